"""GPU check of the FP32 sigmoid of the SwiGLU epilogues and the
shared-expert gate, where(x >= 0, 1, e) / (1 + e) with e = exp(-|x|)
(kaggle/qwen38_tpu/numerics.py:42-45), over every non-NaN BF16 input (the
only inputs its callers pass): the library's quotient must be the correctly
rounded FP32 quotient of its own e, bit for bit, and e must lie within a
couple of ulps of NumPy's float32 exp (the exponential itself is
tolerance-only)."""

import numpy as np
import pytest
import torch

from q6moe import _lib

pytestmark = pytest.mark.gpu


def test_sigmoid_quotient_is_correctly_rounded_for_every_bf16_input(device):
    bits = np.arange(1 << 16, dtype=np.uint32)
    x = (bits << 16).view(np.float32)
    keep = ~np.isnan(x)
    x = x[keep]
    xb = torch.from_numpy(bits[keep].astype(np.uint16).view(np.int16).copy()).to(device)
    n = xb.numel()
    e = torch.empty(n, dtype=torch.float32, device=device)
    s = torch.empty(n, dtype=torch.float32, device=device)
    lib = _lib.load()
    with torch.cuda.device(device):
        rc = lib.q6moe_sigmoid_probe(xb.data_ptr(), n, e.data_ptr(), s.data_ptr(), _lib.stream_handle(device))
    _lib.check(rc, "sigmoid_probe")
    torch.cuda.synchronize(device)
    e = e.cpu().numpy()
    s = s.cpu().numpy()
    num = np.where(x >= 0, np.float32(1), e).astype(np.float32)
    want = (num / (np.float32(1) + e)).astype(np.float32)  # IEEE float32 division
    mismatch = np.flatnonzero(s.view(np.uint32) != want.view(np.uint32))
    assert mismatch.size == 0, f"{mismatch.size} inputs differ, first x = {x[mismatch[:5]]}"
    ref_e = np.exp(-np.abs(x)).astype(np.float32)
    ulps = np.abs(e.view(np.int32).astype(np.int64) - ref_e.view(np.int32).astype(np.int64))
    assert ulps.max() <= 2, f"exp differs from float32 exp by {ulps.max()} ulp"
