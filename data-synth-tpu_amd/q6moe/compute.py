"""BF16 and W8A8 projections of GGUF Q8_0 weights: ``q8_matmul``,
``bf16_q8_matmul`` and ``pack_q8``.

Mirrors kaggle/qwen38_tpu/compute.py:20-49. ``q8_matmul`` quantises the
activations per row and 32-value group (scale max|x| / 127 in FP32, codes
clip(rint(x / scale), -127, 127)), takes each group's INT8 x INT8 dot products
on the matrix cores (v_mfma_i32_16x16x32_i8) and sums (f32(partial) * scale) *
weight_scale over the groups in FP32, rounding the result to BF16
(``q6moe_q8_matmul``). ``bf16_q8_matmul`` decodes the weights to BF16 and
multiplies with FP32 accumulation. ``pack_q8`` is the reference's packer.
"""

import torch

from . import _lib
from .experts import _CACHE, pack_experts
from .quant import dequantize_rows
from .quantize import quantize_q8_0 as pack_q8

__all__ = ["q8_matmul", "bf16_q8_matmul", "pack_q8"]


def _packed_table(packed, k):
    if not isinstance(packed, torch.Tensor) or packed.device.type != "cuda" or packed.dtype != torch.uint8:
        raise ValueError("packed must be Q8_0 bytes [rows, K/32, 34] as a uint8 GPU tensor")
    if packed.ndim != 3 or packed.shape[1:] != (k // 32, 34):
        raise ValueError(f"packed must be Q8_0 bytes [rows, {k // 32}, 34] for x of width {k}")
    return _CACHE.get(packed, "Q8_0", packed.shape[0], k, single=True)


def q8_matmul(x, packed, *, output_dtype=None):
    """W8A8 dot (compute.py:20-34): x [M, K] BF16 on the GPU, packed Q8_0
    [N, K/32, 34] -> [M, N] in ``output_dtype`` (default x's dtype, BF16)."""
    if not isinstance(x, torch.Tensor) or x.device.type != "cuda" or x.dtype != torch.bfloat16 or x.ndim != 2:
        raise ValueError("x must be a BF16 [M, K] GPU tensor")
    m, k = x.shape
    if k % 32 or m < 1:
        raise ValueError("x must be nonempty with a width that is a multiple of 32")
    output_dtype = x.dtype if output_dtype is None else output_dtype
    if output_dtype != torch.bfloat16:
        raise ValueError("q8_matmul returns BF16 (compute_cast of the FP32 sums)")
    table = _packed_table(packed, k)
    x = x.contiguous()
    n = table.rows
    y = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    lib = _lib.load()
    ws = torch.empty(int(lib.q6moe_q8_matmul_workspace_size(m, k)), dtype=torch.uint8, device=x.device)
    with torch.cuda.device(x.device):
        rc = lib.q6moe_q8_matmul(x.data_ptr(), m, k, table.data.data_ptr(), n, y.data_ptr(), ws.data_ptr(),
                                 ws.numel(), _lib.stream_handle(x.device))
    _lib.check(rc, "q8_matmul")
    return y


def bf16_q8_matmul(x, packed):
    """compute.py:36-37: linear(x, dequantize_rows(packed, "Q8_0")): BF16
    weights, FP32 accumulation, BF16 result (library GEMM)."""
    w = dequantize_rows(packed, "Q8_0", x.shape[-1], dtype=torch.bfloat16)
    return torch.mm(w, x.t().contiguous()).t()


def prepack_q8(packed, k, device=None):
    """The unit-major table ``q8_matmul`` runs on, built once (load time)."""
    return pack_experts(packed.reshape(1, -1), "Q8_0", packed.shape[0], k, device)
