"""GGUF row decoding on the GPU: ``block_layout`` and ``dequantize_rows``.

Mirrors kaggle/glm53_offload/gguf_quant.py:57-60,180-216 (and the layout
table and Q4_0/Q4_1/Q5_0/Q5_1/IQ4_NL decoder of kaggle/qwen38_tpu/quant.py:7-55)
with a ``backend="hip"`` decoder for every type in ``BLOCK_LAYOUTS``. Output is
FP32 or BF16 (RNE of the FP32 value, as ``astype(bfloat16)`` does).
"""

import torch

from . import _lib

BLOCK_LAYOUTS = {
    "Q4_K": (256, 144),
    "Q5_K": (256, 176),
    "Q6_K": (256, 210),
    "Q8_0": (32, 34),
    "F16": (1, 2),
    "BF16": (1, 2),
    "F32": (1, 4),
    "Q4_0": (32, 18),
    "Q4_1": (32, 20),
    "Q5_0": (32, 22),
    "Q5_1": (32, 24),
    "IQ4_NL": (32, 18),
}
DEVICE_TYPES = tuple(BLOCK_LAYOUTS)
# GGMLQuantizationType values of the named formats (GGUF file format)
_GGML_IDS = {0: "F32", 1: "F16", 8: "Q8_0", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 30: "BF16"}


def normalize_qtype(qtype):
    """Canonical format name of ``qtype``: an enum member (by its ``name``), a
    string such as "q6_k" or "GGMLQuantizationType.Q6_K" (the part after the
    last dot, upper-cased), or a GGML type id. Accepts the spellings of
    gguf_quant.py:42-54 and raises its ValueError for anything else."""
    def bad():
        return ValueError(f"unsupported GGUF quantization type: {qtype!r}")

    name = getattr(qtype, "name", None)
    if name is None and isinstance(qtype, str):
        name = qtype.split(".")[-1]
    if name is None:
        try:
            name = _GGML_IDS.get(int(qtype))
        except (TypeError, ValueError):
            name = None
        if name is None:
            raise bad()
    name = str(name).upper()
    if name not in BLOCK_LAYOUTS:
        raise bad()
    return name


def block_layout(qtype):
    """(values_per_block, bytes_per_block)."""
    return BLOCK_LAYOUTS[normalize_qtype(qtype)]


def dequantize_rows(raw, qtype, row_width, dtype=None, backend="hip"):
    """Decode uint8 [..., blocks, bytes] on the GPU -> [..., row_width].

    ``dtype`` is torch.float32 (default) or torch.bfloat16.
    """
    name = normalize_qtype(qtype)
    if not isinstance(row_width, int):
        raise TypeError("row_width must be an integer")
    if backend != "hip":
        raise ValueError("backend must be 'hip' (the NumPy decoder is the test oracle)")
    if name not in DEVICE_TYPES:
        raise ValueError(f"backend='hip' decodes {', '.join(DEVICE_TYPES)}; got {name}")
    if not isinstance(raw, torch.Tensor) or raw.device.type != "cuda":
        raise ValueError("raw must be a uint8 torch tensor on a GPU device")
    if raw.dtype != torch.uint8:
        raise TypeError(f"raw must have dtype uint8; got {raw.dtype}")
    values, size = BLOCK_LAYOUTS[name]
    if raw.ndim < 2:
        raise ValueError("raw must have shape (..., blocks_per_row, bytes_per_block)")
    if raw.shape[-1] != size:
        raise ValueError(f"{name} blocks contain {size} bytes; got {raw.shape[-1]}")
    if row_width <= 0:
        raise ValueError("row_width must be a positive integer")
    blocks = (row_width + values - 1) // values
    if raw.shape[-2] != blocks:
        raise ValueError(f"row_width {row_width} requires {blocks} {name} blocks; got {raw.shape[-2]}")
    dtype = torch.float32 if dtype is None else dtype
    if dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("dtype must be torch.float32 or torch.bfloat16")
    lead = tuple(raw.shape[:-2])
    rows = 1
    for s in lead:
        rows *= s
    out = torch.empty(lead + (row_width,), dtype=dtype, device=raw.device)
    lib = _lib.load()
    with torch.cuda.device(raw.device):
        rc = lib.q6moe_gguf_decode(
            _lib.ptr(raw.contiguous()), _lib.GGUF_TYPE_CODES[name], rows, row_width, _lib.ptr(out),
            _lib.BF16 if dtype == torch.bfloat16 else _lib.F32, _lib.stream_handle(raw.device),
        )
    _lib.check(rc, "dequantize_rows")
    return out
