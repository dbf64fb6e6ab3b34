"""Packed-Q6 projection on MI355X: the ``q6_matmul`` operator.

Mirrors kaggle/packed_q6/kernel.py:98-148: same signature, argument checks
and messages, FP32 result of ``x @ decode(W).T`` with BF16 operands and FP32
accumulation, zero-padding of partial K blocks. The work is one launch of the
HIP kernel ``q6_skinny_kernel`` (libq6moe.so); nothing runs on the CPU.

``batch_tile`` is validated as in the reference but does not change the
result (the HIP kernel tiles tokens by 16). ``interpret`` is accepted for
call compatibility and ignored: there is no interpreter or CPU path.
"""

import torch

from . import _lib
from .layout import OUTPUT_TILE, QK, SCALE_FETCH_BYTES, SCALE_TILE_BYTES, TILE_BYTES


def _plane_sizes(output_features, inputs):
    blocks = (inputs + QK - 1) // QK
    tiles = (output_features + OUTPUT_TILE - 1) // OUTPUT_TILE
    scale = tiles * blocks * SCALE_TILE_BYTES
    return tiles * blocks * TILE_BYTES, -(-scale // SCALE_FETCH_BYTES) * SCALE_FETCH_BYTES


def _require_device(*tensors):
    for t in tensors:
        if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
            raise ValueError("q6moe operators take torch tensors on a GPU device")


def q6_matmul(x, packed, scales, *, output_features, batch_tile=8, interpret=False, out_dtype=None):
    """FP32 (or ``out_dtype``) result of BF16 x @ decode(Q6_K).T.

    x: [M, K] torch.bfloat16 on the GPU. packed/scales: flat uint8 planes from
    ``pack_q6`` (moved to the same device). Returns [M, output_features].
    """
    del interpret
    if x.ndim != 2 or min(x.shape) < 1 or x.dtype != torch.bfloat16:
        raise ValueError("x must be a nonempty [M,K] BF16 array")
    if type(output_features) is not int or output_features < 1:
        raise ValueError("output_features must be positive")
    if type(batch_tile) is not int or batch_tile < 8 or batch_tile % 8:
        raise ValueError("batch_tile must be a positive multiple of 8")
    m, inputs = x.shape
    data_size, scale_size = _plane_sizes(output_features, inputs)
    if packed.dtype != torch.uint8 or tuple(packed.shape) != (data_size,):
        raise ValueError("Packed Q6 dtype/shape does not match projection dimensions")
    if scales.dtype != torch.uint8 or tuple(scales.shape) != (scale_size,):
        raise ValueError("Packed Q6 scale dtype/shape does not match projection dimensions")
    _require_device(x, packed, scales)
    out_dtype = torch.float32 if out_dtype is None else out_dtype
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("out_dtype must be torch.float32 or torch.bfloat16")
    x = x if x.stride(1) == 1 else x.contiguous()
    packed, scales = packed.contiguous(), scales.contiguous()
    y = torch.empty((m, output_features), dtype=out_dtype, device=x.device)
    lib = _lib.load()
    with torch.cuda.device(x.device):
        rc = lib.q6moe_q6_matmul(
            _lib.ptr(x), m, inputs, x.stride(0), _lib.ptr(packed), _lib.ptr(scales),
            output_features, _lib.ptr(y), _lib.BF16 if out_dtype == torch.bfloat16 else _lib.F32,
            output_features, _lib.stream_handle(x.device),
        )
    _lib.check(rc, "q6_matmul")
    return y


def q6_decode(packed, scales, *, output_features, input_features):
    """Whole-matrix decode of packed planes -> BF16 [N, K] (bit-exact RNE)."""
    data_size, scale_size = _plane_sizes(output_features, input_features)
    if packed.dtype != torch.uint8 or packed.numel() < data_size:
        raise ValueError("Packed Q6 dtype/shape does not match projection dimensions")
    if scales.dtype != torch.uint8 or scales.numel() < scale_size:
        raise ValueError("Packed Q6 scale dtype/shape does not match projection dimensions")
    _require_device(packed, scales)
    out = torch.empty((output_features, input_features), dtype=torch.bfloat16, device=packed.device)
    lib = _lib.load()
    with torch.cuda.device(packed.device):
        rc = lib.q6moe_q6_decode(
            _lib.ptr(packed.contiguous()), _lib.ptr(scales.contiguous()), output_features,
            input_features, _lib.ptr(out), input_features, _lib.stream_handle(packed.device),
        )
    _lib.check(rc, "q6_decode")
    return out


def q6_pack(raw, input_features):
    """Device GGUF Q6_K [N, KB, 210] uint8 -> (data, scales) SoA planes on the same device.

    Byte-identical to ``pack_q6`` for finite block scales (the host packer also
    rejects non-finite ones; this device repack does not inspect values).
    """
    _require_device(raw)
    if raw.dtype != torch.uint8 or raw.ndim != 3 or raw.shape[2] != 210:
        raise ValueError("Expected [output_features, ceil(input_features / 256), 210]")
    n = raw.shape[0]
    if raw.shape[1] != (input_features + QK - 1) // QK:
        raise ValueError("Expected [output_features, ceil(input_features / 256), 210]")
    data_size, scale_size = _plane_sizes(n, input_features)
    data = torch.empty(data_size, dtype=torch.uint8, device=raw.device)
    scales = torch.empty(scale_size, dtype=torch.uint8, device=raw.device)
    lib = _lib.load()
    with torch.cuda.device(raw.device):
        rc = lib.q6moe_q6_pack(
            _lib.ptr(raw.contiguous()), n, input_features, _lib.ptr(data), _lib.ptr(scales),
            _lib.stream_handle(raw.device),
        )
    _lib.check(rc, "q6_pack")
    return data, scales
