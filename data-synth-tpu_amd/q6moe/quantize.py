"""Build-owned float -> GGUF block quantizers (host, NumPy).

The reference never quantizes Q6_K or Q4_K weights: its checkpoints arrive as
GGUF bytes and ``pack_q6`` only permutes them (kaggle/packed_q6/layout.py:1-6,
kaggle/glm53_offload/gguf_quant.py:5-7). Synthetic workloads need GGUF bytes
from N(0, sigma) weights, so this module supplies deterministic quantizers.
They fix nothing about the decode/matmul semantics, which are defined on the
bytes alone.

* ``quantize_q6_k``: per 16-value sub-block the value of largest magnitude v
  maps to code -32, sub-scale s = v / -32; the block scale is
  d = fp16(s_max / -128) for the sub-scale of largest magnitude; integer
  sub-scales sc = clip(rint(s / d), -128, 127); codes
  clip(rint(w / (d * sc)), -32, 31). (The same extreme-maps-to--32 idea as
  ggml's reference Q6_K quantizer, without its RMSE search.)
* ``quantize_q4_k``: per 32-value sub-block min m = -min(0, min w) and range
  s = (max w + m) / 15; d = fp16(max s / 63), dmin = fp16(max m / 63);
  6-bit sc = rint(s / d), mn = rint(m / dmin); codes
  clip(rint((w + dmin * mn) / (d * sc)), 0, 15).
* ``quantize_q5_k``: as Q4_K with 31 levels, the code's bit 4 in the 32
  high-bit bytes.
* ``quantize_q5_1``: per 32 values m = min w, d = (max w - m) / 31 (FP16),
  codes clip(rint((w - m) / d), 0, 31).
* ``quantize_q8_0``: kaggle/qwen38_tpu/compute.py:41-49 (``pack_q8``).

Rows whose width is not a multiple of the block size are zero-padded.
"""

import numpy as np

_CHUNK_ROWS = 512


def _blocks(w, values):
    w = np.asarray(w, np.float32)
    if w.ndim != 2:
        raise ValueError("weights must be [rows, width]")
    rows, width = w.shape
    nb = -(-width // values)
    if nb * values != width:
        w = np.pad(w, ((0, 0), (0, nb * values - width)))
    return w, rows, nb


def _safe_div(a, b):
    with np.errstate(divide="ignore", invalid="ignore"):
        return np.where(b != 0, a / np.where(b != 0, b, 1), 0).astype(np.float32)


def _q6_rows(w):
    rows = w.shape[0]
    sub = w.reshape(rows, -1, 16, 16)
    idx = np.argmax(np.abs(sub), axis=-1)[..., None]
    v = np.take_along_axis(sub, idx, axis=-1)[..., 0]
    s = (v / np.float32(-32)).astype(np.float32)
    j = np.argmax(np.abs(s), axis=-1)[..., None]
    m = np.take_along_axis(s, j, axis=-1)[..., 0]
    d16 = (m / np.float32(-128)).astype(np.float16)
    d = d16.astype(np.float32)
    sc = np.clip(np.rint(_safe_div(s, d[..., None])), -128, 127).astype(np.int8)
    ds = (d[..., None] * sc.astype(np.float32)).astype(np.float32)
    code = np.clip(np.rint(_safe_div(sub, ds[..., None])), -32, 31).astype(np.int16)
    q = (code + 32).astype(np.uint8).reshape(rows, -1, 2, 4, 32)  # [h, quarter, l]
    ql = ((q[:, :, :, 0:2] & 15) | ((q[:, :, :, 2:4] & 15) << 4)).reshape(rows, -1, 128)
    qh = np.zeros(q.shape[:3] + (32,), np.uint8)
    for quarter in range(4):
        qh |= ((q[:, :, :, quarter] >> 4) & 3) << (2 * quarter)
    out = np.empty((rows, q.shape[1], 210), np.uint8)
    out[..., 0:128] = ql
    out[..., 128:192] = qh.reshape(rows, -1, 64)
    out[..., 192:208] = sc.view(np.uint8)
    out[..., 208:210] = d16.view(np.uint8).reshape(rows, -1, 2)
    return out


def quantize_q6_k(w):
    """FP32 [rows, width] -> GGUF Q6_K bytes [rows, ceil(width/256), 210]."""
    w, rows, nb = _blocks(w, 256)
    out = np.empty((rows, nb, 210), np.uint8)
    for r0 in range(0, rows, _CHUNK_ROWS):
        out[r0 : r0 + _CHUNK_ROWS] = _q6_rows(w[r0 : r0 + _CHUNK_ROWS])
    return out


def _k_rows(w, levels):
    """Q4_K (levels 15) / Q5_K (levels 31) scales, mins and codes of [rows, width]."""
    rows = w.shape[0]
    sub = w.reshape(rows, -1, 8, 32)
    lo = np.minimum(sub.min(-1), 0).astype(np.float32)
    hi = sub.max(-1).astype(np.float32)
    m = (-lo).astype(np.float32)
    s = ((hi - lo) / np.float32(levels)).astype(np.float32)
    d16 = (s.max(-1) / np.float32(63)).astype(np.float16)
    dm16 = (m.max(-1) / np.float32(63)).astype(np.float16)
    d, dm = d16.astype(np.float32), dm16.astype(np.float32)
    sc = np.clip(np.rint(_safe_div(s, d[..., None])), 0, 63).astype(np.uint8)
    mn = np.clip(np.rint(_safe_div(m, dm[..., None])), 0, 63).astype(np.uint8)
    a = (d[..., None] * sc).astype(np.float32)
    b = (dm[..., None] * mn).astype(np.float32)
    q = np.clip(np.rint(_safe_div(sub + b[..., None], a[..., None])), 0, levels).astype(np.uint8)
    head = np.empty((rows, q.shape[1], 16), np.uint8)
    head[..., 0:2] = d16.view(np.uint8).reshape(rows, -1, 2)
    head[..., 2:4] = dm16.view(np.uint8).reshape(rows, -1, 2)
    head[..., 4:8] = (sc[..., :4] & 63) | ((sc[..., 4:] >> 4) << 6)
    head[..., 8:12] = (mn[..., :4] & 63) | ((mn[..., 4:] >> 4) << 6)
    head[..., 12:16] = (sc[..., 4:] & 15) | ((mn[..., 4:] & 15) << 4)
    return head, q


def _nibbles(q):
    """Codes [rows, nb, 8, 32] -> 128 bytes per block: chunk i holds sub-block 2i
    in the low nibbles and 2i + 1 in the high nibbles (gguf_quant.py:137-141)."""
    return ((q[:, :, 0::2] & 15) | ((q[:, :, 1::2] & 15) << 4)).reshape(q.shape[0], -1, 128)


def _q4_rows(w):
    head, q = _k_rows(w, 15)
    return np.concatenate((head, _nibbles(q)), axis=-1)


def _q5k_rows(w):
    head, q = _k_rows(w, 31)
    qh = np.zeros(q.shape[:2] + (32,), np.uint8)
    for j in range(8):  # bit j of byte l: bit 4 of sub-block j's code l (gguf_quant.py:142-147)
        qh |= ((q[:, :, j] >> 4) & 1) << j
    return np.concatenate((head, qh, _nibbles(q)), axis=-1)


def quantize_q4_k(w):
    """FP32 [rows, width] -> GGUF Q4_K bytes [rows, ceil(width/256), 144]."""
    w, rows, nb = _blocks(w, 256)
    out = np.empty((rows, nb, 144), np.uint8)
    for r0 in range(0, rows, _CHUNK_ROWS):
        out[r0 : r0 + _CHUNK_ROWS] = _q4_rows(w[r0 : r0 + _CHUNK_ROWS])
    return out


def quantize_q5_k(w):
    """FP32 [rows, width] -> GGUF Q5_K bytes [rows, ceil(width/256), 176]."""
    w, rows, nb = _blocks(w, 256)
    out = np.empty((rows, nb, 176), np.uint8)
    for r0 in range(0, rows, _CHUNK_ROWS):
        out[r0 : r0 + _CHUNK_ROWS] = _q5k_rows(w[r0 : r0 + _CHUNK_ROWS])
    return out


def quantize_q5_1(w):
    """FP32 [rows, width] -> GGUF Q5_1 bytes [rows, width/32, 24]: per 32 values
    m = fp16(min), d = fp16((max - min) / 31), codes clip(rint((w - m) / d), 0, 31);
    bytes d, m, the 32 high bits, then byte i = code i | code i+16 << 4
    (the layout kaggle/qwen38_tpu/quant.py:34-53 decodes)."""
    w, rows, nb = _blocks(w, 32)
    g = w.reshape(rows, nb, 32)
    m16 = g.min(-1).astype(np.float16)
    d16 = ((g.max(-1) - m16.astype(np.float32)) / np.float32(31)).astype(np.float16)
    d, m = d16.astype(np.float32), m16.astype(np.float32)
    q = np.clip(np.rint(_safe_div(g - m[..., None], np.broadcast_to(d[..., None], g.shape))), 0, 31)
    q = q.astype(np.uint32)
    qh = np.zeros((rows, nb), np.uint32)
    for i in range(32):
        qh |= ((q[..., i] >> 4) & 1) << i
    out = np.empty((rows, nb, 24), np.uint8)
    out[..., 0:2] = d16.view(np.uint8).reshape(rows, nb, 2)
    out[..., 2:4] = m16.view(np.uint8).reshape(rows, nb, 2)
    out[..., 4:8] = qh.astype("<u4").view(np.uint8).reshape(rows, nb, 4)
    out[..., 8:24] = ((q[..., :16] & 15) | ((q[..., 16:] & 15) << 4)).astype(np.uint8)
    return out


def quantize_q8_0(w):
    """FP32 [rows, width] -> GGUF Q8_0 bytes [rows, width/32, 34] (compute.py:41-49)."""
    w, rows, nb = _blocks(w, 32)
    g = w.reshape(rows, nb, 32)
    scale = (np.max(np.abs(g), -1) / np.float32(127)).astype("<f2")
    codes = np.clip(np.rint(g / np.where(scale == 0, 1, scale)[..., None]), -127, 127)
    return np.concatenate(
        (scale.view(np.uint8).reshape(rows, nb, 2), codes.astype(np.int8).view(np.uint8)), axis=-1
    )


QUANTIZERS = {"Q6_K": quantize_q6_k, "Q5_K": quantize_q5_k, "Q4_K": quantize_q4_k, "Q8_0": quantize_q8_0,
              "Q5_1": quantize_q5_1}
