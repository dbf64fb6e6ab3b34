"""NumPy restatement of the reference's GGUF block decoders (test oracle only).

Follows ``kaggle/glm53_offload/gguf_quant.py:21-29`` (block sizes),
``:63-177`` (``_decode``), ``:180-216`` (``dequantize_rows``) and
``kaggle/qwen38_tpu/quant.py:7-55`` (Q4_0/Q4_1/Q5_0/Q5_1/IQ4_NL).

Values are produced in FP32 exactly as the reference does: Q6_K and Q8_0
products are exact in FP32; Q4_K/Q5_K round once at the final subtraction.
"""

import numpy as np

# (values per block, bytes per block) -- gguf_quant.py:21-29, quant.py:8
BLOCKS = {
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

# quant.py:7
IQ4_GRID = np.array(
    (-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113), np.float32
)


def block_layout(qtype):
    return BLOCKS[qtype]


def _half(raw, at):
    """Little-endian FP16 field at byte ``at`` -> FP32 (exact widening)."""
    b = raw[..., at : at + 2].astype(np.uint16)
    return (b[..., 0] | (b[..., 1] << 8)).view(np.float16).astype(np.float32)


def _k_scales(raw):
    """6-bit (scale, min) pairs of Q4_K/Q5_K -- gguf_quant.py:118-135.

    Bytes 4..7 carry the low 6 bits of scales 0-3 (top 2 bits feed 4-7),
    bytes 8..11 the same for mins, bytes 12..15 the low nibbles of 4-7.
    """
    s = raw[..., 4:8].astype(np.uint8)
    m = raw[..., 8:12].astype(np.uint8)
    x = raw[..., 12:16].astype(np.uint8)
    scales = np.concatenate((s & 63, (x & 15) | ((s >> 2) & 48)), axis=-1)
    mins = np.concatenate((m & 63, (x >> 4) | ((m >> 2) & 48)), axis=-1)
    return scales.astype(np.float32), mins.astype(np.float32)


def _decode_block(raw, qtype):
    """raw [..., bytes] -> FP32 [..., values] for one block type."""
    if qtype == "F16":
        return _half(raw, 0)[..., None]
    if qtype == "BF16":
        b = raw.astype(np.uint32)
        return ((b[..., 0] | (b[..., 1] << 8)) << 16).view(np.float32)[..., None]
    if qtype == "F32":
        return np.ascontiguousarray(raw).view("<f4").astype(np.float32)
    if qtype == "Q8_0":  # gguf_quant.py:111-114
        q = raw[..., 2:34].view(np.int8).astype(np.float32)
        return _half(raw, 0)[..., None] * q
    if qtype in ("Q4_K", "Q5_K"):  # gguf_quant.py:115-157
        d, dmin = _half(raw, 0), _half(raw, 2)
        sc, mn = _k_scales(raw)
        if qtype == "Q4_K":
            qs = raw[..., 16:144].reshape(*raw.shape[:-1], 4, 32)
            q = np.stack((qs & 15, qs >> 4), axis=-2)  # sub-block 2i low, 2i+1 high
        else:
            qs = raw[..., 48:176].reshape(*raw.shape[:-1], 4, 32)
            q = np.stack((qs & 15, qs >> 4), axis=-2)
            qh = raw[..., 16:48]
            bits = (qh[..., None, :] >> np.arange(8, dtype=np.uint8)[:, None]) & 1
            q = q.reshape(*raw.shape[:-1], 8, 32) | (bits << 4)
        q = q.reshape(*raw.shape[:-1], 8, 32).astype(np.float32)
        w = d[..., None, None] * sc[..., None] * q - dmin[..., None, None] * mn[..., None]
        return w.reshape(*raw.shape[:-1], 256)
    if qtype == "Q6_K":  # gguf_quant.py:158-173
        ql = raw[..., 0:128].reshape(*raw.shape[:-1], 2, 64)
        lo = np.stack((ql & 15, ql >> 4), axis=-2).reshape(*raw.shape[:-1], 2, 4, 32)
        qh = raw[..., 128:192].reshape(*raw.shape[:-1], 2, 1, 32)
        hi = (qh >> (2 * np.arange(4, dtype=np.uint8))[:, None]) & 3
        # lo stacks (ql[0:32]&15, ql[32:64]&15, ql[0:32]>>4, ql[32:64]>>4) per half
        code = (lo | (hi << 4)).astype(np.int16) - 32
        sc = raw[..., 192:208].view(np.int8).astype(np.float32)
        w = _half(raw, 208)[..., None, None] * sc.reshape(*raw.shape[:-1], 16, 1) * code.reshape(
            *raw.shape[:-1], 16, 16
        ).astype(np.float32)
        return w.reshape(*raw.shape[:-1], 256)
    if qtype in ("Q4_0", "Q4_1", "Q5_0", "Q5_1", "IQ4_NL"):  # kaggle/qwen38_tpu/quant.py:28-55
        affine = qtype in ("Q4_1", "Q5_1")
        base = 4 if affine else 2
        wide = qtype.startswith("Q5")
        low = raw[..., base + (4 if wide else 0) :]
        q = np.concatenate((low & 15, low >> 4), axis=-1).astype(np.int32)
        if wide:
            f = raw[..., base : base + 4].astype(np.uint32)
            word = f[..., 0] | (f[..., 1] << 8) | (f[..., 2] << 16) | (f[..., 3] << 24)
            q |= (((word[..., None] >> np.arange(32, dtype=np.uint32)) & 1) << 4).astype(np.int32)
        if qtype == "IQ4_NL":
            q = IQ4_GRID[q]
        elif not affine:
            q = q - (16 if wide else 8)
        w = _half(raw, 0)[..., None] * q.astype(np.float32)
        if affine:
            w = w + _half(raw, 2)[..., None]
        return w.astype(np.float32)
    raise ValueError(f"unsupported GGUF quantization type: {qtype!r}")


def dequantize_rows(raw, qtype, row_width):
    """raw uint8 [..., blocks, bytes] -> FP32 [..., row_width].

    Same contract as gguf_quant.py:180-216 (numpy backend): the block count
    must be ceil(row_width / values); a partial final block is cropped.
    """
    raw = np.asarray(raw)
    if raw.dtype != np.uint8:
        raise TypeError(f"raw must have dtype uint8; got {raw.dtype}")
    values, size = BLOCKS[qtype]
    blocks = (row_width + values - 1) // values
    if raw.ndim < 2 or raw.shape[-1] != size or raw.shape[-2] != blocks:
        raise ValueError(f"row_width {row_width} requires {blocks} {qtype} blocks of {size} bytes")
    out = _decode_block(raw, qtype)
    return out.reshape(*raw.shape[:-2], blocks * values)[..., :row_width].astype(np.float32)
