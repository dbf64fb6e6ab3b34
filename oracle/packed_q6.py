"""Scalar Q6_K / SoA-layout oracle (test oracle only).

Follows ``kaggle/packed_q6/reference.py:11-57`` (per-position decode, BF16
round-to-nearest-even, FP64 projection, the seeded fixture generator),
``kaggle/packed_q6/kernel.py:27-41`` (exact FP16 -> FP32 from integer
fields) and ``kaggle/packed_q6/layout.py:13-18,71-90`` (the SoA byte map of
layout ``q6_k_soa_n64_k256_v1``), written as independent index formulas.
"""

import numpy as np

QK = 256
BLOCK_BYTES = 210
OUTPUT_TILE = 64
TILE_BYTES = OUTPUT_TILE * 208
SCALE_TILE_BYTES = OUTPUT_TILE * 2
SCALE_FETCH_BYTES = 512


def decode_reference(raw, input_features):
    """GGUF Q6_K bytes [N, KB, 210] -> FP32 [N, input_features].

    Each of the 256 positions p of a block is decoded on its own
    (reference.py:19-31): h = p // 128, q = (p % 128) // 32, l = p % 32,
    low nibble from ql[h*64 + (q%2)*32 + l] >> 4*(q//2), two high bits from
    qh[h*32 + l] >> 2q, code = (lo | hi << 4) - 32, signed sub-scale
    byte[192 + p//16], FP16 d at bytes 208-209, value (d * sc) * code.
    """
    raw = np.asarray(raw)
    if raw.dtype != np.uint8 or raw.ndim != 3 or raw.shape[2] != BLOCK_BYTES:
        raise ValueError("Expected uint8 [N, K_blocks, 210]")
    if input_features < 1 or raw.shape[1] != (input_features + QK - 1) // QK:
        raise ValueError("Input width does not match Q6 block count")
    n, kb, _ = raw.shape
    d = np.ascontiguousarray(raw[:, :, 208:210]).view("<f2").reshape(n, kb).astype(np.float32)
    out = np.empty((n, kb, QK), np.float32)
    for p in range(QK):
        h, q, l = p // 128, (p % 128) // 32, p % 32
        lo = (raw[:, :, h * 64 + (q % 2) * 32 + l].astype(np.int32) >> (4 * (q // 2))) & 15
        hi = (raw[:, :, 128 + h * 32 + l].astype(np.int32) >> (2 * q)) & 3
        code = (lo | (hi << 4)) - 32
        sc = raw[:, :, 192 + p // 16].astype(np.int8).astype(np.float32)
        out[:, :, p] = (d * sc) * code.astype(np.float32)
    return out.reshape(n, kb * QK)[:, :input_features]


def fp16_bits_to_f32(bits):
    """Finite FP16 bit patterns -> exact FP32 from the integer fields.

    kernel.py:27-41: exponent e, mantissa m; e == 0 gives m * 2**-24
    (subnormals and signed zero), otherwise bits ((e + 112) << 23) | m << 13.
    """
    bits = np.asarray(bits, np.uint32)
    e = (bits >> 10) & 31
    m = bits & 1023
    normal = (((e + 112) << 23) | (m << 13)).astype(np.uint32).view(np.float32)
    mag = np.where(e == 0, m.astype(np.float32) * np.float32(2.0**-24), normal).astype(np.float32)
    return (mag.view(np.uint32) | ((bits & 0x8000) << 16)).view(np.float32)


def bf16_round(x):
    """FP32 -> BF16 round-to-nearest-even, returned as FP32 (reference.py:35-41).

    NaN inputs keep their payload and are made quiet (bit 22 set).
    """
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    return np.where(nan, (b | 0x00400000).astype(np.uint32), r).view(np.float32)


def bf16_bits(x):
    """FP32 -> uint16 BF16 bit patterns with RNE."""
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def bf16_to_f32(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def projection_reference(x, raw):
    """FP64 dot of BF16-rounded operands, returned as FP32 (reference.py:44-48)."""
    x = bf16_round(x)
    w = bf16_round(decode_reference(raw, x.shape[1]))
    return (x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32)


def fixture(outputs, inputs, seed=3826):
    """Random legal Q6_K bytes with d in {+-0.003, +-0.001, 0} (reference.py:51-57).

    The draw order (bytes first, then the FP16 choice) is kept so that the
    same seed yields the same bytes as the reference generator.
    """
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, (outputs, (inputs + QK - 1) // QK, BLOCK_BYTES), dtype=np.uint8)
    d = rng.choice(np.array([-0.003, -0.001, 0, 0.001, 0.003], dtype="<f2"), raw.shape[:2])
    raw[:, :, 208:210] = d.view(np.uint8).reshape(*raw.shape[:2], 2)
    return raw


def soa_offsets(output_features, input_features):
    """Where every GGUF byte lands in the SoA planes (layout.py:71-90).

    Returns (plane, offset) arrays of shape [N, KB, 210]: plane 0 is the data
    plane, plane 1 the FP16 scale plane. For tile t = (n // 64) * KB + k and
    row r = n % 64: byte b < 128 -> t*13312 + r*128 + b; 128 <= b < 192 ->
    t*13312 + 8192 + r*64 + (b-128); 192 <= b < 208 -> t*13312 + 12288 +
    r*16 + (b-192); b in {208, 209} -> scale plane (t*64 + r)*2 + (b-208).
    """
    kb = (input_features + QK - 1) // QK
    n = np.arange(output_features)[:, None, None]
    k = np.arange(kb)[None, :, None]
    b = np.arange(BLOCK_BYTES)[None, None, :]
    t = (n // OUTPUT_TILE) * kb + k
    r = n % OUTPUT_TILE
    data = np.where(
        b < 128,
        t * TILE_BYTES + r * 128 + b,
        np.where(b < 192, t * TILE_BYTES + 8192 + r * 64 + (b - 128), t * TILE_BYTES + 12288 + r * 16 + (b - 192)),
    )
    scale = (t * OUTPUT_TILE + r) * 2 + (b - 208)
    shape = (output_features, kb, BLOCK_BYTES)
    plane = np.broadcast_to((b >= 208).astype(np.int64), shape).copy()
    return plane, np.broadcast_to(np.where(b >= 208, scale, data), shape).copy()


def soa_sizes(output_features, input_features):
    """(data bytes, scale-plane bytes) of one packed projection (layout.py:72-77)."""
    kb = (input_features + QK - 1) // QK
    tiles = (output_features + OUTPUT_TILE - 1) // OUTPUT_TILE
    scale = tiles * kb * SCALE_TILE_BYTES
    return tiles * kb * TILE_BYTES, -(-scale // SCALE_FETCH_BYTES) * SCALE_FETCH_BYTES


def decode_soa(data, scales, output_features, input_features):
    """Decode straight from the SoA planes by inverting ``soa_offsets``."""
    plane, off = soa_offsets(output_features, input_features)
    raw = np.where(plane == 0, np.asarray(data)[np.where(plane == 0, off, 0)], np.asarray(scales)[np.where(plane == 1, off, 0)])
    return decode_reference(raw.astype(np.uint8), input_features)
