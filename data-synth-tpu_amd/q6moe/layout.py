"""Lossless GGUF Q6_K -> SoA repack, layout ``q6_k_soa_n64_k256_v1``.

Same interface, error messages and byte layout as the reference packer
(kaggle/packed_q6/layout.py:13-109), so packed planes are interchangeable:

* output rows are grouped in 64-row tiles, K in 256-wide blocks; tile
  t = tile_index * KB + k_block holds 13 312 bytes: the 64 rows' 128 ql
  bytes, then their 64 qh bytes, then their 16 signed sub-scales;
* the FP16 block scales d go to a separate plane, 128 bytes per tile, zero
  padded to a multiple of 512 bytes;
* rows past the end of the last tile are zero bytes; a partial final K
  block keeps its GGUF bytes (the projection zero-pads x).

The repack is a pure byte permutation, written here as one reshape/transpose
of the padded tensor rather than a per-tile loop.
"""

from dataclasses import dataclass

import numpy as np

QK = 256
BLOCK_BYTES = 210
OUTPUT_TILE = 64
TILE_BYTES = OUTPUT_TILE * 208
SCALE_TILE_BYTES = OUTPUT_TILE * 2
SCALE_FETCH_BYTES = 512
LAYOUT = "q6_k_soa_n64_k256_v1"
_REGIONS = ((0, 128), (128, 192), (192, 208))


def input_blocks(input_features):
    return (input_features + QK - 1) // QK


def output_tiles(output_features):
    return (output_features + OUTPUT_TILE - 1) // OUTPUT_TILE


def plane_sizes(output_features, input_features):
    """(data bytes, scale bytes) of one packed projection."""
    tiles, blocks = output_tiles(output_features), input_blocks(input_features)
    scale = tiles * blocks * SCALE_TILE_BYTES
    return tiles * blocks * TILE_BYTES, -(-scale // SCALE_FETCH_BYTES) * SCALE_FETCH_BYTES


@dataclass(frozen=True)
class PackedQ6:
    data: np.ndarray
    scales: np.ndarray
    input_features: int
    output_features: int

    @property
    def input_blocks(self):
        return input_blocks(self.input_features)

    @property
    def output_tiles(self):
        return output_tiles(self.output_features)

    def storage(self):
        original = self.output_features * self.input_blocks * BLOCK_BYTES
        size = self.data.nbytes + self.scales.nbytes
        return dict(
            original_bytes=original,
            packed_bytes=size,
            padding_bytes=size - original,
            padding_ratio=size / original - 1,
            layout=LAYOUT,
            physical_hbm_bytes="requires target allocator measurement",
        )


def _check(raw, input_features):
    if type(input_features) is not int or input_features < 1:
        raise ValueError("input_features must be a positive integer")
    raw = np.asarray(raw)
    if raw.dtype != np.uint8:
        raise TypeError("GGUF Q6_K input must have dtype uint8")
    blocks = input_blocks(input_features)
    if raw.ndim != 3 or raw.shape[0] < 1 or raw.shape[1:] != (blocks, BLOCK_BYTES):
        raise ValueError("Expected [output_features, ceil(input_features / 256), 210]")
    d = np.ascontiguousarray(raw[..., 208:210]).view("<f2")
    if not np.isfinite(d).all():
        raise ValueError("Q6_K block scales must be finite")
    return raw


def pack_q6(raw, input_features):
    """GGUF Q6_K [N, ceil(K/256), 210] uint8 -> PackedQ6 (no arithmetic on values)."""
    raw = _check(raw, input_features)
    n, blocks, _ = raw.shape
    tiles = output_tiles(n)
    padded = np.zeros((tiles * OUTPUT_TILE, blocks, BLOCK_BYTES), np.uint8)
    padded[:n] = raw
    # [tile, row, block, byte] -> [tile, block, row, byte]
    grid = padded.reshape(tiles, OUTPUT_TILE, blocks, BLOCK_BYTES).transpose(0, 2, 1, 3)
    data = np.concatenate(
        [grid[..., a:b].reshape(tiles, blocks, -1) for a, b in _REGIONS], axis=-1
    ).reshape(-1)
    _, scale_size = plane_sizes(n, input_features)
    scales = np.zeros(scale_size, np.uint8)
    used = tiles * blocks * SCALE_TILE_BYTES
    scales[:used] = grid[..., 208:210].reshape(-1)
    return PackedQ6(np.ascontiguousarray(data), scales, input_features, n)


def unpack_q6(packed):
    """Inverse permutation back to GGUF [N, ceil(K/256), 210]."""
    tiles, blocks = packed.output_tiles, packed.input_blocks
    planes = np.asarray(packed.data).reshape(tiles, blocks, TILE_BYTES)
    grid = np.empty((tiles, blocks, OUTPUT_TILE, BLOCK_BYTES), np.uint8)
    start = 0
    for a, b in _REGIONS:
        width = b - a
        grid[..., a:b] = planes[..., start : start + OUTPUT_TILE * width].reshape(
            tiles, blocks, OUTPUT_TILE, width
        )
        start += OUTPUT_TILE * width
    used = tiles * blocks * SCALE_TILE_BYTES
    grid[..., 208:210] = np.asarray(packed.scales)[:used].reshape(tiles, blocks, OUTPUT_TILE, 2)
    rows = grid.transpose(0, 2, 1, 3).reshape(tiles * OUTPUT_TILE, blocks, BLOCK_BYTES)
    return rows[: packed.output_features]


def pack_q6_experts(raw, input_features):
    """Stacked experts [E, N, ceil(K/256), 210] -> (data [E, D], scales [E, S]) uint8."""
    raw = np.asarray(raw)
    if raw.ndim != 4:
        raise ValueError("Expected [experts, output_features, ceil(input_features / 256), 210]")
    parts = [pack_q6(raw[e], input_features) for e in range(raw.shape[0])]
    return np.stack([p.data for p in parts]), np.stack([p.scales for p in parts])
