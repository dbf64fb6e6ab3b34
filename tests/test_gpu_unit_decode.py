"""Bit-exact decode of the unit-major expert tables, through each decoder the
MoE kernels use, against the oracle's ``dequantize_rows`` (gguf_quant.py:111-173).

``q6moe_moe_unpack`` runs the generic kernels' register decode (path 0), the
decode-step kernels' LDS-staged decode (path 1) and the prefill kernels'
whole-block decode (path 2: Q6_K, Q8_0, Q5_1, Q4_K) on a packed table and returns the BF16
weights those kernels feed to the matrix cores. Every weight must equal
RNE_bf16 of the oracle's FP32 value bit for bit; the one allowed difference
is the sign of an exact zero (a Q6_K code of 32 decodes to +0 where d*sc < 0
gives -0 in the reference), which no sum of products can observe.
Inputs: random GGUF bytes with finite, varied FP16 scales (subnormals, signed
zeros, extremes), so every code, sub-scale and scale path is reached.
"""

import numpy as np
import pytest
import torch

from oracle.gguf import block_layout, dequantize_rows
from oracle.packed_q6 import bf16_round
from q6moe.experts import pack_experts, unpack_experts
from q6moe.quantize import QUANTIZERS

pytestmark = pytest.mark.gpu

# FP16 scale bits: normal values across the range, subnormals, signed zeros
_SCALE_BITS = np.array([0x0000, 0x8000, 0x0001, 0x83FF, 0x0400, 0x1C00, 0x2E66, 0xAE66, 0x3C00, 0xBC00,
                        0x2400, 0x1400, 0x5640, 0xD640, 0x7BFF, 0xFBFF], np.uint16)
_SCALE_FIELDS = {"Q6_K": (208,), "Q5_K": (0, 2), "Q4_K": (0, 2), "Q8_0": (0,), "Q5_1": (0, 2)}


def _random_table(qtype, experts, rows, width, seed):
    values, size = block_layout(qtype)
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=(experts, rows, -(-width // values), size), dtype=np.uint8)
    for at in _SCALE_FIELDS[qtype]:
        bits = _SCALE_BITS[rng.integers(0, _SCALE_BITS.size, size=raw.shape[:-1])]
        raw[..., at : at + 2] = bits.astype("<u2").view(np.uint8).reshape(raw.shape[:-1] + (2,))
    return raw


def _want(raw, qtype, rows, width):
    return bf16_round(dequantize_rows(raw, qtype, width)).reshape(raw.shape[0], rows, width)


def _check(got_bf16, want):
    got = got_bf16.float().cpu().numpy()
    assert np.isfinite(want).all()
    # value equality (+0 == -0) and bit equality once signed zeros are merged
    np.testing.assert_array_equal(got, want)
    gb = np.where(got == 0, np.float32(0), got).view(np.uint32)
    wb = np.where(want == 0, np.float32(0), want).view(np.uint32)
    np.testing.assert_array_equal(gb, wb)


@pytest.mark.parametrize("qtype", ["Q6_K", "Q5_K", "Q4_K", "Q8_0", "Q5_1"])
@pytest.mark.parametrize("path", ["generic", "decode"])
@pytest.mark.parametrize("rows,width", [(16, 256), (40, 512), (33, 768)])
def test_unit_decoders_are_bit_exact(device, qtype, path, rows, width):
    raw = _random_table(qtype, 3, rows, width, seed=rows * 7 + width)
    table = pack_experts(raw.reshape(3, -1), qtype, rows, width, device)
    _check(unpack_experts(table, path), _want(raw, qtype, rows, width))


@pytest.mark.parametrize("qtype", ["Q6_K", "Q8_0", "Q5_1", "Q4_K"])
@pytest.mark.parametrize("rows,width", [(16, 256), (48, 768), (33, 512)])
def test_prefill_unit_decoder_is_bit_exact(device, qtype, rows, width):
    raw = _random_table(qtype, 2, rows, width, seed=rows + width)
    table = pack_experts(raw.reshape(2, -1), qtype, rows, width, device)
    _check(unpack_experts(table, "prefill"), _want(raw, qtype, rows, width))


@pytest.mark.parametrize("qtype", ["Q8_0", "Q5_1"])
def test_prefill_unit_decoder_half_block(device, qtype):
    # a width of 640: the last unit holds one used K half and zero padding
    raw = _random_table(qtype, 2, 40, 640, seed=640)
    table = pack_experts(raw.reshape(2, -1), qtype, 40, 640, device)
    _check(unpack_experts(table, "prefill"), _want(raw, qtype, 40, 640))


@pytest.mark.parametrize("qtype,down", [("Q6_K", "Q6_K"), ("Q4_K", "Q4_K"), ("Q6_K", "Q8_0"), ("Q4_K", "Q5_1"),
                                        ("Q5_K", "Q8_0")])
def test_workload_expert_tables_decode_bit_exact(device, qtype, down):
    # Quantized N(0, 0.02) experts of the headline layer shapes (gate [768, 2048],
    # down [2048, 768]) and the Q4 layer shapes (gate [1024, 4096], down [4096, 1024]).
    H, I = (2048, 768) if qtype == "Q6_K" else (4096, 1024)
    rng = np.random.default_rng(5)
    for rows, width, q in ((I, H, qtype), (H, I, down)):
        raw = np.stack([QUANTIZERS[q](rng.normal(0, 0.02, (rows, width)).astype(np.float32)) for _ in range(2)])
        table = pack_experts(raw.reshape(2, -1), q, rows, width, device)
        want = _want(raw, q, rows, width)
        paths = ("generic", "decode", "prefill") if q == "Q6_K" else ("generic", "decode")
        for path in paths:
            _check(unpack_experts(table, path), want)
