"""Host-side checks (no GPU): packer, quantizers, argument validation and the
C-ABI library's exported symbols."""

import ctypes
import re

import numpy as np
import pytest

from oracle import gguf, packed_q6
from q6moe import _lib, layout, pack_q6, unpack_q6
from q6moe.quantize import quantize_q4_k, quantize_q5_1, quantize_q5_k, quantize_q6_k, quantize_q8_0

from .conftest import ROOT


@pytest.mark.parametrize("outputs,inputs", [(1, 1), (65, 257), (320, 2560), (640, 2560), (768, 2048)])
def test_lossless_repack_round_trip_and_padding(outputs, inputs):
    raw = packed_q6.fixture(outputs, inputs)
    packed = pack_q6(raw, inputs)
    np.testing.assert_array_equal(unpack_q6(packed), raw)
    assert packed.data.flags.c_contiguous and packed.data.ndim == 1
    assert packed.storage()["original_bytes"] == raw.nbytes
    assert packed.storage()["layout"] == "q6_k_soa_n64_k256_v1"
    if outputs in (320, 640):
        assert packed.storage()["padding_bytes"] <= 384
        assert packed.storage()["padding_ratio"] < 0.0004


@pytest.mark.parametrize("outputs,inputs", [(1, 1), (65, 300), (128, 512)])
def test_packer_matches_oracle_byte_map(outputs, inputs):
    raw = packed_q6.fixture(outputs, inputs, seed=9)
    packed = pack_q6(raw, inputs)
    plane, off = packed_q6.soa_offsets(outputs, inputs)
    data_size, scale_size = packed_q6.soa_sizes(outputs, inputs)
    assert packed.data.size == data_size and packed.scales.size == scale_size
    np.testing.assert_array_equal(packed.data[off[plane == 0]], raw[plane == 0])
    np.testing.assert_array_equal(packed.scales[off[plane == 1]], raw[plane == 1])
    # everything not addressed by a GGUF byte is zero padding
    mask = np.ones(data_size, bool)
    mask[off[plane == 0]] = False
    assert not packed.data[mask].any()
    smask = np.ones(scale_size, bool)
    smask[off[plane == 1]] = False
    assert not packed.scales[smask].any()
    np.testing.assert_array_equal(
        packed_q6.decode_soa(packed.data, packed.scales, outputs, inputs),
        packed_q6.decode_reference(raw, inputs),
    )


@pytest.mark.parametrize("scale", [np.inf, -np.inf, np.nan])
def test_invalid_block_scale_rejected(scale):
    raw = packed_q6.fixture(1, 256)
    raw[0, 0, 208:] = np.array([scale], dtype="<f2").view(np.uint8)
    with pytest.raises(ValueError, match="finite"):
        pack_q6(raw, 256)


def test_invalid_layout_rejected():
    with pytest.raises(TypeError, match="uint8"):
        pack_q6(np.zeros((64, 1, 210)), 256)
    with pytest.raises(ValueError, match="Expected"):
        pack_q6(np.zeros((64, 1, 211), np.uint8), 256)
    with pytest.raises(ValueError, match="positive integer"):
        pack_q6(np.zeros((64, 1, 210), np.uint8), 0)


def test_q6_matmul_contract_rejected_before_any_device_work():
    torch = pytest.importorskip("torch")
    from q6moe.kernel import q6_matmul

    raw = torch.zeros((layout.TILE_BYTES,), dtype=torch.uint8)
    scales = torch.zeros((layout.SCALE_FETCH_BYTES,), dtype=torch.uint8)
    with pytest.raises(ValueError, match="BF16"):
        q6_matmul(torch.ones((1, 256)), raw, scales, output_features=64)
    with pytest.raises(ValueError, match="multiple of 8"):
        q6_matmul(torch.ones((1, 256), dtype=torch.bfloat16), raw, scales, output_features=64, batch_tile=1)
    with pytest.raises(ValueError, match="dtype/shape"):
        q6_matmul(torch.ones((1, 257), dtype=torch.bfloat16), raw, scales, output_features=64)
    with pytest.raises(ValueError, match="GPU"):
        q6_matmul(torch.ones((1, 256), dtype=torch.bfloat16), raw, scales, output_features=64)


@pytest.mark.parametrize(
    "qtype,fn,bound",
    [("Q6_K", quantize_q6_k, 0.03), ("Q5_K", quantize_q5_k, 0.06), ("Q4_K", quantize_q4_k, 0.12),
     ("Q8_0", quantize_q8_0, 0.01), ("Q5_1", quantize_q5_1, 0.06)],
)
def test_quantizers_round_trip_within_format_error(qtype, fn, bound):
    rng = np.random.default_rng(1)
    w = rng.normal(0, 0.02, (64, 512)).astype(np.float32)
    w[0, :256] = 0  # all-zero blocks must stay finite and decode to zero
    raw = fn(w)
    values, size = gguf.block_layout(qtype)
    assert raw.shape == (64, 512 // values, size)
    dec = gguf.dequantize_rows(raw, qtype, 512)
    assert np.isfinite(dec).all()
    assert np.all(dec[0, :256] == 0)
    rel = np.sqrt(((dec - w) ** 2).mean()) / np.sqrt((w**2).mean())
    assert rel < bound


def test_q8_quantizer_matches_reference_closed_form():
    # pack_q8 (kaggle/qwen38_tpu/compute.py:41-49) restated as a scalar loop.
    rng = np.random.default_rng(2)
    w = rng.normal(size=(3, 64)).astype(np.float32)
    raw = quantize_q8_0(w)
    for r in range(3):
        for b in range(2):
            g = w[r, 32 * b : 32 * b + 32]
            s = np.float16(np.max(np.abs(g)) / np.float32(127))
            codes = np.clip(np.rint(g / np.float32(s)), -127, 127).astype(np.int8)
            assert raw[r, b, :2].view("<f2")[0] == s
            np.testing.assert_array_equal(raw[r, b, 2:].view(np.int8), codes)


def _header_symbols():
    text = (ROOT / "include" / "q6moe.h").read_text()
    return sorted(set(re.findall(r"\b(q6moe_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _header_symbols()
    assert set(declared) == set(_lib.SIGNATURES), "ctypes table must mirror the header"
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.q6moe_version() >= 100


def test_library_rejects_bad_arguments_without_a_device():
    lib = _lib.load()
    rc = lib.q6moe_q6_matmul(None, 1, 256, 256, None, None, 64, None, 0, 64, None)
    assert rc == -1
    assert b"null" in lib.q6moe_last_error()
    rc = lib.q6moe_gguf_decode(ctypes.c_void_p(16), 99, 1, 32, ctypes.c_void_p(16), 0, None)
    assert rc == -3
    rc = lib.q6moe_sigmoid_probe(None, 4, ctypes.c_void_p(16), ctypes.c_void_p(16), None)
    assert rc == -1 and b"null" in lib.q6moe_last_error()
    rc = lib.q6moe_sigmoid_probe(ctypes.c_void_p(16), 0, ctypes.c_void_p(16), ctypes.c_void_p(16), None)
    assert rc == -1 and b"n must be" in lib.q6moe_last_error()


def test_decode_mode_rejects_token_rows_past_32_bit_offsets_without_a_device():
    # 1024 routes x hidden 2^20 BF16 values = 2^31 bytes: the decode-step
    # kernels address token rows with 32-bit byte offsets, so mode 1 refuses
    # the call (mode 0 takes the grouped kernels instead). The checks run
    # before any device work; the pointers are never dereferenced.
    lib = _lib.load()
    fake = ctypes.c_void_p(1 << 20)
    tab = _lib.Table(14, fake, 1 << 40, None, 0)
    args = _lib.MoeArgs(gate=tab, up=tab, down=tab, experts=8, hidden=1 << 20, intermediate=256,
                        x=fake, ids=fake, weights=fake, tokens=256, top_k=4, out=fake, workspace=fake,
                        workspace_bytes=0, mode=1)
    assert lib.q6moe_moe_forward(ctypes.byref(args), None) == -1
    assert b"decode mode" in lib.q6moe_last_error()
    args.hidden = (1 << 20) - 256  # just under the bound: decode mode passes validation (then the workspace check)
    assert lib.q6moe_moe_forward(ctypes.byref(args), None) == -1
    assert b"decode mode" not in lib.q6moe_last_error()


def test_expert_ffn_mode_copies_leave_the_cached_callable_alone():
    from q6moe.experts import expert_parallel

    fn = expert_parallel(None, gate_type="Q6_K", up_type="Q6_K", down_type="Q6_K", hidden=512, intermediate=256)
    assert fn is expert_parallel(None, gate_type="Q6_K", up_type="Q6_K", down_type="Q6_K", hidden=512,
                                 intermediate=256)
    pre = fn.with_mode(2)
    assert (fn.mode, pre.mode) == (0, 2) and pre is not fn
    assert (pre.qtype, pre.down_qtype, pre.hidden, pre.intermediate, pre.compute) == ("Q6_K", "Q6_K", 512, 256, "bf16")
    with pytest.raises(AttributeError):
        fn.mode = 1
    with pytest.raises(ValueError):
        fn.with_mode(3)
