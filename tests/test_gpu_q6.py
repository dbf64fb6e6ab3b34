"""GPU parity for the Q6_K decode and the decode-fused projection (q6_matmul).

Decode must be bit-exact against the oracle; the projection must meet the
reference's own tolerance against its FP64 oracle (rtol 2e-5, atol 2e-4,
kaggle/tests/test_packed_q6.py:51-81) and, with BF16 output, a max relative
error of 1e-2."""

import numpy as np
import pytest
import torch

from oracle import gguf, packed_q6
from q6moe import pack_q6
from q6moe.kernel import q6_decode, q6_matmul, q6_pack
from q6moe.quant import dequantize_rows

pytestmark = pytest.mark.gpu


def _to_dev(packed, device):
    return (torch.from_numpy(packed.data).to(device), torch.from_numpy(packed.scales).to(device))


def _bf16_bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def test_decode_bit_exact_all_codes_subscales_and_fp16_extremes(device):
    raw = packed_q6.fixture(64, 256)
    d = np.array([0, -0.0, 65504, -65504, 2**-24, -(2**-24), 2**-14, 1], dtype="<f2")
    raw[:8, 0, 208:] = d.view(np.uint8).reshape(8, 2)
    raw[..., 192:208] = np.arange(1024, dtype=np.uint16).astype(np.uint8).reshape(64, 1, 16)
    data, scales = _to_dev(pack_q6(raw, 256), device)
    got = _bf16_bits(q6_decode(data, scales, output_features=64, input_features=256))
    want = packed_q6.bf16_bits(packed_q6.decode_reference(raw, 256))
    np.testing.assert_array_equal(got, want)


def test_decode_every_finite_fp16_block_scale(device):
    bits = np.arange(65536, dtype=np.uint32)
    bits = bits[(bits & 0x7C00) != 0x7C00].astype(np.uint16)
    n = bits.size  # 63488 rows, one block each
    raw = packed_q6.fixture(n, 256, seed=17)
    raw[:, 0, 192:208] = 1  # sub-scale 1: value = d * code
    raw[:, 0, 208:210] = bits.view(np.uint8).reshape(n, 2)
    data, scales = _to_dev(pack_q6(raw, 256), device)
    got = _bf16_bits(q6_decode(data, scales, output_features=n, input_features=256))
    want = packed_q6.bf16_bits(packed_q6.decode_reference(raw, 256))
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("outputs,inputs", [(64, 256), (65, 600)])
def test_matmul_operands_equal_decoded_weights(device, outputs, inputs):
    # x = identity rows: y[i, n] = W[n, i] exactly (one nonzero product per
    # sum), so the MFMA operands are pinned value-for-value (+0 == -0).
    raw = packed_q6.fixture(outputs, inputs, seed=21)
    data, scales = _to_dev(pack_q6(raw, inputs), device)
    w = packed_q6.bf16_round(packed_q6.decode_reference(raw, inputs))
    for start in range(0, inputs, 128):
        rows = np.arange(start, min(inputs, start + 128))
        x = np.zeros((rows.size, inputs), np.float32)
        x[np.arange(rows.size), rows] = 1
        y = q6_matmul(torch.from_numpy(x).to(device).to(torch.bfloat16), data, scales,
                      output_features=outputs).cpu().numpy()
        np.testing.assert_array_equal(y, w[:, rows].T)


@pytest.mark.parametrize("outputs,inputs", [(1, 1), (65, 263), (320, 2560), (768, 2048)])
def test_decode_ragged_shapes_bit_exact(device, outputs, inputs):
    raw = packed_q6.fixture(outputs, inputs, seed=outputs + inputs)
    data, scales = _to_dev(pack_q6(raw, inputs), device)
    got = _bf16_bits(q6_decode(data, scales, output_features=outputs, input_features=inputs))
    np.testing.assert_array_equal(got, packed_q6.bf16_bits(packed_q6.decode_reference(raw, inputs)))


@pytest.mark.parametrize(
    "batch,outputs,inputs",
    [(1, 1, 1), (2, 67, 255), (4, 128, 257), (8, 64, 512), (9, 65, 263), (1, 320, 2560),
     (8, 640, 2560), (8, 768, 2048), (16, 64, 256), (17, 130, 600), (70, 96, 512)],
)
def test_projection_matches_fp64_oracle(device, batch, outputs, inputs):
    raw = packed_q6.fixture(outputs, inputs)
    x = np.random.default_rng(721).normal(size=(batch, inputs)).astype(np.float32)
    if batch > 1:
        x[0] = 0
    data, scales = _to_dev(pack_q6(raw, inputs), device)
    xt = torch.from_numpy(x).to(device).to(torch.bfloat16)
    got = q6_matmul(xt, data, scales, output_features=outputs).cpu().numpy()
    want = packed_q6.projection_reference(x, raw)
    assert got.dtype == np.float32 and got.shape == (batch, outputs)
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-4)
    if batch > 1:
        assert np.all(got[0] == 0)


def test_projection_unaligned_x_view(device):
    raw = packed_q6.fixture(64, 300)
    x = np.random.default_rng(5).normal(size=(3, 301)).astype(np.float32)
    data, scales = _to_dev(pack_q6(raw, 300), device)
    xt = torch.from_numpy(x).to(device).to(torch.bfloat16)[:, 1:]  # ldx 301, offset 1 element
    got = q6_matmul(xt, data, scales, output_features=64).cpu().numpy()
    np.testing.assert_allclose(got, packed_q6.projection_reference(x[:, 1:], raw), rtol=2e-5, atol=2e-4)


def test_accumulator_reset_between_row_and_token_tiles(device):
    raw = packed_q6.fixture(128, 512)
    raw[64:] = raw[:64]
    data, scales = _to_dev(pack_q6(raw, 512), device)
    x = np.ones((40, 512), np.float32)
    x[20:] = -1
    got = q6_matmul(torch.from_numpy(x).to(device).to(torch.bfloat16), data, scales,
                    output_features=128).cpu().numpy()
    np.testing.assert_array_equal(got[:, :64], got[:, 64:])
    np.testing.assert_array_equal(got[:20], -got[20:])
    np.testing.assert_array_equal(got[:20], np.broadcast_to(got[0], (20, 128)))


def test_single_projection_workload_bf16_output(device):
    # x bf16 [8, 2048] ~ N(0,1), W [2048 -> 768] ~ N(0, 0.02) quantized to Q6_K, seed 0.
    from q6moe.synth import projection

    w = projection(seed=0)
    data, scales = _to_dev(pack_q6(w["raw"], 2048), device)
    xt = torch.from_numpy(w["x"]).to(device).to(torch.bfloat16)
    got = q6_matmul(xt, data, scales, output_features=768, out_dtype=torch.bfloat16).float().cpu().numpy()
    want32 = packed_q6.projection_reference(w["x"], w["raw"])
    want = packed_q6.bf16_round(want32)
    rel = np.abs(got - want) / np.maximum(np.abs(want), 1e-3 * np.abs(want).max())
    assert rel.max() <= 1e-2
    # bit agreement with RNE of the FP32 result of the same kernel
    f32 = q6_matmul(xt, data, scales, output_features=768)
    np.testing.assert_array_equal(_bf16_bits(f32.to(torch.bfloat16)),
                                  _bf16_bits(torch.from_numpy(got).to(torch.bfloat16)))


def test_repeat_runs_are_bitwise_identical(device):
    raw = packed_q6.fixture(256, 1024)
    data, scales = _to_dev(pack_q6(raw, 1024), device)
    x = torch.randn(8, 1024, generator=torch.Generator().manual_seed(1)).to(device).to(torch.bfloat16)
    a = q6_matmul(x, data, scales, output_features=256)
    b = q6_matmul(x, data, scales, output_features=256)
    assert torch.equal(a, b)


@pytest.mark.parametrize("outputs,inputs", [(1, 1), (65, 263), (768, 2048)])
def test_device_pack_matches_host_pack(device, outputs, inputs):
    raw = packed_q6.fixture(outputs, inputs, seed=3)
    host = pack_q6(raw, inputs)
    data, scales = q6_pack(torch.from_numpy(raw).to(device), inputs)
    np.testing.assert_array_equal(data.cpu().numpy(), host.data)
    np.testing.assert_array_equal(scales.cpu().numpy(), host.scales)


ALL_GGUF_TYPES = ["Q6_K", "Q5_K", "Q4_K", "Q8_0", "Q5_1", "Q5_0", "Q4_1", "Q4_0", "IQ4_NL", "F16", "BF16", "F32"]
_SCALE_AT = {"Q6_K": (208,), "Q5_K": (0, 2), "Q4_K": (0, 2), "Q8_0": (0,), "Q5_1": (0, 2), "Q5_0": (0,),
             "Q4_1": (0, 2), "Q4_0": (0,), "IQ4_NL": (0,)}


def _random_rows(qtype, rows, nb, rng):
    """Random GGUF rows of ``nb`` blocks with finite FP16 scales; for the
    unquantized types finite values incl. signed zeros, subnormals and +-inf."""
    values, size = gguf.block_layout(qtype)
    if qtype in _SCALE_AT:
        raw = rng.integers(0, 256, (rows, nb, size), dtype=np.uint8)
        for off in _SCALE_AT[qtype]:
            raw[..., off : off + 2] = rng.uniform(-0.3, 0.3, (rows, nb)).astype("<f2").view(np.uint8).reshape(
                rows, nb, 2)
        return raw
    special = np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -3e-39, 6e-8, 65504.0], np.float32)
    v = rng.normal(0, 100, (rows, nb)).astype(np.float32)
    v.reshape(-1)[:: 7] = special[rng.integers(0, special.size, v.reshape(-1)[:: 7].size)]
    if qtype == "F32":
        return v.astype("<f4").view(np.uint8).reshape(rows, nb, 4)
    if qtype == "F16":
        return v.astype("<f2").view(np.uint8).reshape(rows, nb, 2)
    return (v.view(np.uint32) >> 16).astype("<u2").view(np.uint8).reshape(rows, nb, 2)  # BF16 (truncated)


@pytest.mark.parametrize("qtype", ALL_GGUF_TYPES)
def test_dequantize_rows_hip_matches_oracle_and_frozen_vectors(device, qtype):
    from .conftest import GOLDEN

    values, size = gguf.block_layout(qtype)
    ref = np.load(GOLDEN / "gguf_py_decoder_reference.npz")
    if f"{qtype}_raw" in ref.files:  # gguf-py 0.19.0 vectors (Q6_K, Q5_K, Q4_K, Q8_0, F16, BF16, F32)
        raw = ref[f"{qtype}_raw"]
        width = raw.shape[-2] * values
        got = dequantize_rows(torch.from_numpy(raw).to(device), qtype, width).cpu().numpy()
        np.testing.assert_array_equal(got.view(np.uint32), ref[f"{qtype}_expected"].view(np.uint32))
    rng = np.random.default_rng(8)
    nb = 3 if values > 1 else 301
    raw = _random_rows(qtype, 37, nb, rng)
    width = nb * values - (5 if values > 1 else 0)
    want = gguf.dequantize_rows(raw, qtype, width)
    got = dequantize_rows(torch.from_numpy(raw).to(device), qtype, width).cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    gotb = dequantize_rows(torch.from_numpy(raw).to(device), qtype, width, dtype=torch.bfloat16)
    np.testing.assert_array_equal(_bf16_bits(gotb), packed_q6.bf16_bits(want))


@pytest.mark.parametrize("case", ["r65_k300", "r130_k520", "r64_k256_all_scales"])
def test_reference_packer_planes_decode_and_repack_on_device(device, case):
    # Planes from the reference's own pack_q6 (tests/golden/packed_q6_soa_reference.npz):
    # the device repack reproduces them byte for byte, and the kernels read them
    # as the reference's layout (decode bit-exact, projection within rtol 2e-5).
    from .conftest import GOLDEN

    ref = np.load(GOLDEN / "packed_q6_soa_reference.npz")
    raw, inputs = ref[f"{case}_raw"], int(ref[f"{case}_inputs"])
    data, scales = ref[f"{case}_data"], ref[f"{case}_scales"]
    outputs = raw.shape[0]
    d_data, d_scales = q6_pack(torch.from_numpy(raw).to(device), inputs)
    np.testing.assert_array_equal(d_data.cpu().numpy(), data)
    np.testing.assert_array_equal(d_scales.cpu().numpy(), scales)
    tdata, tscales = torch.from_numpy(data).to(device), torch.from_numpy(scales).to(device)
    got = q6_decode(tdata, tscales, output_features=outputs, input_features=inputs)
    want = packed_q6.bf16_round(packed_q6.decode_reference(raw, inputs))
    np.testing.assert_array_equal(got.float().cpu().numpy(), want)
    x = np.random.default_rng(3).normal(size=(9, inputs)).astype(np.float32)
    xb = torch.from_numpy(x).to(device).to(torch.bfloat16)
    y = q6_matmul(xb, tdata, tscales, output_features=outputs).cpu().numpy()
    ref_y = packed_q6.projection_reference(xb.float().cpu().numpy(), raw)
    np.testing.assert_allclose(y, ref_y, rtol=2e-5, atol=2e-4)


@pytest.mark.parametrize("qtype", ALL_GGUF_TYPES)
def test_dequantize_rows_hip_staged_and_fallback_paths(device, qtype):
    # 4-byte aligned rows take the LDS-staged vector path, an offset view the
    # byte path; both are bit-exact, with whole and ragged widths and many
    # workgroups (more blocks than one workgroup stages).
    values, size = gguf.block_layout(qtype)
    rng = np.random.default_rng(19)
    rows, nb = 70, (5 if values > 1 else 333)
    raw = _random_rows(qtype, rows, nb, rng)
    for width in ((nb * values, nb * values - 3) if values > 1 else (nb,)):
        want = gguf.dequantize_rows(raw, qtype, width)
        dev = torch.from_numpy(raw).to(device)
        got = dequantize_rows(dev, qtype, width).cpu().numpy()
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
        buf = torch.empty(raw.size + 1, dtype=torch.uint8, device=device)
        buf[1:] = dev.reshape(-1)
        shifted = buf[1:].view(rows, nb, size)  # 1-byte offset: the byte path
        got = dequantize_rows(shifted, qtype, width, dtype=torch.bfloat16)
        np.testing.assert_array_equal(_bf16_bits(got), packed_q6.bf16_bits(want))
