"""Pin the CPU oracle against reference-held vectors, exhaustive enumerations
and closed forms, so that plausible mistakes (a dropped term, a wrong shift, a
transposed index) fail here before the oracle is trusted for GPU parity."""

import numpy as np
import pytest
import torch

from oracle import gguf, kv, moe, numerics, packed_q6, routing

from .conftest import GOLDEN

FROZEN = GOLDEN / "gguf_py_decoder_reference.npz"


@pytest.mark.parametrize("qtype", ["Q4_K", "Q5_K", "Q6_K", "Q8_0", "F16", "BF16", "F32"])
def test_decoder_matches_frozen_gguf_py_vectors(qtype):
    # gguf-py 0.19.0 outputs frozen by the reference (kaggle/REFERENCE_PROVENANCE.json).
    ref = np.load(FROZEN)
    raw, want = ref[f"{qtype}_raw"], ref[f"{qtype}_expected"]
    values, _ = gguf.block_layout(qtype)
    got = gguf.dequantize_rows(raw, qtype, raw.shape[-2] * values)
    assert got.shape == want.shape
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_scalar_q6_oracle_agrees_with_vectorised_decoder_on_all_codes_and_scales():
    raw = packed_q6.fixture(64, 256)
    d = np.array([0, -0.0, 65504, -65504, 2**-24, -(2**-24), 2**-14, 1], dtype="<f2")
    raw[:8, 0, 208:] = d.view(np.uint8).reshape(8, 2)
    raw[..., 192:208] = np.arange(1024, dtype=np.uint16).astype(np.uint8).reshape(64, 1, 16)
    a = packed_q6.decode_reference(raw, 256)
    b = gguf.dequantize_rows(raw, "Q6_K", 256)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
    # every 6-bit code occurs
    ref = np.load(FROZEN)
    a = packed_q6.decode_reference(ref["Q6_K_raw"].reshape(6, 2, 210), 512)
    np.testing.assert_array_equal(a, ref["Q6_K_expected"].reshape(6, 512))


def test_q6_position_map_by_hand():
    # One nonzero code at a time: position p = 200 (h=1, quarter 2, l=8) uses
    # the HIGH nibble of ql[64 + 0*32 + 8] and bits 4-5 of qh[32 + 8].
    raw = np.zeros((1, 1, 210), np.uint8)
    raw[0, 0, 192:208] = 1
    raw[0, 0, 208:210] = np.array([1.0], "<f2").view(np.uint8)
    raw[0, 0, :128] = 0x88  # every code low nibble 8 -> code 8 - 32
    raw[0, 0, 64 + 8] = 0x38  # position 200: low nibble 8 (p=136), high nibble 3
    raw[0, 0, 128 + 32 + 8] = 0b00100000  # quarter 2 high bits = 2
    w = packed_q6.decode_reference(raw, 256)[0]
    assert w[200] == (3 | (2 << 4)) - 32
    assert w[136] == 8 - 32
    assert np.count_nonzero(w != -24) == 1


def test_fp16_expansion_exhaustive():
    bits = np.arange(65536, dtype=np.uint32)
    bits = bits[(bits & 0x7C00) != 0x7C00]
    want = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    got = packed_q6.fp16_bits_to_f32(bits)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_bf16_round_every_bin_below_at_above_halfway():
    high = np.arange(65536, dtype=np.uint32)[:, None] << 16
    low = np.array([0, 0x7FFF, 0x8000, 0x8001], np.uint32)
    src = (high | low).reshape(-1).view(np.float32)
    want = torch.from_numpy(src.copy()).to(torch.bfloat16).float().numpy()
    got = packed_q6.bf16_round(src)
    nan = np.isnan(src)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert np.isnan(got[nan]).all()
    # ties go to even
    assert packed_q6.bf16_round(np.float32(1.00390625)) == np.float32(1.0)
    assert packed_q6.bf16_round(np.float32(1.01171875)) == np.float32(1.015625)


def test_projection_reference_closed_forms():
    raw = packed_q6.fixture(65, 263)
    w = packed_q6.bf16_round(packed_q6.decode_reference(raw, 263))
    eye = np.eye(263, dtype=np.float32)[[0, 100, 262]]
    y = packed_q6.projection_reference(eye, raw)
    np.testing.assert_array_equal(y, w[:, [0, 100, 262]].T)
    x = np.random.default_rng(3).normal(size=(2, 263)).astype(np.float32)
    x = packed_q6.bf16_round(x)
    y1 = packed_q6.projection_reference(x, raw)
    y2 = packed_q6.projection_reference(2 * x, raw)
    np.testing.assert_array_equal(2 * y1, y2)


def test_soa_offsets_are_a_permutation():
    plane, off = packed_q6.soa_offsets(65, 300)
    data_size, scale_size = packed_q6.soa_sizes(65, 300)
    d = off[plane == 0]
    s = off[plane == 1]
    assert len(np.unique(d)) == d.size and d.max() < data_size
    assert len(np.unique(s)) == s.size and s.max() < scale_size


@pytest.mark.parametrize("qtype", ["Q5_1", "IQ4_NL"])
def test_extra_block_types_closed_form(qtype):
    # Scalar enumeration as in the reference test (kaggle/tests/test_qwen38_tpu.py:135-167).
    width = 640 if qtype == "Q5_1" else 160
    size = 24 if qtype == "Q5_1" else 18
    rng = np.random.default_rng(74)
    raw = rng.integers(0, 256, (2, width // 32, size), dtype=np.uint8)
    raw[..., :2] = np.asarray([1.0], "<f2").view(np.uint8)
    if qtype == "Q5_1":
        raw[..., 2:4] = np.asarray([-2.0], "<f2").view(np.uint8)
    expected = []
    for row in raw:
        vals = []
        for blk in row:
            if qtype == "Q5_1":
                high = int.from_bytes(blk[4:8].tobytes(), "little")
                low = blk[8:]
                vals += [((int(low[i % 16]) >> (4 * (i // 16))) & 15) + (((high >> i) & 1) << 4) - 2
                         for i in range(32)]
            else:
                low = blk[2:]
                vals += [int(gguf.IQ4_GRID[(int(low[i % 16]) >> (4 * (i // 16))) & 15]) for i in range(32)]
        expected.append(vals)
    np.testing.assert_array_equal(gguf.dequantize_rows(raw, qtype, width), expected)


@pytest.mark.parametrize("qtype", ["Q4_0", "Q4_1", "Q5_0"])
def test_legacy_block_types_closed_form(qtype):
    # Per-value scalar restatement of the GGML block definitions the reference's
    # decoder follows (kaggle/qwen38_tpu/quant.py:15-55): FP16 d [, FP16 m]
    # [, 32-bit high word], 16 nibble bytes (position i: byte i % 16, nibble
    # i // 16); value d * (q - 8), d * q + m, d * (q - 16). Random FP16 d and m,
    # expected values formed in float64 (exact here) and rounded once.
    size = {"Q4_0": 18, "Q4_1": 20, "Q5_0": 22}[qtype]
    rng = np.random.default_rng(75)
    raw = rng.integers(0, 256, (3, 4, size), dtype=np.uint8)
    d = rng.uniform(-0.5, 0.5, (3, 4)).astype(np.float16)
    m = rng.uniform(-0.5, 0.5, (3, 4)).astype(np.float16)
    raw[..., 0:2] = d.astype("<f2").view(np.uint8).reshape(3, 4, 2)
    if qtype == "Q4_1":
        raw[..., 2:4] = m.astype("<f2").view(np.uint8).reshape(3, 4, 2)
    expected = np.zeros((3, 128), np.float64)
    for r in range(3):
        for b in range(4):
            blk = raw[r, b]
            for i in range(32):
                if qtype == "Q5_0":
                    high = int.from_bytes(blk[2:6].tobytes(), "little")
                    q = ((int(blk[6 + i % 16]) >> (4 * (i // 16))) & 15) | (((high >> i) & 1) << 4)
                    v = float(d[r, b]) * (q - 16)
                elif qtype == "Q4_1":
                    q = (int(blk[4 + i % 16]) >> (4 * (i // 16))) & 15
                    v = float(d[r, b]) * q + float(m[r, b])
                else:
                    q = (int(blk[2 + i % 16]) >> (4 * (i // 16))) & 15
                    v = float(d[r, b]) * (q - 8)
                expected[r, 32 * b + i] = v
    got = gguf.dequantize_rows(raw, qtype, 128 - 7)
    np.testing.assert_array_equal(got, expected[:, : 128 - 7].astype(np.float32))


def test_sigmoid_and_silu_against_fp64():
    x = np.concatenate([np.linspace(-30, 30, 20001), [0.0, -0.0, 1e-30, -1e-30]]).astype(np.float32)
    exact = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    got = numerics.sigmoid(x)
    ulp = np.spacing(np.abs(exact).astype(np.float32))
    assert np.all(np.abs(got - exact) <= 2 * ulp)
    assert numerics.silu_bf16(np.float32(0)) == 0
    s = numerics.silu_bf16(np.float32(1.0))
    assert s == packed_q6.bf16_round(np.float32(1.0 / (1.0 + np.exp(-1.0))))


def test_routing_oracle_brute_force_and_product_router_agree():
    from q6moe.synth import softmax_topk

    rng = np.random.default_rng(11)
    logits = rng.normal(size=(16, 32)).astype(np.float32)
    logits[3, [4, 9]] = 5.0  # tie -> lower id first
    ids, w = routing.route(logits, 4)
    assert ids[3, 0] == 4 and ids[3, 1] == 9
    for b in range(16):
        top = np.argsort(-logits[b], kind="stable")[:4]
        assert list(ids[b]) == list(top)
    np.testing.assert_allclose(w.sum(-1), 1.0, atol=4 * 2**-8)
    pids, pw = softmax_topk(logits, 4)
    np.testing.assert_array_equal(pids, ids)
    np.testing.assert_array_equal(pw, w)


def test_route_weights_sum_duplicates_and_drop_out_of_range():
    ids = np.array([[1, 1, 7], [0, 9, 2]], np.int32)
    w = np.array([[0.25, 0.5, 1.0], [0.125, 1.0, 0.0]], np.float32)
    r = routing.route_weights(ids, w, 8)
    assert r[0, 1] == 0.75 and r[0, 7] == 1.0 and r[1, 0] == 0.125 and r[1, 2] == 0
    assert r.sum() == np.float32(0.75 + 1.0 + 0.125)


def _tiny_moe(seed=5, experts=6, hidden=256, inter=256, tokens=5, top_k=3, qtype="Q6_K"):
    from q6moe.synth import moe_layer

    return moe_layer(seed=seed, experts=experts, top_k=top_k, hidden=hidden, intermediate=inter,
                     tokens=tokens, qtype=qtype, pack=False)


@pytest.mark.parametrize("qtype", ["Q6_K", "Q4_K"])
def test_moe_oracle_two_formulations_agree(qtype):
    L = _tiny_moe(qtype=qtype)
    args = (L["gate"], L["up"], L["down"], L["x"], L["ids"], L["weights"])
    kw = dict(types=(qtype,) * 3, hidden=L["hidden"], intermediate=L["intermediate"])
    a = moe.expert_ffn(*args, **kw)
    b = moe.expert_ffn_per_token(*args, **kw)
    np.testing.assert_array_equal(a, b)
    assert np.isfinite(a).all() and np.any(a != 0)


def test_moe_oracle_zero_routes_give_exact_zero_and_skip_poisoned_experts():
    L = _tiny_moe()
    w = L["weights"].copy()
    w[2] = 0
    gate = L["gate"].copy()
    unused = sorted(set(range(6)) - set(L["ids"][[0, 1, 3, 4]].ravel()))
    for e in unused:  # poison experts nobody routes to (NaN block scales)
        gate[e, ..., 208:210] = np.array([np.nan], "<f2").view(np.uint8)
    out = moe.expert_ffn(gate, L["up"], L["down"], L["x"], L["ids"], w, types=("Q6_K",) * 3,
                         hidden=256, intermediate=256)
    assert np.all(out[2] == 0)
    assert np.isfinite(out).all()


def test_moe_oracle_single_expert_closed_form():
    # One token routed with weight 1 to one expert == that expert's FFN, rounded.
    L = _tiny_moe(tokens=1, top_k=1)
    e = int(L["ids"][0, 0])
    out = moe.expert_ffn(L["gate"], L["up"], L["down"], L["x"], L["ids"], np.ones((1, 1), np.float32),
                         types=("Q6_K",) * 3, hidden=256, intermediate=256)
    x = packed_q6.bf16_round(L["x"])
    gw = packed_q6.bf16_round(packed_q6.decode_reference(L["gate"][e], 256))
    uw = packed_q6.bf16_round(packed_q6.decode_reference(L["up"][e], 256))
    dw = packed_q6.bf16_round(packed_q6.decode_reference(L["down"][e], 256))
    g = packed_q6.bf16_round((x.astype(np.float64) @ gw.T.astype(np.float64)).astype(np.float32))
    u = packed_q6.bf16_round((x.astype(np.float64) @ uw.T.astype(np.float64)).astype(np.float32))
    s = packed_q6.bf16_round(g * (1.0 / (1.0 + np.exp(-g.astype(np.float64)))).astype(np.float32))
    a = packed_q6.bf16_round(s * u)
    y = packed_q6.bf16_round((a.astype(np.float64) @ dw.T.astype(np.float64)).astype(np.float32))
    np.testing.assert_allclose(out, y, rtol=2**-7, atol=1e-6)


def test_kv_quantize_closed_forms_and_rounded_divisor():
    rng = np.random.default_rng(710)
    x = packed_q6.bf16_round(rng.normal(size=(2, 2, 256)).astype(np.float32))
    x[0, 0, :32] = 0
    codes, scale = kv.quantize(x, 32)
    g = x.reshape(2, 2, 8, 32)
    want_scale = packed_q6.bf16_round((np.abs(g).max(-1) / np.float32(127)).astype(np.float32))
    np.testing.assert_array_equal(scale, want_scale)
    div = np.where(want_scale == 0, 1, want_scale)
    np.testing.assert_array_equal(codes.reshape(g.shape), np.clip(np.rint(g / div[..., None]), -127, 127))
    assert np.all(codes.reshape(g.shape)[0, 0, 0] == 0) and scale[0, 0, 0] == 0
    # the rounded divisor differs from the unrounded one somewhere
    full = (np.abs(g).max(-1) / np.float32(127)).astype(np.float32)
    unrounded = np.clip(np.rint(g / np.where(full == 0, 1, full)[..., None]), -127, 127)
    assert np.any(unrounded != codes.reshape(g.shape))


def test_kv_scale_gather_index_rules():
    plane = np.arange(4 * 8, dtype=np.float32).reshape(4, 8)
    idx = np.array([[0, 7, -1, -10, 9], [3, 3, 0, 8, -8]])
    got = kv.gather_scale_plane(plane, idx, 2)
    for b in range(2):
        for s, t in enumerate(idx[b]):
            t = t + 8 if t < 0 else t
            t = min(max(t, 0), 7)
            for g in range(2):
                assert got[b, s, g] == plane[b * 2 + g, t]


def test_kv_paged_read_equals_dense_read_of_the_same_tokens():
    rng = np.random.default_rng(4)
    B, P, pps, H, D = 2, 4, 3, 2, 8
    pool = rng.integers(-127, 128, (B * pps, P, H, D), dtype=np.int8)
    scales = rng.uniform(0, 0.1, (B * pps, P, H)).astype(np.float32)
    table = rng.permutation(B * pps).astype(np.int32).reshape(B, pps)
    got = kv.read_paged(pool, scales, table, P, H, D, D)
    for b in range(B):
        for t in range(pps * P):
            page, slot = table[b, t // P], t % P
            want = packed_q6.bf16_round(pool[page, slot].astype(np.float32) * scales[page, slot][:, None])
            np.testing.assert_array_equal(got[b, t], want)


def test_decode_attention_oracle_closed_forms():
    rng = np.random.default_rng(5)
    b, kvh, r, d, t = 2, 2, 4, 128, 48
    q = packed_q6.bf16_round(rng.standard_normal((b, kvh * r, d)).astype(np.float32))
    v = packed_q6.bf16_round(rng.standard_normal((b, t, kvh, d)).astype(np.float32))
    lengths = np.array([48, 17])
    # equal keys: every attended token has the same score, so prob = RNE(1/n) and
    # out = RNE(RNE(1/n) * sum of the attended values)
    k_eq = np.broadcast_to(v[:, :1], v.shape).copy()
    got = kv.decode_attention(q, k_eq, v, lengths)
    for i, n in enumerate(lengths):
        p = packed_q6.bf16_round(np.float32(1) / np.float32(n))
        want = packed_q6.bf16_round(p * v[i, :n].sum(axis=0, dtype=np.float32))  # [kvh, d]
        np.testing.assert_allclose(got[i].reshape(kvh, r, d), np.repeat(want[:, None], r, axis=1),
                                   rtol=2e-2, atol=2e-2)
    # a dominant key: token 5 of each sequence equals 4x the query of head 0 of
    # its group, so that head attends (almost) only to token 5 and outputs v[5]
    k = packed_q6.bf16_round(0.01 * rng.standard_normal((b, t, kvh, d)).astype(np.float32))
    for i in range(b):
        for g in range(kvh):
            k[i, 5, g] = 4 * q[i, g * r]
    got = kv.decode_attention(q, k, v, lengths)
    for i in range(b):
        for g in range(kvh):
            np.testing.assert_allclose(got[i, g * r], v[i, 5, g], rtol=1e-2, atol=1e-2)
    # against an FP64 softmax attention without the BF16 roundings
    k = packed_q6.bf16_round(rng.standard_normal((b, t, kvh, d)).astype(np.float32))
    got = kv.decode_attention(q, k, v, lengths)
    for i, n in enumerate(lengths):
        for h in range(kvh * r):
            s = (k[i, :n, h // r].astype(np.float64) @ q[i, h].astype(np.float64)) / np.sqrt(d)
            p = np.exp(s - s.max())
            p /= p.sum()
            want = p @ v[i, :n, h // r].astype(np.float64)
            assert np.max(np.abs(got[i, h] - want)) <= 2e-2 * np.abs(want).max() + 1e-3


SOA_GOLDEN = GOLDEN / "packed_q6_soa_reference.npz"
SOA_CASES = ("r65_k300", "r130_k520", "r64_k256_all_scales")


@pytest.mark.parametrize("case", SOA_CASES)
def test_soa_byte_map_matches_reference_packer_output(case):
    # Planes written by the reference's own pack_q6 (kaggle/packed_q6/layout.py:49-90,
    # tests/golden/make_soa_golden.py): the oracle's byte map and the product
    # packer must both reproduce them byte for byte.
    from q6moe import pack_q6

    ref = np.load(SOA_GOLDEN)
    raw, inputs = ref[f"{case}_raw"], int(ref[f"{case}_inputs"])
    data, scales = ref[f"{case}_data"], ref[f"{case}_scales"]
    outputs = raw.shape[0]
    assert int(ref[f"{case}_outputs"]) == outputs
    plane, off = packed_q6.soa_offsets(outputs, inputs)
    assert (data.size, scales.size) == packed_q6.soa_sizes(outputs, inputs)
    np.testing.assert_array_equal(data[off[plane == 0]], raw[plane == 0])
    np.testing.assert_array_equal(scales[off[plane == 1]], raw[plane == 1])
    packed = pack_q6(raw, inputs)
    np.testing.assert_array_equal(packed.data, data)
    np.testing.assert_array_equal(packed.scales, scales)
    np.testing.assert_array_equal(
        packed_q6.decode_soa(data, scales, outputs, inputs).view(np.uint32),
        packed_q6.decode_reference(raw, inputs).view(np.uint32),
    )


def test_shared_gate_oracle_closed_forms():
    # math.py:283: RNE(sigmoid(RNE(x . router))). One-hot routers pick a column
    # of x; sigmoid(0) = 0.5 exactly; large logits saturate. A dot of
    # 1 + 17 * 2^-12 is not a BF16 value: it must round to 1 + 2^-7 before
    # the sigmoid, which changes the gate by one BF16 step.
    x = np.zeros((4, 8), np.float32)
    x[1, 3] = 64.0
    x[2, 3] = -64.0
    x[3, :2] = (1.0, 17 * 2.0**-12)
    router = np.zeros(8, np.float32)
    router[3] = 1.0
    g = moe.shared_gate(x, router)
    assert g[0] == 0.5 and g[1] == 1.0 and g[2] == packed_q6.bf16_round(np.float32(np.exp(-64.0)))
    r2 = np.zeros(8, np.float32)
    r2[:2] = 1.0
    want = packed_q6.bf16_round(np.float32(1.0 / (1.0 + np.exp(-(1.0 + 2.0**-7)))))
    assert moe.shared_gate(x[3:], r2)[0] == want
    unrounded = packed_q6.bf16_round(np.float32(1.0 / (1.0 + np.exp(-(1.0 + 17 * 2.0**-12)))))
    assert want != unrounded


def test_q8_matmul_oracle_closed_form():
    # Activation groups whose max is 127 * 2^e quantise without rounding
    # (codes = x / 2^e), and power-of-two weight scales keep every product and
    # sum exact: the W8A8 dot then equals x . dequant(W) in FP64 exactly. A
    # transposed operand, a wrong group index or a missing scale fails it.
    from oracle import compute
    from q6moe.quantize import quantize_q8_0

    rng = np.random.default_rng(837)
    codes = rng.integers(-127, 128, (5, 4, 32)).astype(np.float32)
    codes[:, :, 0] = 127
    e = rng.integers(-4, 3, (5, 4)).astype(np.float32)
    x = (codes * np.exp2(e)[..., None]).reshape(5, 128)
    x[3] = 0
    wcodes = rng.integers(-127, 128, (7, 4, 32)).astype(np.float32)
    ws = np.exp2(rng.integers(-9, -3, (7, 4))).astype(np.float32)
    raw = np.concatenate([ws.astype("<f2").view(np.uint8).reshape(7, 4, 2),
                          wcodes.astype(np.int8).view(np.uint8)], axis=-1)
    w = (wcodes * ws[..., None]).reshape(7, 128)
    got = compute.q8_matmul(x, raw)
    np.testing.assert_array_equal(got, (x.astype(np.float64) @ w.T.astype(np.float64)).astype(np.float32))
    assert np.all(got[3] == 0)
    # and it matches the pack_q8 quantizer's bytes decoded (compute.py:41-65)
    wf = rng.normal(size=(3, 64)).astype(np.float32)
    raw = quantize_q8_0(wf)
    assert raw.shape == (3, 2, 34)
    xf = rng.normal(size=(2, 64)).astype(np.float32)
    ref = compute.q8_matmul(xf, raw)
    dq = gguf.dequantize_rows(raw, "Q8_0", 64)
    assert np.max(np.abs(ref - xf @ dq.T)) < 0.05 * np.abs(xf @ dq.T).max()
