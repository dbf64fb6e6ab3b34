"""GPU parity at the benchmarked workload shapes, and the reference's own
routed-FFN gate restated.

* Q4_K layer with a shared expert: 64 experts, top-6, hidden 4096,
  intermediate 1024, shared intermediate 4096, N(0, 0.015), seed 3, at 1, 8
  and 64 tokens (the bench's layer: generated once at 64 tokens, the first B
  rows used), against the oracle.
* Paged INT8 KV gather at its full shape: 8 sequences x 32 768 tokens in
  256-token pages, 4 KV heads of 128, FP32 scales, seed 4; two whole
  sequences and a token sample of every sequence bit-exact.
* kaggle/qwen38_tpu/routing_validation.py:15-113 on one device: Q6_K gate/up
  with sub-scales 1..8 and d = 1/2048, Q8_0 down from ``pack_q8``, 5 experts,
  hidden 256, intermediate 32, 273 tokens with a hot expert over three
  128-row tiles, duplicate routes and finished rows; the reference's own
  expected values (per-expert NumPy loop, FP32 matmuls) and its tolerance
  atol = rtol = 3e-3, zero rows exactly zero.

MoE tolerance elsewhere: max relative error 1e-2 and >= 90 % of
outputs bit-identical (see test_gpu_moe.py), plus the reference's
atol = rtol = 3e-3 where it holds.
"""

import numpy as np
import pytest
import torch

from oracle import kv as oracle_kv
from oracle import moe as oracle_moe
from oracle.gguf import dequantize_rows
from oracle.packed_q6 import bf16_bits, bf16_round
from q6moe.experts import expert_parallel, pack_experts

from .test_gpu_moe import assert_moe_close

pytestmark = pytest.mark.gpu

H4, I4, E4, K4, IS4 = 4096, 1024, 64, 6, 4096


@pytest.fixture(scope="module")
def q4_layer():
    from q6moe.synth import moe_layer

    print("generating the Q4_K + shared layer (seed 3) ...", flush=True)
    L = moe_layer(seed=3, experts=E4, top_k=K4, hidden=H4, intermediate=I4, tokens=64, sigma=0.015,
                  qtype="Q4_K", shared_intermediate=IS4, pack=False)
    sh = L["shared"]
    L["shared_dec"] = dict(gate=bf16_round(dequantize_rows(sh["gate"], "Q4_K", H4)),
                           up=bf16_round(dequantize_rows(sh["up"], "Q4_K", H4)),
                           down=bf16_round(dequantize_rows(sh["down"], "Q4_K", IS4)))
    return L


def _q4_run(L, device, b, router=None):
    fn = expert_parallel(None, gate_type="Q4_K", up_type="Q4_K", down_type="Q4_K", hidden=H4, intermediate=I4)
    tabs = fn.prepare(L["gate"].reshape(E4, -1), L["up"].reshape(E4, -1), L["down"].reshape(E4, -1), device)
    sh = L["shared"]
    shared = dict(gate=pack_experts(sh["gate"][None], "Q4_K", IS4, H4, device),
                  up=pack_experts(sh["up"][None], "Q4_K", IS4, H4, device),
                  down=pack_experts(sh["down"][None], "Q4_K", H4, IS4, device))
    if router is not None:
        shared["router"] = torch.from_numpy(router).to(device).to(torch.bfloat16)
    x = torch.from_numpy(L["x"][:b]).to(device).to(torch.bfloat16)
    ids = torch.from_numpy(L["ids"][:b]).to(device)
    w = torch.from_numpy(L["weights"][:b]).to(device).to(torch.bfloat16)
    return fn(*tabs, x, ids, w, shared=shared).float().cpu().numpy()


@pytest.mark.parametrize("tokens", [1, 8, 64])
def test_q4k_shared_layer_full_shape(device, q4_layer, tokens):
    L = q4_layer
    got = _q4_run(L, device, tokens)
    want = oracle_moe.expert_ffn(L["gate"], L["up"], L["down"], L["x"][:tokens], L["ids"][:tokens],
                                 L["weights"][:tokens], types=("Q4_K",) * 3, hidden=H4, intermediate=I4,
                                 shared=L["shared_dec"])
    # The reference's atol = rtol = 3e-3 is its gate for a 256-wide layer; at
    # this shape (4096-wide expert and shared sums, outputs near 1) a differing
    # FP32 summation order flips an intermediate BF16 rounding now and then,
    # which moves an output by a few BF16 steps (2^-7 each near 1). So:
    # the MoE gate, and >= 99.9 % of outputs within the reference's 3e-3.
    assert_moe_close(got, want, ref_gate=False)
    within = np.abs(got - want) <= 3e-3 + 3e-3 * np.abs(want)
    assert within.mean() >= 0.999


def test_q4k_shared_layer_with_device_router_gate(device, q4_layer):
    # The shared output scaled by RNE(sigmoid(RNE(x . router))) computed on the
    # GPU (math.py:283), router BF16 N(0, 0.02) [4096].
    L = q4_layer
    router = bf16_round(np.random.default_rng(33).normal(0, 0.02, H4).astype(np.float32))
    got = _q4_run(L, device, 8, router=router)
    sh = dict(L["shared_dec"], gate_scale=oracle_moe.shared_gate(L["x"][:8], router))
    want = oracle_moe.expert_ffn(L["gate"], L["up"], L["down"], L["x"][:8], L["ids"][:8], L["weights"][:8],
                                 types=("Q4_K",) * 3, hidden=H4, intermediate=I4, shared=sh)
    assert_moe_close(got, want, ref_gate=False)
    assert (np.abs(got - want) <= 3e-3 + 3e-3 * np.abs(want)).mean() >= 0.999


def test_kv_gather_full_shape(device):
    from q6moe.attention_cache import read_paged
    from q6moe.synth import kv_pages

    print("generating the paged KV workload (seed 4) ...", flush=True)
    W = kv_pages(seed=4)
    B, T = W["batch"], W["context"]
    stride = np.arange(0, T, 61)
    for name in ("k", "v"):
        pool = torch.from_numpy(W[name]).to(device)
        scales = torch.from_numpy(W[name + "_scale"]).to(device)
        table = torch.from_numpy(W["page_table"]).to(device)
        got = read_paged(pool, scales, table, page_size=256, kv_heads=4, head_dim=128)
        assert tuple(got.shape) == (B, T, 4, 128)
        bits = got.view(torch.int16).cpu().numpy().view(np.uint16)
        del got
        for b in (0, 5):
            want = oracle_kv.read_paged(W[name], W[name + "_scale"], W["page_table"][b : b + 1], 256, 4, 128, 128)
            np.testing.assert_array_equal(bits[b : b + 1], bf16_bits(want))
        idx = np.broadcast_to(stride, (B, stride.size)).astype(np.int32)
        want = oracle_kv.read_paged(W[name], W[name + "_scale"], W["page_table"], 256, 4, 128, 128, idx)
        np.testing.assert_array_equal(bits[:, stride], bf16_bits(want))


def _pack_q8(weights):
    """pack_q8 (kaggle/qwen38_tpu/compute.py:41-49): scale fp16(max|x| / 127),
    codes clip(rint(x / scale), -127, 127), [rows, K/32, 34]."""
    rows = np.asarray(weights, np.float32).reshape(weights.shape[0], -1, 32)
    scale = (np.max(np.abs(rows), -1) / 127).astype("<f2")
    codes = np.clip(np.rint(rows / np.where(scale == 0, 1, scale)[..., None]), -127, 127).astype(np.int8)
    return np.concatenate((scale.view(np.uint8).reshape(*scale.shape, 2), codes.view(np.uint8)), axis=-1)


def _routing_validation_case(batch):
    """The inputs of routing_validation.py:21-44 for one device (5 experts)."""
    rng = np.random.default_rng(738)
    hidden, inter, count = 256, 32, 5
    packed = {}
    for name in ("gate", "up"):
        raw = rng.integers(0, 256, (count, inter, 1, 210), dtype=np.uint8)
        raw[..., 192:208] = rng.integers(1, 9, raw[..., 192:208].shape, dtype=np.uint8)
        raw[..., 208:210] = np.array([1 / 2048], "<f2").view(np.uint8)
        packed[name] = raw
    packed["down"] = _pack_q8(rng.normal(0, 0.08, (count * hidden, inter)).astype(np.float32)).reshape(
        count, hidden, inter // 32, 34)
    ids = np.stack((np.zeros(batch, np.int32), 1 + np.arange(batch) % (count - 1)), -1).astype(np.int32)
    ids[:8, 1] = 0
    weights = np.full(ids.shape, 0.5, np.float32)
    if batch > 1:
        weights[::37] = 0
    source = rng.normal(0, 0.3, (batch, hidden)).astype(np.float32)
    return packed, ids, weights, source, hidden, inter, count


def _routing_validation_expected(packed, ids, weights, x, hidden, inter, count):
    """The reference gate's own expected values (routing_validation.py:52-71, BF16
    policy): per expert, FP32 matmuls of BF16 operands rounded to BF16, plain
    NumPy sigmoid, FP32 sum of route-weighted outputs, BF16 result."""
    x = bf16_round(x)
    routing = bf16_round(weights)
    expected = np.zeros((x.shape[0], hidden), np.float32)
    for e in range(count):
        route = np.sum(np.where(ids == e, routing, 0).astype(np.float32), -1)

        def project(value, name):
            raw = packed[name][e]
            q, width = ("Q8_0", inter) if name == "down" else ("Q6_K", hidden)
            matrix = bf16_round(dequantize_rows(raw, q, width))
            return bf16_round(value.astype(np.float32) @ matrix.T)

        gate = project(x, "gate")
        activated = bf16_round(gate / (1 + np.exp(-gate)))
        product = bf16_round(activated * project(x, "up"))
        expected += project(product, "down") * route[:, None]
    return bf16_round(expected)


@pytest.mark.parametrize("batch,mode", [(273, 0), (1, 0), (1, 1), (64, 1), (100, 2)])
def test_reference_routing_validation_gate(device, batch, mode):
    packed, ids, weights, source, hidden, inter, count = _routing_validation_case(batch)
    want = _routing_validation_expected(packed, ids, weights, source, hidden, inter, count)
    fn = expert_parallel(None, gate_type="Q6_K", up_type="Q6_K", down_type="Q8_0", hidden=hidden,
                         intermediate=inter)
    tabs = fn.prepare(*(packed[n].reshape(count, -1) for n in ("gate", "up", "down")), device)
    x = torch.from_numpy(source).to(device).to(torch.bfloat16)
    i = torch.from_numpy(ids).to(device)
    w = torch.from_numpy(weights).to(device).to(torch.bfloat16)
    fm = fn.with_mode(mode)
    got = fm(*tabs, x, i, w).float().cpu().numpy()
    zeros = fm(*tabs, x, i, torch.zeros_like(w)).float().cpu().numpy()
    np.testing.assert_allclose(got, want, atol=3e-3, rtol=3e-3)
    np.testing.assert_array_equal(got[np.all(weights == 0, axis=-1)], 0)
    np.testing.assert_array_equal(zeros, 0)
