"""GPU parity of the prefill (tiled grouped-GEMM) expert path against the oracle.

The tiled MFMA kernels run for Q6_K layers whose hidden and intermediate
sizes are multiples of 256 when the call is in prefill mode (mode 2, or
mode 0 with more than 64 tokens). Tolerances are the MoE ones of
test_gpu_moe: max relative error 1e-2 (BF16 output, FP32 accumulation),
elementwise rtol/atol 1e-2, and at least 90 % of outputs bit-identical.
"""

import numpy as np
import pytest
import torch

from oracle import moe as oracle_moe
from q6moe.synth import moe_layer

from .test_gpu_moe import _oracle, _run, assert_moe_close

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("tokens,experts,top_k,hidden,inter", [
    (1, 4, 2, 256, 256),       # one partial tile per expert
    (40, 8, 3, 512, 256),      # partial tiles, several experts
    (300, 6, 2, 512, 512),     # experts with more than one 128-route tile
])
def test_prefill_matches_oracle(device, tokens, experts, top_k, hidden, inter):
    L = moe_layer(seed=100 + tokens, experts=experts, top_k=top_k, hidden=hidden, intermediate=inter,
                  tokens=tokens, bias_sigma=0.5, pack=False)
    got, _ = _run(L, device, mode=2)
    assert_moe_close(got, _oracle(L))


@pytest.mark.parametrize("qtype,down,hidden,inter", [
    ("Q6_K", "Q8_0", 512, 640),   # the Q6 checkpoint's mix; down K = 5 halves of 128
    ("Q8_0", "Q8_0", 384, 384),   # K of 3 halves for both projections
    ("Q4_K", "Q5_1", 512, 384),   # the Q4 checkpoint's mix
    ("Q4_K", "Q4_K", 256, 512),
    ("Q6_K", "Q5_1", 256, 128),   # down K of a single half
    ("Q8_0", "Q6_K", 640, 256),
    ("Q4_K", "Q8_0", 768, 640),
])
def test_tiled_prefill_format_mixes(device, qtype, down, hidden, inter):
    # Every format pair the tiled kernels take, with K not a multiple of 256
    # (odd counts of 128-wide K halves) and skewed routes (partial tiles of
    # every column-group count, experts over several 128-route tiles).
    L = moe_layer(seed=hidden + inter, experts=6, top_k=2, hidden=hidden, intermediate=inter, tokens=300,
                  qtype=qtype, down_qtype=down, bias_sigma=1.0, pack=False)
    got, ctx = _run(L, device, mode=2)
    assert_moe_close(got, _oracle(L))
    fn, tabs, x, ids, w, _ = ctx
    np.testing.assert_array_equal(got, fn(*tabs, x, ids, w).float().cpu().numpy())


def test_prefill_partial_tiles_of_every_width(device):
    # Top-1 routes assigned so that expert e holds counts[e] routes: partial
    # tiles of 1-32, 33-64, 65-96 and 97-128 routes (2, 4, 6 and 8 column
    # groups), exact multiples of 128 and a full tile plus a 1-route tail.
    counts = [1, 17, 32, 33, 50, 64, 65, 90, 96, 97, 113, 127, 128, 129, 256, 200]
    experts = len(counts)
    tokens = sum(counts)
    L = moe_layer(seed=23, experts=experts, top_k=1, hidden=256, intermediate=256, tokens=tokens, pack=False)
    ids = np.repeat(np.arange(experts, dtype=np.int32), counts)
    ids = np.random.default_rng(23).permutation(ids).reshape(tokens, 1)
    w = np.ones((tokens, 1), np.float32)
    got, _ = _run(L, device, mode=2, ids=ids, weights=w)
    assert_moe_close(got, _oracle(L, ids=ids, weights=w))


def test_prefill_and_decode_paths_agree(device):
    # Both paths are checked against the oracle; they share the routing and
    # the rounding boundaries, so they must also agree with each other.
    L = moe_layer(seed=21, experts=16, top_k=4, hidden=1024, intermediate=512, tokens=48, pack=False)
    pre, _ = _run(L, device, mode=2)
    dec, _ = _run(L, device, mode=1)
    want = _oracle(L)
    assert_moe_close(pre, want)
    assert_moe_close(dec, want)
    assert np.mean(pre == dec) >= 0.9


def test_prefill_duplicate_and_dead_routes(device):
    L = moe_layer(seed=22, experts=5, top_k=3, hidden=256, intermediate=256, tokens=200, pack=False)
    ids = L["ids"].copy()
    w = L["weights"].copy()
    ids[:50, 1] = ids[:50, 0]  # duplicated expert in a token: weights add
    w[60:70] = 0  # finished rows give exact zeros
    got, _ = _run(L, device, mode=2, ids=ids, weights=w)
    assert np.all(got[60:70] == 0)
    assert_moe_close(got, _oracle(L, ids=ids, weights=w))


def test_prefill_workload_full_size_sampled(device):
    # 4096 tokens, 128 experts, top-8, hidden 2048, intermediate 768, Q6_K,
    # skewed routing (per-expert logit bias N(0, 0.5)), seed 2. The GPU runs
    # the whole batch; each token's output depends only on its own routes,
    # so the oracle checks a seeded sample of 48 tokens, and a repeat run
    # must be bitwise identical.
    L = moe_layer(seed=2, tokens=4096, bias_sigma=0.5, pack=False)
    got, ctx = _run(L, device, mode=0)
    rows = np.sort(np.random.default_rng(7).choice(4096, 48, replace=False))
    want = oracle_moe.expert_ffn(L["gate"], L["up"], L["down"], L["x"][rows], L["ids"][rows],
                                 L["weights"][rows], types=("Q6_K",) * 3, hidden=2048, intermediate=768)
    assert_moe_close(got[rows], want)
    fn, tabs, x, ids, w, _ = ctx
    again = fn.with_mode(2)(*tabs, x, ids, w).float().cpu().numpy()
    np.testing.assert_array_equal(got, again)
    assert torch.isfinite(torch.from_numpy(got)).all()


def test_prefill_routing_wide_top_k(device):
    # Three routing chunks (256 + 256 + 88 tokens) with 24 routes per token:
    # the staged id/weight rows span several copy rounds per chunk, and the
    # duplicated, out-of-range and zero-weight entries go through the merge.
    L = moe_layer(seed=23, experts=48, top_k=24, hidden=256, intermediate=256, tokens=600, pack=False)
    ids = L["ids"].copy()
    w = L["weights"].copy()
    ids[::5, 2] = ids[::5, 0]
    ids[::7, 3] = 48 + 5
    w[100:110, :] = 0
    w[200:260, 5] = 0
    got, _ = _run(L, device, mode=2, ids=ids, weights=w)
    assert np.all(got[100:110] == 0)
    assert_moe_close(got, _oracle(L, ids=ids, weights=w))
