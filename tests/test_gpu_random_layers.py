"""Seeded sweep of MoE layer configurations against the oracle.

Each case draws a valid layer from its seed: gate/up format, down format
(the checkpoints' mixes and every other allowed pair), hidden and
intermediate sizes (whole blocks of their formats, including 32-value blocks
that leave a partial 256-wide K block), experts, top-k, tokens, kernel family
(mode), an optional shared expert and the W8A8 policy where it applies. The
outputs must meet the MoE gate of test_gpu_moe (max relative error 1e-2,
elementwise 1e-2, at least 90 % bit-identical), and a repeat call must be
bitwise identical.
"""

import numpy as np
import pytest
import torch

from oracle import moe as oracle_moe
from q6moe.experts import expert_parallel, pack_experts
from q6moe.synth import moe_layer

from .test_gpu_moe import _oracle, assert_moe_close

pytestmark = pytest.mark.gpu

GATE_UP = ("Q6_K", "Q5_K", "Q4_K", "Q8_0")
DOWN = ("Q6_K", "Q5_K", "Q4_K", "Q8_0", "Q5_1")
BLOCK = {"Q6_K": 256, "Q5_K": 256, "Q4_K": 256, "Q8_0": 32, "Q5_1": 32}


def draw(seed):
    """One valid layer configuration (a dict) from ``seed``."""
    rng = np.random.default_rng(1000 + seed)
    q = GATE_UP[rng.integers(len(GATE_UP))]
    qd = DOWN[rng.integers(len(DOWN))]
    hb, ib = BLOCK[q], BLOCK[qd]
    hidden = int(hb * rng.integers(1, 3 if hb == 256 else 17))
    inter = int(ib * rng.integers(1, 3 if ib == 256 else 17))
    experts = int(rng.integers(1, 65))
    top_k = int(rng.integers(1, min(experts, 8) + 1))
    tokens = int(rng.choice([1, 2, 5, 8, 16, 17, 33, 64, 65, 96, 128, 200]))
    modes = [0, 2] + ([1] if tokens * top_k <= 1024 else [])
    mode = int(rng.choice(modes))
    w8 = mode != 1 and "Q8_0" in (q, qd) and rng.random() < 0.6
    shared = 0
    if not w8 and rng.random() < 0.4:
        shared = int(ib * rng.integers(1, 3 if ib == 256 else 9))
    return dict(seed=seed, qtype=q, down_qtype=qd, hidden=hidden, intermediate=inter, experts=experts,
                top_k=top_k, tokens=tokens, mode=mode, compute="int8_q8" if w8 else "bf16",
                shared_intermediate=shared)


CASES = [draw(s) for s in range(48)]


@pytest.mark.parametrize("cfg", CASES, ids=[f"{c['qtype']}-{c['down_qtype']}-h{c['hidden']}-i{c['intermediate']}"
                                           f"-e{c['experts']}k{c['top_k']}b{c['tokens']}-m{c['mode']}"
                                           f"-{c['compute']}-s{c['shared_intermediate']}" for c in CASES])
def test_random_layer_matches_oracle(device, cfg):
    q, qd, H, I = cfg["qtype"], cfg["down_qtype"], cfg["hidden"], cfg["intermediate"]
    E, K, B, Is = cfg["experts"], cfg["top_k"], cfg["tokens"], cfg["shared_intermediate"]
    L = moe_layer(seed=cfg["seed"], experts=E, top_k=K, hidden=H, intermediate=I,
                  tokens=B, qtype=q, down_qtype=qd, sigma=0.02, shared_intermediate=Is, pack=False)
    fn = expert_parallel(None, gate_type=q, up_type=q, down_type=qd, hidden=H, intermediate=I,
                         compute=cfg["compute"]).with_mode(cfg["mode"])
    tabs = [pack_experts(L[n], q if n != "down" else qd, I if n != "down" else H, H if n != "down" else I, device)
            for n in ("gate", "up", "down")]
    sh = None
    if Is:
        s = L["shared"]
        sh = dict(gate=pack_experts(s["gate"][None], q, Is, H, device),
                  up=pack_experts(s["up"][None], q, Is, H, device),
                  down=pack_experts(s["down"][None], qd, H, Is, device))
    x = torch.from_numpy(L["x"]).to(device).to(torch.bfloat16)
    ids = torch.from_numpy(L["ids"]).to(device)
    w = torch.from_numpy(L["weights"]).to(device).to(torch.bfloat16)
    got = fn(*tabs, x, ids, w, shared=sh).float().cpu().numpy()
    again = fn(*tabs, x, ids, w, shared=sh).float().cpu().numpy()
    np.testing.assert_array_equal(got, again)
    if cfg["compute"] == "int8_q8":
        want = oracle_moe.expert_ffn(L["gate"], L["up"], L["down"], L["x"], L["ids"], L["weights"],
                                     types=(q, q, qd), hidden=H, intermediate=I, policy="int8_q8")
    else:
        want = _oracle(L, shared=L.get("shared"))
    assert_moe_close(got, want)
