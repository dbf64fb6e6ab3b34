"""Routed SwiGLU expert FFN over packed GGUF experts (test oracle only).

Follows ``kaggle/qwen38_tpu/experts.py:61-131`` and
``kaggle/qwen38_tpu/grouped_experts.py:244-262`` with the rounding points of
``kaggle/qwen38_tpu/math.py:10-20`` and ``precision.py:7-23``:

1. r[b,e] = BF16 sum of the routing weights that name expert e.
2. Active experts (any r != 0) are visited in ascending id.
3. W = RNE_bf16(decode(bytes)).
4. g = RNE(x Wg^T), u = RNE(x Wu^T), FP32 accumulation (here FP64, which
   isolates operand mistakes from reduction order).
5. s = RNE(g * sigmoid(g)); a = RNE(s * u).
6. y = RNE(a Wd^T).
7. out[b] += f32(y[b]) * f32(r[b,e]) in FP32, rows with r == 0 add nothing.
8. RNE to BF16 at the end.

The independent second formulation ``expert_ffn_per_token`` loops over
tokens and their routes instead of experts (routing_validation.py:52-71).
"""

import numpy as np

from .gguf import dequantize_rows
from .numerics import sigmoid, silu_bf16
from .packed_q6 import bf16_round
from .routing import route_weights


def _mm(a, w):
    """a @ w.T for decoded weights (FP64 sums, FP32 result), or w(a) for a
    projection given as a function (the W8A8 policy's integer dot)."""
    if callable(w):
        return w(np.asarray(a, np.float32))
    return (np.asarray(a, np.float64) @ np.asarray(w, np.float64).T).astype(np.float32)


def decode_expert(table, e, qtype, rows, width, policy="bf16"):
    """One expert's weight matrix [rows, width] as BF16 values in FP32; under
    the int8_q8 policy a Q8_0 projection is instead the function running the
    W8A8 integer dot on its bytes (experts.py:85-101, compute.py:20-34)."""
    from .compute import q8_matmul
    from .gguf import block_layout

    values, size = block_layout(qtype)
    raw = np.asarray(table[e]).reshape(rows, -(-width // values), size)
    if policy == "int8_q8" and qtype == "Q8_0":
        return lambda a: q8_matmul(a, raw)
    return bf16_round(dequantize_rows(raw, qtype, width))


def expert_contribution(x, gate_w, up_w, down_w):
    """Steps 4-6 for all rows of x (BF16 values in FP32)."""
    g = bf16_round(_mm(x, gate_w))
    u = bf16_round(_mm(x, up_w))
    a = bf16_round(silu_bf16(g) * u)
    return bf16_round(_mm(a, down_w))


def expert_ffn(gate, up, down, x, ids, weights, *, types, hidden, intermediate, shared=None, workers=1,
               policy="bf16"):
    """x BF16 values [B, hidden] -> BF16 values [B, hidden] as FP32.

    gate/up/down: raw GGUF tables indexable by expert, each expert
    [rows, blocks, bytes] or flat. ``shared`` optionally adds an always-on
    expert (dict of decoded BF16 matrices gate/up/down, optional per-token
    BF16 ``gate_scale``). As in engine.py:199-203 with math.py:282-284 the
    shared output is RNE(y_shared * gate_scale) in BF16 and is added to the
    BF16 routed sum: RNE(f32(routed) + f32(shared)). ``policy`` "int8_q8" runs
    the routed experts' Q8_0 projections as W8A8 integer dots. ``workers`` > 1 computes
    the experts' contributions on a thread pool; they are still added in
    ascending expert id, so the result does not depend on it.
    """
    gt, ut, dt = types
    x = bf16_round(x)
    experts = len(gate)
    r = route_weights(ids, weights, experts)
    active = [e for e in range(experts) if np.any(r[:, e])]

    def contribution(e):
        rows = np.nonzero(r[:, e])[0]
        gw = decode_expert(gate, e, gt, intermediate, hidden, policy)
        uw = decode_expert(up, e, ut, intermediate, hidden, policy)
        dw = decode_expert(down, e, dt, hidden, intermediate, policy)
        return rows, expert_contribution(x[rows], gw, uw, dw)

    if workers > 1 and len(active) > 1:
        from concurrent.futures import ThreadPoolExecutor

        with ThreadPoolExecutor(workers) as pool:
            parts = list(pool.map(contribution, active))
    else:
        parts = [contribution(e) for e in active]
    out = np.zeros((x.shape[0], hidden), np.float32)
    for e, (rows, y) in zip(active, parts):
        out[rows] = (out[rows] + y * r[rows, e][:, None]).astype(np.float32)
    routed = bf16_round(out)
    if shared is None:
        return routed
    y = expert_contribution(x, shared["gate"], shared["up"], shared["down"])
    if shared.get("gate_scale") is not None:
        y = bf16_round(y * bf16_round(np.asarray(shared["gate_scale"], np.float32))[:, None])
    return bf16_round(routed + y)


def shared_gate(x, router):
    """Per-token shared-expert gate of math.py:283 with linear / sigmoid of
    math.py:10-24: RNE_bf16(sigmoid(RNE_bf16(x . router))), x BF16 values
    [B, H], router BF16 values [H] (the checkpoint keeps it BF16,
    checkpoint.py:316-321); the dot in FP64 here, FP32 in the reference."""
    x = bf16_round(np.asarray(x, np.float32))
    w = bf16_round(np.asarray(router, np.float32))
    logit = bf16_round((x.astype(np.float64) @ w.astype(np.float64)).astype(np.float32))
    return bf16_round(sigmoid(logit))


def expert_ffn_per_token(gate, up, down, x, ids, weights, *, types, hidden, intermediate):
    """Second formulation: per token, its distinct experts in ascending id."""
    gt, ut, dt = types
    x = bf16_round(x)
    experts = len(gate)
    r = route_weights(ids, weights, experts)
    out = np.zeros((x.shape[0], hidden), np.float32)
    cache = {}
    for b in range(x.shape[0]):
        acc = np.zeros(hidden, np.float32)
        for e in sorted({int(i) for i in np.asarray(ids)[b] if 0 <= int(i) < experts}):
            if r[b, e] == 0:
                continue
            if e not in cache:
                cache[e] = (
                    decode_expert(gate, e, gt, intermediate, hidden),
                    decode_expert(up, e, ut, intermediate, hidden),
                    decode_expert(down, e, dt, hidden, intermediate),
                )
            y = expert_contribution(x[b : b + 1], *cache[e])[0]
            acc = (acc + y * r[b, e]).astype(np.float32)
        out[b] = acc
    return bf16_round(out)
