"""Router softmax -> top-k -> renormalise -> BF16 (test oracle only).

Follows ``kaggle/qwen38_tpu/math.py:277-281`` (``routes_and_shared``): FP32
softmax of the router logits, ``top_k`` (descending, lower index first on
ties), weights divided by their FP32 sum, inactive rows zeroed, then an RNE
cast to BF16. Written as a per-row brute-force loop.
"""

import numpy as np

from .numerics import softmax
from .packed_q6 import bf16_round


def route(logits, top_k, active=None):
    """logits f32 [B, E] -> (ids int32 [B, k], weights f32 of BF16 values [B, k])."""
    logits = np.asarray(logits, np.float32)
    probs = softmax(logits, -1)
    b, e = probs.shape
    ids = np.zeros((b, top_k), np.int32)
    w = np.zeros((b, top_k), np.float32)
    for row in range(b):
        order = sorted(range(e), key=lambda i: (-float(probs[row, i]), i))[:top_k]
        ids[row] = order
        w[row] = probs[row, order]
    total = np.zeros((b, 1), np.float32)
    for k in range(top_k):  # sequential FP32 sum of the selected probabilities
        total[:, 0] = (total[:, 0] + w[:, k]).astype(np.float32)
    w = (w / total).astype(np.float32)
    if active is not None:
        w = np.where(np.asarray(active, bool)[:, None], w, np.float32(0))
    return ids, bf16_round(w)


def route_weights(ids, weights, experts):
    """r[b, e] = BF16(sum_k [ids[b,k] == e] * weights[b,k]) (experts.py:66-73)."""
    ids = np.asarray(ids)
    weights = np.asarray(weights, np.float32)
    r = np.zeros((ids.shape[0], experts), np.float32)
    for k in range(ids.shape[1]):
        for row in range(ids.shape[0]):
            e = int(ids[row, k])
            if 0 <= e < experts:
                r[row, e] = np.float32(r[row, e] + weights[row, k])
    return bf16_round(r)
