"""Seeded synthetic workloads for the packed-expert path (host, NumPy).

Every generator uses ``np.random.default_rng(seed)`` with a fixed draw order
(documented per function) so the GPU path and the CPU oracle see identical
bytes. Weights are drawn as FP32 N(0, sigma) and quantized with the
build-owned quantizers of ``q6moe.quantize``; activations are FP32 N(0, 1)
rounded to BF16 (RNE) by the caller's cast.

Workloads
---------
* ``projection``  single Q6_K projection, x [8, 2048], W [2048 -> 768], seed 0.
* ``moe_layer``   routed SwiGLU layer: E experts, top-k, hidden H,
  intermediate I; tokens x and router logits (optionally plus a per-expert
  bias for a skewed load). Decode: 128 experts, top-8, H 2048, I 768,
  8 tokens, seed 1. Prefill: same layer, 4096 tokens, bias N(0, 0.5), seed 2.
  Q4_K: 64 experts, top-6, H 4096, I 1024, shared expert I 4096, seed 3.
* ``kv_pages``    INT8 paged KV: 8 sequences x 32 768 tokens in 256-token
  pages, 4 KV heads of 128, FP32 per-token-per-head scales, seed 4.
"""

import numpy as np

from .layout import pack_q6_experts
from .quantize import QUANTIZERS


def _normal(rng, shape, sigma=1.0):
    return rng.standard_normal(shape, dtype=np.float32) * np.float32(sigma)


def projection(seed=0, tokens=8, inputs=2048, outputs=768, sigma=0.02):
    """Draw order: x [tokens, inputs], then W [inputs, outputs]; quantizes W^T rows."""
    rng = np.random.default_rng(seed)
    x = _normal(rng, (tokens, inputs))
    w = _normal(rng, (inputs, outputs), sigma)
    raw = QUANTIZERS["Q6_K"](np.ascontiguousarray(w.T))
    return dict(x=x, raw=raw, inputs=inputs, outputs=outputs)


def softmax_topk(logits, top_k):
    """Router: FP32 softmax -> top-k (ties: lower id) -> renormalise -> BF16 values.

    Same steps as kaggle/qwen38_tpu/math.py:277-281 (routes_and_shared). The
    probabilities use FP64 exp rounded to FP32 and FP32 division.
    """
    logits = np.asarray(logits, np.float32)
    shifted = logits - logits.max(-1, keepdims=True)
    e = np.exp(shifted.astype(np.float64)).astype(np.float32)
    p = (e / e.sum(-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    order = np.lexsort((np.broadcast_to(np.arange(p.shape[1]), p.shape), -p), axis=-1)
    ids = order[:, :top_k].astype(np.int32)
    w = np.take_along_axis(p, ids, -1)
    total = np.zeros(w.shape[0], np.float32)
    for k in range(top_k):
        total = (total + w[:, k]).astype(np.float32)
    w = (w / total[:, None]).astype(np.float32)
    return ids, bf16_values(w)


def bf16_values(x):
    """RNE to BF16, kept as FP32 values (finite inputs)."""
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)


def moe_layer(
    seed=1,
    experts=128,
    top_k=8,
    hidden=2048,
    intermediate=768,
    tokens=8,
    sigma=0.02,
    qtype="Q6_K",
    bias_sigma=None,
    shared_intermediate=0,
    pack=True,
    down_qtype=None,
):
    """Draw order: x [B, H]; logits [B, E]; bias [E] (if bias_sigma); then per expert
    gate [I, H], up [I, H], down [H, I]; then the shared expert gate, up, down.

    Returns raw GGUF tables ``gate/up/down`` [E, rows, blocks, bytes] and, for
    Q6_K with ``pack``, the stacked SoA planes ``*_data`` / ``*_scales``.
    ``down_qtype`` (default ``qtype``) quantizes the down projections (routed
    and shared), e.g. Q6_K gate/up with Q8_0 down.
    """
    rng = np.random.default_rng(seed)
    x = _normal(rng, (tokens, hidden))
    logits = _normal(rng, (tokens, experts))
    if bias_sigma is not None:
        logits = (logits + _normal(rng, (experts,), bias_sigma)[None, :]).astype(np.float32)
    quant = QUANTIZERS[qtype]
    down_qtype = down_qtype or qtype
    quant_d = QUANTIZERS[down_qtype]
    tables = {"gate": [], "up": [], "down": []}
    for _ in range(experts):
        tables["gate"].append(quant(_normal(rng, (intermediate, hidden), sigma)))
        tables["up"].append(quant(_normal(rng, (intermediate, hidden), sigma)))
        tables["down"].append(quant_d(_normal(rng, (hidden, intermediate), sigma)))
    out = dict(x=x, logits=logits, experts=experts, top_k=top_k, hidden=hidden,
               intermediate=intermediate, qtype=qtype, down_qtype=down_qtype)
    for name, parts in tables.items():
        out[name] = np.stack(parts)
    ids, weights = softmax_topk(logits, top_k)
    out.update(ids=ids, weights=weights)
    if shared_intermediate:
        out["shared"] = dict(
            gate=quant(_normal(rng, (shared_intermediate, hidden), sigma)),
            up=quant(_normal(rng, (shared_intermediate, hidden), sigma)),
            down=quant_d(_normal(rng, (hidden, shared_intermediate), sigma)),
            intermediate=shared_intermediate,
        )
    if pack:
        for name, width, q in (("gate", hidden, qtype), ("up", hidden, qtype), ("down", intermediate, down_qtype)):
            if q == "Q6_K":
                out[name + "_data"], out[name + "_scales"] = pack_q6_experts(out[name], width)
    return out


def _expert_weights(seed, e, hidden, intermediate, sigma, quant, quant_d):
    rng = np.random.default_rng([seed, e])
    g = quant(_normal(rng, (intermediate, hidden), sigma))
    u = quant(_normal(rng, (intermediate, hidden), sigma))
    d = quant_d(_normal(rng, (hidden, intermediate), sigma))
    return g, u, d


def wide_moe_layer(
    seed=5,
    experts=512,
    top_k=10,
    hidden=2560,
    intermediate=640,
    tokens=8,
    sigma=0.02,
    qtype="Q6_K",
    down_qtype="Q8_0",
    bias_sigma=None,
    workers=None,
):
    """A wide routed layer whose experts are drawn independently: by default
    the MoE layer of the reference's model (kaggle/qwen38_tpu/config.py:13-19:
    512 experts, top-10, hidden 2560, intermediate 640) in the formats of its
    Q6 checkpoint (checkpoints/q6.json: Q6_K gate/up, Q8_0 down in every layer).

    Draw order: ``default_rng(seed)``: x [B, H], logits [B, E], bias [E] (if
    ``bias_sigma``); then expert e's gate [I, H], up [I, H] and down [H, I],
    each N(0, sigma), from its own ``default_rng([seed, e])``, so the experts
    are quantized on a thread pool (``workers``) with the same bytes for any
    pool size. Returns the same keys as ``moe_layer`` (raw GGUF tables
    [E, rows, blocks, bytes], no SoA planes).
    """
    from concurrent.futures import ThreadPoolExecutor
    import os

    rng = np.random.default_rng(seed)
    x = _normal(rng, (tokens, hidden))
    logits = _normal(rng, (tokens, experts))
    if bias_sigma is not None:
        logits = (logits + _normal(rng, (experts,), bias_sigma)[None, :]).astype(np.float32)
    quant, quant_d = QUANTIZERS[qtype], QUANTIZERS[down_qtype]
    first = _expert_weights(seed, 0, hidden, intermediate, sigma, quant, quant_d)
    tables = {n: np.empty((experts,) + t.shape, np.uint8) for n, t in zip(("gate", "up", "down"), first)}

    def one(e):
        parts = first if e == 0 else _expert_weights(seed, e, hidden, intermediate, sigma, quant, quant_d)
        for n, t in zip(("gate", "up", "down"), parts):
            tables[n][e] = t

    workers = workers or min(16, len(os.sched_getaffinity(0)))
    with ThreadPoolExecutor(workers) as pool:
        list(pool.map(one, range(experts)))
    ids, weights = softmax_topk(logits, top_k)
    out = dict(x=x, logits=logits, experts=experts, top_k=top_k, hidden=hidden, intermediate=intermediate,
               qtype=qtype, down_qtype=down_qtype, ids=ids, weights=weights)
    out.update(tables)
    return out


def kv_pages(seed=4, batch=8, context=32768, page_size=256, kv_heads=4, head_dim=128, q_heads=32):
    """Draw order: K [pages, P, KVH, D]; V (same); page-table permutation; q [B, Hq, D].

    K and V are quantized per token and head (group = head_dim) to int8 with
    FP32 scales max|g| / 127 (codes clip(rint(g / scale), -127, 127)).
    """
    rng = np.random.default_rng(seed)
    pages = batch * context // page_size
    out = {}
    for name in ("k", "v"):
        g = _normal(rng, (pages, page_size, kv_heads, head_dim))
        scale = (np.abs(g).max(-1) / np.float32(127)).astype(np.float32)
        div = np.where(scale == 0, np.float32(1), scale)
        out[name] = np.clip(np.rint(g / div[..., None]), -127, 127).astype(np.int8)
        out[name + "_scale"] = scale
        del g
    out["page_table"] = rng.permutation(pages).astype(np.int32).reshape(batch, context // page_size)
    out["q"] = _normal(rng, (batch, q_heads, head_dim))
    out.update(batch=batch, context=context, page_size=page_size, kv_heads=kv_heads, head_dim=head_dim)
    return out
