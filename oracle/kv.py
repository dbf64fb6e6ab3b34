"""INT8 KV codec, scale-plane gather and dequantising reads (test oracle only).

Follows ``kaggle/qwen38_tpu/attention_cache.py:15-81``:

* ``quantize`` (:15-23): scale = RNE_bf16(max|g| / 127); codes are
  clip(rint(g / divisor), -127, 127) with the ROUNDED scale as divisor (1 for
  an all-zero group). The FP32 per-token-per-head variant keeps the FP32
  quotient max|g| / 127 as scale and divisor.
* ``gather_scale_plane`` (:46-68) and the token gather of ``read_quantized``
  (:71-81) use JAX indexing rules: a negative index adds the extent, then the
  index is clamped into range (the reference test oracle,
  kaggle/tests/test_qwen38_kv_gather.py:22-32).
* ``read_quantized``: RNE_dtype(f32(code) * f32(scale)).

The paged variant (pages of P tokens, page tables per sequence) is the
build's generalisation of the dense [B, T, KVH*D] cache; its arithmetic is
the same per element.
"""

import numpy as np

from .packed_q6 import bf16_round


def quantize(x, group, scale_dtype="bf16"):
    """x [..., C] -> (int8 codes [..., C], FP32 scale values [..., C // group])."""
    g = np.asarray(x, np.float32).reshape(*np.shape(x)[:-1], -1, group)
    full = (np.max(np.abs(g), -1) / np.float32(127)).astype(np.float32)
    scale = bf16_round(full) if scale_dtype == "bf16" else full
    divisor = np.where(scale == 0, np.float32(1), scale).astype(np.float32)
    codes = np.clip(np.rint((g / divisor[..., None]).astype(np.float32)), -127, 127)
    return codes.astype(np.int8).reshape(np.shape(x)), scale


def normalize_index(t, extent):
    t = np.asarray(t, np.int64)
    t = np.where(t < 0, t + extent, t)
    return np.clip(t, 0, extent - 1)


def gather_scale_plane(plane, indices, groups):
    """plane [B*G, T], indices [B, S] -> [B, S, G] (attention_cache.py:46-68)."""
    plane = np.asarray(plane)
    b, s = np.shape(indices)
    t = normalize_index(indices, plane.shape[1])
    out = np.empty((b, s, groups), plane.dtype)
    for row in range(b):
        for g in range(groups):
            out[row, :, g] = plane[row * groups + g, t[row]]
    return out


def read_dense(codes, plane, indices, kv_heads, head_dim, group):
    """Reference layout: codes int8 [B, T, KVH*D], scale plane [B*G, T] (FP32 values).

    Returns FP32 values of the BF16 result [B, S, KVH, D].
    """
    codes = np.asarray(codes)
    b, t_cap, _ = codes.shape
    groups = kv_heads * head_dim // group
    t = normalize_index(indices, t_cap)
    picked = np.stack([codes[row, t[row]] for row in range(b)]).astype(np.float32)
    sc = gather_scale_plane(plane, indices, groups).astype(np.float32)
    vals = picked.reshape(b, t.shape[1], groups, group) * sc[..., None]
    return bf16_round(vals.astype(np.float32)).reshape(b, t.shape[1], kv_heads, head_dim)


def read_paged(pool, scales, page_table, page_size, kv_heads, head_dim, group, indices=None):
    """Paged layout: pool int8 [pages, P, KVH, D], scales FP32 [pages, P, KVH*D/group].

    page_table int32 [B, pages_per_seq]; tokens are 0..capacity-1 or ``indices``.
    Returns FP32 values of the BF16 result [B, S, KVH, D].
    """
    pool = np.asarray(pool)
    table = np.asarray(page_table)
    b, pps = table.shape
    cap = pps * page_size
    if indices is None:
        indices = np.broadcast_to(np.arange(cap), (b, cap))
    t = normalize_index(indices, cap)
    page = table[np.arange(b)[:, None], t // page_size]
    slot = t % page_size
    codes = pool[page, slot].astype(np.float32).reshape(b, t.shape[1], -1, group)
    sc = np.asarray(scales, np.float32)[page, slot]
    vals = (codes * sc[..., None]).astype(np.float32)
    return bf16_round(vals).reshape(b, t.shape[1], kv_heads, head_dim)


def decode_attention(q, keys, values, lengths):
    """Core of the decode attention step, one query token per sequence
    (kaggle/qwen38_tpu/attention_cache.py:159-169): q [B, Hq, D] (BF16 values
    as FP32), keys/values [B, T, KVH, D] (read_quantized values, BF16 as FP32),
    lengths [B] attended tokens (the reference's mask indices <= position:
    lengths = position + 1).

    raw = RNE_bf16(q.k) with FP32 accumulation (:160-162); score =
    RNE_bf16(f32(raw) / float32(sqrt(D))) (:163-165); prob = exp(score - max)
    / sum(exp(score - max)) in FP32 over the attended tokens (numerics.py:48-51,
    masked tokens -inf); out = RNE_bf16(sum_t RNE_bf16(prob) * v) with FP32
    accumulation (:167-169). Returns FP32 values of the BF16 output [B, Hq, D].
    """
    q = np.asarray(q, np.float32)
    keys = np.asarray(keys, np.float32)
    values = np.asarray(values, np.float32)
    b, hq, d = q.shape
    t_cap, kvh = keys.shape[1], keys.shape[2]
    qg = q.reshape(b, kvh, hq // kvh, d)
    raw = bf16_round(np.einsum("bkrd,btkd->bkrt", qg, keys, dtype=np.float32).astype(np.float32))
    score = bf16_round((raw / np.float32(d ** 0.5)).astype(np.float32))
    mask = np.arange(t_cap)[None, :] < np.asarray(lengths)[:, None]
    score = np.where(mask[:, None, None, :], score, np.float32(-np.inf)).astype(np.float32)
    e = np.exp((score - score.max(axis=-1, keepdims=True)).astype(np.float32)).astype(np.float32)
    prob = (e / e.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    out = np.einsum("bkrt,btkd->bkrd", bf16_round(prob), values, dtype=np.float32).astype(np.float32)
    return bf16_round(out).reshape(b, hq, d)
