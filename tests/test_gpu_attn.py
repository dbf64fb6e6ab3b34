"""GPU parity of the fused paged decode attention against the oracle.

The oracle (oracle.kv.decode_attention on oracle.kv.read_paged values) keeps
the reference's rounding points; the kernel accumulates in a different order
(MFMA blocks of 32 channels for the scores, token pairs and 256-token chunks
for P.V), so outputs are compared with a max relative error of 1e-2 (BF16
output, FP32 accumulation) and most of them must be bit-identical.
"""

import numpy as np
import pytest
import torch

from oracle import kv as oracle_kv
from q6moe.attention_cache import paged_decode_attention

pytestmark = pytest.mark.gpu


def _case(seed, batch, kvh, r, pages, page_size, pps):
    rng = np.random.default_rng(seed)
    d = 128
    pools, scales = [], []
    for _ in range(2):
        g = rng.standard_normal((pages, page_size, kvh, d)).astype(np.float32)
        sc = (np.abs(g).max(-1) / np.float32(127)).astype(np.float32)
        codes = np.clip(np.rint(g / sc[..., None]), -127, 127).astype(np.int8)
        pools.append(codes.reshape(pages, page_size, kvh * d))
        scales.append(sc)
    table = np.stack([rng.permutation(pages)[:pps] for _ in range(batch)]).astype(np.int32)
    q = rng.standard_normal((batch, kvh * r, d)).astype(np.float32)
    return pools, scales, table, q


def _run(device, pools, scales, table, q, lengths, page_size, kvh):
    qt = torch.from_numpy(q).to(device).to(torch.bfloat16)
    out = paged_decode_attention(
        qt, torch.from_numpy(pools[0]).to(device), torch.from_numpy(scales[0]).to(device),
        torch.from_numpy(pools[1]).to(device), torch.from_numpy(scales[1]).to(device),
        torch.from_numpy(table).to(device), torch.from_numpy(np.asarray(lengths, np.int32)).to(device),
        page_size=page_size, kv_heads=kvh)
    return out.float().cpu().numpy(), qt.float().cpu().numpy()


def _want(pools, scales, table, qv, lengths, page_size, kvh, rows=None):
    rows = range(table.shape[0]) if rows is None else rows
    outs = []
    for b in rows:
        kv = [oracle_kv.read_paged(pools[i].reshape(pools[i].shape[0], page_size, kvh, 128), scales[i],
                                   table[b:b + 1], page_size, kvh, 128, 128) for i in range(2)]
        outs.append(oracle_kv.decode_attention(qv[b:b + 1], kv[0], kv[1], np.asarray(lengths)[b:b + 1])[0])
    return np.stack(outs)


def _check(got, want):
    assert np.isfinite(got).all()
    err = np.max(np.abs(got - want)) / np.abs(want).max()
    assert err <= 1e-2, err
    np.testing.assert_allclose(got, want, rtol=1e-2, atol=1e-2 * np.abs(want).max())
    assert np.mean(got == want) >= 0.5


@pytest.mark.parametrize("batch,kvh,r,page_size,pps,lengths", [
    (2, 2, 8, 64, 8, [512, 300]),        # full and partial last chunk
    (3, 1, 3, 128, 3, [1, 129, 384]),    # one token; group of 3 heads; chunk edges
    (1, 4, 8, 256, 2, [257]),            # one token past the first chunk
    (2, 2, 4, 64, 40, [2560, 2049]),     # two 2048-token P.V chunks, the second partial
    (2, 1, 8, 256, 16, [2048, 4096]),    # lengths on P.V chunk boundaries, one and two whole chunks
])
def test_decode_attention_matches_oracle(device, batch, kvh, r, page_size, pps, lengths):
    pools, scales, table, q = _case(100 + batch * pps, batch, kvh, r, pages=batch * pps + 3,
                                    page_size=page_size, pps=pps)
    got, qv = _run(device, pools, scales, table, q, lengths, page_size, kvh)
    _check(got, _want(pools, scales, table, qv, lengths, page_size, kvh))


def test_decode_attention_unmapped_pages_read_as_zero_and_repeat_is_bitwise(device):
    pools, scales, table, q = _case(7, 2, 2, 4, pages=10, page_size=64, pps=4)
    table[1, 2] = -1   # unmapped page inside the attended range: its codes read as 0
    table[0, 3] = 99   # past the pool
    lengths = [256, 200]
    got, qv = _run(device, pools, scales, table, q, lengths, 64, 2)
    # the oracle reads unmapped pages as zero codes with zero scales
    pz = [np.concatenate([p, np.zeros((1,) + p.shape[1:], p.dtype)]) for p in pools]
    sz = [np.concatenate([s, np.zeros((1,) + s.shape[1:], s.dtype)]) for s in scales]
    tz = np.where((table < 0) | (table >= 10), 10, table).astype(np.int32)
    _check(got, _want(pz, sz, tz, qv, lengths, 64, 2))
    again, _ = _run(device, pools, scales, table, q, lengths, 64, 2)
    np.testing.assert_array_equal(got, again)


def test_decode_attention_c5_shape_sampled(device):
    # batch 8, 32 query heads over 4 KV heads, head_dim 128, 32768 tokens per
    # sequence in pages of 256, random page tables; the oracle checks two
    # sequences (each sequence's output depends only on its own pages).
    B, KVH, R, P, PPS = 8, 4, 8, 256, 128
    pools, scales, table, q = _case(4, B, KVH, R, pages=B * PPS, page_size=P, pps=PPS)
    lengths = [32768, 32768, 20001, 32768, 1, 32768, 32768, 16384]
    got, qv = _run(device, pools, scales, table, q, lengths, P, KVH)
    rows = [2, 7]
    _check(got[rows], _want(pools, scales, table, qv, lengths, P, KVH, rows=rows))


def _sweep_case(seed):
    """A seeded attention shape: batch, KV heads, query heads per KV head, page
    size, pages per sequence, ragged lengths and a few unmapped table entries."""
    rng = np.random.default_rng(500 + seed)
    batch = int(rng.integers(1, 6))
    kvh = int(rng.choice([1, 2, 4]))
    r = int(rng.integers(1, 9))
    page_size = int(rng.choice([64, 128, 256]))
    pps = int(rng.integers(1, 13))
    lengths = [int(rng.integers(1, pps * page_size + 1)) for _ in range(batch)]
    unmapped = int(rng.integers(0, 3)) if pps > 1 else 0
    return batch, kvh, r, page_size, pps, lengths, unmapped


@pytest.mark.parametrize("seed", range(16))
def test_decode_attention_seeded_sweep(device, seed):
    batch, kvh, r, page_size, pps, lengths, unmapped = _sweep_case(seed)
    pages = batch * pps + 2
    pools, scales, table, q = _case(900 + seed, batch, kvh, r, pages=pages, page_size=page_size, pps=pps)
    rng = np.random.default_rng(seed)
    for _ in range(unmapped):  # -1 or past the pool: read as zero codes and scales
        table[rng.integers(batch), rng.integers(pps)] = -1 if rng.random() < 0.5 else pages + 5
    print(f"[sweep] batch {batch} kvh {kvh} r {r} page {page_size} pps {pps} lengths {lengths}", flush=True)
    got, qv = _run(device, pools, scales, table, q, lengths, page_size, kvh)
    pz = [np.concatenate([p, np.zeros((1,) + p.shape[1:], p.dtype)]) for p in pools]
    sz = [np.concatenate([s, np.zeros((1,) + s.shape[1:], s.dtype)]) for s in scales]
    tz = np.where((table < 0) | (table >= pages), pages, table).astype(np.int32)
    _check(got, _want(pz, sz, tz, qv, lengths, page_size, kvh))
