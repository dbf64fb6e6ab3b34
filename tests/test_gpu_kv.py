"""GPU parity of the INT8 KV gather + dequant (bit-exact against the oracle)."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import kv as oracle_kv
from oracle.packed_q6 import bf16_bits, bf16_round
from q6moe.attention_cache import gather_scale_plane, read_paged, read_quantized

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def test_dense_reference_cache_read_bit_exact(device):
    rng = np.random.default_rng(413)
    B, T, H, D, group = 3, 64, 2, 256, 32
    G = H * D // group
    codes = rng.integers(-127, 128, (B, T, H * D), dtype=np.int8)
    plane = bf16_round(rng.uniform(0, 0.03, (B * G, T)).astype(np.float32))
    plane[:, 0] = 0
    idx = np.tile(np.array([0, 0, 1, T // 8, T - 1, -1, -T - 2, T + 3, 17]), (B, 1)).astype(np.int32)
    c = SimpleNamespace(kv_heads=H, head_dim=D, cache_group=group)
    cache = {"k": torch.from_numpy(codes).to(device),
             "k_scale": torch.from_numpy(plane).to(device).to(torch.bfloat16)}
    got = read_quantized(cache, "k", torch.from_numpy(idx).to(device), c)
    want = oracle_kv.read_dense(codes, plane, idx, H, D, group)
    np.testing.assert_array_equal(_bits(got), bf16_bits(want))
    got32 = read_quantized(cache, "k", torch.from_numpy(idx).to(device), c, torch.float32).cpu().numpy()
    t = oracle_kv.normalize_index(idx, T)
    sc = oracle_kv.gather_scale_plane(plane, idx, G)
    for b in range(B):
        want32 = codes[b, t[b]].astype(np.float32).reshape(len(idx[b]), G, group) * sc[b][..., None]
        np.testing.assert_array_equal(got32[b].reshape(len(idx[b]), -1), want32.reshape(len(idx[b]), -1))


@pytest.mark.parametrize("method", ["indexed", "rowwise"])
def test_scale_plane_gather_matches_oracle(device, method):
    rng = np.random.default_rng(629)
    plane = bf16_round(rng.normal(size=(2 * 16, 32)).astype(np.float32))
    idx = np.tile(np.array([0, 0, 1, 4, 31, -1, -34, 35]), (2, 1))
    got = gather_scale_plane(torch.from_numpy(plane).to(device), torch.from_numpy(idx).to(device), 16,
                             method=method).cpu().numpy()
    np.testing.assert_array_equal(got, oracle_kv.gather_scale_plane(plane, idx, 16))


def test_paged_read_bit_exact_and_unmapped_pages_read_zero(device):
    rng = np.random.default_rng(4)
    B, P, pps, H, D = 2, 16, 5, 4, 128
    pages = B * pps + 1
    pool = rng.integers(-127, 128, (pages, P, H, D), dtype=np.int8)
    scales = rng.uniform(0, 0.05, (pages, P, H)).astype(np.float32)
    table = rng.permutation(pages)[: B * pps].astype(np.int32).reshape(B, pps)
    got = read_paged(torch.from_numpy(pool).to(device), torch.from_numpy(scales).to(device),
                     torch.from_numpy(table).to(device), page_size=P, kv_heads=H, head_dim=D)
    want = oracle_kv.read_paged(pool, scales, table, P, H, D, D)
    np.testing.assert_array_equal(_bits(got), bf16_bits(want))
    idx = rng.integers(-pps * P - 3, pps * P + 3, (B, 37)).astype(np.int32)
    got = read_paged(torch.from_numpy(pool).to(device), torch.from_numpy(scales).to(device),
                     torch.from_numpy(table).to(device), page_size=P, kv_heads=H, head_dim=D,
                     indices=torch.from_numpy(idx).to(device))
    np.testing.assert_array_equal(_bits(got), bf16_bits(oracle_kv.read_paged(pool, scales, table, P, H, D, D, idx)))
    bad = table.copy()
    bad[1, 2] = pages + 7
    got = read_paged(torch.from_numpy(pool).to(device), torch.from_numpy(scales).to(device),
                     torch.from_numpy(bad).to(device), page_size=P, kv_heads=H, head_dim=D).float().cpu().numpy()
    assert np.all(got[1, 2 * P : 3 * P] == 0)


def test_odd_shapes_take_the_scalar_path(device):
    rng = np.random.default_rng(7)
    B, P, pps, H, D, group = 2, 3, 2, 3, 10, 5
    pool = rng.integers(-127, 128, (B * pps, P, H, D), dtype=np.int8)
    scales = rng.uniform(0, 0.05, (B * pps, P, H * D // group)).astype(np.float32)
    table = np.arange(B * pps, dtype=np.int32).reshape(B, pps)
    got = read_paged(torch.from_numpy(pool).to(device), torch.from_numpy(scales).to(device),
                     torch.from_numpy(table).to(device), page_size=P, kv_heads=H, head_dim=D, group=group)
    np.testing.assert_array_equal(_bits(got), bf16_bits(oracle_kv.read_paged(pool, scales, table, P, H, D, group)))


def test_kv_pages_workload_reduced_shape(device):
    # Same generator as the bench workload (paged int8 K/V, FP32 per-token-per-head
    # scales, random page permutation), at 2 sequences x 4096 tokens.
    from q6moe.synth import kv_pages

    W = kv_pages(seed=4, batch=2, context=4096)
    for name in ("k", "v"):
        got = read_paged(torch.from_numpy(W[name]).to(device), torch.from_numpy(W[name + "_scale"]).to(device),
                         torch.from_numpy(W["page_table"]).to(device), page_size=256, kv_heads=4, head_dim=128)
        want = oracle_kv.read_paged(W[name], W[name + "_scale"], W["page_table"], 256, 4, 128, 128)
        np.testing.assert_array_equal(_bits(got), bf16_bits(want))


def test_gather_scale_plane_bf16_and_f32_planes_on_device(device):
    # q6moe_kv_gather_scales: values copied bitwise, JAX index rules
    rng = np.random.default_rng(630)
    idx = rng.integers(-70, 70, (3, 41)).astype(np.int32)
    for dt in (torch.bfloat16, torch.float32):
        plane = torch.from_numpy(rng.normal(size=(3 * 8, 64)).astype(np.float32)).to(dt)
        got = gather_scale_plane(plane.to(device), torch.from_numpy(idx).to(device), 8)
        assert got.dtype == dt and tuple(got.shape) == (3, 41, 8)
        want = oracle_kv.gather_scale_plane(plane.float().numpy(), idx, 8)
        np.testing.assert_array_equal(got.float().cpu().numpy(), want)


def test_decode_attention_output_for_a_permuted_query(device):
    # a dense but permuted q: the output keeps the logical [B, Hq, 128] order
    from q6moe.attention_cache import paged_decode_attention
    from q6moe.synth import kv_pages

    W = kv_pages(seed=8, batch=2, context=512, q_heads=8)
    args = [torch.from_numpy(W[n]).to(device) for n in ("k", "k_scale", "v", "v_scale", "page_table")]
    lengths = torch.tensor([512, 300], dtype=torch.int32, device=device)
    q = torch.from_numpy(W["q"]).to(device).to(torch.bfloat16)
    qp = q.permute(1, 0, 2).contiguous().permute(1, 0, 2)  # same values, permuted strides
    a = paged_decode_attention(q, *args[:2], *args[2:4], args[4], lengths, page_size=256, kv_heads=4)
    b = paged_decode_attention(qp, *args[:2], *args[2:4], args[4], lengths, page_size=256, kv_heads=4)
    np.testing.assert_array_equal(_bits(a), _bits(b))
    with pytest.raises(ValueError, match="out must be"):
        paged_decode_attention(q, *args[:2], *args[2:4], args[4], lengths, page_size=256, kv_heads=4,
                               out=torch.empty((2, 8, 64), dtype=torch.bfloat16, device=device))


@pytest.mark.parametrize("seed", range(12))
def test_paged_read_seeded_sweep(device, seed):
    # Seeded shapes: page size, pages per sequence, KV heads, head_dim (vector
    # path when its rows split into 16-byte groups, scalar path otherwise),
    # scale group, FP32 or BF16 scales, BF16 or FP32 output, and explicit
    # indices (negative and past-the-end ones normalized as the reference does).
    rng = np.random.default_rng(300 + seed)
    B = int(rng.integers(1, 5))
    P = int(rng.choice([1, 3, 16, 64, 256]))
    pps = int(rng.integers(1, 6))
    H = int(rng.integers(1, 5))
    D = int(rng.choice([16, 32, 64, 128, 10, 48]))
    group = int(rng.choice([g for g in (D, 16, 32, 8) if D % g == 0]))
    pages = B * pps + int(rng.integers(0, 3))
    pool = rng.integers(-127, 128, (pages, P, H, D), dtype=np.int8)
    scales = rng.uniform(0, 0.05, (pages, P, H * D // group)).astype(np.float32)
    sdt = torch.bfloat16 if rng.random() < 0.5 else torch.float32
    if sdt == torch.bfloat16:
        scales = bf16_round(scales)
    odt = torch.bfloat16 if rng.random() < 0.5 else torch.float32
    table = rng.permutation(pages)[: B * pps].astype(np.int32).reshape(B, pps)
    idx = None
    if rng.random() < 0.6:
        idx = rng.integers(-pps * P - 3, pps * P + 3, (B, int(rng.integers(1, 40)))).astype(np.int32)
    print(f"[sweep] B {B} P {P} pps {pps} H {H} D {D} group {group} scales {sdt} out {odt} "
          f"indices {None if idx is None else idx.shape}", flush=True)
    got = read_paged(torch.from_numpy(pool).to(device), torch.from_numpy(scales).to(device).to(sdt),
                     torch.from_numpy(table).to(device), page_size=P, kv_heads=H, head_dim=D, group=group,
                     indices=None if idx is None else torch.from_numpy(idx).to(device), dtype=odt)
    want = oracle_kv.read_paged(pool, scales, table, P, H, D, group, idx)  # BF16 values as FP32
    if odt == torch.bfloat16:
        np.testing.assert_array_equal(_bits(got), bf16_bits(want))
    else:
        t = oracle_kv.normalize_index(np.broadcast_to(np.arange(pps * P), (B, pps * P)) if idx is None else idx,
                                      pps * P)
        page = table[np.arange(B)[:, None], t // P]
        exact = (pool[page, t % P].astype(np.float32).reshape(B, t.shape[1], -1, group)
                 * scales[page, t % P][..., None]).reshape(want.shape)
        np.testing.assert_array_equal(got.cpu().numpy(), exact)
