"""GPU parity of the routed SwiGLU expert FFN against the NumPy oracle.

Tolerance (BF16 output, FP32 accumulation vs. the oracle's FP64 sums):
  * max relative error max|got - want| / max|want| <= 1e-2;
  * elementwise |got - want| <= 1e-2 * |want| + 1e-2 * max|want|;
  * at least 90 % of outputs bit-identical to the oracle (a differing FP32
    summation order only flips an intermediate BF16 rounding now and then,
    moving a few outputs by one BF16 ulp; a wrong index or term would not).
Structural invariants are exact: zero routes give exact zeros, poisoned
unrouted experts never leak, repeat runs are bitwise identical."""

import numpy as np
import pytest
import torch

from oracle import moe as oracle_moe
from oracle import routing as oracle_routing
from oracle.packed_q6 import bf16_round as bf16_round_np
from q6moe.experts import expert_parallel, pack_experts
from q6moe.synth import moe_layer

pytestmark = pytest.mark.gpu

REL = 1e-2


def _max_rel(got, want):
    return float(np.max(np.abs(got - want)) / max(np.abs(want).max(), 1e-30))


def assert_moe_close(got, want, exact_frac=0.9, ref_gate=True):
    """The MoE gate (max relative error 1e-2, >= 90 % bit-identical) and, with
    ``ref_gate``, the reference's own routed-FFN tolerance atol = rtol = 3e-3
    (kaggle/qwen38_tpu/routing_validation.py:90,105)."""
    assert np.isfinite(got).all()
    assert _max_rel(got, want) <= REL
    np.testing.assert_allclose(got, want, rtol=REL, atol=REL * np.abs(want).max())
    assert np.mean(got == want) >= exact_frac
    if ref_gate:
        np.testing.assert_allclose(got, want, atol=3e-3, rtol=3e-3)


def _run(L, device, mode=0, shared=None, weights=None, ids=None):
    q, H, I = L["qtype"], L["hidden"], L["intermediate"]
    qd = L.get("down_qtype", q)
    fn = expert_parallel(None, gate_type=q, up_type=q, down_type=qd, hidden=H, intermediate=I)
    tabs = [pack_experts(L[n], q if n != "down" else qd, I if n != "down" else H, H if n != "down" else I, device)
            for n in ("gate", "up", "down")]
    x = torch.from_numpy(L["x"]).to(device).to(torch.bfloat16)
    ids = torch.from_numpy(L["ids"] if ids is None else ids).to(device)
    w = torch.from_numpy(L["weights"] if weights is None else weights).to(device).to(torch.bfloat16)
    sh = None
    if shared is not None:
        Is = shared["intermediate"]
        sh = dict(gate=pack_experts(shared["gate"][None], q, Is, H, device),
                  up=pack_experts(shared["up"][None], q, Is, H, device),
                  down=pack_experts(shared["down"][None], qd, H, Is, device))
    fn = fn.with_mode(mode)
    out = fn(*tabs, x, ids, w, shared=sh)
    return out.float().cpu().numpy(), (fn, tabs, x, ids, w, sh)


def _oracle(L, shared=None, weights=None, ids=None):
    q = L["qtype"]
    qd = L.get("down_qtype", q)
    sh = None
    if shared is not None:
        from oracle.gguf import dequantize_rows
        from oracle.packed_q6 import bf16_round

        H, Is = L["hidden"], shared["intermediate"]
        sh = dict(gate=bf16_round(dequantize_rows(shared["gate"], q, H)),
                  up=bf16_round(dequantize_rows(shared["up"], q, H)),
                  down=bf16_round(dequantize_rows(shared["down"], qd, Is)))
    return oracle_moe.expert_ffn(L["gate"], L["up"], L["down"], L["x"],
                                 L["ids"] if ids is None else ids,
                                 L["weights"] if weights is None else weights,
                                 types=(q, q, qd), hidden=L["hidden"], intermediate=L["intermediate"],
                                 shared=sh)


@pytest.mark.parametrize("qtype", ["Q6_K", "Q4_K"])
@pytest.mark.parametrize("tokens,experts,top_k", [(1, 8, 2), (8, 16, 4), (20, 12, 3), (33, 16, 4), (70, 6, 2)])
def test_small_layers_match_oracle(device, qtype, tokens, experts, top_k):
    L = moe_layer(seed=tokens + experts, experts=experts, top_k=top_k, hidden=512, intermediate=256,
                  tokens=tokens, qtype=qtype, pack=False)
    got, _ = _run(L, device)
    assert_moe_close(got, _oracle(L))


@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("tokens,top_k", [(3, 12), (5, 16), (40, 10)])
def test_top_k_above_eight_matches_oracle(device, mode, tokens, top_k):
    # More than 8 routes per token: the decode-step combine sums the rank rows
    # past the first eight in a second loop, and the routing kernels of every
    # path take their 16-entry register branches.
    L = moe_layer(seed=60 + tokens + top_k, experts=20, top_k=top_k, hidden=512, intermediate=256,
                  tokens=tokens, pack=False)
    got, _ = _run(L, device, mode=mode)
    assert_moe_close(got, _oracle(L))


def test_decode_workload_full_size(device):
    # 128 experts, top-8, hidden 2048, intermediate 768, Q6_K, 8 tokens, seed 1.
    L = moe_layer(seed=1, pack=False)
    got, ctx = _run(L, device)
    want = _oracle(L)
    assert_moe_close(got, want)
    # repeat run is bitwise identical (no atomics on values)
    fn, tabs, x, ids, w, _ = ctx
    again = fn(*tabs, x, ids, w).float().cpu().numpy()
    np.testing.assert_array_equal(got, again)


def test_one_launch_decode_on_a_reused_workspace(device):
    # Routes spread thin (512 experts, top-10, 8 tokens: 80 routes) take the
    # one-launch decode kernel, whose down items wait on per-call flags in the
    # workspace. Consecutive calls on one workspace, with new inputs each time,
    # and a workspace whose bytes start as zeros or all ones, must all give the
    # oracle's values; a repeat call is bitwise identical.
    L = moe_layer(seed=66, experts=512, top_k=10, hidden=512, intermediate=256, tokens=40, pack=False)
    fn = expert_parallel(None, gate_type="Q6_K", up_type="Q6_K", down_type="Q6_K", hidden=512,
                         intermediate=256).with_mode(1)
    tabs = fn.prepare(*(L[n].reshape(512, -1) for n in ("gate", "up", "down")), device)
    need = fn.workspace_bytes(8, 10, 512)
    for fill in (0, 255):
        ws = torch.full((need,), fill, dtype=torch.uint8, device=device)
        for r in range(5):
            rows = slice(8 * r, 8 * r + 8)
            x = torch.from_numpy(L["x"][rows]).to(device).to(torch.bfloat16)
            ids = torch.from_numpy(L["ids"][rows]).to(device)
            w = torch.from_numpy(L["weights"][rows]).to(device).to(torch.bfloat16)
            got = fn(*tabs, x, ids, w, workspace=ws).float().cpu().numpy()
            want = oracle_moe.expert_ffn(L["gate"], L["up"], L["down"], L["x"][rows], L["ids"][rows],
                                         L["weights"][rows], types=("Q6_K",) * 3, hidden=512, intermediate=256)
            assert_moe_close(got, want)
            np.testing.assert_array_equal(got, fn(*tabs, x, ids, w, workspace=ws).float().cpu().numpy())


def test_duplicate_routes_sum_and_zero_rows_are_exact_zero(device):
    L = moe_layer(seed=9, experts=6, top_k=3, hidden=256, intermediate=256, tokens=9, pack=False)
    ids = L["ids"].copy()
    w = L["weights"].copy()
    ids[:3, 1] = ids[:3, 0]  # duplicate expert in one token: weights add
    w[4] = 0  # finished request
    got, _ = _run(L, device, ids=ids, weights=w)
    want = _oracle(L, ids=ids, weights=w)
    assert np.all(got[4] == 0)
    assert_moe_close(got, want)
    zero, _ = _run(L, device, ids=ids, weights=np.zeros_like(w))
    assert np.all(zero == 0)


@pytest.mark.parametrize("tokens,top_k,experts", [
    (6, 8, 64),      # one launch, a group of 8 lanes per token
    (40, 16, 128),   # one launch, 4 lanes per token
    (100, 32, 256),  # one launch, 2 lanes per token, top-k above 16
    (256, 8, 64),    # one launch, one lane per token
    (180, 20, 48),   # one launch, one lane per token, top-k above 16
    (513, 8, 16),    # count, then scan and placement in one launch, three chunks
    (600, 24, 96),   # the same, top-k above 16
    (8448, 2, 16),   # 33 chunks: count, scan and placement in three launches
    (257, 4, 1024),  # two chunks, the second of one token; workgroups of 1024 lanes
    (300, 2, 2),     # two experts: every token routes to both
])
def test_grouped_routing_edge_entries(device, tokens, top_k, experts):
    # The grouped family's routing in each of its branches, fed a token whose
    # entries all name one expert, repeats at both ends of a row, ids past the
    # last expert and -1, an all-zero row and a lone zero weight: the result
    # meets the oracle's gate and, where the decode family takes the call, is
    # bitwise equal to it.
    L = moe_layer(seed=70 + top_k, experts=experts, top_k=top_k, hidden=256, intermediate=256, tokens=tokens,
                  pack=False)
    ids = L["ids"].copy()
    w = L["weights"].copy()
    ids[0, :] = ids[0, 0]
    ids[1, -1] = ids[1, 0]
    ids[2, 1] = experts + 5
    ids[2, -1] = -1
    w[3] = 0
    w[4, top_k // 2] = 0
    got, _ = _run(L, device, mode=2, ids=ids, weights=w)
    assert np.all(got[3] == 0)
    assert_moe_close(got, _oracle(L, ids=ids, weights=w))
    if tokens <= 256 and tokens * top_k <= 1024:
        np.testing.assert_array_equal(got, _run(L, device, mode=1, ids=ids, weights=w)[0])


def test_poisoned_unrouted_experts_do_not_leak(device):
    L = moe_layer(seed=10, experts=8, top_k=2, hidden=256, intermediate=256, tokens=4, pack=False)
    used = set(L["ids"].ravel().tolist())
    for e in set(range(8)) - used:
        for n in ("gate", "up", "down"):
            L[n][e, ..., 208:210] = np.array([np.nan], "<f2").view(np.uint8)
    got, _ = _run(L, device)
    assert_moe_close(got, _oracle(L))


def test_out_of_range_ids_are_ignored(device):
    L = moe_layer(seed=12, experts=6, top_k=2, hidden=256, intermediate=256, tokens=3, pack=False)
    ids = L["ids"].copy()
    ids[0, 1] = 99
    ids[1, 0] = -1
    got, _ = _run(L, device, ids=ids)
    assert_moe_close(got, _oracle(L, ids=ids))


@pytest.mark.parametrize("tokens", [1, 8])
def test_q4_with_shared_expert(device, tokens):
    L = moe_layer(seed=3, experts=8, top_k=3, hidden=512, intermediate=256, tokens=tokens, qtype="Q4_K",
                  sigma=0.015, shared_intermediate=512, pack=False)
    got, _ = _run(L, device, shared=L["shared"])
    assert_moe_close(got, _oracle(L, shared=L["shared"]))


@pytest.mark.parametrize("qtype,tokens,mode", [("Q4_K", 8, 1), ("Q4_K", 100, 2), ("Q6_K", 100, 2), ("Q6_K", 20, 1)])
def test_shared_expert_repeated_calls(device, qtype, tokens, mode):
    # Decode-shaped (mode 1) and prefill-shaped (mode 2) calls with a shared
    # expert: three calls in a row on the same stream and workspace, with no
    # synchronisation between them, each bitwise equal to the first.
    L = moe_layer(seed=31, experts=8, top_k=3, hidden=512, intermediate=256, tokens=tokens, qtype=qtype,
                  sigma=0.015, shared_intermediate=768, pack=False)
    want = _oracle(L, shared=L["shared"])
    got, ctx = _run(L, device, mode=mode, shared=L["shared"])
    assert_moe_close(got, want)
    fn, tabs, x, ids, w, sh = ctx  # fn runs ``mode``
    outs = [fn(*tabs, x, ids, w, shared=sh) for _ in range(3)]
    for o in outs:
        np.testing.assert_array_equal(o.float().cpu().numpy(), got)


def test_raw_gguf_tables_match_packed_tables(device):
    L = moe_layer(seed=13, experts=4, top_k=2, hidden=512, intermediate=256, tokens=5, pack=False)
    got, ctx = _run(L, device)
    fn, tabs, x, ids, w, _ = ctx
    raw = [torch.from_numpy(L[n].reshape(4, -1)).to(device) for n in ("gate", "up", "down")]
    out = fn(*raw, x, ids, w).float().cpu().numpy()
    np.testing.assert_array_equal(got, out)


def test_route_weights_match_oracle_merging(device):
    # The combine uses the oracle's merged BF16 route weights; check them
    # indirectly through a single-expert layer where out = RNE(y * r).
    L = moe_layer(seed=14, experts=2, top_k=2, hidden=256, intermediate=256, tokens=2, pack=False)
    ids = np.array([[1, 1], [0, 0]], np.int32)
    w = np.array([[0.375, 0.25], [0.5, 0.5]], np.float32)
    got, _ = _run(L, device, ids=ids, weights=w)
    r = oracle_routing.route_weights(ids, w, 2)
    assert r[0, 1] == 0.625 and r[1, 0] == 1.0
    assert_moe_close(got, _oracle(L, ids=ids, weights=w))


def _q6_codes(blk):
    """Six-bit codes [..., 256] of GGUF Q6_K blocks [..., 210] (gguf_quant.py:159-167)."""
    ql, qh = blk[..., :128].astype(np.uint32), blk[..., 128:192].astype(np.uint32)
    p = np.arange(256)
    n, q, l = p >> 7, (p >> 5) & 3, p & 31
    lo = ql[..., 64 * n + l + 32 * (q & 1)]
    nib = np.where(q >= 2, lo >> 4, lo) & 15
    return (nib | (((qh[..., 32 * n + l] >> (2 * q)) & 3) << 4)).astype(np.uint32)


def _unit_major(raw, qtype, rows, width):
    """The unit-major expert table, restated with NumPy: units of 16 rows x one
    256-wide K block ordered [row group][K block], rows padded with zeros.
    Q4_K: 16-byte chunk c of row j at 16*(16c + j). Q6_K (bit-planar): lane l
    (row j = l % 16, jA = l // 16) holds sub-blocks 4g + jA; its code word g of
    chunk c sits at 1024c + 16l + 4g with pair k (positions 2k, 2k+1, low/high
    16 bits) at bits 4+6(k%2) of word k//2 for k < 6, and for k = 6, 7 the low
    nibbles in word k-6 bits 0-3 and the high two bits in word 2 bits 2(k-6);
    then the lanes' sub-scales (3072 + 4l + g) and the rows' FP16 scales."""
    bs = 210 if qtype == "Q6_K" else 144
    E, kbs, groups = raw.shape[0], -(-width // 256), -(-rows // 16)
    pad = np.zeros((E, groups * 16, kbs, bs), np.uint8)
    pad[:, :rows] = raw.reshape(E, rows, kbs, bs)
    blk = pad.reshape(E, groups, 16, kbs, bs).transpose(0, 1, 3, 2, 4)  # [E, g, kb, row, bs]
    if qtype != "Q6_K":
        return blk.reshape(E, groups, kbs, 16, 9, 16).transpose(0, 1, 2, 4, 3, 5).reshape(E, -1)
    codes = _q6_codes(blk)  # [E, g, kb, row, 256]
    lane = np.arange(64)
    j, jA = lane % 16, lane // 16
    pos = 64 * np.arange(4)[None, :, None] + 16 * jA[:, None, None] + np.arange(16)[None, None, :]
    c = codes[..., j[:, None, None], pos]  # [E, g, kb, lane, group, 16]

    def pair(k, h):
        return c[..., 2 * k + h]

    words = np.zeros(c.shape[:-1] + (3,), np.uint32)
    for h in range(2):
        for w in range(3):
            words[..., w] |= (pair(2 * w, h) << (4 + 16 * h)) | (pair(2 * w + 1, h) << (10 + 16 * h))
        for t in range(2):
            words[..., t] |= (pair(6 + t, h) & 15) << (16 * h)
            words[..., 2] |= (pair(6 + t, h) >> 4) << (2 * t + 16 * h)
    # words [E, g, kb, lane, group, chunk] -> bytes at 1024*chunk + 16*lane + 4*group
    code_bytes = np.ascontiguousarray(words.transpose(0, 1, 2, 5, 3, 4).astype("<u4"))
    code_bytes = code_bytes.view(np.uint8).reshape(E, groups, kbs, 3072)
    sc = blk[..., 192:208][..., j[:, None], 4 * np.arange(4)[None, :] + jA[:, None]]  # [E, g, kb, lane, 4]
    d = blk[..., 208:210].reshape(E, groups, kbs, 32)
    unit = np.concatenate([code_bytes, sc.reshape(E, groups, kbs, 256), d], axis=-1)
    return unit.reshape(E, -1)


@pytest.mark.parametrize("qtype", ["Q6_K", "Q4_K"])
@pytest.mark.parametrize("rows,width", [(40, 512), (16, 256), (33, 768)])
def test_pack_is_the_unit_major_byte_permutation(device, qtype, rows, width):
    bs = 210 if qtype == "Q6_K" else 144
    raw = np.random.default_rng(rows + width).integers(0, 256, size=(3, rows * (width // 256) * bs), dtype=np.uint8)
    table = pack_experts(raw, qtype, rows, width, device)
    np.testing.assert_array_equal(table.data.cpu().numpy(), _unit_major(raw, qtype, rows, width))



def _q8_unit_major(raw, rows, width):
    """Q8_0 unit-major table restated with NumPy: 16 rows x 8 blocks of 34 B
    per unit; lane l (row j = l % 16, jA = l // 16) holds at 1024g + 16l the
    16 codes of K positions 64g + 16jA + [0, 16), i.e. codes 16(jA % 2) + [0, 16)
    of block 2g + jA // 2; the rows' FP16 block scales follow at
    4096 + 8(2j + h) + 2g (block 2g + h). Missing rows and blocks are zero."""
    E, nb, kbs, groups = raw.shape[0], width // 32, -(-width // 256), -(-rows // 16)
    pad = np.zeros((E, groups * 16, kbs * 8, 34), np.uint8)
    pad[:, :rows, :nb] = raw.reshape(E, rows, nb, 34)
    blk = pad.reshape(E, groups, 16, kbs, 8, 34).transpose(0, 1, 3, 2, 4, 5)  # [E, g, kb, row, block, 34]
    lane = np.arange(64)
    j, jA = lane % 16, lane // 16
    chunks = np.arange(4)
    b = 2 * chunks[:, None] + (jA // 2)[None, :]                               # [chunk, lane]
    off = 2 + 16 * (jA % 2)[None, :, None] + np.arange(16)[None, None, :]      # [1, lane, 16]
    codes = blk[:, :, :, j[None, :, None], b[:, :, None], off]                 # [E, g, kb, chunk, lane, 16]
    h, g = np.meshgrid(np.arange(2), chunks, indexing="ij")
    d = blk[:, :, :, :, (2 * g + h).reshape(-1), 0:2]                          # [E, g, kb, row, 8 (h, g), 2]
    unit = np.concatenate([codes.reshape(E, groups, kbs, 4096), d.reshape(E, groups, kbs, 256)], axis=-1)
    return unit.reshape(E, -1)


@pytest.mark.parametrize("rows,width", [(40, 512), (16, 256), (33, 288)])
def test_pack_q8_0_is_the_unit_major_byte_permutation(device, rows, width):
    raw = np.random.default_rng(rows * width).integers(0, 256, size=(3, rows * (width // 32) * 34), dtype=np.uint8)
    table = pack_experts(raw, "Q8_0", rows, width, device)
    np.testing.assert_array_equal(table.data.cpu().numpy(), _q8_unit_major(raw, rows, width))


@pytest.mark.parametrize("qtype,tokens,mode,shared", [
    ("Q6_K", 8, 1, 0), ("Q6_K", 20, 1, 512), ("Q4_K", 8, 1, 512),
    ("Q6_K", 100, 2, 0), ("Q6_K", 300, 0, 512), ("Q4_K", 100, 2, 0)])
def test_q8_0_down_matches_oracle(device, qtype, tokens, mode, shared):
    # The real checkpoint's mix: Q6_K (or Q4_K) gate/up with Q8_0 down, through
    # the decode kernels (mode 1) and the prefill path (mode 2, or 0 above 64
    # tokens: tiled Q6_K gate/up, generic Q8_0 down).
    L = moe_layer(seed=41 + tokens, experts=8, top_k=3, hidden=512, intermediate=256, tokens=tokens,
                  qtype=qtype, down_qtype="Q8_0", sigma=0.02, shared_intermediate=shared, pack=False)
    sh = L.get("shared")
    got, _ = _run(L, device, mode=mode, shared=sh)
    assert_moe_close(got, _oracle(L, shared=sh))


def test_raw_table_cache_follows_the_tensor_not_its_address(device):
    # A raw table freed and a different one allocated in its place (the caching
    # allocator hands the block straight back, same shape, same version) must
    # be repacked: the output follows the new weights.
    from q6moe import experts as ex

    L = moe_layer(seed=15, experts=4, top_k=2, hidden=256, intermediate=256, tokens=3, pack=False)
    L2 = moe_layer(seed=16, experts=4, top_k=2, hidden=256, intermediate=256, tokens=3, pack=False)
    fn = expert_parallel(None, gate_type="Q6_K", up_type="Q6_K", down_type="Q6_K", hidden=256, intermediate=256)
    x = torch.from_numpy(L["x"]).to(device).to(torch.bfloat16)
    ids = torch.from_numpy(L["ids"]).to(device)
    w = torch.from_numpy(L["weights"]).to(device).to(torch.bfloat16)
    gate, up, down = (torch.from_numpy(L[n].reshape(4, -1)).to(device) for n in ("gate", "up", "down"))
    first = fn(gate, up, down, x, ids, w).float().cpu().numpy()
    ptr = gate.data_ptr()
    before = len(ex._CACHE)
    del gate
    torch.cuda.synchronize()
    assert len(ex._CACHE) == before - 1
    gate = torch.from_numpy(L2["gate"].reshape(4, -1)).to(device)
    assert gate.data_ptr() == ptr  # the same block, reused
    second = fn(gate, up, down, x, ids, w).float().cpu().numpy()
    L3 = dict(L, gate=L2["gate"])
    assert_moe_close(second, _oracle(L3))
    assert not np.array_equal(first, second)


def test_raw_table_repack_warns_of_the_doubled_memory(device, monkeypatch):
    # The first device repack of a raw table in a process warns that the raw
    # and packed bytes are both held; packed tables never warn.
    import warnings

    from q6moe import experts as ex

    monkeypatch.setattr(ex._CACHE, "warned", False)
    L = moe_layer(seed=18, experts=2, top_k=1, hidden=256, intermediate=256, tokens=2, pack=False)
    fn = expert_parallel(None, gate_type="Q6_K", up_type="Q6_K", down_type="Q6_K", hidden=256, intermediate=256)
    x = torch.from_numpy(L["x"]).to(device).to(torch.bfloat16)
    ids = torch.from_numpy(L["ids"]).to(device)
    w = torch.from_numpy(L["weights"]).to(device).to(torch.bfloat16)
    raw = [torch.from_numpy(L[n].reshape(2, -1)).to(device) for n in ("gate", "up", "down")]
    with pytest.warns(ResourceWarning, match="held twice"):
        fn(*raw, x, ids, w)
    packed = fn.prepare(*raw, device)
    monkeypatch.setattr(ex._CACHE, "warned", False)
    with warnings.catch_warnings():
        warnings.simplefilter("error", ResourceWarning)
        fn(*packed, x, ids, w)


def test_raw_table_cache_packs_each_live_table_once(device, monkeypatch):
    # 48 layers x 3 raw tables: the first pass packs each of the 144 tables,
    # later passes pack nothing.
    from q6moe import experts as ex

    calls = []
    real = ex.pack_experts
    monkeypatch.setattr(ex, "pack_experts", lambda *a, **k: calls.append(1) or real(*a, **k))
    L = moe_layer(seed=17, experts=2, top_k=1, hidden=256, intermediate=256, tokens=2, pack=False)
    fn = expert_parallel(None, gate_type="Q6_K", up_type="Q6_K", down_type="Q6_K", hidden=256, intermediate=256)
    x = torch.from_numpy(L["x"]).to(device).to(torch.bfloat16)
    ids = torch.from_numpy(L["ids"]).to(device)
    w = torch.from_numpy(L["weights"]).to(device).to(torch.bfloat16)
    layers = [[torch.from_numpy(L[n].reshape(2, -1)).to(device) for n in ("gate", "up", "down")] for _ in range(48)]
    outs = []
    for rep in range(3):
        for g, u, d in layers:
            outs.append(fn(g, u, d, x, ids, w))
        if rep == 0:
            assert len(calls) == 144
    assert len(calls) == 144
    ref = outs[0].float().cpu().numpy()
    for o in outs[1:]:
        np.testing.assert_array_equal(o.float().cpu().numpy(), ref)
    g = layers[0][0]
    g.add_(0)  # an in-place update bumps the version: repacked on the next call
    fn(g, layers[0][1], layers[0][2], x, ids, w)
    assert len(calls) == 145


def test_shared_expert_router_gate_on_device(device):
    for tokens, mode in ((8, 1), (100, 2)):
        L = moe_layer(seed=51, experts=8, top_k=3, hidden=512, intermediate=256, tokens=tokens, qtype="Q6_K",
                      sigma=0.02, shared_intermediate=512, pack=False)
        router = bf16_round_np(np.random.default_rng(52).normal(0, 0.05, 512).astype(np.float32))
        fn = expert_parallel(None, gate_type="Q6_K", up_type="Q6_K", down_type="Q6_K", hidden=512, intermediate=256)
        tabs = fn.prepare(*(L[n].reshape(8, -1) for n in ("gate", "up", "down")), device)
        sh = L["shared"]
        # raw shared tables: the shared intermediate comes from their size
        shared = {n: torch.from_numpy(sh[n].reshape(1, -1)).to(device) for n in ("gate", "up", "down")}
        shared["router"] = torch.from_numpy(router).to(device).to(torch.bfloat16)
        x = torch.from_numpy(L["x"]).to(device).to(torch.bfloat16)
        ids = torch.from_numpy(L["ids"]).to(device)
        w = torch.from_numpy(L["weights"]).to(device).to(torch.bfloat16)
        fm = fn.with_mode(mode)
        got = fm(*tabs, x, ids, w, shared=shared).float().cpu().numpy()
        scale = torch.from_numpy(oracle_moe.shared_gate(L["x"], router)).to(device).to(torch.bfloat16)
        got2 = fm(*tabs, x, ids, w, shared=dict(shared, router=None, scale=scale)).float().cpu().numpy()
        from oracle.gguf import dequantize_rows

        dec = dict(gate=bf16_round_np(dequantize_rows(sh["gate"], "Q6_K", 512)),
                   up=bf16_round_np(dequantize_rows(sh["up"], "Q6_K", 512)),
                   down=bf16_round_np(dequantize_rows(sh["down"], "Q6_K", 512)),
                   gate_scale=oracle_moe.shared_gate(L["x"], router))
        want = oracle_moe.expert_ffn(L["gate"], L["up"], L["down"], L["x"], L["ids"], L["weights"],
                                     types=("Q6_K",) * 3, hidden=512, intermediate=256, shared=dec)
        assert_moe_close(got, want)
        assert_moe_close(got2, want)
        # a non-unit gate changes the output (the scale path is live)
        plain = oracle_moe.expert_ffn(L["gate"], L["up"], L["down"], L["x"], L["ids"], L["weights"],
                                      types=("Q6_K",) * 3, hidden=512, intermediate=256,
                                      shared=dict(dec, gate_scale=None))
        assert not np.allclose(want, plain)


def test_out_and_workspace_are_validated(device):
    L = moe_layer(seed=18, experts=2, top_k=1, hidden=256, intermediate=256, tokens=2, pack=False)
    fn = expert_parallel(None, gate_type="Q6_K", up_type="Q6_K", down_type="Q6_K", hidden=256, intermediate=256)
    tabs = fn.prepare(*(L[n].reshape(2, -1) for n in ("gate", "up", "down")), device)
    x = torch.from_numpy(L["x"]).to(device).to(torch.bfloat16)
    ids = torch.from_numpy(L["ids"]).to(device)
    w = torch.from_numpy(L["weights"]).to(device).to(torch.bfloat16)
    for bad in (torch.empty((2, 255), dtype=torch.bfloat16, device=device),
                torch.empty((2, 256), dtype=torch.float32, device=device),
                torch.empty((256, 2), dtype=torch.bfloat16, device=device).t()):
        with pytest.raises(ValueError, match="out must be"):
            fn(*tabs, x, ids, w, out=bad)
    with pytest.raises(ValueError, match="workspace holds"):
        fn(*tabs, x, ids, w, workspace=torch.empty(16, dtype=torch.uint8, device=device))


@pytest.mark.parametrize("qtype,down,tokens,mode", [
    ("Q4_K", "Q5_1", 8, 1), ("Q4_K", "Q5_1", 100, 2), ("Q5_K", "Q8_0", 8, 1), ("Q5_K", "Q8_0", 100, 2),
    ("Q8_0", "Q8_0", 8, 1), ("Q8_0", "Q8_0", 100, 2), ("Q6_K", "Q5_1", 20, 1), ("Q6_K", "Q5_1", 300, 0),
    ("Q5_K", "Q5_K", 33, 1)])
def test_checkpoint_format_mixes_match_oracle(device, qtype, down, tokens, mode):
    # The real checkpoints' layer mixes (kaggle/qwen38_tpu/checkpoints/q4.json, q6.json,
    # q8.json): Q4_K gate/up with Q5_1 down (43 of 48 Q4 layers), Q5_K gate/up with
    # Q8_0 down, all-Q8_0 layers; plus Q6_K with Q5_1 down and an all-Q5_K layer,
    # through the decode kernels (mode 1) and the grouped path (mode 2 / 0).
    L = moe_layer(seed=71 + tokens, experts=8, top_k=3, hidden=512, intermediate=256, tokens=tokens,
                  qtype=qtype, down_qtype=down, sigma=0.02, shared_intermediate=512 if mode == 1 else 0,
                  pack=False)
    sh = L.get("shared")
    got, _ = _run(L, device, mode=mode, shared=sh)
    assert_moe_close(got, _oracle(L, shared=sh))


@pytest.mark.parametrize("tokens,mode", [(8, 1), (300, 2)])
def test_profiling_events_leave_results_and_bracket_gate_up(device, tokens, mode):
    """The optional profiling events: the output is bitwise the one without
    them, the five events are ordered, and the second and third (the gate/up
    kernel's own start and end on the decode-step and tiled prefill paths)
    span a positive part of the call."""
    L = moe_layer(seed=5, experts=16, top_k=4, hidden=512, intermediate=256, tokens=tokens, pack=False)
    plain, (fn, tabs, x, ids, w, _) = _run(L, device, mode=mode)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(5)]
    for ev in evs:
        ev.record()
    torch.cuda.synchronize()
    for _ in range(3):
        got = fn(*tabs, x, ids, w, events=evs)
        torch.cuda.synchronize()
        assert np.array_equal(got.float().cpu().numpy().view(np.uint32), plain.view(np.uint32))
        ms = [evs[i].elapsed_time(evs[i + 1]) for i in range(4)]
        assert all(m >= 0.0 for m in ms), ms
        assert 0.0 < ms[1] <= evs[0].elapsed_time(evs[4]), ms


@pytest.fixture(scope="module")
def largest_layer(device):
    L = moe_layer(seed=77, experts=1024, top_k=32, hidden=256, intermediate=256, tokens=300, pack=False,
                  down_qtype="Q8_0")
    fn = expert_parallel(None, gate_type="Q6_K", up_type="Q6_K", down_type="Q8_0", hidden=256, intermediate=256)
    tabs = fn.prepare(*(L[n].reshape(1024, -1) for n in ("gate", "up", "down")), device)
    return L, fn, tabs


@pytest.mark.parametrize("tokens", [1, 8, 32, 100, 300])
def test_largest_layer_every_family(device, largest_layer, tokens):
    # The operator's limits: 1024 experts and top-32. 32 tokens x 32 routes is
    # the decode-step kernels' most entries (1024); 100 tokens route in one
    # launch (one chunk of 256 tokens), 300 in three passes over two chunks.
    # Every family the call can take agrees bitwise with the others, and the
    # result meets the oracle's gate.
    L, fn, tabs = largest_layer
    rows = slice(0, tokens)
    x = torch.from_numpy(L["x"][rows]).to(device).to(torch.bfloat16)
    ids = torch.from_numpy(L["ids"][rows]).to(device)
    w = torch.from_numpy(L["weights"][rows]).to(device).to(torch.bfloat16)
    modes = [0, 2] + ([1] if tokens * 32 <= 1024 else [])
    outs = [fn.with_mode(m)(*tabs, x, ids, w).float().cpu().numpy() for m in modes]
    for o in outs[1:]:
        np.testing.assert_array_equal(outs[0], o)
    want = oracle_moe.expert_ffn(L["gate"], L["up"], L["down"], L["x"][rows], L["ids"][rows], L["weights"][rows],
                                 types=("Q6_K", "Q6_K", "Q8_0"), hidden=256, intermediate=256, workers=8)
    assert_moe_close(outs[0], want)
