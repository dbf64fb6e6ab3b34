"""GPU parity of the INT8 KV codec and cache writes (bit-exact against the oracle).

quantize (kaggle/qwen38_tpu/attention_cache.py:15-23): scale = RNE_bf16(max|g|/127),
divisor = the ROUNDED scale (1 for an all-zero group), codes = clip(rint(g/divisor)).
write_quantized (:26-43): rows with active[b] store codes at cache[name][b, t_b]
and scales at cache[name + "_scale"][b*G + g, t_b]; other rows are unchanged.
"""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import kv as oracle_kv
from oracle.packed_q6 import bf16_round
from q6moe.attention_cache import quantize, read_paged, read_quantized, write_paged, write_quantized

pytestmark = pytest.mark.gpu


def _bf16_cuda(a, device):
    return torch.from_numpy(np.asarray(a, np.float32)).to(device).to(torch.bfloat16)


def _codec_inputs():
    rng = np.random.default_rng(31)
    x = bf16_round(rng.normal(size=(6, 512)).astype(np.float32) * rng.uniform(0.01, 4, (6, 1)))
    x[0, :32] = 0                      # all-zero group: scale 0, divisor 1
    x[1, :32] = 0.0
    x[1, 5] = -3.0                     # max at a negative value
    x[2, 32:64] = bf16_round(np.linspace(-1.0, 1.0, 32, dtype=np.float32))
    # ties: with max 127 the BF16 scale is 1.0, so g/divisor hits k + 0.5 exactly
    x[3, 64:96] = np.array([127.0] + [k + 0.5 for k in range(-15, 16)], np.float32)
    return x


@pytest.mark.parametrize("group", [32, 128])
@pytest.mark.parametrize("scale_dtype", [torch.bfloat16, torch.float32])
def test_quantize_bit_exact(device, group, scale_dtype):
    x = _codec_inputs()
    codes, scale = quantize(_bf16_cuda(x, device), group, scale_dtype=scale_dtype)
    want_codes, want_scale = oracle_kv.quantize(x, group, "bf16" if scale_dtype == torch.bfloat16 else "f32")
    np.testing.assert_array_equal(codes.cpu().numpy(), want_codes)
    np.testing.assert_array_equal(scale.float().cpu().numpy(), want_scale)
    if group == 32 and scale_dtype == torch.bfloat16:
        assert np.all(want_codes[0, :32] == 0) and want_scale[0, 0] == 0
        # rint halves to even: k + 0.5 -> the even neighbour
        np.testing.assert_array_equal(want_codes[3, 65:96], [2 * round((k + 0.5) / 2) for k in range(-15, 16)])


def test_quantize_uses_the_rounded_divisor(device):
    # A group whose BF16-rounded scale differs from max/127 gives different
    # codes with the exact quotient as divisor; the kernel must follow the
    # reference's rounded divisor.
    g = np.zeros((1, 32), np.float32)
    g[0, 0] = bf16_round(np.float32(100.3))
    g[0, 1:] = bf16_round(np.linspace(0.1, 90.0, 31).astype(np.float32))
    codes, scale = quantize(_bf16_cuda(g, device), 32)
    want_codes, want_scale = oracle_kv.quantize(g, 32)
    exact = np.clip(np.rint(g / (np.abs(g).max() / np.float32(127))), -127, 127)
    assert not np.array_equal(want_codes.astype(np.float32), exact)  # the case has teeth
    np.testing.assert_array_equal(codes.cpu().numpy(), want_codes)
    np.testing.assert_array_equal(scale.float().cpu().numpy(), want_scale)


def test_write_quantized_reference_case(device):
    # kaggle/tests/test_qwen38_compute.py:101-118 restated: two rows, one active.
    c = SimpleNamespace(kv_heads=2, head_dim=256, cache_group=32)
    rng = np.random.default_rng(81)
    source = bf16_round(rng.normal(size=(2, 2, 256)).astype(np.float32))
    cache = {n: torch.zeros((2, 8, 512), dtype=torch.int8, device=device) for n in ("k", "v")}
    cache.update({n: torch.zeros((32, 8), dtype=torch.bfloat16, device=device) for n in ("k_scale", "v_scale")})
    src = _bf16_cuda(source, device)
    out = write_quantized(cache, src, src, torch.tensor([3, 7]), torch.tensor([True, False]), c)
    assert out is cache
    actual = read_quantized(cache, "k", torch.tensor([[3], [7]], device=device), c, torch.float32)
    actual = actual.cpu().numpy()[:, 0].reshape(2, 512)
    grouped = source[0].reshape(2, 8, 32)
    scale = bf16_round(np.max(np.abs(grouped), -1) / np.float32(127))
    codes = np.clip(np.rint(grouped / np.where(scale == 0, 1, scale)[..., None]), -127, 127)
    np.testing.assert_array_equal(actual[0], (codes * scale[..., None]).reshape(512))
    np.testing.assert_array_equal(actual[1], 0)
    for name in ("k_scale", "v_scale"):
        np.testing.assert_array_equal(cache[name].float().cpu().numpy()[16:], 0)
    zero, zscale = quantize(torch.zeros((2, 2, 256), device=device), 32)
    assert not zero.any() and not zscale.float().any()


def test_write_paged_then_read_bit_exact(device):
    rng = np.random.default_rng(5)
    B, pps, P, H, D = 3, 4, 16, 4, 128
    pages = B * pps + 2
    table = rng.permutation(pages)[: B * pps].reshape(B, pps).astype(np.int32)
    table[2, 3] = pages + 5  # unmapped page: writes there are dropped
    pool = torch.full((pages, P, H * D), 7, dtype=torch.int8, device=device)
    scales = torch.full((pages, P, H), 0.5, dtype=torch.float32, device=device)
    x = bf16_round(rng.normal(size=(B, H * D)).astype(np.float32))
    slots = np.array([5, -1, 3 * P + 2], np.int32)  # row 1: last slot; row 2: unmapped page
    active = np.array([1, 1, 1], np.uint8)
    write_paged(pool, scales, torch.from_numpy(table).to(device), _bf16_cuda(x, device),
                torch.from_numpy(slots).to(device), page_size=P, kv_heads=H, head_dim=D,
                active=torch.from_numpy(active).to(device))
    want_codes, want_scale = oracle_kv.quantize(x, D, "f32")
    pool_h, sc_h = pool.cpu().numpy(), scales.cpu().numpy()
    for b, t in ((0, 5), (1, pps * P - 1)):
        pg, sl = table[b, t // P], t % P
        np.testing.assert_array_equal(pool_h[pg, sl], want_codes[b])
        np.testing.assert_array_equal(sc_h[pg, sl], want_scale[b])
    written = {(table[0, 0], 5), (table[1, pps - 1], P - 1)}
    for pg in range(pages):
        for sl in range(P):
            if (pg, sl) not in written:
                assert np.all(pool_h[pg, sl] == 7) and np.all(sc_h[pg, sl] == 0.5)
    # read back through the paged gather: the written token dequantises exactly
    tab = torch.from_numpy(table[:2]).to(device)
    got = read_paged(pool, scales, tab, page_size=P, kv_heads=H, head_dim=D,
                     indices=torch.tensor([[5], [pps * P - 1]], dtype=torch.int32, device=device),
                     dtype=torch.float32).cpu().numpy().reshape(2, H * D)
    want = (want_codes[:2].astype(np.float32).reshape(2, H, D) * want_scale[:2][..., None]).reshape(2, H * D)
    np.testing.assert_array_equal(got, want)


def test_inactive_and_out_of_range_rows_leave_the_cache_unchanged(device):
    c = SimpleNamespace(kv_heads=1, head_dim=64, cache_group=32)
    cache = {n: torch.full((3, 4, 64), 9, dtype=torch.int8, device=device) for n in ("k", "v")}
    cache.update({n: torch.full((6, 4), 2.0, dtype=torch.bfloat16, device=device) for n in ("k_scale", "v_scale")})
    x = torch.randn(3, 64, device=device).to(torch.bfloat16)
    write_quantized(cache, x, x, torch.tensor([1, 9, 2]), torch.tensor([False, True, True]), c)
    k = cache["k"].cpu().numpy()
    assert np.all(k[0] == 9) and np.all(k[1] == 9)  # row 0 inactive, row 1 slot 9 out of range
    want_codes, want_scale = oracle_kv.quantize(x.float().cpu().numpy(), 32)
    np.testing.assert_array_equal(k[2, 2], want_codes[2])
    assert np.all(np.delete(k[2], 2, axis=0) == 9)
    np.testing.assert_array_equal(cache["k_scale"].float().cpu().numpy()[4:, 2], want_scale[2])
    assert np.all(cache["k_scale"].float().cpu().numpy()[:4] == 2.0)
