"""INT8 KV cache on the GPU: ``quantize``, ``write_quantized``, ``read_quantized``
and the paged variants.

Mirrors kaggle/qwen38_tpu/attention_cache.py:15-81:

* dense reference cache: ``cache[name]`` int8 [B, T, KVH*D], ``cache[name +
  "_scale"]`` BF16 [B*G, T] with G = KVH*D/cache_group; ``indices`` [B, S]
  follow JAX gather rules (negative adds T, then clamp);
* result ``compute_cast(f32(code) * f32(scale), dtype)``, i.e. RNE to BF16.

``read_paged`` / ``write_paged`` are the paged generalisation (page tables
per sequence, FP32 per-token-per-head scales). Reads run the HIP kernel
``q6moe_kv_read``; ``quantize`` runs ``q6moe_kv_quantize`` and the writes
``q6moe_kv_write``, ``gather_scale_plane`` runs ``q6moe_kv_gather_scales``
with the reference contract and error messages.
"""

import ctypes

import torch

from . import _lib


def _dtype_code(dtype):
    if dtype == torch.bfloat16:
        return _lib.BF16
    if dtype == torch.float32:
        return _lib.F32
    raise ValueError("dtype must be torch.bfloat16 or torch.float32")


def _run(args, device):
    lib = _lib.load()
    with torch.cuda.device(device):
        rc = lib.q6moe_kv_read(ctypes.byref(args), _lib.stream_handle(device))
    _lib.check(rc, "kv_read")


def _group_of(c):
    return getattr(c, "cache_group", None) or getattr(c, "group")


def quantize(x, group, scale_dtype=torch.bfloat16):
    """attention_cache.py:15-23 on the GPU: x [..., C] (BF16/FP32) -> (int8 codes
    [..., C], scale [..., C // group]). A BF16 scale is RNE_bf16(max|g| / 127)
    and is also the divisor (1 for an all-zero group); FP32 keeps the quotient."""
    if not isinstance(x, torch.Tensor) or x.device.type != "cuda":
        raise ValueError("x must be a GPU tensor")
    if x.shape[-1] % group:
        raise ValueError("group must divide the last dimension")
    xx = x.contiguous()
    rows, chans = xx.numel() // x.shape[-1], x.shape[-1]
    codes = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    scale = torch.empty((*x.shape[:-1], chans // group), dtype=scale_dtype, device=x.device)
    lib = _lib.load()
    with torch.cuda.device(x.device):
        rc = lib.q6moe_kv_quantize(xx.data_ptr(), _dtype_code(xx.dtype), rows, chans, group, codes.data_ptr(),
                                   scale.data_ptr(), _dtype_code(scale_dtype), _lib.stream_handle(x.device))
    _lib.check(rc, "kv_quantize")
    return codes, scale


def _write(x, codes, scales, *, layout, indices, active, batch, capacity, heads, dim, group, table=None,
           pool_pages=0, pages_per_seq=0, page_size=0):
    xx = x.reshape(batch, heads * dim).contiguous()
    idx = indices.to(device=codes.device, dtype=torch.int32).contiguous()
    if idx.numel() != batch:
        raise ValueError("indices must hold one token slot per row")
    act = None
    if active is not None:
        act = active.to(device=codes.device).reshape(batch).to(torch.uint8).contiguous()
    a = _lib.KvWriteArgs()
    a.x, a.x_dtype = xx.data_ptr(), _dtype_code(xx.dtype)
    a.codes, a.scales = codes.data_ptr(), scales.data_ptr()
    a.scale_dtype, a.scale_layout = _dtype_code(scales.dtype), layout
    a.page_table = None if table is None else table.data_ptr()
    a.pool_pages, a.pages_per_seq, a.page_size = pool_pages, pages_per_seq, page_size
    a.indices = idx.data_ptr()
    a.active = None if act is None else act.data_ptr()
    a.batch, a.capacity = batch, capacity
    a.kv_heads, a.head_dim, a.group = heads, dim, group
    lib = _lib.load()
    with torch.cuda.device(codes.device):
        rc = lib.q6moe_kv_write(ctypes.byref(a), _lib.stream_handle(codes.device))
    _lib.check(rc, "kv_write")


def write_quantized(cache, key, value, indices, active, c):
    """attention_cache.py:26-43: quantise the new token's key/value rows
    ([B, kv_heads*head_dim] or [B, kv_heads, head_dim]) and store codes at
    cache[name][b, indices[b]] and scales at cache[name + "_scale"][b*G + g,
    indices[b]] for rows with ``active[b]``. The cache tensors are updated in
    place (the reference's functional update with buffer donation) and the
    dict is returned."""
    group = _group_of(c)
    for name, token in (("k", key), ("v", value)):
        codes, plane = cache[name], cache[name + "_scale"]
        if codes.dtype != torch.int8 or codes.ndim != 3 or codes.shape[2] != c.kv_heads * c.head_dim:
            raise ValueError("cache codes must be int8 [batch, time, kv_heads * head_dim]")
        if not codes.is_contiguous() or not plane.is_contiguous():
            raise ValueError("cache tensors must be contiguous")
        batch, time, chans = codes.shape
        if plane.shape != (batch * (chans // group), time):
            raise ValueError("Scale plane must be [batch * groups, time]")
        _write(token, codes, plane, layout=0, indices=indices, active=active, batch=batch, capacity=time,
               heads=c.kv_heads, dim=c.head_dim, group=group)
    return cache


def write_paged(pool, scales, page_table, x, indices, *, page_size, kv_heads, head_dim, group=None, active=None):
    """Paged write: quantise x [B, kv_heads*head_dim] and store row b at token
    slot indices[b] of sequence b (page page_table[b, t // page_size])."""
    group = head_dim if group is None else group
    if pool.dtype != torch.int8 or pool.ndim < 3 or pool.shape[1] != page_size or not pool.is_contiguous():
        raise ValueError("pool must be contiguous int8 [pages, page_size, ...]")
    table = page_table.to(device=pool.device, dtype=torch.int32).contiguous()
    batch, pps = table.shape
    _write(x, pool, scales, layout=1, indices=indices, active=active, batch=batch, capacity=pps * page_size,
           heads=kv_heads, dim=head_dim, group=group, table=table, pool_pages=pool.shape[0],
           pages_per_seq=pps, page_size=page_size)


def read_quantized(cache, name, indices, c, dtype=torch.bfloat16, *, scale_gather=None):
    """Gather + dequantize cached tokens -> dtype [B, S, kv_heads, head_dim].

    ``c`` needs ``kv_heads``, ``head_dim`` and ``cache_group`` (or ``group``).
    ``scale_gather`` ("indexed" / "rowwise") is validated; both reference
    methods give identical values, and the HIP kernel implements that value.
    """
    if scale_gather not in (None, "indexed", "rowwise"):
        raise ValueError("Scale gather method must be indexed or rowwise")
    codes = cache[name]
    plane = cache[name + "_scale"]
    heads, dim = c.kv_heads, c.head_dim
    group = _group_of(c)
    if codes.dtype != torch.int8 or codes.ndim != 3 or codes.shape[2] != heads * dim:
        raise ValueError("cache codes must be int8 [batch, time, kv_heads * head_dim]")
    batch, time, chans = codes.shape
    groups = chans // group
    if indices.ndim != 2 or plane.ndim != 2 or plane.shape[0] != indices.shape[0] * groups:
        raise ValueError("Scale plane must be [batch * groups, time] for [batch, selected] indices")
    if indices.shape[0] != batch or plane.shape[1] != time:
        raise ValueError("indices and the scale plane must match the cache's batch and time")
    if plane.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("scale plane must be BF16 or FP32")
    idx = indices.to(device=codes.device, dtype=torch.int32).contiguous()
    out = torch.empty((batch, idx.shape[1], heads, dim), dtype=dtype, device=codes.device)
    codes, plane = codes.contiguous(), plane.contiguous()
    a = _lib.KvArgs()
    a.codes, a.scales = codes.data_ptr(), plane.data_ptr()
    a.scale_dtype = _dtype_code(plane.dtype)
    a.scale_layout = 0
    a.indices = idx.data_ptr()
    a.batch, a.selected, a.capacity = batch, idx.shape[1], time
    a.kv_heads, a.head_dim, a.group = heads, dim, group
    a.out, a.out_dtype = out.data_ptr(), _dtype_code(dtype)
    _run(a, codes.device)
    return out


def read_paged(pool, scales, page_table, *, page_size, kv_heads, head_dim, group=None, indices=None,
               dtype=torch.bfloat16, out=None):
    """Paged cache -> dtype [B, S, kv_heads, head_dim].

    pool int8 [pages, page_size, kv_heads*head_dim]; scales [pages, page_size,
    kv_heads*head_dim/group] (FP32 or BF16); page_table int32 [B, pages_per_seq];
    indices int32 [B, S] or None for every token of every page.
    """
    group = head_dim if group is None else group
    if pool.dtype != torch.int8 or pool.ndim < 3 or pool.shape[1] != page_size:
        raise ValueError("pool must be int8 [pages, page_size, ...]")
    chans = kv_heads * head_dim
    if pool[0, 0].numel() != chans:
        raise ValueError("pool rows must hold kv_heads * head_dim codes")
    if scales[0, 0].numel() != chans // group:
        raise ValueError("scales must hold kv_heads * head_dim / group values per token")
    table = page_table.to(device=pool.device, dtype=torch.int32).contiguous()
    batch, pps = table.shape
    cap = pps * page_size
    idx = None if indices is None else indices.to(device=pool.device, dtype=torch.int32).contiguous()
    sel = cap if idx is None else idx.shape[1]
    if out is None:
        out = torch.empty((batch, sel, kv_heads, head_dim), dtype=dtype, device=pool.device)
    elif (not isinstance(out, torch.Tensor) or out.dtype not in (torch.bfloat16, torch.float32)
          or tuple(out.shape) != (batch, sel, kv_heads, head_dim) or out.device != pool.device
          or not out.is_contiguous()):
        raise ValueError(f"out must be a contiguous BF16 or FP32 [{batch}, {sel}, {kv_heads}, {head_dim}] tensor "
                         f"on {pool.device}")
    pool, scales = pool.contiguous(), scales.contiguous()
    a = _lib.KvArgs()
    a.codes, a.scales = pool.data_ptr(), scales.data_ptr()
    a.scale_dtype = _dtype_code(scales.dtype)
    a.scale_layout = 1
    a.page_table = table.data_ptr()
    a.pool_pages, a.pages_per_seq, a.page_size = pool.shape[0], pps, page_size
    a.indices = None if idx is None else idx.data_ptr()
    a.batch, a.selected, a.capacity = batch, sel, cap
    a.kv_heads, a.head_dim, a.group = kv_heads, head_dim, group
    a.out, a.out_dtype = out.data_ptr(), _dtype_code(out.dtype)
    _run(a, pool.device)
    return out


def paged_decode_attention(q, k_pool, k_scales, v_pool, v_scales, page_table, lengths, *, page_size, kv_heads,
                           workspace=None, out=None):
    """Decode attention over the paged INT8 cache with the dequant fused in
    (attention_cache.py:159-169 after read_quantized :71-81): q BF16 [B, Hq, 128]
    -> BF16 [B, Hq, 128], the attention output before the reference's gate and
    out projection. Pools int8 [pages, page_size, kv_heads*128], scales FP32
    [pages, page_size, kv_heads] (one per token and head), page_table int32
    [B, pages_per_seq], lengths int32 [B] attended tokens (the reference's
    position + 1). No BF16 copy of K or V is made.
    """
    head_dim = 128
    if q.dtype != torch.bfloat16 or q.ndim != 3 or q.shape[2] != head_dim:
        raise ValueError("q must be BF16 [batch, query_heads, 128]")
    for pool in (k_pool, v_pool):
        if pool.dtype != torch.int8 or pool.ndim < 3 or pool.shape[1] != page_size or \
                pool[0, 0].numel() != kv_heads * head_dim:
            raise ValueError("pools must be int8 [pages, page_size, kv_heads * 128]")
    for sc in (k_scales, v_scales):
        if sc.dtype != torch.float32 or sc.numel() != k_pool.shape[0] * page_size * kv_heads:
            raise ValueError("scales must be FP32 [pages, page_size, kv_heads]")
    batch, hq = q.shape[0], q.shape[1]
    table = page_table.to(device=q.device, dtype=torch.int32).contiguous()
    lens = lengths.to(device=q.device, dtype=torch.int32).contiguous()
    if table.shape[0] != batch or lens.shape != (batch,):
        raise ValueError("page_table must be [batch, pages_per_seq] and lengths [batch]")
    pps = table.shape[1]
    lib = _lib.load()
    need = int(lib.q6moe_attn_workspace_size(batch, hq, kv_heads, pps, page_size))
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    elif (not isinstance(workspace, torch.Tensor) or workspace.dtype != torch.uint8 or workspace.device != q.device
          or not workspace.is_contiguous() or workspace.numel() < need):
        raise ValueError(f"workspace must be a contiguous uint8 tensor of at least {need} bytes on {q.device}")
    q = q.contiguous()
    if out is None:
        out = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
    elif (not isinstance(out, torch.Tensor) or out.dtype != torch.bfloat16 or tuple(out.shape) != tuple(q.shape)
          or out.device != q.device or not out.is_contiguous()):
        raise ValueError(f"out must be a contiguous BF16 {list(q.shape)} tensor on {q.device}")
    k_pool, v_pool, k_scales, v_scales = (t.contiguous() for t in (k_pool, v_pool, k_scales, v_scales))
    a = _lib.AttnArgs()
    a.q, a.k_codes, a.v_codes = q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr()
    a.k_scales, a.v_scales = k_scales.data_ptr(), v_scales.data_ptr()
    a.page_table, a.lengths = table.data_ptr(), lens.data_ptr()
    a.batch, a.query_heads, a.kv_heads, a.head_dim = batch, hq, kv_heads, head_dim
    a.pool_pages, a.pages_per_seq, a.page_size = k_pool.shape[0], pps, page_size
    a.out = out.data_ptr()
    a.workspace, a.workspace_bytes = workspace.data_ptr(), workspace.numel()
    with torch.cuda.device(q.device):
        rc = lib.q6moe_kv_decode_attention(ctypes.byref(a), _lib.stream_handle(q.device))
    _lib.check(rc, "kv_decode_attention")
    return out


def gather_scale_plane(plane, indices, groups, *, method="indexed"):
    """[B*G, T] scale plane, [B, S] indices -> [B, S, G] (attention_cache.py:46-68),
    on the GPU (``q6moe_kv_gather_scales``). Both reference methods ("indexed",
    "rowwise") give the same values: a negative index adds T, then the index is
    clamped into [0, T)."""
    if indices.ndim != 2 or plane.ndim != 2 or plane.shape[0] != indices.shape[0] * groups:
        raise ValueError("Scale plane must be [batch * groups, time] for [batch, selected] indices")
    if method not in ("indexed", "rowwise"):
        raise ValueError("Scale gather method must be indexed or rowwise")
    if not isinstance(plane, torch.Tensor) or plane.device.type != "cuda":
        raise ValueError("plane must be a GPU tensor")
    batch, sel = indices.shape
    plane = plane.contiguous()
    idx = indices.to(device=plane.device, dtype=torch.int32).contiguous()
    out = torch.empty((batch, sel, groups), dtype=plane.dtype, device=plane.device)
    lib = _lib.load()
    with torch.cuda.device(plane.device):
        rc = lib.q6moe_kv_gather_scales(plane.data_ptr(), _dtype_code(plane.dtype), idx.data_ptr(), batch, sel,
                                        groups, plane.shape[1], out.data_ptr(), _lib.stream_handle(plane.device))
    _lib.check(rc, "kv_gather_scales")
    return out
