"""Routed SwiGLU expert FFN over packed experts: ``expert_parallel``.

Mirrors the factory of kaggle/qwen38_tpu/experts.py:17-140 (and
grouped_experts.py:21-163): same keywords, validation messages and returned
callable ``fn(gate, up, down, x, ids, weights) -> x.dtype [B, hidden]``, with
the numerics contract of the reference (BF16 weights decoded exactly, FP32
accumulation, BF16 rounding of g, u, silu(g), the SwiGLU product and the
down output, FP32 weighted sum over experts in ascending id, BF16 result).

``compute="int8_q8"`` runs the Q8_0 projections W8A8 on the INT8 matrix
cores, as the reference's ``q8_matmul`` (compute.py:20-34, experts.py:85-101);
other projections stay BF16.

One GPU holds every expert, so ``mesh``, ``group_size`` and
``tensor_parallel`` do not change the computation (the reference's grouped
and tensor-parallel variants are defined to produce the same values); they
are validated the way the reference validates them. All device work is HIP:
``q6moe_moe_forward`` in libq6moe.so (route sort, fused gate/up + SwiGLU,
down projection, deterministic combine).

Expert tables are either ``ExpertTable`` objects from ``pack_experts`` or, as
in the reference, raw GGUF byte tables ``uint8 [E, bytes_per_expert]`` on the
GPU; raw tables are repacked on the device to the unit-major layout of the
kernels (16 rows x one 256-wide K block per contiguous unit, bytes permuted
only) once per live tensor object and version, and the packed copy is freed
with the raw tensor.
"""

import ctypes
import warnings
import weakref
from dataclasses import dataclass
from functools import lru_cache

import numpy as np
import torch

from . import _lib
from .quant import BLOCK_LAYOUTS

EXPERT_ROW_TILE = 128
SUPPORTED = ("Q6_K", "Q5_K", "Q4_K", "Q8_0", "Q5_1")  # tables pack_experts takes
GATE_UP_TYPES = ("Q6_K", "Q5_K", "Q4_K", "Q8_0")       # gate/up types the kernels run; down: any of SUPPORTED


@dataclass(frozen=True)
class ExpertTable:
    """One projection for all experts, resident on the GPU.

    ``data`` [E, q6moe_moe_table_bytes] unit-major tables (Q6_K, Q5_K, Q4_K,
    Q8_0 or Q5_1); the scales live inside the units, so ``scales`` is None.
    """

    qtype: str
    data: torch.Tensor
    scales: object
    rows: int
    width: int

    @property
    def experts(self):
        return self.data.shape[0]

    def c_table(self):
        t = _lib.Table()
        t.qtype = _lib.QTYPE_CODES[self.qtype]
        t.data = self.data.data_ptr()
        t.data_stride = self.data.stride(0) if self.data.ndim > 1 else 0
        if self.scales is not None:
            t.scales = self.scales.data_ptr()
            t.scale_stride = self.scales.stride(0) if self.scales.ndim > 1 else 0
        return t

    def nbytes(self):
        return self.data.numel() + (0 if self.scales is None else self.scales.numel())


def _raw_view(raw, qtype, rows, width):
    values, size = BLOCK_LAYOUTS[qtype]
    blocks = (width + values - 1) // values
    experts = raw.shape[0]
    if raw.numel() != experts * rows * blocks * size:
        raise ValueError(f"{qtype} table must hold [experts, {rows}, {blocks}, {size}] bytes per expert")
    return raw.reshape(experts, rows, blocks, size)


def pack_experts(raw, qtype, rows, width, device=None):
    """GGUF expert table [E, rows, blocks, bytes] (or [E, bytes]) -> ExpertTable on the GPU."""
    if qtype not in SUPPORTED:
        raise ValueError(f"expert tables must be one of {SUPPORTED}; got {qtype}")
    if isinstance(raw, np.ndarray):
        if raw.dtype != np.uint8:
            raise TypeError("expert tables must have dtype uint8")
        raw = torch.from_numpy(np.ascontiguousarray(raw))
    if raw.dtype != torch.uint8:
        raise TypeError("expert tables must have dtype uint8")
    device = torch.device(device) if device is not None else (raw.device if raw.is_cuda else torch.device("cuda"))
    raw = _raw_view(raw.to(device), qtype, rows, width).contiguous()
    experts = raw.shape[0]
    lib = _lib.load()
    code = _lib.QTYPE_CODES[qtype]
    size = int(lib.q6moe_moe_table_bytes(code, rows, width))
    if size == 0:
        raise ValueError(f"cannot pack a {qtype} table of [{rows}, {width}]")
    data = torch.empty((experts, size), dtype=torch.uint8, device=device)
    with torch.cuda.device(device):
        rc = lib.q6moe_moe_pack(_lib.ptr(raw), code, experts, rows, width, _lib.ptr(data), _lib.stream_handle(device))
        _lib.check(rc, "moe_pack")
    return ExpertTable(qtype, data, None, rows, width)


UNPACK_PATHS = {"generic": 0, "decode": 1, "prefill": 2}


def unpack_experts(table, path="generic"):
    """Decode a unit-major ExpertTable back to BF16 [E, rows, width] with the
    decoder one family of MoE kernels uses (``path``: "generic", "decode" or
    "prefill"), through ``q6moe_moe_unpack``: each weight is RNE_bf16 of its
    GGUF value, as ``dequantize_rows(..., dtype=bfloat16)`` gives it
    (gguf_quant.py:111-173); Q6_K weights with code 32 come out as +0."""
    if not isinstance(table, ExpertTable):
        raise TypeError("unpack_experts takes an ExpertTable")
    data = table.data
    out = torch.empty((table.experts, table.rows, table.width), dtype=torch.bfloat16, device=data.device)
    lib = _lib.load()
    with torch.cuda.device(data.device):
        rc = lib.q6moe_moe_unpack(_lib.ptr(data), _lib.QTYPE_CODES[table.qtype], table.experts, table.rows,
                                  table.width, data.stride(0), UNPACK_PATHS[path], _lib.ptr(out),
                                  _lib.stream_handle(data.device))
    _lib.check(rc, "moe_unpack")
    return out


def stacked_table(data, qtype, rows, width):
    """Wrap an already-packed device table [E, q6moe_moe_table_bytes] (from ``q6moe_moe_pack``)."""
    return ExpertTable(qtype, data, None, rows, width)


class _PackCache:
    """Device repack of raw GGUF expert tables, one entry per live tensor.

    An entry belongs to the tensor object it was made from: it is found by
    that object's identity and removed by a finaliser when the object is
    freed, so a later table that the caching allocator places at the same
    address never sees another table's packed bytes. The entry also records
    the tensor's version counter, pointer, shape and strides, and is rebuilt
    when any of them changes (an in-place update). Entries live exactly as
    long as their raw tables, whatever their number: a 48-layer model that
    passes the same 144 table objects on every call packs each one once.
    A view made afresh on every call (``table[layer]`` inside the layer loop)
    is a new object each time and is repacked each time; pass the same
    object, or pack once at load time with ``pack_experts`` /
    ``ExpertFFN.prepare``. While an entry lives, the raw bytes and the packed
    copy are both held (at the reference model's size, 512 experts x 4.43 MB
    per layer): the first repack of a process issues a ResourceWarning that
    says so.
    """

    def __init__(self):
        self.entries = {}
        self.warned = False  # one ResourceWarning per process for the doubled memory

    def get(self, raw, qtype, rows, width, single=False):
        """``single``: ``raw`` is one projection [rows, blocks, bytes], packed as one expert."""
        key = id(raw)
        sig = (raw._version, raw.data_ptr(), tuple(raw.shape), tuple(raw.stride()), qtype, rows, width, single)
        hit = self.entries.get(key)
        if hit is not None and hit[0] == sig:
            return hit[1]
        table = pack_experts(raw.reshape(1, -1) if single else raw, qtype, rows, width, raw.device)
        if hit is None:
            weakref.finalize(raw, self.entries.pop, key, None)
            if not self.warned:
                self.warned = True
                warnings.warn(
                    f"a raw GGUF expert table ({raw.numel()} bytes) was repacked on the device for this call; the "
                    "packed copy lives as long as the raw tensor, so the layer's expert memory is held twice. "
                    "Pack once at load time (ExpertFFN.prepare / pack_experts) and pass the packed tables, "
                    "or free the raw tensor.", ResourceWarning, stacklevel=4)
        self.entries[key] = (sig, table)
        return table

    def __len__(self):
        return len(self.entries)


_CACHE = _PackCache()


def _as_table(t, qtype, rows, width, name):
    if isinstance(t, ExpertTable):
        if t.qtype != qtype or t.rows != rows or t.width != width:
            raise ValueError(f"{name} table holds {t.qtype} [{t.rows}, {t.width}], expected {qtype} [{rows}, {width}]")
        if t.data.device.type != "cuda":
            raise ValueError("expert tables must be on a GPU device")
        return t
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise ValueError(f"{name} must be an ExpertTable or a uint8 GPU tensor [experts, bytes]")
    if t.dtype != torch.uint8:
        raise TypeError("expert tables must have dtype uint8")
    return _CACHE.get(t, qtype, rows, width)


def _rows_of(t, qtype, width):
    """Output rows of one expert's projection: an ExpertTable's, or those a raw
    GGUF table [1, bytes] (or [rows, blocks, bytes]) of row width ``width`` holds."""
    if isinstance(t, ExpertTable):
        return t.rows
    values, size = BLOCK_LAYOUTS[qtype]
    per_row = -(-width // values) * size
    n = t.numel() // (t.shape[0] if t.ndim in (2, 4) else 1)
    if n % per_row:
        raise ValueError(f"shared expert table does not hold whole {qtype} rows of width {width}")
    return n // per_row


def _check_bf16_out(out, shape, device, name="out"):
    if out is None:
        return torch.empty(shape, dtype=torch.bfloat16, device=device)
    if (not isinstance(out, torch.Tensor) or out.dtype != torch.bfloat16 or tuple(out.shape) != tuple(shape)
            or out.device != device or not out.is_contiguous()):
        raise ValueError(f"{name} must be a contiguous BF16 {list(shape)} tensor on {device}")
    return out


def _check_workspace(workspace, need, device):
    if workspace is None:
        return torch.empty(need, dtype=torch.uint8, device=device)
    if (not isinstance(workspace, torch.Tensor) or workspace.dtype != torch.uint8 or workspace.device != device
            or not workspace.is_contiguous()):
        raise ValueError(f"workspace must be a contiguous uint8 tensor on {device}")
    if workspace.numel() < need:
        raise ValueError(f"workspace holds {workspace.numel()} bytes; this call needs {need}")
    return workspace


MODES = (0, 1, 2)  # kernel family: by token count, decode-step kernels, grouped (prefill) kernels


class ExpertFFN:
    """Callable returned by ``expert_parallel``.

    ``expert_parallel`` caches its result, so one object serves every caller
    with the same configuration; it holds no per-call state. ``mode`` picks the
    kernel family: 0 (the default) the decode-step kernels up to 64 tokens
    (without a shared expert, only while tokens x top-k x experts < 2^17) and
    the grouped ones otherwise, 1 always the decode-step kernels, 2 always the
    grouped kernels. ``with_mode`` returns a copy that runs another family.
    """

    def __init__(self, qtype, hidden, intermediate, mode=0, down_qtype=None, compute="bf16"):
        if mode not in MODES:
            raise ValueError(f"mode must be one of {MODES}")
        self.qtype = qtype
        self.down_qtype = down_qtype or qtype
        self.hidden = hidden
        self.intermediate = intermediate
        self._mode = mode
        self.compute = compute

    @property
    def mode(self):
        return self._mode

    def with_mode(self, mode):
        """This FFN with the kernel family ``mode`` (0, 1 or 2)."""
        return ExpertFFN(self.qtype, self.hidden, self.intermediate, mode, self.down_qtype, self.compute)

    def workspace_bytes(self, tokens, top_k, experts, shared_intermediate=0):
        return int(_lib.load().q6moe_moe_workspace_size(
            tokens, top_k, experts, self.hidden, self.intermediate, shared_intermediate))

    def prepare(self, gate, up, down, device=None):
        """Pack a layer's raw GGUF tables ([E, bytes_per_expert] uint8, host or
        GPU) once, at load time: returns the (gate, up, down) ExpertTables that
        calls take in place of the raw tables, so no call ever repacks."""
        H, I = self.hidden, self.intermediate
        return (pack_experts(gate, self.qtype, I, H, device), pack_experts(up, self.qtype, I, H, device),
                pack_experts(down, self.down_qtype, H, I, device))

    def __call__(self, gate, up, down, x, ids, weights, *, shared=None, workspace=None, out=None,
                 events=None):
        """Routed FFN of x [B, hidden] BF16 through ``q6moe_moe_forward``; see ``args``."""
        args, out, keep = self.args(gate, up, down, x, ids, weights, shared=shared, workspace=workspace, out=out,
                                    events=events)
        lib = _lib.load()
        with torch.cuda.device(x.device):
            rc = lib.q6moe_moe_forward(ctypes.byref(args), _lib.stream_handle(x.device))
        _lib.check(rc, "moe_forward")
        del keep
        return out

    def args(self, gate, up, down, x, ids, weights, *, shared=None, workspace=None, out=None, events=None,
             with_workspace=True):
        """The ``q6moe_moe_args`` of one call, its output tensor and the tensors
        the arguments point into (keep them alive until the call is issued).

        Routed FFN of x [B, hidden] BF16 with ids/weights [B, top_k].

        ``shared`` adds the always-on shared expert (engine.py:199-203,
        math.py:282-283): a dict with ``gate``, ``up`` (rows = shared
        intermediate) and ``down`` tables, and optionally either ``router``
        (BF16 [hidden]: the output is scaled per token by
        RNE(sigmoid(RNE(x . router))), computed on the GPU) or ``scale``
        (BF16 [B], that per-token factor precomputed by the caller).
        ``out`` (BF16 [B, hidden]) and ``workspace`` (uint8, at least
        ``workspace_bytes(...)``) are optional preallocated buffers on x's
        device. ``events``: optional 5 timing events (torch.cuda.Event,
        already recorded once so they exist) stamped before routing, after
        routing, after gate/up, after down and after the combine."""
        H, I, q, qd = self.hidden, self.intermediate, self.qtype, self.down_qtype
        gate = _as_table(gate, q, I, H, "gate")
        up = _as_table(up, q, I, H, "up")
        down = _as_table(down, qd, H, I, "down")
        experts = gate.experts
        if up.experts != experts or down.experts != experts:
            raise ValueError("gate, up and down must hold the same number of experts")
        if not isinstance(x, torch.Tensor) or x.device.type != "cuda":
            raise ValueError("x must be a GPU tensor")
        if x.dtype != torch.bfloat16 or x.ndim != 2 or x.shape[1] != H or x.shape[0] < 1:
            raise ValueError(f"x must be a nonempty BF16 [tokens, {H}] tensor")
        if ids.ndim != 2 or ids.shape[0] != x.shape[0] or tuple(weights.shape) != tuple(ids.shape):
            raise ValueError("ids and weights must both be [tokens, top_k]")
        if weights.dtype != x.dtype:
            raise ValueError("routing weights must have x's dtype (BF16)")
        B, K = ids.shape
        x = x.contiguous()
        ids = ids.to(device=x.device, dtype=torch.int32).contiguous()
        weights = weights.to(x.device).contiguous()
        args = _lib.MoeArgs()
        args.gate, args.up, args.down = gate.c_table(), up.c_table(), down.c_table()
        args.experts, args.hidden, args.intermediate = experts, H, I
        args.x, args.ids, args.weights = x.data_ptr(), ids.data_ptr(), weights.data_ptr()
        args.tokens, args.top_k = B, K
        Is = 0
        keep = []
        if shared is not None:
            Is = int(shared.get("intermediate") or _rows_of(shared["gate"], q, H))
            sg = _as_table(shared["gate"], q, Is, H, "shared gate")
            su = _as_table(shared["up"], q, Is, H, "shared up")
            sd = _as_table(shared["down"], qd, H, Is, "shared down")
            args.shared_gate, args.shared_up, args.shared_down = sg.c_table(), su.c_table(), sd.c_table()
            args.shared_intermediate = Is
            scale, router = shared.get("scale"), shared.get("router")
            if scale is not None and router is not None:
                raise ValueError("give the shared expert either a router or a precomputed scale, not both")
            if scale is not None:
                scale = scale.to(device=x.device, dtype=torch.bfloat16).contiguous()
                if scale.numel() != B:
                    raise ValueError("shared scale must hold one BF16 value per token")
                keep.append(scale)
                args.shared_scale = scale.data_ptr()
            if router is not None:
                if not isinstance(router, torch.Tensor) or router.dtype != torch.bfloat16 or router.numel() != H:
                    raise ValueError(f"shared router must be a BF16 [{H}] tensor")
                router = router.to(x.device).contiguous()
                keep.append(router)
                args.shared_router = router.data_ptr()
        if with_workspace:
            need = self.workspace_bytes(B, K, experts, Is)
            workspace = _check_workspace(workspace, need, x.device)
            keep.append(workspace)
            args.workspace = workspace.data_ptr()
            args.workspace_bytes = workspace.numel()
        out = _check_bf16_out(out, (B, H), x.device)
        args.out = out.data_ptr()
        args.mode = self.mode
        args.compute = 1 if self.compute == "int8_q8" else 0
        if events is not None:
            if len(events) != 5:
                raise ValueError("events must hold 5 timing events")
            handles = (ctypes.c_void_p * 5)(*[ctypes.c_void_p(ev.cuda_event) for ev in events])
            keep.append(handles)
            args.events = ctypes.cast(handles, ctypes.POINTER(ctypes.c_void_p))
        keep += [x, ids, weights, gate, up, down]
        return args, out, keep


@lru_cache(maxsize=32)
def expert_parallel(
    mesh=None,
    *,
    gate_type,
    up_type,
    down_type,
    hidden,
    intermediate,
    compute="bf16",
    row_tile=EXPERT_ROW_TILE,
    group_size=1,
    tensor_parallel=1,
):
    """Return the routed FFN ``fn(gate, up, down, x, ids, weights)`` (experts.py:17-140)."""
    del mesh
    if compute not in {"bf16", "int8_q8"}:
        raise ValueError("Unknown expert compute policy")
    if row_tile is not None and (type(row_tile) is not int or row_tile < 1):
        raise ValueError("Expert row tile must be a positive integer or None")
    if type(group_size) is not int or group_size < 1:
        raise ValueError("Expert group size must be a positive integer")
    if type(tensor_parallel) is not int or tensor_parallel < 1:
        raise ValueError("Tensor parallel size must divide the device count")
    if intermediate % tensor_parallel or (intermediate // tensor_parallel) % BLOCK_LAYOUTS[down_type][0]:
        raise ValueError("Tensor slices must contain whole down quantization blocks")
    if gate_type != up_type or gate_type not in GATE_UP_TYPES or down_type not in SUPPORTED:
        raise NotImplementedError(
            f"this build runs gate/up of one type in {GATE_UP_TYPES} with down in {SUPPORTED}; got "
            f"{gate_type}/{up_type}/{down_type}"
        )
    return ExpertFFN(gate_type, hidden, intermediate, down_qtype=down_type, compute=compute)


def grouped_expert_parallel(mesh=None, *, gate_type, up_type, down_type, hidden, intermediate,
                            compute="bf16", row_tile=128, group_size=4):
    """grouped_experts.py:21-163: same values as ``expert_parallel`` on one GPU."""
    if type(row_tile) is not int or row_tile < 1:
        raise ValueError("Expert row tile must be a positive integer")
    return expert_parallel(mesh, gate_type=gate_type, up_type=up_type, down_type=down_type,
                           hidden=hidden, intermediate=intermediate, compute=compute,
                           row_tile=row_tile, group_size=group_size)
