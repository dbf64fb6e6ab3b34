"""Routed SwiGLU expert FFN over packed experts: ``expert_parallel``.

Mirrors the factory of kaggle/qwen38_tpu/experts.py:17-140 (and
grouped_experts.py:21-163): same keywords, validation messages and returned
callable ``fn(gate, up, down, x, ids, weights) -> x.dtype [B, hidden]``, with
the numerics contract of the reference (BF16 weights decoded exactly, FP32
accumulation, BF16 rounding of g, u, silu(g), the SwiGLU product and the
down output, FP32 weighted sum over experts in ascending id, BF16 result).

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
only) once and cached per tensor version.
"""

import ctypes
from dataclasses import dataclass
from functools import lru_cache

import numpy as np
import torch

from . import _lib
from .quant import BLOCK_LAYOUTS

EXPERT_ROW_TILE = 128
SUPPORTED = ("Q6_K", "Q4_K", "Q8_0")  # tables pack_experts takes
GATE_UP_TYPES = ("Q6_K", "Q4_K")       # gate/up types the kernels run; down is that type or Q8_0


@dataclass(frozen=True)
class ExpertTable:
    """One projection for all experts, resident on the GPU.

    ``data`` [E, q6moe_moe_table_bytes] unit-major tables (Q6_K or Q4_K); the
    scales live inside the units, so ``scales`` is None.
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


def stacked_table(data, qtype, rows, width):
    """Wrap an already-packed device table [E, q6moe_moe_table_bytes] (from ``q6moe_moe_pack``)."""
    return ExpertTable(qtype, data, None, rows, width)


class _PackCache:
    """Device repack of raw GGUF expert tables, keyed by (pointer, version, shape)."""

    def __init__(self):
        self.entries = {}

    def get(self, raw, qtype, rows, width):
        key = (raw.data_ptr(), raw._version, tuple(raw.shape), qtype, rows, width)
        hit = self.entries.get(key)
        if hit is None:
            if len(self.entries) > 16:
                self.entries.clear()
            hit = self.entries[key] = pack_experts(raw, qtype, rows, width, raw.device)
        return hit


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


class ExpertFFN:
    """Callable returned by ``expert_parallel``."""

    def __init__(self, qtype, hidden, intermediate, mode=0, down_qtype=None):
        self.qtype = qtype
        self.down_qtype = down_qtype or qtype
        self.hidden = hidden
        self.intermediate = intermediate
        self.mode = mode

    def workspace_bytes(self, tokens, top_k, experts, shared_intermediate=0):
        return int(_lib.load().q6moe_moe_workspace_size(
            tokens, top_k, experts, self.hidden, self.intermediate, shared_intermediate))

    def __call__(self, gate, up, down, x, ids, weights, *, shared=None, workspace=None, out=None,
                 events=None):
        """``events``: optional 5 timing events (torch.cuda.Event, already
        recorded once so they exist) stamped before routing, after routing,
        after gate/up, after down and after the combine."""
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
            sg, su, sd = shared["gate"], shared["up"], shared["down"]
            Is = sg.rows
            sg = _as_table(sg, q, Is, H, "shared gate")
            su = _as_table(su, q, Is, H, "shared up")
            sd = _as_table(sd, qd, H, Is, "shared down")
            args.shared_gate, args.shared_up, args.shared_down = sg.c_table(), su.c_table(), sd.c_table()
            args.shared_intermediate = Is
            scale = shared.get("scale")
            if scale is not None:
                scale = scale.to(device=x.device, dtype=torch.bfloat16).contiguous()
                if scale.numel() != B:
                    raise ValueError("shared scale must hold one BF16 value per token")
                keep.append(scale)
                args.shared_scale = scale.data_ptr()
        need = self.workspace_bytes(B, K, experts, Is)
        if workspace is None or workspace.numel() < need:
            workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
        out = torch.empty((B, H), dtype=torch.bfloat16, device=x.device) if out is None else out
        args.out = out.data_ptr()
        args.workspace = workspace.data_ptr()
        args.workspace_bytes = workspace.numel()
        args.mode = self.mode
        if events is not None:
            if len(events) != 5:
                raise ValueError("events must hold 5 timing events")
            handles = (ctypes.c_void_p * 5)(*[ctypes.c_void_p(ev.cuda_event) for ev in events])
            keep.append(handles)
            args.events = ctypes.cast(handles, ctypes.POINTER(ctypes.c_void_p))
        lib = _lib.load()
        with torch.cuda.device(x.device):
            rc = lib.q6moe_moe_forward(ctypes.byref(args), _lib.stream_handle(x.device))
        _lib.check(rc, "moe_forward")
        return out


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
    if gate_type != up_type or gate_type not in GATE_UP_TYPES or down_type not in (gate_type, "Q8_0"):
        raise NotImplementedError(
            f"this build runs Q6_K or Q4_K gate/up with down of the same type or Q8_0; got "
            f"{gate_type}/{up_type}/{down_type}"
        )
    if compute == "int8_q8":
        raise NotImplementedError("the int8_q8 (W8A8) policy is not part of this build")
    return ExpertFFN(gate_type, hidden, intermediate, down_qtype=down_type)


def grouped_expert_parallel(mesh=None, *, gate_type, up_type, down_type, hidden, intermediate,
                            compute="bf16", row_tile=128, group_size=4):
    """grouped_experts.py:21-163: same values as ``expert_parallel`` on one GPU."""
    if type(row_tile) is not int or row_tile < 1:
        raise ValueError("Expert row tile must be a positive integer")
    return expert_parallel(mesh, gate_type=gate_type, up_type=up_type, down_type=down_type,
                           hidden=hidden, intermediate=intermediate, compute=compute,
                           row_tile=row_tile, group_size=group_size)
