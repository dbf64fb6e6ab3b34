"""Streaming load of GGUF expert tensors into unit-major device tables.

The reference loads one expert projection at a time from the checkpoint
(``Checkpoint.resident_experts``, kaggle/qwen38_tpu/checkpoint.py:225-261):
it reads the tensor's bytes ([E, bytes_per_expert], GGUF blocks per row)
in expert groups through ``Checkpoint.read(name, offset, size)`` and places
each group on its device. ``stream_expert_table`` takes the same kind of
reader and streams the bytes in groups of experts through two pinned host
buffers: while the GPU copies group i and repacks it (``q6moe_moe_pack``)
straight into its slice of the unit-major table, the host reads group i+1.
Host staging is bounded by two groups; no full raw copy is made on either
side.
"""

import torch

from . import _lib
from .experts import SUPPORTED, ExpertTable
from .quant import BLOCK_LAYOUTS


def stream_expert_table(read, qtype, experts, rows, width, device=None, group_experts=8):
    """``read(offset, size)`` returns ``size`` bytes (any buffer-protocol object)
    of the GGUF tensor [experts, rows, width/values_per_block, block_bytes]
    starting at byte ``offset``. Returns the ExpertTable ``pack_experts`` would
    build from the whole tensor."""
    if qtype not in SUPPORTED:
        raise ValueError(f"expert tables must be one of {SUPPORTED}; got {qtype}")
    values, block = BLOCK_LAYOUTS[qtype]
    if width % values or experts < 1 or rows < 1 or group_experts < 1:
        raise ValueError("bad expert tensor shape")
    device = torch.device(device) if device is not None else torch.device("cuda")
    stride = rows * (width // values) * block  # raw bytes per expert
    lib = _lib.load()
    code = _lib.QTYPE_CODES[qtype]
    size = int(lib.q6moe_moe_table_bytes(code, rows, width))
    if size == 0:
        raise ValueError(f"cannot pack a {qtype} table of [{rows}, {width}]")
    g = min(group_experts, experts)
    table = torch.empty((experts, size), dtype=torch.uint8, device=device)
    host = [torch.empty(g * stride, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
    stage = [torch.empty(g * stride, dtype=torch.uint8, device=device) for _ in range(2)]
    done = [None, None]  # event after the group that last used buffer i was packed
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device)
        for i, e0 in enumerate(range(0, experts, g)):
            n = min(g, experts - e0)
            b = i % 2
            if done[b] is not None:
                done[b].synchronize()  # its previous copy and pack have finished
            chunk = read(e0 * stride, n * stride)
            view = memoryview(chunk).cast("B")
            if len(view) != n * stride:
                raise ValueError("read returned the wrong number of bytes")
            host[b][: n * stride].numpy()[:] = view
            stage[b][: n * stride].copy_(host[b][: n * stride], non_blocking=True)
            rc = lib.q6moe_moe_pack(_lib.ptr(stage[b]), code, n, rows, width, _lib.ptr(table[e0]),
                                    _lib.stream_handle(device))
            _lib.check(rc, "moe_pack")
            done[b] = torch.cuda.Event()
            done[b].record(stream)
        torch.cuda.current_stream(device).synchronize()
    return ExpertTable(qtype, table, None, rows, width)
