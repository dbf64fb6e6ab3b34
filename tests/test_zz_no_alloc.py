"""The no-allocation routed-FFN entry point ``q6moe_moe_forward_noalloc``
against ``q6moe_moe_forward``, through the C ABI.

The entry point takes the same arguments without a workspace and uses the
library's static per-device scratch instead. Its outputs must equal the
workspace entry point's bit for bit (the same kernels run on the same inputs),
on consecutive calls with shrinking inputs (the scratch keeps the previous
call's contents), on the decode and the grouped paths, and a call whose
regions exceed the scratch must be rejected with a message.
"""

import ctypes

import numpy as np
import pytest
import torch

from q6moe import _lib
from q6moe.experts import expert_parallel
from q6moe.synth import moe_layer

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20  # Q6MOE_NOALLOC_SCRATCH_BYTES


def _noalloc():
    return _lib.load().q6moe_moe_forward_noalloc


def _inputs(L, device, tokens):
    x = torch.from_numpy(L["x"][:tokens]).to(device).to(torch.bfloat16)
    ids = torch.from_numpy(L["ids"][:tokens]).to(device)
    w = torch.from_numpy(L["weights"][:tokens]).to(device).to(torch.bfloat16)
    return x, ids, w


def _both(fn, tabs, device, x, ids, w, mode, shared=None):
    fn = fn.with_mode(mode)
    want = fn(*tabs, x, ids, w, shared=shared)
    args, out, keep = fn.args(*tabs, x, ids, w, shared=shared, with_workspace=False)
    with torch.cuda.device(device):
        rc = _noalloc()(ctypes.byref(args), _lib.stream_handle(device))
    _lib.check(rc, "moe_forward_noalloc")
    torch.cuda.synchronize()
    del keep
    return want.view(torch.int16).cpu().numpy(), out.view(torch.int16).cpu().numpy()


def test_noalloc_matches_workspace_entry_point_on_consecutive_calls(device):
    # decode step (128 experts, top-8, H 2048, I 768, 8 tokens), then the same
    # layer with 3 tokens: the second call must not see the first one's scratch
    L = moe_layer(seed=1, pack=False)
    fn = expert_parallel(None, gate_type="Q6_K", up_type="Q6_K", down_type="Q6_K", hidden=2048, intermediate=768)
    tabs = fn.prepare(*(L[n].reshape(128, -1) for n in ("gate", "up", "down")), device)
    for tokens in (8, 3):
        want, got = _both(fn, tabs, device, *_inputs(L, device, tokens), mode=0)
        np.testing.assert_array_equal(got, want)


def test_noalloc_grouped_path_and_shared_expert(device):
    # the grouped (prefill-shaped) kernels at 200 then 70 tokens, and the decode
    # kernels with a shared expert and its device router gate
    L = moe_layer(seed=61, experts=16, top_k=4, hidden=512, intermediate=256, tokens=200, qtype="Q6_K",
                  shared_intermediate=512, pack=False)
    fn = expert_parallel(None, gate_type="Q6_K", up_type="Q6_K", down_type="Q6_K", hidden=512, intermediate=256)
    tabs = fn.prepare(*(L[n].reshape(16, -1) for n in ("gate", "up", "down")), device)
    sh = L["shared"]
    shared = {n: torch.from_numpy(sh[n].reshape(1, -1)).to(device) for n in ("gate", "up", "down")}
    shared["router"] = torch.from_numpy(np.random.default_rng(62).normal(0, 0.05, 512).astype(np.float32)).to(
        device).to(torch.bfloat16)
    for tokens, mode in ((200, 2), (70, 2), (16, 1), (5, 1)):
        want, got = _both(fn, tabs, device, *_inputs(L, device, tokens), mode=mode, shared=shared)
        np.testing.assert_array_equal(got, want)


def test_noalloc_rejects_calls_beyond_the_scratch(device):
    L = moe_layer(seed=63, experts=4, top_k=2, hidden=2048, intermediate=768, tokens=1, pack=False)
    fn = expert_parallel(None, gate_type="Q6_K", up_type="Q6_K", down_type="Q6_K", hidden=2048, intermediate=768)
    tabs = fn.prepare(*(L[n].reshape(4, -1) for n in ("gate", "up", "down")), device)
    tokens = 4096  # grouped path: activations and expert outputs alone exceed 32 MiB
    x = torch.zeros((tokens, 2048), dtype=torch.bfloat16, device=device)
    ids = torch.zeros((tokens, 2), dtype=torch.int32, device=device)
    w = torch.zeros((tokens, 2), dtype=torch.bfloat16, device=device)
    assert fn.workspace_bytes(tokens, 2, 4) > SCRATCH_BYTES
    args, out, keep = fn.args(*tabs, x, ids, w, with_workspace=False)
    with torch.cuda.device(device):
        rc = _noalloc()(ctypes.byref(args), _lib.stream_handle(device))
    assert rc == -1
    assert b"static scratch" in _lib.load().q6moe_last_error()
    # a caller workspace is refused: the entry point uses only its own scratch
    args.workspace, args.workspace_bytes = x.data_ptr(), 1 << 20
    with torch.cuda.device(device):
        rc = _noalloc()(ctypes.byref(args), _lib.stream_handle(device))
    assert rc == -1
    assert b"takes no workspace" in _lib.load().q6moe_last_error()
    del keep


@pytest.mark.parametrize("case", ["decode", "grouped", "thin"])
def test_noalloc_call_replays_in_a_captured_graph(device, case):
    # The entry point captured once in a HIP graph (after a first eager call on
    # the device), then replayed with new inputs written in place into the
    # captured x / ids / weights, with eager work of the program between the
    # replays: each replay must equal q6moe_moe_forward on the same inputs bit
    # for bit (decode kernels at 8 tokens; grouped kernels at 200 tokens).
    if case == "decode":
        E, H, I, B, mode = 128, 2048, 768, 8, 0
        L = moe_layer(seed=1, tokens=4 * B, pack=False)
    elif case == "thin":  # 512 experts, top-10, 8 tokens: the one-launch decode kernel and its call counter
        E, H, I, B, mode = 512, 512, 256, 8, 0
        L = moe_layer(seed=65, experts=E, top_k=10, hidden=H, intermediate=I, tokens=4 * B, pack=False)
    else:
        E, H, I, B, mode = 16, 512, 256, 200, 2
        L = moe_layer(seed=64, experts=E, top_k=4, hidden=H, intermediate=I, tokens=4 * B, pack=False)
    fn = expert_parallel(None, gate_type="Q6_K", up_type="Q6_K", down_type="Q6_K", hidden=H,
                         intermediate=I).with_mode(mode)
    tabs = fn.prepare(*(L[n].reshape(E, -1) for n in ("gate", "up", "down")), device)
    x, ids, w = (t.clone() for t in _inputs(L, device, B))
    args, out, keep = fn.args(*tabs, x, ids, w, with_workspace=False)
    call = _noalloc()
    with torch.cuda.device(device):
        assert call(ctypes.byref(args), _lib.stream_handle(device)) == 0  # first use on this device
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream(device)
    s.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.graph(g, stream=s):
        rc = call(ctypes.byref(args), _lib.stream_handle(device))
    torch.cuda.current_stream(device).wait_stream(s)
    assert rc == 0
    for r in range(1, 4):
        xs, ids_s, ws_ = _inputs(L, device, 4 * B)
        x.copy_(xs[r * B:(r + 1) * B])
        ids.copy_(ids_s[r * B:(r + 1) * B])
        w.copy_(ws_[r * B:(r + 1) * B])
        g.replay()
        torch.cuda.synchronize()
        got = out.view(torch.int16).cpu().numpy()
        want = fn(*tabs, x, ids, w).view(torch.int16).cpu().numpy()  # eager, with a workspace
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got, want)
        assert not np.array_equal(got, np.zeros_like(got))
    del keep
