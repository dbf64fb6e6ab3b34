#!/usr/bin/env python3
"""Benchmark of the packed-Q6 routed-expert decode step on one MI355X.

Workload (default): one MoE expert-FFN decode step with Q6_K experts --
128 experts, top-8 routing, hidden 2048, expert intermediate 768, SwiGLU,
8 tokens, weights N(0, 0.02) quantized to Q6_K, x N(0, 1) BF16, router
logits N(0, 1) -> softmax -> top-8 -> renormalised BF16 weights, seed 1.

A step is one call of the routed FFN (route sort, fused gate/up + SwiGLU,
down projection, combine). Steps rotate over ``--layers`` copies of the
layer's expert tables at distinct HBM addresses (default 4: about 0.8 GB of
active expert bytes per rotation, over 3x the 256 MB Infinity Cache), so the
weights stream from HBM. The metric is algorithmic bytes per step (active
experts' packed weights + activations + routing inputs + output) / time.

Output: one JSON line (rank 0) with the ``roofline`` of the dominant kernel
(moe_dec_gate_up_kernel, timed with HIP events on the stream it runs on), the
``cpu_baseline`` (the NumPy oracle on this host, one step, one thread) and a
``prefill`` block: the same layer shapes with 4096 tokens, skewed routing
(per-expert logit bias N(0, 0.5)), seed 2, whose FLOPs (2 * 4096 * 8 * 3 *
2048 * 768) over the step time give TFLOP/s against the 2.5 PFLOP/s dense
BF16 MFMA peak.
"""

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "data-synth-tpu_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "Q6 expert-GEMM HBM GB/s (decode) + TFLOP/s (prefill), % of MI355X roofline"
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0
EXPERTS, TOP_K, HIDDEN, INTER, TOKENS, SEED = 128, 8, 2048, 768, 8, 1
PREFILL_TOKENS, PREFILL_SEED, PREFILL_BIAS = 4096, 2, 0.5
PREFILL_FLOPS = 2 * PREFILL_TOKENS * TOP_K * 3 * HIDDEN * INTER
Q6_PROJ_BYTES = 768 * 8 * 210  # one 768x2048 (or 2048x768) Q6_K projection: 210 bytes per 256 weights
# L2-to-fabric bytes per launch measured with rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE over this script, scaled by a 512 MiB device copy in the same run
# (profiles/moe_q6k_e128_top8_h2048_i768__hbm_bytes.txt); they change only
# when the kernels do and are re-measured with them.
TRAFFIC_BYTES = {"moe_dec_gate_up_kernel": 129_900_000, "moe_pf_gate_up_kernel": 644_420_000}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def step_bytes(active, routes):
    """Algorithmic HBM bytes of one decode step (each needed byte once)."""
    weights = active * 3 * Q6_PROJ_BYTES
    x = TOKENS * HIDDEN * 2
    out = TOKENS * HIDDEN * 2
    routing = TOKENS * TOP_K * (4 + 2)
    return weights + x + out + routing


def gate_up_bytes(active, routes):
    """Algorithmic bytes of one moe_dec_gate_up_kernel launch: gate+up of the active
    experts, the token activations it reads and the SwiGLU rows it writes."""
    return active * 2 * Q6_PROJ_BYTES + TOKENS * HIDDEN * 2 + routes * INTER * 2


def measure_prefill(dev, steps, warmup):
    """Prefill step (routing, gate/up, down, combine) on the seed-2 4096-token layer."""
    import numpy as np
    import torch

    from q6moe.experts import expert_parallel, pack_experts
    from q6moe.synth import moe_layer

    L = moe_layer(seed=PREFILL_SEED, experts=EXPERTS, top_k=TOP_K, hidden=HIDDEN, intermediate=INTER,
                  tokens=PREFILL_TOKENS, bias_sigma=PREFILL_BIAS, pack=False)
    tabs = [pack_experts(L[n], "Q6_K", INTER if n != "down" else HIDDEN, HIDDEN if n != "down" else INTER, dev)
            for n in ("gate", "up", "down")]
    x = torch.from_numpy(L["x"]).to(dev).to(torch.bfloat16)
    ids = torch.from_numpy(L["ids"]).to(dev)
    w = torch.from_numpy(L["weights"]).to(dev).to(torch.bfloat16)
    fn = expert_parallel(None, gate_type="Q6_K", up_type="Q6_K", down_type="Q6_K", hidden=HIDDEN,
                         intermediate=INTER)
    ws = torch.empty(fn.workspace_bytes(PREFILL_TOKENS, TOP_K, EXPERTS), dtype=torch.uint8, device=dev)
    out = torch.empty((PREFILL_TOKENS, HIDDEN), dtype=torch.bfloat16, device=dev)
    for _ in range(warmup):
        fn(*tabs, x, ids, w, workspace=ws, out=out)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        fn(*tabs, x, ids, w, workspace=ws, out=out)
    b.record()
    torch.cuda.synchronize()
    step_us = a.elapsed_time(b) / steps * 1e3
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in range(steps)]
    for row in evs:
        for ev in row:
            ev.record()
    torch.cuda.synchronize()
    for i in range(steps):
        fn(*tabs, x, ids, w, workspace=ws, out=out, events=evs[i])
    torch.cuda.synchronize()
    ph = np.array([[row[j].elapsed_time(row[j + 1]) for j in range(4)] for row in evs]).mean(0) * 1e3
    gu_flops = PREFILL_FLOPS * 2 / 3
    gu_tflops = gu_flops / (ph[1] * 1e-6) / 1e12
    tflops = PREFILL_FLOPS / (step_us * 1e-6) / 1e12
    return {
        "workload": "moe_prefill_q6k_e128_top8_h2048_i768_t4096_skew0.5",
        "value": round(tflops, 1),
        "unit": "TFLOP/s",
        "us_per_step": round(step_us, 1),
        "mfma_fraction": round(tflops / MFMA_PEAK_TFLOPS, 4),
        "flops_per_step": PREFILL_FLOPS,
        "phases_us": {k: round(float(v), 1) for k, v in zip(("route", "gate_up", "down", "combine"), ph)},
        "roofline": {
            "kernel": "moe_pf_gate_up_kernel",
            "bound": "mfma",
            "achieved": round(gu_tflops, 1),
            "peak": MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(gu_tflops / MFMA_PEAK_TFLOPS, 4),
            "traffic": TRAFFIC_BYTES["moe_pf_gate_up_kernel"],
            "flops_per_launch": int(gu_flops),
            "avg_launch_us": round(float(ph[1]), 1),
        },
    }


def _time_calls(fn, calls, warmup=3):
    """Mean device time (us) of ``calls`` back-to-back invocations of fn(i)."""
    import torch

    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(calls):
        fn(i)
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / calls * 1e3


def measure_projection(dev):
    """Single packed-Q6 projection, x bf16 [8, 2048] x W [2048 -> 768], seed 0, BF16 output.
    Hot: the same 1.3 MB weights every call (us per call, cache-resident). Cold:
    640 distinct weight copies (826 MB, over 3x the Infinity Cache) in rotation."""
    import torch

    from q6moe import pack_q6
    from q6moe.kernel import q6_matmul
    from q6moe.synth import projection

    w = projection(seed=0)
    packed = pack_q6(w["raw"], 2048)
    data = torch.from_numpy(packed.data).to(dev)
    scales = torch.from_numpy(packed.scales).to(dev)
    x = torch.from_numpy(w["x"]).to(dev).to(torch.bfloat16)
    hot = _time_calls(lambda i: q6_matmul(x, data, scales, output_features=768, out_dtype=torch.bfloat16), 200)
    copies = 640
    datas = data.repeat(copies, 1)
    scaless = scales.repeat(copies, 1)
    cold = _time_calls(lambda i: q6_matmul(x, datas[i % copies], scaless[i % copies], output_features=768,
                                           out_dtype=torch.bfloat16), copies)
    nbytes = 1_290_240 + 32_768 + 12_288
    return {"workload": "q6_projection_x8x2048_w2048to768", "hot_us_per_call": round(hot, 2),
            "cold_us_per_call": round(cold, 2), "cold_GBps": round(nbytes / (cold * 1e-6) / 1e9, 1),
            "bytes_per_call": nbytes, "cold_copies": copies}


def measure_q4_shared(dev):
    """Q4_K decode with an always-on shared expert: 64 experts, top-6, H 4096, I 1024,
    shared I 4096, N(0, 0.015), seed 3; tokens 1, 8, 64. The routed and shared weight tables
    rotate over enough copies that the active bytes of one rotation exceed 3x the Infinity
    Cache."""
    import numpy as np
    import torch

    from q6moe.experts import expert_parallel, pack_experts
    from q6moe.synth import moe_layer

    H4, I4, E4, K4, IS = 4096, 1024, 64, 6, 4096
    L = moe_layer(seed=3, experts=E4, top_k=K4, hidden=H4, intermediate=I4, tokens=64, sigma=0.015,
                  qtype="Q4_K", shared_intermediate=IS, pack=False)
    sh = L["shared"]
    base = [pack_experts(L[n], "Q4_K", I4 if n != "down" else H4, H4 if n != "down" else I4, dev)
            for n in ("gate", "up", "down")]
    base += [pack_experts(sh["gate"][None], "Q4_K", IS, H4, dev), pack_experts(sh["up"][None], "Q4_K", IS, H4, dev),
             pack_experts(sh["down"][None], "Q4_K", H4, IS, dev)]
    fn = expert_parallel(None, gate_type="Q4_K", up_type="Q4_K", down_type="Q4_K", hidden=H4, intermediate=I4)
    per_expert, shared_bytes = 7_077_888, 28_311_552
    out = {"workload": "moe_decode_q4k_e64_top6_h4096_i1024_shared4096", "batches": {}}
    layers = [base]
    for b in (1, 8, 64):
        active = len(np.unique(L["ids"][:b]))
        nbytes = active * per_expert + shared_bytes + 2 * b * H4 * 2
        want = min(12, max(2, -(-3 * 256 * 2**20 // nbytes)))
        while len(layers) < want:
            layers.append([type(t)(t.qtype, t.data.clone(), None, t.rows, t.width) for t in base])
        x = torch.from_numpy(L["x"][:b]).to(dev).to(torch.bfloat16)
        ids = torch.from_numpy(L["ids"][:b]).to(dev)
        w = torch.from_numpy(L["weights"][:b]).to(dev).to(torch.bfloat16)
        ws = torch.empty(fn.workspace_bytes(b, K4, E4, IS), dtype=torch.uint8, device=dev)
        o = torch.empty((b, H4), dtype=torch.bfloat16, device=dev)
        def call(i):
            g, u, d, sg, su, sd = layers[i % want]
            fn(g, u, d, x, ids, w, shared=dict(gate=sg, up=su, down=sd), workspace=ws, out=o)

        us = _time_calls(call, 100)
        out["batches"][str(b)] = {"us_per_step": round(us, 2), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
                                  "hbm_fraction": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                                  "active_experts": active, "bytes_per_step": nbytes, "layer_copies": want}
    return out


def measure_q8_down(dev):
    """The decode step of the headline layer (128 experts, top-8, H 2048, I 768, 8 tokens,
    seed 1) with the checkpoint's mix: Q6_K gate/up and Q8_0 down. Layer copies rotate so
    that one rotation's active bytes exceed 3x the Infinity Cache."""
    import numpy as np
    import torch

    from q6moe.experts import expert_parallel, pack_experts
    from q6moe.synth import moe_layer

    L = moe_layer(seed=1, experts=EXPERTS, top_k=TOP_K, hidden=HIDDEN, intermediate=INTER, tokens=TOKENS,
                  down_qtype="Q8_0", pack=False)
    base = [pack_experts(L["gate"], "Q6_K", INTER, HIDDEN, dev), pack_experts(L["up"], "Q6_K", INTER, HIDDEN, dev),
            pack_experts(L["down"], "Q8_0", HIDDEN, INTER, dev)]
    fn = expert_parallel(None, gate_type="Q6_K", up_type="Q6_K", down_type="Q8_0", hidden=HIDDEN,
                         intermediate=INTER)
    active = len(np.unique(L["ids"]))
    down_bytes = HIDDEN * (INTER // 32) * 34
    nbytes = active * (2 * Q6_PROJ_BYTES + down_bytes) + 2 * TOKENS * HIDDEN * 2 + TOKENS * TOP_K * 6
    copies = max(2, -(-3 * 256 * 2**20 // nbytes))
    layers = [base] + [[type(t)(t.qtype, t.data.clone(), None, t.rows, t.width) for t in base]
                       for _ in range(copies - 1)]
    x = torch.from_numpy(L["x"]).to(dev).to(torch.bfloat16)
    ids = torch.from_numpy(L["ids"]).to(dev)
    w = torch.from_numpy(L["weights"]).to(dev).to(torch.bfloat16)
    ws = torch.empty(fn.workspace_bytes(TOKENS, TOP_K, EXPERTS), dtype=torch.uint8, device=dev)
    o = torch.empty((TOKENS, HIDDEN), dtype=torch.bfloat16, device=dev)
    us = _time_calls(lambda i: fn(*layers[i % copies], x, ids, w, workspace=ws, out=o), 200)
    return {"workload": "moe_decode_q6k_gateup_q8_0_down_e128_top8_h2048_i768_b8", "us_per_step": round(us, 2),
            "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
            "hbm_fraction": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "active_experts": active,
            "bytes_per_step": nbytes, "layer_copies": copies}


def measure_kv_gather(dev):
    """Paged INT8 KV gather + dequant of every cached token: batch 8, 4 KV heads x 128,
    32768 tokens per sequence in pages of 256, FP32 per-token-per-head scales, seed 4.
    One call reads K and V (codes, scales, page tables) and writes BF16 [8, 32768, 4, 128]
    for each; three pool copies rotate so the 276 MB of codes are not cache-resident."""
    import torch

    from q6moe.attention_cache import read_paged
    from q6moe.synth import kv_pages

    K = kv_pages(seed=4)
    P, H, D = K["page_size"], K["kv_heads"], K["head_dim"]
    table = torch.from_numpy(K["page_table"]).to(dev)
    pools = []
    for _ in range(3):
        pools.append({n: torch.from_numpy(K[n]).to(dev) for n in ("k", "k_scale", "v", "v_scale")})
    ok = torch.empty((8, K["context"], H, D), dtype=torch.bfloat16, device=dev)
    ov = torch.empty_like(ok)

    def call(i):
        p = pools[i % 3]
        read_paged(p["k"], p["k_scale"], table, page_size=P, kv_heads=H, head_dim=D, out=ok)
        read_paged(p["v"], p["v_scale"], table, page_size=P, kv_heads=H, head_dim=D, out=ov)

    us = _time_calls(call, 30)
    nbytes = 813_699_072
    return {"workload": "kv_paged_gather_b8_kvh4_d128_ctx32768_p256_f32scale", "us_per_call": round(us, 1),
            "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
            "hbm_fraction": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "bytes_per_call": nbytes}


def measure_kv_attention(dev):
    """Fused decode attention over the same paged INT8 cache as the gather (batch 8, 32
    query heads over 4 KV heads, head_dim 128, 32768 attended tokens per sequence, pages of
    256, FP32 per-token-per-head scales, seed 4): the work of the gather plus the two
    attention einsums, without the BF16 copy. Three pool copies rotate."""
    import torch

    from q6moe.attention_cache import paged_decode_attention
    from q6moe.synth import kv_pages

    K = kv_pages(seed=4)
    P, H = K["page_size"], K["kv_heads"]
    table = torch.from_numpy(K["page_table"]).to(dev)
    pools = [{n: torch.from_numpy(K[n]).to(dev) for n in ("k", "k_scale", "v", "v_scale")} for _ in range(3)]
    q = torch.from_numpy(K["q"]).to(dev).to(torch.bfloat16)
    lengths = torch.full((K["batch"],), K["context"], dtype=torch.int32, device=dev)
    o = torch.empty_like(q)
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=dev)

    def call(i):
        p = pools[i % 3]
        paged_decode_attention(q, p["k"], p["k_scale"], p["v"], p["v_scale"], table, lengths, page_size=P,
                               kv_heads=H, workspace=ws, out=o)

    us = _time_calls(call, 30)
    nbytes = sum(pools[0][n].numel() * pools[0][n].element_size() for n in pools[0]) + table.numel() * 4 + \
        2 * q.numel() * 2
    return {"workload": "kv_paged_decode_attention_b8_hq32_kvh4_d128_ctx32768_p256_f32scale",
            "us_per_call": round(us, 1), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
            "hbm_fraction": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "bytes_per_call": nbytes}


def cpu_baseline(L):
    """The NumPy oracle (one thread) on one full decode step of the same workload."""
    from threadpoolctl import threadpool_limits

    from oracle import moe as oracle_moe

    with threadpool_limits(1):
        t0 = time.perf_counter()
        oracle_moe.expert_ffn(L["gate"], L["up"], L["down"], L["x"], L["ids"], L["weights"],
                              types=("Q6_K",) * 3, hidden=HIDDEN, intermediate=INTER)
        return time.perf_counter() - t0


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the single-projection, Q4_K+shared and KV-gather measurements")
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="first copy a buffer of this many MiB device-to-device 5 times (a known-size "
                         "kernel for scaling hardware byte counters)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        log("bench.py measures one GPU: the packed-expert path runs on a single MI355X here "
            "(sharding is by expert, see the design notes); run with --gpus 1")
        return 2
    if not (1 <= args.steps <= 100000 and 0 <= args.warmup <= 10000 and 1 <= args.layers <= 16):
        log("steps must be 1..100000, warmup 0..10000, layers 1..16")
        return 2

    import numpy as np
    import torch

    from q6moe.experts import expert_parallel, pack_experts
    from q6moe.synth import moe_layer

    dev = torch.device("cuda", 0)
    if args.calib_copy_mb > 0:
        src = torch.ones(args.calib_copy_mb << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    log("generating the decode workload (seed 1) ...")
    t0 = time.perf_counter()
    L = moe_layer(seed=SEED, experts=EXPERTS, top_k=TOP_K, hidden=HIDDEN, intermediate=INTER,
                  tokens=TOKENS, pack=False)
    log(f"  quantized {EXPERTS} experts in {time.perf_counter() - t0:.1f}s")
    base = [pack_experts(L[n], "Q6_K", INTER if n != "down" else HIDDEN, HIDDEN if n != "down" else INTER, dev)
            for n in ("gate", "up", "down")]
    layers = [base]
    for _ in range(args.layers - 1):
        layers.append([type(t)(t.qtype, t.data.clone(), None, t.rows, t.width) for t in base])
    x = torch.from_numpy(L["x"]).to(dev).to(torch.bfloat16)
    ids = torch.from_numpy(L["ids"]).to(dev)
    w = torch.from_numpy(L["weights"]).to(dev).to(torch.bfloat16)
    fn = expert_parallel(None, gate_type="Q6_K", up_type="Q6_K", down_type="Q6_K", hidden=HIDDEN,
                         intermediate=INTER)
    ws = torch.empty(fn.workspace_bytes(TOKENS, TOP_K, EXPERTS), dtype=torch.uint8, device=dev)
    out = torch.empty((TOKENS, HIDDEN), dtype=torch.bfloat16, device=dev)
    active = len(np.unique(L["ids"]))
    routes = int(np.count_nonzero(L["weights"]))

    def step(i, events=None):
        g, u, d = layers[i % len(layers)]
        fn(g, u, d, x, ids, w, workspace=ws, out=out, events=events)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # Whole-step throughput: K back-to-back steps between two synchronisations.
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    start.record()
    for i in range(args.steps):
        step(i)
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    gpu_ms = start.elapsed_time(end)
    ms_per_step = max(wall * 1e3, gpu_ms) / args.steps
    nbytes = step_bytes(active, routes)
    value = nbytes / (ms_per_step * 1e-3) / 1e9

    # Per-kernel durations with HIP events recorded between the launches.
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in range(args.steps)]
    for row in evs:
        for ev in row:
            ev.record()
    torch.cuda.synchronize()
    for i in range(args.steps):
        step(i, events=evs[i])
    torch.cuda.synchronize()
    phase = np.array([[row[j].elapsed_time(row[j + 1]) for j in range(4)] for row in evs]) * 1e3  # us
    ph = phase.mean(0)
    gu_bytes = gate_up_bytes(active, routes)
    achieved = gu_bytes / (ph[1] * 1e-6) / 1e9

    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations/logits, N(0,0.02) weights quantized to Q6_K)",
        "config": {
            "workload": "moe_decode_q6k_e128_top8_h2048_i768_b8",
            "experts": EXPERTS, "top_k": TOP_K, "hidden": HIDDEN, "intermediate": INTER,
            "tokens": TOKENS, "seed": SEED, "active_experts": active, "layer_copies": args.layers,
            "bytes_per_step": nbytes,
        },
        "hbm_fraction": round(value / HBM_PEAK_GBS, 4),
        "phases_us": {k: round(float(v), 2) for k, v in zip(("pre", "gate_up", "down", "combine"), ph)},
        "roofline": {
            "kernel": "moe_dec_gate_up_kernel",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": TRAFFIC_BYTES["moe_dec_gate_up_kernel"],
            "bytes_per_launch": gu_bytes,
            "avg_launch_us": round(float(ph[1]), 3),
        },
    }
    if not args.no_prefill:
        log("timing the prefill step (4096 tokens, seed 2) ...")
        result["prefill"] = measure_prefill(dev, steps=10, warmup=2)
    if not args.no_extras:
        log("timing the single projection, the Q4_K + shared layer, the Q8_0-down layer, the KV gather and attention ...")
        result["extras"] = {"projection": measure_projection(dev), "q4k_shared": measure_q4_shared(dev),
                            "q8_0_down": measure_q8_down(dev), "kv_gather": measure_kv_gather(dev),
                            "kv_attention": measure_kv_attention(dev)}
    if not args.no_cpu_baseline:
        log("timing the CPU oracle on one step (one thread) ...")
        secs = cpu_baseline(L)
        result["cpu_baseline"] = {
            "value": round(nbytes / secs / 1e9, 4),
            "unit": "GB/s",
            "cores": 1,
            "kind": "port",
            "sample": f"one full decode step of the same workload ({active} active experts decoded, "
                      f"SwiGLU FFN, combine) by the NumPy oracle: {secs:.2f} s",
        }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
