"""Benchmark of the MI355X FP4 MoE expert path (headline metric: FP4 MoE decode us/layer + HBM TB/s; prefill
grouped-GEMM MXFP4 TFLOPS).

Step (the headline, configs[1]): one MoE decode layer at batch 1 -- softmax top-8 routing of fresh N(0,1)
logits over 384 experts, then the routed FP4 experts (hidden 7168, intermediate 1664, packed E2M1 + E8M0,
tile_fp4 layout). value = selected-expert bytes (8 x 19,009,536 B) / step time, in TB/s.
Timing: K steps captured in one hipGraph, bracketed by a synchronize on both sides, timed with HIP events;
steps rotate over 4 resident copies of the layer (separate seeds) with fresh routing each step, so the
>= 456 MB streamed between two uses of a copy exceeds the 256 MB Infinity Cache (no MALL reuse).
Also reported (extra keys): the full layer with the bf16 shared expert, M = 4 / 8 / 16, the
dominant kernel's roofline (HIP events around that kernel alone, same inputs), configs[0] (one FP4 GEMV) on the
GPU and the CPU, configs[3] prefill, configs[4] 20-layer stack, and on this host's cores the reference's CPU MoE
library (oracle/_ref, compiled from the reference sources; cpu_baseline) beside this build's own host library
(cpu_port).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import ctypes
import gc
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "deepseekv4.1-a100-custom_amd"))
sys.path.insert(0, REPO)

HBM_PEAK = 8.0e12          # MI355X HBM3E, bytes/s
E, H, I, TOPK = 384, 7168, 1664, 8
LIMIT = 10.0               # swiglu_limit of the reference tests (test_cpumoe.py:23)
N_COPIES = 4
# HBM bytes per launch of the dominant kernel (moe_decode_up_kernel, M = 1): rocprofv3 FETCH_SIZE 49,706.1 KiB and
# WRITE_SIZE 16.5 KiB per dispatch (medians of 2048), scaled by what the same counters read for a plain 512 MiB device
# copy (FETCH x 2.000, WRITE x 1.000); summary and commands in profiles/moe_decode_up_kernel__configs1_decode_m1.txt
UP_TRAFFIC_BYTES = int(round((49706.0625 * 2.0 + 16.46875 * 1.0) * 1024))


def expert_bytes():
    return 2 * I * (H // 2) + 2 * I * (H // 32) + H * (I // 2) + H * (I // 32)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--quick", action="store_true", help="headline only (no extra configs)")
    ap.add_argument("--prefill-only", action="store_true", help="only the configs[3] prefill (2048 tokens; for profiling its kernels)")
    ap.add_argument("--prefill-tokens", type=int, default=2048, help="tokens of --prefill-only (2048: configs[3]; 16384: the probe)")
    ap.add_argument("--decode-m", type=int, default=0, help="only the configs[2] decode of this many tokens (for profiling its kernels)")
    ap.add_argument("--stack-only", action="store_true", help="only the configs[4] 20-layer decode stack (for profiling its kernels)")
    ap.add_argument("--surfaces-only", action="store_true", help="only the reference-shaped drop-in surfaces (for profiling their kernels)")
    ap.add_argument("--shared-only", choices=["bf16", "fp8"], default=None,
                    help="only the configs[1] layer with its shared expert fused into the decode launches (for profiling them)")
    ap.add_argument("--fp8-only", action="store_true", help="only the FP8 dense GEMV at the reference's test shapes (for profiling it)")
    ap.add_argument("--fp8-rows", type=int, default=1, help="token rows of --fp8-only (1: the GEMV; 5..64: fp8_gemm_kernel)")
    ap.add_argument("--mfma-rate", action="store_true", help="only the MFMA issue-rate probe (block-scaled 16x16x128, three operand "
                    "mixes): the attainable matrix rate the prefill kernels are measured against")
    ap.add_argument("--stream-probe", action="store_true", help="only the HBM stream-rate probe: the decode byte volumes read in "
                    "several launch shapes (and with a per-step workgroup barrier), graph-timed over rotating regions")
    ap.add_argument("--calib", action="store_true", help="also time a plain 512 MiB device copy (the reference kernel for "
                                                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes)")
    return ap.parse_args()


def make_layers(torch, dev, n, seed):
    from dsv41_amd import moe
    layers = []
    for c in range(n):
        g = torch.Generator(device=dev).manual_seed(seed + c)
        # random bytes are random in any layout: generated directly as the tile_fp4 layout
        w13 = torch.randint(0, 256, (E, 2 * I, H // 2), generator=g, dtype=torch.uint8, device=dev)
        s13 = torch.randint(119, 124, (E, 2 * I, H // 32), generator=g, dtype=torch.uint8, device=dev)
        w2 = torch.randint(0, 256, (E, H, I // 2), generator=g, dtype=torch.uint8, device=dev)
        s2 = torch.randint(119, 124, (E, H, I // 32), generator=g, dtype=torch.uint8, device=dev)
        ex = moe.ExpertWeights(w13, s13, w2, s2, tiled=True)
        ex.check()
        layers.append(ex)
    return layers


REPLAYS = 50   # timed replays of each captured graph; the median is reported (p10 / p90 kept in graph_time.stats)


def settle(torch):
    """Free what the previous measurement left (Python garbage, torch's cached blocks) now, with the device idle: a
    collection that falls inside the next measurement's timed replays cost it ~1.5 us per step (the drop-in decode
    sequences after the offload leg: 40.5 instead of 38.9 us)."""
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def graph_time(torch, fn_steps, steps, warmup, replays=None):
    """Capture `steps` calls (fn_steps(i) for i in range(steps)) in one graph; replay it for warm-up, then REPLAYS times
    back to back with one HIP event pair around each replay (one synchronisation before and after the set). Returns
    (median seconds per step, graph); graph_time.stats holds the p10 / median / p90 per step and the replay count."""
    settle(torch)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())   # inputs were produced on the current stream
    with torch.cuda.stream(s):
        for i in range(min(steps, 4)):
            fn_steps(i)                       # eager warm-up: workspaces allocated outside capture
    torch.cuda.synchronize()
    # a first capture, replayed once and dropped: the first graph captured after another workload ran ~1 us per step slow
    # through all its replays (the drop-in decode sequences: 40.4-40.9 against 38.9 us; the next capture of the same calls
    # was not; gc, an emptied allocator cache, 25 ms of warm-up replays and a 10 s idle did not remove it)
    g0 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g0, stream=s):
        for i in range(steps):
            fn_steps(i)
    g0.replay()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(steps):
            fn_steps(i)
    del g0
    for _ in range(max(1, warmup // max(1, steps) + 1)):
        g.replay()
    # and at least ~25 ms of replays, so the clocks have settled at the load this graph puts on the device (a leg after a
    # mostly idle one measured ~1.5 us per step slow on its first short warm-up)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g.replay()
    torch.cuda.synchronize()
    for _ in range(min(200, int(0.025 / max(time.perf_counter() - t0, 1e-6)))):
        g.replay()
    n = replays or REPLAYS
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    torch.cuda.synchronize()
    for e0, e1 in ev:
        e0.record()
        g.replay()
        e1.record()
    torch.cuda.synchronize()
    times = sorted(e0.elapsed_time(e1) / 1e3 / steps for e0, e1 in ev)
    q = lambda f: times[min(n - 1, int(round(f * (n - 1))))]
    graph_time.stats = {"replays": n, "steps_per_replay": steps, "p10_us": round(q(0.1) * 1e6, 3), "median_us": round(statistics.median(times) * 1e6, 3),
                        "p90_us": round(q(0.9) * 1e6, 3)}
    return statistics.median(times), g


def routing_stream(torch, dev, steps, M, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    return torch.randn(steps, M, E, generator=g, device=dev)


def bench_decode(torch, dev, layers, steps, warmup, M, shared=None, shared_mode="fused", seed=7, limit=LIMIT):
    """One decode layer per step over the rotating layer copies; shared: list of SharedExpert copies (bf16 or FP8),
    rotated with the layers, computed inside the two decode launches ("fused") or, bf16, as its own launches first
    ("separate"), or of (w8.W8 w13, w8.W8 w2) FP8 copies run as two FP8 GEMMs and a SwiGLU first ("fp8"). Returns
    (seconds per step, mean unique experts per step)."""
    from dsv41_amd import moe, quant
    logits = routing_stream(torch, dev, steps, M, seed)
    gx = torch.Generator(device=dev).manual_seed(seed + 1)
    x = torch.randn(M, H, generator=gx, device=dev).to(torch.bfloat16)
    xq = quant.fake_quant_fp8(x)
    eid = torch.empty(steps, M, TOPK, dtype=torch.int32, device=dev)
    wt = torch.empty(steps, M, TOPK, dtype=torch.float32, device=dev)
    out = torch.empty(M, H, dtype=torch.bfloat16, device=dev)
    ys = torch.empty(M, H, dtype=torch.bfloat16, device=dev)

    def step(i):
        ex = layers[i % len(layers)]
        route = (xq, logits[i], None, 1.0, TOPK, 1.0, "softmax", True, ex, limit)
        if shared is None:
            moe.moe_route_experts(*route, out=out, eid_out=eid[i], wt_out=wt[i])
        elif shared_mode == "fused":
            moe.moe_route_experts(*route, out=out, eid_out=eid[i], wt_out=wt[i], shared=shared[i % len(shared)], ys_out=ys)
        elif shared_mode == "fp8":
            w13, w2 = shared[i % len(shared)]
            y_s = moe.shared_expert_rows(xq, w13, w2, I, LIMIT)
            moe.moe_route_experts(*route, ys=y_s, out=out, eid_out=eid[i], wt_out=wt[i])
        else:
            sw = shared[i % len(shared)]
            y_s = moe.shared_expert(xq, sw.w13, sw.w2, LIMIT, ys=ys, tiled=sw.tiled)
            moe.moe_route_experts(*route, ys=y_s, out=out, eid_out=eid[i], wt_out=wt[i])

    t, g = graph_time(torch, step, steps, warmup)
    # unique experts per step (selected-expert bytes: each unique expert is read once)
    uniq = [len(set(eid[i].reshape(-1).tolist())) for i in range(steps)]
    return t, statistics.mean(uniq)


def bench_stack(torch, dev, layers, steps, warmup, n_layers=20):
    """batch-1 decode through n_layers independent MoE layers in one graph, with device routing.
    Per layer: one launch for the router (x <- rmsnorm(x + y_prev), logits = G_l . x with G_l [384, 7168] bf16
    ~N(0, 1/sqrt(7168)), fused with the FP8 fake-quantisation of x; our choice of chaining, unit norm weight),
    then the routed experts (softmax top-8). The first len(layers) layers reuse the headline copies; the rest get
    their own seeds. Returns (seconds per step, bytes per step)."""
    from dsv41_amd import moe
    stack = list(layers) + make_layers(torch, dev, n_layers - len(layers), 2000)
    g = torch.Generator(device=dev).manual_seed(77)
    routers = [(torch.randn(E, H, generator=g, device=dev) / H ** 0.5).to(torch.bfloat16) for _ in range(n_layers)]
    xs = [torch.randn(1, H, generator=g, device=dev).to(torch.bfloat16), torch.empty(1, H, dtype=torch.bfloat16, device=dev)]
    xq = torch.empty(1, H, dtype=torch.bfloat16, device=dev)
    y = torch.zeros(1, H, dtype=torch.bfloat16, device=dev)
    part = torch.empty(H // 1024, 1, E, dtype=torch.float32, device=dev)

    def step(i):
        for l in range(n_layers):
            moe.router_logits(xs[l % 2], y, routers[l], None, 1e-6, part=part, xn=xs[(l + 1) % 2], xq=xq)
            moe.moe_route_experts(xq, part, None, 1.0, TOPK, 1.0, "softmax", True, stack[l], LIMIT, out=y)

    t, _ = graph_time(torch, step, steps, warmup)
    del stack, routers
    return t, n_layers * (TOPK * expert_bytes() + E * H * 2)


MXFP4_PEAK = 10.1e15       # MI355X dense MXFP4 MFMA, FLOP/s
FP8_PEAK = 5.0e15          # dense FP8 rate (the fp4 x fp8 block-scaled MFMA)


def zipf_routing(T, seed, s=1.1):
    """configs[3] routing: Zipf(s) popularity over the 384 expert ranks, permuted by seed; 8 distinct experts per
    token drawn without replacement proportionally to popularity; weights = softmax of per-token N(0,1) logits
    over the 8."""
    import numpy as np
    rng = np.random.default_rng(seed)
    pop = 1.0 / np.arange(1, E + 1) ** s
    pop = pop[rng.permutation(E)]
    pop /= pop.sum()
    eid = np.stack([rng.choice(E, TOPK, replace=False, p=pop) for _ in range(T)]).astype(np.int32)
    lg = rng.standard_normal((T, TOPK))
    wt = (np.exp(lg) / np.exp(lg).sum(1, keepdims=True)).astype(np.float32)
    return eid, wt


def bench_prefill(torch, dev, ex, T, iters=20, seed=31):
    """prefill of T tokens (x bf16 ~N(0,1) -> FP8 fake-quant -> codes; Zipf routing) through the
    expert path: quantise + dispatch, w13 GEMM + SwiGLU, w2 GEMM, combine. Times each stage with HIP events
    (median over iters) and returns a dict."""
    import numpy as np
    from dsv41_amd import moe, quant
    settle(torch)
    eid_np, wt_np = zipf_routing(T, seed)
    eid, wt = torch.from_numpy(eid_np).to(dev), torch.from_numpy(wt_np).to(dev)
    g = torch.Generator(device=dev).manual_seed(seed)
    xq = quant.fake_quant_fp8(torch.randn(T, H, generator=g, device=dev).to(torch.bfloat16))
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    counts = np.bincount(eid_np.reshape(-1), minlength=E)
    touched = int((counts > 0).sum())
    flops = T * TOPK * (2 * 2 * I * H + 2 * H * I)
    wbytes = touched * expert_bytes()
    rec = {"total": [], "up": [], "down": []}
    for it in range(iters + 1):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        torch.cuda.synchronize()
        ev[0].record()
        st = moe.prefill_up(xq, eid, wt, ex, LIMIT)
        ev[1].record()
        moe.prefill_down(st, ex, out=out)
        ev[2].record()
        torch.cuda.synchronize()
        if it > 0:
            rec["up"].append(ev[0].elapsed_time(ev[1]) / 1e3)
            rec["down"].append(ev[1].elapsed_time(ev[2]) / 1e3)
            rec["total"].append(ev[0].elapsed_time(ev[2]) / 1e3)
        del st
    t = statistics.median(rec["total"])
    t_hbm = wbytes / HBM_PEAK
    return {"tokens": T, "pairs": T * TOPK, "experts_touched": touched, "max_pairs_per_expert": int(counts.max()),
            "us": round(t * 1e6, 1), "us_up_with_quant_dispatch": round(statistics.median(rec["up"]) * 1e6, 1),
            "us_down_with_combine": round(statistics.median(rec["down"]) * 1e6, 1), "TFLOPS": round(flops / t / 1e12, 1),
            "frac_mxfp4_peak": round(flops / t / MXFP4_PEAK, 4), "frac_fp8_rate": round(flops / t / FP8_PEAK, 4),
            "weight_GBps": round(wbytes / t / 1e9, 1),
            "attainable_frac": round(max(t_hbm, flops / FP8_PEAK) / t, 4), "flop": flops, "weight_bytes": wbytes}


def bench_up_kernel(torch, dev, layers, steps, warmup):
    """The dominant kernel alone (dsv41_moe_decode_up at M = 1: routing + w13 + SwiGLU): average launch duration
    from HIP events on its launch stream, over the same rotating layers and fresh logits."""
    from dsv41_amd import moe, quant
    logits = routing_stream(torch, dev, steps, 1, 11)
    xq = quant.fake_quant_fp8(torch.randn(1, H, device=dev).to(torch.bfloat16))

    def step(i):
        moe.decode_up(xq, layers[i % len(layers)], LIMIT, TOPK, logits=logits[i], gate=(None, 1.0, 1.0, "softmax", True))

    t, _ = graph_time(torch, step, steps, warmup)
    return t


def host_info():
    """lscpu fields the CPU numbers depend on, and the CPUs this process may use."""
    import subprocess
    info = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            if k.strip() in ("Model name", "Socket(s)", "Core(s) per socket", "Thread(s) per core", "NUMA node(s)", "L3 cache"):
                info[k.strip()] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    info["cpus_allowed"] = len(os.sched_getaffinity(0))
    return info


def _ref_lib():
    """The reference's CPU MoE library (dsv41/cpu/moe_cpu.cpp built by oracle/Makefile into oracle/_ref), or None."""
    lib = os.path.join(REPO, "oracle", "_ref", "libmoe_cpu_ref.so")
    flags = open("/proc/cpuinfo").read()
    if not os.path.exists(lib) or not all(f in flags for f in ("avx512f", "avx512bw", "avx512_vnni", "avx512vbmi", "avx512_bf16")):
        return None
    L = ctypes.CDLL(lib)
    L.cpumoe_alloc.restype = ctypes.c_void_p
    L.cpumoe_alloc.argtypes = [ctypes.c_size_t]
    L.cpumoe_init_list.restype = ctypes.c_int
    L.cpumoe_forward_ids.restype = ctypes.c_int
    L.cpumoe_forward_ids.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_size_t] * 4 + [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                     ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                     ctypes.c_void_p, ctypes.c_void_p]
    return L


def _time_layer_calls(L, bufs, Es, steps_cap, budget_s, it0=0):
    """Median time of forward_ids over 8 of Es resident experts, expert ids rotating every call
    (test_cpumoe.py:32-35); x is N(0,1) bf16, routing weights 1/8."""
    import numpy as np
    b13, bs13, b2, bs2 = 2 * I * (H // 2), 2 * I * (H // 32), H * (I // 2), H * (I // 32)
    rng = np.random.default_rng(4)
    x = rng.standard_normal(H).astype(np.float32)
    xb = (x.view(np.uint32) >> 16).astype(np.uint16)
    out = np.zeros(H, np.float32)
    gu = np.zeros(16 * 2 * I, np.float32)
    hb = np.zeros(16 * I, np.uint16)
    wts = np.full(TOPK, 1.0 / TOPK, np.float32)
    times = []
    t_end = time.perf_counter() + budget_s
    for it in range(it0, it0 + steps_cap):
        ids = np.array([(j * 5 + 8 * it) % Es for j in range(TOPK)], np.int32)
        t0 = time.perf_counter()
        r = L.cpumoe_forward_ids(bufs[0], bufs[1], bufs[2], bufs[3], b13, bs13, b2, bs2, ids.ctypes.data, TOPK, xb.ctypes.data,
                                 wts.ctypes.data, out.ctypes.data, H, I, H, ctypes.c_float(LIMIT), gu.ctypes.data, hb.ctypes.data)
        times.append(time.perf_counter() - t0)
        assert r == 0
        if time.perf_counter() > t_end:
            break
    return statistics.median(times[1:] if len(times) > 1 else times), len(times)


def llc_bytes() -> int:
    """The largest cache of cpu0 from sysfs (the last-level cache), in bytes; 0 when unreadable."""
    best = 0
    base = "/sys/devices/system/cpu/cpu0/cache"
    try:
        for d in os.listdir(base):
            try:
                v = open(os.path.join(base, d, "size")).read().strip()
            except OSError:
                continue
            mult = {"K": 1 << 10, "M": 1 << 20, "G": 1 << 30}.get(v[-1:].upper(), 1)
            best = max(best, int(v.rstrip("KkMmGg")) * mult)
    except OSError:
        pass
    return best


def cpu_baselines(steps_cap=80):
    """CPU numbers, all on the same host buffers and the same worker CPUs (this process's CPUs minus one core
    per NUMA node, as cpumoe.default_cpu_list):
      cpu_baseline  the reference's CPU MoE library (oracle/_ref), default W4A8 int8 mode (cpumoe.py:36), on a
                    bounded sample of configs[1]: a 48-expert subset of the layer shapes (0.91 GB, larger than
                    the host caches), 8 experts per call with rotating ids (test_cpumoe.py:32-35);
      cpu_port      this build's host library (libdsv41_cpu.so), same sample and mode;
      cpu_gemv_configs0  this build's single FP4 GEMV (configs[0], W [2048, 4096]) over 128 resident copies
                    (571 MB, so no copy is cache-resident between uses);
      host          lscpu fields and the library's measured DRAM read bandwidth."""
    import numpy as np
    from dsv41_amd import cpumoe
    res = {"host": host_info()}
    try:
        M = cpumoe.load_raw()
    except RuntimeError as err:
        return {"value": None, "note": str(err)}, res
    lst = cpumoe._expand(cpumoe.default_cpu_list() or ",".join(str(c) for c in sorted(os.sched_getaffinity(0))))
    per_node = int(os.environ.get("DSV41_CORES_PER_NODE", str(len(lst))))
    arr = (ctypes.c_int * len(lst))(*lst)
    M.cpumoe_init_list(arr, len(lst), per_node)
    M.cpumoe_set_int8(2)
    res["host"]["worker_cpus"] = len(lst)
    res["host"]["workers_pinned"] = M.cpumoe_threads_pinned()
    # the host's DRAM read rate with every worker: a 1 GiB stream (32x the 32 MiB L3 and more) read with plain loads and
    # with the expert kernels' 8 KB software prefetch; probed before, between and after the timed blocks (the host's
    # clocks settle during the first calls), the best reading reported
    bw_bytes = 1 << 30
    pbw = M.cpumoe_alloc(bw_bytes)
    np.frombuffer((ctypes.c_uint8 * bw_bytes).from_address(pbw), dtype=np.uint8)[:] = 1
    probes = []

    def probe(when):
        for pf in (0, 8192):
            M.cpumoe_set_prefetch(pf)
            probes.append({"when": when, "prefetch_bytes": pf, "GBps": round(M.cpumoe_bw_test(pbw, bw_bytes, 5, -1), 1)})
        M.cpumoe_set_prefetch(int(os.environ.get("DSV41_CPU_PF", "8192")))   # the kernels' setting again
    probe("before warm-up")

    # the expert subset: at least 48 experts (0.91 GB) and at least 4x the last-level cache, so no call finds its
    # experts cache-resident (rotating ids; 8 of the subset per call)
    llc = llc_bytes()
    Es = min(E, max(48, -(-4 * llc // expert_bytes())))
    res["host"]["llc_bytes"] = llc
    b13, bs13, b2, bs2 = 2 * I * (H // 2), 2 * I * (H // 32), H * (I // 2), H * (I // 32)
    rng = np.random.default_rng(3)
    sizes = (Es * b13, Es * bs13, Es * b2, Es * bs2)
    bufs = []
    for nbytes, (lo, hi) in zip(sizes, ((0, 256), (119, 124), (0, 256), (119, 124))):
        p = M.cpumoe_alloc(nbytes)
        np.frombuffer((ctypes.c_uint8 * nbytes).from_address(p), dtype=np.uint8)[:] = rng.integers(lo, hi, nbytes, dtype=np.uint8)
        bufs.append(p)
    sel = TOPK * expert_bytes()
    sample = (f"configs[1] layer shapes, {Es}-expert subset ({Es * expert_bytes() / 1e9:.2f} GB, {Es * expert_bytes() / max(llc, 1):.0f}x the "
              f"last-level cache), top-8 per call with rotating ids, int8 W4A8 mode, {len(lst)} pinned worker CPUs")
    baseline = {"value": None, "note": "oracle/_ref not built or host lacks its ISA"}
    R = _ref_lib()
    libs = [M]
    if R is not None:
        R.cpumoe_init_list(arr, len(lst), per_node)
        R.cpumoe_set_int8(2)
        libs = [R, M]
    # both libraries warm up first (the host's first few hundred calls run slow: page and clock settling), then
    # they are timed in alternating blocks of 10 calls, so neither gains from running later
    for L in libs:
        _time_layer_calls(L, bufs, Es, 1 << 20, 1.5)
    probe("after warm-up")
    meds = {id(L): [] for L in libs}
    n_blk = max(1, steps_cap // 10)
    for blk in range(n_blk):
        for L in libs:
            meds[id(L)].append(_time_layer_calls(L, bufs, Es, 11, 5.0, it0=11 * blk)[0])
        if blk == n_blk // 2:
            probe("between timing blocks")
    probe("after the timed blocks")
    M.cpumoe_free(pbw, bw_bytes)
    best_bw = max(p["GBps"] for p in probes)
    res["host"]["dram_read_GBps"] = best_bw
    res["host"]["dram_read_probes"] = probes
    if R is not None:
        med = statistics.median(meds[id(R)])
        baseline = {"value": round(med * 1e6, 1), "unit": "us/layer", "gbps": round(sel / med / 1e9, 1), "cores": len(lst),
                    "kind": "reference", "sample": sample + f", median of {len(meds[id(R)])} blocks of 10 calls, alternating with cpu_port"}
    rates = [sel / statistics.median(meds[id(L)]) / 1e9 for L in libs]
    res["host"]["layer_rate_within_dram_read"] = bool(max(rates) <= best_bw)
    med = statistics.median(meds[id(M)])
    res["cpu_port"] = {"value": round(med * 1e6, 1), "unit": "us/layer", "gbps": round(sel / med / 1e9, 1), "cores": len(lst),
                       "kind": "port", "sample": sample + f", median of {len(meds[id(M)])} blocks of 10 calls, alternating with cpu_baseline",
                       "note": "libdsv41_cpu.so: this build's restatement (bit-exact with the reference library in int8 mode "
                               "for inter % 256 == 0; computes the I = 1664 tail the reference skips)"}
    for p, nbytes in zip(bufs, sizes):
        M.cpumoe_free(p, nbytes)

    # configs[0] on the CPU: 128 copies of W [2048, 4096] + S, rotating
    N0, K0, copies = 2048, 4096, 128
    wb, sb = N0 * K0 // 2, N0 * K0 // 32
    pw, ps = M.cpumoe_alloc(copies * wb), M.cpumoe_alloc(copies * sb)
    np.frombuffer((ctypes.c_uint8 * (copies * wb)).from_address(pw), dtype=np.uint8)[:] = rng.integers(0, 256, copies * wb, dtype=np.uint8)
    np.frombuffer((ctypes.c_uint8 * (copies * sb)).from_address(ps), dtype=np.uint8)[:] = rng.integers(119, 124, copies * sb, dtype=np.uint8)
    x = (rng.standard_normal(K0).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    out = np.zeros(N0, np.float32)
    times = []
    for it in range(3 * copies):
        c = (it * 37) % copies
        t0 = time.perf_counter()
        assert M.cpumoe_gemv(pw + c * wb, ps + c * sb, N0, K0, x.ctypes.data, out.ctypes.data) == 0
        times.append(time.perf_counter() - t0)
    med = statistics.median(times[copies:])
    res["cpu_gemv_configs0"] = {"us": round(med * 1e6, 1), "GBps": round((wb + sb + 2 * K0 + 4 * N0) / med / 1e9, 1), "cores": len(lst),
                                "sample": f"median of {2 * copies} calls over 128 rotating copies (571 MB), int8 W4A8 mode"}
    M.cpumoe_free(pw, copies * wb)
    M.cpumoe_free(ps, copies * sb)
    return baseline, res


def bench_gemv_gpu(torch, dev, steps, warmup):
    """configs[0] on the GPU: one FP4 GEMV W [2048, 4096] x fq8(x) (cukern.fp4_gemv_pairs with one pair) per step,
    over 64 resident copies (290 MB > the 256 MB Infinity Cache); launch-bound at this size."""
    from dsv41_amd import hipkern, quant
    N0, K0, copies = 2048, 4096, 64
    g = torch.Generator(device=dev).manual_seed(9)
    w = torch.randint(0, 256, (copies, N0, K0 // 2), generator=g, dtype=torch.uint8, device=dev)
    s = torch.randint(119, 124, (copies, N0, K0 // 32), generator=g, dtype=torch.uint8, device=dev)
    x = quant.fake_quant_fp8(torch.randn(1, K0, generator=g, device=dev).to(torch.bfloat16))
    row_in = torch.zeros(1, dtype=torch.int32, device=dev)
    wt = torch.ones(1, dtype=torch.float32, device=dev)
    ids = [torch.full((1,), c, dtype=torch.int32, device=dev) for c in range(copies)]

    def step(i):
        hipkern.fp4_gemv_pairs(x, w, s, row_in, ids[(i * 37) % copies], wt, 1)

    t, _ = graph_time(torch, step, steps, warmup)
    nbytes = N0 * K0 // 2 + N0 * K0 // 32 + 2 * K0 + 4 * N0
    return {"us": round(t * 1e6, 2), "GBps": round(nbytes / t / 1e9, 1), "bytes": nbytes,
            "note": "x quantisation + GEMV launches per step, in one graph"}


FP8_SHAPES = [(5120, 8192), (4608, 5120), (32768, 1280), (1280, 5120), (5120, 2304)]   # test_fp8_tc.py:19 (V4.1 dims)


def bench_fp8_dense(torch, dev, steps, warmup, rows=1, with_bf16=True):
    """The FP8 dense-weight GEMV (w8.linear_w on a W8 weight, `rows` tokens, one by default) at the reference's own
    test shapes, each over enough resident copies to exceed the 256 MB Infinity Cache, against torch's bf16 F.linear
    (hipBLASLt) on bf16 copies of the same shape. Bytes: the FP8 weights plus their E8M0 scales."""
    from dsv41_amd import w8
    out = {}
    g = torch.Generator(device=dev).manual_seed(17)
    for (N, Kd) in FP8_SHAPES:
        copies = max(2, int(600e6 // (N * Kd)) + 1)
        Ws = [w8.W8(torch.randint(0, 256, (N, Kd), generator=g, dtype=torch.uint8, device=dev) & 0x7E,
                    torch.randint(115, 130, (N // 32, Kd // 32), generator=g, dtype=torch.uint8, device=dev)) for _ in range(copies)]
        x = torch.randn(rows, Kd, generator=g, device=dev).to(torch.bfloat16)
        t8, _ = graph_time(torch, lambda i: w8.linear_w(x, Ws[i % copies]), max(steps, copies), warmup)
        del Ws
        nbytes = N * Kd + (N // 32) * (Kd // 32)
        if not with_bf16:
            out[f"{N}x{Kd}"] = {"us": round(t8 * 1e6, 2), "GBps": round(nbytes / t8 / 1e9, 1)}
            continue
        Wb = [torch.randn(N, Kd, generator=g, device=dev).to(torch.bfloat16) for _ in range(max(2, copies // 2))]
        tb, _ = graph_time(torch, lambda i: torch.nn.functional.linear(x, Wb[i % len(Wb)]), max(steps, len(Wb)), warmup)
        del Wb
        out[f"{N}x{Kd}"] = {"us": round(t8 * 1e6, 2), "GBps": round(nbytes / t8 / 1e9, 1),
                            "bf16_linear_us": round(tb * 1e6, 2), "speedup_vs_bf16": round(tb / t8, 2)}
        torch.cuda.empty_cache()
    return out


def bench_offload(torch, dev, n_experts=64, tokens=20, seed=23):
    """The single-GPU offload paths on a configs[1]-shaped layer cut to `n_experts` experts held in pinned host memory
    (offload.OffloadMoE): one-token decode by gathering the 8 selected experts over PCIe; one-token decode with half the
    experts resident in a GPU slot table and the rest on the host library, run at the same time; and a 2048-token
    prefill that streams every expert through GPU staging. Wall-clock per call (host syncs included: these paths sync
    once per layer by design). PCIe-inclusive; no HBM roofline applies."""
    import time
    from dsv41_amd import cpumoe, moe, offload, quant
    g = torch.Generator(device=dev).manual_seed(seed)
    u8 = lambda *shape, lo=0, hi=256: torch.randint(lo, hi, shape, generator=g, dtype=torch.uint8, device=dev)
    w13, s13, w2, s2 = u8(n_experts, 2 * I, H // 2), u8(n_experts, 2 * I, H // 32, lo=119, hi=124), u8(n_experts, H, I // 2), \
        u8(n_experts, H, I // 32, lo=119, hi=124)
    hx = offload.HostExpertWeights.of(moe.ExpertWeights(quant.tile_fp4(w13), quant.tile_fp4_scales(s13), quant.tile_fp4(w2),
                                                        quant.tile_fp4_scales(s2), True))
    gate_w = torch.randn(n_experts, H, generator=g, device=dev) / H ** 0.5
    x1 = torch.randn(1, H, generator=g, device=dev).to(torch.bfloat16)
    out = {"n_experts": n_experts, "expert_bytes": hx.expert_bytes()}

    def wall(fn, n):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n

    layer = offload.OffloadMoE(hx, gate_w, topk=TOPK, swiglu_limit=LIMIT, device=dev)
    t_g = wall(lambda: layer(x1), tokens)
    out["decode_gather_us"] = round(t_g * 1e6, 1)
    out["decode_gather_h2d_GBps"] = round(TOPK * hx.expert_bytes() / t_g / 1e9, 1)
    if cpumoe.isa_ok():
        cw = [t.cpu() for t in (w13, s13, w2, s2)]
        he = cpumoe.HostExperts(n_experts, I, H)
        he.load_layer([cw[0][e, :I] for e in range(n_experts)], [cw[0][e, I:] for e in range(n_experts)],
                      [cw[1][e, :I] for e in range(n_experts)], [cw[1][e, I:] for e in range(n_experts)],
                      [cw[2][e] for e in range(n_experts)], [cw[3][e] for e in range(n_experts)])
        del cw
        layer_c = offload.OffloadMoE(hx, gate_w, topk=TOPK, swiglu_limit=LIMIT, device=dev, host=he,
                                     hot_ids=list(range(n_experts // 2)))
        t_c = wall(lambda: layer_c(x1), tokens)
        out["decode_hot_cold_us"] = round(t_c * 1e6, 1)
        out["hot_slots"] = n_experts // 2
        del layer_c
        he.close()
    xp = torch.randn(2048, H, generator=g, device=dev).to(torch.bfloat16)
    t_p = wall(lambda: layer(xp), 2)
    out["prefill_2048_us"] = round(t_p * 1e6, 1)
    out["prefill_h2d_GBps"] = round(n_experts * hx.expert_bytes() / t_p / 1e9, 1)
    del layer, hx
    torch.cuda.empty_cache()
    return out


def bench_surfaces(torch, dev, layers, steps, warmup):
    """The reference-shaped kernel surfaces called the way the reference calls them:
      * configs[1] decode through cukern.fp4_gemm_tc (decode.py:324-327: w13 GEMM, swiglu_quant(permute), w2 GEMM, sum)
        and through cukern.fp4_gemv_pairs (model.py:578-581), one layer per step over the rotating layer copies;
      * configs[3] prefill through GroupedPairs + moe_kernels.grouped_fp4_gemm (model.py:583-589, block_m 64: the
        128-pair tile kernel), stage times from HIP events."""
    from dsv41_amd import fused, hipkern, moe_kernels, quant
    logits = routing_stream(torch, dev, steps, 1, 7)
    top = [torch.topk(logits[i, 0], TOPK) for i in range(steps)]
    eids = [t.indices.to(torch.int32).contiguous() for t in top]
    wts = [torch.softmax(t.values, 0).contiguous() for t in top]
    xq = quant.fake_quant_fp8(torch.randn(1, H, device=dev).to(torch.bfloat16))
    xqp = hipkern.permute_x(xq)
    starts = torch.arange(TOPK + 1, device=dev, dtype=torch.int32)
    tok = torch.zeros(TOPK, device=dev, dtype=torch.int32)
    rows = torch.arange(TOPK, device=dev, dtype=torch.int32)
    ones = torch.ones(TOPK, device=dev)

    def tc_step(i):
        ex = layers[i % len(layers)]
        gu = hipkern.fp4_gemm_tc(xqp, ex.w13, ex.s13, eids[i], starts, tok, TOPK, 1)
        hqp = fused.swiglu_quant(gu, wts[i], I, LIMIT, permute=True)
        return hipkern.fp4_gemm_tc(hqp, ex.w2, ex.s2, eids[i], starts, rows, TOPK, 1, zero_out=True).sum(0)

    def gp_step(i):
        ex = layers[i % len(layers)]
        gu = hipkern.fp4_gemv_pairs(xq, ex.w13, ex.s13, tok, eids[i], ones, TOPK, tiled=True)
        hq = fused.swiglu_quant(gu, wts[i], I, LIMIT)
        return hipkern.fp4_gemv_pairs(hq, ex.w2, ex.s2, rows, eids[i], ones, TOPK, tiled=True).sum(0)

    out = {}
    t, _ = graph_time(torch, tc_step, steps, warmup)
    out["configs1_decode_fp4_gemm_tc_us"] = round(t * 1e6, 2)
    t, _ = graph_time(torch, gp_step, steps, warmup)
    out["configs1_decode_fp4_gemv_pairs_us"] = round(t * 1e6, 2)
    T = 2048
    eid_np, wt_np = zipf_routing(T, 31)
    eid = torch.from_numpy(eid_np).to(dev).reshape(-1)
    wt = torch.from_numpy(wt_np).to(dev).reshape(-1)
    xp = quant.fake_quant_fp8(torch.randn(T, H, device=dev).to(torch.bfloat16))
    P = T * TOPK
    tokp = torch.arange(T, device=dev, dtype=torch.int32).repeat_interleave(TOPK)
    pr = torch.arange(P, device=dev, dtype=torch.int32)
    onesp = torch.ones(P, device=dev)
    ex = layers[0]
    rec = []
    for it in range(4):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        torch.cuda.synchronize()
        ev[0].record()
        gu = moe_kernels.grouped_fp4_gemm(xp, ex.w13, ex.s13, moe_kernels.GroupedPairs(eid, tokp, pr, onesp, 64, n_experts=E), P, tiled=True)
        ev[1].record()
        hq = fused.swiglu_quant(gu, wt, I, LIMIT)
        ev[2].record()
        y = moe_kernels.grouped_fp4_gemm(hq, ex.w2, ex.s2, moe_kernels.GroupedPairs(eid, pr, pr, onesp, 64, n_experts=E), P,
                                         tiled=True).view(T, TOPK, H).sum(1)
        ev[3].record()
        torch.cuda.synchronize()
        if it:
            rec.append([ev[0].elapsed_time(ev[1]), ev[1].elapsed_time(ev[2]), ev[2].elapsed_time(ev[3]), ev[0].elapsed_time(ev[3])])
        del gu, hq, y
    m = [statistics.median(c) * 1e3 for c in zip(*rec)]
    out["configs3_prefill_grouped_fp4_gemm_us"] = {"w13_with_pairs_and_quant": round(m[0], 1), "swiglu": round(m[1], 1),
                                                   "w2_with_pairs_quant_and_sum": round(m[2], 1), "total": round(m[3], 1)}
    out["note"] = ("drop-in surfaces with the reference's own call sequences; the fused paths (us_per_layer, prefill_2048) "
                   "are this build's own orchestration of the same math")
    return out


def mfma_rate(torch, dev, iters=2000):
    """PFLOP/s of back-to-back independent block-scaled 16x16x128 MFMAs (dsv41_selftest_mfma_rate), median of 5 launches,
    per operand mix and grid size."""
    import ctypes
    from dsv41_amd import _lib
    out = torch.zeros(4, device=dev)
    res = {"iters": iters, "peaks_PFLOPs": {"fp8": FP8_PEAK / 1e15, "mxfp4": MXFP4_PEAK / 1e15}}
    for mode, name in ((0, "fp4xfp8"), (1, "fp8xfp8"), (2, "fp4xfp4")):
        for blocks in (1024, 4096):
            _lib.call("dsv41_selftest_mfma_rate", mode, blocks, 10, _lib.ptr(out), _lib.stream(dev))
            torch.cuda.synchronize()
            ts = []
            for _ in range(5):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                _lib.call("dsv41_selftest_mfma_rate", mode, blocks, iters, _lib.ptr(out), _lib.stream(dev))
                e1.record()
                torch.cuda.synchronize()
                ts.append(e0.elapsed_time(e1) / 1e3)
            flop = blocks * 4 * iters * 8 * 2 * 16 * 16 * 128
            res[f"{name}_blocks{blocks}_PFLOPs"] = round(flop / statistics.median(ts) / 1e15, 3)
    return res


def plain_read_us(torch, dev, buf, nbytes, blocks, waves, sync=0, steps=20):
    """Seconds per launch of a plain read of nbytes (dsv41_selftest_stream) in one launch shape, graph-timed (steps launches
    per graph, median of the replays) over rotating regions of buf: 160 MiB regions (4 of them, 640 MiB > the 256 MB
    Infinity Cache) below 1 GiB, else two regions of nbytes."""
    from dsv41_amd import _lib
    out = torch.zeros(4, dtype=torch.int32, device=dev)
    reg, nreg = (160 << 20, 4) if nbytes < (1 << 30) else (nbytes, 2)
    assert buf.numel() >= reg * nreg

    def launch(i):
        _lib.call("dsv41_selftest_stream", buf.data_ptr() + (i % nreg) * reg, nbytes // 1024, blocks, waves, sync, _lib.ptr(out), _lib.stream(dev))

    t, _ = graph_time(torch, launch, steps, 4)
    return t


def stream_probe(torch, dev):
    """What a plain read of the decode byte volumes attains: the down projection's 50.7 MB, the up projection's 101.4 MB,
    the layer's 152.1 MB and 1 GiB, each in several launch shapes (workgroups x waves), plain_read_us each; and 96 MiB
    read by 16 .. 512 workgroups (how fast part of the chip streams). sync: a
    workgroup barrier after every second tile, as the prefill kernels synchronise each k-step. fit: t = F + bytes / R by
    least squares over the four volumes for one shape."""
    import numpy as np
    buf = torch.empty(2 << 30, dtype=torch.uint8, device=dev)
    buf.random_(0, 256)
    vols = {"down_50.7MB": 50692096, "up_101.4MB": 101384192, "layer_152.1MB": 152076288, "1GiB": 1 << 30}
    shapes = [(256, 8), (416, 8), (448, 8), (512, 8), (1024, 8), (2048, 4)]
    res = {"us": {}, "TBps": {}}
    for vname, nb in vols.items():
        for blocks, waves, sync in [(b, w, 0) for b, w in shapes] + [(416, 8, 1), (512, 8, 1)]:
            t = plain_read_us(torch, dev, buf, nb, blocks, waves, sync)
            key = f"{vname}_{blocks}x{waves}" + ("_sync" if sync else "")
            res["us"][key] = round(t * 1e6, 2)
            res["TBps"][key] = round(nb / t / 1e12, 3)
    # part of the chip streaming: 96 MiB over 16 .. 512 workgroups of 8 waves (one per CU up to 256), the per-CU rate
    # a kernel reaches when other CUs are busy with something else
    for blocks in (16, 32, 64, 128, 192, 256, 512):
        t = plain_read_us(torch, dev, buf, 96 << 20, blocks, 8, 0)
        res["us"][f"cus_96MiB_{blocks}x8"] = round(t * 1e6, 2)
        res["TBps"][f"cus_96MiB_{blocks}x8"] = round((96 << 20) / t / 1e12, 3)
    for blocks, waves in ((416, 8), (512, 8)):
        xs = np.array([float(v) for v in vols.values()])
        ys = np.array([res["us"][f"{k}_{blocks}x{waves}"] * 1e-6 for k in vols])
        (F, invR), *_ = np.linalg.lstsq(np.stack([np.ones_like(xs), xs], 1), ys, rcond=None)
        res[f"fit_{blocks}x{waves}"] = {"F_us": round(F * 1e6, 2), "R_TBps": round(1 / invR / 1e12, 3)}
    return res


def progress(msg):
    """One line per finished phase on stderr (the JSON result is the only stdout line)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_shared_bf16(torch, dev, g):
    """N_COPIES bf16 shared experts of configs[1]'s dims (one per layer copy, in the fused launches' tiled layout)."""
    from dsv41_amd import moe
    return [moe.SharedExpert.prepare((torch.randn(2 * I, H, generator=g, device=dev) / H ** 0.5).to(torch.bfloat16),
                                     (torch.randn(H, I, generator=g, device=dev) / I ** 0.5).to(torch.bfloat16), tiled=True)
            for _ in range(N_COPIES)]


def make_shared_fp8(torch, dev, g):
    """N_COPIES shared experts as the checkpoint stores them (FP8 E4M3 with 32 x 32 E8M0 block scales, w8.W8 pairs)."""
    from dsv41_amd import w8
    return [(w8.W8(torch.randint(0, 256, (2 * I, H), generator=g, dtype=torch.uint8, device=dev) & 0x7E,
                   torch.randint(118, 122, (2 * I // 32, H // 32), generator=g, dtype=torch.uint8, device=dev)),
             w8.W8(torch.randint(0, 256, (H, I), generator=g, dtype=torch.uint8, device=dev) & 0x7E,
                   torch.randint(118, 122, (H // 32, I // 32), generator=g, dtype=torch.uint8, device=dev)))
            for _ in range(N_COPIES)]


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only: every GPU box here has one GPU, and the expert "
                                   "path's multi-GPU form (expert parallelism) is a design note, not a measured path",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    import dsv41_amd  # noqa: F401
    from dsv41_amd import _lib
    _lib.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    K, W = args.steps, args.warmup
    if args.mfma_rate:
        print(json.dumps(mfma_rate(torch, dev)))
        return
    if args.stream_probe:
        print(json.dumps({"stream_probe": stream_probe(torch, dev)}))
        return
    if args.fp8_only:
        print(json.dumps({"workload": f"FP8 dense weights x {args.fp8_rows} bf16 row(s), the reference's test shapes",
                          "fp8_dense": bench_fp8_dense(torch, dev, K, W, rows=args.fp8_rows, with_bf16=False)}))
        return
    if args.prefill_only:
        layers = make_layers(torch, dev, 1, 1000)
        T = args.prefill_tokens
        print(json.dumps(dict(bench_prefill(torch, dev, layers[0], T, iters=K),
                              workload=("configs[3]: " if T == 2048 else "") + f"{T} tokens x top-8, Zipf(1.1) routing, full expert path")))
        return
    layers = make_layers(torch, dev, N_COPIES, 1000)
    eb = expert_bytes()
    if args.decode_m:
        M = args.decode_m
        t_m, uniq = bench_decode(torch, dev, layers, K, W, M, seed=100 + M)
        print(json.dumps({"workload": f"configs[2] decode, M = {M}", "us": round(t_m * 1e6, 2), "unique_experts": round(uniq, 2),
                          "TBps": round(uniq * eb / t_m / 1e12, 3), "w2_bytes_per_expert": H * (I // 2) + H * (I // 32)}))
        return
    if args.surfaces_only:
        print(json.dumps({"workload": "drop-in surfaces: configs[1] fp4_gemm_tc / fp4_gemv_pairs, configs[3] GroupedPairs + grouped_fp4_gemm",
                          **bench_surfaces(torch, dev, layers, min(K, 40), W)}))
        return
    if args.stack_only:
        t_s, b_s = bench_stack(torch, dev, layers, max(2, min(K, 10)), W)
        print(json.dumps({"workload": "configs[4]: 20 layers, batch-1 decode, one graph", "us_per_step": round(t_s * 1e6, 1),
                          "bytes_per_step": b_s, "GBps": round(b_s / t_s / 1e9, 1)}))
        return
    if args.shared_only:
        # the configs[1] layer with its shared expert inside the two decode launches, for profiling those kernels
        from dsv41_amd import moe
        g = torch.Generator(device=dev).manual_seed(5)
        if args.shared_only == "bf16":
            shared, sh_bytes = make_shared_bf16(torch, dev, g), 2 * I * H * 2 + H * I * 2
        else:
            shared, sh_bytes = [moe.SharedExpert.of(p) for p in make_shared_fp8(torch, dev, g)], 3 * I * H + 3 * (I // 32) * (H // 32)
        t_l, _ = bench_decode(torch, dev, layers, K, W, 1, shared=shared, shared_mode="fused")
        print(json.dumps({"workload": f"configs[1] decode, M = 1, {args.shared_only} shared expert in the two launches",
                          "us": round(t_l * 1e6, 2), "bytes": TOPK * eb + sh_bytes, "TBps": round((TOPK * eb + sh_bytes) / t_l / 1e12, 3),
                          "shared_bytes": sh_bytes}))
        return
    sel_bytes = TOPK * eb

    progress("layers resident")
    t_routed, _ = bench_decode(torch, dev, layers, K, W, 1)
    timing = {"layer": dict(graph_time.stats)}
    progress(f"configs[1] decode layer {t_routed * 1e6:.2f} us")
    value = sel_bytes / t_routed / 1e12
    extra = {}
    # dominant kernel roofline: the fused up kernel at M = 1 (8 experts x (W13 + S13) bytes per launch; the
    # logits and activations it also reads are < 0.03 % of that and not counted)
    w13_bytes = TOPK * (2 * I * (H // 2) + 2 * I * (H // 32))
    t_up = bench_up_kernel(torch, dev, layers, K, W)
    timing["up_kernel"] = dict(graph_time.stats)
    roof = {"bound": "hbm", "kernel": "moe_decode_up_kernel<1,8,6,1> (routing + w13 + SwiGLU, M=1)", "achieved": round(w13_bytes / t_up / 1e9, 1),
            "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": round(w13_bytes / t_up / HBM_PEAK, 4), "traffic": UP_TRAFFIC_BYTES,
            "traffic_over_algorithmic": round(UP_TRAFFIC_BYTES / w13_bytes, 4), "avg_launch_us": round(t_up * 1e6, 2),
            "algorithmic_bytes": w13_bytes}
    extra["down_sum_us_est"] = round((t_routed - t_up) * 1e6, 2)
    progress(f"up kernel alone {t_up * 1e6:.2f} us")
    # the floor this layer is measured against on the same box: plain reads of the two launches' byte volumes in the
    # kernels' own launch shapes (up: 416 workgroups x 8 waves over 8 x (W13 + S13); down: 448 x 8 over 8 x (W2 + S2))
    buf = torch.empty(640 << 20, dtype=torch.uint8, device=dev)
    buf.random_(0, 256)
    w2_bytes = sel_bytes - w13_bytes
    r_up = plain_read_us(torch, dev, buf, w13_bytes, I // 32 * TOPK, 8)
    r_dn = plain_read_us(torch, dev, buf, w2_bytes, H // 16, 8)
    del buf
    extra["plain_read_floor"] = {"up_volume_us": round(r_up * 1e6, 2), "down_volume_us": round(r_dn * 1e6, 2),
                                 "two_reads_us": round((r_up + r_dn) * 1e6, 2), "layer_over_two_reads": round((r_up + r_dn) / t_routed, 4),
                                 "up_kernel_over_its_read": round(r_up / t_up, 4),
                                 "note": "dsv41_selftest_stream: a bare read of the same bytes in the same launch shape, same box, "
                                         "graph-timed over rotating regions; the layer adds routing, the down launch's table fetch, "
                                         "the MFMAs and the reductions to two such reads"}
    progress(f"plain reads of the two volumes {(r_up + r_dn) * 1e6:.2f} us")
    if not args.quick:
        # the same layer with the SwiGLU clamp disabled (swiglu_limit 0: the second setting configs[1] is run at)
        t_nolim, _ = bench_decode(torch, dev, layers, K, W, 1, limit=0.0)
        extra["layer_us_swiglu_limit_0"] = round(t_nolim * 1e6, 2)
        # the bf16 shared expert, one copy per layer copy (4 x 71.6 MB: with the routed bytes between two uses of a copy,
        # more than the 256 MB Infinity Cache holds)
        from dsv41_amd import moe
        g = torch.Generator(device=dev).manual_seed(5)
        shared = make_shared_bf16(torch, dev, g)
        t_layer, _ = bench_decode(torch, dev, layers, K, W, 1, shared=shared, shared_mode="fused")
        t_sep, _ = bench_decode(torch, dev, layers, K, W, 1, shared=shared, shared_mode="separate")
        sh_bytes = 2 * I * H * 2 + H * I * 2
        extra["layer_us_with_shared_expert"] = round(t_layer * 1e6, 2)
        extra["shared_expert"] = {"bytes": sh_bytes, "us_added_fused": round((t_layer - t_routed) * 1e6, 2),
                                  "layer_us_separate_launches": round(t_sep * 1e6, 2), "us_added_separate": round((t_sep - t_routed) * 1e6, 2),
                                  "layer_TBps_fused": round((sel_bytes + sh_bytes) / t_layer / 1e12, 3),
                                  "note": "fused: its gate/up row blocks are extra workgroups of the up launch and its down projection "
                                          "rides in the down launch; separate: three launches (gate/up GEMV, SwiGLU, down GEMV) before "
                                          "the routed experts; 4 rotating copies"}
        del shared
        # the same shared expert as the checkpoint stores it (FP8 E4M3, 32 x 32 E8M0 block scales, kept as w8.W8)
        shared8 = make_shared_fp8(torch, dev, g)
        t_fp8, _ = bench_decode(torch, dev, layers, K, W, 1, shared=shared8, shared_mode="fp8")
        t_fp8f, _ = bench_decode(torch, dev, layers, K, W, 1, shared=[moe.SharedExpert.of(p) for p in shared8], shared_mode="fused")
        fp8_bytes = 3 * I * H + 3 * (I // 32) * (H // 32)
        extra["shared_expert"].update({"fp8_bytes": fp8_bytes, "layer_us_fp8_fused": round(t_fp8f * 1e6, 2),
                                       "us_added_fp8_fused": round((t_fp8f - t_routed) * 1e6, 2),
                                       "layer_TBps_fp8_fused": round((sel_bytes + fp8_bytes) / t_fp8f / 1e12, 3),
                                       "layer_us_fp8_separate": round(t_fp8 * 1e6, 2), "us_added_fp8_separate": round((t_fp8 - t_routed) * 1e6, 2)})
        del shared8
        progress("layer with shared expert")
        extra["fp8_dense_gemv"] = bench_fp8_dense(torch, dev, K, W)
        # and 16 rows (the 5-16-row kernel, test_fp8_tc.py:19's 16-row case), FP8 only
        extra["fp8_dense_gemm_16_rows"] = bench_fp8_dense(torch, dev, K, W, rows=16, with_bf16=False)
        progress("FP8 dense GEMV")
        # the drop-in surfaces beside the other decode-sized legs (their decode sequences are the headline's shape)
        extra["drop_in_surfaces"] = bench_surfaces(torch, dev, layers, min(K, 40), W)
        progress("drop-in surfaces")
        for M in (4, 8, 16):
            t_m, uniq = bench_decode(torch, dev, layers, K, W, M, seed=100 + M)
            extra[f"decode_M{M}"] = {"us": round(t_m * 1e6, 2), "unique_experts": round(uniq, 2),
                                     "TBps": round(uniq * eb / t_m / 1e12, 3), "frac_hbm": round(uniq * eb / t_m / HBM_PEAK, 4),
                                     "p10_us": graph_time.stats["p10_us"], "p90_us": graph_time.stats["p90_us"]}
        progress("decode M = 4 / 8 / 16")
        extra["prefill_2048"] = dict(bench_prefill(torch, dev, layers[0], 2048),
                                     workload="configs[3]: 2048 tokens x top-8, Zipf(1.1) routing, full expert path")
        extra["prefill_16384_probe"] = dict(bench_prefill(torch, dev, layers[1], 16384, iters=10),
                                            workload="16,384-token probe (~341 pairs per expert)")
        ks = max(2, min(K, 10))
        t_s, b_s = bench_stack(torch, dev, layers, ks, 1)
        progress("prefill")
        extra["stack20"] = {"workload": "configs[4]: 20 layers, batch-1 decode; per layer rmsnorm + router GEMV (one launch), then "
                                        "gate + routed experts (two launches); one graph", "steps": ks, "us_per_step": round(t_s * 1e6, 1),
                            "bytes_per_step": b_s, "GBps": round(b_s / t_s / 1e9, 1), "frac_hbm": round(b_s / t_s / HBM_PEAK, 4)}
    if args.calib:
        src = torch.empty(512 << 20, dtype=torch.uint8, device=dev).random_(0, 256)
        dst = torch.empty_like(src)
        t_copy, _ = graph_time(torch, lambda i: dst.copy_(src), 4, 2)
        extra["copy_calibration"] = {"bytes_read": src.numel(), "bytes_written": dst.numel(), "us": round(t_copy * 1e6, 2),
                                     "GBps_read": round(src.numel() / t_copy / 1e9, 1)}
        del src, dst
    if not args.quick:
        extra["gemv_configs0_gpu"] = bench_gemv_gpu(torch, dev, K, W)
        progress("configs[4] stack and configs[0] GEMV")
        extra["offload"] = bench_offload(torch, dev)
        progress("offload paths")
    if args.no_cpu:
        cpu = {"value": None, "note": "skipped"}
    else:
        cpu, cpu_extra = cpu_baselines()
        progress("CPU baselines")
        extra.update(cpu_extra)
    result = {
        "metric": "FP4 MoE decode us/layer + HBM TB/s; prefill grouped-GEMM MXFP4 TFLOPS",
        "value": round(value, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(t_routed * 1e3, 5),
        "us_per_layer": round(t_routed * 1e6, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp4(e2m1)xfp8(e4m3)->fp32",
        "data": "synthetic: random E2M1 bytes, E8M0 scale bytes 119..123, N(0,1) bf16 activations, N(0,1) router logits",
        "config": {"workload": "configs[1]: one 384-expert top-8 FP4 MoE layer, decode batch 1, hidden 7168, intermediate 1664 "
                               "(routing + routed experts; shared expert reported as layer_us_with_shared_expert)",
                   "selected_expert_bytes": sel_bytes, "layer_copies": N_COPIES, "parallelism": "single GPU"},
        "frac_hbm_peak": round(value * 1e12 / HBM_PEAK, 4),
        "roofline": roof,
        "cpu_baseline": cpu,
        "timing": dict(timing, protocol=f"each figure: one graph of `steps` calls, replayed {REPLAYS} times back to back with an "
                                        "event pair per replay, median per step (p10 / p90 beside it)"),
    }
    result.update(extra)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
