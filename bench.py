#!/usr/bin/env python3
"""Benchmark of the MI355X 4-bit dequant matmul path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W]
    python bench.py --summarize-trace DIR     (a rocprofv3 output folder of this script)

Workload (benchmark config 2): one Llama-3.2-3B decode layer's projections at
M = 1 with MLX 4-bit group-64 weights -- q/o [3072x3072], k/v [1024x3072],
gate+up [8192x3072] fused with SiLU x up, down [3072x8192].  A step is one
layer: 4 launches (q/k/v rows concatenated at load time into one [5120x3072]
weight, o, gate/up+SiLU, down), down consuming the gate/up output.  Step i
uses layer copy i mod --copies (default 40 copies, 2.27 GB of weights), so the
256 MB MALL cannot hold the working set.

value      = algorithmic bytes of exactly K steps / GPU time of those K
             steps: W warm-up steps and then K timed steps, each a HIP graph
             of that many steps (graph replay removes the host launch cost, as
             a decode loop would), bracketed by torch.cuda.synchronize() and
             timed by events recorded around the replay on its stream (the
             host wall clock around it, which adds one replay's launch and
             synchronize latency, is in timing.host_wall_gbs).  Before the
             warm-up every layer copy is read once by a plain read kernel
             (not a step), so that the timed steps read weights the GPU has
             read before, as decode tokens after the first do.
stats      = the same layer over >= 50 replays (and >= 200 ms) of a graph of
             one rotation over the copies, an event after each replay:
             median and quartiles of the time per step.
roofline   = the dominant kernel (fused gate/up GEMV, 28.33 MB per launch):
             a graph of its 40 rotated launches alone, >= 50 replays with an
             event after each; avg_us = the median over replays of the time
             per launch.  `--summarize-trace` computes the same statistic from
             a kernel trace (the median over replays of the replay's mean
             kernel duration).  measured_ceiling: a read-only stream
             (csrc/bench/hbm_read.hip, in lib/libswiftltx_bench.so) and a
             device copy, same replay method.
extra      = the other benchmark configs and the paths around the GEMV, each
             by the same replay method: config 1 (q_proj GEMV over >= 2 GB of
             rotated copies), config 4a (lm_head GEMV over 10 rotated copies,
             2.2 GB), the fused-norm decode layer, the
             decode token (greedy / sampled), the 750-token prefill, token
             selection, small M (2..256) and the M > 1 MFMA GEMMs (configs 3,
             4b, 5) against the 2.5 PFLOP/s dense fp16/bf16 peak.
configs    = the last key of the line: every benchmark config as us and
             fraction of its roofline (a log that keeps only the line's tail
             still holds them).
cpu_baseline = C restatements of the same dequant matmul (Swift, the
             reference's host language, is not installed): single-thread
             scalar and all-cores 8-wide SIMD, median of 5 runs per config.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

METRIC = "4-bit GEMV HBM GB/s + GEMM TFLOP/s (% roofline) at Llama-3.2-3B shapes, 1 GPU"
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense fp16 / bf16
G = 64
MIN_REPLAYS = 50
MIN_MS = 200.0


def gemv_bytes(N, K, nsets=1, M=1, g=G):
    """Algorithmic bytes of a 4-bit matmul: packed codes, fp16 scales and
    biases of each weight set, fp16 x [M, K] and y [M, N]."""
    return nsets * (N * K // 2 + 4 * N * (K // g)) + 2 * M * K + 2 * M * N


# (name, N, K, weight sets).  q [3072], k [1024] and v [1024] rows are
# concatenated at load time into one [5120, 3072] weight (one launch, same
# matmulQ4 entry point); gate and up stay separate weights fused in one launch.
DECODE = [("qkv_proj", 5120, 3072, 1), ("o_proj", 3072, 3072, 1),
          ("gate_up_proj", 8192, 3072, 2), ("down_proj", 3072, 8192, 1)]
LAYER_BYTES = sum(gemv_bytes(N, K, n) for _, N, K, n in DECODE)  # 56,696,832
DOMINANT = "gate_up_proj"
DOMINANT_KERNEL = "q4_gemv_kernel<32, 3, true, false, 0, 1>"   # one x row
DOMINANT_BYTES = gemv_bytes(8192, 3072, 2)  # 28,334,080


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=80)
    ap.add_argument("--copies", type=int, default=40)
    ap.add_argument("--no-gemm", action="store_true", help="skip the M>1 GEMM and small-M legs")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--traffic", action="store_true",
                    help="only: 24 launches of the dominant kernel over 12 weight copies, then a "
                         "256 MiB torch copy (the calibration kernel), for rocprofv3 --pmc runs")
    ap.add_argument("--traffic-m", default="1",
                    help="with --traffic: activation rows of the gate/up launches, a comma list "
                         "(1: the GEMV; 2 and 8: the small-M kernel; at 1 < M <= 4 also the "
                         "down projection on the narrow kernel)")
    ap.add_argument("--gemm-pmc", action="store_true",
                    help="only: 10 launches each of the M=750 prefill gate/up (SiLU) and down "
                         "GEMMs, for rocprofv3 --pmc MFMA-utilisation runs")
    ap.add_argument("--token-select", action="store_true",
                    help="only: the token-selection leg (graphs), then TRACE_CALLS eager calls of "
                         "each sampling case, for rocprofv3 --kernel-trace; with "
                         "--summarize-trace: summarize such a trace per case and kernel")
    ap.add_argument("--small-m", action="store_true",
                    help="only: the small-M legs (graphs of rotated weights), for rocprofv3 "
                         "--kernel-trace runs of the narrow and small-M kernels")
    ap.add_argument("--summarize-pmc", metavar="DIR",
                    help="print the mean of the counter per kernel (dispatch count, KiB) of a "
                         "rocprofv3 --pmc output folder (rocpd .db or counter_collection.csv); "
                         "no GPU needed")
    ap.add_argument("--summarize-trace", metavar="DIR",
                    help="print a markdown summary of a rocprofv3 --kernel-trace output folder "
                         "(rocpd .db or kernel_trace.csv) of this script; no GPU needed")
    return ap.parse_args()


# --------------------------------------------------------------- timing ---

def replay_stats(torch, replay, units, min_reps=MIN_REPLAYS, min_ms=MIN_MS, max_reps=20000):
    """Times `replay` (enqueues one graph replay, or one eager sequence, on
    the current stream): one untimed call, then at least min_reps calls and
    at least min_ms of GPU time, an event recorded on the same stream after
    each.  Returns us per unit (units = launches or steps per call): median,
    25th / 75th percentiles, and the count."""
    import numpy as np
    replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    replay()
    e1.record()
    torch.cuda.synchronize()
    one = max(e0.elapsed_time(e1), 1e-3)
    reps = int(min(max_reps, max(min_reps, math.ceil(min_ms / one))))
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    evs[0].record()
    for i in range(reps):
        replay()
        evs[i + 1].record()
    torch.cuda.synchronize()
    per = np.array([evs[i].elapsed_time(evs[i + 1]) for i in range(reps)]) * 1e3 / units
    q25, q50, q75 = np.percentile(per, [25, 50, 75])
    return {"median_us": round(float(q50), 3), "p25_us": round(float(q25), 3),
            "p75_us": round(float(q75), 3), "replays": reps, "units_per_replay": units,
            "timed_ms": round(float(per.sum() * units / 1e3), 1)}


def upload_graph(g, stream):
    """hipGraphUpload of a captured graph's executable on `stream`, so that
    the replay in the timed region does not also pay the upload of its
    kernel packets to the device (the timed region holds that one replay)."""
    import ctypes
    try:
        exe = g.raw_cuda_graph_exec()
        hip = ctypes.CDLL("libamdhip64.so")
    except (AttributeError, OSError, RuntimeError):
        return False
    hip.hipGraphUpload.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    hip.hipGraphUpload.restype = ctypes.c_int
    return hip.hipGraphUpload(ctypes.c_void_p(exe), ctypes.c_void_p(stream.cuda_stream)) == 0


def capture(torch, fn, stream, warm=None):
    """A HIP graph of fn() captured on `stream`, after warm() (default fn)
    has run there eagerly once: the library sizes per-stream workspaces on
    first use and never allocates while a stream is being captured."""
    with torch.cuda.stream(stream):
        (warm or fn)()
    stream.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        fn()
    torch.cuda.synchronize()
    return g


def rate(st, nbytes=None, flops=None):
    """Adds GB/s (HBM fraction) or TFLOP/s (MFMA fraction) of the median."""
    us = st["median_us"]
    if nbytes:
        gbs = nbytes / (us * 1e-6) / 1e9
        st.update({"gbs": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                   "bytes": nbytes})
    if flops:
        tf = flops / (us * 1e-6) / 1e12
        st.update({"tflops": round(tf, 1), "frac_mfma": round(tf / MFMA_PEAK_TFLOPS, 4)})
    return st


# ----------------------------------------------------------------- data ---

def rand_q4(torch, N, K, gen, dev):
    w = torch.randint(-2**31, 2**31 - 1, (N, K // 8), generator=gen, device=dev,
                      dtype=torch.int64).to(torch.int32)
    s = (torch.randn(N, K // G, generator=gen, device=dev) * 0.02).abs().to(torch.float16)
    b = (s.float() * -8.0).to(torch.float16)
    return w, s, b


def q4(pkg, torch, N, K, gen, dev):
    return pkg.Q4Weight(*rand_q4(torch, N, K, gen, dev), K, G)


class Layer:
    def __init__(self, pkg, torch, gen, dev):
        self.w = {}
        for name, N, K, n in DECODE:
            self.w[name] = [q4(pkg, torch, N, K, gen, dev) for _ in range(n)]


def _wsb(q):
    return q.weight, q.scales, q.biases


# ----------------------------------------------------------------- main ---

def main():
    args = parse()
    if args.summarize_pmc:
        print(summarize_pmc(args.summarize_pmc))
        return
    if args.summarize_trace:
        if args.token_select:
            print(summarize_token_select_trace(args.summarize_trace))
        elif args.small_m:
            print(summarize_small_m_trace(args.summarize_trace))
        else:
            print(summarize_trace(args.summarize_trace, args.copies))
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(no sharding or collectives); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0 or args.copies < 1:
        print("--steps must be >= 1, --warmup >= 0, --copies >= 1", file=sys.stderr)
        sys.exit(2)

    import torch
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    pkg.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)

    if args.traffic:
        traffic_run(pkg, torch, gen, dev, tuple(int(m) for m in args.traffic_m.split(",")))
        return
    if args.gemm_pmc:
        gemm_pmc_run(pkg, torch, gen, dev)
        return
    if args.small_m:
        print(json.dumps(small_m_legs(pkg, torch, gen, dev, torch.cuda.Stream())), flush=True)
        return
    if args.token_select:
        print(json.dumps(token_select_leg(pkg, torch, gen, dev)), flush=True)
        for name, fn in token_select_cases(pkg, torch, gen, dev):
            if name.startswith("sample_"):
                s = torch.cuda.Stream()
                for _ in range(TRACE_CALLS):
                    fn(s)
                torch.cuda.synchronize()
        print("eager trace section:", ", ".join(SAMPLE_CASES), flush=True)
        return

    C = args.copies
    layers = [Layer(pkg, torch, gen, dev) for _ in range(C)]
    x = torch.randn(1, 3072, generator=gen, device=dev).half()
    attn = torch.randn(1, 3072, generator=gen, device=dev).half()
    x2 = torch.randn(1, 3072, generator=gen, device=dev).half()
    outs = {name: torch.empty(1, N, device=dev, dtype=torch.float16) for name, N, _, _ in DECODE}
    cap = torch.cuda.Stream()

    def step(i):
        w = layers[i % C].w
        pkg.matmul_q4(x, *_wsb(w["qkv_proj"][0]), 1, 3072, 5120, G, out=outs["qkv_proj"])
        pkg.matmul_q4(attn, *_wsb(w["o_proj"][0]), 1, 3072, 3072, G, out=outs["o_proj"])
        pkg.matmul_q4_silu_mul(x2, w["gate_up_proj"][0], w["gate_up_proj"][1], 1, 3072, 8192,
                               out=outs["gate_up_proj"])
        pkg.matmul_q4(outs["gate_up_proj"], *_wsb(w["down_proj"][0]), 1, 8192, 3072, G,
                      out=outs["down_proj"])

    # The library's per-device state is set up by a call that is not a step
    # (sltx_init), so that no step runs outside the warm-up and the timed
    # region.  Steps 0..W-1 are the warm-up graph, W..W+K-1 the timed graph.
    pkg.check(pkg.lib().sltx_init())
    torch.cuda.synchronize()

    def graph_of(first, n):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cap):
            for i in range(first, first + n):
                step(i)
        return g

    g_warm = graph_of(0, args.warmup) if args.warmup > 0 else None
    g_timed = graph_of(args.warmup, args.steps)
    uploaded = upload_graph(g_timed, cap)
    # Every weight copy is read once (a read kernel, not a step) before the
    # warm-up: the timed steps then read weights the GPU has read before, as
    # every decode token after the first does.  Measured without it, the
    # timed replay (the first read of those copies since their
    # initialization wrote them) took 21.0 us/step against 18.0 for a replay
    # of the same graph right after it; with it, 18.8.
    prime_weights(torch, dev, layers)
    torch.cuda.synchronize()
    if g_warm is not None:
        g_warm.replay()
    # Exactly K steps, one replay, bracketed by synchronizes.  The time is
    # the GPU's (events on the replaying stream, as the benchmark's rules time
    # kernels); the host wall clock around it, which adds the launch and
    # synchronize latency of one replay (~75 us), is reported beside it.
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record()
    g_timed.replay()
    ev1.record()
    torch.cuda.synchronize()
    host_wall = time.perf_counter() - t0
    wall = ev0.elapsed_time(ev1) / 1e3
    value = args.steps * LAYER_BYTES / wall / 1e9
    del g_warm, g_timed

    # the same layer, >= 50 replays of one rotation: median and quartiles
    g_rot = graph_of(0, C)
    layer_st = rate(replay_stats(torch, g_rot.replay, C), nbytes=LAYER_BYTES)
    del g_rot

    # dominant kernel: its C rotated launches alone
    def gate_up(i):
        w = layers[i % C].w["gate_up_proj"]
        pkg.matmul_q4_silu_mul(x2, w[0], w[1], 1, 3072, 8192, out=outs["gate_up_proj"])

    g_dom = capture(torch, lambda: [gate_up(i) for i in range(C)], cap, warm=lambda: gate_up(0))
    dom = replay_stats(torch, g_dom.replay, C)
    del g_dom
    dom_us = dom["median_us"]
    achieved = DOMINANT_BYTES / (dom_us * 1e-6) / 1e9

    ceilings = hbm_ceilings(pkg, torch, dev, cap)
    legs = {}
    legs["config1_q_proj_gemv_m1"] = config1_leg(pkg, torch, gen, dev, cap)
    legs["lm_head_gemv_m1_cold"] = lm_head_cold_leg(pkg, torch, gen, dev, cap)
    legs["decode_layer_fused_norms"] = fused_layer_leg(pkg, torch, gen, dev, layers, cap)
    model = synthetic_llama(pkg, torch, gen, dev, layers)
    legs["decode_token_greedy"] = decode_token_leg(pkg, torch, gen, dev, model)
    legs["prefill_750"] = prefill_leg(pkg, torch, gen, dev, model)
    del model
    legs["token_select"] = token_select_leg(pkg, torch, gen, dev)
    del layers, outs
    torch.cuda.empty_cache()
    if not args.no_gemm:
        legs["gemm"] = gemm_legs(pkg, torch, gen, dev, cap)
        legs["small_m"] = small_m_legs(pkg, torch, gen, dev, cap)
    cpu = None if args.no_cpu else cpu_baseline()

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * wall / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4xf16->f32",
        "data": "synthetic (the benchmark's distributions: x~N(0,1) fp16, codes uniform 0..15, "
                "scales |N(0,0.02)| fp16, biases -8*scale)",
        "config": {"workload": "Llama-3.2-3B decode layer projections, M=1, MLX 4-bit g64 "
                               "(q,k,v rows concatenated at load, o, gate+up fused SiLU*up, "
                               f"down); {C} distinct layer copies rotated",
                   "bytes_per_step": LAYER_BYTES, "launches_per_step": len(DECODE),
                   "timed": f"one HIP graph of exactly {args.steps} steps after one of "
                            f"{args.warmup} warm-up steps, between synchronizes; GPU time from "
                            f"events around the replay"},
        "timing": {"gpu_ms": round(wall * 1e3, 4), "host_wall_ms": round(host_wall * 1e3, 4),
                   "host_wall_gbs": round(args.steps * LAYER_BYTES / host_wall / 1e9, 1),
                   "graph_uploaded": uploaded},
        "stats": {**layer_st, "ms_per_step_median": round(layer_st["median_us"] / 1e3, 5),
                  "what": f"per step, over replays of a graph of one {C}-copy rotation"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profiles(),
                     "kernel": f"{DOMINANT_KERNEL} (gate/up fused SiLU*up)",
                     "avg_us": dom_us, "p25_us": dom["p25_us"], "p75_us": dom["p75_us"],
                     "replays": dom["replays"], "bytes_per_launch": DOMINANT_BYTES,
                     "timing": f"median over {dom['replays']} replays of a graph of the {C} "
                               "rotated gate/up launches of the time per launch (an event "
                               "after each replay, on the stream the graph runs on)",
                     "measured_ceiling": {**ceilings,
                                          "frac_of_read": round(achieved / ceilings["read_gbs"],
                                                                4)}},
        "cpu_baseline": cpu,
        "extra": legs,
    }
    line["configs"] = config_summary(value, args.steps, wall, layer_st, dom_us, legs)
    print(json.dumps(line))


def config_summary(value, steps, wall, layer_st, dom_us, legs):
    """Every benchmark config in a few numbers, for the end of the JSON line
    (whose tail is what a log keeps): us and fraction of the HBM (GEMV) or
    dense MFMA (GEMM) peak."""
    def hbm(st):
        return {"us": st["median_us"], "frac_hbm": st["frac_hbm"]} if st else None

    def mfma(st):
        return {"us": st["median_us"], "frac_mfma": st["frac_mfma"]} if st else None

    gemm = legs.get("gemm", {})

    def small(name, M):
        st = legs.get("small_m", {}).get(name, {}).get(f"m{M}")
        return {"us": st["median_us"], "frac_hbm": st["frac_hbm"], "frac_mfma": st["frac_mfma"],
                "route": st["route"]} if st else None

    return {
        "c1_q_proj_gemv": hbm(legs.get("config1_q_proj_gemv_m1")),
        "c2_decode_layer": {"value_us_per_step": round(1e6 * wall / steps, 3),
                            "value_frac_hbm": round(value / HBM_PEAK_GBS, 4),
                            "stats_us": layer_st["median_us"],
                            "stats_frac_hbm": layer_st["frac_hbm"],
                            "gate_up_us": dom_us,
                            "gate_up_frac_hbm": round(DOMINANT_BYTES / (dom_us * 1e-6)
                                                      / 1e9 / HBM_PEAK_GBS, 4),
                            "fused_norms_us": legs["decode_layer_fused_norms"]["median_us"]},
        "c3_prefill_gate_up_silu_m750": mfma(gemm.get("prefill_gate_up_silu_m750")),
        "c3_prefill_down_m750": mfma(gemm.get("prefill_down_m750")),
        "c4a_lm_head_gemv_cold": hbm(legs.get("lm_head_gemv_m1_cold")),
        "c4b_lm_head_gemm_m750": mfma(gemm.get("lm_head_gemm_m750")),
        "c5_dit_up_gelu_m6144": mfma(gemm.get("dit_ffn_up_gelu_m6144_bf16")),
        "c5_dit_down_m6144": mfma(gemm.get("dit_ffn_down_m6144_bf16")),
        "c5_dit_up_m6144_f32in": mfma(gemm.get("dit_ffn_up_gelu_m6144_f32in")),
        "m128_llama_gate_up_silu": small("llama_gate_up_silu", 128),
        "m128_t5_ffn_wo": small("t5_ffn_wo", 128),
    }


# ------------------------------------------------------------ ceilings ---

_BENCH_LIB = None


def bench_lib():
    """lib/libswiftltx_bench.so: measurement kernels built beside the product
    library (swift-ltx_amd/csrc/bench/) and loaded only here."""
    global _BENCH_LIB
    if _BENCH_LIB is None:
        import ctypes
        path = os.path.join(REPO, "swift-ltx_amd", "lib", "libswiftltx_bench.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: run python swift-ltx_amd/build.py")
        L = ctypes.CDLL(path)
        L.sltx_bench_hbm_read_blocks.argtypes = []
        L.sltx_bench_hbm_read_blocks.restype = ctypes.c_int
        L.sltx_bench_hbm_read.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p,
                                          ctypes.c_int32, ctypes.c_void_p]
        L.sltx_bench_hbm_read.restype = ctypes.c_int
        _BENCH_LIB = L
    return _BENCH_LIB


def hbm_read(torch, src, sink, lds=False):
    """Streams the bytes of device tensor src (contiguous, a multiple of 16)
    through the GPU's loads into registers (or, lds, through direct global ->
    LDS copies); sink: int32 [bench_lib().sltx_bench_hbm_read_blocks()]."""
    rc = bench_lib().sltx_bench_hbm_read(src.data_ptr(), src.numel() * src.element_size(),
                                         sink.data_ptr(), 1 if lds else 0,
                                         torch.cuda.current_stream().cuda_stream)
    if rc != 0:
        raise RuntimeError(f"sltx_bench_hbm_read failed: {rc}")


def prime_weights(torch, dev, layers):
    """One read of every layer copy's packed weights, scales and biases with
    the bench library's read kernel (csrc/bench/hbm_read.hip)."""
    sink = torch.empty(bench_lib().sltx_bench_hbm_read_blocks(), device=dev, dtype=torch.int32)
    for lay in layers:
        for ws in lay.w.values():
            for w in ws:
                for t in (w.weight, w.scales, w.biases):
                    hbm_read(torch, t, sink)


def hbm_ceilings(pkg, torch, dev, cap, read_gib=4, copy_gib=1):
    """Measured HBM ceilings: a read-only stream of read_gib GiB (16-byte
    nontemporal loads over the whole GPU, XOR-reduced; csrc/bench/hbm_read.hip),
    the same stream through direct global -> LDS copies, and a device copy of
    copy_gib GiB (torch copy_, bytes read + written)."""
    src = torch.empty(read_gib * 2 ** 30 // 4, device=dev, dtype=torch.int32)
    src.random_()
    sink = torch.empty(bench_lib().sltx_bench_hbm_read_blocks(), device=dev, dtype=torch.int32)
    g = capture(torch, lambda: hbm_read(torch, src, sink), cap)
    rd = rate(replay_stats(torch, g.replay, 1), nbytes=src.numel() * 4)
    del g
    g = capture(torch, lambda: hbm_read(torch, src, sink, lds=True), cap)
    rl = rate(replay_stats(torch, g.replay, 1), nbytes=src.numel() * 4)
    del g, src
    n = copy_gib * 2 ** 30 // 2
    a = torch.empty(n, device=dev, dtype=torch.float16).normal_()
    b = torch.empty_like(a)
    g = capture(torch, lambda: b.copy_(a), cap)
    cp = rate(replay_stats(torch, g.replay, 1), nbytes=2 * n * 2)
    del g, a, b
    torch.cuda.empty_cache()
    return {"read_gbs": rd["gbs"], "read_frac_of_peak": rd["frac_hbm"],
            "read_what": f"register read of {read_gib} GiB, median of {rd['replays']} replays",
            "read_lds_gbs": rl["gbs"],
            "read_lds_what": f"direct global -> LDS copies of {read_gib} GiB, "
                             f"median of {rl['replays']} replays",
            "copy_gbs": cp["gbs"],
            "copy_what": f"{copy_gib} GiB device copy (read + written), median of "
                         f"{cp['replays']} replays"}


# --------------------------------------------------------- config legs ---

def config1_leg(pkg, torch, gen, dev, cap, copies=400):
    """Benchmark config 1: one q_proj GEMV [3072 x 3072], M = 1, rotated over
    `copies` weight copies (400 x 5.31 MB = 2.12 GB)."""
    ws = [q4(pkg, torch, 3072, 3072, gen, dev) for _ in range(copies)]
    xx = torch.randn(1, 3072, generator=gen, device=dev).half()
    y = torch.empty(1, 3072, device=dev, dtype=torch.float16)
    run = lambda w: pkg.matmul_q4(xx, *_wsb(w), 1, 3072, 3072, G, out=y)
    g = capture(torch, lambda: [run(w) for w in ws], cap, warm=lambda: run(ws[0]))
    st = rate(replay_stats(torch, g.replay, copies), nbytes=gemv_bytes(3072, 3072))
    del g, ws
    torch.cuda.empty_cache()
    st["copies"] = copies
    st["working_set_gb"] = round(copies * gemv_bytes(3072, 3072) / 1e9, 2)
    return st


def lm_head_cold_leg(pkg, torch, gen, dev, cap, copies=10):
    """Benchmark config 4a: the tied lm_head GEMV [128256 x 3072], M = 1,
    rotated over `copies` weight copies (10 x 222.6 MB = 2.23 GB, beyond the
    256 MB MALL)."""
    V = 128256
    ws = [q4(pkg, torch, V, 3072, gen, dev) for _ in range(copies)]
    xx = torch.randn(1, 3072, generator=gen, device=dev).half()
    y = torch.empty(1, V, device=dev, dtype=torch.float16)
    run = lambda w: pkg.matmul_q4(xx, *_wsb(w), 1, 3072, V, G, out=y)
    g = capture(torch, lambda: [run(w) for w in ws], cap, warm=lambda: run(ws[0]))
    st = rate(replay_stats(torch, g.replay, copies), nbytes=gemv_bytes(V, 3072))
    del g, ws
    torch.cuda.empty_cache()
    st["copies"] = copies
    st["working_set_gb"] = round(copies * gemv_bytes(V, 3072) / 1e9, 2)
    return st


def fused_layer_leg(pkg, torch, gen, dev, layers, cap):
    """The same decode layer with the operators around the projections fused
    in (LlamaModel.swift:288-331): rms_norm -> q|k|v, o, residual add +
    rms_norm -> gate/up + SiLU x up, down + residual add.  Still 4 launches;
    the norm weights (fp32) and the residual vectors add a few KB per layer.
    Rotated over the layer copies."""
    K, F = 3072, 8192
    n1 = (1.0 + 0.1 * torch.randn(K, generator=gen, device=dev)).float()
    n2 = (1.0 + 0.1 * torch.randn(K, generator=gen, device=dev)).float()
    x = torch.randn(1, K, generator=gen, device=dev).half()
    attn = torch.randn(1, K, generator=gen, device=dev).half()
    qkv = torch.empty(1, 5120, device=dev, dtype=torch.float16)
    o = torch.empty(1, K, device=dev, dtype=torch.float16)
    res = torch.empty(1, K, device=dev, dtype=torch.float16)
    act = torch.empty(1, F, device=dev, dtype=torch.float16)
    out = torch.empty(1, K, device=dev, dtype=torch.float16)

    def step(L):
        w = L.w
        pkg.rmsnorm_matmul_q4(x, n1, 1e-5, w["qkv_proj"][0], 5120, out=qkv)
        pkg.linear(attn, w["o_proj"][0], 1, K, K, out=o)
        pkg.residual_rmsnorm_matmul_q4_silu_mul(x, o, n2, 1e-5, w["gate_up_proj"][0],
                                                w["gate_up_proj"][1], F, residual_out=res,
                                                out=act)
        pkg.matmul_q4_residual(act, w["down_proj"][0], res, 1, K, out=out)

    g = capture(torch, lambda: [step(L) for L in layers], cap, warm=lambda: step(layers[0]))
    nbytes = LAYER_BYTES + 2 * K * 4 + 5 * 2 * K
    st = rate(replay_stats(torch, g.replay, len(layers)), nbytes=nbytes)
    del g
    st.update({"launches_per_layer": 4,
               "note": "rms_norm, residual add + rms_norm and the final residual add run inside "
                       "the projections' kernels"})
    return st


def synthetic_llama(pkg, torch, gen, dev, layers, L=28):
    """Llama-3.2-3B with random 4-bit weights, in ModelWeights' shape (q|k|v
    concatenated, tied 4-bit embedding / lm_head over 128256 tokens): the
    first L of the rotated layer copies; layer norm weights 0.05 (1 + 0.1
    N(0,1)), so that the residual stream stays inside fp16 over 28 layers
    (nothing bounds it without attention: with weights near 1 it overflows and
    every logit is NaN); final norm weights 1 + 0.1 N(0,1), which gives peaked
    logits like a trained model's."""
    from types import SimpleNamespace
    from swiftltx_amd.weights import LayerWeights
    K, V = 3072, 128256
    norm = lambda: (0.05 * (1.0 + 0.1 * torch.randn(K, generator=gen, device=dev))).float()
    fnorm = lambda: (1.0 + 0.1 * torch.randn(K, generator=gen, device=dev)).float()
    embed = q4(pkg, torch, V, K, gen, dev)
    lws = []
    for lay in layers[:L]:
        w = lay.w
        lws.append(LayerWeights(q_proj=None, k_proj=None, v_proj=None, o_proj=w["o_proj"][0],
                                gate_proj=w["gate_up_proj"][0], up_proj=w["gate_up_proj"][1],
                                down_proj=w["down_proj"][0], input_norm_weight=norm(),
                                post_norm_weight=norm(), qkv_proj=w["qkv_proj"][0]))
    cfg = SimpleNamespace(hidden_size=K, intermediate_size=8192, num_attention_heads=24,
                          num_key_value_heads=8, head_dim=128, vocab_size=V, rms_norm_eps=1e-5)
    return SimpleNamespace(config=cfg, embed_tokens=embed, lm_head=embed, norm_weight=fnorm(),
                           layers=lws)


def decode_token_leg(pkg, torch, gen, dev, mw):
    """A Llama-3.2-3B decode step's matmul path (swiftltx_amd.decode), greedy
    and sampled: 4-bit embedding gather, 28 layers (RMSNorm + q|k|v, o,
    residual + RMSNorm + gate/up SiLU, down + residual), final RMSNorm + tied
    4-bit lm_head over 128256 tokens, argmax (or top-p sampling) -- one HIP
    graph per token, the token id fed back on the device.  Attention is
    outside the path: its stand-in is the q rows (a view, no launch).  mw:
    synthetic_llama()."""
    from swiftltx_amd.decode import DecodeStep
    K, V, L = mw.config.hidden_size, mw.config.vocab_size, len(mw.layers)
    s = torch.cuda.Stream()
    ds = DecodeStep(mw, stream=s)
    ds.capture()
    st = replay_stats(torch, ds.replay, 1)
    # the same step sampling (temperature 0.7, top-p 0.9, penalty 1.1) from a
    # SamplerState: 64 prompt ids, the history and the draws on the device
    state = pkg.SamplerState(8192, draws=8192, generator=gen, device=dev,
                             history=torch.randint(0, V, (64,), generator=gen,
                                                   device=dev).tolist())
    ds2 = DecodeStep(mw, stream=s)
    ds2.capture(temperature=0.7, top_p=0.9, repetition_penalty=1.1, state=state)
    st2 = replay_stats(torch, ds2.replay, 1, max_reps=4000)
    nbytes = (L * (LAYER_BYTES + 2 * K * 4) + gemv_bytes(V, K) + K * 4 + K // 2 + 4 * K // G
              + 2 * K)
    us, us_s = st["median_us"], st2["median_us"]
    return {**rate(st, nbytes=nbytes), "tokens_per_s": round(1e6 / us, 1),
            "launches_per_token": 1 + 4 * L + 1 + 2, "layers": L,
            "sampled": {**st2, "tokens_per_s": round(1e6 / us_s, 1),
                        "launches_per_token": 1 + 4 * L + 1 + 4,
                        "sampler": "temperature 0.7, top-p 0.9, repetition penalty 1.1, "
                                   "history and draws in device memory (SamplerState)"},
            "note": "attention (RoPE, KV cache, softmax) is outside the 4-bit path; stand-in = "
                    "the q rows"}


def prefill_leg(pkg, torch, gen, dev, mw, S=750):
    """A Llama-3.2-3B prefill of S = 750 prompt tokens (swiftltx_amd.prefill;
    LlamaModel.swift:168-203): 4-bit embedding gather of S ids, 28 layers of
    q|k|v GEMM, o GEMM + residual + rms_norm (one call), gate/up GEMM with the
    SiLU x up epilogue, down GEMM + residual + the next layer's rms_norm (one
    call), then rms_norm + lm_head on the last row -- one HIP graph per prompt
    (layer 0's input norm is its own launch).  Attention is outside
    the path: its stand-in copies the q columns (a torch copy, inside the
    timed graph).  flops: the matmuls only, 2 * S * (q|k|v + o + gate + up +
    down) per layer plus the last row's lm_head."""
    from swiftltx_amd.prefill import PrefillStep
    c = mw.config
    K, F, L = c.hidden_size, c.intermediate_size, len(mw.layers)
    qkv = (c.num_attention_heads + 2 * c.num_key_value_heads) * c.head_dim
    q = c.num_attention_heads * c.head_dim
    s = torch.cuda.Stream()
    ps = PrefillStep(mw, S, stream=s)
    ps.tokens.copy_(torch.randint(0, c.vocab_size, (S,), generator=gen, device=dev,
                                  dtype=torch.int32))
    torch.cuda.synchronize()
    ps.capture()
    st = replay_stats(torch, ps.replay, 1)
    flops = 2 * S * L * (K * qkv + q * K + 2 * K * F + F * K) + 2 * K * c.vocab_size
    rate(st, flops=flops)
    st.update({"ms_per_prompt": round(st["median_us"] / 1e3, 3),
               "prompt_tokens_per_s": round(S / (st["median_us"] * 1e-6), 1),
               "tokens": S, "layers": L,
               "note": "matmul flops only; attention stand-in = a copy of the q columns"})
    return st


# ------------------------------------------------------- token selection ---

SAMPLE_CASES = ("sample_top_p", "sample_top_p_flat", "sample_top_p_two_levels",
                "sample_top_p_near_flat", "sample_top_p_two_clusters")
SAMPLE_KERNELS = ("scale", "prob", "gather", "narrow", "select")
TRACE_CALLS = 20


def token_select_cases(pkg, torch, gen, dev, vocab=128256):
    """(name, fn(stream)) for argmax and the sampling cases of
    token_select_leg, over fresh seeded logits."""
    peaked = (3.0 * torch.randn(vocab, generator=gen, device=dev)).half()
    flat = torch.zeros(vocab, device=dev, dtype=torch.float16)
    half = torch.rand(vocab, generator=gen, device=dev) < 0.5
    two_levels = torch.where(half, 0.0, 1.0).half()
    near_flat = (1e-3 * torch.randn(vocab, generator=gen, device=dev)).half()
    clusters = (torch.where(half, 0.0, 0.3) +
                1e-3 * torch.randn(vocab, generator=gen, device=dev)).half()
    seen = torch.randint(0, vocab, (64,), generator=gen, device=dev, dtype=torch.int32)
    out = torch.empty(1, device=dev, dtype=torch.int32)

    def samp(lg):
        return lambda s: pkg.sample(lg, 0.7, 0.9, 1.1, seen, 0.5, out=out, stream=s)

    return (("argmax", lambda s: pkg.argmax(peaked, out=out, stream=s)),
            ("sample_top_p", samp(peaked)), ("sample_top_p_flat", samp(flat)),
            ("sample_top_p_two_levels", samp(two_levels)),
            ("sample_top_p_near_flat", samp(near_flat)),
            ("sample_top_p_two_clusters", samp(clusters)))


def token_select_leg(pkg, torch, gen, dev, vocab=128256):
    """Token selection after the lm_head (LlamaModel.swift:153,161): argmax
    and temperature 0.7 / top-p 0.9 / repetition penalty 1.1 sampling (u =
    0.5) over Llama 3.2's 128256 fp16 logits with 64 seen ids, for N(0, 3^2)
    logits (a nucleus of a few tokens, as for a trained model) and for the
    degenerate distributions that are the sampler's worst cases: flat (every
    token tied: the nucleus is the whole vocabulary), two tied levels (half
    the tokens at each of two probabilities), near-flat (N(0, 1e-3^2) logits:
    one level-0 bin of 128256 near-equal keys) and two dense clusters.  Each
    is a graph of 10 calls on its own stream (after one eager call there,
    which sizes the workspace); us per call includes the graph's launch gaps.
    "worst_us" is the largest sampling median."""
    res = {}
    for name, fn in token_select_cases(pkg, torch, gen, dev, vocab):
        s = torch.cuda.Stream()
        g = capture(torch, lambda: [fn(s) for _ in range(10)], s, warm=lambda: fn(s))
        res[name] = replay_stats(torch, g.replay, 10)
        del g
    res["worst_us"] = max(v["median_us"] for k, v in res.items() if k.startswith("sample_"))
    res["vocab"] = vocab
    res["launches"] = {"argmax": 2, "sample_top_p": len(SAMPLE_KERNELS)}
    return res


# ---------------------------------------------------------------- GEMMs ---

def gemm_legs(pkg, torch, gen, dev, cap, min_gb=2.0):
    """Benchmark configs 3 (M = 750 prefill gate/up + SiLU and down), 4b
    (lm_head M = 750) and 5 (LTX DiT FFN, M = 6144 bf16, and the up projection
    with fp32 activations): graphs of launches
    over weight copies rotated to >= min_gb GB (the measurement rule: one
    resident weight would be served from the 256 MB MALL, as a prefill's
    layers never are), then, for comparison, `resident`: the same launch
    repeated on one weight."""
    res = {}

    def leg(fn_w, make_w, flops, reps, wbytes):
        copies = max(2, math.ceil(min_gb * 1e9 / wbytes))
        ws = [make_w() for _ in range(copies)]
        g = capture(torch, lambda: [fn_w(w) for w in ws], cap, warm=lambda: fn_w(ws[0]))
        st = rate(replay_stats(torch, g.replay, copies), flops=flops)
        del g
        g = capture(torch, lambda: [fn_w(ws[0]) for _ in range(reps)], cap,
                    warm=lambda: fn_w(ws[0]))
        warm = rate(replay_stats(torch, g.replay, reps), flops=flops)
        del g, ws
        torch.cuda.empty_cache()
        st["weight_copies"] = copies
        st["resident"] = {k: warm[k] for k in ("median_us", "tflops", "frac_mfma")}
        return st

    def wb(N, K, sets=1):   # packed weights, scales and biases of one copy
        return sets * (N * K // 2 + 4 * N * K // 64)

    M = 750
    xa = torch.randn(M, 3072, generator=gen, device=dev).half()
    h = torch.empty(M, 8192, device=dev, dtype=torch.float16)
    res["prefill_gate_up_silu_m750"] = leg(
        lambda w: pkg.matmul_q4_silu_mul(xa, w[0], w[1], M, 3072, 8192, out=h),
        lambda: [q4(pkg, torch, 8192, 3072, gen, dev) for _ in range(2)],
        2 * 2 * M * 8192 * 3072, 10, wb(8192, 3072, 2))
    y = torch.empty(M, 3072, device=dev, dtype=torch.float16)
    res["prefill_down_m750"] = leg(
        lambda w: pkg.matmul_q4_fast(h, *_wsb(w), M, 8192, 3072, G, out=y),
        lambda: q4(pkg, torch, 3072, 8192, gen, dev),
        2 * M * 3072 * 8192, 10, wb(3072, 8192))
    yl = torch.empty(M, 128256, device=dev, dtype=torch.float16)
    res["lm_head_gemm_m750"] = leg(
        lambda w: pkg.matmul_q4_fast(xa, *_wsb(w), M, 3072, 128256, G, out=yl),
        lambda: q4(pkg, torch, 128256, 3072, gen, dev),
        2 * M * 128256 * 3072, 5, wb(128256, 3072))
    del yl
    Md = 6144
    xd = torch.randn(Md, 2048, generator=gen, device=dev).bfloat16()
    hd = torch.empty(Md, 8192, device=dev, dtype=torch.bfloat16)
    yd = torch.empty(Md, 2048, device=dev, dtype=torch.float32)
    res["dit_ffn_up_gelu_m6144_bf16"] = leg(
        lambda w: pkg.matmul_q4_ex(xd, w, Md, 8192, out=hd, epilogue=pkg.SLTX_EPI_GELU_TANH),
        lambda: q4(pkg, torch, 8192, 2048, gen, dev),
        2 * Md * 8192 * 2048, 5, wb(8192, 2048))
    res["dit_ffn_down_m6144_bf16"] = leg(
        lambda w: pkg.matmul_q4_ex(hd, w, Md, 2048, out=yd),
        lambda: q4(pkg, torch, 2048, 8192, gen, dev),
        2 * Md * 2048 * 8192, 5, wb(2048, 8192))
    # DiTLinear.applyF32in with fp32 activations (DiTModel.swift:102-125):
    # the cast with the +-65504 clamp, one pass into a per-stream buffer at
    # this output width, then the fp16 GEMM
    xf = torch.randn(Md, 2048, generator=gen, device=dev)
    res["dit_ffn_up_gelu_m6144_f32in"] = leg(
        lambda w: pkg.matmul_q4_ex(xf, w, Md, 8192, out=hd, epilogue=pkg.SLTX_EPI_GELU_TANH),
        lambda: q4(pkg, torch, 8192, 2048, gen, dev),
        2 * Md * 8192 * 2048, 5, wb(8192, 2048))
    del xd, hd, yd, xf
    torch.cuda.empty_cache()
    return res


SMALL_M = (2, 4, 8, 32, 64, 128, 256)


def small_m_legs(pkg, torch, gen, dev, cap, min_gb=2.0):
    """Small M (T5 encoder layers at S <= 256, T5Encoder.swift:140-205, and
    short prompts): the Llama gate/up + SiLU and q|k|v shapes and the T5-XXL
    shapes (K = 4096: q/k/v/o [4096 x 4096], gelu FFN wi_0/wi_1 [10240 x 4096]
    in one launch, wo [4096 x 10240]) at M in SMALL_M, each over
    weight copies rotated to >= min_gb GB, with the route each launch takes.
    GB/s = weight + activation bytes per launch / median time; bound: HBM
    (every weight byte read once per launch)."""
    shapes = (("llama_gate_up_silu", 8192, 3072, 2, "silu"),
              ("llama_qkv", 5120, 3072, 1, None),
              ("t5_attn_proj", 4096, 4096, 1, None),
              ("t5_ffn_wi_gelu", 10240, 4096, 2, "gelu"),
              ("t5_ffn_wo", 4096, 10240, 1, None))
    res = {}
    for name, N, K, nsets, epi in shapes:
        per = gemv_bytes(N, K, nsets, M=0)
        copies = max(1, math.ceil(min_gb * 1e9 / per))
        ws = [[q4(pkg, torch, N, K, gen, dev) for _ in range(nsets)] for _ in range(copies)]
        row = {"N": N, "K": K, "weight_sets": nsets, "copies": copies}
        for M in SMALL_M:
            xx = torch.randn(M, K, generator=gen, device=dev).half()
            y = torch.empty(M, N, device=dev, dtype=torch.float16)

            def run(w, xx=xx, y=y, M=M):
                if epi == "silu":
                    pkg.matmul_q4_silu_mul(xx, w[0], w[1], M, K, N, out=y)
                elif epi == "gelu":
                    pkg.matmul_q4_geglu(xx, w[0], w[1], M, K, N, out=y)
                else:
                    pkg.matmul_q4(xx, *_wsb(w[0]), M, K, N, G, out=y)

            g = capture(torch, lambda: [run(w) for w in ws], cap, warm=lambda: run(ws[0]))
            st = rate(replay_stats(torch, g.replay, copies),
                      nbytes=gemv_bytes(N, K, nsets, M=M), flops=2 * M * N * K * nsets)
            del g
            st["route"] = pkg.gemm_route(M, N, K, gated=nsets == 2)
            row[f"m{M}"] = st
        res[name] = row
        del ws
        torch.cuda.empty_cache()
    return res


# ------------------------------------------------------------ PMC modes ---

def traffic_run(pkg, torch, gen, dev, ms=(1,)):
    """Workload for the FETCH_SIZE / WRITE_SIZE passes: the fused gate/up +
    SiLU x up launch at each M of `ms` (M = 1: the dominant GEMV) 24 times
    over 12 distinct weight copies -- and, at 1 < M <= 4, the down
    projection (3072 x 8192, one weight set: the narrow route) 24 times over
    12 copies -- then one 256 MiB copy_ whose counters give the
    bytes-per-count calibration."""
    sets = [[q4(pkg, torch, 8192, 3072, gen, dev) for _ in range(2)] for _ in range(12)]
    downs = None
    for M in ms:
        x = torch.randn(M, 3072, generator=gen, device=dev).half()
        y = torch.empty(M, 8192, device=dev, dtype=torch.float16)
        for _ in range(2):
            for gate, up in sets:
                pkg.matmul_q4_silu_mul(x, gate, up, M, 3072, 8192, out=y)
        if 1 < M <= 4:
            if downs is None:
                downs = [q4(pkg, torch, 3072, 8192, gen, dev) for _ in range(12)]
            a = torch.randn(M, 8192, generator=gen, device=dev).half()
            z = torch.empty(M, 3072, device=dev, dtype=torch.float16)
            for _ in range(2):
                for w in downs:
                    pkg.linear(a, w, M, 8192, 3072, fast=True, out=z)
    src = torch.empty(256 * 2 ** 20 // 4, device=dev, dtype=torch.float32).normal_()
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    print("traffic run done", flush=True)


def gemm_pmc_run(pkg, torch, gen, dev):
    """Workload for the MFMA-utilisation passes: the M=750 prefill GEMMs
    (gate/up with SiLU x up, and down), then the wide-M route at M = 128 (the
    Llama gate/up pair, and T5 wo 4096 x 10240, which splits K), 11
    launches each (the first is the warm-up)."""
    M, K, F = 750, 3072, 8192
    x = torch.randn(M, K, generator=gen, device=dev).half()
    a = torch.randn(M, F, generator=gen, device=dev).half()
    gate = q4(pkg, torch, F, K, gen, dev)
    up = q4(pkg, torch, F, K, gen, dev)
    down = q4(pkg, torch, K, F, gen, dev)
    y = torch.empty(M, F, device=dev, dtype=torch.float16)
    z = torch.empty(M, K, device=dev, dtype=torch.float16)
    for _ in range(11):
        pkg.matmul_q4_silu_mul(x, gate, up, M, K, F, out=y)
    for _ in range(11):
        pkg.linear(a, down, M, F, K, fast=True, out=z)
    m, kt5, nt5 = 128, 10240, 4096
    x128 = x[:m].contiguous()
    wo = q4(pkg, torch, nt5, kt5, gen, dev)
    xt5 = torch.randn(m, kt5, generator=gen, device=dev).half()
    y128 = torch.empty(m, F, device=dev, dtype=torch.float16)
    zt5 = torch.empty(m, nt5, device=dev, dtype=torch.float16)
    for _ in range(11):
        pkg.matmul_q4_silu_mul(x128, gate, up, m, K, F, out=y128)
    for _ in range(11):
        pkg.linear(xt5, wo, m, kt5, nt5, fast=True, out=zt5)
    torch.cuda.synchronize()
    print("gemm pmc run done", flush=True)


def traffic_from_profiles():
    """HBM bytes per dominant launch from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, copy-calibrated), if present."""
    path = os.path.join(REPO, "profiles", "gemv_gate_up_decode_traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            try:
                return int(float(line.split(":", 1)[1].strip()))
            except ValueError:
                return None
    return None


# --------------------------------------------------------- CPU baseline ---

def cpu_baseline(runs=5):
    """The reference's CPU plan: the same dequant matmul (w = s*q + b, group 64,
    fp32 accumulate, fp16 out; gate/up with SiLU x up) as C restatements in
    oracle/q4_cpu_baseline.c -- a substitute for Swift, which is not
    installed: single-thread scalar (matmulCPU's loop order,
    LlamaModel.swift:478-493) and all-cores 8-wide SIMD (SIMD8<Float>), the
    median of `runs` wall-clock runs per config.  Config 3's scalar figure is
    timed on the first rows of x and scaled to 750 rows (the scalar loop's
    cost is linear in the rows)."""
    import numpy as np
    from oracle import q4_oracle as o
    o.cpu_lib()
    try:
        host = len(os.sched_getaffinity(0))
    except AttributeError:
        host = os.cpu_count() or 1
    threads = max(1, min(host, 16))
    configs = {
        "config1_q_proj_m1": (1, [("q_proj", 3072, 3072)], False),
        "config2_decode_layer_m1": (1, [("q_proj", 3072, 3072), ("k_proj", 1024, 3072),
                                        ("v_proj", 1024, 3072), ("o_proj", 3072, 3072),
                                        ("gate_proj", 8192, 3072), ("up_proj", 8192, 3072),
                                        ("down_proj", 3072, 8192)], True),
        "config3_prefill_m750": (750, [("gate_proj", 8192, 3072), ("up_proj", 8192, 3072),
                                       ("down_proj", 3072, 8192)], True),
    }
    out = {}
    for cname, (M, projs, silu) in configs.items():
        jobs = []
        for i, (name, N, K) in enumerate(projs):
            xx, [(w, s, b)] = o.make_inputs(M, N, K, G, seed=200 + i)
            jobs.append(o.CpuQ4(xx, w, s, b, G))
        rows = M if M == 1 else 4
        nbytes = sum(gemv_bytes(j.N, j.K, M=M) for j in jobs)
        flops = sum(2 * M * j.N * j.K for j in jobs)
        res = {"M": M, "matmuls": [n for n, _, _ in projs], "bytes": nbytes, "flops": flops}
        for kind in ("scalar", "simd"):
            ts = []
            for _ in range(runs):
                t0 = time.perf_counter()
                ys = [j.scalar(rows) if kind == "scalar" else j.simd(threads) for j in jobs]
                if silu:
                    o.c_silu_mul(ys[-3], ys[-2])
                ts.append(time.perf_counter() - t0)
            t = float(np.median(ts)) * (M / rows if kind == "scalar" else 1.0)
            res[kind] = {"us": round(t * 1e6, 1), "gbs": round(nbytes / t / 1e9, 3),
                         "gflops": round(flops / t / 1e9, 2),
                         "threads": 1 if kind == "scalar" else threads, "runs": runs,
                         **({"rows_timed": rows} if kind == "scalar" and rows != M else {})}
        out[cname] = res
    c2 = out["config2_decode_layer_m1"]["simd"]
    return {"value": c2["gbs"], "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"benchmark config 2 decode layer (7 projections + silu_mul, "
                      f"{out['config2_decode_layer_m1']['bytes']} algorithmic bytes), 8-wide "
                      f"SIMD C on {threads} threads, median of {runs} runs",
            "substitute": "C restatement of the Swift scalar / SIMD8<Float> CPU plan (no Swift "
                          "toolchain on the box)",
            "host_cpus": host, "per_config": out}


# --------------------------------------------------------- trace summary ---

def _trace_rows(folder):
    """(name, start_ns, end_ns, blocks, threads, vgpr, agpr, lds) of every
    kernel dispatch in a rocprofv3 output folder, in start order."""
    import csv
    import glob
    import sqlite3
    dbs = sorted(glob.glob(os.path.join(folder, "**", "*.db"), recursive=True))
    rows = []
    if dbs:
        for db in dbs:
            c = sqlite3.connect(db)
            try:   # blocks over every grid dimension, where the database has them
                q = c.execute("select name, start, end, grid_x, workgroup_x, vgpr_count, "
                              "accum_vgpr_count, lds_size, grid_y, workgroup_y, grid_z, "
                              "workgroup_z from kernels").fetchall()
            except sqlite3.Error:
                q = [r + (1, 1, 1, 1) for r in c.execute(
                    "select name, start, end, grid_x, workgroup_x, vgpr_count, "
                    "accum_vgpr_count, lds_size from kernels")]
            for r in q:
                blocks = int(r[3]) // max(1, int(r[4]))
                blocks *= (int(r[8] or 1) // max(1, int(r[9] or 1))) * \
                    (int(r[10] or 1) // max(1, int(r[11] or 1)))
                rows.append((r[0], int(r[1]), int(r[2]), blocks, int(r[4]), r[5], r[6], r[7]))
    else:
        for f in sorted(glob.glob(os.path.join(folder, "**", "*kernel_trace.csv"),
                                  recursive=True)):
            for r in csv.DictReader(open(f)):
                wg = int(r.get("Workgroup_Size_X", r.get("Workgroup_Size", 1)) or 1)
                gr = int(r.get("Grid_Size_X", r.get("Grid_Size", 1)) or 1)
                blocks = gr // max(1, wg)
                for d in ("Y", "Z"):   # split launches spread their blocks over y and z
                    gd = int(r.get(f"Grid_Size_{d}", 1) or 1)
                    blocks *= gd // max(1, int(r.get(f"Workgroup_Size_{d}", 1) or 1))
                rows.append((r["Kernel_Name"], int(r["Start_Timestamp"]),
                             int(r["End_Timestamp"]), blocks, wg,
                             r.get("Arch_VGPR_Count", ""), r.get("Accum_VGPR_Count", ""),
                             r.get("LDS_Block_Size", r.get("Group_Segment_Size", ""))))
    rows.sort(key=lambda r: r[1])
    return rows


def _short(name):
    n = name[5:] if name.startswith("void ") else name
    n = n.replace("sltx::", "").replace("(anonymous namespace)::", "")
    i = n.find("(")
    if i > 0 and not n.startswith("at::"):
        n = n[:i]
    return n if len(n) <= 90 else n[:87] + "..."


def summarize_trace(folder, copies=40):
    """Markdown summary of a kernel trace of this script: every kernel
    (median / mean / min / max duration per launch shape) and the dominant
    kernel's replay statistic, computed the way the bench computes avg_us:
    the trace's runs of `copies` back-to-back dominant launches (the gate/up
    graph's replays) -> the mean kernel duration of each replay -> the median
    over replays."""
    import numpy as np
    rows = _trace_rows(folder)
    if not rows:
        return f"no kernel dispatches found under {folder}"
    groups = {}
    for r in rows:
        groups.setdefault((_short(r[0]), r[3], r[4]), []).append(r)
    out = ["| kernel | blocks x threads | calls | median us | mean us | min us | max us | "
           "VGPR | AGPR | LDS B |", "|---|---|---|---|---|---|---|---|---|---|"]
    order = sorted(groups.items(), key=lambda kv: -sum(r[2] - r[1] for r in kv[1]))
    for (name, blocks, thr), rs in order[:40]:
        d = np.array([(r[2] - r[1]) / 1e3 for r in rs])
        out.append(f"| `{name}` | {blocks} x {thr} | {len(rs)} | {np.median(d):.3f} | "
                   f"{d.mean():.3f} | {d.min():.3f} | {d.max():.3f} | {rs[0][5]} | {rs[0][6]} | "
                   f"{rs[0][7]} |")
    # dominant kernel: maximal runs of consecutive dominant launches
    runs, cur = [], []
    for r in rows:
        if DOMINANT_KERNEL in r[0]:
            cur.append(r)
        else:
            if len(cur) >= copies:
                runs.append(cur)
            cur = []
    if len(cur) >= copies:
        runs.append(cur)
    reps = []
    for run in runs:
        for i in range(0, len(run) - copies + 1, copies):
            chunk = run[i:i + copies]
            reps.append(np.mean([(r[2] - r[1]) / 1e3 for r in chunk]))
    out.append("")
    if reps:
        med = float(np.median(reps))
        p25, p75 = np.percentile(reps, [25, 75])
        gbs = DOMINANT_BYTES / (med * 1e-6) / 1e9
        out += [f"dominant kernel `{DOMINANT_KERNEL}`: {len(reps)} replays of {copies} "
                f"back-to-back launches",
                f"replay_median_us: {med:.3f}",
                f"replay_p25_us: {p25:.3f}",
                f"replay_p75_us: {p75:.3f}",
                f"achieved_gbs: {gbs:.1f}",
                f"frac_of_8000_gbs: {gbs / HBM_PEAK_GBS:.4f}"]
    else:
        out.append(f"no run of {copies} back-to-back `{DOMINANT_KERNEL}` launches in the trace")
    return "\n".join(out)


def summarize_token_select_trace(folder):
    """Markdown table of a kernel trace of `bench.py --token-select`: the
    median duration of each sampler kernel per case, over the eager section's
    TRACE_CALLS calls of each case (the trace's last sampler dispatches, in
    SAMPLE_CASES order)."""
    import numpy as np
    rows = [r for r in _trace_rows(folder) if "sample_" in r[0] and "_kernel" in r[0]]
    per_call = len(SAMPLE_KERNELS)
    need = len(SAMPLE_CASES) * TRACE_CALLS * per_call
    if len(rows) < need:
        return f"expected {need} sampler dispatches in the eager section, found {len(rows)}"
    rows = rows[-need:]
    out = ["| case | " + " | ".join(f"{k} us" for k in SAMPLE_KERNELS) + " | sum us |",
           "|---|" + "---|" * (per_call + 1)]
    for ci, case in enumerate(SAMPLE_CASES):
        seg = rows[ci * TRACE_CALLS * per_call:(ci + 1) * TRACE_CALLS * per_call]
        meds = []
        for k, kname in enumerate(SAMPLE_KERNELS):
            ks = seg[k::per_call]
            assert all(f"sample_{kname}_kernel" in r[0] for r in ks), (case, kname)
            meds.append(float(np.median([(r[2] - r[1]) / 1e3 for r in ks])))
        out.append(f"| {case} | " + " | ".join(f"{m:.1f}" for m in meds) +
                   f" | {sum(meds):.1f} |")
    return "\n".join(out)


def summarize_pmc(folder):
    """Per kernel of a rocprofv3 --pmc run: dispatches and the mean value of
    each counter collected (one line per kernel and counter)."""
    import csv
    import glob
    import sqlite3
    vals = {}
    for db in sorted(glob.glob(os.path.join(folder, "**", "*.db"), recursive=True)):
        c = sqlite3.connect(db)
        for name, ctr, v in c.execute("select kernel_name, counter_name, value "
                                      "from counters_collection"):
            vals.setdefault((name, ctr), []).append(float(v))
    if not vals:
        for f in sorted(glob.glob(os.path.join(folder, "**", "*counter_collection.csv"),
                                  recursive=True)):
            for r in csv.DictReader(open(f)):
                vals.setdefault((r["Kernel_Name"], r["Counter_Name"]), []).append(
                    float(r["Counter_Value"]))
    out = []
    for (name, ctr), v in vals.items():
        out.append(f"{ctr} {len(v):5d} dispatches  mean {sum(v) / len(v):14.1f}  {_short(name)}")
    return "\n".join(out)


def summarize_small_m_trace(folder):
    """Markdown table of a kernel trace of `bench.py --small-m`: the legs run
    in SMALL_M order per shape, and each (shape, M) is one unbroken run of
    this library's dispatches (torch kernels that make the next inputs
    separate them; the one-call warm-up before each graph is dropped).  Per
    run: the kernels, blocks x threads, dispatches and the median duration of
    each kernel."""
    import numpy as np
    runs, cur = [], []
    for r in _trace_rows(folder):
        if "q4_" in r[0] and "_kernel" in r[0] and "at::" not in r[0]:
            cur.append(r)
        elif cur:
            runs.append(cur)
            cur = []
    if cur:
        runs.append(cur)
    runs = [r for r in runs if len(r) >= MIN_REPLAYS]   # drop the one-call warm-ups
    names = ["llama_gate_up_silu", "llama_qkv", "t5_attn_proj", "t5_ffn_wi_gelu", "t5_ffn_wo"]
    want = len(names) * len(SMALL_M)
    if len(runs) != want:
        return f"expected {want} runs of q4 dispatches, found {len(runs)}"
    out = ["| shape | M | kernel | blocks x threads | dispatches | median us |",
           "|---|---|---|---|---|---|"]
    for i, run in enumerate(runs):
        shape, M = names[i // len(SMALL_M)], SMALL_M[i % len(SMALL_M)]
        kinds = {}
        for r in run:
            kinds.setdefault((_short(r[0]), r[3], r[4]), []).append((r[2] - r[1]) / 1e3)
        for (k, blocks, threads), d in kinds.items():
            out.append(f"| {shape} | {M} | `{k}` | {blocks} x {threads} | {len(d)} | "
                       f"{float(np.median(d)):.2f} |")
    return "\n".join(out)


if __name__ == "__main__":
    main()
