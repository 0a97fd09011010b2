"""WKV-7 forward+backward throughput on one MI355X.

One step = one pass of the hot path over one batch: ``forward_with_aux``
(y, S_T and the checkpoints) followed by ``backward`` (all six vector
gradients and dS0), both through the HIP backend's callables -- the
callables the reference's FFI registry binds (src/rwkv7m/kernels/
wkv_ffi.py:21-34).  Inputs (vectors, S0, dy, dS_T) are synthetic, with the
model's input distributions, and resident in HBM before timing starts.

Three timings.  The headline: ``--settle`` untimed steps (the first few
dozen steps over freshly allocated device memory run slower), W untimed
warmup steps, then K steps back to back between two device
synchronisations; tokens/s = B*T / seconds per step, with kernel durations
from HIP events recorded on the stream the kernels run on.  ``graph``: the
same step captured once in a HIP graph and replayed (no host work between
kernels, as in the reference's compiled step).  ``reference_method``
repeats the reference's WKV microbenchmark
(scripts/benchmark_wkv_accelerator.py:88-97, :162-185): each call
host-synchronised, median / p95 / min over ``--ref-iters`` iterations, for
the forward alone and for forward+backward.
``cpu_baseline`` times the CPU restatement of the reference scan (oracle/,
fp32, OpenMP over (b, h)) on a bounded sample of the same workload on the
host cores.

Prints ONE JSON line.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--settle", type=int, default=40,
                   help="untimed steps before the warmup (the first few "
                        "dozen steps over fresh device allocations are "
                        "slower)")
    p.add_argument("--graph-steps", type=int, default=-1,
                   help="replays of the HIP-graph-captured step to time "
                        "(-1: as many as --steps; 0: skip)")
    p.add_argument("--config", type=int, default=2,
                   help="benchmark configuration index (2 = the headline shape; "
                        "3 = the decode loop)")
    p.add_argument("--chunk", type=int, default=0,
                   help="checkpoint interval / chunk length (0 = library "
                        "default)")
    p.add_argument("--head-size", type=int, default=0,
                   help="run the configuration at this head size, with H "
                        "scaled to keep H * N (0 = the configuration's N); "
                        "sizes other than 64 take the sequential kernels")
    p.add_argument("--fp32", action="store_true",
                   help="fp32 vectors instead of the configuration's bf16 "
                        "(the sequential kernels)")
    p.add_argument("--layout", choices=("tbhn", "bthn"), default="tbhn",
                   help="vector layout: time-major [T,B,H,N] (the "
                        "reference's WKV contract) or batch-major "
                        "[B,T,H,N] (the _bthn entry points)")
    p.add_argument("--path", choices=("wkv", "timemix", "screening"),
                   default="wkv",
                   help="wkv: the WKV-7 call (the headline); timemix: the "
                        "fused time-mix section around it (producers, "
                        "batch-major WKV, consumer), forward and backward; "
                        "screening: the state-level screening read path of "
                        "the 0.185B preset at config 1's B and T")
    p.add_argument("--screen-phase", default="read_screening_only",
                   choices=("read_screening_only", "read_write"),
                   help="screening phase for --path screening")
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="target CPU-baseline sample duration (0 = skip)")
    p.add_argument("--ref-iters", type=int, default=100,
                   help="iterations of the reference's per-call "
                        "synchronised timing (0 = skip)")
    p.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                   help="before warmup, run one plain device copy of this "
                        "many MiB (the reference kernel for scaling HBM "
                        "counters under rocprofv3 --pmc)")
    return p.parse_args()


def algorithmic_bytes(T, B, H, N, eb):
    """Compulsory HBM traffic: fwd reads 6 vectors and S0 and writes y and
    S_T; bwd reads 6 vectors, dy, dS_T and S0 and writes 6 gradients and
    dS0.  Checkpoint traffic is implementation overhead and not counted."""
    V = T * B * H * N * eb
    S = B * H * N * N * 4
    return 7 * V + 2 * S, 13 * V + 3 * S


def measured_traffic(kernel, config, chunk, layout="tbhn"):
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE measurement, or None if none matches."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            rows = json.load(f)["measurements"]
    except (OSError, ValueError, KeyError):
        return None
    for row in rows:
        if (row.get("kernel") == kernel and row.get("config") == config
                and row.get("chunk") == chunk
                and row.get("layout", "tbhn") == layout):
            return row.get("bytes_per_launch")
    return None


def mfma_diagnostic(kernel, config, chunk):
    """MFMA utilisation of ``kernel`` from the committed rocprofv3 counter
    run (profiles/mfma_util.json), or None if none matches."""
    path = os.path.join(ROOT, "profiles", "mfma_util.json")
    try:
        with open(path) as f:
            rows = json.load(f)["measurements"]
    except (OSError, ValueError, KeyError):
        return None
    for row in rows:
        if (row.get("kernel") == kernel and row.get("config") == config
                and row.get("chunk") == chunk):
            return {"tflops": row["mfma_tflops"], "util": row["mfma_util"],
                    "busy": row["mfma_busy"],
                    "peak_tflops": 2500.0,
                    "source": "profiles/mfma_util.json (rocprofv3 --pmc)"}
    return None


def cpu_threads():
    """(threads used, CPUs in this process's affinity set): the thread pool
    is pinned to the affinity set, one thread per CPU in it."""
    cpus = len(os.sched_getaffinity(0))
    return cpus, cpus


def timing_summary(samples_ms):
    """The reference's per-call summary (benchmark_wkv_accelerator.py:
    72-85): median, mean, min, p95 and max in milliseconds."""
    import statistics
    xs = sorted(samples_ms)
    p95 = xs[min(len(xs) - 1, int(round(0.95 * (len(xs) - 1))))]
    return {"median_ms": statistics.median(xs),
            "mean_ms": statistics.fmean(xs), "min_ms": xs[0],
            "p95_ms": p95, "max_ms": xs[-1], "iterations": len(xs)}


def per_call_timing(fn, iters, warmup=3):
    """Host-synchronised wall time of each of ``iters`` calls of fn (the
    reference's _measure, benchmark_wkv_accelerator.py:88-97)."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    samples = []
    for _ in range(iters):
        t0 = time.perf_counter_ns()
        fn()
        torch.cuda.synchronize()
        samples.append((time.perf_counter_ns() - t0) / 1e6)
    return timing_summary(samples)


def cpu_baseline(cfg, target_s):
    """Time the CPU restatement (oracle, fp32, OpenMP over (b, h)) on the
    config's (B, H, N) the reference's way (one warmup, then synchronised
    iterations, median; forward and forward+backward separately), at a
    reduced T chosen so that the iterations take about ``target_s``."""
    import numpy as np

    import oracle
    from rwkv7m_amd.synthetic import make_inputs

    threads, cpus = cpu_threads()
    B, H, N = cfg["B"], cfg["H"], cfg["N"]

    def run(T):
        """(forward seconds, backward seconds) of one iteration."""
        inp = make_inputs(T, B, H, N, dtype=cfg["dtype"], seed=7,
                          state_std=cfg.get("state_std", 0.0),
                          dstate_std=cfg.get("dstate_std", 0.0),
                          slow_decay=cfg.get("slow_decay", False))
        arrs = {k: v.float().numpy() for k, v in inp.items()}
        vecs = [arrs[n] for n in ("r", "w", "k", "v", "neg_kk", "kka")]
        t0 = time.perf_counter()
        oracle.forward(*vecs, arrs["s0"], precision="f32", threads=threads)
        t1 = time.perf_counter()
        oracle.backward(*vecs, arrs["s0"], arrs["dy"], arrs["ds_t"],
                        precision="f32", threads=threads)
        return t1 - t0, time.perf_counter() - t1

    import statistics
    probe_T = 16
    dt = sum(run(probe_T))
    # one warmup and three timed iterations in about target_s
    T = int(max(probe_T,
                min(cfg["T"], probe_T * target_s / 4 / max(dt, 1e-6))))
    run(T)
    iters = [run(T) for _ in range(3)]
    fwd = statistics.median(f for f, _ in iters)
    step = statistics.median(f + b for f, b in iters)
    return {
        "value": B * T / step,
        "unit": "tokens/s",
        "forward_tokens_per_s": B * T / fwd,
        "cores": threads,
        "threads": threads,
        "kind": "port",
        "sample": (f"fp32 C restatement of the reference scan, B={B} T={T} "
                   f"H={H} N={N}: 1 warmup + 3 iterations, median fwd+bwd "
                   f"{step:.2f} s (fwd {fwd:.2f} s), one thread per CPU of "
                   f"the affinity set ({cpus})"),
    }


def decode_cpu_baseline(cfg, target_s):
    """Time the CPU restatement (oracle, fp32, OpenMP over (b, h)) of one
    decode step at the config's (B, H, N), repeated for about target_s."""
    import oracle
    from rwkv7m_amd.synthetic import make_inputs

    threads, cpus = cpu_threads()
    B, H, N = cfg["B"], cfg["H"], cfg["N"]
    inp = make_inputs(1, B, H, N, dtype=cfg["dtype"], seed=7,
                      state_std=cfg.get("state_std", 0.0))
    arrs = {k: v.float().numpy() for k, v in inp.items()}
    vecs = [arrs[n] for n in ("r", "w", "k", "v", "neg_kk", "kka")]
    reps, dt = 0, 0.0
    while reps == 0 or dt < 0.8 * target_s:
        t0 = time.perf_counter()
        oracle.forward(*vecs, arrs["s0"], precision="f32", threads=threads)
        dt += time.perf_counter() - t0
        reps += 1
    return {
        "value": reps * B / dt,
        "unit": "tokens/s",
        "cores": threads,
        "affinity_cpus": cpus,
        "kind": "port",
        "sample": (f"fp32 C restatement of one reference step, B={B} H={H} "
                   f"N={N}, {reps} step(s), {dt:.1f} s on {threads} "
                   f"threads ({cpus} CPUs in the affinity set)"),
    }


def bench_decode(args, cfg, inp, stream):
    """Config 3: the reference's eager decode loop
    (src/rwkv7m/infer/generate.py:74-99) -- one WKV call per token with the
    whole state, updated in place, fresh vectors each step.  A step is one
    ``decode_inplace`` call; tokens/s = B per step."""
    import torch

    from rwkv7m_amd.kernels import wkv_hip
    from rwkv7m_amd.synthetic import make_inputs

    B, H, N, dtype = cfg["B"], cfg["H"], cfg["N"], cfg["dtype"]
    nsteps = args.warmup + args.steps
    seq = make_inputs(nsteps, B, H, N, dtype=dtype, seed=cfg["seed"],
                      device=stream.device, generator="torch")
    vecs = [seq[n] for n in ("r", "w", "k", "v", "neg_kk", "kka")]
    state = inp["s0"].clone()
    for t in range(args.warmup):
        wkv_hip.decode_inplace(*(x[t] for x in vecs), state)
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(2)]
           for _ in range(args.steps)]
    t0 = time.perf_counter()
    for i in range(args.steps):
        t = args.warmup + i
        evs[i][0].record(stream)
        wkv_hip.decode_inplace(*(x[t] for x in vecs), state)
        evs[i][1].record(stream)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    event_ms = sum(e[0].elapsed_time(e[1]) for e in evs) / args.steps
    ms_per_step = elapsed * 1e3 / args.steps
    # the kernel's own duration: the eager loop leaves the device idle
    # between calls (host time per call is about the kernel's), so each event
    # pair also spans part of a launch gap.  The same K steps captured in one
    # HIP graph run back to back; events around a replay give the kernel time.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        wkv_hip.decode_inplace(*(x[0] for x in vecs), state)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(args.steps):
            wkv_hip.decode_inplace(*(x[args.warmup + i] for x in vecs),
                                   state)
    graph.replay()
    torch.cuda.synchronize()
    g0 = torch.cuda.Event(enable_timing=True)
    g1 = torch.cuda.Event(enable_timing=True)
    g0.record(stream)
    graph.replay()
    g1.record(stream)
    torch.cuda.synchronize()
    kern_ms = g0.elapsed_time(g1) / args.steps
    del graph
    eb = 2 if dtype == torch.bfloat16 else 4
    step_bytes = 2 * B * H * N * N * 4 + 7 * B * H * N * eb
    achieved = step_bytes / (kern_ms / 1e3) / 1e9
    result = {
        "metric": "WKV-7 decode tokens/sec at B=256,H=64,N=64 (in place)",
        "value": B / (ms_per_step / 1e3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if eb == 2 else "f32",
        "data": "synthetic (model input distributions, device RNG)",
        "config": {
            "workload": (f"config {args.config}: WKV-7 decode B={B} H={H} "
                         f"N={N}, one token per step, state in place"),
            "B": B, "T": 1, "H": H, "N": N,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "decode",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": measured_traffic("decode", args.config, 0),
            "algorithmic_bytes": step_bytes,
            "avg_ms": kern_ms,
        },
        "kernels_ms": {"decode": kern_ms, "decode_eager_events": event_ms},
    }
    result["cpu_baseline"] = (decode_cpu_baseline(cfg, args.cpu_seconds)
                              if args.cpu_seconds > 0 else None)
    print(json.dumps(result), flush=True)

def copy_probe(mib, dev):
    """One plain device copy of ``mib`` MiB (0: none) -- the reference
    kernel for scaling HBM counters under rocprofv3 --pmc."""
    if mib <= 0:
        return
    import torch
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def timemix_cpu_baseline(cfg, target_s):
    """Time the CPU restatements of the time-mix section on the host cores:
    the numpy producers/consumer oracle (fp32 arrays) around the C WKV
    oracle (fp32, OpenMP over (b, h)), forward and backward, on the
    config's (B, H, N) at a reduced T."""
    import numpy as np

    import oracle
    from oracle import timemix_oracle as tmo

    threads, cpus = cpu_threads()
    B, H, N = cfg["B"], cfg["H"], cfg["N"]
    C = H * N
    rng = np.random.default_rng(7)

    def run(T):
        rows = B * T
        f = {n: rng.standard_normal((rows, C), dtype=np.float32)
             for n in ("w_raw", "k", "a", "r", "v", "g", "dout")}
        par = np.ones(C, np.float32)
        s0 = np.zeros((B, H, N, N), np.float32)

        def tmaj(x):
            return np.ascontiguousarray(
                x.reshape(B, T, H, N).transpose(1, 0, 2, 3))

        def bmaj(x):
            return x.transpose(1, 0, 2, 3).reshape(rows, C)

        t0 = time.perf_counter()
        w, kp, nkk, kka = tmo.wkv_inputs(f["w_raw"], f["k"], f["a"], par,
                                         par, N)
        vecs = [tmaj(x) for x in (f["r"], w, kp, f["v"], nkk, kka)]
        y, _ = oracle.forward(*vecs, s0, precision="f32", threads=threads)
        args = (bmaj(y), f["r"], kp, f["v"], f["g"], par, par, par)
        tmo.wkv_output(*args, N)
        dy, _, dk_c, *_ = tmo.wkv_output_backward(*args, f["dout"], N)
        g = oracle.backward(*vecs, s0, tmaj(dy), s0, precision="f32",
                            threads=threads)
        tmo.wkv_inputs_backward(f["w_raw"], f["k"], f["a"], par, par,
                                bmaj(g[1]), bmaj(g[2]) + dk_c, bmaj(g[4]),
                                bmaj(g[5]), N)
        return time.perf_counter() - t0

    probe_T = 16
    dt = run(probe_T)
    T = int(max(probe_T, min(cfg["T"], probe_T * target_s / max(dt, 1e-6))))
    reps, dt = 0, 0.0
    while reps == 0 or dt < 0.8 * target_s:
        dt += run(T)
        reps += 1
    return {
        "value": reps * B * T / dt,
        "unit": "tokens/s",
        "cores": threads,
        "affinity_cpus": cpus,
        "kind": "port",
        "sample": (f"numpy time-mix producers/consumer (fp32) around the "
                   f"fp32 C WKV restatement, fwd+bwd, B={B} T={T} H={H} "
                   f"N={N}, {reps} run(s), {dt:.1f} s on {threads} threads"),
    }


def bench_timemix(args, cfg):
    """The fused WKV section of the time mix (src/rwkv7m/model/
    nnx_model.py:630-727 without the projections) on batch-major [B, T, C]
    activations: producers, batch-major WKV forward_with_aux, consumer, then
    consumer, WKV (with the consumer's cotangents of r, k' and v summed into
    its stores) and producer backward -- the calls
    ``rwkv7m_amd.time_mix_wkv`` makes.  Each stage is bracketed by HIP
    events on the launch stream; the algorithmic bytes of a fused kernel
    are its activation reads and writes."""
    import torch

    from rwkv7m_amd.kernels import timemix_hip, wkv_hip

    T, B, H, N, dtype = cfg["T"], cfg["B"], cfg["H"], cfg["N"], cfg["dtype"]
    C = H * N
    dev = torch.device("cuda:0")
    copy_probe(args.copy_probe, dev)
    gen = torch.Generator(device=dev).manual_seed(cfg["seed"])

    def act(scale=1.0, shift=0.0):
        return (torch.randn(B, T, C, generator=gen, device=dev) * scale +
                shift).to(dtype)

    x = {"r": act(), "w_raw": act(0.5, -0.5), "k": act(), "v": act(),
         "a": torch.sigmoid(act().float()).to(dtype), "g": act(),
         "dout": act()}
    par = {"k_k": torch.full((C,), 0.7, device=dev),
           "k_a": torch.full((C,), 1.02, device=dev),
           "r_k": torch.full((C,), -0.04, device=dev),
           "scale": torch.full((C,), 0.8, device=dev),
           "bias": torch.zeros(C, device=dev)}
    s0 = torch.zeros(B, H, N, N, device=dev)
    ds_t = torch.zeros_like(s0)
    hv = (B, T, H, N)
    stream = torch.cuda.current_stream(dev)
    torch.cuda.synchronize()
    stages = ("inputs_fwd", "wkv_fwd", "output_fwd", "output_bwd", "wkv_bwd",
              "inputs_bwd")

    def step(evs=None):
        def mark(i):
            if evs:
                evs[i].record(stream)
        mark(0)
        w, kp, nkk, kka = (t.view(hv) for t in timemix_hip.inputs_forward(
            x["w_raw"], x["k"], x["a"], par["k_k"], par["k_a"], N))
        mark(1)
        r_h, v_h = x["r"].view(hv), x["v"].view(hv)
        vecs = (r_h, w, kp, v_h, nkk, kka, s0)
        (y, s_t), aux = wkv_hip.forward_with_aux(*vecs, layout="bthn")
        mark(2)
        out = timemix_hip.output_forward(y, r_h, kp, v_h, x["g"],
                                         par["r_k"], par["scale"],
                                         par["bias"], N)
        mark(3)
        dy, dr_c, dk_c, dv_c, dg, *pg = timemix_hip.output_backward(
            y, r_h, kp, v_h, x["g"], par["r_k"], par["scale"], par["bias"],
            x["dout"], N)
        mark(4)
        dr, dw, dk_w, dv, dnkk, dkka, ds0 = wkv_hip.backward(
            *vecs, dy, ds_t, *aux, layout="bthn",
            add=(dr_c.view(hv), dk_c.view(hv), dv_c.view(hv)))
        mark(5)
        gi = timemix_hip.inputs_backward(
            x["w_raw"], x["k"], x["a"], par["k_k"], par["k_a"], dw, dk_w,
            dnkk, dkka, N)
        mark(6)
        return out, s_t, dr, dv, dg, gi, pg, ds0

    settle(step, args.settle)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(7)]
           for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(evs[i])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    stage_ms = {name: sum(e[j].elapsed_time(e[j + 1]) for e in evs) /
                args.steps for j, name in enumerate(stages)}
    ms_per_step = elapsed * 1e3 / args.steps
    eb = 2 if dtype == torch.bfloat16 else 4
    M = B * T * C * eb
    # activations each fused kernel reads and writes (the producers'
    # backward: w_raw, k, a and the four WKV input cotangents in, three out)
    moved = {"inputs_fwd": 7 * M, "output_fwd": 6 * M, "output_bwd": 11 * M,
             "inputs_bwd": 10 * M}
    kernels = {name: {"ms": stage_ms[name],
                      "algorithmic_bytes": moved[name],
                      "GB/s": moved[name] / (stage_ms[name] / 1e3) / 1e9}
               for name in moved}
    dominant = max(moved, key=lambda n: stage_ms[n])
    ach = kernels[dominant]["GB/s"]
    result = {
        "metric": ("time-mix WKV section (fused producers + WKV-7 + "
                   "consumer) fwd+bwd tokens/sec at H=32,N=64,T=4096 bf16"),
        "value": B * T / (ms_per_step / 1e3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if eb == 2 else "f32",
        "data": "synthetic (normal activations, device RNG)",
        "config": {
            "workload": (f"config {args.config}: time-mix WKV section "
                         f"fwd+bwd B={B} T={T} H={H} N={N} batch-major "
                         f"[B,T,C] activations, fp32 state"),
            "B": B, "T": T, "H": H, "N": N, "layout": "bthn",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dominant,
            "achieved": ach,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": ach / HBM_PEAK_GBS,
            "traffic": measured_traffic(dominant, args.config, 0, "bthn"),
            "algorithmic_bytes": moved[dominant],
            "avg_ms": stage_ms[dominant],
        },
        "stages_ms": stage_ms,
        "fused_kernels": kernels,
    }
    result["cpu_baseline"] = (timemix_cpu_baseline(cfg, args.cpu_seconds)
                              if args.cpu_seconds > 0 else None)
    print(json.dumps(result), flush=True)


def screening_cpu_baseline(cfg_d, P, B, T, target_s,
                           phase="read_screening_only"):
    """Time the CPU restatement of the reference's read-only screening scan
    (numpy float64, one step per token, forward only) on a reduced T."""
    import numpy as np

    from oracle import screening_oracle as so

    C, ds, M = cfg_d["d_model"], cfg_d["d_slot"], cfg_d["n_slots"]
    rng = np.random.default_rng(7)

    def run(t):
        x = rng.normal(size=(B, t, C))
        h = rng.normal(size=(B, t, C))
        t0 = time.perf_counter()
        so.read_forward(x, h, np.zeros((B, M, ds)), np.zeros((B, M)),
                        np.zeros((B, M)), P, cfg_d, phase=phase)
        return time.perf_counter() - t0

    dt = run(8)
    t = int(max(8, min(T, 8 * target_s / max(dt, 1e-6))))
    reps, dt = 0, 0.0
    while reps == 0 or dt < 0.8 * target_s:
        dt += run(t)
        reps += 1
    return {
        "value": reps * B * t / dt,
        "unit": "tokens/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"numpy float64 per-step scan of the {phase} screening "
                   f"(the reference's algorithm), forward only, B={B} T={t}, "
                   f"{reps} run(s), {dt:.1f} s"),
    }


def bench_screening(args):
    """State-level screening read path (phase read_screening_only) of the
    0.185B preset (src/rwkv7m/model/presets.py:93-104: d_model 768,
    d_slot 128, d_k 64, d_v 64, 16 slots in banks 8/4/4) at config 1's
    B=8, T=512, bf16: one step = StateLevelScreening forward and the
    backward of all its inputs and parameters from a cotangent of h, captured
    in a HIP graph and replayed (``eager_ms_per_step``: the same step
    launched op by op).  The HIP kernels (the slot scan, or in phase
    read_write the write recurrence, and the read) are also timed alone with
    HIP events."""
    import numpy as np
    import torch

    from oracle import screening_oracle as so
    from rwkv7m_amd.kernels import screening_hip
    from rwkv7m_amd.screening import (ScreeningConfig, StateLevelScreening,
                                      init_screen_state)

    B, T = 8, 512
    cfg_d = so.default_config(d_model=768, d_slot=128, d_k=64, d_v=64,
                              n_slots=16,
                              bank_ids=(0,) * 8 + (1,) * 4 + (2,) * 4,
                              use_write_screening=True)
    phase = args.screen_phase
    cfg = ScreeningConfig(**cfg_d)
    dev = torch.device("cuda:0")
    mod = StateLevelScreening(cfg, compute_dtype=torch.bfloat16, device=dev)
    gen = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(B, T, 768, generator=gen, device=dev).to(torch.bfloat16)
    h = torch.randn(B, T, 768, generator=gen, device=dev).to(torch.bfloat16)
    x.requires_grad_(True)
    h.requires_grad_(True)
    dh = torch.randn(B, T, 768, generator=gen, device=dev).to(torch.bfloat16)
    state = init_screen_state(B, cfg, device=dev)
    state = state._replace(slots=0.1 * torch.randn(
        B, 16, 128, generator=gen, device=dev))
    stream = torch.cuda.current_stream(dev)

    def step():
        out, new, _ = mod(x, h, state, phase=phase)
        (out.float() * dh.float()).sum().backward()
        return out

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3 / args.steps

    # the same step captured once in a HIP graph and replayed: the step is
    # launch-bound (about 200 small launches for 4096 tokens)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            mod.zero_grad(set_to_none=True)
            x.grad = h.grad = None
            step()
    torch.cuda.current_stream().wait_stream(side)
    mod.zero_grad(set_to_none=True)
    x.grad = h.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        graph.replay()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps

    # the kernels alone, on the step's shapes
    base = torch.randn(B, T, 128, generator=gen, device=dev).to(torch.bfloat16)
    st = 0.3 * torch.randn(16, 128, generator=gen, device=dev)
    mu = torch.full((16,), 0.02, device=dev)
    seq, _, _ = screening_hip.slot_scan(base, st, mu, state.slots)
    proj = torch.randn(B, T, 16, 128, generator=gen, device=dev).to(
        torch.bfloat16)
    q = torch.nn.functional.normalize(
        torch.randn(B, T, 64, generator=gen, device=dev), dim=-1)
    tau = torch.tensor(-0.2, device=dev)
    du = torch.randn(B, T, 64, generator=gen, device=dev).to(torch.bfloat16)
    dseq = torch.randn_like(seq)
    calls = {
        "scan_fwd": (lambda: screening_hip.slot_scan(base, st, mu,
                                                     state.slots),
                     B * T * 128 * 2 + B * T * 16 * 128 * 2),
        "scan_bwd": (lambda: screening_hip.slot_scan_backward(
            base, st, mu, seq, dseq),
                     B * T * 128 * 2 + 2 * B * T * 16 * 128 * 2
                     + B * T * 16 * 128 * 4),
        "read_fwd": (lambda: screening_hip.read(q, proj, tau, None, cfg, 64),
                     B * T * 16 * 128 * 2 + B * T * 64 * 4 + B * T * 64 * 2),
        "read_bwd": (lambda: screening_hip.read_backward(
            q, proj, tau, None, cfg, 64, du),
                     2 * B * T * 16 * 128 * 2 + B * T * 64 * (4 + 2 + 4)),
    }
    if phase == "read_write":
        # the write-phase recurrence replaces the slot scan
        se = 0.1 * torch.randn(16, 128, generator=gen, device=dev)
        kw = torch.randn(128, 64, generator=gen, device=dev) / 128 ** 0.5
        tau_w = torch.tensor(0.1, device=dev)
        ages0 = torch.zeros(B, 16, device=dev)
        wargs = (base, st, se, kw, q, tau_w, mu, 0.05, 1e-6)
        wout = screening_hip.write(*wargs, state.slots, ages0)
        wseq, ws32 = wout[0], wout[1]
        dwseq = torch.randn_like(wseq)
        btm = B * T * 16
        del calls["scan_fwd"], calls["scan_bwd"]
        calls["write_fwd"] = (
            lambda: screening_hip.write(*wargs, state.slots, ages0),
            B * T * 128 * 2 + B * T * 64 * 4 + btm * 128 * (2 + 4)
            + btm * 16)
        calls["write_bwd"] = (
            lambda: screening_hip.write_backward(*wargs, ws32, dwseq),
            B * T * 128 * 2 + B * T * 64 * 4 + btm * 128 * (4 + 2 + 4)
            + btm * 64 * 8 + btm * 4)
    kernels = {}
    for name, (fn, nbytes) in calls.items():
        fn()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(20):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / 20
        kernels[name] = {"ms": ms, "algorithmic_bytes": nbytes,
                         "GB/s": nbytes / (ms / 1e3) / 1e9}
    dominant = max(kernels, key=lambda n: kernels[n]["ms"])
    ach = kernels[dominant]["GB/s"]
    result = {
        "metric": (f"screening {phase} fwd+bwd tokens/sec at the 0.185B "
                   "preset (B=8, T=512, bf16)"),
        "value": B * T / (ms_per_step / 1e3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (normal activations, random-init parameters)",
        "config": {
            "workload": (f"StateLevelScreening {phase} fwd+bwd, "
                         "0.185B preset (d_model 768, d_slot 128, d_k 64, "
                         "d_v 64, 16 slots), B=8 T=512"),
            "B": B, "T": T, "phase": phase,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dominant,
            "achieved": ach,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": ach / HBM_PEAK_GBS,
            "traffic": None,
            "algorithmic_bytes": kernels[dominant]["algorithmic_bytes"],
            "avg_ms": kernels[dominant]["ms"],
        },
        "screen_kernels": kernels,
        "eager_ms_per_step": eager_ms,
    }
    if args.cpu_seconds > 0:
        P = {k: np.asarray(getattr(mod, {"ln_scale": "screen_ln_scale",
                                         "ln_bias": "screen_ln_bias"}.get(
                                             k, k)).detach().double().cpu())
             for k in so.PARAM_NAMES}
        if phase == "read_write":
            for k in ("q_proj_w", "k_proj_w", "tau_w_raw"):
                P[k] = np.asarray(getattr(mod, k).detach().double().cpu())
        result["cpu_baseline"] = screening_cpu_baseline(
            cfg_d, P, B, T, args.cpu_seconds, phase)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


def graph_step_ms(step, settle_calls: int, warmup: int, steps: int) -> float:
    """Milliseconds per replay of `step` captured once in a HIP graph (its
    own memory pool, so settled again), after `warmup` untimed replays."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    settle(graph.replay, settle_calls)
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        graph.replay()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    del graph
    return ms


def settle(fn, calls: int = 40) -> None:
    """Run fn `calls` times, untimed: the first few dozen uses of freshly
    allocated device memory are slower, a one-off cost that a training loop
    pays once."""
    import torch
    for _ in range(calls):
        fn()
    torch.cuda.synchronize()


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: the WKV-7 path shards over "
              "(batch, head) with no exchange, so each GPU runs this same "
              "single-GPU kernel on its share; run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from rwkv7m_amd.kernels import wkv_hip
    from rwkv7m_amd.synthetic import CONFIGS, make_inputs

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    wkv_hip.load_library()
    cfg = dict(CONFIGS[args.config])
    variant = bool(args.head_size or args.fp32)
    if args.head_size:
        cfg["H"] = cfg["H"] * cfg["N"] // args.head_size
        cfg["N"] = args.head_size
    if args.fp32:
        cfg["dtype"] = torch.float32
    if variant and args.path != "wkv":
        print("--head-size and --fp32 apply to --path wkv", file=sys.stderr)
        sys.exit(2)
    if args.path == "timemix":
        return bench_timemix(args, cfg)
    if args.path == "screening":
        return bench_screening(args)
    T, B, H, N, dtype = cfg["T"], cfg["B"], cfg["H"], cfg["N"], cfg["dtype"]
    dev = torch.device("cuda:0")
    inp = make_inputs(T, B, H, N, dtype=dtype, seed=cfg["seed"],
                      slow_decay=cfg.get("slow_decay", False),
                      state_std=cfg.get("state_std", 0.0),
                      dstate_std=cfg.get("dstate_std", 0.0),
                      device=dev, generator="torch")
    vecs = [inp[n] for n in ("r", "w", "k", "v", "neg_kk", "kka")]
    s0, dy, ds_t = inp["s0"], inp["dy"], inp["ds_t"]
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream(dev)
    copy_probe(args.copy_probe, dev)
    if T == 1:
        return bench_decode(args, cfg, inp, stream)
    if args.layout == "bthn":
        # batch-major copies, made before the timed region
        vecs = [x.transpose(0, 1).contiguous() for x in vecs]
        dy = dy.transpose(0, 1).contiguous()
        del inp
        torch.cuda.synchronize()

    def step(evs=None):
        if evs:
            evs[0].record(stream)
        (y, s_t), aux = wkv_hip.forward_with_aux(
            *vecs, s0, checkpoint_interval=args.chunk, layout=args.layout)
        if evs:
            evs[1].record(stream)
        grads = wkv_hip.backward(*vecs, s0, dy, ds_t, *aux,
                                 layout=args.layout)
        if evs:
            evs[2].record(stream)
        return y, s_t, grads

    # settle: the step's output buffers are allocated fresh by the first
    # steps, and the first few dozen steps over freshly allocated device
    # memory run up to 25 % slower, recovering step by step (measured: the
    # same drift follows a graph capture's new pool; buffers already in use
    # show none).  A training loop pays this once; the settling steps come
    # before the warmup proper.
    settle(step, args.settle)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    # the forward / backward split from HIP events around each call, over
    # another K steps (each event adds a few microseconds between the
    # kernels, so the step time above is taken without them)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)]
           for _ in range(args.steps)]
    for i in range(args.steps):
        step(evs[i])
    torch.cuda.synchronize()

    fwd_ms = sum(e[0].elapsed_time(e[1]) for e in evs) / args.steps
    bwd_ms = sum(e[1].elapsed_time(e[2]) for e in evs) / args.steps
    ms_per_step = elapsed * 1e3 / args.steps
    eb = 2 if dtype == torch.bfloat16 else 4
    fwd_bytes, bwd_bytes = algorithmic_bytes(T, B, H, N, eb)
    tokens = B * T
    value = tokens / (ms_per_step / 1e3)

    dominant = "backward" if bwd_ms >= fwd_ms else "forward"
    dom_bytes = bwd_bytes if dominant == "backward" else fwd_bytes
    dom_ms = bwd_ms if dominant == "backward" else fwd_ms
    achieved = dom_bytes / (dom_ms / 1e3) / 1e9
    step_gbs = (fwd_bytes + bwd_bytes) / (ms_per_step / 1e3) / 1e9

    ci = args.chunk or wkv_hip.default_checkpoint_interval(dtype, N)
    result = {
        "metric": "WKV-7 fwd+bwd tokens/sec at H=32,N=64,T=4096 bf16",
        "value": value,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if dtype == torch.bfloat16 else "f32",
        "data": "synthetic (model input distributions, device RNG)",
        "config": {
            "workload": (f"config {args.config}: WKV-7 fwd+bwd B={B} T={T} "
                         f"H={H} N={N} "
                         f"{'bf16' if eb == 2 else 'fp32'} vectors "
                         f"({'time' if args.layout == 'tbhn' else 'batch'}"
                         f"-major), fp32 state"),
            "B": B, "T": T, "H": H, "N": N, "chunk": ci,
            "layout": args.layout,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dominant,
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": None if variant else measured_traffic(
                dominant, args.config, ci, args.layout),
            "algorithmic_bytes": dom_bytes,
            "avg_ms": dom_ms,
            "mfma": None if variant else mfma_diagnostic(dominant,
                                                         args.config, ci),
        },
        "kernels_ms": {"forward": fwd_ms, "backward": bwd_ms},
        "step_roofline_frac": step_gbs / HBM_PEAK_GBS,
    }
    # the same step captured once in a HIP graph and replayed (the
    # reference's step runs as one compiled XLA program, with no host work
    # between its kernels): the step without launch gaps
    gsteps = args.steps if args.graph_steps < 0 else args.graph_steps
    if gsteps > 0:
        graph_ms = graph_step_ms(step, args.settle, args.warmup, gsteps)
        result["graph"] = {"ms_per_step": graph_ms, "steps": gsteps,
                           "tokens_per_s": tokens / (graph_ms / 1e3)}
    if args.ref_iters > 0:
        # the reference's method: every call host-synchronised, median over
        # the iterations, forward alone and forward+backward
        def fwd_only():
            wkv_hip.forward(*vecs, s0, layout=args.layout)

        fwd_t = per_call_timing(fwd_only, args.ref_iters)
        step_t = per_call_timing(step, args.ref_iters)
        result["reference_method"] = {
            "forward": fwd_t,
            "forward_backward": step_t,
            "fwd_bwd_tokens_per_s_median": tokens / (step_t["median_ms"] /
                                                     1e3),
            "fwd_tokens_per_s_median": tokens / (fwd_t["median_ms"] / 1e3),
        }
    if args.cpu_seconds > 0:
        result["cpu_baseline"] = cpu_baseline(cfg, args.cpu_seconds)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
