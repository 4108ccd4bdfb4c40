#!/usr/bin/env python
"""Benchmark of the MI355X selective-scan engine (one JSON line on stdout).

Metric: selective-scan fwd+bwd Mtok/s and % HBM peak at B16 L512 D512 N16
fp32 (config 1: z gate + D skip, upstream grad dy ~ N(0,1)).  A step is one forward and one
backward of the fused scan over the batch, inputs resident in HBM.  W untimed warmup steps,
then exactly K steps between two torch.cuda.synchronize() calls.  The step is timed in three
launch modes in the same run: eager (Python + autograd launch every step; the kernels' HIP-event
timer is off in the timed loop), captured once in a HIP graph and replayed, and 10 consecutive
steps captured in one graph (as a training loop captures its iteration) replayed K/10 times;
every replayed step's outputs are checked bitwise against the eager step's.  `value` is the
fastest mode and `step_mode` names it: the eager step is host-bound when the host is busy, and
each graph replay adds a fixed launch gap of several microseconds, which the 10-step graph
pays once per 10 steps.  `--eager` times the eager step only.  Every mode's time is in the
record.

Per-entry device times come from HIP events recorded on the launch stream around every
C-ABI call (ssm_scan.KernelTimer); the dominant entry (ssm_bwd: the backward kernel plus its
small fixed-order reduction kernel) gives the roofline: algorithmic bytes per launch /
average duration, against 8 TB/s.  The CPU baseline is the torch-CPU restatement of the
reference's CPU path (oracle/cpu_chunked.py), timed on a bounded sample of the same workload.

The default c1 run appends, as extra keys of the same line, the other two north_star targets
(c2's L = 131072 fp32 forward time with the CPU baseline's seconds and cores and the GPU/CPU
time fraction; c4's decode latency per layer at batch 64) and the long-sequence fwd+bwd times
(`--no-extras` leaves them out).

Other workloads (--workload): c0 (forward, B1 L512), c2 / c2bf16 (long-sequence forward) --
both timed in the same three launch modes as c1 --
c3 (10-layer Mamba LM fwd+bwd), c4 (decode latency per layer at batch 64, HIP-graph replay),
long (B1 D512 N16 fwd+bwd at L 4096 / 16384 / 65536, the reference's bench_scan shape),
refdecode (the reference's own decode benchmark: batch 1, 11 layers, bf16 autocast),
scans (the composed path's linear-scan algorithms and discretization, GB/s per kernel),
copy (a plain device copy of known size, for PMC counter calibration).
"""

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "mamba-ssm-benchmark_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0
METRIC = "selective-scan fwd+bwd Mtok/s and % HBM peak, B16 L512 D512 N16 fp32"


def alg_bytes(B, L, D, N, s=4, gate=True, skip=True, last=True):
    """Algorithmic HBM bytes per pass: every tensor read or written once (workspace excluded).
    fwd: x, delta, B, C, z read; y written; A, D read; last written.
    bwd: x, delta, B, C, z, A, D re-read; dy read; dx, ddelta, dz, dB, dC, dA, dD written."""
    BL = B * L
    fwd = s * BL * (2 * D + 2 * N) + (s * BL * D if gate else 0) + s * BL * D + 4 * D * N \
        + (4 * D if skip else 0) + (4 * B * D * N if last else 0)
    bwd = s * BL * (2 * D + 2 * N) + (s * BL * D if gate else 0) + 4 * D * N + (4 * D if skip else 0) \
        + s * BL * D + (3 if gate else 2) * s * BL * D + 2 * s * BL * N + 4 * D * N + (4 * D if skip else 0)
    return fwd, bwd


def load_traffic(name):
    path = os.path.join(ROOT, "profiles", f"traffic_{name}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("bytes_per_launch")


def cpu_baseline_c1(t, budget_s=12.0):
    """Time oracle/cpu_chunked.fwd_bwd on batch row 0 (1 x 512 tokens) of config 1."""
    from oracle import cpu_chunked
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    rows = slice(0, 1)
    args = [t[k][rows].contiguous().float() for k in ("u", "delta")] + [t["A"]] + \
        [t[k][rows].contiguous().float() for k in ("Bm", "Cm")] + [t["D"], t["z"][rows].contiguous(),
                                                                    t["dy"][rows].contiguous()]
    cpu_chunked.fwd_bwd(*args)                      # warm-up
    reps, t0 = 0, time.perf_counter()
    while reps < 1 or (time.perf_counter() - t0 < budget_s and reps < 10000):
        cpu_chunked.fwd_bwd(*args)
        reps += 1
    dt = time.perf_counter() - t0
    tokens = args[0].shape[0] * args[0].shape[1] * reps
    return {"value": tokens / dt / 1e6, "unit": "Mtok/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"config-1 batch row 0 (1x512 tokens, D512 N16 fp32, z gate + D skip), fwd+bwd of the "
                      f"torch-CPU restatement of the reference CPU path (SelectiveScanFn + scan_chunked), "
                      f"{reps} reps in {dt:.1f} s"}


def cpu_baseline_fwd(L, budget_s=20.0, label="config-2"):
    """Time the reference CPU path's forward (oracle/cpu_chunked.fwd: SelectiveScanFn over
    channel tiles of d_block = 2^24 // (L N), scan_chunked inside) at B1 D512 N16 on a bounded
    sample: whole channel tiles, as many as fit the budget; the full forward is that time x
    (number of tiles) / (tiles run), since the tiles are independent and equal."""
    from oracle import cpu_chunked
    from ssm_scan.synthetic import baseline_inputs
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    D, N = 512, 16
    t = baseline_inputs(1, L, D, N)
    tiles = cpu_chunked._blocks(1, L, D, N)
    i, j = tiles[0]
    args = [t[k][..., i:j].contiguous() for k in ("u", "delta")] + [t["A"][i:j]] + \
        [t[k].contiguous() for k in ("Bm", "Cm")]
    cpu_chunked.fwd(*args)                          # warm-up
    reps, t0 = 0, time.perf_counter()
    while reps < 1 or (time.perf_counter() - t0 < budget_s and reps < len(tiles)):
        cpu_chunked.fwd(*args)
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    full_s = dt * len(tiles)
    return {"value": L / full_s / 1e6, "unit": "Mtok/s", "cores": torch.get_num_threads(), "kind": "port",
            "seconds_full_forward": full_s,
            "sample": f"{label} forward B1 L{L} D512 N16 fp32 on the torch-CPU restatement of the reference "
                      f"CPU path (SelectiveScanFn + scan_chunked, d_block {j - i}): {reps} of its {len(tiles)} "
                      f"independent channel tiles timed ({dt:.2f} s each), scaled to all tiles"}


def _read_first(paths, pick):
    for path in paths:
        try:
            with open(path) as f:
                v = pick(f.read())
            if v:
                return v
        except OSError:
            continue
    return None


def env_record(dev):
    """The environment the line was measured in: torch/HIP versions, the GPU, its engine-clock
    levels (sysfs pp_dpm_sclk, the current one marked *) and the host CPU model."""
    import glob
    props = torch.cuda.get_device_properties(dev)
    cpu = _read_first(["/proc/cpuinfo"], lambda t: next((ln.split(":", 1)[1].strip() for ln in t.splitlines()
                                                          if ln.startswith("model name")), None))
    sclk = _read_first(sorted(glob.glob("/sys/class/drm/card*/device/pp_dpm_sclk")),
                       lambda t: " | ".join(ln.strip() for ln in t.splitlines() if ln.strip()))
    return {"torch": torch.__version__, "hip": torch.version.hip, "gpu": props.name,
            "arch": getattr(props, "gcnArchName", None), "compute_units": props.multi_processor_count,
            "sclk_levels": sclk, "host_cpus": os.cpu_count(), "host_cpu_model": cpu}


def time_stats(samples):
    """Median, quartiles and count of a list of per-launch times (ms)."""
    if len(samples) < 2:
        return {"median": samples[0] if samples else None, "q1": None, "q3": None, "n": len(samples)}
    q = statistics.quantiles(samples, n=4)
    return {"median": statistics.median(samples), "q1": q[0], "q3": q[2], "n": len(samples)}


def flush_buffer(dev):
    return torch.empty(512 * 1024 * 1024 // 4, dtype=torch.float32, device=dev)


GRAPH_STEPS = 10  # consecutive steps captured in one graph by the multi-step graph mode


def time_steps(step, args, multi=False):
    """(eager ms/step, graph-replay ms/step or None, replay outputs == eager outputs or None).

    Eager: W warmup steps, then K steps between two synchronizations.  Graph: the step captured
    once on a side stream and replayed W + K times; the replay's outputs are compared bitwise
    with the eager step's (the kernels are deterministic).  multi=True: GRAPH_STEPS consecutive
    steps captured in one graph (as a training loop captures its iteration), replayed so that
    exactly K steps run in the timed region (K rounded up to a multiple of GRAPH_STEPS); every
    step's outputs are compared with the eager step's."""
    for _ in range(args.warmup):
        ref = step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    if args.eager:
        return eager_ms, None, None
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    per = GRAPH_STEPS if multi else 1
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gouts = [step() for _ in range(per)]
    reps = (args.steps + per - 1) // per
    for _ in range(max(1, args.warmup // per)):
        graph.replay()
    torch.cuda.synchronize()
    ok = all(torch.equal(a, b) for gout in gouts for a, b in zip(gout, ref))
    t0 = time.perf_counter()
    for _ in range(reps):
        graph.replay()
    torch.cuda.synchronize()
    return eager_ms, (time.perf_counter() - t0) * 1e3 / (reps * per), ok


def bench_c1(args, dev):
    import ssm_scan
    from ssm_scan.synthetic import baseline_inputs
    B, L, D, N = args.batch, 512, 512, 16
    t = baseline_inputs(B, L, D, N, gate=True, with_dy=True)
    names = ("u", "delta", "A", "Bm", "Cm", "D", "z")
    leaves = [t[k].to(dev).requires_grad_() for k in names]
    dy = t["dy"].to(dev)

    def step():
        out = ssm_scan.selective_scan_fn(leaves[0], leaves[1], leaves[2], leaves[3], leaves[4],
                                         D=leaves[5], z=leaves[6])
        return torch.autograd.grad(out, leaves, dy)

    eager_ms, graph_ms, graph_ok = time_steps(step, args)
    modes = {"eager launches": eager_ms}
    if graph_ok:
        modes["hip-graph replay of the fwd+bwd step"] = graph_ms
    multi_ms = multi_ok = None
    if not args.eager:
        _, multi_ms, multi_ok = time_steps(step, args, multi=True)
        if multi_ok:
            modes[f"hip-graph replay of {GRAPH_STEPS} consecutive fwd+bwd steps"] = multi_ms
    step_mode = min(modes, key=modes.get)
    ms_step = modes[step_mode]

    with ssm_scan.KernelTimer() as timer:
        for _ in range(args.steps):
            step()
    times = timer.times_ms()
    fwd_ms = statistics.mean(times["ssm_fwd"])
    bwd_ms = statistics.mean(times["ssm_bwd"])
    fb, bb = alg_bytes(B, L, D, N)

    # cold caches: flush MALL + L2 with a 512 MB write before each step (flush not timed)
    flush = flush_buffer(dev)
    with ssm_scan.KernelTimer() as cold:
        for _ in range(min(args.steps, 10)):
            flush.fill_(1.0)
            step()
    ct = cold.times_ms()
    del flush
    cold_f, cold_b = statistics.mean(ct["ssm_fwd"]), statistics.mean(ct["ssm_bwd"])
    kstats = {"ssm_fwd": time_stats(times["ssm_fwd"]), "ssm_bwd": time_stats(times["ssm_bwd"]),
              "ssm_fwd_cold": time_stats(ct["ssm_fwd"]), "ssm_bwd_cold": time_stats(ct["ssm_bwd"])}

    achieved = bb / (bwd_ms * 1e-3) / 1e9
    rec = {
        "metric": METRIC,
        "value": B * L / (ms_step * 1e-3) / 1e6,
        "unit": "Mtok/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"config 1: fused selective-scan fwd+bwd, B{B} L512 D512 N16 fp32, "
                               "zoh, z gate + D skip, channel-major (B,D,L) storage"
                               + ("" if B == 16 else " (config 1 is B16; this is a batch sweep point)"),
                   "batch": B, "seqlen": L, "dim": D, "dstate": N, "method": "zoh"},
        "hbm_frac_step": (fb + bb) / (ms_step * 1e-3) / (HBM_PEAK_GBS * 1e9),
        "step_mode": step_mode,
        "eager_ms_per_step": eager_ms, "graph_ms_per_step": graph_ms, "graph_matches_eager": graph_ok,
        "graph_multi_ms_per_step": multi_ms, "graph_multi_matches_eager": multi_ok,
        "kernels_ms": {"ssm_fwd": fwd_ms, "ssm_bwd": bwd_ms, "ssm_fwd_cold": cold_f, "ssm_bwd_cold": cold_b},
        "kernels_ms_stats": kstats,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": load_traffic("ssm_bwd_c1") if B == 16 else None,
                     "kernel": "ssm_bwd (k_bwdw + k_bwd_finalize)", "alg_bytes_per_launch": bb,
                     "fwd_achieved": fb / (fwd_ms * 1e-3) / 1e9},
    }
    if not args.no_cpu_baseline:
        rec["cpu_baseline"] = cpu_baseline_c1(t)
    return rec


def bench_fwd(args, dev, B, L, dtype, workload):
    import ssm_scan
    from ssm_scan.synthetic import baseline_inputs
    D, N = 512, 16
    t = baseline_inputs(B, L, D, N, dtype=dtype)
    ins = [t[k].to(dev) for k in ("u", "delta", "A", "Bm", "Cm")]
    Dv = t["D"].to(dev)                      # D_skip = ones(D), no gate (BASELINE configs 0 and 2)

    def step():
        with torch.no_grad():
            return ssm_scan.selective_scan_fn(*ins, D=Dv, return_last_state=True, segments=args.segments)

    eager_ms, graph_ms, graph_ok = time_steps(step, args)
    modes = {"eager launches": eager_ms}
    if graph_ok:
        modes["hip-graph replay"] = graph_ms
    multi_ms = multi_ok = None
    if not args.eager:
        _, multi_ms, multi_ok = time_steps(step, args, multi=True)
        if multi_ok:
            modes[f"hip-graph replay of {GRAPH_STEPS} consecutive forwards"] = multi_ms
    step_mode = min(modes, key=modes.get)
    ms = modes[step_mode]
    with ssm_scan.KernelTimer() as timer:
        for _ in range(args.steps):
            step()
    fwd_ms = statistics.mean(timer.times_ms()["ssm_fwd"])
    s = torch.tensor([], dtype=dtype).element_size()
    fb, _ = alg_bytes(B, L, D, N, s=s, gate=False)
    achieved = fb / (fwd_ms * 1e-3) / 1e9
    rec = {"metric": f"selective-scan fwd Mtok/s, {workload}", "value": B * L / (ms * 1e-3) / 1e6,
            "unit": "Mtok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": {torch.float32: "f32", torch.bfloat16: "bf16"}[dtype], "data": "synthetic",
            "config": {"workload": workload, "batch": B, "seqlen": L, "dim": D, "dstate": N},
            "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": achieved / HBM_PEAK_GBS, "traffic": None, "kernel": "ssm_fwd",
                         "alg_bytes_per_launch": fb},
           "segments": args.segments or "auto",
           "step_mode": step_mode, "eager_ms_per_step": eager_ms,
           "graph_ms_per_step": graph_ms, "graph_matches_eager": graph_ok,
           "graph_multi_ms_per_step": multi_ms, "graph_multi_matches_eager": multi_ok, "kernel_ms": fwd_ms}
    if not args.no_cpu_baseline and B == 1:
        cb = cpu_baseline_fwd(L, label="config-0" if L == 512 else "config-2")
        rec["cpu_baseline"] = cb
        rec["gpu_time_frac_of_cpu"] = fwd_ms * 1e-3 / cb["seconds_full_forward"]
    return rec


REF_LONG_MS = {4096: 10.7207, 16384: 41.8723, 65536: 525.1975}   # results/csv/bench_scan.csv:25-27


def bench_long(args, dev, lengths=(4096, 16384, 65536)):
    """The reference's own scan benchmark shape (benchmarks/bench_scan.py:25-66): one layer's
    scan at B1 D512 N16 fp32 for growing L, forward + backward of out.sum() (dy = ones), inputs
    as its make_inputs (x, B, C ~ N(0,1) in (B, L, .) storage, delta ~ U[1e-3, 0.101], A =
    -(1..16)), no D skip and no gate.  B x D alone leaves the GPU short of work, so forward
    and backward walk time segments.  `value` is Mtok/s at the longest L; every length's
    fwd+bwd and forward-only times are in `lengths`, beside the reference's published fused
    Triton fwd+bwd times (RTX 3050 Laptop GPU)."""
    import ssm_scan
    D, N = 512, 16
    per = {}
    for L in lengths:
        g = torch.Generator().manual_seed(0)
        x = torch.randn(1, L, D, generator=g)
        delta = torch.rand(1, L, D, generator=g) * 0.1 + 1e-3
        A = -torch.arange(1, N + 1, dtype=torch.float32).repeat(D, 1)
        Bm = torch.randn(1, L, N, generator=g)
        Cm = torch.randn(1, L, N, generator=g)
        leaves = [t.to(dev).requires_grad_() for t in (x, delta, A, Bm, Cm)]
        dy = torch.ones(1, L, D, device=dev)

        def step():
            out = ssm_scan.selective_scan_fn(*leaves)
            return torch.autograd.grad(out, leaves, dy)

        def fwd():
            with torch.no_grad():
                return (ssm_scan.selective_scan_fn(*leaves),)

        eager_ms, graph_ms, graph_ok = time_steps(step, args)
        ms = min(eager_ms, graph_ms) if graph_ok else eager_ms
        f_eager, f_graph, f_ok = time_steps(fwd, args)
        with ssm_scan.KernelTimer() as timer:
            for _ in range(min(args.steps, 20)):
                step()
        tt = timer.times_ms()
        fwd_k, bwd_k = statistics.mean(tt["ssm_fwd"]), statistics.mean(tt["ssm_bwd"])
        fb, bb = alg_bytes(1, L, D, N, gate=False, skip=False)
        per[L] = {"fwd_bwd_ms": ms, "fwd_ms": min(f_eager, f_graph) if f_ok else f_eager,
                  "kernels_ms": {"ssm_fwd": fwd_k, "ssm_bwd": bwd_k},
                  "hbm_frac_bwd": bb / (bwd_k * 1e-3) / (HBM_PEAK_GBS * 1e9),
                  "hbm_frac_fwd": fb / (fwd_k * 1e-3) / (HBM_PEAK_GBS * 1e9),
                  "graph_matches_eager": graph_ok and f_ok,
                  "reference_published_fwd_bwd_ms": REF_LONG_MS.get(L)}
        del leaves, dy, x, delta, Bm, Cm
        torch.cuda.empty_cache()
    L = max(lengths)
    top = per[L]
    value = L / (top["fwd_bwd_ms"] * 1e-3) / 1e6
    fb, bb = alg_bytes(1, L, D, N, gate=False, skip=False)
    achieved = bb / (top["kernels_ms"]["ssm_bwd"] * 1e-3) / 1e9
    ref = REF_LONG_MS.get(L)
    return {"metric": f"selective-scan fwd+bwd Mtok/s, B1 L{L} D512 N16 fp32 (reference bench_scan shape)",
            "value": value, "unit": "Mtok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": top["fwd_bwd_ms"], "higher_is_better": True, "scaling": "weak",
            "vs_baseline": value / (L / (ref * 1e-3) / 1e6) if ref else None,
            "baseline_note": "vs the reference's published fused Triton fwd+bwd time at this shape "
                             "(RTX 3050 Laptop GPU, results/csv/bench_scan.csv)",
            "dtype": "f32", "data": "synthetic",
            "config": {"workload": "config 2 shape fwd+bwd: B1 D512 N16, L in "
                                   + "/".join(str(v) for v in lengths) + ", zoh, no gate, no D skip, (B, L, D) "
                                   "storage, dy = ones (bench_scan.py's out.sum().backward())",
                       "batch": 1, "seqlen": L, "dim": D, "dstate": N, "method": "zoh"},
            "lengths": {str(k): v for k, v in per.items()},
            "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                         "kernel": "ssm_bwd (summary, carry, main pass, finalize)", "alg_bytes_per_launch": bb}}


def bench_lm(args, dev):
    """Config 3: the 10-layer byte-level Mamba LM (d_model 256, d_inner 512, N 16), forward +
    backward of the next-byte cross-entropy at B16 L512, float32, random init and random bytes.
    Scan, conv1d and RMSNorm run in the engine's kernels, the projections in torch.  Timed
    eager, with torch's backward threading on and off, the faster named in step_mode (the step
    is not captured in a HIP graph: a capture of a smaller LM step crashed
    inside the runtime's end of capture)."""
    import ssm_scan
    from ssm_scan.block import MambaLM
    torch.manual_seed(0)
    model = MambaLM(n_layers=10).to(dev)
    g = torch.Generator().manual_seed(1)
    idx = torch.randint(0, 256, (16, 513), generator=g).to(dev)
    inp, tgt = idx[:, :-1], idx[:, 1:]
    params = list(model.parameters())

    def step():
        logits = model(inp)
        loss = torch.nn.functional.cross_entropy(logits.reshape(-1, 256), tgt.reshape(-1))
        return torch.autograd.grad(loss, params)

    def timed(threaded):
        # torch runs a CUDA backward on its device worker thread by default; with it off the
        # backward runs on this thread, which saves the hand-offs between the two threads that
        # every backward node written in Python (the engine's autograd functions) costs
        with torch.autograd.set_multithreading_enabled(threaded):
            for _ in range(args.warmup):
                step()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(args.steps):
                step()
            torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / args.steps

    modes = {"eager launches, backward on the autograd worker thread": timed(True),
             "eager launches, backward on the calling thread": timed(False)}
    step_mode = min(modes, key=modes.get)
    ms = modes[step_mode]
    with ssm_scan.KernelTimer() as timer:
        for _ in range(min(args.steps, 10)):
            step()
    tt = {k: sum(v) / len(v) for k, v in timer.times_ms().items()}
    per_step = {k: tt[k] * 10 for k in tt}   # ten layers call each entry once per step
    return {"metric": "Mamba LM (10 layers, d_model 256) fwd+bwd tokens/s, B16 L512 fp32", "value": 16 * 512 / (ms * 1e-3),
            "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
            "data": "synthetic (uniform random bytes, random-init weights)",
            "config": {"workload": "config 3: byte-level Mamba LM fwd+bwd", "layers": 10, "batch": 16, "seqlen": 512,
                       "d_model": 256, "d_inner": 512, "dstate": 16, "params_non_embedding": model.num_params()},
            "step_mode": step_mode, "modes_ms_per_step": modes, "engine_ms_per_step": per_step}


def bench_decode(args, dev):
    """Config 4: recurrent decode of the config-3 model at batch 64 (fp32 state ~ N(0,1), one
    random byte per step).  The token step -- one ssm_decode_stack call: the embedding rows, two
    launches per block (the in_proj and out_proj GEMMs inside), the final norm and head in one
    more -- is timed over 256 back-to-back steps issued eagerly and as HIP-graph replays; `value`
    is the faster of the two.  Beside it: the per-block path (in_proj GEMM, the fused
    ssm_decode_step launch, out_proj + residual GEMM per block), and the module decode path
    (models/mamba.py's structure: conv step and scan step kernels between torch ops), eager and
    graph-replayed; `--decode-path stack` times the token step alone."""
    from ssm_scan.block import MambaLM
    from ssm_scan.decode import FastDecoder
    torch.manual_seed(0)
    model = MambaLM(n_layers=10).to(dev).eval()
    B = 64
    states = model.init_state(B, 1, dev)
    g = torch.Generator().manual_seed(2)
    for s in states:
        s.ssm.copy_(torch.randn(s.ssm.shape, generator=g))
        s.conv.copy_(torch.randn(s.conv.shape, generator=g))
    tok = torch.zeros(B, 1, dtype=torch.long, device=dev)
    toks = torch.randint(0, 256, (args.decode_steps + 64, B, 1), generator=g).to(dev)

    def module_step():
        with torch.no_grad():
            return model(tok, states, 0)

    fast = FastDecoder(model)
    block = FastDecoder(model, path="block")

    def fast_step():
        return fast.step(tok, states)

    def block_step():
        return block.step(tok, states)

    def eager_time(step):
        for _ in range(3):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(args.decode_steps):
            tok.copy_(toks[i])
            step()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / args.decode_steps

    def graph_time(step):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                step()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        for i in range(20):
            tok.copy_(toks[i])
            graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(args.decode_steps):
            tok.copy_(toks[i])
            graph.replay()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / args.decode_steps

    eager_ms = module_graph_ms = block_ms = None
    every_path = args.decode_path == "all"   # "stack": the token step alone (profiling runs)
    if every_path:
        eager_ms = eager_time(module_step)
        module_graph_ms = None if args.eager else graph_time(module_step)
    fast_eager_ms = eager_time(fast_step)
    if every_path and not args.eager:
        block_ms = graph_time(block_step)
    fast_graph_ms = None if args.eager else graph_time(fast_step)
    ms = min(fast_eager_ms, fast_graph_ms or fast_eager_ms)   # the faster way of issuing the same token step
    timing = "graph" if fast_graph_ms is not None and fast_graph_ms <= fast_eager_ms else "eager"
    rec_cpu = None if args.no_cpu_baseline else cpu_baseline_decode(model, B)
    return {"metric": "Mamba LM decode latency per token per layer, batch 64 (10 layers)", "value": ms * 1e3 / 10,
            "unit": "us/layer", "n_gpus": 1, "steps": args.decode_steps, "warmup": 20, "ms_per_step": ms,
            "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
            "data": "synthetic (random bytes, random-init weights, N(0,1) states)",
            "config": {"workload": f"config 4: recurrent decode step of the 10-layer LM, back-to-back token steps "
                                   f"({timing} launch, the faster of HIP-graph replay and eager) "
                                   f"({fast.path} path: " + ("ssm_decode_stack, 2 launches per layer)" if fast.path == "stack"
                                                             else "fused ssm_decode_step + 2 GEMMs per layer)"),
                       "batch": B, "layers": 10, "d_model": 256, "d_inner": 512, "dstate": 16, "conv_width": 4},
            "ms_per_token_model": ms, "timing": timing,
            "fused_ms_per_token_model": {"eager": fast_eager_ms, "graph": fast_graph_ms},
            "block_path_graph_ms_per_token_model": block_ms,
            "module_path_ms_per_token_model": {"eager": eager_ms, "graph": module_graph_ms},
            "tokens_per_s": B / (ms * 1e-3), **({"cpu_baseline": rec_cpu} if rec_cpu else {})}


REF_DECODE_MS = 0.9188  # results/csv/bench_decode.csv:9 (mamba, context 128, graph replay)


def bench_refdecode(args, dev):
    """The reference's own decode benchmark (benchmarks/bench_decode.py:27-61, the "mamba" preset
    of models/lm.py:150-152): the 11-layer Mamba LM (d_model 256), batch 1, one token step inside
    a bf16 autocast region with a bf16 conv state and a float32 SSM state (N(0,1)).  `value` is
    the fused token step FastDecoder(model) takes by default at this shape, the stack path
    (ssm_decode_stack: the embedding row, two launches per block with the in_proj, x_proj,
    dt_proj and out_proj products inside, and the final norm + head; computed in float32, the
    conv state kept in bf16) replayed from a HIP graph; `block_path_graph_ms_per_token_model`
    holds the per-block path (an in_proj GEMM, the fused decode layer and an out_proj + residual
    GEMM per block) replayed the same way; beside them the model's own decode path under
    autocast (the structure of
    models/mamba.py: the engine's conv and scan step kernels between bf16 GEMMs), eager and
    replayed.  The reference's published time is on an RTX 3050 Laptop GPU (0.919 ms/token,
    graph replay)."""
    from ssm_scan.block import MambaLM
    from ssm_scan.decode import FastDecoder
    torch.manual_seed(0)
    model = MambaLM(n_layers=11).to(dev).eval()
    g = torch.Generator().manual_seed(1)

    def fresh_states(dtype):
        st = model.init_state(1, 129, dev, dtype=dtype)
        for s_ in st:
            s_.conv.copy_(torch.randn(s_.conv.shape, generator=g))
            s_.ssm.copy_(torch.randn(s_.ssm.shape, generator=g))
        return st

    tok = torch.randint(0, 256, (1, 1), generator=g).to(dev)
    states = fresh_states(torch.bfloat16)

    def module_step():
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, cache_enabled=False):
            return model(tok, states, 128)

    fast = FastDecoder(model)
    block = FastDecoder(model, path="block")
    fstates = fresh_states(torch.bfloat16)

    def fast_step():
        with torch.autocast("cuda", dtype=torch.bfloat16, cache_enabled=False):
            return fast.step(tok, fstates)

    def block_step():
        with torch.autocast("cuda", dtype=torch.bfloat16, cache_enabled=False):
            return block.step(tok, fstates)

    def timed(fn, n):
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / n

    def graphed(step):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                step()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        return graph

    n = max(args.decode_steps, 50)
    eager_ms = timed(module_step, n)
    graph_ms = timed(graphed(module_step).replay, n)
    fast_eager_ms = timed(fast_step, n)
    block_graph_ms = timed(graphed(block_step).replay, n)
    fast_graph_ms = timed(graphed(fast_step).replay, n)
    return {"metric": "Mamba LM decode latency per token, batch 1, 11 layers, bf16 autocast (reference bench_decode)",
            "value": fast_graph_ms, "unit": "ms/token", "n_gpus": 1, "steps": n, "warmup": 10,
            "ms_per_step": fast_graph_ms, "higher_is_better": False, "scaling": "weak",
            "vs_baseline": fast_graph_ms / REF_DECODE_MS,
            "baseline_note": "value / the reference's published 0.919 ms/token (RTX 3050 Laptop GPU, graph replay, "
                             "results/csv/bench_decode.csv:9)",
            "dtype": "f32", "data": "synthetic (random byte, random-init weights, N(0,1) states)",
            "config": {"workload": "reference decode benchmark: mamba preset (11 Mamba layers, d_model 256), batch 1, "
                                   "in a bf16 autocast region, conv state bf16, ssm state f32, HIP-graph replay of the "
                                   f"fused token step (float32 compute, {fast.path} path)",
                       "batch": 1, "layers": 11, "d_model": 256, "d_inner": 512, "dstate": 16},
            "fused_ms_per_token": {"eager": fast_eager_ms, "graph": fast_graph_ms, "path": fast.path},
            "block_path_graph_ms_per_token": block_graph_ms,
            "module_path_bf16_autocast_ms_per_token": {"eager": eager_ms, "graph": graph_ms}}


def cpu_baseline_decode(model, B, budget_s=10.0):
    """The reference's decode step on the host: the torch-CPU restatement of models/mamba.py's
    recurrent step inside models/lm.py's LM (oracle/lm_ref, float32 here), one token for the
    batch through all 10 layers with conv and SSM states, repeated within a time budget."""
    from oracle import lm_ref
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    p = {k: v.detach().cpu().float() for k, v in model.state_dict().items()}
    g = torch.Generator().manual_seed(3)
    states = [{"conv": torch.randn(B, 512, 3, generator=g), "ssm": torch.randn(B, 512, 16, generator=g)}
              for _ in range(10)]
    tok = torch.randint(0, 256, (B, 1), generator=g)
    with torch.no_grad():
        lm_ref.lm_forward(p, tok, n_layers=10, states=states)
        reps, t0 = 0, time.perf_counter()
        while reps < 3 or (time.perf_counter() - t0 < budget_s and reps < 200):
            lm_ref.lm_forward(p, tok, n_layers=10, states=states)
            reps += 1
    per_tok = (time.perf_counter() - t0) / reps
    return {"value": per_tok * 1e6 / 10, "unit": "us/layer", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"batch {B}, one token through the 10-layer LM on the torch-CPU restatement of the "
                      f"reference decode path (oracle/lm_ref, float32), {reps} tokens timed"}


def bench_scans(args, dev):
    """The composed path's kernels (models/scan.py's algorithms on the engine): each linear-scan
    algorithm on (B, L, M) = (2, 4096, 16384) float32 (a, b read, h written: 3 x 4 x B L M
    algorithmic bytes), and the materialized ZOH discretization on (B, L, D, N) =
    (2, 4096, 1024, 16) (a, b written; delta, x, B read) and its backward (da, db read;
    ddelta, dx, dBm, dA written).  Device time per launch from HIP events on the launch
    stream, against 8 TB/s."""
    import ssm_scan
    from ssm_scan import scan as S
    B, L, M = 2, 4096, 16384
    g = torch.Generator().manual_seed(0)
    a = torch.rand(B, L, M, generator=g).to(dev) * 0.5 + 0.5
    b = torch.randn(B, L, M, generator=g).to(dev)
    lines = {}
    for name in ("sequential", "hillis_steele", "blelloch", "chunked"):
        fn = S.SCANS[name]
        with torch.no_grad():
            for _ in range(2):
                fn(a, b)
            with ssm_scan.KernelTimer() as tm:
                for _ in range(args.steps):
                    fn(a, b)
        t = statistics.median(tm.times_ms()["ssm_lscan"])
        nbytes = 3 * 4 * B * L * M
        lines[name] = {"ms": t, "GB/s": nbytes / (t * 1e-3) / 1e9, "frac": nbytes / (t * 1e-3) / (HBM_PEAK_GBS * 1e9),
                       "alg_bytes": nbytes}
    del a, b
    D, N = 1024, 16
    delta = (torch.rand(B, L, D, generator=g) * 0.1).to(dev)
    x = torch.randn(B, L, D, generator=g).to(dev)
    Bm = torch.randn(B, L, N, generator=g).to(dev)
    A = -torch.arange(1, N + 1, dtype=torch.float32).repeat(D, 1).to(dev)
    with torch.no_grad():
        for _ in range(2):
            S.discretize(delta, A, Bm, x)
        with ssm_scan.KernelTimer() as tm:
            for _ in range(args.steps):
                S.discretize(delta, A, Bm, x)
    t = statistics.median(tm.times_ms()["ssm_disc_fwd"])
    nbytes = 2 * 4 * B * L * D * N + 4 * (2 * B * L * D + B * L * N + D * N)
    lines["discretize_zoh"] = {"ms": t, "GB/s": nbytes / (t * 1e-3) / 1e9,
                               "frac": nbytes / (t * 1e-3) / (HBM_PEAK_GBS * 1e9), "alg_bytes": nbytes}
    # its backward: da, db read; ddelta, dx, dBm, dA written (delta, x, Bm, A re-read)
    leaves = [v.clone().requires_grad_() for v in (delta, A, Bm, x)]
    with torch.enable_grad():
        a_, b_ = S.discretize(*leaves)
    ga, gb = torch.randn_like(a_), torch.randn_like(b_)
    for _ in range(2):
        torch.autograd.grad((a_, b_), leaves, (ga, gb), retain_graph=True)
    with ssm_scan.KernelTimer() as tm:
        for _ in range(args.steps):
            torch.autograd.grad((a_, b_), leaves, (ga, gb), retain_graph=True)
    t = statistics.median(tm.times_ms()["ssm_disc_bwd"])
    nbytes = 2 * 4 * B * L * D * N + 4 * (4 * B * L * D + 2 * B * L * N + 2 * D * N)
    lines["discretize_zoh_bwd"] = {"ms": t, "GB/s": nbytes / (t * 1e-3) / 1e9,
                                   "frac": nbytes / (t * 1e-3) / (HBM_PEAK_GBS * 1e9), "alg_bytes": nbytes}
    del a_, b_, ga, gb, leaves
    best = max(lines, key=lambda k: lines[k]["frac"])
    rec = {"metric": "composed-path kernels, HBM GB/s (linear scans B2 L4096 M16384, discretize B2 L4096 D1024 N16)",
           "value": lines[best]["GB/s"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": 2,
           "ms_per_step": lines[best]["ms"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "f32", "data": "synthetic", "config": {"workload": "composed path (models/scan.py algorithms)",
                                                            "best": best},
           "kernels": lines}
    if not args.no_cpu_baseline:
        rec["cpu_baseline"] = cpu_baseline_scans(B, L, M, lines["chunked"]["ms"])
    return rec


def cpu_baseline_scans(B, L, M, gpu_ms, budget_s=10.0, m_sample=2048):
    """The reference's CPU scan (scan_chunked, models/scan.py:142-165, restated in torch in
    oracle/cpu_chunked.py) on a column sample of the scans workload; the columns are
    independent recurrences, so the full scan's time is the sample's x M / m_sample."""
    from oracle import cpu_chunked
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    g = torch.Generator().manual_seed(0)
    a = torch.rand(B, L, m_sample, generator=g) * 0.5 + 0.5
    b = torch.randn(B, L, m_sample, generator=g)
    cpu_chunked.scan_chunked(a, b)                  # warm-up
    reps, t0 = 0, time.perf_counter()
    while reps < 1 or (time.perf_counter() - t0 < budget_s and reps < 200):
        cpu_chunked.scan_chunked(a, b)
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    full_s = dt * M / m_sample
    return {"value": 3 * 4 * B * L * M / full_s / 1e9, "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port", "seconds_full_scan": full_s, "gpu_chunked_fraction": gpu_ms * 1e-3 / full_s,
            "sample": f"scan_chunked of the torch-CPU restatement of the reference (oracle/cpu_chunked.py) on "
                      f"(B, L, M) = ({B}, {L}, {m_sample}) float32, {reps} reps of {dt * 1e3:.1f} ms, scaled to "
                      f"M = {M}"}


def bench_copy(args, dev):
    """A plain device copy of 256 MiB (reads 256 MiB, writes 256 MiB): PMC calibration, and the
    read + write bandwidth a plain copy reaches (the practical ceiling of the HBM-bound kernels)."""
    src = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(args.warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(args.steps):
        dst.copy_(src)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    gbs = 2 * src.numel() * 4 / (ms * 1e-3) / 1e9
    return {"metric": "device copy 256 MiB (PMC calibration)", "value": 256.0, "unit": "MiB",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_copy": ms,
            "read_write_GBps": gbs, "frac_of_peak": gbs / HBM_PEAK_GBS}


def c1_extras(args, dev):
    """The other north_star targets and the long-sequence fwd+bwd, measured in the default run
    beside the c1 line: c2's L = 131072 fp32 forward against the CPU baseline, c4's decode
    latency per layer at batch 64 (graph replay), config 3's 10-layer LM training step (B16
    L512, eager), and B1 D512 N16 fwd+bwd at L 4096..65536."""
    sub = argparse.Namespace(**vars(args))
    sub.steps, sub.warmup = min(args.steps, 20), min(args.warmup, 5)
    sub.segments = 0
    out = {}
    c2 = bench_fwd(sub, dev, 1, 131072, torch.float32, "config 2: fwd B1 L131072 D512 N16")
    cb = c2.get("cpu_baseline", {})
    out["c2_fwd_L131072"] = {"ms": c2["ms_per_step"], "kernel_ms": c2["kernel_ms"],
                             "hbm_frac": c2["roofline"]["frac"],
                             "cpu_baseline_seconds": cb.get("seconds_full_forward"),
                             "cpu_baseline_cores": cb.get("cores"), "cpu_baseline_kind": cb.get("kind"),
                             "gpu_time_frac_of_cpu": c2.get("gpu_time_frac_of_cpu"), "target_frac": 0.02}
    torch.cuda.empty_cache()
    sub.decode_path = "stack"   # only the token step's time is reported here
    c4 = bench_decode(sub, dev)
    out["c4_decode_us_per_layer"] = c4["value"]
    out["c4_decode"] = {"us_per_layer": c4["value"], "ms_per_token_model": c4["ms_per_token_model"],
                        "step_mode": c4["timing"], "path": "ssm_decode_stack", "batch": 64, "target_us_per_layer": 20.0,
                        "cpu_baseline_us_per_layer": c4.get("cpu_baseline", {}).get("value")}
    torch.cuda.empty_cache()
    sub3 = argparse.Namespace(**vars(sub))
    sub3.steps, sub3.warmup = min(args.steps, 10), min(args.warmup, 3)
    c3 = bench_lm(sub3, dev)
    out["c3_lm"] = {"ms_per_step": c3["ms_per_step"], "tokens_per_s": c3["value"], "step_mode": c3["step_mode"],
                    "modes_ms_per_step": c3["modes_ms_per_step"],
                    "steps": sub3.steps, "engine_ms_per_step": c3["engine_ms_per_step"],
                    "workload": "config 3: 10-layer Mamba LM fwd+bwd, B16 L512 fp32, next-byte cross-entropy"}
    del c3
    torch.cuda.empty_cache()
    lg = bench_long(sub, dev)
    out["long_fwd_bwd"] = {"Mtok_s_L65536": lg["value"], "vs_reference_published": lg["vs_baseline"],
                           "lengths": {k: {"fwd_bwd_ms": v["fwd_bwd_ms"], "fwd_ms": v["fwd_ms"],
                                           "reference_published_fwd_bwd_ms": v["reference_published_fwd_bwd_ms"]}
                                       for k, v in lg["lengths"].items()}}
    return out


def parser():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="c1", choices=["c1", "c0", "c2", "c2bf16", "c3", "c4", "long", "refdecode",
                                                                 "scans", "copy"])
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--decode-path", default="all", choices=["all", "stack"],
                    help="c4: time every decode path, or only the token step FastDecoder runs")
    ap.add_argument("--seqlen", type=int, default=131072)
    ap.add_argument("--lengths", default="4096,16384,65536", help="long: the sequence lengths")
    ap.add_argument("--segments", type=int, default=0, help="forward time segments (0 = automatic)")
    ap.add_argument("--batch", type=int, default=16,
                    help="c1 only: batch rows (16 = config 1; other values are points of a batch sweep)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--eager", action="store_true", help="report the eager step (no HIP-graph replay)")
    ap.add_argument("--no-extras", action="store_true",
                    help="c1 only: skip the c2 / c4 / long-sequence keys appended to the line")
    return ap


def main():
    args = parser().parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (--gpus {args.gpus} requested): the hot path here is the "
              "single-GPU scan kernel; it is not sharded across GPUs in this build.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda", 0)
    if args.workload == "c1":
        rec = bench_c1(args, dev)
        if not args.no_extras:
            rec.update(c1_extras(args, dev))
    elif args.workload == "c0":
        rec = bench_fwd(args, dev, 1, 512, torch.float32, "config 0: fwd B1 L512 D512 N16 fp32")
    elif args.workload in ("c2", "c2bf16"):
        dt = torch.bfloat16 if args.workload == "c2bf16" else torch.float32
        rec = bench_fwd(args, dev, 1, args.seqlen, dt, f"config 2: fwd B1 L{args.seqlen} D512 N16")
    elif args.workload == "c3":
        rec = bench_lm(args, dev)
    elif args.workload == "c4":
        rec = bench_decode(args, dev)
    elif args.workload == "refdecode":
        rec = bench_refdecode(args, dev)
    elif args.workload == "long":
        rec = bench_long(args, dev, tuple(int(v) for v in args.lengths.split(",")))
    elif args.workload == "scans":
        rec = bench_scans(args, dev)
    else:
        rec = bench_copy(args, dev)
    rec["env"] = env_record(dev)
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
