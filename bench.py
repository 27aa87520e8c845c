#!/usr/bin/env python3
"""Benchmark of the fused causal long convolution on one MI355X.

Metric: ms per B=8 x H=768 batch (one fused launch = one step) at the workload
L=1024, fp32 I/O: u ~ N(0,1) [8,768,1024], k ~ N(0,1) exp(-n/256)/sqrt(L) [768,1024],
N=2048 two-stage 64x32 plan. Inputs are synthetic and resident in HBM before the
timed region. By default every step uses another of several disjoint (u, y, spectrum)
buffer sets totalling more than 512 MB, so the 256 MB Infinity Cache cannot hold
the working set across steps (the warm, single-buffer time is reported beside it).

Prints ONE JSON line (rank 0). Roofline: algorithmic bytes per launch =
B*H*L*(in+out bytes) + H*2L*8 (u read once, y written once, complex64 spectrum
read once) divided by the average launch duration measured with HIP events on the
launch stream, against 8 TB/s.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--B", type=int, default=8)
    ap.add_argument("--H", type=int, default=768)
    ap.add_argument("--L", type=int, default=1024)
    ap.add_argument("--io", choices=["fp32", "bf16"], default="fp32")
    ap.add_argument("--plan", default=None, help="e.g. 64x32 (default: the tuned plan for L/io)")
    ap.add_argument("--waves", type=int, default=None)
    ap.add_argument("--seqs", type=int, default=None)
    ap.add_argument("--mode", type=int, default=None, help="0: workgroup per transform, 1: wavefront per pair")
    ap.add_argument("--channels", type=int, default=None, help="mode 1: channels per workgroup")
    ap.add_argument("--acc", type=int, default=0)
    ap.add_argument("--rotate-mb", type=float, default=600.0,
                    help="minimum total size of the rotated buffer sets (0 = one warm set)")
    ap.add_argument("--cpu-baseline", type=int, default=1, help="time the fp64 CPU baseline (rank 0, N=1)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU sample budget (seconds)")
    ap.add_argument("--check", type=int, default=1, help="verify the output against the fp64 oracle")
    ap.add_argument("--work-mb", type=float, default=0.0,
                    help="multi-pass plans: workspace size in MB (0: the library's default chunking)")
    ap.add_argument("--copy-mb", type=float, default=0.0,
                    help="instead of the convolution, time a plain device-to-device copy of this many MB "
                         "(bandwidth reference and the calibration run for HBM byte counters)")
    return ap.parse_args()


def profiled_traffic(workload: str, plan) -> "int | None":
    """HBM bytes per launch measured by rocprofv3 PMC runs (FETCH_SIZE, WRITE_SIZE,
    calibrated on a plain copy) for this workload and plan, from the committed
    summaries under profiles/ (their `workload:`, `plan:` and
    `traffic_bytes_per_launch:` lines); None when no summary covers them."""
    import glob
    import re

    want_plan = (f"plan: {plan.name()} waves={plan.waves} seqs={plan.seqs} mode={plan.mode} "
                 f"channels={plan.channels}")
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*.md"))):
        text = open(path).read()
        if f"workload: {workload}\n" in text and want_plan + "\n" in text:
            m = re.search(r"^traffic_bytes_per_launch: (\d+)$", text, re.M)
            if m:
                return int(m.group(1))
    return None


def copy_reference(a):
    """Times a plain copy of known size (reads and writes copy_mb MB per step), K copies
    captured as one HIP graph and replayed between events, as the convolution is."""
    import torch

    n = int(a.copy_mb * 1e6) // 4
    x = torch.randn(n, device="cuda:0")
    y = torch.empty_like(x)
    for _ in range(a.warmup):
        y.copy_(x)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(a.steps):
            y.copy_(x)
    graph.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(torch.cuda.current_stream())
    graph.replay()
    e1.record(torch.cuda.current_stream())
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / a.steps
    gbs = 2 * n * 4 / (ms * 1e-3) / 1e9
    print(json.dumps({"copy_bytes_per_step": 2 * n * 4, "ms_per_step": ms, "GB/s": round(gbs, 1),
                      "frac_of_8TBps": round(gbs / HBM_PEAK_GBS, 4)}), flush=True)


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {a.gpus}); the convolution "
              "shards across GPUs by channel with no communication (each GPU takes H/N channels "
              "and their filters). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if a.copy_mb > 0:
        copy_reference(a)
        return
    import numpy as np
    import torch

    import sffft_amd as sf

    dev = torch.device("cuda:0")
    B, H, L, io = a.B, a.H, a.L, a.io
    base = sf.default_plan(L, io, B, acc=a.acc)
    spec, waves, seqs, mode, channels = base.name(), base.waves, base.seqs, base.mode, base.channels
    if a.plan:
        spec = a.plan
    if a.waves:
        waves = a.waves
    if a.seqs:
        seqs = a.seqs
    if a.mode is not None:
        mode = a.mode
    if a.channels:
        channels = a.channels
    if mode == 0:
        channels = 1
    plan = sf.make_plan(spec, waves, acc=a.acc, cached=1, seqs=seqs, mode=mode, channels=channels)
    rc = sf.plan_check(L, plan)
    if rc:
        raise SystemExit(f"plan {plan!r} unusable for L={L}: {sf.strerror(rc)}")

    # ---- synthetic inputs (the benchmark workload), resident in HBM -------------
    g = torch.Generator(device=dev).manual_seed(0)
    decay = 256.0 if L <= 2048 else 2048.0
    n = torch.arange(L, device=dev, dtype=torch.float32)
    s_io = 4 if io == "fp32" else 2
    set_bytes = B * H * L * 2 * s_io + H * 2 * L * 8
    # one set already larger than the rotation size defeats the Infinity Cache by itself
    nsets = 1 if a.rotate_mb <= 0 or set_bytes > a.rotate_mb * 1e6 else \
        max(3, int(np.ceil(a.rotate_mb * 1e6 / set_bytes)))
    sets = []
    for i in range(nsets):
        k = torch.randn(H, L, device=dev, generator=g) * torch.exp(-n / decay) / L ** 0.5
        u32 = torch.randn(B, H, L, device=dev, generator=g)
        u = sf.to_bf16(u32) if io == "bf16" else u32
        kf = sf.spectrum(k, L, plan)
        y = torch.empty_like(u)
        sets.append((u, kf, y, k, u32 if i == 0 else None))
    # multi-pass plans: one workspace for every step (the steps run in stream order)
    work = None
    if plan.mode == 2:
        wb = int(a.work_mb * 1e6) if a.work_mb > 0 else sf.work_bytes(B, H, L, plan)
        work = torch.empty(wb, dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()

    def step(i):
        u, kf, y = sets[i % nsets][:3]
        sf.conv(u, kf, plan, out=y, work=work)

    # ---- timed region ----------------------------------------------------------
    # W eager warmup steps; then the K steps are captured once as a HIP graph and
    # the graph is replayed between two events on the capture-replay stream (what a
    # production caller does to keep host launch overhead off the GPU timeline).
    # The same K steps launched eagerly are timed beside it.
    stream = torch.cuda.current_stream()
    for i in range(a.warmup):
        step(i)
    for i in range(nsets):  # every buffer set once more, untimed: the eager outputs
        step(i)
    torch.cuda.synchronize()
    y_eager = [s_[2].clone() for s_ in sets]

    def timed(fn, reps):
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(torch.cuda.current_stream())
        fn()
        e1.record(torch.cuda.current_stream())
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps, time.perf_counter() - t0

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(a.steps):
            step(i)
    graph.replay()  # untimed replay
    torch.cuda.synchronize()
    replay_exact = all(torch.equal(s_[2], y0) for s_, y0 in zip(sets, y_eager))
    ms, wall = timed(graph.replay, a.steps)
    replay_exact = replay_exact and all(torch.equal(s_[2], y0) for s_, y0 in zip(sets, y_eager))
    ms_eager, _ = timed(lambda: [step(i) for i in range(a.steps)], a.steps)

    # warm (single buffer set, cache-resident for small L) for comparison
    warm_graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(warm_graph):
        for i in range(a.steps):
            step(0)
    warm_graph.replay()
    ms_warm, _ = timed(warm_graph.replay, a.steps)

    # dispatch floor: a body-less kernel with the same grid, block and LDS size,
    # K launches replayed as a graph like the convolution (first call eager: it
    # sets the kernel's LDS attribute, which is not a stream operation)
    ms_floor = None
    if plan.mode != 2:  # multi-pass steps are three launches of different shapes
        sf.dispatch_floor(B, H, L, plan)
        floor_graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(floor_graph):
            for i in range(a.steps):
                sf.dispatch_floor(B, H, L, plan)
        floor_graph.replay()
        ms_floor, _ = timed(floor_graph.replay, a.steps)

    # ---- correctness of the measured configuration ----------------------------
    rel_err = None
    if a.check:
        import oracle

        u, kf, y, k, u32 = sets[0]
        step(0)
        torch.cuda.synchronize()
        nchk = min(B * H, 96 if L <= 16384 else 32)
        idx = np.linspace(0, B * H - 1, nchk).astype(np.int64)
        u_np = u32.cpu().numpy().reshape(B * H, L)[idx]  # fp32 input: bf16 error includes I/O rounding
        y_np = y.float().cpu().numpy().reshape(B * H, L)[idx]
        k_np = k.cpu().numpy()
        ks = np.stack([k_np[int(s) % H] for s in idx])
        # fp64 direct convolution (the reference's check) up to L = 16384, fp64 FFT beyond
        ref = (oracle.direct_conv if L <= 16384 else oracle.fft_conv)(u_np[None], ks)[0]
        rel_err = oracle.rel_l2(y_np, ref)

    algo_bytes = B * H * L * 2 * s_io + H * 2 * L * 8
    achieved = algo_bytes / (ms * 1e-3) / 1e9

    # ---- CPU baseline: the reference's fp64 direct convolution (oracle port) ----
    # A bounded sample of the same workload: whole-batch passes repeated for about
    # cpu_seconds when a pass is short, otherwise the first sequences of one pass.
    cpu = None
    if a.cpu_baseline:
        import oracle

        cores = oracle.threads()
        u, k = sets[0][4], sets[0][3]
        u_np = u.cpu().numpy()
        k_np = k.cpu().numpy()
        t1 = time.perf_counter()
        oracle.direct_conv(u_np[:1, :1], k_np[:1], nthreads=1)
        per_seq = max(time.perf_counter() - t1, 1e-6)
        est_batch = per_seq * B * H / cores
        if est_batch <= a.cpu_seconds:
            reps, done = 0, 0.0
            t1 = time.perf_counter()
            while done < a.cpu_seconds or reps == 0:
                oracle.direct_conv(u_np, k_np, nthreads=cores)
                reps += 1
                done = time.perf_counter() - t1
            value = done * 1e3 / reps
            sample = (f"fp64 direct convolution (src/sffft.cu:377 loop order) of the whole batch "
                      f"({B * H} sequences at L={L}) repeated {reps} times, {done:.1f} s on {cores} threads")
        else:
            nseq = max(cores, int(a.cpu_seconds * cores / per_seq) // cores * cores)
            us = u_np.reshape(B * H, L)[:nseq].reshape(1, nseq, L)
            ks = np.stack([k_np[s_ % H] for s_ in range(nseq)])
            t1 = time.perf_counter()
            oracle.direct_conv(us, ks, nthreads=cores)
            done = time.perf_counter() - t1
            value = done * 1e3 * (B * H) / nseq
            sample = (f"fp64 direct convolution (src/sffft.cu:377 loop order) of the first {nseq} of {B * H} "
                      f"sequences at L={L}, {done:.1f} s on {cores} threads, scaled linearly to the batch")
        cpu = {"value": round(value, 3), "unit": "ms per batch", "cores": cores, "kind": "port", "sample": sample}

    out = {
        "metric": "ms per B=8xH=768 batch vs L (fp32/bf16 I/O); % HBM roofline; rel L2 err",
        "value": round(ms, 6),
        "unit": "ms",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 MFMA operands, f32 accumulate",
        "data": "synthetic (u ~ N(0,1), k ~ N(0,1) exp(-n/%g)/sqrt(L), torch.Generator seed 0)" % decay,
        "config": {"workload": f"causal long convolution B={B} H={H} L={L} {io} I/O", "B": B, "H": H, "L": L,
                   "io": io, "plan": plan.name(), "waves": plan.waves, "seqs_per_transform": plan.seqs,
                   "mode": ("workgroup per transform", "wavefront per pair",
                            "multi-pass: columns, rows, columns; complex fp16 workspace")[plan.mode],
                   "channels_per_workgroup": plan.channels,
                   "acc": "fp16" if plan.acc else "fp32", "rotated_sets": nsets,
                   "workspace_bytes": None if work is None else work.numel(),
                   "rotated_bytes": nsets * set_bytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic(f"B={B} H={H} L={L} {io}", plan)},
        "cpu_baseline": cpu,
        "ms_warm": round(ms_warm, 6),
        "ms_eager": round(ms_eager, 6),
        "ms_dispatch_floor": None if ms_floor is None else round(ms_floor, 6),
        "io_only_frac": round(B * H * L * 2 * s_io / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "timing": "HIP graph of the K steps replayed between events; ms_eager: the same steps launched one by one",
        "graph_replay_bitexact": bool(replay_exact),
        "rel_l2_vs_fp64": rel_err,
        "algorithmic_bytes": algo_bytes,
        "wall_s": round(wall, 3),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
