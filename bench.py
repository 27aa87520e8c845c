#!/usr/bin/env python3
"""Benchmark of the fused causal long convolution on one MI355X.

Metric: ms per B=8 x H=768 batch vs L (fp32/bf16 I/O), % of the HBM roofline, rel-L2
error. One step = one fused launch over one batch. The headline (`value`) is the
workload L=1024, fp32 I/O: u ~ N(0,1) [8,768,1024], k ~ N(0,1) exp(-n/256)/sqrt(L)
[768,1024], N=2048 two-stage 64x32 plan. The `sweep` key carries every L from 128 to
8192 in fp32 and bf16 I/O (the reference's README table, src/sffft.cu:506-513), each
beside the rocFFT pad/R2C/multiply/C2R/slice pipeline timed the same way.

Inputs are synthetic and resident in HBM before the timed region. Every step uses
another of several disjoint (u, y, spectrum) buffer sets totalling more than 512 MB, so
the 256 MB Infinity Cache cannot hold the working set across steps (the warm,
single-buffer time is reported beside it). The K steps are captured once as a HIP graph;
before the start event the stream runs a spin kernel long enough for the host to enqueue
the whole replay, so the events bracket back-to-back dispatches only, not the host's
launch latency.

Prints ONE JSON line (rank 0). Roofline: algorithmic bytes per launch =
B*H*L*(in+out bytes) + H*2L*8 (u read once, y written once, complex64 spectrum read
once) divided by the average launch duration measured with HIP events on the launch
stream, against 8 TB/s.
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
SWEEP_LENGTHS = (128, 256, 512, 1024, 2048, 4096, 8192)


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
    ap.add_argument("--repeats", type=int, default=5,
                    help="timed replays of the K-step graph per measurement; ms is their median")
    ap.add_argument("--configs", type=int, default=1,
                    help="also time the other benchmark configurations (the `configs` key): L=2048 bf16 "
                         "16x16x16 with fp32 and fp16 accumulation, and B=4 H=1536 L=16384 bf16")
    ap.add_argument("--gpu-warm-ms", type=float, default=300.0,
                    help="before the timed steps, replay the captured steps for about this long so the GPU "
                         "runs at its steady clocks (untimed)")
    ap.add_argument("--rotate-mb", type=float, default=600.0,
                    help="minimum total size of the rotated buffer sets (0 = one warm set)")
    ap.add_argument("--sweep", type=int, default=1,
                    help="also time every L of the reference table (128..8192) in fp32 and bf16 I/O "
                         "with the rocFFT pipeline beside each (the `sweep` key)")
    ap.add_argument("--cpu-baseline", type=int, default=1, help="time the fp64 CPU baseline (rank 0, N=1)")
    ap.add_argument("--cpu-seconds", type=float, default=8.0, help="CPU sample budget per leg (seconds)")
    ap.add_argument("--check", type=int, default=1, help="verify every output against the fp64 oracle")
    ap.add_argument("--work-mb", type=float, default=0.0,
                    help="multi-pass plans: workspace size in MB (0: the library's default chunking)")
    ap.add_argument("--floor-shapes", type=int, default=0,
                    help="1: instead of the convolution, time the body-less kernel over a set of launch shapes "
                         "(the dispatch floor against grid, block and LDS size)")
    ap.add_argument("--copy-mb", type=float, default=0.0,
                    help="instead of the convolution, time a plain device-to-device copy of this many MB "
                         "(bandwidth reference and the calibration run for HBM byte counters)")
    return ap.parse_args()


def profiled_traffic(workload: str, plan, stamp: str) -> "int | None":
    """HBM bytes per launch measured by rocprofv3 PMC runs (FETCH_SIZE, WRITE_SIZE,
    calibrated on a plain copy) for this workload and plan, from the committed
    summaries under profiles/ (their `workload:`, `plan:`, `kernel_sources_sha:` and
    `traffic_bytes_per_launch:` lines). Only a summary measured on a build of the same
    kernel sources counts; None otherwise."""
    import glob
    import re

    want_plan = (f"plan: {plan.name()} waves={plan.waves} seqs={plan.seqs} mode={plan.mode} "
                 f"channels={plan.channels}")
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*.md"))):
        text = open(path).read()
        if (f"workload: {workload}\n" in text and want_plan + "\n" in text
                and f"kernel_sources_sha: {stamp}\n" in text):
            m = re.search(r"^traffic_bytes_per_launch: (\d+)$", text, re.M)
            if m:
                return int(m.group(1))
    return None


class Cover:
    """A spin kernel (torch.cuda._sleep) queued ahead of a timed region keeps the GPU busy
    while the host enqueues the region's launches, so the start event is followed by
    back-to-back dispatches and the host's launch latency stays outside the events."""

    def __init__(self):
        import torch

        self.torch = torch
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1 << 16)  # first launch loads the kernel
        e0.record()
        torch.cuda._sleep(1 << 22)
        e1.record()
        torch.cuda.synchronize()
        self.cycles_per_ms = (1 << 22) / max(e0.elapsed_time(e1), 1e-3)

    def __call__(self, ms: float) -> int:
        cycles = int(self.cycles_per_ms * ms)
        self.torch.cuda._sleep(cycles)
        return cycles


class Clocks:
    """GFX clock (SCLK), memory clock (MCLK), socket power, hotspot temperature and GFX
    activity of the GPU behind cuda:0, read through amdsmi (matched by PCI address).
    start() begins sampling every couple of milliseconds on a host thread, stop() returns the
    median, min and max of each field over the samples and how many distinct readings there
    were. On the boxes measured the metrics table refreshed far more slowly than the timed
    regions last (one reading through a whole 300 ms window, idle values during load), so
    the GFX clock of a timed region comes from its spin kernel instead (events_ms); these
    readings describe the box, not the region. Reading only; an "error" entry where the
    library or the device is unavailable."""

    FIELDS = (("sclk_mhz", ("current_gfxclk", "current_gfxclks", "average_gfxclk_frequency")),
              ("mclk_mhz", ("current_uclk", "average_uclk_frequency")),
              ("power_w", ("current_socket_power", "average_socket_power")),
              ("hotspot_c", ("temperature_hotspot",)),
              ("gfx_activity_pct", ("average_gfx_activity",)))

    def __init__(self, period_s=0.002):
        self.h, self.error, self.period = None, None, period_s
        self._thread, self._samples = None, []
        try:
            import amdsmi
            import torch

            self.amdsmi = amdsmi
            amdsmi.amdsmi_init()
            p = torch.cuda.get_device_properties(0)
            want = f"{p.pci_domain_id:04x}:{p.pci_bus_id:02x}:{p.pci_device_id:02x}"
            handles = amdsmi.amdsmi_get_processor_handles()
            for h in handles:
                if amdsmi.amdsmi_get_gpu_device_bdf(h).lower().startswith(want):
                    self.h = h
            if self.h is None and len(handles) == 1:
                self.h = handles[0]
            if self.h is None:
                self.error = f"no amdsmi device at {want}"
        except Exception as e:  # noqa: BLE001  (reported, never fatal)
            self.error = f"{type(e).__name__}: {e}"

    @staticmethod
    def _num(v):
        if isinstance(v, (list, tuple)):
            vals = [x for x in v if isinstance(x, (int, float)) and 0 < x < 1 << 31]
            return round(sum(vals) / len(vals), 1) if vals else None
        return v if isinstance(v, (int, float)) and 0 <= v < 1 << 31 else None

    def read(self):
        """One sample: {field: value or None}, or {"error": ...}."""
        if self.h is None:
            return {"error": self.error}
        try:
            m = self.amdsmi.amdsmi_get_gpu_metrics_info(self.h)
        except Exception as e:  # noqa: BLE001
            return {"error": f"{type(e).__name__}: {e}"}
        out = {}
        for key, names in self.FIELDS:
            out[key] = None
            for n in names:
                v = self._num(m.get(n))
                if v is not None:
                    out[key] = v
                    break
        return out

    def start(self):
        import threading

        self._samples = []
        if self.h is None:
            return
        self._stop = threading.Event()

        def run():
            while not self._stop.is_set():
                self._samples.append(self.read())
                self._stop.wait(self.period)

        self._thread = threading.Thread(target=run, daemon=True)
        self._thread.start()

    def stop(self):
        import statistics

        if self._thread is None:
            return {"error": self.error}
        self._stop.set()
        self._thread.join()
        self._thread = None
        good = [x for x in self._samples if "error" not in x]
        out = {"samples": len(good), "distinct": len({tuple(sorted(x.items())) for x in good})}
        for key, _ in self.FIELDS:
            vals = [x[key] for x in good if x.get(key) is not None]
            out[key] = ({"median": statistics.median(vals), "min": min(vals), "max": max(vals)} if vals else None)
        return out


def clock_brief(c):
    """The spin-measured GFX clock of the timed replays and the amdsmi power reading, for
    the progress lines."""
    import statistics

    spin = c.get("sclk_mhz_spin") or []
    a = c.get("amdsmi") or {}
    pw = a.get("power_w") if isinstance(a, dict) else None
    return (f"sclk {statistics.median(spin) if spin else None} MHz (spin), amdsmi "
            f"{pw['median'] if isinstance(pw, dict) else None} W")


def events_ms(cover, fn, reps, host_ms, sclk=None):
    """Average ms per rep of fn() between two events on the current stream, with the
    spin kernel covering the host's enqueue time (host_ms, measured beforehand). The spin
    counts shader-clock cycles (s_memtime), so its own duration gives the GFX clock just
    before the timed region: appended to `sclk` in MHz when a list is given."""
    import torch

    torch.cuda.synchronize()
    es, e0, e1 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
    es.record()
    cycles = cover(max(0.3, 3.0 * host_ms + 0.1))
    e0.record()
    fn()
    e1.record()
    torch.cuda.synchronize()
    if sclk is not None:
        sclk.append(round(cycles / es.elapsed_time(e0) / 1e3, 1))
    return e0.elapsed_time(e1) / reps


def host_time_ms(fn):
    import torch

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    fn()
    t1 = time.perf_counter()
    torch.cuda.synchronize()
    return (t1 - t0) * 1e3


def reference_protocol_ms(cover, fn, L):
    """src/sffft.cu:321-327: 3 warm-ups, synchronise, an event pair around
    clamp(20000/L, 10, 200) back-to-back launches on one buffer set. The launches are
    eager, as in the reference; the spin kernel covers their host enqueue time so the
    events see the GPU's back-to-back dispatches (the reference enqueues from C++, whose
    launch rate keeps ahead of the GPU; this process enqueues through Python)."""
    import torch

    iters = min(200, max(10, 20000 // L))
    for _ in range(3):
        fn()
    run = lambda: [fn() for _ in range(iters)]  # noqa: E731
    return events_ms(cover, run, iters, host_time_ms(run))


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
    host = host_time_ms(graph.replay)
    ms = events_ms(Cover(), graph.replay, a.steps, host)
    gbs = 2 * n * 4 / (ms * 1e-3) / 1e9
    print(json.dumps({"copy_bytes_per_step": 2 * n * 4, "ms_per_step": ms, "GB/s": round(gbs, 1),
                      "frac_of_8TBps": round(gbs / HBM_PEAK_GBS, 4)}), flush=True)


FLOOR_SHAPES = ((1, 64, 0), (256, 768, 129024), (256, 768, 0), (256, 256, 129024), (256, 256, 0),
                (256, 1024, 0), (768, 256, 92160), (768, 256, 0), (3072, 256, 40960), (3072, 256, 0),
                (6144, 128, 9216), (6144, 128, 0))


def floor_shapes(a):
    """The dispatch floor per launch shape (grid workgroups, block lanes, LDS bytes): K
    launches of the body-less kernel captured as one HIP graph and replayed between events,
    as the convolution is; median of `repeats` replays per shape. Separates what the launch
    shape of a plan controls (workgroup count, size, LDS request) from the per-kernel cost."""
    import statistics

    import torch

    import sffft_amd as sf

    cover = Cover()
    rows = []
    for grid, block, lds in FLOOR_SHAPES:
        sf.dispatch_floor_shape(grid, block, lds)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(a.steps):
                sf.dispatch_floor_shape(grid, block, lds)
        graph.replay()
        host = host_time_ms(graph.replay)
        runs = [events_ms(cover, graph.replay, a.steps, host) for _ in range(max(1, a.repeats))]
        rows.append({"grid": grid, "block": block, "lds_bytes": lds, "us": round(statistics.median(runs) * 1e3, 3),
                     "us_min": round(min(runs) * 1e3, 3)})
        print(f"# floor grid {grid} block {block} lds {lds}: {rows[-1]['us']:.3f} us", file=sys.stderr, flush=True)
    print(json.dumps({"dispatch_floor_shapes": rows, "steps": a.steps, "repeats": a.repeats}), flush=True)


def sinusoid_filters(torch, dev, H, L, g):
    """Hyena-style long filters: k[h, n] = sum_{i<16} A_hi sin(w_hi n) exp(-a_h n) with
    w ~ U(0, pi), A ~ N(0, 1) and a_h log-uniform in [1e-4, 1e-2], evaluated in float64 on
    the device (128 channels at a time), returned as float32."""
    import math

    w = torch.rand(H, 16, device=dev, dtype=torch.float64, generator=g) * math.pi
    amp = torch.randn(H, 16, device=dev, dtype=torch.float64, generator=g)
    lo, hi = math.log(1e-4), math.log(1e-2)
    alpha = torch.exp(lo + (hi - lo) * torch.rand(H, device=dev, dtype=torch.float64, generator=g))
    n = torch.arange(L, device=dev, dtype=torch.float64)
    k = torch.empty(H, L, device=dev, dtype=torch.float64)
    for h in range(0, H, 128):
        s = slice(h, h + 128)
        k[s] = (amp[s, :, None] * torch.sin(w[s, :, None] * n)).sum(1) * torch.exp(-alpha[s, None] * n)
    return k.float()


def make_workload(sf, torch, dev, B, H, L, io, plan, rotate_mb, seed=0, filters="decay"):
    """Rotated (u, spectrum, y) buffer sets of the benchmark workload, synthetic, in HBM.
    filters: "decay" (k ~ N(0,1) exp(-n/decay)/sqrt(L)) or "sines" (sinusoid_filters)."""
    import numpy as np

    g = torch.Generator(device=dev).manual_seed(seed)
    decay = 256.0 if L <= 2048 else 2048.0
    n = torch.arange(L, device=dev, dtype=torch.float32)
    s_io = 4 if io == "fp32" else 2
    set_bytes = B * H * L * 2 * s_io + H * 2 * L * 8
    # one set already larger than the rotation size defeats the Infinity Cache by itself
    nsets = 1 if rotate_mb <= 0 or set_bytes > rotate_mb * 1e6 else max(3, int(np.ceil(rotate_mb * 1e6 / set_bytes)))
    sets = []
    for i in range(nsets):
        if filters == "sines":
            k = sinusoid_filters(torch, dev, H, L, g)
        else:
            k = torch.randn(H, L, device=dev, generator=g) * torch.exp(-n / decay) / L ** 0.5
        u32 = torch.randn(B, H, L, device=dev, generator=g)
        u = sf.to_bf16(u32) if io == "bf16" else u32
        kf = sf.spectrum(k, L, plan)
        y = torch.empty_like(u)
        sets.append({"u": u, "kf": kf, "y": y, "k": k, "u32": u32 if i == 0 else None})
    return sets, decay, set_bytes


def time_fused(sf, torch, cover, sets, plan, steps, warmup, work=None, warm=True, gpu_warm_ms=0.0, repeats=5,
               clocks=None):
    """K graph-replayed steps over the rotated sets, timed `repeats` times: ms per step as the
    median of the replays, with their min, max and every value; the GPU clocks before and
    after the timed replays; the same steps launched eagerly; the warm single-set time (median
    of as many replays); and whether the replays reproduced the eager outputs bit for bit.
    Before the timed replays the captured steps are replayed, untimed, for about gpu_warm_ms,
    so the GPU leaves its idle clocks first."""
    import statistics

    nsets = len(sets)

    def step(i):
        s = sets[i % nsets]
        sf.conv(s["u"], s["kf"], plan, out=s["y"], work=work)

    for i in range(warmup):
        step(i)
    for i in range(nsets):  # every buffer set once more, untimed: the eager outputs
        step(i)
    torch.cuda.synchronize()
    y_eager = [s["y"].clone() for s in sets]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(steps):
            step(i)
    graph.replay()  # untimed replay
    if clocks:  # sampled through the untimed and the timed replays
        clocks.start()
    t_warm = time.perf_counter()
    while (time.perf_counter() - t_warm) * 1e3 < gpu_warm_ms:
        graph.replay()
        torch.cuda.synchronize()
    host = host_time_ms(graph.replay)
    exact = all(torch.equal(s["y"], y0) for s, y0 in zip(sets, y_eager))
    sclk = []
    runs = [events_ms(cover, graph.replay, steps, host, sclk) for _ in range(max(1, repeats))]
    clk = clocks.stop() if clocks else {}
    clk = {"sclk_mhz_spin": sclk, "amdsmi": clk}
    exact = exact and all(torch.equal(s["y"], y0) for s, y0 in zip(sets, y_eager))
    eager = lambda: [step(i) for i in range(steps)]  # noqa: E731
    ms_eager = events_ms(cover, eager, steps, host_time_ms(eager))
    del y_eager
    ms_warm = None
    if warm:
        warm_graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(warm_graph):
            for i in range(steps):
                step(0)
        warm_graph.replay()
        host_w = host_time_ms(warm_graph.replay)
        ms_warm = statistics.median(events_ms(cover, warm_graph.replay, steps, host_w)
                                    for _ in range(max(1, repeats)))
        del warm_graph
    del graph
    return {"ms": statistics.median(runs), "ms_min": min(runs), "ms_max": max(runs), "ms_runs": runs,
            "ms_eager": ms_eager, "ms_warm": ms_warm, "exact": exact, "step": step,
            "clocks": clk}


def all_output_error(oracle, np, sets, B, H, L, y=None):
    """rel-L2 of every B*H*L output against the fp64 oracle (src/sffft.cu:394-399): the
    direct convolution up to L = 2048, the fp64 FFT convolution beyond it, cross-checked
    against the direct sum on sequences {0, BH/2, BH-1} (src/sffft.cu:376). The bf16 error
    includes the I/O rounding: its reference is the fp32 input's."""
    s0 = sets[0]
    u_np = s0["u32"].cpu().numpy()
    k_np = s0["k"].cpu().numpy()
    if L <= 2048:
        ref = oracle.direct_conv(u_np, k_np)
        xcheck = None
    else:
        ref = oracle.fft_conv(u_np, k_np)
        seqs = [0, B * H // 2, B * H - 1]
        d = oracle.direct_conv_seqs(u_np, k_np, seqs)
        xcheck = oracle.rel_l2(ref.reshape(B * H, L)[seqs], d)
    return ref, xcheck


def cpu_baseline(oracle, np, u_np, k_np, B, H, L, seconds, cores):
    """The reference's fp64 direct convolution (src/sffft.cu:377 loop order, the oracle's C
    restatement) on `cores` host threads: whole-batch passes repeated for about `seconds`
    when a pass is short, otherwise the first sequences of one pass, scaled to the batch."""
    t1 = time.perf_counter()
    oracle.direct_conv(u_np[:1, :1], k_np[:1], nthreads=1)
    per_seq = max(time.perf_counter() - t1, 1e-6)
    if per_seq * B * H / cores <= seconds:
        reps, done = 0, 0.0
        t1 = time.perf_counter()
        while done < seconds or reps == 0:
            oracle.direct_conv(u_np, k_np, nthreads=cores)
            reps += 1
            done = time.perf_counter() - t1
        value = done * 1e3 / reps
        sample = (f"fp64 direct convolution (src/sffft.cu:377 loop order) of the whole batch "
                  f"({B * H} sequences at L={L}) repeated {reps} times, {done:.1f} s on {cores} thread(s)")
    else:
        nseq = max(cores, int(seconds * cores / per_seq) // cores * cores)
        us = u_np.reshape(B * H, L)[:nseq].reshape(1, nseq, L)
        ks = np.stack([k_np[s_ % H] for s_ in range(nseq)])
        t1 = time.perf_counter()
        oracle.direct_conv(us, ks, nthreads=cores)
        done = time.perf_counter() - t1
        value = done * 1e3 * (B * H) / nseq
        sample = (f"fp64 direct convolution (src/sffft.cu:377 loop order) of the first {nseq} of {B * H} "
                  f"sequences at L={L}, {done:.1f} s on {cores} thread(s), scaled linearly to the batch")
    return {"value": round(value, 3), "unit": "ms per batch", "cores": cores, "kind": "port", "sample": sample}


def sweep(a, sf, torch, np, dev, cover, clocks):
    """Every L of the reference table in fp32 and bf16 I/O (src/sffft.cu:506-513,
    README.md:27-35): graph-timed rotated ms, roofline fraction, all-output rel-L2
    against fp64, and the reference's own warm protocol for the fused launch and the
    rocFFT pipeline (fp32, src/sffft.cu:372-381), whose ratio is the speedup."""
    import oracle

    B, H = a.B, a.H
    rows = []
    for L in SWEEP_LENGTHS:
        ref = xcheck = None
        rocfft_ms = rocfft_core_ms = rocfft_err = None
        for io in ("fp32", "bf16"):
            t0 = time.perf_counter()
            plan = sf.default_plan(L, io, B)
            sets, _, set_bytes = make_workload(sf, torch, dev, B, H, L, io, plan, a.rotate_mb)
            t = time_fused(sf, torch, cover, sets, plan, a.steps, 3, warm=True, gpu_warm_ms=a.gpu_warm_ms,
                           repeats=a.repeats, clocks=clocks)
            ms, ms_warm, exact, step = t["ms"], t["ms_warm"], t["exact"], t["step"]
            ms_ref = reference_protocol_ms(cover, lambda: step(0), L)
            s_io = 4 if io == "fp32" else 2
            algo = B * H * L * 2 * s_io + H * 2 * L * 8
            if ref is None:
                ref, xcheck = all_output_error(oracle, np, sets, B, H, L)
            step(0)
            torch.cuda.synchronize()
            err = oracle.rel_l2(sets[0]["y"].float().cpu().numpy(), ref)
            # the same plan in the fp16-accumulation mode (its packed fp16 products), on the
            # same buffers: the reference's speed-for-precision trade (README.md:112-122)
            plan16 = plan.replace(acc=1)
            t16 = time_fused(sf, torch, cover, sets, plan16, a.steps, 3, warm=False, gpu_warm_ms=a.gpu_warm_ms,
                             repeats=a.repeats)
            t16["step"](0)
            torch.cuda.synchronize()
            err16 = oracle.rel_l2(sets[0]["y"].float().cpu().numpy(), ref)
            if io == "fp32":
                s0 = sets[0]
                rp = sf.RocfftPipeline(B, H, L, s0["k"])
                yr = torch.empty_like(s0["u32"])
                rocfft_ms = reference_protocol_ms(cover, lambda: rp.full(s0["u32"], yr), L)
                rocfft_core_ms = reference_protocol_ms(cover, rp.core, L)
                rp.full(s0["u32"], yr)
                torch.cuda.synchronize()
                rocfft_err = oracle.rel_l2(yr.cpu().numpy(), ref)
                rp.close()
                del yr
            row = {"L": L, "io": io, "plan": plan.name(), "waves": plan.waves, "mode": plan.mode,
                   "channels": plan.channels, "ms": round(ms, 6), "ms_min": round(t["ms_min"], 6),
                   "ms_max": round(t["ms_max"], 6), "ms_warm": round(ms_warm, 6), "clocks": t["clocks"],
                   "roofline_frac": round(algo / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                   "rel_l2_vs_fp64": err, "ms_reference_protocol": round(ms_ref, 6),
                   "rocfft_pipeline_ms": None if rocfft_ms is None else round(rocfft_ms, 6),
                   "rocfft_core_ms": None if rocfft_core_ms is None else round(rocfft_core_ms, 6),
                   "rocfft_rel_l2_vs_fp64": rocfft_err,
                   "speedup_vs_rocfft": None if rocfft_ms is None else round(rocfft_ms / ms_ref, 2),
                   "graph_replay_bitexact": bool(exact), "rotated_sets": len(sets),
                   "fp16acc": {"ms": round(t16["ms"], 6), "ms_min": round(t16["ms_min"], 6),
                               "ms_max": round(t16["ms_max"], 6),
                               "roofline_frac": round(algo / (t16["ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                               "rel_l2_vs_fp64": err16, "graph_replay_bitexact": bool(t16["exact"])}}
            if xcheck is not None:
                row["oracle_fft_vs_direct"] = xcheck
            rows.append(row)
            print(f"# sweep L={L} {io} {plan.name()}: {ms * 1e3:.2f} us (min {t['ms_min'] * 1e3:.2f} max "
                  f"{t['ms_max'] * 1e3:.2f}) frac {row['roofline_frac']} err {err:.3e}; fp16 acc "
                  f"{t16['ms'] * 1e3:.2f} us err {err16:.3e}; rocfft {rocfft_ms} "
                  f"clocks {clock_brief(t['clocks'])} ({time.perf_counter() - t0:.1f} s)", file=sys.stderr,
                  flush=True)
            del sets
            torch.cuda.empty_cache()
    # the fp32 rocFFT pipeline is the comparator of both I/O rows of a length
    by_L = {r["L"]: r for r in rows if r["io"] == "fp32"}
    for r in rows:
        if r["io"] == "bf16":
            f = by_L[r["L"]]
            r["speedup_vs_rocfft"] = round(f["rocfft_pipeline_ms"] / r["ms_reference_protocol"], 2)
    return rows


# The benchmark configurations beside the headline and the sweep: (name, B, H, L, io, plan
# spec, waves, seqs, mode, channels, acc, filters); plan None = the tuned default.
CONFIG_ROWS = (
    ("L=2048 bf16 16x16x16, fp32 accumulation", 8, 768, 2048, "bf16", "16x16x16", 4, 2, 0, 1, 0, "decay"),
    ("L=2048 bf16 16x16x16, fp16 accumulation", 8, 768, 2048, "bf16", "16x16x16", 4, 2, 0, 1, 1, "decay"),
    ("Hyena-style long filter B=4 H=1536 L=16384 bf16", 4, 1536, 16384, "bf16", None, 0, 0, 0, 0, 0, "sines"),
)


def config_rows(a, sf, torch, np, dev, cover, clocks):
    """The other benchmark configurations (CONFIG_ROWS), each timed like the sweep rows
    (median of the graph replays over rotated sets, warm time, the reference protocol)
    with its all-output error against the fp64 oracle."""
    import oracle

    rows = []
    for name, B, H, L, io, spec, waves, seqs, mode, channels, acc, filters in CONFIG_ROWS:
        t0 = time.perf_counter()
        if spec is None:
            plan = sf.default_plan(L, io, B, acc=acc)
        else:
            plan = sf.make_plan(spec, waves, acc=acc, cached=1, seqs=seqs, mode=mode, channels=channels)
        sets, _, set_bytes = make_workload(sf, torch, dev, B, H, L, io, plan, a.rotate_mb, filters=filters)
        t = time_fused(sf, torch, cover, sets, plan, a.steps, 3, warm=True, gpu_warm_ms=a.gpu_warm_ms,
                       repeats=a.repeats, clocks=clocks)
        ms_ref = reference_protocol_ms(cover, lambda: t["step"](0), L)
        ref, xcheck = all_output_error(oracle, np, sets, B, H, L)
        t["step"](0)
        torch.cuda.synchronize()
        err = oracle.rel_l2(sets[0]["y"].float().cpu().numpy(), ref)
        del ref
        s_io = 4 if io == "fp32" else 2
        algo = B * H * L * 2 * s_io + H * 2 * L * 8
        row = {"config": name, "B": B, "H": H, "L": L, "io": io, "plan": plan.name(), "waves": plan.waves,
               "seqs": plan.seqs, "mode": plan.mode, "channels": plan.channels,
               "acc": "fp16" if plan.acc else "fp32", "filters": filters, "ms": round(t["ms"], 6),
               "ms_min": round(t["ms_min"], 6), "ms_max": round(t["ms_max"], 6), "ms_warm": round(t["ms_warm"], 6),
               "ms_reference_protocol": round(ms_ref, 6),
               "roofline_frac": round(algo / (t["ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "rel_l2_vs_fp64": err,
               "oracle_fft_vs_direct": xcheck, "graph_replay_bitexact": bool(t["exact"]),
               "rotated_sets": len(sets), "clocks": t["clocks"]}
        rows.append(row)
        print(f"# config {name} {plan.name()} w{plan.waves}: {t['ms'] * 1e3:.2f} us (min {t['ms_min'] * 1e3:.2f} "
              f"max {t['ms_max'] * 1e3:.2f}) frac {row['roofline_frac']} err {err:.3e} "
              f"clocks {clock_brief(t['clocks'])} ({time.perf_counter() - t0:.1f} s)", file=sys.stderr, flush=True)
        del sets
        torch.cuda.empty_cache()
    return rows


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
    if a.floor_shapes:
        floor_shapes(a)
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

    t_start = time.perf_counter()
    cover = Cover()
    clocks = Clocks()
    # ---- synthetic inputs (the benchmark workload), resident in HBM -------------
    sets, decay, set_bytes = make_workload(sf, torch, dev, B, H, L, io, plan, a.rotate_mb)
    s_io = 4 if io == "fp32" else 2
    # multi-pass plans: one workspace for every step (the steps run in stream order)
    work = None
    if plan.mode == 2:
        wb = int(a.work_mb * 1e6) if a.work_mb > 0 else sf.work_bytes(B, H, L, plan)
        work = torch.empty(wb, dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()

    # ---- timed region ----------------------------------------------------------
    # W eager warmup steps; then the K steps are captured once as a HIP graph and the
    # graph is replayed between two events on the replay stream, behind a spin kernel
    # that covers the host's enqueue time. The same K steps launched eagerly are timed
    # beside it, and the same K steps on one buffer set (warm).
    timed = time_fused(sf, torch, cover, sets, plan, a.steps, a.warmup, work, gpu_warm_ms=a.gpu_warm_ms,
                       repeats=a.repeats, clocks=clocks)
    ms, ms_eager, ms_warm, replay_exact, step = (timed["ms"], timed["ms_eager"], timed["ms_warm"], timed["exact"],
                                                 timed["step"])

    # dispatch floor: a body-less kernel with the same grid, block and LDS size, K
    # launches replayed as a graph like the convolution (first call eager: it sets the
    # kernel's LDS attribute, which is not a stream operation)
    ms_floor = None
    if plan.mode != 2:  # multi-pass steps are three launches of different shapes
        sf.dispatch_floor(B, H, L, plan)
        floor_graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(floor_graph):
            for i in range(a.steps):
                sf.dispatch_floor(B, H, L, plan)
        floor_graph.replay()
        ms_floor = events_ms(cover, floor_graph.replay, a.steps, host_time_ms(floor_graph.replay))

    # ---- correctness of the measured configuration: every output ---------------
    rel_err = xcheck = None
    if a.check:
        import oracle

        if L <= 16384:
            ref, xcheck = all_output_error(oracle, np, sets, B, H, L)
        else:  # multi-pass lengths: the fp64 FFT convolution of 32 sampled sequences
            idx = np.linspace(0, B * H - 1, 32).astype(np.int64)
            u_np = sets[0]["u32"].cpu().numpy().reshape(B * H, L)[idx]
            k_np = sets[0]["k"].cpu().numpy()
            ref = oracle.fft_conv(u_np[None], np.stack([k_np[int(s) % H] for s in idx]))[0]
        step(0)
        torch.cuda.synchronize()
        y = sets[0]["y"].float().cpu().numpy()
        if L > 16384:
            y = y.reshape(B * H, L)[idx]
        rel_err = oracle.rel_l2(y, ref)
        del ref, y

    algo_bytes = B * H * L * 2 * s_io + H * 2 * L * 8
    achieved = algo_bytes / (ms * 1e-3) / 1e9
    u32_np, k_np = sets[0]["u32"].cpu().numpy(), sets[0]["k"].cpu().numpy()
    nsets, work_bytes = len(sets), None if work is None else work.numel()
    del sets, work
    torch.cuda.empty_cache()

    rows = sweep(a, sf, torch, np, dev, cover, clocks) if a.sweep and plan.mode != 2 else None
    cfg_rows = config_rows(a, sf, torch, np, dev, cover, clocks) if a.configs and plan.mode != 2 else None

    # ---- CPU baseline: the reference's fp64 direct convolution (oracle port) ----
    # A bounded sample of the same workload on all host threads, and on one thread.
    cpu = cpu1 = None
    if a.cpu_baseline:
        import oracle

        cpu = cpu_baseline(oracle, np, u32_np, k_np, B, H, L, a.cpu_seconds, oracle.threads())
        cpu1 = cpu_baseline(oracle, np, u32_np, k_np, B, H, L, a.cpu_seconds, 1)

    stamp = sf.kernel_sources_sha(plan.mode)
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
                   "rotated_bytes": nsets * set_bytes,
                   "workspace_bytes": work_bytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic(f"B={B} H={H} L={L} {io}", plan, stamp)},
        "cpu_baseline": cpu,
        "cpu_baseline_1core": cpu1,
        "ms_min": round(timed["ms_min"], 6),
        "ms_max": round(timed["ms_max"], 6),
        "ms_runs": [round(x, 6) for x in timed["ms_runs"]],
        "repeats": a.repeats,
        "clocks": timed["clocks"],
        "ms_warm": round(ms_warm, 6),
        "ms_eager": round(ms_eager, 6),
        "ms_dispatch_floor": None if ms_floor is None else round(ms_floor, 6),
        "io_only_frac": round(B * H * L * 2 * s_io / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "timing": ("HIP graph of the K steps replayed between events behind a spin kernel that covers the "
                   "host enqueue, after W eager warmup steps and untimed replays for gpu_warm_ms; value: the median "
                   "ms per step of `repeats` such replays (ms_min, ms_max, ms_runs); clocks: the GFX clock before each "
                   "timed replay from its spin kernel (shader-clock cycles over event time), and amdsmi readings "
                   "sampled through the replays (a slowly refreshed table); ms_eager: the same steps launched one "
                   "by one"),
        "gpu_warm_ms": a.gpu_warm_ms,
        "graph_replay_bitexact": bool(replay_exact),
        "rel_l2_vs_fp64": rel_err,
        "rel_l2_outputs": "all B*H*L" if L <= 16384 else "32 sampled sequences",
        "oracle_fft_vs_direct": xcheck,
        "algorithmic_bytes": algo_bytes,
        "kernel_sources_sha": stamp,
        "sweep": rows,
        "configs": cfg_rows,
        "wall_s": round(time.perf_counter() - t_start, 1),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
