#!/usr/bin/env python3
"""Benchmark of the quantized-weight matmul hot path on one MI355X.

Headline workload (value): batch-1 Q4_K GEMV, weight 9728 x 2560 in GGUF
144-byte super-blocks, fp32 activation quantized to Q8_K on the device, fp32
output — one step is one qmm_gemm_multi_dispatch call (quantize + GEMV, one
kernel launch). Steps rotate over enough weight replicas (>= 512 MB) that
every step streams its weights from HBM rather than the 256 MB Infinity
Cache. Timing (see timed): HIP graphs timed with HIP events on the
library's stream, each right behind >= 4 ms of untimed GPU work; a step's
time is (T(lead-in + K steps) - T(lead-in)) / K over a short lead-in, so
what a graph launch costs once cancels and the figure does not depend on
--steps; the plain K-step graph time is reported beside it.

Also reported: the 16-B streaming-read floor over the same replicas, the
tree-verify GEMMs (M = 8..64, int8 TOPS), the FFN block, the M = 512
prefill layer, task groups of several types in one launch, the Q6_K LM head
(GEMV, argmax epilogue, chunked scan with early exit), and the reference's
own CPU dot path timed on this host. Roofline objects of the GEMMs carry
rocprofv3 counter figures from the committed summary under profiles/.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1]
Prints one JSON line on stdout; progress goes to stderr.
Counter runs: python bench.py --pmc-run (the GEMM workloads alone, launched
directly, one marker launch between workloads) under rocprofv3 --pmc, then
python bench.py --pmc-summarize DIR... > profiles/qmm_gemm_kernels_pmc.txt.
"""
import argparse
import csv
import glob
import json
import math
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "npu880-mtk-npu-llm-runtime_amd"))

import numpy as np  # noqa: E402

import qmm_hip  # noqa: E402
import synth  # noqa: E402

METRIC = "Q4_K GEMV HBM GB/s (% of peak) at 2560x9728; tree-verify GEMM int8 TOPS"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
DECODE_BYTES_PER_TOKEN = 36 * 72_120_320 + 319_065_600  # 36 layers + Q6_K LM head
ROTATE_BYTES = 512 << 20
DIRECT = False  # --direct: launch steps one by one instead of replaying a HIP graph
PMC_SUMMARY = os.path.join(ROOT, "profiles", "qmm_gemm_kernels_pmc.txt")
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "gemv_q4k_fused_9728x2560_pmc.txt")
CHUNK_THRESH = [19.5, 16.0, 13.5, 11.5, 10.5, 10.0, 10.0, 10.0, 10.0, -1e30]  # chunk_thresh, E:11245
SWEEP_MULTS = (1, 2, 4, 8)  # the size sweep: Q4_K GEMVs of 9728 * m rows x 2560
SWEEP_GRIDS = ((512, 4), (1024, 4), (2048, 4), (512, 8), (1024, 8), (2048, 8))  # stream-read grids tried per size
SWEEP_PROFILE = os.path.join(ROOT, "profiles", "gemv_q4k_size_sweep_kernel_trace.txt")
SWEEP_MARKER_BASE = 3000  # workgroups of the marker launch before sweep section i: 3000 + i


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def under_profiler():
    """True when a ROCm profiler is attached to this process: its tool
    library is mapped (rocprofv3 preloads it) or its environment is set.
    Graph replays crashed the host process under rocprofv3 --kernel-trace
    (a SIGSEGV below hipGraphLaunch), so such runs launch directly."""
    if any(k.startswith(("ROCPROF", "ROCPROFILER")) for k in os.environ):
        return True
    if "rocprof" in os.environ.get("LD_PRELOAD", ""):
        return True
    try:
        with open("/proc/self/maps") as f:
            return any("rocprofiler" in ln or "rocprofv3" in ln or "roctracer" in ln for ln in f)
    except OSError:
        return False


WARM_MS = 4.0  # untimed GPU work right before each timed graph: clocks at their steady state


def timed(ctx, fn, steps, warmup, period=1):
    """(ms per step, ms per step of a plain K-step graph) for `steps` calls.

    fn(i) works on weight replica i mod `period`. After `warmup` untimed
    direct calls (which also give a first per-call estimate), graphs are
    captured over whole rotations of the replicas: W = >= WARM_MS of calls
    (untimed), A = the lead-in fn(0) .. fn(L - 1) (L >= 16 calls), and B =
    the same lead-in followed by the timed calls fn(L) .. fn(L + steps - 1).
    A and B are each launched right behind W and timed with HIP events on
    the library's stream; the per-step figure is (T(B) - T(A)) / steps,
    median of five trials. What a graph launch costs once (the gap before
    its first kernel, the host's submission) is in both and cancels; the
    clocks are at their steady state; every timed call finds its replica
    last touched one full rotation earlier, as in a long run; and A and B
    are short, so their difference keeps its precision — the figure does
    not depend on --steps. The second figure is the plain one: one K-step
    graph between two events right behind W. With --direct the calls are
    launched one by one between host events (for profilers that do not
    follow graphs)."""
    ctx.sync()
    ctx.timer_begin()
    for i in range(max(1, warmup)):
        fn(i)
    est = ctx.timer_end() / max(1, warmup)
    rot = lambda n: period * max(1, math.ceil(n / period))  # noqa: E731
    lead = rot(16)
    nwarm = rot(max(16, WARM_MS / max(est, 1e-4)))
    if DIRECT:
        for i in range(nwarm):
            fn(i)
        ctx.timer_begin()
        for i in range(steps):
            fn(nwarm + i)
        ms = ctx.timer_end()
        return ms / steps, ms / steps

    def capture(lo, hi):
        ctx.graph_begin()
        for i in range(lo, hi):
            fn(i)
        return ctx.graph_end()

    gW = capture(0, nwarm)
    gA = capture(0, lead)
    gB = capture(0, lead + steps)
    gK = capture(lead, lead + steps)
    for g in (gW, gA, gB, gK):
        ctx.graph_launch(g)
    ctx.sync()

    def after_warm(g):
        ctx.graph_launch(gW)
        ctx.timer_begin()
        ctx.graph_launch(g)
        return ctx.timer_end()

    trials = [(after_warm(gB) - after_warm(gA)) / steps for _ in range(5)]
    plain = after_warm(gK) / steps
    for g in (gW, gA, gB, gK):
        ctx.graph_destroy(g)
    return float(np.median(trials)), plain


class Replicated:
    """One tensor replicated R times in one allocation (stride 4 KB-aligned)."""

    def __init__(self, ctx, type_id, N, K, R, seed, host=None):
        self.ctx, self.type, self.N, self.K = ctx, type_id, N, K
        self.rb = synth.row_bytes(type_id, K)
        self.bytes = N * self.rb
        self.stride = (self.bytes + 4095) // 4096 * 4096
        self.R = R if R > 0 else max(1, math.ceil(ROTATE_BYTES / self.bytes))
        if host is None:
            host = synth.float_rows(type_id, N, K, seed) if type_id in (0, 1) else synth.weights(type_id, N, K, seed)
        self.host = host
        self.buf = ctx.malloc(self.R * self.stride)
        ctx.h2d(self.buf, host)
        for r in range(1, self.R):
            ctx.d2d(self.buf.ptr + r * self.stride, self.buf.ptr, self.bytes)

    def ptr(self, i):
        return self.buf.ptr + (i % self.R) * self.stride

    def task(self, i, dst, ldy=None, res=None):
        ldy = ldy or self.N
        return qmm_hip.MatrixTask(self.ptr(i), self.type, self.N, self.K, dst, ldy, residual=res,
                                  res_stride=ldy if res is not None else 0)

    def free(self):
        self.ctx.free(self.buf)


class Acts:
    """fp32 activations [M][K] and their Q8_K / Q8_0 buffers."""

    def __init__(self, ctx, M, K, seed):
        self.ctx, self.M, self.K = ctx, M, K
        self.host = synth.activations(M, K, seed=seed)
        self.x = ctx.upload(self.host)
        self.q8k = ctx.malloc(ctx.lib.qmm_q8k_bytes(M, K))
        ctx.quantize_q8k(self.x, M, K, self.q8k)
        self.q80 = None
        if K % 32 == 0:
            self.q80 = ctx.malloc(ctx.lib.qmm_q8_0_bytes(M, K))
            ctx.quantize_q8_0(self.x, M, K, self.q80)

    def free(self):
        for b in (self.x, self.q8k, self.q80):
            if b is not None:
                self.ctx.free(b)


def gbs(nbytes, ms):
    return nbytes / (ms * 1e-3) / 1e9


# ------------------------------------------------------------------ headline
def bench_headline(ctx, args):
    N, K = synth.GEMV_Q4K["N"], synth.GEMV_Q4K["K"]
    W = Replicated(ctx, synth.TYPE_Q4_K, N, K, args.replicas, seed=0)
    a = Acts(ctx, 1, K, seed=1)
    y = ctx.malloc(N * 4)
    ctx.reserve(1, K)
    parity = check_against_oracle(ctx, W, a, y)
    step_bytes = N * 1440 + K * 4 + N * 4          # weights + fp32 x + fp32 y
    kern_bytes = N * 1440 + (K + 4 * K // 256 + 4 * K // 32) + N * 4  # weights + Q8_K x + y

    def step(i):  # quantize + GEMV: one dispatch, one launch
        ctx.gemm_multi_dispatch(a.x, 1, K, [W.task(i, y)])

    def pre(i):  # on prequantized Q8_K activations
        ctx.gemm_multi_dispatch_prequantized(a.q8k, None, 1, K, [W.task(i, y)])

    ms, wall = timed(ctx, step, args.steps, args.warmup, W.R)
    ms_pre, _ = timed(ctx, pre, args.steps, args.warmup, W.R)
    log(f"step (quantize + GEMV), {W.R} replicas: {ms * 1e3:.3f} us/step "
        f"({wall * 1e3:.3f} us/step in a plain {args.steps}-step graph), {gbs(step_bytes, ms):.1f} GB/s")
    hot = Replicated(ctx, synth.TYPE_Q4_K, N, K, 1, seed=0, host=W.host)

    def hot_step(i):
        ctx.gemm_multi_dispatch(a.x, 1, K, [hot.task(i, y)])

    ms_hot, _ = timed(ctx, hot_step, args.steps, args.warmup, 1)
    hot.free()
    log(f"GEMV on prequantized Q8_K: {ms_pre * 1e3:.3f} us; one replica (cache-resident): {ms_hot * 1e3:.3f} us")
    floor = bench_stream_floor(ctx, W, args)
    out = dict(ms=ms, wall=wall, step_bytes=step_bytes, parity=parity, R=W.R, wbytes=W.bytes,
               gemv_prequantized={"kernel": "gemv_persist_kernel<FmtQ4K4, 4, 3, false, 6, false, false> on Q8_K input",
                                  "us_per_launch": round(ms_pre * 1e3, 3), "algorithmic_bytes": kern_bytes,
                                  "gbs": round(gbs(kern_bytes, ms_pre), 1)},
               cache_resident_us_per_launch=round(ms_hot * 1e3, 3), hbm_read_floor=floor)
    for b in (y,):
        ctx.free(b)
    a.free()
    W.free()
    return out


def bench_stream_floor(ctx, W, args):
    """The same rotated 14 MB replicas read by the plain 16-B streaming-read
    kernel (no compute): the best grid of several, µs per launch, and one
    512 MB read for the sustained rate."""
    sink = ctx.malloc(4 * 4096)
    best = None
    sweep = {}
    for wgs in (256, 512, 1024, 2048):
        for nl in (2, 4, 8):
            ms, _ = timed(ctx, lambda i: ctx.stream_read(W.ptr(i), W.bytes, wgs, nl, sink), args.steps,
                          args.warmup, W.R)
            sweep[f"{wgs}x{nl}"] = round(ms * 1e3, 3)
            if best is None or ms < best[0]:
                best = (ms, wgs, nl)
    big = ctx.malloc(ROTATE_BYTES)
    ms_big, _ = timed(ctx, lambda i: ctx.stream_read(big, ROTATE_BYTES, 4096, 4, sink), 20, 3)
    ctx.free(big)
    ctx.free(sink)
    ms, wgs, nl = best
    log(f"streaming-read floor, {W.bytes} B: {ms * 1e3:.3f} us ({gbs(W.bytes, ms):.1f} GB/s) at {wgs} workgroups x "
        f"{nl} loads; 512 MiB: {gbs(ROTATE_BYTES, ms_big):.1f} GB/s")
    return {"kernel": "stream_read_kernel (16-B non-temporal loads, no compute)", "bytes": W.bytes,
            "us_per_launch": round(ms * 1e3, 3), "gbs": round(gbs(W.bytes, ms), 1),
            "best_grid": f"{wgs} workgroups x {nl} KB in flight per wave", "sweep_us": sweep,
            "gbs_512MiB_one_launch": round(gbs(ROTATE_BYTES, ms_big), 1)}


def check_against_oracle(ctx, W, a, y):
    """The benchmarked path gives the oracle's result (bit-exact) on replica 0."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    ctx.gemm_multi_dispatch(a.x, 1, W.K, [W.task(0, y)])
    ctx.sync()
    got = ctx.d2h(y, np.float32, (1, W.N))
    ref = O.load_oracle().gemm(W.type, W.host, W.N, a.host)
    err = float(np.abs(got - ref).max() / np.abs(ref).max())
    exact = bool(np.array_equal(got.view(np.uint32), ref.view(np.uint32)))
    log(f"parity {qmm_hip.TYPE_NAMES[W.type]} {W.N}x{W.K} M=1: norm err {err:.2e}, bit-exact {exact}")
    return {"norm_err": err, "bit_exact": exact}


# ---------------------------------------------------------------- size sweep
def fit_time(points):
    """Least-squares T = t0 + bytes / BW over (bytes, us) points: the fixed
    per-launch time t0 and the marginal rate BW of the bytes themselves."""
    xs = np.array([p[0] for p in points], np.float64)
    ys = np.array([p[1] for p in points], np.float64)
    A = np.vstack([np.ones_like(xs), xs]).T
    (t0, slope), *_ = np.linalg.lstsq(A, ys, rcond=None)
    bw = 1.0 / (slope * 1e-6) / 1e9 if slope > 0 else float("inf")
    return {"t0_us": round(float(t0), 3), "marginal_gbs": round(float(bw), 1),
            "marginal_frac": round(float(bw / HBM_PEAK_GBS), 4),
            "max_residual_us": round(float(np.abs(ys - (t0 + slope * xs)).max()), 3)}


def sweep_weights(ctx, m, seed=0):
    """The headline tensor's shape at 9728 * m rows (independent rows per
    size), rotated over >= 512 MB of replicas."""
    N, K = 9728 * m, 2560
    return Replicated(ctx, synth.TYPE_Q4_K, N, K, 0, seed=seed + m)


def bench_size_sweep(ctx, args):
    """The fused Q4_K GEMV (the headline step) and the streaming-read floor
    at 9728 x {1, 2, 4, 8} rows (K = 2560, rotated replicas), graph-timed as
    the headline; T = t0 + bytes / BW fitted to each separates the fixed
    per-launch cost t0 from the marginal rate of the bytes."""
    K = 2560
    a = Acts(ctx, 1, K, seed=1)
    sink = ctx.malloc(4 * 8192)
    steps = max(50, args.steps // 4)
    gemv, stream = {}, {}
    for m in SWEEP_MULTS:
        W = sweep_weights(ctx, m)
        N = W.N
        y = ctx.malloc(N * 4)
        ms, _ = timed(ctx, lambda i: ctx.gemm_multi_dispatch(a.x, 1, K, [W.task(i, y)]), steps, 10, W.R)
        alg = N * 1440 + K * 4 + N * 4
        best = None
        for wgs, nl in SWEEP_GRIDS:
            mss, _ = timed(ctx, lambda i: ctx.stream_read(W.ptr(i), W.bytes, wgs, nl, sink), steps, 10, W.R)
            if best is None or mss < best[0]:
                best = (mss, wgs, nl)
        gemv[N] = {"us": round(ms * 1e3, 3), "algorithmic_bytes": alg, "gbs": round(gbs(alg, ms), 1)}
        stream[N] = {"us": round(best[0] * 1e3, 3), "bytes": W.bytes, "gbs": round(gbs(W.bytes, best[0]), 1),
                     "grid": f"{best[1]}x{best[2]}"}
        log(f"size sweep N={N}: fused GEMV {gemv[N]['us']} us ({gemv[N]['gbs']} GB/s); "
            f"stream read {stream[N]['us']} us ({stream[N]['gbs']} GB/s, {stream[N]['grid']})")
        ctx.free(y)
        W.free()
    ctx.free(sink)
    a.free()
    out = {"K": K, "rows": list(gemv), "gemv_fused_q4k": gemv, "stream_read": stream,
           "fit_gemv": fit_time([(v["algorithmic_bytes"], v["us"]) for v in gemv.values()]),
           "fit_stream_read": fit_time([(v["bytes"], v["us"]) for v in stream.values()]),
           "timing": "graph-timed, as the headline"}
    log(f"size sweep fits: GEMV {out['fit_gemv']}, stream read {out['fit_stream_read']}")
    return out


def sweep_run(args):
    """The size sweep launched directly, for rocprofv3 --kernel-trace: per
    size, a marker launch (the streaming-read kernel on 3000 + 2i workgroups)
    then 16 fused GEMVs; a marker (3000 + 2i + 1) then 16 launches of each
    streaming-read grid, all over rotated replicas."""
    ctx = qmm_hip.Context(0)
    K = 2560
    a = Acts(ctx, 1, K, seed=1)
    sink = ctx.malloc(4 * 8192)
    src = ctx.malloc(4096)
    for i, m in enumerate(SWEEP_MULTS):
        W = sweep_weights(ctx, m)
        y = ctx.malloc(W.N * 4)
        for s in range(W.R):  # every replica touched once before the traced launches
            ctx.stream_read(W.ptr(s), W.bytes, 2048, 4, sink)
        ctx.sync()
        ctx.stream_read(src, 4096, SWEEP_MARKER_BASE + 2 * i, 1, sink)
        for s in range(16):
            ctx.gemm_multi_dispatch(a.x, 1, K, [W.task(s, y)])
        ctx.sync()
        ctx.stream_read(src, 4096, SWEEP_MARKER_BASE + 2 * i + 1, 1, sink)
        for wgs, nl in SWEEP_GRIDS:
            for s in range(16):
                ctx.stream_read(W.ptr(s), W.bytes, wgs, nl, sink)
        ctx.sync()
        log(f"sweep run N={W.N} done")
        ctx.free(y)
        W.free()
    ctx.close()


def sweep_summarize(dirs):
    """Per size, from rocprofv3 kernel-trace CSVs: the mean traced duration
    of the fused GEMV and the best grid's mean of the streaming read, then
    the fits."""
    rows = []
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True):
            with open(f) as fh:
                rows += list(csv.DictReader(fh))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    sec = None
    gemv, stream, names = {}, {}, {}
    for r in rows:
        kn = r["Kernel_Name"]
        wg = int(r["Grid_Size_X"]) // max(1, int(r["Workgroup_Size_X"]))
        us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3
        if "stream_read_kernel" in kn and SWEEP_MARKER_BASE <= wg < SWEEP_MARKER_BASE + 2 * len(SWEEP_MULTS):
            sec = wg - SWEEP_MARKER_BASE
            continue
        if sec is None:
            continue
        m = SWEEP_MULTS[sec // 2]
        if sec % 2 == 0 and "gemv_persist_kernel" in kn:
            gemv.setdefault(m, []).append(us)
            names[m] = kn
        elif sec % 2 == 1 and "stream_read_kernel" in kn:
            stream.setdefault(m, {}).setdefault((wg, kn), []).append(us)
    return gemv, stream, names


def sweep_write(dirs):
    gemv, stream, names = sweep_summarize(dirs)
    print("# Size sweep under rocprofv3 --kernel-trace --stats: the fused Q4_K GEMV (the headline")
    print("# step: fp32 x quantized to Q8_K in the launch, then the GEMV) and the 16-B streaming-read")
    print("# floor at 9728 x {1, 2, 4, 8} rows of K = 2560, weights rotated over >= 512 MB of")
    print("# replicas, every dispatch launched directly (16 per size and kernel). Command (run from")
    print("# /tmp with TMPDIR=/tmp; paths relative to the repository root):")
    print("#   rocprofv3 --kernel-trace --stats -d prof/sweep_trace -o run --output-format csv \\")
    print("#     -- python3 bench.py --sweep-run")
    print(f"#   python3 bench.py --sweep-summarize prof/sweep_trace > {os.path.relpath(SWEEP_PROFILE, ROOT)}")
    print("# Each traced dispatch runs alone (its own ramp-up and drain under the profiler's completion")
    print("# signal), so a duration here is the graph-timed step's time plus a fixed per-dispatch cost;")
    print("# the fit T = t0 + bytes / BW puts that cost into t0, and its slope (the marginal rate) is")
    print("# what both regimes share. fit lines: t0_us, marginal GB/s, marginal fraction of 8 TB/s.")
    print("# rows  gemv_us  gemv_alg_bytes  stream_us  stream_bytes  stream_grid")
    gp, sp = [], []
    for m in SWEEP_MULTS:
        if m not in gemv or m not in stream:
            continue
        N = 9728 * m
        alg = N * 1440 + 2560 * 4 + N * 4
        g = float(np.mean(gemv[m]))
        (wg, kn), v = min(stream[m].items(), key=lambda kv: np.mean(kv[1]))
        st = float(np.mean(v))
        nl = kn.split("stream_read_kernel<", 1)[1].split(">", 1)[0] if "stream_read_kernel<" in kn else "?"
        print(f"{N:6d}  {g:7.3f}  {alg:14d}  {st:9.3f}  {N * 1440:12d}  {wg}x{nl}")
        print(f"gemv.N{N}.us: {g:.3f}")
        print(f"stream.N{N}.us: {st:.3f}")
        gp.append((alg, g))
        sp.append((N * 1440, st))
    if gp:
        print(f"gemv.kernel: {names[SWEEP_MULTS[0]]}")
        fg, fs = fit_time(gp), fit_time(sp)
        for k, v in fg.items():
            print(f"fit_gemv.{k}: {v}")
        for k, v in fs.items():
            print(f"fit_stream.{k}: {v}")
        print(f"gemv.N9728.frac_of_peak: {gp[0][0] / (gp[0][1] * 1e-6) / 1e9 / HBM_PEAK_GBS:.4f}")


def sweep_profile():
    """Figures of the committed size-sweep trace summary (or {})."""
    out = {}
    try:
        with open(SWEEP_PROFILE) as f:
            for ln in f:
                if ":" in ln and not ln.startswith("#"):
                    k, v = ln.split(":", 1)
                    out[k.strip()] = v.strip()
    except OSError:
        pass
    return out


# ---------------------------------------------------------------- GEMM lines
PMC = None


def pmc_fields(name):
    """Counter figures of one workload from the committed rocprofv3 summary."""
    global PMC
    if PMC is None:
        PMC = {}
        try:
            with open(PMC_SUMMARY) as f:
                for ln in f:
                    if ":" in ln and not ln.startswith("#"):
                        k, v = ln.split(":", 1)
                        PMC[k.strip()] = v.strip()
        except OSError:
            pass
    out = {}
    for k in ("kernel", "us_under_profiler", "mfma_busy_frac", "valu_insts", "mfma_insts", "valu_per_mfma",
              "int8_ops_executed", "int8_ops_over_algorithmic", "lds_bank_conflict_frac", "hbm_bytes",
              "hbm_bytes_over_algorithmic"):
        v = PMC.get(f"{name}.{k}")
        if v is not None:
            try:
                out[k] = float(v) if k != "kernel" else v
            except ValueError:
                out[k] = v
    return out or None


def gemm_line(name, M, N, K, type_id, ms, extra_bytes=0):
    ops = 2.0 * M * N * K
    byts = N * synth.row_bytes(type_id, K) + M * K * 4 + M * N * 4 + extra_bytes
    tops = ops / (ms * 1e-3) / 1e12
    g = gbs(byts, ms)
    roof = {"bound": "hbm", "achieved": round(g, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(g / HBM_PEAK_GBS, 4), "int8_tops": round(tops, 2),
            "int8_frac": round(tops / INT8_PEAK_TOPS, 4), "algorithmic_bytes": byts, "int8_ops": ops,
            "counters": pmc_fields(name)}
    us_prof = (roof["counters"] or {}).get("us_under_profiler")
    if us_prof:  # the same figures over the kernel's duration under the profiler (direct launches)
        roof["frac_profiled"] = round(byts / (us_prof * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
        roof["int8_frac_profiled"] = round(ops / (us_prof * 1e-6) / 1e12 / INT8_PEAK_TOPS, 4)
    return {"us_gemm_kernel": round(ms * 1e3, 3), "tops": round(tops, 3), "gbs": round(g, 1), "roofline": roof}


def bench_tree(ctx, args):
    steps = max(50, args.steps // 4)
    out = {}
    for label, (t, N, K) in (("q4k_9728x2560", synth.TREE_VERIFY["q4k"]), ("q5k_4096x2560", synth.TREE_VERIFY["q5k"]),
                             ("q6k_2560x9728", synth.TREE_VERIFY["q6k"])):
        W = Replicated(ctx, t, N, K, 0, seed=10 + t)
        lines = {}
        for M in synth.TREE_VERIFY["M"]:
            a = Acts(ctx, M, K, seed=20 + M)
            y = ctx.malloc(M * N * 4)
            ms, _ = timed(ctx, lambda i: ctx.gemm_multi_dispatch_prequantized(a.q8k, None, M, K, [W.task(i, y)]),
                          steps, 10, W.R)
            ms_step, _ = timed(ctx, lambda i: ctx.gemm_multi_dispatch(a.x, M, K, [W.task(i, y)]), steps, 10, W.R)
            ln = gemm_line(f"tree_{label.split('_')[0]}_m{M}", M, N, K, t, ms)
            ln["us_per_step_with_quantize"] = round(ms_step * 1e3, 3)
            lines[f"M{M}"] = ln
            log(f"tree-verify {label} M={M}: {ln['us_gemm_kernel']} us, {ln['tops']} TOPS, {ln['gbs']} GB/s "
                f"(with the quantizer {ln['us_per_step_with_quantize']} us)")
            ctx.free(y)
            a.free()
        out[f"tree_verify_{label}"] = lines
        W.free()
    return out


def bench_prefill(ctx, args):
    """One prefill layer's projections at M = 512 tokens: QKV Q5_K 6144x2560,
    O Q4_K 2560x4096, gate+up Q4_K 9728x2560 (one dispatch), down Q6_K
    2560x9728, Q8_0 2560x2560; each dispatch quantizes its fp32 input."""
    M = synth.PREFILL_LAYER["M"]
    T = synth.PREFILL_LAYER["tensors"]
    layer = sum(N * synth.row_bytes(t, K) for t, N, K in T.values())
    R = max(1, math.ceil(ROTATE_BYTES / layer))
    W = {name: Replicated(ctx, t, N, K, R, 100 + j) for j, (name, (t, N, K)) in enumerate(T.items())}
    acts = {K: Acts(ctx, M, K, seed=200 + K) for K in (2560, 4096, 9728)}
    ys = {name: ctx.malloc(M * N * 4) for name, (t, N, K) in T.items()}
    ctx.reserve(M, 9728)

    def step(i):
        ctx.gemm_multi_dispatch(acts[2560].x, M, 2560, [W["qkv"].task(i, ys["qkv"])])
        ctx.gemm_multi_dispatch(acts[4096].x, M, 4096, [W["o"].task(i, ys["o"])])
        ctx.gemm_multi_dispatch(acts[2560].x, M, 2560, [W["gate"].task(i, ys["gate"]), W["up"].task(i, ys["up"])])
        ctx.gemm_multi_dispatch(acts[9728].x, M, 9728, [W["down"].task(i, ys["down"])])
        ctx.gemm_multi_dispatch(acts[2560].x, M, 2560, [W["q8_0"].task(i, ys["q8_0"])])

    steps = max(5, args.steps // 200)
    ms, _ = timed(ctx, step, steps, 3, R)
    per = {}
    for name, (t, N, K) in T.items():
        if name == "up":
            continue
        tasks = [W[name]] + ([W["up"]] if name == "gate" else [])
        q8 = acts[K].q80 if t == synth.TYPE_Q8_0 else None
        q8k = None if t == synth.TYPE_Q8_0 else acts[K].q8k
        ms_t, _ = timed(ctx, lambda i: ctx.gemm_multi_dispatch_prequantized(
            q8k, q8, M, K, [w.task(i, ys["gate" if w is W["gate"] else ("up" if w is W["up"] else name)])
                            for w in tasks]), max(10, steps), 3, R)
        n_all = N * len(tasks)
        per[name if name != "gate" else "gate_up"] = gemm_line(f"prefill_{name}", M, n_all, K, t, ms_t)
    ops = sum(2.0 * M * N * K for t, N, K in T.values())
    byts = layer + sum(M * K * 4 + M * N * 4 for t, N, K in T.values())
    for w in W.values():
        w.free()
    for a in acts.values():
        a.free()
    for b in ys.values():
        ctx.free(b)
    tops = ops / (ms * 1e-3) / 1e12
    out = {"us_per_layer": round(ms * 1e3, 2), "tops": round(tops, 2), "mfma_frac": round(tops / INT8_PEAK_TOPS, 4),
           "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": INT8_PEAK_TOPS, "unit": "TOP/s (int8)",
                        "frac": round(tops / INT8_PEAK_TOPS, 4), "hbm_gbs": round(gbs(byts, ms), 1),
                        "algorithmic_bytes": byts, "int8_ops": ops},
           "prefill_36_layers_ms": round(36 * ms, 3), "prefill_tokens_per_s": round(M / (36 * ms * 1e-3), 1),
           "replicas": R, "per_dispatch_kernel_only": per}
    log(f"prefill layer M=512: {out['us_per_layer']} us, {out['tops']} TOPS; per dispatch: "
        + ", ".join(f"{k} {v['us_gemm_kernel']} us" for k, v in per.items()))
    return out


def bench_mixed(ctx, args):
    """The engine's {qkv Q5_K 8192, gate Q4_K 4096, alpha F32 32, beta F32 32}
    x 2560 group (E:7954-7959): one dispatch (one launch) against one
    dispatch per type (three launches), at M = 1 (fused quantizer) and M = 8
    (prequantized input)."""
    K = 2560
    specs = [(synth.TYPE_Q5_K, 8192), (synth.TYPE_Q4_K, 4096), (synth.TYPE_F32, 32), (synth.TYPE_F32, 32)]
    group_bytes = sum(n * synth.row_bytes(t, K) for t, n in specs)
    R = max(1, math.ceil(ROTATE_BYTES / group_bytes))
    Ws = [Replicated(ctx, t, n, K, R, 400 + i) for i, (t, n) in enumerate(specs)]
    out = {}
    steps = max(50, args.steps // 4)
    for M in (1, 8):
        a = Acts(ctx, M, K, seed=410 + M)
        ys = [ctx.malloc(M * n * 4) for _, n in specs]

        def one(i):
            tasks = [w.task(i, y) for w, y in zip(Ws, ys)]
            if M == 1:
                ctx.gemm_multi_dispatch(a.x, 1, K, tasks)
            else:
                ctx.gemm_multi_dispatch_prequantized(a.q8k, None, M, K, tasks)

        def per_type(i):
            tasks = [w.task(i, y) for w, y in zip(Ws, ys)]
            for grp in (tasks[0:1], tasks[1:2], tasks[2:4]):
                if M == 1:
                    ctx.gemm_multi_dispatch(a.x, 1, K, grp)
                else:
                    ctx.gemm_multi_dispatch_prequantized(a.q8k, None, M, K, grp)

        ms1, _ = timed(ctx, one, steps, 10, R)
        ms3, _ = timed(ctx, per_type, steps, 10, R)
        byts = group_bytes + M * K * 4 + M * sum(n for _, n in specs) * 4
        out[f"M{M}"] = {"us_one_launch": round(ms1 * 1e3, 3), "us_per_type_launches": round(ms3 * 1e3, 3),
                        "launches": "1 vs 3", "gbs_one_launch": round(gbs(byts, ms1), 1), "algorithmic_bytes": byts}
        log(f"mixed group M={M}: one launch {ms1 * 1e3:.3f} us, per-type launches {ms3 * 1e3:.3f} us")
        for y in ys:
            ctx.free(y)
        a.free()
    for w in Ws:
        w.free()
    out["group"] = "Q5_K 8192 + Q4_K 4096 + F32 32 + F32 32, K 2560"
    return out


def bench_ffn(ctx, args):
    """FFN block at batch 1: gate+up Q4_K 9728x2560 on one input row,
    SiLU(gate)*up -> Q8_K, down Q6_K 2560x9728 with its residual —
    qmm_ffn_block (gate/up with SwiGLU in its epilogue, then the down GEMV
    on h in fp16: two launches), and beside it the three separate calls
    (dispatch, swiglu, prequantized dispatch); then the block behind its
    input RMSNorm: the norm's launch followed by qmm_ffn_block on its Q8_K
    row, against qmm_ffn_block_rmsnorm (the norm in the gate/up launch's
    fill: two launches in all)."""
    H, F = 2560, 9728
    tg, tu, td = synth.FFN["gate"], synth.FFN["up"], synth.FFN["down"]
    block = 2 * F * synth.row_bytes(tg[0], H) + H * synth.row_bytes(td[0], F)
    R = max(1, math.ceil(ROTATE_BYTES / block))
    wg = Replicated(ctx, tg[0], F, H, R, 71)
    wu = Replicated(ctx, tu[0], F, H, R, 72)
    wd = Replicated(ctx, td[0], H, F, R, 73)
    x = ctx.upload(synth.activations(1, H, seed=70))
    res = ctx.upload(synth.activations(1, H, seed=74))
    g, u, h, y = ctx.malloc(F * 4), ctx.malloc(F * 4), ctx.malloc(F * 4), ctx.malloc(H * 4)
    q = ctx.malloc(ctx.lib.qmm_q8k_bytes(1, F))
    ctx.reserve(1, F)

    def block_call(i):
        ctx.ffn_block(x, None, H, wg.task(i, g), wu.task(i, u), wd.task(i, y, res=res), None)

    def three_calls(i):
        ctx.gemm_multi_dispatch(x, 1, H, [wg.task(i, g), wu.task(i, u)])
        ctx.swiglu_q8k(g, u, 1, F, h, q)
        ctx.gemm_multi_dispatch_prequantized(q, None, 1, F, [wd.task(i, y, res=res)])

    gm = ctx.upload(np.random.default_rng(75).uniform(0.5, 1.5, H).astype(np.float32))
    xq = ctx.malloc(ctx.lib.qmm_q8k_bytes(1, H))

    def norm_then_block(i):
        ctx.rmsnorm_q8k(x, gm, 1, H, None, xq)
        ctx.ffn_block(None, xq, H, wg.task(i, g), wu.task(i, u), wd.task(i, y, res=res), None)

    def norm_block(i):
        ctx.ffn_block_rmsnorm(x, gm, H, wg.task(i, g), wu.task(i, u), wd.task(i, y, res=res), None)

    steps = max(50, args.steps // 10)
    ms, _ = timed(ctx, block_call, steps, 10, R)
    ms3, _ = timed(ctx, three_calls, steps, 10, R)
    ms_n2, _ = timed(ctx, norm_then_block, steps, 10, R)
    ms_n1, _ = timed(ctx, norm_block, steps, 10, R)
    alg = block + H * 4 + H * 4 + H * 4  # weights + fp32 x, residual in + fp32 y out (the fused minimum)
    for b in (wg, wu, wd):
        b.free()
    for b in (x, res, g, u, h, y, q, gm, xq):
        ctx.free(b)
    out = {"us_per_block": round(ms * 1e3, 3), "algorithmic_bytes": alg, "gbs": round(gbs(alg, ms), 1),
           "replicas": R, "launches": "qmm_ffn_block: gate+up with SwiGLU (one launch), down GEMV on fp16 h",
           "three_calls_us": round(ms3 * 1e3, 3),
           "with_input_rmsnorm": {"us_norm_then_block": round(ms_n2 * 1e3, 3),
                                  "us_ffn_block_rmsnorm": round(ms_n1 * 1e3, 3)}}
    log(f"FFN block: {out}")
    return out


def bench_rmsnorm_gemv(ctx, args):
    """RMSNorm -> Q8_K (qmm_rmsnorm_q8k) then the Q4_K 9728 x 2560 GEMV on the
    prequantized row, against the RMSNorm alone (M = 1, K = 2560), and the
    same pair as one call (qmm_gemm_multi_dispatch_rmsnorm: the norm inside
    the GEMV's activation fill, one launch)."""
    N, K = synth.GEMV_Q4K["N"], synth.GEMV_Q4K["K"]
    w = Replicated(ctx, synth.TYPE_Q4_K, N, K, 0, 0)
    x = ctx.upload(synth.activations(1, K, seed=1))
    gm = ctx.upload(np.random.default_rng(2).uniform(0.5, 1.5, K).astype(np.float32))
    q = ctx.malloc(ctx.lib.qmm_q8k_bytes(1, K))
    y = ctx.malloc(N * 4)
    steps = max(200, args.steps // 4)
    ms_norm, _ = timed(ctx, lambda i: ctx.rmsnorm_q8k(x, gm, 1, K, None, q), steps, 10)

    def step(i):
        ctx.rmsnorm_q8k(x, gm, 1, K, None, q)
        ctx.gemm_multi_dispatch_prequantized(q, None, 1, K, [w.task(i, y)])

    ms, _ = timed(ctx, step, steps, 10, w.R)
    ms_fused, _ = timed(ctx, lambda i: ctx.gemm_multi_dispatch_rmsnorm(x, gm, 1, K, [w.task(i, y)]), steps, 10, w.R)
    w.free()
    for b in (x, gm, q, y):
        ctx.free(b)
    nbytes = N * 1440 + 2 * K * 4 + N * 4  # weights + fp32 x + gamma + fp32 y
    out = {"us_rmsnorm_q8k": round(ms_norm * 1e3, 3), "us_rmsnorm_then_gemv": round(ms * 1e3, 3),
           "us_rmsnorm_fused_gemv": round(ms_fused * 1e3, 3), "gbs_fused": round(gbs(nbytes, ms_fused), 1)}
    log(f"RMSNorm->Q8_K + GEMV: {out}")
    return out


def bench_lm_head(ctx, args):
    """The Q6_K LM head 151936 x 2560 at M = 1 on a prequantized row: the
    GEMV, the GEMV with its argmax epilogue, and the chunked scan
    (24832-row chunks, chunk_thresh) on a tensor whose chunk 0 holds a row
    at logit 25 (the scan stops after chunk 0) against the same scan
    without thresholds (one launch) and with a threshold at every chunk that
    no chunk meets (chunk 0's launch, then the later chunks in one launch;
    all 7 chunks either way)."""
    N, K = synth.GEMV_Q6K_LMHEAD["N"], synth.GEMV_Q6K_LMHEAD["K"]
    rb = synth.row_bytes(synth.TYPE_Q6_K, K)
    a = Acts(ctx, 1, K, seed=21)
    lm = {}
    # the GEMV and the argmax epilogue over the random tensor (2 replicas: 640 MB)
    W = Replicated(ctx, synth.TYPE_Q6_K, N, K, 2, 20)
    y = ctx.malloc(N * 4)
    steps = max(100, args.steps // 10)
    ms_g, _ = timed(ctx, lambda i: ctx.gemm_multi_dispatch_prequantized(a.q8k, None, 1, K, [W.task(i, y)]), steps, 5,
                    W.R)
    lm_bytes = N * rb + (K + 40 + 320) + N * 4
    lm["gemv"] = {"us_gemv_kernel": round(ms_g * 1e3, 2), "gbs": round(gbs(lm_bytes, ms_g), 1),
                  "roofline_frac": round(gbs(lm_bytes, ms_g) / HBM_PEAK_GBS, 4)}
    bv, bi = ctx.upload(np.full(1, -1e30, np.float32)), ctx.upload(np.zeros(1, np.uint32))

    def one(i):
        ctx.lm_head_argmax(a.q8k, None, 1, K, W.ptr(i), synth.TYPE_Q6_K, N, 0, None, bv, bi)

    def chunked(i):
        for r0 in range(0, N, 24832):
            ctx.lm_head_argmax(a.q8k, None, 1, K, W.ptr(i) + r0 * rb, synth.TYPE_Q6_K, min(24832, N - r0), r0, None,
                               bv, bi)

    ms1, _ = timed(ctx, one, steps, 3, W.R)
    ms7, _ = timed(ctx, chunked, steps, 3, W.R)
    lm["argmax"] = {"us_one_call": round(ms1 * 1e3, 2), "us_7_chunks": round(ms7 * 1e3, 2),
                    "gbs_one_call": round(gbs(N * rb, ms1), 1)}
    W.free()
    ctx.free(y)
    # the scan: small random logits, one planted row at 25 in chunk 0; 7 replicas so the chunk-0 reads
    # (7 x 52 MB) do not fit the Infinity Cache either
    host = synth.lm_head_small_logits(N, K, seed=22)
    host[1234 * rb:1235 * rb] = synth.q6k_row_following(a.host[0], 25.0)
    S = Replicated(ctx, synth.TYPE_Q6_K, N, K, 7, 0, host=host)
    st = ctx.upload(np.zeros(4, np.int32))

    def scan(thr):
        return lambda i: ctx.lm_head_scan(a.q8k, None, 1, K, S.ptr(i), synth.TYPE_Q6_K, N, 24832, thresholds=thr,
                                          best_val=bv, best_id=bi, scan_state=st)

    res = {}
    for label, thr in (("early_exit", CHUNK_THRESH), ("all_chunks", None),
                       ("all_chunks_thresholds_unmet", [1e30] * 7)):
        ms_s, _ = timed(ctx, scan(thr), max(50, args.steps // 20), 3, S.R)
        state = ctx.d2h(st, np.int32, (4,))
        best = int(ctx.d2h(bi, np.uint32, (1,))[0])
        chunks = int(state[0])
        read = sum(min(24832, N - c * 24832) for c in range(chunks)) * rb
        res[label] = {"us": round(ms_s * 1e3, 2), "chunks_read": chunks, "stopped_early": bool(state[2]),
                      "best_row": best, "weight_bytes_read": read, "gbs_effective": round(gbs(read, ms_s), 1)}
        log(f"LM-head scan {label}: {res[label]}")
    # the early-exit scan behind the final RMSNorm: gamma = the row's rms, so the normed row is the row
    # (to fp16 rounding) and the planted row still ends the scan after chunk 0
    xr = a.host[0:1].astype(np.float32)
    xb = ctx.upload(xr)
    gm = ctx.upload(np.full(K, np.sqrt(np.mean(xr.astype(np.float64) ** 2) + 1e-6), np.float32))
    qn = ctx.malloc(ctx.lib.qmm_q8k_bytes(1, K))

    def norm_then_scan(i):
        ctx.rmsnorm_q8k(xb, gm, 1, K, None, qn)
        ctx.lm_head_scan(qn, None, 1, K, S.ptr(i), synth.TYPE_Q6_K, N, 24832, thresholds=CHUNK_THRESH, best_val=bv,
                         best_id=bi, scan_state=st)

    def scan_rmsnorm(i):
        ctx.lm_head_scan_rmsnorm(xb, gm, 1, K, S.ptr(i), synth.TYPE_Q6_K, N, 24832, thresholds=CHUNK_THRESH,
                                 best_val=bv, best_id=bi, scan_state=st)

    nres = {}
    for label, fn in (("us_norm_then_scan", norm_then_scan), ("us_scan_rmsnorm", scan_rmsnorm)):
        ms_s, _ = timed(ctx, fn, max(50, args.steps // 20), 3, S.R)
        nres[label] = round(ms_s * 1e3, 2)
        nres[label.replace("us_", "chunks_read_")] = int(ctx.d2h(st, np.int32, (4,))[0])
    log(f"LM-head scan early_exit behind the final norm: {nres}")
    res["early_exit_behind_final_rmsnorm"] = nres
    lm["scan_151936_chunks_24832"] = res
    S.free()
    for b in (bv, bi, st, xb, gm, qn):
        ctx.free(b)
    a.free()
    return lm


def launch_floor(ctx, args):
    """µs per launch of the smallest kernel the library has (Q8_K quantizer
    of one 256-value block), graph-captured: the per-launch floor."""
    x = ctx.upload(synth.activations(1, 256, seed=5))
    q = ctx.malloc(ctx.lib.qmm_q8k_bytes(1, 256))
    ms, wall = timed(ctx, lambda i: ctx.quantize_q8k(x, 1, 256, q), max(200, args.steps // 4), 10, 1)
    ctx.free(x)
    ctx.free(q)
    return {"us": round(ms * 1e3, 3), "us_plain_graph": round(wall * 1e3, 3)}


def traffic(path):
    """HBM bytes per launch of the headline kernel, from the committed
    rocprofv3 --pmc summary (FETCH_SIZE and WRITE_SIZE per dispatch, each
    scaled by the counter's reading on a copy of known size); None if the
    summary is absent."""
    try:
        vals = {}
        with open(path) as f:
            for ln in f:
                if ":" in ln and not ln.startswith("#"):
                    k, v = ln.split(":", 1)
                    vals[k.strip()] = v.strip()
        return int(float(vals["hbm_bytes_per_launch"]))
    except (OSError, KeyError, ValueError):
        return None


# -------------------------------------------------------------- CPU baseline
def cpu_info():
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    l3 = None
    try:
        ids = set()
        total = 0
        for p in glob.glob("/sys/devices/system/cpu/cpu*/cache/index3"):
            sid = open(os.path.join(p, "shared_cpu_list")).read().strip()
            if sid not in ids:
                ids.add(sid)
                s = open(os.path.join(p, "size")).read().strip()
                total += int(s[:-1]) * (1024 if s.endswith("K") else 1 << 20 if s.endswith("M") else 1)
        l3 = total or None
    except (OSError, ValueError):
        pass
    return {"model": model, "nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)), "l3_bytes": l3}


def cpu_baseline(N, K, seconds):
    """The reference's own portable Q4_K path (quantize_row_fp16_to_q8_k +
    eval_single_lm_row_dot, compiled from its C source into oracle/_ref,
    x86-64-v3) on this host's cores, row-parallel pthreads, weights rotated
    over replicas that exceed the last-level cache; then the C restatement
    compiled here with -O3 -march=native (OpenMP rows)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    info = cpu_info()
    w = synth.weights(synth.TYPE_Q4_K, N, K, seed=0)
    x = synth.activations(1, K, seed=1)
    x16 = x.astype(np.float16).view(np.uint16).reshape(-1)
    share = min(16, info["affinity"])  # this GPU's share of the host's cores
    nbytes = N * 1440 + K * 4 + N * 4
    llc = info["l3_bytes"] or (256 << 20)
    reps = max(2, math.ceil(2 * llc / w.size), math.ceil((256 << 20) / w.size))  # past any host L3
    wr = np.tile(w, reps)
    ref = O.load_reference()
    out = {"cpu": info, "replicas": reps, "replica_bytes": int(w.size)}
    if ref is not None:
        legs = {}
        for T, budget in ((share, seconds), (4, seconds / 2)):
            t1, _ = ref.bench_gemv(synth.TYPE_Q4_K, wr, N, K, x16, T, 2, reps)
            iters = max(3, int(budget / max(t1 / 2, 1e-4)))
            t, _ = ref.bench_gemv(synth.TYPE_Q4_K, wr, N, K, x16, T, iters, reps)
            legs[T] = (nbytes * iters / t / 1e9, iters, t)
            log(f"cpu reference T={T}: {legs[T][0]:.2f} GB/s ({iters} GEMVs in {t:.1f} s, {reps} replicas)")
        g, iters, t = legs[share]
        out.update({"value": round(g, 3), "unit": "GB/s", "cores": share, "kind": "reference",
                    "sample": f"{iters} Q4_K GEMVs 9728x2560 (quantize x + eval_single_lm_row_dot per row) in "
                              f"{t:.1f} s, {share} pthreads, weights rotated over {reps} replicas "
                              f"({reps * w.size >> 20} MiB, past the {llc >> 20} MiB L3), same algorithmic bytes "
                              f"as the GPU line; reference built -O3 -march=x86-64-v3 -ffp-contract=off",
                    "t4_reference_pool": {"value": round(legs[4][0], 3), "cores": 4}})
    # the restatement, built here for this host's own ISA
    so = "/tmp/qmm_oracle_native.so"
    try:
        subprocess.run(["gcc", "-O3", "-march=native", "-std=gnu11", "-fPIC", "-shared", "-ffp-contract=off",
                        "-fopenmp", os.path.join(ROOT, "oracle", "qmm_oracle.c"), "-o", so, "-lm"], check=True,
                       capture_output=True, timeout=120)
        orc = O.Oracle(so)
        env_t = os.environ.get("OMP_NUM_THREADS")
        t0 = time.perf_counter()
        iters = 0
        while time.perf_counter() - t0 < seconds / 2:
            orc.gemm(synth.TYPE_Q4_K, wr[(iters % reps) * w.size:(iters % reps + 1) * w.size], N, x)
            iters += 1
        t = time.perf_counter() - t0
        out["port_native"] = {"value": round(nbytes * iters / t / 1e9, 3), "unit": "GB/s",
                              "cores": int(env_t) if env_t else share, "kind": "port",
                              "sample": f"{iters} GEMVs with the C restatement built -O3 -march=native "
                                        f"-ffp-contract=off, OpenMP rows, {t:.1f} s"}
        log(f"cpu restatement -march=native: {out['port_native']['value']} GB/s")
    except (OSError, subprocess.SubprocessError) as e:
        out["port_native"] = {"error": str(e)[:200]}
    if "value" not in out:  # no compiled reference here: the restatement is the baseline
        pn = out["port_native"]
        out.update({k: pn[k] for k in ("value", "unit", "cores", "kind", "sample") if k in pn})
    return out


# -------------------------------------------------------------- counter runs
PMC_WORKLOADS = [
    # name, type, N, K, M (prequantized input, the GEMM kernel alone)
    ("gemv_q4k_m1", synth.TYPE_Q4_K, 9728, 2560, 1),
    ("tree_q4k_m8", synth.TYPE_Q4_K, 9728, 2560, 8),
    ("tree_q4k_m16", synth.TYPE_Q4_K, 9728, 2560, 16),
    ("tree_q4k_m32", synth.TYPE_Q4_K, 9728, 2560, 32),
    ("tree_q4k_m64", synth.TYPE_Q4_K, 9728, 2560, 64),
    ("tree_q5k_m8", synth.TYPE_Q5_K, 4096, 2560, 8),
    ("tree_q5k_m16", synth.TYPE_Q5_K, 4096, 2560, 16),
    ("tree_q5k_m32", synth.TYPE_Q5_K, 4096, 2560, 32),
    ("tree_q5k_m64", synth.TYPE_Q5_K, 4096, 2560, 64),
    ("tree_q6k_m8", synth.TYPE_Q6_K, 2560, 9728, 8),
    ("tree_q6k_m16", synth.TYPE_Q6_K, 2560, 9728, 16),
    ("tree_q6k_m32", synth.TYPE_Q6_K, 2560, 9728, 32),
    ("tree_q6k_m64", synth.TYPE_Q6_K, 2560, 9728, 64),
    ("prefill_qkv", synth.TYPE_Q5_K, 6144, 2560, 512),
    ("prefill_o", synth.TYPE_Q4_K, 2560, 4096, 512),
    ("prefill_gate", synth.TYPE_Q4_K, 9728, 2560, 512),
    ("prefill_down", synth.TYPE_Q6_K, 2560, 9728, 512),
    ("prefill_q8_0", synth.TYPE_Q8_0, 2560, 2560, 512),
]
PMC_MARKER_BASE = 1000  # workgroups of the marker launch before workload i: 1000 + i


def pmc_run(args):
    """The GEMM workloads one after another, each as 8 directly launched
    dispatches over rotated replicas, with a marker launch (the streaming-read
    kernel on 1000 + i workgroups) before workload i."""
    ctx = qmm_hip.Context(0)
    sink = ctx.malloc(4 * 8192)
    src = ctx.malloc(4096)
    for i, (name, t, N, K, M) in enumerate(PMC_WORKLOADS):
        W = Replicated(ctx, t, N, K, 0, seed=30 + i)
        a = Acts(ctx, M, K, seed=40 + i)
        y = ctx.malloc(M * N * 4)
        ctx.sync()
        ctx.stream_read(src, 4096, PMC_MARKER_BASE + i, 1, sink)
        for s in range(8):
            if t == synth.TYPE_Q8_0:
                ctx.gemm_multi_dispatch_prequantized(None, a.q80, M, K, [W.task(s, y)])
            else:
                ctx.gemm_multi_dispatch_prequantized(a.q8k, None, M, K, [W.task(s, y)])
        ctx.sync()
        log(f"pmc workload {name} done")
        ctx.free(y)
        a.free()
        W.free()
    ctx.close()


def pmc_summarize(dirs):
    """Per workload, from rocprofv3 --pmc CSVs (one directory per pass): the
    mean per dispatch of each counter over the workload's GEMM dispatches,
    and the derived figures."""
    rows = []
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(f) as fh:
                rows += list(csv.DictReader(fh))
    per_pass = {}  # process (one per pass) -> dispatch -> (row, counters)
    for r in rows:
        per_pass.setdefault(r["Process_Id"], {}).setdefault(r["Dispatch_Id"], {"r": r, "c": {}})
        per_pass[r["Process_Id"]][r["Dispatch_Id"]]["c"][r["Counter_Name"]] = float(r["Counter_Value"])
    acc = {}  # workload -> counter -> list
    names = {}
    dur = {}
    for pid, disp in per_pass.items():
        cur = None
        for did in sorted(disp, key=lambda v: int(v)):
            r, c = disp[did]["r"], disp[did]["c"]
            kn = r["Kernel_Name"]
            grid_wg = int(r["Grid_Size"]) // max(1, int(r["Workgroup_Size"]))
            if "stream_read_kernel" in kn and PMC_MARKER_BASE <= grid_wg < PMC_MARKER_BASE + len(PMC_WORKLOADS):
                cur = PMC_WORKLOADS[grid_wg - PMC_MARKER_BASE][0]
                continue
            if cur is None or "quantize" in kn or "copyBuffer" in kn:
                continue
            names.setdefault(cur, kn)
            if kn != names[cur]:
                continue
            for k, v in c.items():
                acc.setdefault(cur, {}).setdefault(k, []).append(v)
            dur.setdefault(cur, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3)
    return acc, names, dur


def pmc_write(dirs):
    acc, names, dur = pmc_summarize(dirs)
    cmd = " ".join(sys.argv)
    print("# rocprofv3 counters of the GEMM workloads (the kernel alone, on prequantized input, weights")
    print("# rotated over >= 512 MB of replicas; 8 dispatches each, launched directly, one at a time under")
    print("# the profiler). Passes (run from /tmp with TMPDIR=/tmp; paths relative to the repository root):")
    print("#   rocprofv3 --pmc SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_VALU_MFMA_MOPS_I8 SQ_VALU_MFMA_BUSY_CYCLES \\")
    print("#     SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_WAVES GRBM_GUI_ACTIVE -d prof/gpmc1 -o run \\")
    print("#     --output-format csv -- python3 bench.py --pmc-run")
    print("#   rocprofv3 --pmc FETCH_SIZE -d prof/gpmc2 ... ; rocprofv3 --pmc WRITE_SIZE -d prof/gpmc3 ...")
    print("#   rocprofv3 --pmc SQ_WAVE_CYCLES SQ_WAIT_ANY SQ_WAIT_INST_ANY SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_LDS \\")
    print("#     SQ_VALU_MFMA_COEXEC_CYCLES SQ_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_F16 -d prof/gpmc4 ...")
    print(f"# summary: {cmd}")
    print("# derived: mfma_busy_frac = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 XCDs * 1024 SIMDs)")
    print("#   (rocprof's MfmaUtil); valu_per_mfma = SQ_INSTS_VALU / SQ_INSTS_MFMA; int8_ops_executed =")
    print("#   SQ_INSTS_VALU_MFMA_MOPS_I8 * 512; lds_bank_conflict_frac = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE;")
    print("#   hbm_bytes = FETCH_SIZE * 1.9966 + WRITE_SIZE * 1.0 KiB (the factors the same counters read on a")
    print("#   device copy of known size, profiles/gemv_q4k_fused_9728x2560_pmc.txt); wave time (SQ_WAVE_CYCLES,")
    print("#   quad-cycles summed over waves): valu_active_frac = SQ_ACTIVE_INST_VALU / SQ_WAVE_CYCLES,")
    print("#   wait_any_frac = SQ_WAIT_ANY / SQ_WAVE_CYCLES (waitcnt / barrier), wait_issue_frac =")
    print("#   SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES (ready instruction not issued); mfma_coexec_frac =")
    print("#   SQ_VALU_MFMA_COEXEC_CYCLES / SQ_VALU_MFMA_BUSY_CYCLES (MFMA-busy cycles in which a VALU issued)")
    for name, t, N, K, M in PMC_WORKLOADS:
        if name not in acc:
            continue
        c = {k: float(np.mean(v)) for k, v in acc[name].items()}
        ops = 2.0 * M * N * K
        byts = N * synth.row_bytes(t, K) + M * K * 4 + M * N * 4
        print(f"{name}.kernel: {names[name]}")
        print(f"{name}.shape: {qmm_hip.TYPE_NAMES[t]} {N}x{K} M={M}")
        print(f"{name}.us_under_profiler: {np.mean(dur[name]):.3f}")
        for k in ("SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_VALU_MFMA_MOPS_I8", "SQ_INSTS_VALU_MFMA_MOPS_F16",
                  "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_VALU_MFMA_COEXEC_CYCLES", "SQ_LDS_BANK_CONFLICT",
                  "SQ_LDS_IDX_ACTIVE", "SQ_WAVES", "SQ_WAVE_CYCLES", "SQ_WAIT_ANY", "SQ_WAIT_INST_ANY",
                  "SQ_ACTIVE_INST_VALU", "SQ_ACTIVE_INST_LDS", "SQ_BUSY_CYCLES", "GRBM_GUI_ACTIVE", "FETCH_SIZE",
                  "WRITE_SIZE"):
            if k in c:
                print(f"{name}.{k}: {c[k]:.6g}")
        if "SQ_INSTS_VALU" in c:
            print(f"{name}.valu_insts: {c['SQ_INSTS_VALU']:.6g}")
            print(f"{name}.mfma_insts: {c['SQ_INSTS_MFMA']:.6g}")
            if c["SQ_INSTS_MFMA"] > 0:
                print(f"{name}.valu_per_mfma: {c['SQ_INSTS_VALU'] / c['SQ_INSTS_MFMA']:.3f}")
        if "SQ_VALU_MFMA_BUSY_CYCLES" in c and c.get("GRBM_GUI_ACTIVE"):
            print(f"{name}.mfma_busy_frac: {c['SQ_VALU_MFMA_BUSY_CYCLES'] / (c['GRBM_GUI_ACTIVE'] / 8 * 1024):.4f}")
        if c.get("SQ_WAVE_CYCLES"):
            wc = c["SQ_WAVE_CYCLES"]
            for k, lab in (("SQ_ACTIVE_INST_VALU", "valu_active_frac"), ("SQ_WAIT_ANY", "wait_any_frac"),
                           ("SQ_WAIT_INST_ANY", "wait_issue_frac")):
                if k in c:
                    print(f"{name}.{lab}: {c[k] / wc:.3f}")
        if c.get("SQ_VALU_MFMA_BUSY_CYCLES") and "SQ_VALU_MFMA_COEXEC_CYCLES" in c:
            print(f"{name}.mfma_coexec_frac: {c['SQ_VALU_MFMA_COEXEC_CYCLES'] / c['SQ_VALU_MFMA_BUSY_CYCLES']:.3f}")
        if "SQ_INSTS_VALU_MFMA_MOPS_I8" in c:
            ex = c["SQ_INSTS_VALU_MFMA_MOPS_I8"] * 512
            print(f"{name}.int8_ops_executed: {ex:.6g}")
            print(f"{name}.int8_ops_over_algorithmic: {ex / ops:.3f}")
        if c.get("SQ_LDS_IDX_ACTIVE"):
            print(f"{name}.lds_bank_conflict_frac: {c['SQ_LDS_BANK_CONFLICT'] / c['SQ_LDS_IDX_ACTIVE']:.4f}")
        if "FETCH_SIZE" in c and "WRITE_SIZE" in c:
            hb = (c["FETCH_SIZE"] * 1.9966 + c["WRITE_SIZE"]) * 1024
            print(f"{name}.hbm_bytes: {hb:.0f}")
            print(f"{name}.hbm_bytes_over_algorithmic: {hb / byts:.3f}")


# ------------------------------------------------------------------------ main
def main():
    global DIRECT
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--replicas", type=int, default=0, help="0 = enough for >= 512 MB")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--only", default="",
                    help="comma list of extra sections: tree,prefill,mixed,ffn,rms,lm,sweep,floor")
    ap.add_argument("--direct", action="store_true",
                    help="launch steps directly, not from a HIP graph (for rocprofv3 runs)")
    ap.add_argument("--pmc-run", action="store_true", help="the GEMM workloads alone, for rocprofv3 --pmc")
    ap.add_argument("--pmc-summarize", nargs="+", metavar="DIR", help="print the counter summary of rocprofv3 CSVs")
    ap.add_argument("--sweep-run", action="store_true", help="the size sweep launched directly, for rocprofv3")
    ap.add_argument("--sweep-summarize", nargs="+", metavar="DIR", help="print the size sweep's trace summary")
    args = ap.parse_args()
    if args.pmc_summarize:
        pmc_write(args.pmc_summarize)
        return
    if args.sweep_summarize:
        sweep_write(args.sweep_summarize)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py runs on one GPU only: this build measures the single-GPU hot path "
              "(row-sharding across GPUs is a design note, not built)", file=sys.stderr)
        sys.exit(2)
    if args.pmc_run:
        pmc_run(args)
        return
    if args.sweep_run:
        sweep_run(args)
        return
    DIRECT = args.direct
    if not DIRECT and under_profiler():
        log("a profiler is attached: steps are launched directly (graph replays are not run under a profiler)")
        DIRECT = True

    ctx = qmm_hip.Context(0)
    info = ctx.device_info()
    log(f"device {info}")
    N, K = synth.GEMV_Q4K["N"], synth.GEMV_Q4K["K"]
    head = bench_headline(ctx, args)
    ms = head["ms"]
    value = gbs(head["step_bytes"], ms)

    extra = {}
    only = set(filter(None, args.only.split(",")))
    want = (lambda s: not only or s in only)
    if not args.no_extra:
        if want("sweep"):  # right after the headline, in the same conditions
            extra["size_sweep_q4k_gemv"] = bench_size_sweep(ctx, args)
        if want("tree"):
            extra.update(bench_tree(ctx, args))
        if want("mixed"):
            extra["task_group_one_launch"] = bench_mixed(ctx, args)
        if want("ffn"):
            extra["ffn_block_q4k_q6k"] = bench_ffn(ctx, args)
        if want("prefill"):
            extra["prefill_layer_m512"] = bench_prefill(ctx, args)
        if want("rms"):
            extra["rmsnorm_q8k_then_gemv_q4k_9728x2560"] = bench_rmsnorm_gemv(ctx, args)
        if want("lm"):
            extra["lm_head_q6k_151936x2560"] = bench_lm_head(ctx, args)
        extra["launch_floor_us"] = launch_floor(ctx, args)
        log(f"launch floor: {extra['launch_floor_us']}")
    ctx.close()

    cpu = None if args.no_cpu else cpu_baseline(N, K, args.cpu_seconds)
    floor = head["hbm_read_floor"]
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "Q4_K GEMV batch 1 (fp32 x -> Q8_K on device, then GEMV), "
                               "weight 9728 x 2560 GGUF super-blocks, fp32 out",
                   "N": N, "K": K, "M": 1, "replicas": head["R"], "replica_bytes": head["wbytes"],
                   "timing": ("direct launches, HIP events" if DIRECT else
                              "HIP graphs each behind >= 4 ms of untimed GPU work, HIP events on the library's "
                              "stream; per step = (T(lead-in + K steps) - T(lead-in)) / K, median of 5, the "
                              "lead-in >= 16 steps of whole rotations of the replicas")},
        "plain_graph_ms_per_step": round(head["wall"], 6),
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "tokens_per_s_equiv": round(value * 1e9 / DECODE_BYTES_PER_TOKEN, 1),
        "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4), "traffic": traffic(TRAFFIC_PROFILE),
                     "kernel": "gemv_persist_kernel<FmtQ4K4, 4, 3, true, 6, false, false> (fused Q8_K quantizer)",
                     "us_per_launch": round(ms * 1e3, 3), "algorithmic_bytes": head["step_bytes"],
                     "floor_us_per_launch": floor["us_per_launch"],
                     "frac_of_measured_floor": round(floor["us_per_launch"] / (ms * 1e3), 4)},
        "hbm_read_floor": floor,
        "roofline_regimes": ("roofline.frac: algorithmic bytes / the graph-timed step (HIP events on the library's "
                             "stream around graph replays); roofline.frac_profiled: the same over the kernel's mean "
                             "duration under rocprofv3 --kernel-trace, launched directly "
                             f"({os.path.relpath(SWEEP_PROFILE, ROOT)}); fit_graph / fit_profiled: T = t0 + bytes / "
                             "BW over 9728 x {1, 2, 4, 8} rows in each regime, t0 the fixed per-launch time, "
                             "marginal_frac = BW / 8 TB/s"),
        "gemv_prequantized": head["gemv_prequantized"],
        "cache_resident_us_per_launch": head["cache_resident_us_per_launch"],
        "parity": head["parity"],
        "cpu_baseline": cpu,
        "device": info,
    }
    prof = sweep_profile()
    roof = line["roofline"]
    if "gemv.N9728.frac_of_peak" in prof:
        roof["frac_profiled"] = float(prof["gemv.N9728.frac_of_peak"])
        roof["us_per_launch_profiled"] = float(prof["gemv.N9728.us"])
        roof["fit_profiled"] = {k.split(".", 1)[1]: float(v) for k, v in prof.items() if k.startswith("fit_gemv.")}
        roof["fit_profiled_stream_read"] = {k.split(".", 1)[1]: float(v) for k, v in prof.items()
                                            if k.startswith("fit_stream.")}
    if "size_sweep_q4k_gemv" in extra:
        roof["fit_graph"] = extra["size_sweep_q4k_gemv"]["fit_gemv"]
        roof["fit_graph_stream_read"] = extra["size_sweep_q4k_gemv"]["fit_stream_read"]
    line.update(extra)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
