#!/usr/bin/env python3
"""Benchmark of the quantized-weight matmul hot path on one MI355X.

Headline workload (value): batch-1 Q4_K GEMV, weight 9728 x 2560 in GGUF
144-byte super-blocks, fp32 activation quantized to Q8_K on the device, fp32
output — one step is one qmm_gemm_multi_dispatch call (quantize + GEMV).
Steps rotate over enough weight replicas (>= 512 MB) that every step streams
its weights from HBM rather than the 256 MB Infinity Cache. Steps are
captured in a HIP graph and timed with HIP events on the library's stream.

Also reported: the GEMV kernel alone (roofline), the same with one replica
(cache-resident), the tree-verify GEMM (M = 8..64, int8 TOPS), the Q6_K
LM-head GEMV, and the reference's own CPU dot path timed on this host.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1]
Prints one JSON line on stdout; progress goes to stderr.
"""
import argparse
import json
import math
import os
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


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Workload:
    """N x K weights of one type, replicated R times in one HBM allocation."""

    def __init__(self, ctx, type_id, N, K, M, replicas, seed):
        self.ctx, self.type, self.N, self.K, self.M = ctx, type_id, N, K, M
        self.rb = synth.row_bytes(type_id, K)
        self.wbytes = N * self.rb
        self.stride = (self.wbytes + 4095) // 4096 * 4096
        self.R = replicas if replicas > 0 else max(1, math.ceil(ROTATE_BYTES / self.wbytes))
        self.w_host = synth.weights(type_id, N, K, seed=seed)
        self.w = ctx.malloc(self.R * self.stride)
        ctx.h2d(self.w, self.w_host)
        for r in range(1, self.R):
            ctx.d2d(self.w.ptr + r * self.stride, self.w.ptr, self.wbytes)
        self.x_host = synth.activations(M, K, seed=seed + 1)
        self.x = ctx.upload(self.x_host)
        self.y = ctx.malloc(M * N * 4)
        self.q = ctx.malloc(ctx.lib.qmm_q8k_bytes(M, K))
        ctx.quantize_q8k(self.x, M, K, self.q)
        ctx.reserve(M, K)
        ctx.sync()

    def task(self, i):
        return qmm_hip.MatrixTask(self.w.ptr + (i % self.R) * self.stride, self.type, self.N,
                                  self.K, self.y, self.N)

    def step(self, i):  # quantize + matmul (the dispatcher)
        self.ctx.gemm_multi_dispatch(self.x, self.M, self.K, [self.task(i)])

    def kernel_only(self, i):  # matmul on prequantized activations
        self.ctx.gemm_multi_dispatch_prequantized(self.q, None, self.M, self.K, [self.task(i)])

    def time(self, fn, steps, warmup):
        """ms per step over exactly `steps` graph-captured calls of fn (or, with
        DIRECT set, `steps` direct calls: for profilers that do not follow
        graph launches; per-kernel durations are the same, the gaps between
        kernels are host launch time)."""
        ctx = self.ctx
        for i in range(warmup):
            fn(i)
        ctx.sync()
        if DIRECT:
            ctx.timer_begin()
            for i in range(steps):
                fn(i)
            return ctx.timer_end() / steps
        ctx.graph_begin()
        for i in range(steps):
            fn(i)
        g = ctx.graph_end()
        ctx.graph_launch(g)  # untimed replay: instantiation and first-touch costs
        ctx.sync()
        ctx.timer_begin()
        ctx.graph_launch(g)
        ms = ctx.timer_end()
        ctx.graph_destroy(g)
        return ms / steps

    def free(self):
        for b in (self.w, self.x, self.y, self.q):
            self.ctx.free(b)


class Replicated:
    """One tensor replicated R times in one allocation (rotation defeats the
    256 MB Infinity Cache for multi-tensor steps)."""

    def __init__(self, ctx, type_id, N, K, R, seed):
        self.type, self.N, self.K = type_id, N, K
        self.bytes = N * synth.row_bytes(type_id, K)
        self.stride = (self.bytes + 4095) // 4096 * 4096
        self.R = R
        self.buf = ctx.malloc(R * self.stride)
        ctx.h2d(self.buf, synth.weights(type_id, N, K, seed=seed))
        for r in range(1, R):
            ctx.d2d(self.buf.ptr + r * self.stride, self.buf.ptr, self.bytes)

    def task(self, i, dst, ldy, res=None):
        return qmm_hip.MatrixTask(self.buf.ptr + (i % self.R) * self.stride, self.type, self.N,
                                  self.K, dst, ldy, residual=res, res_stride=ldy if res is not None else 0)


def timed(ctx, fn, steps, warmup):
    """ms per call of fn(i) over exactly `steps` calls, graph-captured (or direct)."""
    for i in range(warmup):
        fn(i)
    ctx.sync()
    if DIRECT:
        ctx.timer_begin()
        for i in range(steps):
            fn(i)
        return ctx.timer_end() / steps
    ctx.graph_begin()
    for i in range(steps):
        fn(i)
    g = ctx.graph_end()
    ctx.graph_launch(g)
    ctx.sync()
    ctx.timer_begin()
    ctx.graph_launch(g)
    ms = ctx.timer_end()
    ctx.graph_destroy(g)
    return ms / steps


def bench_ffn(ctx, steps):
    """FFN block at batch 1: gate+up Q4_K 9728x2560 on one shared Q8_K input
    (one dispatch), SiLU(gate)*up -> Q8_K, down Q6_K 2560x9728 (prequantized)."""
    H, F = 2560, 9728
    tg, tu, td = synth.FFN["gate"], synth.FFN["up"], synth.FFN["down"]
    block = 2 * F * synth.row_bytes(tg[0], H) + H * synth.row_bytes(td[0], F)
    R = max(1, math.ceil(ROTATE_BYTES / block))
    wg = Replicated(ctx, tg[0], F, H, R, 71)
    wu = Replicated(ctx, tu[0], F, H, R, 72)
    wd = Replicated(ctx, td[0], H, F, R, 73)
    x = ctx.upload(synth.activations(1, H, seed=70))
    g, u, h, y = ctx.malloc(F * 4), ctx.malloc(F * 4), ctx.malloc(F * 4), ctx.malloc(H * 4)
    q = ctx.malloc(ctx.lib.qmm_q8k_bytes(1, F))
    ctx.reserve(1, F)

    def step(i):
        ctx.gemm_multi_dispatch(x, 1, H, [wg.task(i, g, F), wu.task(i, u, F)])
        ctx.swiglu_q8k(g, u, 1, F, h, q)
        ctx.gemm_multi_dispatch_prequantized(q, None, 1, F, [wd.task(i, y, H)])

    ms = timed(ctx, step, steps, 10)
    alg = block + H * 4 + H * 4  # weights + fp32 x in + fp32 y out (the fused minimum)
    for b in (wg.buf, wu.buf, wd.buf, x, g, u, h, y, q):
        ctx.free(b)
    return {"us_per_block": round(ms * 1e3, 3), "algorithmic_bytes": alg,
            "gbs": round(alg / (ms * 1e-3) / 1e9, 1), "replicas": R,
            "launches": "gemv(gate+up, one launch), swiglu+Q8_K, gemv(down)"}


def bench_prefill(ctx, steps):
    """One prefill layer's projections at M = 512 tokens: QKV Q5_K 6144x2560,
    O Q4_K 2560x4096, gate+up Q4_K 9728x2560 (one dispatch), down Q6_K
    2560x9728, Q8_0 2560x2560; each dispatch quantizes its fp32 input."""
    M = synth.PREFILL_LAYER["M"]
    T = synth.PREFILL_LAYER["tensors"]
    layer = sum(N * synth.row_bytes(t, K) for t, N, K in T.values())
    R = max(1, math.ceil(ROTATE_BYTES / layer))
    W = {name: Replicated(ctx, t, N, K, R, 100 + j) for j, (name, (t, N, K)) in enumerate(T.items())}
    xs = {K: ctx.upload(synth.activations(M, K, seed=200 + K)) for K in (2560, 4096, 9728)}
    ys = {name: ctx.malloc(M * N * 4) for name, (t, N, K) in T.items()}
    ctx.reserve(M, 9728)

    def step(i):
        ctx.gemm_multi_dispatch(xs[2560], M, 2560, [W["qkv"].task(i, ys["qkv"], 6144)])
        ctx.gemm_multi_dispatch(xs[4096], M, 4096, [W["o"].task(i, ys["o"], 2560)])
        ctx.gemm_multi_dispatch(xs[2560], M, 2560, [W["gate"].task(i, ys["gate"], 9728),
                                                     W["up"].task(i, ys["up"], 9728)])
        ctx.gemm_multi_dispatch(xs[9728], M, 9728, [W["down"].task(i, ys["down"], 2560)])
        ctx.gemm_multi_dispatch(xs[2560], M, 2560, [W["q8_0"].task(i, ys["q8_0"], 2560)])

    ms = timed(ctx, step, steps, 3)
    ops = sum(2.0 * M * N * K for t, N, K in T.values())
    for w in W.values():
        ctx.free(w.buf)
    for b in list(xs.values()) + list(ys.values()):
        ctx.free(b)
    per_layer = ms * 1e-3
    return {"us_per_layer": round(ms * 1e3, 2), "tops": round(ops / per_layer / 1e12, 2),
            "mfma_frac": round(ops / per_layer / 1e12 / INT8_PEAK_TOPS, 4),
            "prefill_36_layers_ms": round(36 * ms, 3),
            "prefill_tokens_per_s": round(M / (36 * per_layer), 1), "replicas": R}


def bench_rmsnorm_gemv(ctx, steps):
    """The decode projection with its producer fused: RMSNorm -> Q8_K
    (qmm_rmsnorm_q8k) then the Q4_K 9728 x 2560 GEMV on the prequantized
    row, against the RMSNorm alone (M = 1, K = 2560)."""
    N, K = synth.GEMV_Q4K["N"], synth.GEMV_Q4K["K"]
    w = Replicated(ctx, synth.TYPE_Q4_K, N, K, max(1, math.ceil(ROTATE_BYTES / (N * 1440))), 0)
    x = ctx.upload(synth.activations(1, K, seed=1))
    gm = ctx.upload(np.random.default_rng(2).uniform(0.5, 1.5, K).astype(np.float32))
    q = ctx.malloc(ctx.lib.qmm_q8k_bytes(1, K))
    y = ctx.malloc(N * 4)
    ms_norm = timed(ctx, lambda i: ctx.rmsnorm_q8k(x, gm, 1, K, None, q), steps, 10)

    def step(i):
        ctx.rmsnorm_q8k(x, gm, 1, K, None, q)
        ctx.gemm_multi_dispatch_prequantized(q, None, 1, K, [w.task(i, y, N)])

    ms = timed(ctx, step, steps, 10)
    for b in (w.buf, x, gm, q, y):
        ctx.free(b)
    return {"us_rmsnorm_q8k": round(ms_norm * 1e3, 3), "us_rmsnorm_then_gemv": round(ms * 1e3, 3)}


def bench_lm_head_argmax(ctx, steps):
    """The LM head with its argmax epilogue (Q6_K 151936 x 2560, M = 1,
    prequantized row): one call over all rows, and the reference's chunking
    (24832-row chunks chained through the running best)."""
    N, K = synth.GEMV_Q6K_LMHEAD["N"], synth.GEMV_Q6K_LMHEAD["K"]
    w = Replicated(ctx, synth.TYPE_Q6_K, N, K, 2, 20)
    rb = synth.row_bytes(synth.TYPE_Q6_K, K)
    q = ctx.malloc(ctx.lib.qmm_q8k_bytes(1, K))
    ctx.quantize_q8k(ctx.upload(synth.activations(1, K, seed=21)), 1, K, q)
    bv, bi = ctx.upload(np.full(1, -1e30, np.float32)), ctx.upload(np.zeros(1, np.uint32))

    def one(i):
        base = w.buf.ptr + (i % w.R) * w.stride
        ctx.lm_head_argmax(q, None, 1, K, base, synth.TYPE_Q6_K, N, 0, None, bv, bi)

    def chunked(i):
        base = w.buf.ptr + (i % w.R) * w.stride
        for r0 in range(0, N, 24832):
            rows = min(24832, N - r0)
            ctx.lm_head_argmax(q, None, 1, K, base + r0 * rb, synth.TYPE_Q6_K, rows, r0, None, bv, bi)

    one(0)
    chunked(0)
    ctx.sync()
    ms1 = timed(ctx, one, steps, 3)
    ms7 = timed(ctx, chunked, steps, 3)
    for b in (w.buf, q, bv, bi):
        ctx.free(b)
    byts = N * rb
    return {"us_one_call": round(ms1 * 1e3, 2), "us_7_chunks": round(ms7 * 1e3, 2),
            "gbs_one_call": round(byts / (ms1 * 1e-3) / 1e9, 1)}


def launch_floor(ctx, steps):
    """µs per launch of the smallest kernel the library has (Q8_K quantizer
    of one 256-value block), graph-captured: the per-launch floor."""
    x = ctx.upload(synth.activations(1, 256, seed=5))
    q = ctx.malloc(ctx.lib.qmm_q8k_bytes(1, 256))
    ms = timed(ctx, lambda i: ctx.quantize_q8k(x, 1, 256, q), steps, 10)
    ctx.free(x)
    ctx.free(q)
    return round(ms * 1e3, 3)


def check_against_oracle(wl):
    """The benchmarked path gives the oracle's result (bit-exact) on replica 0."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    wl.step(0)
    wl.ctx.sync()
    y = wl.ctx.d2h(wl.y, np.float32, (wl.M, wl.N))
    ref = O.load_oracle().gemm(wl.type, wl.w_host, wl.N, wl.x_host)
    err = float(np.abs(y - ref).max() / np.abs(ref).max())
    exact = bool(np.array_equal(y.view(np.uint32), ref.view(np.uint32)))
    log(f"parity {qmm_hip.TYPE_NAMES[wl.type]} {wl.N}x{wl.K} M={wl.M}: norm err {err:.2e}, bit-exact {exact}")
    return {"norm_err": err, "bit_exact": exact}


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "gemv_q4k_fused_9728x2560_pmc.txt")


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


def cpu_baseline(N, K, seconds):
    """The reference's own portable Q4_K path (quantize_row_fp16_to_q8_k +
    eval_single_lm_row_dot, compiled from its C source into oracle/_ref) on
    this host's cores, row-parallel pthreads; falls back to the restatement."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    w = synth.weights(synth.TYPE_Q4_K, N, K, seed=0)
    x = synth.activations(1, K, seed=1)
    x16 = x.astype(np.float16).view(np.uint16).reshape(-1)
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    nbytes = N * 1440 + K * 4 + N * 4
    ref = O.load_reference()
    out = {}
    if ref is not None:
        for T, budget in ((threads, seconds), (4, seconds / 2)):
            t1, _ = ref.bench_gemv(synth.TYPE_Q4_K, w, N, K, x16, T, 1)
            iters = max(3, int(budget / max(t1, 1e-4)))
            t, _ = ref.bench_gemv(synth.TYPE_Q4_K, w, N, K, x16, T, iters)
            out[T] = (nbytes * iters / t / 1e9, iters, t)
            log(f"cpu reference T={T}: {out[T][0]:.2f} GB/s ({iters} GEMVs in {t:.1f} s)")
        gbs, iters, t = out[threads]
        return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "reference",
                "sample": f"{iters} Q4_K GEMVs 9728x2560 (quantize x + eval_single_lm_row_dot per row) "
                          f"in {t:.1f} s, {threads} pthreads, same algorithmic bytes as the GPU line",
                "t4_reference_pool": {"value": round(out[4][0], 3), "cores": 4}}
    orc = O.load_oracle()
    t0 = time.perf_counter()
    iters = 0
    while time.perf_counter() - t0 < seconds:
        orc.gemm(synth.TYPE_Q4_K, w, N, x)
        iters += 1
    t = time.perf_counter() - t0
    return {"value": round(nbytes * iters / t / 1e9, 3), "unit": "GB/s",
            "cores": int(os.environ.get("OMP_NUM_THREADS", threads)), "kind": "port",
            "sample": f"{iters} Q4_K GEMVs 9728x2560 with the C restatement (OpenMP rows) in {t:.1f} s"}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--replicas", type=int, default=0, help="0 = enough for >= 512 MB")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--direct", action="store_true",
                    help="launch steps directly, not from a HIP graph (for rocprofv3 runs)")
    args = ap.parse_args()
    global DIRECT
    DIRECT = args.direct
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py runs on one GPU only: this build measures the single-GPU hot path "
              "(row-sharding across GPUs is a design note, not built)", file=sys.stderr)
        sys.exit(2)

    ctx = qmm_hip.Context(0)
    info = ctx.device_info()
    log(f"device {info}")
    N, K = synth.GEMV_Q4K["N"], synth.GEMV_Q4K["K"]
    wl = Workload(ctx, synth.TYPE_Q4_K, N, K, 1, args.replicas, seed=0)
    parity = check_against_oracle(wl)
    step_bytes = N * 1440 + K * 4 + N * 4          # weights + fp32 x + fp32 y
    kern_bytes = N * 1440 + (K + 4 * K // 256 + 4 * K // 32) + N * 4  # weights + Q8_K x + y

    ms = wl.time(wl.step, args.steps, args.warmup)
    value = step_bytes / (ms * 1e-3) / 1e9
    log(f"step (quantize + GEMV), {wl.R} replicas: {ms * 1e3:.2f} us/step, {value:.1f} GB/s")
    # the step is one launch of the fused kernel (quantizer + GEMV): its
    # roofline is the step's algorithmic bytes over the step's duration
    ach = value
    ms_k = wl.time(wl.kernel_only, args.steps, args.warmup)
    ach_pre = kern_bytes / (ms_k * 1e-3) / 1e9
    log(f"GEMV on prequantized Q8_K activations: {ms_k * 1e3:.2f} us/launch, {ach_pre:.1f} GB/s")
    hot = Workload(ctx, synth.TYPE_Q4_K, N, K, 1, 1, seed=0)
    ms_hot = hot.time(hot.kernel_only, args.steps, args.warmup)
    hot.free()
    log(f"GEMV kernel, one replica (cache-resident): {ms_hot * 1e3:.2f} us/launch")

    extra = {}
    if not args.no_extra:
        tv = {}
        for M in synth.TREE_VERIFY["M"]:
            t = Workload(ctx, synth.TYPE_Q4_K, N, K, M, 0, seed=10 + M)
            steps = max(50, args.steps // 4)
            m_step = t.time(t.step, steps, 10)
            m_k = t.time(t.kernel_only, steps, 10)
            ops = 2.0 * M * N * K
            byts = N * 1440 + M * K * 4 + M * N * 4
            tv[f"M{M}"] = {"us_per_step": round(m_step * 1e3, 3), "us_gemm_kernel": round(m_k * 1e3, 3),
                           "tops": round(ops / (m_k * 1e-3) / 1e12, 3),
                           "gbs": round(byts / (m_step * 1e-3) / 1e9, 1)}
            log(f"tree-verify Q4_K M={M}: {tv[f'M{M}']}")
            t.free()
        extra["tree_verify_q4k_9728x2560"] = tv
        t5 = synth.TREE_VERIFY["q5k"]
        t = Workload(ctx, t5[0], t5[1], t5[2], 64, 0, seed=80)
        m_k = t.time(t.kernel_only, max(50, args.steps // 4), 10)
        extra["tree_verify_q5k_4096x2560_M64"] = {
            "us_gemm_kernel": round(m_k * 1e3, 3),
            "tops": round(2.0 * 64 * t5[1] * t5[2] / (m_k * 1e-3) / 1e12, 3)}
        log(f"tree-verify Q5_K 4096x2560 M=64: {extra['tree_verify_q5k_4096x2560_M64']}")
        t.free()
        extra["ffn_block_q4k_q6k"] = bench_ffn(ctx, max(50, args.steps // 10))
        log(f"FFN block: {extra['ffn_block_q4k_q6k']}")
        extra["prefill_layer_m512"] = bench_prefill(ctx, max(5, args.steps // 200))
        log(f"prefill layer M=512: {extra['prefill_layer_m512']}")
        extra["rmsnorm_q8k_then_gemv_q4k_9728x2560"] = bench_rmsnorm_gemv(ctx, max(200, args.steps // 4))
        log(f"RMSNorm->Q8_K + GEMV: {extra['rmsnorm_q8k_then_gemv_q4k_9728x2560']}")
        extra["lm_head_argmax_q6k_151936x2560"] = bench_lm_head_argmax(ctx, max(200, args.steps // 10))
        log(f"LM head + argmax: {extra['lm_head_argmax_q6k_151936x2560']}")
        extra["launch_floor_us"] = launch_floor(ctx, max(200, args.steps // 4))
        log(f"launch floor: {extra['launch_floor_us']} us")
        lm = Workload(ctx, synth.TYPE_Q6_K, 151936, 2560, 1, 2, seed=20)
        # a graph of >= 500 launches: shorter ones read high (100 launches: +16 %)
        m_lm = lm.time(lm.kernel_only, max(500, args.steps // 4), 5)
        lm_bytes = 151936 * 2100 + (2560 + 40 + 320) + 151936 * 4
        extra["lm_head_q6k_151936x2560"] = {"us_gemv_kernel": round(m_lm * 1e3, 2),
                                            "gbs": round(lm_bytes / (m_lm * 1e-3) / 1e9, 1)}
        log(f"LM head Q6_K GEMV: {extra['lm_head_q6k_151936x2560']}")
        lm.free()

    wl.free()
    ctx.close()

    cpu = None if args.no_cpu else cpu_baseline(N, K, args.cpu_seconds)
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
                   "N": N, "K": K, "M": 1, "replicas": wl.R,
                   "replica_bytes": wl.wbytes,
                   "timing": "direct launches, HIP events" if DIRECT else "HIP graph of all steps, HIP events"},
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "tokens_per_s_equiv": round(value * 1e9 / DECODE_BYTES_PER_TOKEN, 1),
        "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic(TRAFFIC_PROFILE),
                     "kernel": "gemv_persist_kernel<FmtQ4K4, 4, 3, true, 6, false> (fused Q8_K quantizer)",
                     "us_per_launch": round(ms * 1e3, 3), "algorithmic_bytes": step_bytes},
        "gemv_prequantized": {"kernel": "gemv_persist_kernel<FmtQ4K4, 4, 3, false, 6, false> on Q8_K input", "us_per_launch": round(ms_k * 1e3, 3),
                              "algorithmic_bytes": kern_bytes, "gbs": round(ach_pre, 1)},
        "cache_resident_us_per_launch": round(ms_hot * 1e3, 3),
        "parity": parity,
        "cpu_baseline": cpu,
        "device": info,
    }
    line.update(extra)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
