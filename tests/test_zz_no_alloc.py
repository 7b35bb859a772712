"""qmm_gemm_multi_dispatch_noalloc against qmm_gemm_multi_dispatch, through
the C ABI: two calls in a row on the device scratch (the second with a
smaller input, so stale scratch from the first is present), each equal bit
for bit to the allocating dispatcher's outputs; a call past the scratch's
size is refused before anything is launched."""
import numpy as np
import pytest

import qmm_hip
import synth
from gpu_util import say
from oracle import TYPE_F32, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0

pytestmark = pytest.mark.gpu


def _weights(type_id, rows, K, seed):
    if type_id == TYPE_F32:
        return (synth.activations(rows, K, seed=seed) * np.float32(0.05)).view(np.uint8).reshape(-1)
    return synth.weights(type_id, rows, K, seed=seed)


def _both(ctx, specs, M, K, seed):
    """Outputs of the allocating and the no-allocation dispatch on the same
    input and weights."""
    x = synth.activations(M, K, seed=seed)
    xb = ctx.upload(x)
    bufs = [xb]
    ta, tb = [], []
    for i, (t, n) in enumerate(specs):
        wb = ctx.weight_upload(_weights(t, n, K, seed + 1 + i), t, n, K)
        ya, yb = ctx.malloc(M * n * 4), ctx.malloc(M * n * 4)
        bufs += [wb, ya, yb]
        ta.append(qmm_hip.MatrixTask(wb, t, n, K, ya, n))
        tb.append(qmm_hip.MatrixTask(wb, t, n, K, yb, n))
    ctx.gemm_multi_dispatch(xb, M, K, ta)
    ctx.gemm_multi_dispatch_noalloc(xb, M, K, tb)
    ctx.sync()
    out = [(ctx.d2h(a.dst, np.float32, (M, a.rows)), ctx.d2h(b.dst, np.float32, (M, b.rows))) for a, b in zip(ta, tb)]
    for b in bufs:
        ctx.free(b)
    return out


def _same(pairs, what):
    for i, (a, b) in enumerate(pairs):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{what}: task {i} differs"


def test_noalloc_matches_dispatch_twice(ctx):
    K = 2560
    say("noalloc call 1: M=48, Q4_K + Q8_0 + F32 + Q6_K")
    _same(_both(ctx, [(TYPE_Q4_K, 300), (TYPE_Q8_0, 70), (TYPE_F32, 20), (TYPE_Q6_K, 64)], 48, K, seed=500),
          "first call")
    say("noalloc call 2: M=5, Q5_K (smaller)")
    _same(_both(ctx, [(TYPE_Q5_K, 130)], 5, K, seed=510), "second call")
    say("noalloc call 3: M=1")
    _same(_both(ctx, [(TYPE_Q4_K, 257), (TYPE_Q8_0, 33)], 1, K, seed=520), "batch-1 call")


def test_noalloc_refuses_inputs_past_the_scratch(ctx):
    say("noalloc size limit")
    cap = int(ctx.lib.qmm_noalloc_scratch_bytes())
    assert cap == 32 << 20
    K = 9728
    M = 1
    while ctx.lib.qmm_q8k_bytes(M, K) <= cap:
        M *= 2
    w = ctx.weight_upload(synth.weights(TYPE_Q6_K, 16, K, seed=530), TYPE_Q6_K, 16, K)
    y = ctx.malloc(16 * 4)
    x = ctx.malloc(16)  # never read: the call is refused before any launch
    t = (qmm_hip._Task * 1)(qmm_hip._Task(int(w), TYPE_Q6_K, qmm_hip.row_bytes(TYPE_Q6_K, K), int(y), 16, None, 16,
                                          16, K, 0))
    rc = ctx.status_of("qmm_gemm_multi_dispatch_noalloc", qmm_hip._p(int(x)), M, K, t, 1)
    assert rc == qmm_hip.QMM_ESHAPE and "scratch" in ctx.last_error()
    ctx.sync()
    for b in (w, y, x):
        ctx.free(b)


def test_noalloc_captures_in_a_fresh_context():
    """The point of the entry point: a context that never reserved or
    allocated activation buffers captures the dispatch into a HIP graph (a
    call that needed a buffer would fail the capture with QMM_ENOMEM), and
    every replay — with eager work, fresh inputs and synchronizations in
    between — equals the eager allocating dispatch bit for bit, at M = 48
    (the scratch path) and M = 1 (the fused batch-1 path)."""
    K = 2560
    with qmm_hip.Context(0) as fresh, qmm_hip.Context(0) as eager:
        for M, specs, seed in ((48, [(TYPE_Q4_K, 300), (TYPE_Q8_0, 70), (TYPE_F32, 20)], 540),
                               (1, [(TYPE_Q4_K, 257), (TYPE_Q6_K, 64)], 550)):
            say(f"noalloc graph capture in a fresh context: M={M}")
            xb = fresh.malloc(M * K * 4)
            ws, tf, te = [], [], []
            for i, (t, n) in enumerate(specs):
                host = _weights(t, n, K, seed + 1 + i)
                wf, we = fresh.weight_upload(host, t, n, K), eager.weight_upload(host, t, n, K)
                yf, ye = fresh.malloc(M * n * 4), eager.malloc(M * n * 4)
                ws += [(fresh, wf), (eager, we), (fresh, yf), (eager, ye)]
                tf.append(qmm_hip.MatrixTask(wf, t, n, K, yf, n))
                te.append(qmm_hip.MatrixTask(we, t, n, K, ye, n))
            fresh.graph_begin()
            fresh.gemm_multi_dispatch_noalloc(xb, M, K, tf)
            g = fresh.graph_end()
            try:
                for r in range(3):
                    x = synth.activations(M, K, seed=seed + 10 + r)
                    fresh.h2d(xb, x)
                    for a in tf:  # a replay that skipped a task would leave this pattern
                        fresh.h2d(a.dst, np.full(M * a.rows, np.nan, np.float32))
                    fresh.sync()
                    fresh.graph_launch(g)
                    fresh.sync()
                    xe = eager.upload(x)
                    eager.gemm_multi_dispatch(xe, M, K, te)
                    eager.sync()
                    eager.free(xe)
                    for i, (a, b) in enumerate(zip(tf, te)):
                        got = fresh.d2h(a.dst, np.float32, (M, a.rows))
                        ref = eager.d2h(b.dst, np.float32, (M, b.rows))
                        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), \
                            f"M={M} replay {r}: task {i} differs from the eager dispatch"
            finally:
                fresh.graph_destroy(g)
            for c, b in ws:
                c.free(b)
            fresh.free(xb)
