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
