"""Dispatches captured into a HIP graph and replayed give the eager result on
every replay, with eager work and synchronisation between replays."""
import numpy as np
import pytest

import qmm_hip
import synth
from gpu_util import say
from oracle import TYPE_Q4_K, TYPE_Q6_K

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M", [1, 8])
def test_graph_replay_matches_eager(ctx, M):
    K, N = 2560, 512
    say(f"graph replay M={M}")
    w = ctx.weight_upload(synth.weights(TYPE_Q4_K, N, K, seed=5), TYPE_Q4_K, N, K)
    w6 = ctx.weight_upload(synth.weights(TYPE_Q6_K, 64, K, seed=6), TYPE_Q6_K, 64, K)
    xb = ctx.upload(synth.activations(M, K, seed=7))
    y_e, y_g = ctx.malloc(M * N * 4), ctx.malloc(M * N * 4)
    z_e, z_g = ctx.malloc(M * 64 * 4), ctx.malloc(M * 64 * 4)
    ctx.reserve(M, K)
    ctx.gemm_multi_dispatch(xb, M, K, [qmm_hip.MatrixTask(w, TYPE_Q4_K, N, K, y_e),
                                       qmm_hip.MatrixTask(w6, TYPE_Q6_K, 64, K, z_e)])
    ctx.sync()
    eager = ctx.d2h(y_e, np.float32, (M, N)), ctx.d2h(z_e, np.float32, (M, 64))
    ctx.graph_begin()
    ctx.gemm_multi_dispatch(xb, M, K, [qmm_hip.MatrixTask(w, TYPE_Q4_K, N, K, y_g),
                                       qmm_hip.MatrixTask(w6, TYPE_Q6_K, 64, K, z_g)])
    g = ctx.graph_end()
    for rep in range(3):
        ctx.h2d(y_g, np.zeros((M, N), np.float32))
        ctx.h2d(z_g, np.zeros((M, 64), np.float32))
        ctx.graph_launch(g)
        ctx.sync()
        assert np.array_equal(ctx.d2h(y_g, np.float32, (M, N)), eager[0]), rep
        assert np.array_equal(ctx.d2h(z_g, np.float32, (M, 64)), eager[1]), rep
        # eager work between replays
        ctx.gemm_multi_dispatch(xb, M, K, [qmm_hip.MatrixTask(w, TYPE_Q4_K, N, K, y_e)])
        ctx.sync()
    ctx.graph_destroy(g)
    for b in (w, w6, xb, y_e, y_g, z_e, z_g):
        ctx.free(b)


def test_graph_keeps_its_buffers_when_eager_calls_grow(ctx):
    """A graph captured at a small size keeps using the activation buffer it
    was captured with after an eager call at a larger size replaced it; the
    replays stay equal to the eager result (the replaced buffer is freed only
    with the last graph)."""
    K, N = 2560, 256
    say("graph buffers after growth")
    w = ctx.weight_upload(synth.weights(TYPE_Q4_K, N, K, seed=8), TYPE_Q4_K, N, K)
    xs = ctx.upload(synth.activations(2, K, seed=9))
    xl = ctx.upload(synth.activations(48, K, seed=10))
    ys, yl, ye = ctx.malloc(2 * N * 4), ctx.malloc(48 * N * 4), ctx.malloc(2 * N * 4)
    with qmm_hip.Context(0) as c2:  # a fresh context: its buffers are sized by this test alone
        c2.reserve(2, K)
        c2.gemm_multi_dispatch(xs, 2, K, [qmm_hip.MatrixTask(w, TYPE_Q4_K, N, K, ye)])
        c2.sync()
        eager = c2.d2h(ye, np.float32, (2, N))
        c2.graph_begin()
        c2.gemm_multi_dispatch(xs, 2, K, [qmm_hip.MatrixTask(w, TYPE_Q4_K, N, K, ys)])
        g = c2.graph_end()
        c2.gemm_multi_dispatch(xl, 48, K, [qmm_hip.MatrixTask(w, TYPE_Q4_K, N, K, yl)])  # grows the buffers
        c2.sync()
        for rep in range(3):
            c2.h2d(ys, np.zeros((2, N), np.float32))
            c2.graph_launch(g)
            c2.sync()
            assert np.array_equal(c2.d2h(ys, np.float32, (2, N)), eager), rep
            c2.gemm_multi_dispatch(xl, 48, K, [qmm_hip.MatrixTask(w, TYPE_Q4_K, N, K, yl)])
            c2.sync()
        c2.graph_destroy(g)
        c2.gemm_multi_dispatch(xs, 2, K, [qmm_hip.MatrixTask(w, TYPE_Q4_K, N, K, ye)])
        c2.sync()
        assert np.array_equal(c2.d2h(ye, np.float32, (2, N)), eager)
    for b in (w, xs, xl, ys, yl, ye):
        ctx.free(b)
