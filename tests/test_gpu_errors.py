"""Argument validation of the C ABI: every bad call returns a status code
(the reference's dispatcher has none, E:4188-4262). The failing calls launch
no kernel; a context is needed, hence the gpu mark."""
import ctypes as C

import numpy as np
import pytest

import qmm_hip
import synth
from oracle import TYPE_Q4_K, TYPE_Q6_K

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def bufs(ctx):
    K, N = 512, 8
    w = ctx.weight_upload(synth.weights(TYPE_Q4_K, N, K, seed=1), TYPE_Q4_K, N, K)
    x = ctx.upload(synth.activations(1, K, seed=2))
    y = ctx.malloc(4 * N * 4)
    yield dict(w=w, x=x, y=y, K=K, N=N)
    for b in (w, x, y):
        ctx.free(b)


def _dispatch(ctx, x, M, K, task):
    arr = (qmm_hip._Task * 1)(task)
    return ctx.lib.qmm_gemm_multi_dispatch(ctx._h, C.c_void_p(int(x)), M, K, arr, 1)


def _task(b, **kw):
    t = dict(w_base=int(b["w"]), type=TYPE_Q4_K, row_bytes=qmm_hip.row_bytes(TYPE_Q4_K, b["K"]),
             dst=int(b["y"]), dst_stride=b["N"], residual=None, res_stride=0, rows=b["N"],
             cols=b["K"], start_row=0)
    t.update(kw)
    return qmm_hip._Task(**t)


def test_valid_call_is_ok(ctx, bufs):
    assert _dispatch(ctx, bufs["x"], 1, bufs["K"], _task(bufs)) == qmm_hip.QMM_OK
    ctx.sync()


@pytest.mark.parametrize("kw,code", [
    (dict(type=2), qmm_hip.QMM_ETYPE),  # Q4_0: not on this path
    (dict(type=99), qmm_hip.QMM_ETYPE),
    (dict(cols=256), qmm_hip.QMM_ESHAPE),
    (dict(row_bytes=100), qmm_hip.QMM_ESHAPE),
    (dict(dst=None), qmm_hip.QMM_EINVAL),
    (dict(w_base=None), qmm_hip.QMM_EINVAL),
    (dict(rows=-1), qmm_hip.QMM_EINVAL),
])
def test_bad_task_fields(ctx, bufs, kw, code):
    t = _task(bufs, **kw)
    if "w_base" in kw:
        t.w_base = None
    if "dst" in kw:
        t.dst = None
    assert _dispatch(ctx, bufs["x"], 1, bufs["K"], t) == code
    assert ctx.last_error()


def test_misaligned_pointers(ctx, bufs):
    t = _task(bufs)
    t.w_base = int(bufs["w"]) + 8  # Q4_K rows must be 16-B aligned
    assert _dispatch(ctx, bufs["x"], 1, bufs["K"], t) == qmm_hip.QMM_EALIGN
    assert _dispatch(ctx, int(bufs["x"]) + 4, 1, bufs["K"], _task(bufs)) == qmm_hip.QMM_EALIGN
    t = _task(bufs)
    t.dst = int(bufs["y"]) + 2
    assert _dispatch(ctx, bufs["x"], 1, bufs["K"], t) == qmm_hip.QMM_EALIGN


def test_bad_sizes(ctx, bufs):
    assert _dispatch(ctx, bufs["x"], 0, bufs["K"], _task(bufs)) == qmm_hip.QMM_EINVAL
    assert _dispatch(ctx, bufs["x"], 1, 300, _task(bufs, cols=300)) == qmm_hip.QMM_ESHAPE
    t = _task(bufs, dst_stride=1)
    assert _dispatch(ctx, bufs["x"], 4, bufs["K"], t) == qmm_hip.QMM_EINVAL
    # M * K past 2^31 at M >= 2 (checked before any allocation or launch)
    assert _dispatch(ctx, bufs["x"], (1 << 31) // bufs["K"], bufs["K"], _task(bufs)) == qmm_hip.QMM_ESHAPE
    arr = (qmm_hip._Task * 1)(_task(bufs))
    assert ctx.lib.qmm_gemm_multi_dispatch(ctx._h, C.c_void_p(int(bufs["x"])), 1, bufs["K"], arr, 0) == qmm_hip.QMM_EINVAL
    assert ctx.lib.qmm_gemm_multi_dispatch(ctx._h, None, 1, bufs["K"], arr, 1) == qmm_hip.QMM_EINVAL


def test_prequantized_requires_activations(ctx, bufs):
    arr = (qmm_hip._Task * 1)(_task(bufs))
    rc = ctx.lib.qmm_gemm_multi_dispatch_prequantized(ctx._h, None, None, 1, bufs["K"], arr, 1)
    assert rc == qmm_hip.QMM_EINVAL


def test_other_entry_points(ctx, bufs):
    L, h = ctx.lib, ctx._h
    out = ctx.malloc(L.qmm_q8k_bytes(1, 512))
    assert L.qmm_quantize_q8k(h, C.c_void_p(int(bufs["x"])), 1, 300, C.c_void_p(int(out))) == qmm_hip.QMM_ESHAPE
    assert L.qmm_quantize_q8_0(h, C.c_void_p(int(bufs["x"])), 1, 33, C.c_void_p(int(out))) == qmm_hip.QMM_ESHAPE
    assert L.qmm_quantize_q8k(h, None, 1, 256, C.c_void_p(int(out))) == qmm_hip.QMM_EINVAL
    assert L.qmm_dequantize_f16(h, C.c_void_p(int(bufs["w"])), 5, 1, 256, C.c_void_p(int(out))) == qmm_hip.QMM_ETYPE
    assert L.qmm_dequantize_f16(h, C.c_void_p(int(bufs["w"])), TYPE_Q6_K, 1, 100, C.c_void_p(int(out))) == qmm_hip.QMM_ESHAPE
    assert L.qmm_swiglu_q8k(h, None, None, 1, 256, None, None) == qmm_hip.QMM_EINVAL
    p = C.c_void_p()
    blocks = np.zeros(144, np.uint8)
    assert L.qmm_weight_upload(h, C.c_void_p(blocks.ctypes.data), 3, 1, 256, C.byref(p)) == qmm_hip.QMM_ETYPE
    assert L.qmm_weight_upload(h, C.c_void_p(blocks.ctypes.data), TYPE_Q4_K, 1, 100, C.byref(p)) == qmm_hip.QMM_ESHAPE
    assert L.qmm_malloc(h, 1 << 62, C.byref(p)) == qmm_hip.QMM_ENOMEM
    ctx.free(out)
    ctx.sync()
