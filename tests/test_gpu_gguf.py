"""GGUF residency: tensors uploaded from a GGUF file (qmm_gguf_upload) and
used by the dispatcher give the oracle's results on the file's bytes."""
import numpy as np
import pytest

import gguf_writer as gw
import qmm_hip
import synth
from gpu_util import check_outputs, say
from oracle import TYPE_Q4_K, TYPE_Q6_K

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M", [1, 5])
def test_gguf_upload_and_dispatch(tmp_path, ctx, oracle, M):
    say(f"gguf upload M={M}")
    K = 2560
    wq4 = synth.weights(TYPE_Q4_K, 300, K, seed=31)
    wq6 = synth.weights(TYPE_Q6_K, 200, K, seed=32)
    path = tmp_path / "t.gguf"
    gw.write(path, [("general.architecture", gw.STR, "test")],
             [("a.weight", [K, 300], TYPE_Q4_K, wq4.tobytes()), ("b.weight", [K, 200], TYPE_Q6_K, wq6.tobytes())],
             align=64)
    x = synth.activations(M, K, seed=33)
    xb = ctx.upload(x)
    with qmm_hip.Gguf(str(path)) as g:
        pa, ia = g.upload(ctx, "a.weight")
        pb, ib = g.upload(ctx, "b.weight")
    assert (ia["type"], ia["dims"][:2]) == (TYPE_Q4_K, [K, 300])
    ya, yb = ctx.malloc(M * 300 * 4), ctx.malloc(M * 200 * 4)
    ctx.gemm_multi_dispatch(xb, M, K, [qmm_hip.MatrixTask(pa, TYPE_Q4_K, 300, K, ya, 300),
                                       qmm_hip.MatrixTask(pb, TYPE_Q6_K, 200, K, yb, 200)])
    ctx.sync()
    ra, rb = oracle.gemm_multi(x, [dict(w=wq4, type=TYPE_Q4_K, rows=300), dict(w=wq6, type=TYPE_Q6_K, rows=200)])
    check_outputs(ctx.d2h(ya, np.float32, (M, 300)), ra, "gguf Q4_K")
    check_outputs(ctx.d2h(yb, np.float32, (M, 200)), rb, "gguf Q6_K")
    for b in (xb, ya, yb):
        ctx.free(b)
    ctx.lib.qmm_free(ctx._h, pa)
    ctx.lib.qmm_free(ctx._h, pb)
