"""The FFN block at batch 1 (gate + up Q4_K 9728 x 2560 on one shared Q8_K
input, SiLU(gate) * up, Q8_K requant, down Q6_K 2560 x 9728) — the CPU
fallback sequence of the reference (E:8290-8296) on the HIP path."""
import numpy as np
import pytest

import qmm_hip
import synth
from gpu_util import check_outputs, norm_err, say
from oracle import TYPE_Q4_K, TYPE_Q6_K

pytestmark = pytest.mark.gpu


def test_ffn_block(ctx, oracle):
    H, F = 2560, 9728
    say("ffn block")
    x = synth.activations(1, H, seed=70)
    wg = synth.weights(TYPE_Q4_K, F, H, seed=71)
    wu = synth.weights(TYPE_Q4_K, F, H, seed=72)
    wd = synth.weights(TYPE_Q6_K, H, F, seed=73)
    bg, bu, bd = (ctx.weight_upload(wg, TYPE_Q4_K, F, H), ctx.weight_upload(wu, TYPE_Q4_K, F, H),
                  ctx.weight_upload(wd, TYPE_Q6_K, H, F))
    xb = ctx.upload(x)
    g, u, h = ctx.malloc(F * 4), ctx.malloc(F * 4), ctx.malloc(F * 4)
    q = ctx.malloc(ctx.lib.qmm_q8k_bytes(1, F))
    y = ctx.malloc(H * 4)
    ctx.gemm_multi_dispatch(xb, 1, H, [qmm_hip.MatrixTask(bg, TYPE_Q4_K, F, H, g),
                                       qmm_hip.MatrixTask(bu, TYPE_Q4_K, F, H, u)])
    ctx.swiglu_q8k(g, u, 1, F, h, q)
    ctx.gemm_multi_dispatch_prequantized(q, None, 1, F, [qmm_hip.MatrixTask(bd, TYPE_Q6_K, H, F, y)])
    ctx.sync()
    g_np, u_np = ctx.d2h(g, np.float32, (1, F)), ctx.d2h(u, np.float32, (1, F))
    h_np, y_np = ctx.d2h(h, np.float32, (1, F)), ctx.d2h(y, np.float32, (1, H))
    rg, ru = oracle.gemm_multi(x, [dict(w=wg, type=TYPE_Q4_K, rows=F), dict(w=wu, type=TYPE_Q4_K, rows=F)])
    check_outputs(g_np, rg, "gate")
    check_outputs(u_np, ru, "up")
    # stage by stage: the down projection on the device's own requant is exact
    qd = ctx.read_q8k(q, 1, F)
    eq = oracle.quantize_q8k(h_np)
    for a, b in zip(qd, eq):
        assert np.array_equal(a, b)
    ry = oracle.gemm_multi(h_np, [dict(w=wd, type=TYPE_Q6_K, rows=H)], prequantized=(eq, None))[0]
    check_outputs(y_np, ry, "down")
    # end to end against the oracle's own SiLU (host expf): tolerance only
    rh, rq = oracle.swiglu_q8k(rg, ru)
    ry2 = oracle.gemm_multi(rh, [dict(w=wd, type=TYPE_Q6_K, rows=H)], prequantized=(rq, None))[0]
    assert norm_err(y_np, ry2) <= 1e-3
    for b in (bg, bu, bd, xb, g, u, h, q, y):
        ctx.free(b)
