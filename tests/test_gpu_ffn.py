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


# --------------------------------------------- the block as one call
def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


class _Ffn:
    """One FFN block's weights and buffers on the device."""

    def __init__(self, ctx, K, F, H, tg, td, seed, residual=False):
        self.ctx, self.K, self.F, self.H, self.tg, self.td = ctx, K, F, H, tg, td
        self.x = synth.activations(1, K, seed=seed)
        self.wg = synth.weights(tg, F, K, seed=seed + 1)
        self.wu = synth.weights(tg, F, K, seed=seed + 2)
        self.wd = synth.weights(td, H, F, seed=seed + 3)
        self.bg, self.bu = ctx.weight_upload(self.wg, tg, F, K), ctx.weight_upload(self.wu, tg, F, K)
        self.bd = ctx.weight_upload(self.wd, td, H, F)
        self.xb = ctx.upload(self.x)
        self.res = synth.activations(1, H, seed=seed + 4) if residual else None
        self.rb = ctx.upload(self.res) if residual else None
        self.xq = ctx.malloc(ctx.lib.qmm_q8k_bytes(1, K))
        ctx.quantize_q8k(self.xb, 1, K, self.xq)
        self.bufs = [self.bg, self.bu, self.bd, self.xb, self.xq] + ([self.rb] if residual else [])

    def out(self):
        b = [self.ctx.malloc(n * 4) for n in (self.F, self.F, self.F, self.H)]
        self.bufs += b
        return b

    def tasks(self, g, u, y):
        return (qmm_hip.MatrixTask(self.bg, self.tg, self.F, self.K, g),
                qmm_hip.MatrixTask(self.bu, self.tg, self.F, self.K, u),
                qmm_hip.MatrixTask(self.bd, self.td, self.H, self.F, y, residual=self.rb))

    def three_calls(self, prequantized=False):
        ctx = self.ctx
        g, u, h, y = self.out()
        q = ctx.malloc(ctx.lib.qmm_q8k_bytes(1, self.F))
        self.bufs.append(q)
        tg, tu, td = self.tasks(g, u, y)
        if prequantized:
            ctx.gemm_multi_dispatch_prequantized(self.xq, None, 1, self.K, [tg, tu])
        else:
            ctx.gemm_multi_dispatch(self.xb, 1, self.K, [tg, tu])
        ctx.swiglu_q8k(g, u, 1, self.F, h, q)
        ctx.gemm_multi_dispatch_prequantized(q, None, 1, self.F, [td])
        return g, u, h, y

    def one_call(self, prequantized=False, h_out=True):
        g, u, h, y = self.out()
        tg, tu, td = self.tasks(g, u, y)
        if prequantized:
            self.ctx.ffn_block(None, self.xq, self.K, tg, tu, td, h if h_out else None)
        else:
            self.ctx.ffn_block(self.xb, None, self.K, tg, tu, td, h if h_out else None)
        return g, u, h, y

    def read(self, bufs):
        g, u, h, y = bufs
        F, H = self.F, self.H
        return (self.ctx.d2h(g, np.float32, (1, F)), self.ctx.d2h(u, np.float32, (1, F)),
                self.ctx.d2h(h, np.float32, (1, F)), self.ctx.d2h(y, np.float32, (1, H)))

    def free(self):
        for b in self.bufs:
            self.ctx.free(b)


def _same(a, b, h=True):
    names = ("gate", "up", "h", "down")
    for i, (p, q) in enumerate(zip(a, b)):
        if i == 2 and not h:
            continue
        nbad = int(np.count_nonzero(_bits(p) != _bits(q)))
        assert nbad == 0, f"{names[i]}: {nbad} of {p.size} values differ from the separate calls"


@pytest.mark.parametrize("case", [
    # K, F, H, gate/up type, down type, prequantized input, residual
    (2560, 9728, 2560, TYPE_Q4_K, TYPE_Q6_K, False, True),    # the model's block: 1 down row per wave
    (2560, 9728, 2560, TYPE_Q4_K, TYPE_Q4_K, True, False),    # Q4_K down, Q8_K input
    (3072, 12288, 3072, TYPE_Q4_K, TYPE_Q6_K, False, False),  # 7 loads per group, 3 rounds of h
    (2560, 3072, 8192, TYPE_Q4_K, TYPE_Q6_K, True, True),     # 4 down rows per wave
    (2560, 4096, 1000, TYPE_Q4_K, TYPE_Q6_K, False, True),    # down too short for the persistent grid
    (2560, 4096, 2560, qmm_hip.TYPE_Q5_K, TYPE_Q6_K, False, True),  # Q5_K gate/up, down too short
    (2560, 9728, 2560, qmm_hip.TYPE_Q5_K, TYPE_Q6_K, False, True),  # Q5_K gate/up: 7 loads per group
    (3072, 12288, 3072, qmm_hip.TYPE_Q5_K, TYPE_Q4_K, True, False),  # Q5_K at K = 3072: 9 loads per group
], ids=["model", "q4k_down_prequant", "k3072_f12288", "f3072_h8192", "h1000_separate", "q5k_separate", "q5k_model",
        "q5k_k3072"])
def test_ffn_block_one_call(ctx, oracle, case):
    K, F, H, tg, td, pre, res = case
    say(f"ffn_block K={K} F={F} H={H} gate={tg} down={td} pre={pre} res={res}")
    ctx.reserve(1, F)
    blk = _Ffn(ctx, K, F, H, tg, td, seed=K + F + H, residual=res)
    ref = blk.three_calls(prequantized=pre)
    got = blk.one_call(prequantized=pre)
    ctx.sync()
    a, b = blk.read(got), blk.read(ref)
    _same(a, b)
    if case[0:3] == (2560, 9728, 2560) and not pre:
        # and against the oracle, stage by stage, at the model's shape
        g_np, u_np, h_np, y_np = a
        rg, ru = oracle.gemm_multi(blk.x, [dict(w=blk.wg, type=tg, rows=F), dict(w=blk.wu, type=tg, rows=F)])
        check_outputs(g_np, rg, "gate")
        check_outputs(u_np, ru, "up")
        eq = oracle.quantize_q8k(h_np)
        ry = oracle.gemm_multi(h_np, [dict(w=blk.wd, type=td, rows=H)], prequantized=(eq, None))[0]
        if res:
            ry = (ry.astype(np.float32) + blk.res.astype(np.float32)).astype(np.float32)
        check_outputs(y_np, ry, "down")
    blk.free()


def test_ffn_block_repeated_and_without_h(ctx):
    """Calls back to back; h_out may be NULL."""
    K, F, H = 2560, 9728, 2560
    say("ffn_block repeated")
    ctx.reserve(1, F)
    blks = [_Ffn(ctx, K, F, H, TYPE_Q4_K, TYPE_Q6_K, seed=500 + 10 * i, residual=i == 1) for i in range(3)]
    refs = [b.three_calls() for b in blks]
    gots = [b.one_call(h_out=(i != 2)) for i, b in enumerate(blks)]
    again = [b.one_call() for b in blks]
    ctx.sync()
    for i, b in enumerate(blks):
        _same(b.read(gots[i]), b.read(refs[i]), h=(i != 2))
        _same(b.read(again[i]), b.read(refs[i]))
    for b in blks:
        b.free()


def test_ffn_block_graph_replays(ctx):
    """Captured in a graph and replayed several times, with eager work and
    synchronizations between the replays: every replay equals the eager
    result."""
    K, F, H = 2560, 9728, 2560
    say("ffn_block graph")
    ctx.reserve(1, F)
    blk = _Ffn(ctx, K, F, H, TYPE_Q4_K, TYPE_Q6_K, seed=900, residual=True)
    ref = blk.read(blk.three_calls())
    got = blk.out()
    tg, tu, td = blk.tasks(*got[:2], got[3])
    ctx.graph_begin()
    ctx.ffn_block(blk.xb, None, K, tg, tu, td, got[2])
    gr = ctx.graph_end()
    for rep in range(4):
        for b, n in zip(got, (F, F, F, H)):  # stale values a replay must overwrite
            ctx.h2d(b, np.full(n, np.nan if rep % 2 else 7.0, np.float32))
        blk.three_calls()  # eager work between the replays
        ctx.graph_launch(gr)
        ctx.sync()
        _same(blk.read(got), ref)
    ctx.graph_destroy(gr)
    blk.free()


@pytest.mark.parametrize("case", [
    # K, F, H, gate/up type, down type, residual
    (2560, 9728, 2560, TYPE_Q4_K, TYPE_Q6_K, True),            # the model's block: the norm in the gate/up fill
    (3072, 12288, 3072, qmm_hip.TYPE_Q5_K, TYPE_Q4_K, False),  # Q5_K gate/up at K = 3072
    (2560, 4096, 1000, TYPE_Q4_K, TYPE_Q6_K, True),            # down too short: the norm's kernel, three steps
    (4096, 4096, 2560, TYPE_Q4_K, TYPE_Q6_K, False),           # K past the fill: the norm's kernel, three steps
], ids=["model", "q5k_k3072", "three_steps", "k4096_three_steps"])
def test_ffn_block_rmsnorm(ctx, oracle, case):
    """qmm_ffn_block_rmsnorm equals qmm_rmsnorm_q8k followed by qmm_ffn_block
    on that prequantized row, bit for bit (gate, up, h, down)."""
    K, F, H, tg, td, residual = case
    say(f"ffn block rmsnorm K={K} F={F} H={H}")
    f = _Ffn(ctx, K, F, H, tg, td, seed=90 + K + F, residual=residual)
    gamma = np.random.default_rng(K + F).uniform(0.5, 1.5, K).astype(np.float32)
    gb = ctx.upload(gamma)
    f.bufs.append(gb)
    g, u, h, y = f.out()
    tg_, tu_, td_ = f.tasks(g, u, y)
    ctx.ffn_block_rmsnorm(f.xb, gb, K, tg_, tu_, td_, h)
    nq = ctx.malloc(ctx.lib.qmm_q8k_bytes(1, K))
    f.bufs.append(nq)
    ctx.rmsnorm_q8k(f.xb, gb, 1, K, None, nq)
    g2, u2, h2, y2 = f.out()
    tg2, tu2, td2 = f.tasks(g2, u2, y2)
    ctx.ffn_block(None, nq, K, tg2, tu2, td2, h2)
    ctx.sync()
    _same(f.read((g, u, h, y)), f.read((g2, u2, h2, y2)))
    f.free()
