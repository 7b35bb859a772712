"""Seeded sweeps of batch-1 shapes through the C ABI against the oracle, bit
for bit: every k-quant format and Q8_0 over heights that land on the
persistent grid and off it, ragged last row groups, K up to 3072 and 9728,
residuals; and the FFN block entry point over gate/up and down shapes."""
import numpy as np
import pytest

import qmm_hip
import synth
from gpu_util import check_outputs, say
from oracle import TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0

pytestmark = pytest.mark.gpu
NAMES = {TYPE_Q4_K: "Q4_K", TYPE_Q5_K: "Q5_K", TYPE_Q6_K: "Q6_K", TYPE_Q8_0: "Q8_0"}


def _cases(n, seed):
    g = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        t = int(g.choice([TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0]))
        K = int(g.choice([256, 512, 768, 1280, 2560, 3072, 4096, 9728]))
        if t == TYPE_Q8_0:
            K = int(g.choice([32, 96, 288, 1024, 2560]))
        N = int(g.choice([int(g.integers(1, 700)), int(g.integers(4000, 9000)), int(g.integers(9000, 24000))]))
        out.append((t, N, K, bool(g.integers(0, 2)), int(g.integers(0, 1 << 30))))
    return out


@pytest.mark.parametrize("case", _cases(24, 7), ids=lambda c: f"{NAMES[c[0]]}-N{c[1]}-K{c[2]}-r{int(c[3])}")
def test_gemv_sweep(ctx, oracle, case):
    t, N, K, residual, seed = case
    say(f"sweep {NAMES[t]} N={N} K={K} residual={residual}")
    w = synth.weights(t, N, K, seed=seed)
    x = synth.activations(1, K, seed=seed + 1)
    res = synth.activations(1, N, seed=seed + 2) if residual else None
    wb = ctx.weight_upload(w, t, N, K)
    y = ctx.gemm(t, wb, N, K, x, res)
    ctx.free(wb)
    task = dict(w=w, type=t, rows=N)
    if res is not None:
        task["residual"] = res
    check_outputs(y, oracle.gemm_multi(x, [task])[0], f"sweep {NAMES[t]} N={N} K={K}")


def _ffn_cases(n, seed):
    g = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        K = int(g.choice([256, 1024, 2560, 3072]))
        F = 256 * int(g.integers(8, 48))
        H = int(g.choice([int(g.integers(100, 2000)), int(g.integers(2048, 6000))]))
        td = int(g.choice([TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K]))
        out.append((K, F, H, td, bool(g.integers(0, 2)), int(g.integers(0, 1 << 30))))
    return out


@pytest.mark.parametrize("case", _ffn_cases(8, 11), ids=lambda c: f"K{c[0]}-F{c[1]}-H{c[2]}-{NAMES[c[3]]}")
def test_ffn_block_sweep(ctx, oracle, case):
    """qmm_ffn_block (two launches where they apply, three elsewhere) against
    the oracle stage by stage: gate and up bit-exact, h's Q8_K codes equal
    to the oracle's quantizer on the device's h, down bit-exact on them."""
    K, F, H, td, residual, seed = case
    say(f"ffn sweep K={K} F={F} H={H} down={NAMES[td]} residual={residual}")
    x = synth.activations(1, K, seed=seed)
    wg = synth.weights(TYPE_Q4_K, F, K, seed=seed + 1)
    wu = synth.weights(TYPE_Q4_K, F, K, seed=seed + 2)
    wd = synth.weights(td, H, F, seed=seed + 3)
    res = synth.activations(1, H, seed=seed + 4) if residual else None
    bg, bu = ctx.weight_upload(wg, TYPE_Q4_K, F, K), ctx.weight_upload(wu, TYPE_Q4_K, F, K)
    bd = ctx.weight_upload(wd, td, H, F)
    xb = ctx.upload(x)
    rb = ctx.upload(res) if residual else None
    g, u, h, y = ctx.malloc(F * 4), ctx.malloc(F * 4), ctx.malloc(F * 4), ctx.malloc(H * 4)
    ctx.reserve(1, F)
    ctx.ffn_block(xb, None, K, qmm_hip.MatrixTask(bg, TYPE_Q4_K, F, K, g), qmm_hip.MatrixTask(bu, TYPE_Q4_K, F, K, u),
                  qmm_hip.MatrixTask(bd, td, H, F, y, residual=rb), h)
    ctx.sync()
    g_np, u_np = ctx.d2h(g, np.float32, (1, F)), ctx.d2h(u, np.float32, (1, F))
    h_np, y_np = ctx.d2h(h, np.float32, (1, F)), ctx.d2h(y, np.float32, (1, H))
    rg, ru = oracle.gemm_multi(x, [dict(w=wg, type=TYPE_Q4_K, rows=F), dict(w=wu, type=TYPE_Q4_K, rows=F)])
    check_outputs(g_np, rg, "gate")
    check_outputs(u_np, ru, "up")
    eq = oracle.quantize_q8k(h_np)
    task = dict(w=wd, type=td, rows=H)
    if residual:
        task["residual"] = res
    check_outputs(y_np, oracle.gemm_multi(h_np, [task], prequantized=(eq, None))[0], "down")
    for b in (bg, bu, bd, xb, g, u, h, y) + ((rb,) if residual else ()):
        ctx.free(b)


def _gemm_cases(n, seed):
    g = np.random.default_rng(seed)
    out = []
    for i in range(n):
        t = int(g.choice([TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0]))
        K = int(g.choice([256, 768, 2560, 3072, 4096])) if t != TYPE_Q8_0 else int(g.choice([64, 288, 2560]))
        if i % 3 == 2:  # the prefill kernels, on short tensors (the scalar oracle's time)
            M, N = int(g.integers(65, 300)), int(g.integers(16, 700))
        else:
            M, N = int(g.integers(2, 81)), int(g.integers(16, 6000))
        out.append((t, N, K, M, bool(g.integers(0, 2)), int(g.integers(0, 1 << 30))))
    return out


@pytest.mark.parametrize("case", _gemm_cases(18, 13), ids=lambda c: f"{NAMES[c[0]]}-N{c[1]}-K{c[2]}-M{c[3]}-r{int(c[4])}")
def test_gemm_sweep(ctx, oracle, case):
    t, N, K, M, residual, seed = case
    say(f"sweep {NAMES[t]} N={N} K={K} M={M} residual={residual}")
    w = synth.weights(t, N, K, seed=seed)
    x = synth.activations(M, K, seed=seed + 1)
    res = synth.activations(M, N, seed=seed + 2) if residual else None
    wb = ctx.weight_upload(w, t, N, K)
    y = ctx.gemm(t, wb, N, K, x, res)
    ctx.free(wb)
    task = dict(w=w, type=t, rows=N)
    if res is not None:
        task["residual"] = res
    check_outputs(y, oracle.gemm_multi(x, [task])[0], f"sweep {NAMES[t]} N={N} K={K} M={M}")


def _small_m_cases(n, seed):
    g = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        t = int(g.choice([TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0]))
        M = int(g.choice([int(g.integers(2, 5)), int(g.integers(5, 17)), int(g.integers(17, 33)), int(g.integers(33, 65))]))
        K = int(g.choice([256, 768, 2560, 3072, 3328, 4352, 9728]))
        if t == TYPE_Q8_0:
            K = int(g.choice([32, 288, 1024, 2560, 4096]))
        hi = 10000 if K <= 3072 else 3200  # (keeps the oracle's share of the sweep to seconds)
        N = int(g.choice([int(g.integers(1, 700)), int(g.integers(2000, 3000)), int(g.integers(3000, hi))]))
        out.append((t, M, N, K, bool(g.integers(0, 2)), int(g.integers(0, 1 << 30))))
    return out


@pytest.mark.parametrize("case", _small_m_cases(24, 13),
                         ids=lambda c: f"{NAMES[c[0]]}-M{c[1]}-N{c[2]}-K{c[3]}-r{int(c[4])}")
def test_gemm_small_m_sweep(ctx, oracle, case):
    """2..64 tokens: whichever kernel the dispatcher picks for the shape
    (the batch-1 shape for a few tokens, resident tiles, part tiles on token
    groups, chunked tiles, decoded slabs split over K), bit for bit."""
    t, M, N, K, residual, seed = case
    say(f"small-M sweep {NAMES[t]} M={M} N={N} K={K} residual={residual}")
    w = synth.weights(t, N, K, seed=seed)
    x = synth.activations(M, K, seed=seed + 1)
    res = synth.activations(M, N, seed=seed + 2) if residual else None
    wb = ctx.weight_upload(w, t, N, K)
    y = ctx.gemm(t, wb, N, K, x, res)
    ctx.free(wb)
    task = dict(w=w, type=t, rows=N)
    if res is not None:
        task["residual"] = res
    check_outputs(y, oracle.gemm_multi(x, [task])[0], f"small-M sweep {NAMES[t]} M={M} N={N} K={K}")


def _prefill_cases(n, seed):
    g = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        t = int(g.choice([TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0]))
        M = int(g.integers(65, 300))
        K = int(g.choice([256, 1280, 2560, 3072, 4352, 9728]))
        if t == TYPE_Q8_0:
            K = int(g.choice([64, 1024, 2560, 4096]))
        N = int(g.integers(1, 1500 if K <= 3072 else 500))
        out.append((t, M, N, K, bool(g.integers(0, 2)), int(g.integers(0, 1 << 30))))
    return out


@pytest.mark.parametrize("case", _prefill_cases(12, 17),
                         ids=lambda c: f"{NAMES[c[0]]}-M{c[1]}-N{c[2]}-K{c[3]}-r{int(c[4])}")
def test_gemm_prefill_sweep(ctx, oracle, case):
    """65..300 tokens on ragged shapes: the slab kernels (packed or decoded,
    each slab shape the launcher picks) and the Q8_0 tiles, bit for bit."""
    t, M, N, K, residual, seed = case
    say(f"prefill sweep {NAMES[t]} M={M} N={N} K={K} residual={residual}")
    w = synth.weights(t, N, K, seed=seed)
    x = synth.activations(M, K, seed=seed + 1)
    res = synth.activations(M, N, seed=seed + 2) if residual else None
    wb = ctx.weight_upload(w, t, N, K)
    y = ctx.gemm(t, wb, N, K, x, res)
    ctx.free(wb)
    task = dict(w=w, type=t, rows=N)
    if res is not None:
        task["residual"] = res
    check_outputs(y, oracle.gemm_multi(x, [task])[0], f"prefill sweep {NAMES[t]} M={M} N={N} K={K}")
