"""HIP quantizers and dequantizer vs the oracle: bit-exact."""
import numpy as np
import pytest

import synth
from gpu_util import say
from oracle import TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0

pytestmark = pytest.mark.gpu


def _inputs(M, K, seed):
    x = synth.activations(M, K, seed) * 2
    if M >= 3:
        x[1, :256] = 0                       # zero block
        x[2, :256] = 0
        x[2, :8] = [127, 2.5, 3.5, -2.5, 0.5, 1.5, -0.5, 126.5]  # exact .5 ties
    return x.astype(np.float32)


@pytest.mark.parametrize("M,K", [(1, 256), (3, 2560), (5, 9728), (37, 768), (64, 2560)])
def test_quantize_q8k_bit_exact(ctx, oracle, M, K):
    say(f"quantize_q8k M={M} K={K}")
    x = _inputs(M, K, seed=M * 31 + K)
    xb = ctx.upload(x)
    out = ctx.malloc(ctx.lib.qmm_q8k_bytes(M, K))
    ctx.quantize_q8k(xb, M, K, out)
    ctx.sync()
    d, qs, bs = ctx.read_q8k(out, M, K)
    ed, eqs, ebs = oracle.quantize_q8k(x)
    assert np.array_equal(d.view(np.uint32), ed.view(np.uint32))
    assert np.array_equal(qs, eqs)
    assert np.array_equal(bs, ebs)
    # the tiles section: the same codes in matrix-core operand order
    assert np.array_equal(ctx.read_q8k_tiles(out, M, K), qs)
    # the h section: the fp16 values the codes came from
    assert np.array_equal(ctx.read_q8k_h(out, M, K), oracle.f32_to_fp16(x))
    # the bh section: sums of 16 codes (pairs of them are the bsum32 values)
    bh = ctx.read_q8k_bh(out, M, K)
    assert np.array_equal(bh, eqs.reshape(M, K // 16, 16).astype(np.int32).sum(axis=2).astype(np.float32))
    assert np.array_equal(bh.reshape(M, K // 32, 2).sum(axis=2).astype(np.int32), ebs)
    ctx.free(xb)
    ctx.free(out)


@pytest.mark.parametrize("M,K", [(1, 32), (3, 2560), (7, 96)])
def test_quantize_q8_0_bit_exact(ctx, oracle, M, K):
    say(f"quantize_q8_0 M={M} K={K}")
    x = _inputs(M, K, seed=M + K) if K >= 256 else synth.activations(M, K, seed=3)
    xb = ctx.upload(x)
    out = ctx.malloc(ctx.lib.qmm_q8_0_bytes(M, K))
    ctx.quantize_q8_0(xb, M, K, out)
    ctx.sync()
    d, qs = ctx.read_q8_0(out, M, K)
    ed, eqs = oracle.quantize_q8_0(x)
    assert np.array_equal(d.view(np.uint32), ed.view(np.uint32))
    assert np.array_equal(qs, eqs)
    ctx.free(xb)
    ctx.free(out)


def test_swiglu_requant(ctx, oracle):
    M, N = 2, 9728
    say(f"swiglu_q8k M={M} N={N}")
    g = synth.activations(M, N, seed=41) * 3
    u = synth.activations(M, N, seed=42)
    gb, ub = ctx.upload(g), ctx.upload(u)
    hb = ctx.malloc(M * N * 4)
    out = ctx.malloc(ctx.lib.qmm_q8k_bytes(M, N))
    ctx.swiglu_q8k(gb, ub, M, N, hb, out)
    ctx.sync()
    h = ctx.d2h(hb, np.float32, (M, N))
    d, qs, bs = ctx.read_q8k(out, M, N)
    # SiLU uses the device expf: values within a few ulp of the host libm's
    eh, _ = oracle.swiglu_q8k(g, u)
    assert np.allclose(h, eh, rtol=1e-5, atol=1e-30)
    # the requant is pinned by composition: host quantizer on the device's h
    ed, eqs, ebs = oracle.quantize_q8k(h)
    assert np.array_equal(d.view(np.uint32), ed.view(np.uint32))
    assert np.array_equal(qs, eqs) and np.array_equal(bs, ebs)
    assert np.array_equal(ctx.read_q8k_tiles(out, M, N), qs)
    assert np.array_equal(ctx.read_q8k_bh(out, M, N),
                          qs.reshape(M, N // 16, 16).astype(np.int32).sum(axis=2).astype(np.float32))
    assert np.array_equal(ctx.read_q8k_h(out, M, N), oracle.f32_to_fp16(h))
    for b in (gb, ub, hb, out):
        ctx.free(b)


def test_swiglu_rounds_gate_and_up_to_fp16(ctx, oracle):
    """fp32 gate / up that are not fp16 values: SiLU sees fp16(g) and fp16(u)
    (E:4352-4353), so the device's h equals the device's h on the rounded
    inputs bit for bit, and its codes are the quantizer's codes of that h."""
    M, N = 1, 2560
    say("swiglu fp16 inputs")
    g = synth.activations(M, N, seed=43) * np.float32(3.0001)
    u = synth.activations(M, N, seed=44) * np.float32(1.0001)
    g16 = oracle.fp16_to_f32(oracle.f32_to_fp16(g))
    u16 = oracle.fp16_to_f32(oracle.f32_to_fp16(u))
    assert not np.array_equal(g16, g)
    outs = []
    for gi, ui in ((g, u), (g16, u16)):
        gb, ub = ctx.upload(gi), ctx.upload(ui)
        hb, out = ctx.malloc(M * N * 4), ctx.malloc(ctx.lib.qmm_q8k_bytes(M, N))
        ctx.swiglu_q8k(gb, ub, M, N, hb, out)
        ctx.sync()
        outs.append((ctx.d2h(hb, np.float32, (M, N)), ctx.read_q8k(out, M, N)))
        for b in (gb, ub, hb, out):
            ctx.free(b)
    assert np.array_equal(outs[0][0].view(np.uint32), outs[1][0].view(np.uint32))
    for a, b in zip(outs[0][1], outs[1][1]):
        assert np.array_equal(a, b)
    eh, _ = oracle.swiglu_q8k(g, u)
    assert np.allclose(outs[0][0], eh, rtol=1e-5, atol=1e-30)


def _weights(type_id, rows, cols, seed):
    if type_id in (0, 1):  # F32 / F16 rows
        v = synth.activations(rows, cols, seed=seed) * np.float32(40.0)
        return (v if type_id == 0 else v.astype(np.float16)).view(np.uint8).reshape(-1)
    return synth.weights(type_id, rows, cols, seed=seed)


@pytest.mark.parametrize("type_id,rows,cols", [(TYPE_Q4_K, 37, 512), (TYPE_Q5_K, 37, 512),
                                               (TYPE_Q6_K, 37, 512), (TYPE_Q8_0, 37, 512),
                                               (TYPE_Q6_K, 64, 2560), (0, 5, 2560), (1, 5, 2560)])
def test_dequant_bit_exact(ctx, oracle, type_id, rows, cols):
    say(f"dequant type={type_id} {rows}x{cols}")
    w = _weights(type_id, rows, cols, seed=type_id + rows)
    wb = ctx.weight_upload(w, type_id, rows, cols)
    yb = ctx.malloc(rows * cols * 2)
    ctx.dequantize_f16(wb, type_id, rows, cols, yb)
    ctx.sync()
    y = ctx.d2h(yb, np.uint16, (rows, cols))
    assert np.array_equal(y, oracle.dequant_rows(type_id, w, rows, cols))
    ctx.free(wb)
    ctx.free(yb)
