"""Pins the oracle's row dots (eval_single_lm_row_dot E:10986-11105,
sdot_row_q5_k/q6_k/q8_0_batch E:3109-3408) and the dispatcher's task
semantics (E:3491-3619, E:4188-4262) with blocks of known parameters:
exact integer partials, fp64 brute force, unit-scale reduction to a plain
int8 dot."""
import numpy as np
import pytest

import kquant_pack as kp
import synth
from oracle import TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0


def _random_kquant_row(g, type_id, nb):
    """(packed row, per-value fp64 weights, per-block params)."""
    blocks, wvals, params = [], [], []
    for _ in range(nb):
        d = float(np.float16(g.uniform(1e-3, 4e-3)))
        dmin = float(np.float16(g.uniform(1e-3, 4e-3)))
        if type_id == TYPE_Q6_K:
            sc = g.integers(-32, 32, 16)
            codes = g.integers(0, 64, 256)
            blocks.append(kp.pack_q6_k(d, sc, codes))
            grp = np.array([kp.q6_group_of_value(k) for k in range(256)])
            wvals.append(d * sc[grp] * (codes - 32.0))
            params.append(dict(d=d, sc=sc, codes=codes, grp=grp))
        else:
            sc, m = g.integers(0, 64, 8), g.integers(0, 64, 8)
            hi = 16 if type_id == TYPE_Q4_K else 32
            codes = g.integers(0, hi, 256)
            pack = kp.pack_q4_k if type_id == TYPE_Q4_K else kp.pack_q5_k
            blocks.append(pack(d, dmin, sc, m, codes))
            wvals.append(d * kp.expand_sub(sc) * codes - dmin * kp.expand_sub(m))
            params.append(dict(d=d, dmin=dmin, sc=sc, m=m, codes=codes))
    return np.concatenate(blocks), np.concatenate(wvals), params


@pytest.mark.parametrize("type_id", [TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K])
def test_block_partials_exact(oracle, type_id):
    g = np.random.default_rng(type_id)
    row, _, params = _random_kquant_row(g, type_id, 2)
    x = g.standard_normal((1, 512)).astype(np.float32)
    d, qs, bs = oracle.quantize_q8k(x)
    S, Mb = oracle.block_partials(type_id, row, 512, qs[0], bs[0])
    for b, p in enumerate(params):
        q = qs[0, 256 * b:256 * (b + 1)].astype(np.int64)
        if type_id == TYPE_Q6_K:
            assert S[b] == int(np.sum(p["sc"][p["grp"]] * (p["codes"] - 32) * q))
            assert Mb[b] == 0
        else:
            assert S[b] == int(np.sum(kp.expand_sub(p["sc"]) * p["codes"] * q))
            assert Mb[b] == int(np.sum(p["m"] * bs[0, 8 * b:8 * (b + 1)]))


@pytest.mark.parametrize("type_id", [TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K])
def test_dot_vs_fp64_brute_force(oracle, type_id):
    g = np.random.default_rng(50 + type_id)
    row, wv, _ = _random_kquant_row(g, type_id, 2)
    x = g.standard_normal((1, 512)).astype(np.float32)
    d, qs, bs = oracle.quantize_q8k(x)
    xq = np.repeat(d[0].astype(np.float64), 256) * qs[0]
    exact = float(np.dot(wv, xq))
    got = oracle.dot_row(type_id, row, 512, d[0], qs[0], bs[0])
    assert abs(got - exact) <= 1e-5 * np.abs(wv * xq).sum()


def test_dot_q8_0_vs_fp64(oracle):
    g = np.random.default_rng(77)
    blocks, wv = [], []
    for _ in range(8):
        dd = float(np.float16(g.uniform(1e-3, 4e-3)))
        c = g.integers(-127, 128, 32)
        blocks.append(kp.pack_q8_0(dd, c))
        wv.append(dd * c)
    row, wv = np.concatenate(blocks), np.concatenate(wv)
    x = g.standard_normal((1, 256)).astype(np.float32)
    d, qs = oracle.quantize_q8_0(x)
    exact = float(np.dot(wv, np.repeat(d[0].astype(np.float64), 32) * qs[0]))
    got = oracle.dot_row(TYPE_Q8_0, row, 256, d[0], qs[0])
    assert abs(got - exact) <= 1e-5 * np.abs(wv).sum()


def test_unit_scales_reduce_to_int8_dot(oracle):
    g = np.random.default_rng(5)
    codes = g.integers(0, 16, 256)
    row = kp.pack_q4_k(1.0, 0.0, np.ones(8, int), np.zeros(8, int), codes)
    q = g.integers(-127, 128, 256).astype(np.int8)
    got = oracle.dot_row(TYPE_Q4_K, row, 256, np.ones(1, np.float32), q, np.zeros(8, np.int32))
    assert got == float(np.dot(codes, q.astype(np.int64)))
    # with mins: dot - dmin * sum(m * bsum)
    row = kp.pack_q4_k(1.0, 1.0, np.ones(8, int), np.full(8, 2), codes)
    bsum = q.astype(np.int32).reshape(8, 32).sum(-1)
    got = oracle.dot_row(TYPE_Q4_K, row, 256, np.ones(1, np.float32), q, bsum)
    assert got == float(np.dot(codes, q.astype(np.int64)) - 2 * bsum.sum())


def test_gemm_multi_task_semantics(oracle):
    K, M = 512, 3
    x = synth.activations(M, K, seed=1)
    w1 = synth.weights(TYPE_Q4_K, 5, K, seed=2)
    w2 = synth.weights(TYPE_Q6_K, 3, K, seed=3)
    w3 = synth.weights(TYPE_Q8_0, 4, K, seed=4)
    res = np.random.default_rng(0).standard_normal((M, 3)).astype(np.float32)
    outs = oracle.gemm_multi(x, [dict(w=w1, type=TYPE_Q4_K, rows=5),
                                 dict(w=w2, type=TYPE_Q6_K, rows=3, residual=res),
                                 dict(w=w3, type=TYPE_Q8_0, rows=4)])
    d, qs, bs = oracle.quantize_q8k(x)
    d0, q0 = oracle.quantize_q8_0(x)
    for m in range(M):
        for r in range(5):
            assert outs[0][m, r] == oracle.dot_row(TYPE_Q4_K, w1[r * 288:(r + 1) * 288], K, d[m], qs[m], bs[m])
        for r in range(3):
            v = oracle.dot_row(TYPE_Q6_K, w2[r * 420:(r + 1) * 420], K, d[m], qs[m], bs[m])
            assert outs[1][m, r] == np.float32(v) + res[m, r]
        for r in range(4):
            assert outs[2][m, r] == oracle.dot_row(TYPE_Q8_0, w3[r * 544:(r + 1) * 544], K, d0[m], q0[m])


def test_gemm_multi_rejects_bad_tasks(oracle):
    x = synth.activations(1, 512, seed=1)
    w = synth.weights(TYPE_Q4_K, 2, 512, seed=2)
    with pytest.raises(ValueError):
        oracle.gemm_multi(x[:, :300], [dict(w=w, type=TYPE_Q4_K, rows=2)])
    with pytest.raises(ValueError):
        oracle.gemm_multi(x, [dict(w=w, type=2, rows=2)])  # Q4_0 is not on this path


def test_float_rows_closed_forms(oracle):
    """F32 / F16 rows (E:3410-3440): unit weights sum the inputs exactly while
    the partial sums stay integers below 2^24; the sum is in row order —
    2^24 followed by ones stays 2^24 (each + 1 is a tie to even), where any
    other order of the ones first would give 2^24 + 2k."""
    K = 2560
    x16 = np.ones(K, np.float16).view(np.uint16)
    ones32 = np.ones(K, np.float32).view(np.uint8)
    ones16 = np.ones(K, np.float16).view(np.uint8)
    assert oracle.dot_row_float(0, ones32, K, x16) == K
    assert oracle.dot_row_float(1, ones16, K, x16) == K
    w = np.ones(K, np.float32)
    w[0] = 2.0 ** 24
    assert oracle.dot_row_float(0, w.view(np.uint8), K, x16) == 2.0 ** 24
    w[0], w[-1] = 1.0, 2.0 ** 24
    # ones first: the exact integer 2559, then one rounding of 2^24 + 2559
    assert oracle.dot_row_float(0, w.view(np.uint8), K, x16) == np.float32(2.0 ** 24 + K - 1)


@pytest.mark.parametrize("type_id", [0, 1])
def test_float_rows_vs_fp64(oracle, type_id):
    g = np.random.default_rng(11 + type_id)
    K = 2048
    x = g.standard_normal(K).astype(np.float16)
    w = (g.standard_normal(K) * 0.1).astype(np.float32 if type_id == 0 else np.float16)
    exact = float(np.dot(w.astype(np.float64), x.astype(np.float64)))
    got = oracle.dot_row_float(type_id, w.view(np.uint8), K, x.view(np.uint16))
    assert abs(got - exact) <= K * 2.0 ** -23 * float(np.abs(w.astype(np.float64) * x).sum())
