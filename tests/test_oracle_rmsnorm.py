"""The RMSNorm -> Q8_K producer of the oracle (rmsnorm_fp16_rows_fast,
E:4264-4314, scalar branch): bit-exact against the compiled reference where
it is built, and pinned without it by closed forms and an fp64 restatement."""
import numpy as np
import pytest


def _rows(M, K, seed, scale=1.0):
    g = np.random.default_rng(seed)
    return (g.standard_normal((M, K)) * scale).astype(np.float32)


def _gamma(K, seed):
    return np.random.default_rng(seed).uniform(0.5, 1.5, K).astype(np.float32)


@pytest.mark.parametrize("M,K", [(1, 256), (3, 2560), (2, 9216)])
def test_rmsnorm_matches_reference(oracle, ref, M, K):
    x16 = oracle.f32_to_fp16(_rows(M, K, seed=K + M))
    g16 = oracle.f32_to_fp16(_gamma(K, seed=K))
    y, (d, qs, bs) = oracle.rmsnorm_q8k_f16(x16, g16)
    ry, (rd, rqs, rbs) = ref.rmsnorm_q8k(x16, g16)
    assert np.array_equal(y, ry)
    assert np.array_equal(d.view(np.uint32), rd.view(np.uint32))
    assert np.array_equal(qs, rqs)
    assert np.array_equal(bs, rbs)


def test_rmsnorm_fp64_restatement(oracle):
    """y within one fp16 rounding (plus the fp32 sum's error) of
    x / sqrt(mean(x^2) + 1e-6) * gamma in fp64, including a row whose mean
    square is comparable to the epsilon (a wrong epsilon fails it)."""
    K = 2560
    x = np.concatenate([_rows(2, K, seed=3), _rows(1, K, seed=4, scale=1e-3)])
    gm = _gamma(K, seed=5)
    y, _ = oracle.rmsnorm_q8k(x, gm)
    x64 = oracle.fp16_to_f32(oracle.f32_to_fp16(x)).astype(np.float64)
    g64 = oracle.fp16_to_f32(oracle.f32_to_fp16(gm)).astype(np.float64)
    exp = x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + 1e-6) * g64
    rel = np.abs(y - exp) / np.maximum(np.abs(exp), 6.1e-5)
    assert rel.max() < 2e-3  # fp16 half-ulp is 4.9e-4; sum and products add a few fp32 ulps


def test_rmsnorm_closed_forms(oracle):
    """Constant rows with unit gamma normalise to sign(c) / sqrt(1 + 1e-6/c^2);
    the Q8_K of y is then the quantizer applied to y (composition)."""
    K = 512
    c = np.array([[1.0], [-2.0], [0.25]], np.float32)
    x = np.repeat(c, K, axis=1)
    y, (d, qs, bs) = oracle.rmsnorm_q8k(x, np.ones(K, np.float32))
    exp = np.sign(c) / np.sqrt(1.0 + 1e-6 / (c.astype(np.float64) ** 2))
    assert np.allclose(y, exp, rtol=1e-3, atol=0)
    ed, eqs, ebs = oracle.quantize_q8k(y)
    assert np.array_equal(qs, eqs) and np.array_equal(bs, ebs)
    assert np.array_equal(d.view(np.uint32), ed.view(np.uint32))
