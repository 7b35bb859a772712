"""Pins the oracle's activation quantizers (quantize_row_fp16_to_q8_k
E:925-990, quantize_row_fp16_to_q8_0 E:1016-1064) by invariants and special
cases with known answers."""
import numpy as np
import pytest


def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("K", [256, 2560])
def test_q8k_invariants_random(oracle, K):
    x = np.random.default_rng(K).standard_normal((3, K)).astype(np.float32) * 3
    d, qs, bs = oracle.quantize_q8k(x)
    assert np.abs(qs.astype(int)).max() <= 127
    assert np.array_equal(bs, qs.reshape(3, -1, 32).astype(np.int32).sum(-1))
    # d = amax / 127 of the fp16-rounded block; the element holding amax maps to +-127
    xh = x.astype(np.float16).astype(np.float32).reshape(3, -1, 256)
    amax = np.abs(xh).max(-1)
    assert np.array_equal(d, (amax / np.float32(127)).astype(np.float32))
    qb = qs.reshape(3, -1, 256)
    arg = np.abs(xh).argmax(-1)
    assert np.all(np.abs(np.take_along_axis(qb, arg[..., None], -1)) == 127)
    # codes lie within half a step of x * 127 / amax
    err = np.abs(xh * (127 / amax[..., None]) - qb)
    assert err.max() <= 0.5 + 1e-4


def test_q8k_zero_block_and_single_nonzero(oracle):
    x = np.zeros((1, 512), np.float32)
    x[0, 300] = -0.75
    d, qs, bs = oracle.quantize_q8k(x)
    assert d[0, 0] == 0.0 and not qs[0, :256].any() and not bs[0, :8].any()
    assert d[0, 1] == np.float32(0.75) / np.float32(127)
    assert qs[0, 300] == -127 and np.count_nonzero(qs[0]) == 1
    assert bs[0, 300 // 32] == -127


def test_q8k_round_half_to_even(oracle):
    # amax = 127 makes id = 1 exactly, so x*id hits exact .5 ties
    x = np.zeros((1, 256), np.float32)
    x[0, :8] = [127, 2.5, 3.5, -2.5, 0.5, 1.5, -0.5, 126.5]
    d, qs, _ = oracle.quantize_q8k(x)
    assert d[0, 0] == 1.0
    assert list(qs[0, :8]) == [127, 2, 4, -2, 0, 2, 0, 126]


def test_q8k_integer_grid_is_fixed_point(oracle):
    g = np.random.default_rng(4)
    q = g.integers(-127, 128, (2, 768)).astype(np.float32)
    q[:, ::256] = 127  # every block reaches 127 -> d = 1, id = 1
    d, qs, _ = oracle.quantize_q8k(q)
    assert np.all(d == 1.0)
    assert np.array_equal(qs.astype(np.float32), q)


def test_q8k_fp32_contract_rounds_through_fp16(oracle):
    x = np.random.default_rng(9).standard_normal((2, 512)).astype(np.float32)
    d, qs, bs = oracle.quantize_q8k(x)
    for m in range(2):
        d2, q2, b2 = oracle.quantize_row_q8k_f16(_f16(x[m]))
        assert np.array_equal(d[m], d2) and np.array_equal(qs[m], q2) and np.array_equal(bs[m], b2)


def test_q8_0_invariants(oracle):
    x = np.random.default_rng(11).standard_normal((2, 320)).astype(np.float32)
    x[1, 32:64] = 0
    d, qs = oracle.quantize_q8_0(x)
    assert d[1, 1] == 0 and not qs[1, 32:64].any()
    xh = x.astype(np.float16).astype(np.float32).reshape(2, -1, 32)
    amax = np.abs(xh).max(-1)
    assert np.array_equal(d, (amax / np.float32(127)).astype(np.float32))
    assert np.abs(qs.astype(int)).max() <= 127
    x2 = np.zeros((1, 32), np.float32)
    x2[0, :4] = [127, 2.5, -3.5, 0.5]
    d2, q2 = oracle.quantize_q8_0(x2)
    assert d2[0, 0] == 1.0 and list(q2[0, :4]) == [127, 2, -4, 0]
