"""The oracle against the committed known-answer vectors
(tests/golden/golden_vectors.npz, written by tests/golden/make_golden.py from
the reference's own scalar code). Runs everywhere, including where the
compiled reference is absent."""
import os

import numpy as np
import pytest

from oracle import TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0

TYPES = {"q4_k": TYPE_Q4_K, "q5_k": TYPE_Q5_K, "q6_k": TYPE_Q6_K, "q8_0": TYPE_Q8_0}
PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_vectors.npz")


@pytest.fixture(scope="module")
def gold():
    with np.load(PATH, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_fp16_cast(oracle, gold):
    assert np.array_equal(oracle.f32_to_fp16(gold["fp16_in"]), gold["fp16_out"])


@pytest.mark.parametrize("name", list(TYPES))
def test_dequant(oracle, gold, name):
    t = TYPES[name]
    qk = 32 if t == TYPE_Q8_0 else 256
    y = gold[f"dq_{name}_y"]
    got = oracle.dequant_rows(t, gold[f"dq_{name}_w"], y.shape[0], qk)
    assert np.array_equal(got, y)


def test_quantizers(oracle, gold):
    for i, x16 in enumerate(gold["q_x16"]):
        d, qs, bs = oracle.quantize_row_q8k_f16(x16)
        assert np.array_equal(d, gold["q8k_d"][i])
        assert np.array_equal(qs, gold["q8k_qs"][i])
        assert np.array_equal(bs, gold["q8k_bs"][i])
        d0, q0 = oracle.quantize_row_q8_0_f16(x16)
        assert np.array_equal(d0, gold["q80_d"][i]) and np.array_equal(q0, gold["q80_qs"][i])


@pytest.mark.parametrize("name", list(TYPES))
def test_dots(oracle, gold, name):
    t = TYPES[name]
    x = gold["dot_x"]
    M, K = x.shape
    y = gold[f"dot_{name}_y"]
    outs = oracle.gemm_multi(x, [dict(w=gold[f"dot_{name}_w"], type=t, rows=y.shape[1])])[0]
    assert np.array_equal(outs.view(np.uint32), y.view(np.uint32))


def test_swiglu(oracle, gold):
    g = oracle.fp16_to_f32(gold["sw_gate"])
    u = oracle.fp16_to_f32(gold["sw_up"])
    h, (d, qs, bs) = oracle.swiglu_q8k(g, u)
    assert np.array_equal(oracle.f32_to_fp16(h), gold["sw_h"])
    assert np.array_equal(d, gold["sw_d"]) and np.array_equal(qs, gold["sw_qs"])
    assert np.array_equal(bs, gold["sw_bs"])
