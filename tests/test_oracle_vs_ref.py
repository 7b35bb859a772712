"""The oracle against the reference's own scalar code compiled in place
(oracle/_ref/libref.so, built from src/v182_r22_breakthrough_engine.c by
oracle/Makefile): dequant bits, Q8_K / Q8_0 codes and fp32 dot sums must be
identical. Skipped where the compiled reference is absent."""
import numpy as np
import pytest

import kquant_pack as kp
import synth
from oracle import BLOCK_BYTES, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0

ALL = [TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0]


def _special_blocks(type_id):
    if type_id == TYPE_Q4_K:
        return [kp.pack_q4_k(0.0, 0.5, np.zeros(8, int), np.full(8, 63), np.full(256, 15)),
                kp.pack_q4_k(65504.0, 65504.0, np.full(8, 63), np.full(8, 63), np.arange(256) % 16)]
    if type_id == TYPE_Q5_K:
        return [kp.pack_q5_k(1.0, 0.0, np.ones(8, int), np.zeros(8, int), np.arange(256) % 32),
                kp.pack_q5_k(6e-5, 2.0, np.full(8, 63), np.full(8, 63), np.full(256, 31))]
    if type_id == TYPE_Q6_K:
        return [kp.pack_q6_k(1.0, np.full(16, -128), np.arange(256) % 64),
                kp.pack_q6_k(0.0, np.full(16, 127), np.full(256, 63))]
    return [kp.pack_q8_0(1.0, np.arange(-16, 16)), kp.pack_q8_0(65504.0, np.full(32, -128))]


@pytest.mark.parametrize("type_id", ALL)
def test_dequant_matches_reference(oracle, ref, type_id):
    qk = 32 if type_id == TYPE_Q8_0 else 256
    rnd = synth.blocks(type_id, 40, seed=type_id).reshape(-1)
    w = np.concatenate([rnd] + _special_blocks(type_id))
    nblk = w.size // BLOCK_BYTES[type_id]
    got = oracle.dequant_rows(type_id, w, nblk, qk)
    exp = ref.dequant_rows(type_id, w, nblk, qk)
    assert np.array_equal(got, exp)


def _quant_inputs():
    g = np.random.default_rng(21)
    rows = [g.standard_normal(768).astype(np.float32),
            (g.standard_normal(768) * 1e-3).astype(np.float32),
            (g.standard_normal(768) * 1e4).astype(np.float32),
            np.zeros(768, np.float32)]
    tie = np.zeros(768, np.float32)
    tie[:8] = [127, 2.5, 3.5, -2.5, 0.5, 1.5, -0.5, 126.5]
    tie[256] = -6e-8  # fp16 subnormal amax
    tie[512:520] = [1, -1, 0.5, 0.25, 1e-8, -65504, 65504, 3]
    rows.append(tie)
    return [r.astype(np.float16).view(np.uint16) for r in rows]


def test_quantizers_match_reference(oracle, ref):
    for x16 in _quant_inputs():
        for a, b in zip(oracle.quantize_row_q8k_f16(x16), ref.quantize_row_q8k_f16(x16)):
            assert np.array_equal(a, b)
        for a, b in zip(oracle.quantize_row_q8_0_f16(x16), ref.quantize_row_q8_0_f16(x16)):
            assert np.array_equal(a, b)


@pytest.mark.parametrize("type_id", ALL)
@pytest.mark.parametrize("K", [256, 2560])
def test_dots_match_reference(oracle, ref, type_id, K):
    M = 3
    x = synth.activations(M, K, seed=K + type_id)
    w = synth.weights(type_id, 4, K, seed=type_id * 7 + K)
    rb = w.size // 4
    if type_id == TYPE_Q8_0:
        d, qs = oracle.quantize_q8_0(x)
        bs = None
    else:
        d, qs, bs = oracle.quantize_q8k(x)
    for r in range(4):
        row = w[r * rb:(r + 1) * rb]
        got = np.array([oracle.dot_row(type_id, row, K, d[m], qs[m], None if bs is None else bs[m])
                        for m in range(M)], np.float32)
        kernels = [True] if type_id == TYPE_Q8_0 else ([False, True] if type_id != TYPE_Q4_K else [False])
        for batch in kernels:
            exp = ref.dot_rows(type_id, row, K, d, qs, bs, batch_kernel=batch)
            assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), (type_id, K, r, batch)


def test_swiglu_requant_matches_reference(oracle, ref):
    g = np.random.default_rng(5)
    gate = (g.standard_normal((2, 512)) * 3).astype(np.float16)
    up = g.standard_normal((2, 512)).astype(np.float16)
    h16, (d, qs, bs) = ref.swiglu_q8k(gate.view(np.uint16), up.view(np.uint16))
    h, (d2, qs2, bs2) = oracle.swiglu_q8k(gate.astype(np.float32), up.astype(np.float32))
    # both use the host libm expf; the reference stores h as fp16 (E:4355)
    assert np.array_equal(oracle.f32_to_fp16(h), h16)
    assert np.array_equal(d, d2) and np.array_equal(qs, qs2) and np.array_equal(bs, bs2)


@pytest.mark.parametrize("type_id", [0, 1])
@pytest.mark.parametrize("K", [32, 2560])
def test_float_rows_match_reference(oracle, ref, type_id, K):
    """sdot_row_f32_batch / sdot_row_f16_batch (E:3410-3440): bit for bit."""
    g = np.random.default_rng(K + type_id)
    x16 = (g.standard_normal((3, K)) * 2).astype(np.float16).view(np.uint16)
    for r in range(3):
        if type_id == 0:
            row = (g.standard_normal(K) * 0.05).astype(np.float32).view(np.uint8)
        else:
            row = (g.standard_normal(K) * 0.05).astype(np.float16).view(np.uint8)
        got = np.array([oracle.dot_row_float(type_id, row, K, x16[m]) for m in range(3)], np.float32)
        exp = ref.dot_rows_float(type_id, row, K, x16)
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


@pytest.mark.parametrize("type_id", [0, 1])
def test_float_dequant_matches_reference(oracle, ref, type_id):
    """dequant_contiguous_fast of F32 / F16 rows (E:3857-3860, E:3876-3879)."""
    g = np.random.default_rng(3 + type_id)
    v = g.standard_normal(600) * 300
    v[:6] = [65519.0, 65520.0, 1e-8, -6e-8, 0.0, -0.0]
    with np.errstate(over="ignore"):  # 65520 and above round to inf in fp16
        w = (v.astype(np.float32) if type_id == 0 else v.astype(np.float16)).view(np.uint8)
    got = oracle.dequant_rows(type_id, w, 20, 30)
    exp = ref.dequant_contiguous(type_id, w, 600)
    assert np.array_equal(got.reshape(-1), exp)


def test_swiglu_fp32_inputs_match_reference(oracle, ref):
    """fp32 gate / up that are not fp16 values: the oracle rounds them to fp16
    first, as the reference's gate / up are the dispatcher's fp16 outputs."""
    g = np.random.default_rng(6)
    gate = (g.standard_normal((2, 512)) * 3).astype(np.float32) + np.float32(1e-4)
    up = g.standard_normal((2, 512)).astype(np.float32) * np.float32(1.0001)
    assert not np.array_equal(gate.astype(np.float16).astype(np.float32), gate)
    h16, (d, qs, bs) = ref.swiglu_q8k(oracle.f32_to_fp16(gate), oracle.f32_to_fp16(up))
    h, (d2, qs2, bs2) = oracle.swiglu_q8k(gate, up)
    assert np.array_equal(oracle.f32_to_fp16(h), h16)
    assert np.array_equal(d, d2) and np.array_equal(qs, qs2) and np.array_equal(bs, bs2)
