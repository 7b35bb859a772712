"""Pins the oracle's block formats and dequantizers (E:364-374, E:598-853):
row sizes, the 6-bit scale packing, and every dequantizer against closed
forms of blocks built from known parameters."""
import numpy as np
import pytest

import kquant_pack as kp
from oracle import TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0


def test_row_bytes_known_values(oracle):
    L = oracle.lib
    assert L.qo_row_bytes(TYPE_Q4_K, 2560) == 1440
    assert L.qo_row_bytes(TYPE_Q5_K, 2560) == 1760
    assert L.qo_row_bytes(TYPE_Q6_K, 2560) == 2100
    assert L.qo_row_bytes(TYPE_Q8_0, 2560) == 2720
    assert L.qo_row_bytes(TYPE_Q4_K, 4096) == 2304
    assert L.qo_row_bytes(TYPE_Q6_K, 9728) == 7980
    assert L.qo_row_bytes(99, 2560) == 0


def test_scale_min_k4_roundtrip_all_values(oracle):
    # every (sc, m) in 0..63 at every sub-block position
    g = np.random.default_rng(1)
    for trial in range(64):
        sc = (np.arange(8) * 8 + trial) % 64
        m = g.integers(0, 64, 8)
        packed = kp.pack_scales_k4(sc, m)
        for j in range(8):
            assert oracle.get_scale_min_k4(j, packed) == (sc[j], m[j])


def _f16_of(v):
    return np.asarray(v, np.float32).astype(np.float16).view(np.uint16)


def _params(g):
    d = float(np.float16(g.uniform(1e-3, 4e-3)))
    dmin = float(np.float16(g.uniform(1e-3, 4e-3)))
    return d, dmin, g.integers(0, 64, 8), g.integers(0, 64, 8)


@pytest.mark.parametrize("seed", range(6))
def test_dequant_q4_k_closed_form(oracle, seed):
    g = np.random.default_rng(seed)
    d, dmin, sc, m = _params(g)
    codes = g.integers(0, 16, 256)
    blk = kp.pack_q4_k(d, dmin, sc, m, codes)
    # y = fp16(d*sc*q - dmin*m): both products exact in fp32 (<= 21 bits)
    d32, dm32 = np.float32(d), np.float32(dmin)
    w = (d32 * kp.expand_sub(sc).astype(np.float32)) * codes.astype(np.float32) - dm32 * kp.expand_sub(m).astype(np.float32)
    assert np.array_equal(oracle.dequant_rows(TYPE_Q4_K, blk, 1, 256)[0], _f16_of(w))


@pytest.mark.parametrize("seed", range(6))
def test_dequant_q5_k_closed_form(oracle, seed):
    g = np.random.default_rng(100 + seed)
    d, dmin, sc, m = _params(g)
    codes = g.integers(0, 32, 256)
    blk = kp.pack_q5_k(d, dmin, sc, m, codes)
    d32, dm32 = np.float32(d), np.float32(dmin)
    w = (d32 * kp.expand_sub(sc).astype(np.float32)) * codes.astype(np.float32) - dm32 * kp.expand_sub(m).astype(np.float32)
    assert np.array_equal(oracle.dequant_rows(TYPE_Q5_K, blk, 1, 256)[0], _f16_of(w))


@pytest.mark.parametrize("seed", range(6))
def test_dequant_q6_k_closed_form(oracle, seed):
    g = np.random.default_rng(200 + seed)
    d = float(np.float16(g.uniform(1e-3, 4e-3)))
    sc = g.integers(-128, 128, 16)
    codes = g.integers(0, 64, 256)
    blk = kp.pack_q6_k(d, sc, codes)
    grp = np.array([kp.q6_group_of_value(k) for k in range(256)])
    w = (np.float32(d) * sc[grp].astype(np.float32)) * (codes - 32).astype(np.float32)
    assert np.array_equal(oracle.dequant_rows(TYPE_Q6_K, blk, 1, 256)[0], _f16_of(w))


def test_dequant_q8_0_closed_form(oracle):
    g = np.random.default_rng(3)
    for _ in range(8):
        d = float(np.float16(g.uniform(1e-3, 4e-3)))
        codes = g.integers(-128, 128, 32)
        blk = kp.pack_q8_0(d, codes)
        w = np.float32(d) * codes.astype(np.float32)
        assert np.array_equal(oracle.dequant_rows(TYPE_Q8_0, blk, 1, 32)[0], _f16_of(w))


def test_dequant_special_cases(oracle):
    # d = 0: every output is -dmin*m of its sub-block; sc = 0 likewise
    sc = np.zeros(8, int)
    m = np.full(8, 63)
    codes = np.full(256, 15)
    blk = kp.pack_q4_k(0.0, 0.5, sc, m, codes)
    out = oracle.fp16_to_f32(oracle.dequant_rows(TYPE_Q4_K, blk, 1, 256)[0])
    assert np.all(out == np.float32(-31.5))
    # maximal codes and scales: d*63*15 - 0
    blk = kp.pack_q4_k(1.0, 0.0, np.full(8, 63), np.zeros(8, int), np.full(256, 15))
    assert np.all(oracle.fp16_to_f32(oracle.dequant_rows(TYPE_Q4_K, blk, 1, 256)[0]) == 945.0)
    # Q5_K code 31 uses the high bit in every position
    blk = kp.pack_q5_k(1.0, 0.0, np.ones(8, int), np.zeros(8, int), np.full(256, 31))
    assert np.all(oracle.fp16_to_f32(oracle.dequant_rows(TYPE_Q5_K, blk, 1, 256)[0]) == 31.0)
    # Q6_K codes 0 and 63 map to -32 and +31
    blk = kp.pack_q6_k(1.0, np.ones(16, int), np.where(np.arange(256) % 2, 63, 0))
    out = oracle.fp16_to_f32(oracle.dequant_rows(TYPE_Q6_K, blk, 1, 256)[0])
    assert np.array_equal(out, np.where(np.arange(256) % 2, 31.0, -32.0).astype(np.float32))


def test_dequant_rows_multi_row_layout(oracle):
    # rows are consecutive blocks: dequant of 3 rows == per-block dequant
    import synth
    w = synth.weights(TYPE_Q6_K, 3, 512, seed=5)
    full = oracle.dequant_rows(TYPE_Q6_K, w, 3, 512)
    for r in range(3):
        for b in range(2):
            blk = w[(r * 2 + b) * 210:(r * 2 + b + 1) * 210]
            assert np.array_equal(full[r, 256 * b:256 * (b + 1)], oracle.dequant_rows(TYPE_Q6_K, blk, 1, 256)[0])
