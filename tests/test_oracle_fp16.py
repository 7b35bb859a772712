"""Pins the oracle's fp16 conversions (the reference's __fp16 casts,
E:592-596) against numpy's IEEE binary16 conversion (round to nearest even)
and against the compiled reference."""
import numpy as np
import pytest


def _bits_equal_or_both_nan(got, exp):
    nan = np.isnan(exp)
    assert np.isnan(got[nan]).all()
    assert np.array_equal(got[~nan].view(np.uint32), exp[~nan].view(np.uint32))


def test_fp16_to_f32_exhaustive(oracle):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    _bits_equal_or_both_nan(oracle.fp16_to_f32(h), h.view(np.float16).astype(np.float32))


def _boundary_floats():
    """Every finite half, the fp32 midpoints between neighbours, and the fp32
    neighbours of those midpoints (where round-to-nearest-even decides)."""
    h = np.arange(0, 0x7C00, dtype=np.uint32).astype(np.uint16)
    v = h.view(np.float16).astype(np.float64)
    nxt = np.append(v[1:], 65536.0)  # above 65504 the next step is the overflow threshold
    mid = ((v + nxt) / 2).astype(np.float32)
    up = np.nextafter(mid, np.float32(np.inf))
    dn = np.nextafter(mid, np.float32(-np.inf))
    pos = np.concatenate([v.astype(np.float32), mid, up, dn])
    return np.concatenate([pos, -pos, np.array([np.inf, -np.inf, 1e-30, -1e-30, 1e30], np.float32)])


def test_f32_to_fp16_rounding_boundaries(oracle):
    x = _boundary_floats()
    with np.errstate(over="ignore"):
        exp = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f32_to_fp16(x), exp)


def test_f32_to_fp16_strided_sweep(oracle):
    bits = (np.arange(0, 1 << 20, dtype=np.uint64) * 4093).astype(np.uint32)
    x = bits.view(np.float32)
    keep = ~np.isnan(x)
    x = x[keep]
    with np.errstate(over="ignore"):
        exp = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f32_to_fp16(x), exp)


def test_fp16_matches_compiled_reference(oracle, ref):
    g = np.random.default_rng(7)
    x = np.concatenate([_boundary_floats()[::37], g.standard_normal(2000).astype(np.float32) * 100])
    got = oracle.f32_to_fp16(x)
    exp = np.array([ref.f32_to_fp16(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, exp)
    h = np.arange(0, 65536, 97, dtype=np.uint32).astype(np.uint16)
    back = oracle.fp16_to_f32(h)
    exp_back = np.array([ref.fp16_to_f32(int(v)) for v in h], np.float32)
    _bits_equal_or_both_nan(back, exp_back)
