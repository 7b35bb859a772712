"""The LM-head running argmax of the oracle (E:11172-11183: row order,
fp16-rounded logits, replace only on a strictly greater value) against a
different restatement — first position of the maximum, then a strict
comparison with the seed — on planted ties, NaNs and seed-equal values."""
import numpy as np


def _first_max_then_strict(lg, bv, bi, round16, ids, row_base, oracle):
    v = lg.astype(np.float32)
    if round16:
        v = oracle.fp16_to_f32(oracle.f32_to_fp16(v))
    outv, outi = bv.copy(), bi.copy()
    for m in range(v.shape[0]):
        row = np.where(np.isnan(v[m]), -np.inf, v[m])
        j = int(np.argmax(row))  # first occurrence of the maximum
        if row[j] > outv[m]:
            outv[m] = row[j]
            outi[m] = ids[j] if ids is not None else row_base + j
    return outv, outi


def test_chunk_argmax_semantics(oracle):
    g = np.random.default_rng(7)
    lg = g.standard_normal((4, 3000)).astype(np.float32) * 8
    lg[0, [10, 2000, 2999]] = 100.0         # ties: the first wins
    lg[1, 5] = np.nan                       # never taken
    lg[1, 100] = 90.0
    lg[2, :] = -5.0                         # all equal to the seed: nothing replaces
    lg[3, 700] = 100.01                     # rounds to the same fp16 as 100.0 ...
    lg[3, 701] = 100.0                      # ... so the earlier one wins after rounding
    seed_v = np.array([-1e30, -1e30, -5.0, -1e30], np.float32)
    seed_i = np.array([0, 0, 77, 0], np.uint32)
    for round16 in (True, False):
        got = oracle.chunk_argmax(lg, seed_v, seed_i, round16, None, 1000)
        exp = _first_max_then_strict(lg, seed_v, seed_i, round16, None, 1000, oracle)
        assert np.array_equal(got[0].view(np.uint32), exp[0].view(np.uint32))
        assert np.array_equal(got[1], exp[1])
    v, i = oracle.chunk_argmax(lg, seed_v, seed_i, True, None, 1000)
    assert i[0] == 1010 and i[1] == 1100 and i[2] == 77 and i[3] == 1700


def test_chunk_argmax_chains_like_one_pass(oracle):
    g = np.random.default_rng(8)
    lg = g.standard_normal((2, 5000)).astype(np.float32)
    lg[:, 4000] = lg[:, 100] = 9.0  # tie across chunks: the earlier chunk keeps it
    seed_v = np.full(2, -1e30, np.float32)
    seed_i = np.zeros(2, np.uint32)
    one = oracle.chunk_argmax(lg, seed_v, seed_i, True, None, 0)
    bv, bi = seed_v, seed_i
    for r0, r1 in ((0, 1234), (1234, 4000), (4000, 5000)):
        bv, bi = oracle.chunk_argmax(lg[:, r0:r1], bv, bi, True, None, r0)
    assert np.array_equal(one[0], bv) and np.array_equal(one[1], bi)
    assert list(bi) == [100, 100]


def test_indexed_rows_report_ids(oracle):
    lg = np.array([[1.0, 3.0, 3.0, 2.0]], np.float32)
    ids = np.array([50, 7, 9, 3], np.uint32)
    v, i = oracle.chunk_argmax(lg, np.array([-1e30], np.float32), np.zeros(1, np.uint32), False, ids, 0)
    assert v[0] == 3.0 and i[0] == 7
