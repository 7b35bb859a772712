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


# ---------------------------------------------------------------------------
# The chunked vocabulary scan (E:11138-11256): outcomes fixed by planted
# logits. Random rows give logits below 1; planted rows give chosen ones.
import lm_plant  # noqa: E402
import synth  # noqa: E402
from oracle import TYPE_Q6_K  # noqa: E402

V, CH, K = 20000, 4096, 2560  # 5 chunks, the last 3616 rows


def _scan_setup(oracle, M, seed):
    w = lm_plant.base_tensor(V + 16, K, seed)  # 16 rows past the vocabulary, never scanned
    q = oracle.quantize_q8k(synth.activations(M, K, seed=seed + 1))
    return w, q


def test_scan_random_logits_stay_small(oracle):
    w, q = _scan_setup(oracle, 1, 900)
    bv, bi, n, act, stp = oracle.lm_head_scan(q, w, TYPE_Q6_K, V, K, CH, lm_plant.CHUNK_THRESH)
    assert abs(bv[0]) < 2.0 and n == 5 and stp == 0 and act == 1


def test_scan_exits_at_the_first_met_threshold(oracle):
    w, q = _scan_setup(oracle, 1, 901)
    # 14 in chunk 2: below 19.5 and 16 (chunks 0, 1), above 13.5 (chunk 2)
    (v,) = lm_plant.plant(w, oracle, q, [(2 * CH + 77, 0, 14.0)], K)
    assert 13.5 < v < 16.0
    bv, bi, n, act, stp = oracle.lm_head_scan(q, w, TYPE_Q6_K, V, K, CH, lm_plant.CHUNK_THRESH)
    assert (n, stp, int(bi[0])) == (3, 1, 2 * CH + 77)
    assert bv[0] == np.float32(np.float16(v))  # chunk logits compare as fp16
    # a chunk-0 row above 19.5 ends the scan after one chunk
    lm_plant.plant(w, oracle, q, [(5, 0, 25.0)], K)
    bv, bi, n, act, stp = oracle.lm_head_scan(q, w, TYPE_Q6_K, V, K, CH, lm_plant.CHUNK_THRESH)
    assert (n, stp, int(bi[0])) == (1, 1, 5)
    # with the first checkpoint at chunk 3 (all chunks required up to it), chunk 3's 11.5 ends it
    bv, bi, n, act, stp = oracle.lm_head_scan(q, w, TYPE_Q6_K, V, K, CH, lm_plant.CHUNK_THRESH, first_checkpoint=3)
    assert (n, stp, int(bi[0])) == (4, 1, 5)
    # no thresholds: every chunk is read
    bv, bi, n, act, stp = oracle.lm_head_scan(q, w, TYPE_Q6_K, V, K, CH, None)
    assert (n, stp, int(bi[0])) == (5, 0, 5)


def test_scan_pre_rows_and_candidates(oracle):
    M = 3
    w, q = _scan_setup(oracle, M, 902)
    eos = [V - 2, V - 4]
    draft = np.array([0, 600, V + 7], np.uint32)  # token 1's candidate is past the vocabulary
    (ve, vc) = lm_plant.plant(w, oracle, q, [(V - 4, 0, 30.0), (600, 0, 3.0)], K)
    bv, bi, n, act, stp = oracle.lm_head_scan(q, w, TYPE_Q6_K, V, K, CH, None, pre_ids=eos, draft_ids=draft)
    # token 0: the second pre row (fp32 value) wins and no chunk beats it
    assert int(bi[0]) == V - 4 and bv[0] == np.float32(ve)
    # token 0's best is not its candidate (600) and beats it: the active batch ends at 1
    assert act == 1 and n == 5


def test_scan_pruning_freezes_later_positions(oracle):
    M = 4
    w, q = _scan_setup(oracle, M, 903)
    draft = np.array([0, 100, 200, 300], np.uint32)
    # token 0: its candidate 100 has logit 5, row 1500 (chunk 0) has 8 -> prune to 1 after chunk 0;
    # tokens 1..3: rows in chunk 1 with 12 — never seen, since they are no longer active
    plan = [(100, 0, 5.0), (1500, 0, 8.0), (CH + 10, 1, 12.0), (CH + 20, 2, 12.0), (CH + 30, 3, 12.0)]
    lm_plant.plant(w, oracle, q, plan, K)
    bv, bi, n, act, stp = oracle.lm_head_scan(q, w, TYPE_Q6_K, V, K, CH, None, draft_ids=draft)
    assert act == 1 and int(bi[0]) == 1500
    assert all(bv[p] < 2.0 for p in (1, 2, 3))
    # without draft ids nothing is pruned and the chunk-1 rows win
    bv, bi, n, act, stp = oracle.lm_head_scan(q, w, TYPE_Q6_K, V, K, CH, None)
    assert act == M and [int(i) for i in bi[1:]] == [CH + 10, CH + 20, CH + 30]


# ---------------------------------------------------------------------------
# The script-gated exit (E:9716-9733 at batch 1, E:11185-11241 batched):
# outcomes fixed by planted logits and script tables.
def _tables(rows_cyr=(), rows_cjk=()):
    is_cyr = np.zeros(V, np.uint8)
    is_cjk = np.zeros(V, np.uint8)
    is_cyr[list(rows_cyr)] = 1
    is_cjk[list(rows_cjk)] = 1
    return is_cyr, is_cjk


def test_script_scan_without_a_script_is_the_plain_scan(oracle):
    M = 3
    w, q = _scan_setup(oracle, M, 910)
    draft = np.array([0, 700, 9000], np.uint32)
    lm_plant.plant(w, oracle, q, [(700, 0, 4.0), (CH + 3, 0, 6.0), (2 * CH + 9, 1, 14.0), (9000, 1, 3.0)], K)
    is_cyr, is_cjk = _tables()
    for thr in (lm_plant.CHUNK_THRESH, None):
        plain = oracle.lm_head_scan(q, w, TYPE_Q6_K, V, K, CH, thr, pre_ids=[V - 3], draft_ids=draft)
        got = oracle.lm_head_scan_script(q, w, TYPE_Q6_K, V, K, CH, thr, pre_ids=[V - 3], draft_ids=draft,
                                         is_cyr=is_cyr, is_cjk=is_cjk, cyr_rows=[5, 6], cjk_rows=[7])
        assert np.array_equal(plain[0].view(np.uint32), got[0].view(np.uint32))
        assert np.array_equal(plain[1], got[1]) and plain[2:] == got[2:5]
        assert got[5:] == (False, False)


def test_script_exit_batched(oracle):
    M = 1
    w, q = _scan_setup(oracle, M, 911)
    ext = [3 * CH + 5, 3 * CH + 6]  # extended rows outside chunk 0
    is_cyr, is_cjk = _tables(rows_cyr=ext)
    (v,) = lm_plant.plant(w, oracle, q, [(3 * CH + 6, 0, 12.0)], K)
    assert 11.5 < v < 13.5
    kw = dict(is_cyr=is_cyr, is_cjk=is_cjk, cyr_rows=ext)
    # the session already writes Cyrillic: after chunk 0 the extended rows give 12 on a Cyrillic token,
    # >= 11.5, so the scan ends after one chunk with that row (fp32 value)
    bv, bi, n, act, stp, hc, hj = oracle.lm_head_scan_script(q, w, TYPE_Q6_K, V, K, CH, lm_plant.CHUNK_THRESH,
                                                             has_cyr=True, **kw)
    assert (n, stp, int(bi[0]), hc) == (1, 1, 3 * CH + 6, True) and bv[0] == np.float32(v)
    # no script in the session: the row is found when chunk 3 is scanned (fp16 value), and chunk 3's
    # threshold 11.5 ends the scan there; that best token then sets the session's flag (for later
    # tokens: the extended rows run only after chunk 0)
    bv, bi, n, act, stp, hc, hj = oracle.lm_head_scan_script(q, w, TYPE_Q6_K, V, K, CH, lm_plant.CHUNK_THRESH, **kw)
    assert (n, stp, int(bi[0]), hc) == (4, 1, 3 * CH + 6, True) and bv[0] == np.float32(np.float16(v))
    # the full scan is required: no script exit, and with 5 chunks no checkpoint (they start at chunk 6)
    bv, bi, n, act, stp, hc, hj = oracle.lm_head_scan_script(q, w, TYPE_Q6_K, V, K, CH, lm_plant.CHUNK_THRESH,
                                                             has_cyr=True, require_full=True, **kw)
    assert (n, stp, int(bi[0])) == (5, 0, 3 * CH + 6)


def test_script_exit_needs_an_in_script_best_or_20(oracle):
    w, q = _scan_setup(oracle, 1, 912)
    ext = [4 * CH + 1]
    is_cyr, is_cjk = _tables(rows_cjk=ext)
    # chunk 0 holds 15 on a token of no script: the session has CJK (set below by chunk 0's best), so
    # the extended rows run, but the best is not CJK and 15 < 20: no script exit; 15 < 19.5 and 16,
    # >= 13.5 at chunk 2
    (v0, v1) = lm_plant.plant(w, oracle, q, [(900, 0, 15.0), (4 * CH + 1, 0, 11.0)], K)
    is_cjk[900] = 0
    bv, bi, n, act, stp, hc, hj = oracle.lm_head_scan_script(q, w, TYPE_Q6_K, V, K, CH, lm_plant.CHUNK_THRESH,
                                                             is_cyr=is_cyr, is_cjk=is_cjk, cjk_rows=ext,
                                                             has_cjk=True)
    assert (n, stp, int(bi[0])) == (3, 1, 900)
    # chunk 0's best is itself a CJK token: it sets the session's flag, the extended rows run, and
    # 15 on an in-script token clears 11.5
    is_cjk[900] = 1
    bv, bi, n, act, stp, hc, hj = oracle.lm_head_scan_script(q, w, TYPE_Q6_K, V, K, CH, lm_plant.CHUNK_THRESH,
                                                             is_cyr=is_cyr, is_cjk=is_cjk, cjk_rows=ext)
    assert (n, stp, int(bi[0]), hj) == (1, 1, 900, True)


def test_script_exit_batch1_rule_is_10_5(oracle):
    w, q = _scan_setup(oracle, 1, 913)
    ext = [2 * CH + 40]
    is_cyr, is_cjk = _tables(rows_cyr=ext)
    (v,) = lm_plant.plant(w, oracle, q, [(2 * CH + 40, 0, 11.0)], K)
    assert 10.5 < v < 11.5
    kw = dict(is_cyr=is_cyr, is_cjk=is_cjk, cyr_rows=ext, has_cyr=True)
    bv, bi, n, act, stp, hc, hj = oracle.lm_head_scan_script(q, w, TYPE_Q6_K, V, K, CH, lm_plant.CHUNK_THRESH,
                                                             batch1=True, **kw)
    assert (n, stp, int(bi[0])) == (1, 1, 2 * CH + 40) and bv[0] == np.float32(v)
    # the batched rule wants 11.5 for an in-script token: the scan goes on to chunk 4 (10.5)
    bv, bi, n, act, stp, hc, hj = oracle.lm_head_scan_script(q, w, TYPE_Q6_K, V, K, CH, lm_plant.CHUNK_THRESH, **kw)
    assert (n, stp, int(bi[0])) == (5, 1, 2 * CH + 40)


def test_script_rows_then_pruning(oracle):
    M = 3
    w, q = _scan_setup(oracle, M, 914)
    ext = [3 * CH + 100]
    is_cyr, is_cjk = _tables(rows_cyr=ext + [600])
    draft = np.array([0, 600, 601], np.uint32)
    # token 0: candidate 600 (Cyrillic, logit 9 in chunk 0: sets the flag, best == candidate, no pruning
    # after chunk 0); the extended row gives it 12 on another row -> pruned to 1 active position, and
    # 12 >= 11.5 on a Cyrillic token ends the scan; tokens 1, 2 keep their chunk-0 bests
    plan = [(600, 0, 9.0), (3 * CH + 100, 0, 12.0), (601, 1, 2.0), (CH + 50, 2, 13.0)]
    lm_plant.plant(w, oracle, q, plan, K)
    bv, bi, n, act, stp, hc, hj = oracle.lm_head_scan_script(q, w, TYPE_Q6_K, V, K, CH, lm_plant.CHUNK_THRESH,
                                                             draft_ids=draft, is_cyr=is_cyr, is_cjk=is_cjk,
                                                             cyr_rows=ext)
    assert (n, stp, act, int(bi[0]), hc) == (1, 1, 1, 3 * CH + 100, True)
    assert int(bi[2]) != CH + 50  # chunk 1 was never scanned
