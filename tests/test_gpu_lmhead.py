"""The LM-head epilogue on the HIP path: chunked running argmax over fp16
logits and indexed-row evaluation, bit-exact against the oracle (values,
ids and logits), including planted ties across and inside chunks."""
import numpy as np
import pytest

import synth
from gpu_util import check_outputs, say
from oracle import TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K

pytestmark = pytest.mark.gpu


def _setup(ctx, oracle, type_id, N, K, M, seed):
    w = synth.weights(type_id, N, K, seed=seed)
    x = synth.activations(M, K, seed=seed + 1)
    q = oracle.quantize_q8k(x)
    qb = ctx.malloc(ctx.lib.qmm_q8k_bytes(M, K))
    ctx.write_q8k(qb, *q)
    return w, q, qb


@pytest.mark.parametrize("type_id,M", [(TYPE_Q6_K, 1), (TYPE_Q6_K, 3), (TYPE_Q4_K, 2)])
def test_lm_head_chunks(ctx, oracle, type_id, M):
    N, K = 20000, 2560
    say(f"lm head argmax type={type_id} M={M}")
    w, q, qb = _setup(ctx, oracle, type_id, N, K, M, seed=600 + M)
    rb = synth.row_bytes(type_id, K)
    # plant ties with the first maximum: copies of it later in its chunk and in a later chunk
    lg_all, _, _ = oracle.lm_head_argmax(q, w, type_id, N, 0, np.full(M, -1e30, np.float32), np.zeros(M, np.uint32))
    top = int(np.argmax(lg_all[0]))
    for dst in (top + 1 + (N - top - 2) // 3, N - 1):
        if dst != top:
            w[dst * rb:(dst + 1) * rb] = w[top * rb:(top + 1) * rb]
    wb = ctx.weight_upload(w, type_id, N, K)
    bv = ctx.upload(np.full(M, -1e30, np.float32))
    bi = ctx.upload(np.zeros(M, np.uint32))
    lgb = ctx.malloc(M * N * 4)
    ebv, ebi = np.full(M, -1e30, np.float32), np.zeros(M, np.uint32)
    chunks = [(0, 7000), (7000, 14500), (14500, N)]
    for r0, r1 in chunks:
        ctx.lm_head_argmax(qb, None, M, K, wb.ptr + r0 * rb, type_id, r1 - r0, r0,
                           lgb.ptr + 0, bv, bi) if r0 == 0 else \
            ctx.lm_head_argmax(qb, None, M, K, wb.ptr + r0 * rb, type_id, r1 - r0, r0, None, bv, bi)
        elg, ebv, ebi = oracle.lm_head_argmax(q, w[r0 * rb:r1 * rb], type_id, r1 - r0, r0, ebv, ebi)
        if r0 == 0:
            ctx.sync()
            check_outputs(ctx.d2h(lgb, np.float32, (M, r1 - r0)), elg, "chunk 0 logits")
    ctx.sync()
    got_v, got_i = ctx.d2h(bv, np.float32, (M,)), ctx.d2h(bi, np.uint32, (M,))
    assert np.array_equal(got_v.view(np.uint32), ebv.view(np.uint32)), (got_v, ebv)
    assert np.array_equal(got_i, ebi), (got_i, ebi)
    for b in (wb, bv, bi, lgb, qb):
        ctx.free(b)


@pytest.mark.parametrize("M", [1, 4])
def test_eval_rows(ctx, oracle, M):
    N, K = 3000, 2560
    say(f"eval rows M={M}")
    w, q, qb = _setup(ctx, oracle, TYPE_Q6_K, N, K, M, seed=700 + M)
    ids = np.random.default_rng(M).integers(0, N, 517).astype(np.uint32)
    ids[100] = ids[3]  # a duplicate: the earlier position keeps a tie
    wb = ctx.weight_upload(w, TYPE_Q6_K, N, K)
    idb = ctx.upload(ids)
    vb = ctx.malloc(M * len(ids) * 4)
    bv = ctx.upload(np.full(M, -1e30, np.float32))
    bi = ctx.upload(np.zeros(M, np.uint32))
    ctx.eval_rows_argmax(qb, None, M, K, wb, N, TYPE_Q6_K, idb, len(ids), vb, bv, bi)
    ctx.sync()
    vals, ev, ei = oracle.eval_rows_argmax(q, w, TYPE_Q6_K, K, ids, np.full(M, -1e30, np.float32),
                                           np.zeros(M, np.uint32))
    check_outputs(ctx.d2h(vb, np.float32, (M, len(ids))), vals, "indexed rows")
    assert np.array_equal(ctx.d2h(bv, np.float32, (M,)).view(np.uint32), ev.view(np.uint32))
    assert np.array_equal(ctx.d2h(bi, np.uint32, (M,)), ei)
    for b in (wb, idb, vb, bv, bi, qb):
        ctx.free(b)


@pytest.mark.parametrize("type_id", [TYPE_Q6_K, TYPE_Q4_K, TYPE_Q5_K])
def test_lm_head_tall_chunks(ctx, oracle, type_id):
    """One row, no logits requested, chunks tall enough for the persistent
    GEMV grid. Ties planted inside a chunk and across chunks (the earlier row
    must win)."""
    N, K = 60000, 2560
    say(f"tall lm head chunks type={type_id}")
    w, q, qb = _setup(ctx, oracle, type_id, N, K, 1, seed=650 + type_id)
    rb = synth.row_bytes(type_id, K)
    lg_all, _, _ = oracle.lm_head_argmax(q, w, type_id, N, 0, np.full(1, -1e30, np.float32), np.zeros(1, np.uint32))
    top = int(np.argmax(lg_all[0]))
    for dst in (min(top + 9001, N - 1), (top + 30011) % N):
        if dst != top:
            w[dst * rb:(dst + 1) * rb] = w[top * rb:(top + 1) * rb]
    wb = ctx.weight_upload(w, type_id, N, K)
    bv = ctx.upload(np.full(1, -1e30, np.float32))
    bi = ctx.upload(np.zeros(1, np.uint32))
    ebv, ebi = np.full(1, -1e30, np.float32), np.zeros(1, np.uint32)
    for r0, r1 in [(0, 25000), (25000, N)]:
        ctx.lm_head_argmax(qb, None, 1, K, wb.ptr + r0 * rb, type_id, r1 - r0, r0, None, bv, bi)
        _, ebv, ebi = oracle.lm_head_argmax(q, w[r0 * rb:r1 * rb], type_id, r1 - r0, r0, ebv, ebi)
    ctx.sync()
    got_v, got_i = ctx.d2h(bv, np.float32, (1,)), ctx.d2h(bi, np.uint32, (1,))
    assert np.array_equal(got_v.view(np.uint32), ebv.view(np.uint32)), (got_v, ebv)
    assert np.array_equal(got_i, ebi), (got_i, ebi)
    for b in (wb, bv, bi, qb):
        ctx.free(b)


def test_eval_rows_many(ctx, oracle):
    """9000 indexed rows at M = 1 without the values requested (list
    positions mapped to row ids, no fp16 rounding)."""
    N, K = 12000, 2560
    say("many eval rows")
    w, q, qb = _setup(ctx, oracle, TYPE_Q6_K, N, K, 1, seed=760)
    ids = np.random.default_rng(9).integers(0, N, 9000).astype(np.uint32)
    ids[7000] = ids[5]  # a duplicate: the earlier position keeps the tie
    wb = ctx.weight_upload(w, TYPE_Q6_K, N, K)
    idb = ctx.upload(ids)
    bv = ctx.upload(np.full(1, -1e30, np.float32))
    bi = ctx.upload(np.zeros(1, np.uint32))
    ctx.eval_rows_argmax(qb, None, 1, K, wb, N, TYPE_Q6_K, idb, len(ids), None, bv, bi)
    ctx.sync()
    _, ev, ei = oracle.eval_rows_argmax(q, w, TYPE_Q6_K, K, ids, np.full(1, -1e30, np.float32),
                                        np.zeros(1, np.uint32))
    assert np.array_equal(ctx.d2h(bv, np.float32, (1,)).view(np.uint32), ev.view(np.uint32))
    assert np.array_equal(ctx.d2h(bi, np.uint32, (1,)), ei)
    for b in (wb, idb, bv, bi, qb):
        ctx.free(b)


def test_lm_head_nan_row(ctx, oracle):
    """A row whose logit is NaN (a NaN scale in its first Q6_K block: d at
    byte 208) at the position of the maximum, in a chunk tall enough for the
    GEMV's fused argmax: never taken, as under the reference's strict `>`."""
    N, K = 30000, 2560
    say("lm head NaN row")
    w, q, qb = _setup(ctx, oracle, TYPE_Q6_K, N, K, 1, seed=680)
    rb = synth.row_bytes(TYPE_Q6_K, K)
    lg_all, _, _ = oracle.lm_head_argmax(q, w, TYPE_Q6_K, N, 0, np.full(1, -1e30, np.float32), np.zeros(1, np.uint32))
    top = int(np.argmax(lg_all[0]))
    w[top * rb + 208:top * rb + 210] = [0x00, 0x7E]  # fp16 NaN
    wb = ctx.weight_upload(w, TYPE_Q6_K, N, K)
    bv = ctx.upload(np.full(1, -1e30, np.float32))
    bi = ctx.upload(np.zeros(1, np.uint32))
    ctx.lm_head_argmax(qb, None, 1, K, wb, TYPE_Q6_K, N, 0, None, bv, bi)
    ctx.sync()
    lg, ebv, ebi = oracle.lm_head_argmax(q, w, TYPE_Q6_K, N, 0, np.full(1, -1e30, np.float32), np.zeros(1, np.uint32))
    assert np.isnan(lg[0, top]) and ebi[0] != top
    got_v, got_i = ctx.d2h(bv, np.float32, (1,)), ctx.d2h(bi, np.uint32, (1,))
    assert np.array_equal(got_v.view(np.uint32), ebv.view(np.uint32)), (got_v, ebv)
    assert np.array_equal(got_i, ebi), (got_i, ebi)
    for b in (wb, bv, bi, qb):
        ctx.free(b)


def test_eval_rows_past_the_tensor(ctx, oracle):
    """Ids at or past tensor_rows are never read and count as -1e30 (E:11150):
    the tensor is uploaded with 16 more rows than tensor_rows says, so the
    ids past the bound still lie inside the allocation."""
    N, K, M = 3000, 2560, 2
    say("eval rows past the tensor")
    w, q, qb = _setup(ctx, oracle, TYPE_Q6_K, N + 16, K, M, seed=770)
    ids = np.array([5, N + 3, 17, N, N + 15, 9], np.uint32)
    wb = ctx.weight_upload(w, TYPE_Q6_K, N + 16, K)
    idb = ctx.upload(ids)
    vb = ctx.malloc(M * len(ids) * 4)
    for seed_v, label in ((-1e30, "seed -1e30"), (-np.inf, "seed -inf")):
        bv = ctx.upload(np.full(M, seed_v, np.float32))
        bi = ctx.upload(np.full(M, 123, np.uint32))
        ctx.eval_rows_argmax(qb, None, M, K, wb, N, TYPE_Q6_K, idb, len(ids), vb, bv, bi)
        ctx.sync()
        vals = ctx.d2h(vb, np.float32, (M, len(ids)))
        inb = [i for i, r in enumerate(ids) if r < N]
        exp_vals, ev, ei = oracle.eval_rows_argmax(q, w, TYPE_Q6_K, K, ids[inb], np.full(M, seed_v, np.float32),
                                                   np.full(M, 123, np.uint32))
        assert np.array_equal(vals[:, inb].view(np.uint32), exp_vals.view(np.uint32)), label
        assert np.all(vals[:, [1, 3, 4]] == np.float32(-1e30)), label
        got_v, got_i = ctx.d2h(bv, np.float32, (M,)), ctx.d2h(bi, np.uint32, (M,))
        assert np.array_equal(got_v.view(np.uint32), ev.view(np.uint32)), label
        assert np.array_equal(got_i, ei), label
        ctx.free(bv)
        ctx.free(bi)
    for b in (wb, idb, vb, qb):
        ctx.free(b)


# ------------------------------------------------- the chunked vocabulary scan
import lm_plant  # noqa: E402

V, CH = 20000, 4096  # 5 chunks


def _scan(ctx, oracle, M, seed, plan, thresholds, first_checkpoint=0, pre=None, draft=None, V=V, CH=CH):
    K = 2560
    w = lm_plant.base_tensor(V + 16, K, seed)
    x = synth.activations(M, K, seed=seed + 1)
    q = oracle.quantize_q8k(x)
    lm_plant.plant(w, oracle, q, plan, K)
    qb = ctx.malloc(ctx.lib.qmm_q8k_bytes(M, K))
    ctx.write_q8k(qb, *q, x16=oracle.f32_to_fp16(x))
    wb = ctx.weight_upload(w, TYPE_Q6_K, V + 16, K)
    bv, bi = ctx.malloc(M * 4), ctx.malloc(M * 4)
    st = ctx.upload(np.full(4, -7, np.int32))
    preb = ctx.upload(np.asarray(pre, np.uint32)) if pre is not None else None
    drb = ctx.upload(np.asarray(draft, np.uint32)) if draft is not None else None
    ctx.lm_head_scan(qb, None, M, K, wb, TYPE_Q6_K, V, CH, thresholds=thresholds, first_checkpoint=first_checkpoint,
                     pre_ids=preb, n_pre=0 if pre is None else len(pre), draft_ids=drb, best_val=bv, best_id=bi,
                     scan_state=st)
    ctx.sync()
    got = (ctx.d2h(bv, np.float32, (M,)), ctx.d2h(bi, np.uint32, (M,)), ctx.d2h(st, np.int32, (4,)))
    exp = oracle.lm_head_scan(q, w, TYPE_Q6_K, V, K, CH, thresholds, first_checkpoint, 1e-3, pre, draft)
    for b in (qb, wb, bv, bi, st, preb, drb):
        if b is not None:
            ctx.free(b)
    return got, exp


def _same(got, exp, want_chunks, want_active, want_stopped):
    (gv, gi, st), (ev, ei, n, act, stp) = got, exp
    assert (n, act, stp) == (want_chunks, want_active, want_stopped)  # the plan's outcome, on the oracle
    assert np.array_equal(gv.view(np.uint32), ev.view(np.uint32)), (gv, ev)
    assert np.array_equal(gi, ei), (gi, ei)
    assert list(st) == [n, act, stp, 0], st


@pytest.mark.parametrize("M", [1, 3])
def test_scan_early_exit(ctx, oracle, M):
    say(f"lm scan early exit M={M}")
    T = lm_plant.CHUNK_THRESH
    # every token above 19.5 in chunk 0: one chunk read
    plan0 = [(5 + 11 * p, p, 25.0) for p in range(M)]
    _same(*_scan(ctx, oracle, M, 910 + M, plan0, T), 1, M, 1)
    # 14 in chunk 2 for every token: three chunks
    plan2 = [(2 * CH + 77 + p, p, 14.0) for p in range(M)]
    _same(*_scan(ctx, oracle, M, 920 + M, plan2, T), 3, M, 1)
    # checkpoints from chunk 3 only: four chunks
    _same(*_scan(ctx, oracle, M, 930 + M, plan0, T, first_checkpoint=3), 4, M, 1)
    # no thresholds: all five chunks (the last one partial)
    _same(*_scan(ctx, oracle, M, 940 + M, plan0, None), 5, M, 0)


def test_scan_one_token_short_of_the_threshold(ctx, oracle):
    """Two tokens above 19.5 in chunk 0, the third only at 17: not all above,
    so chunk 0 does not end the scan; chunk 1's 16 does."""
    say("lm scan one token short")
    plan = [(5, 0, 25.0), (16, 1, 25.0), (27, 2, 17.0)]
    _same(*_scan(ctx, oracle, 3, 950, plan, lm_plant.CHUNK_THRESH), 2, 3, 1)


@pytest.mark.parametrize("M", [3, 4])
def test_scan_candidates_and_pruning(ctx, oracle, M):
    say(f"lm scan pruning M={M}")
    draft = [0, 100, 200, 300][:M]
    # token 0: its candidate (100) at 5, row 1500 (chunk 0) at 8: the active batch ends at 1 after chunk 0;
    # the other tokens' chunk-1 rows at 12 are never seen
    plan = [(100, 0, 5.0), (1500, 0, 8.0)] + [(CH + 10 * p, p, 12.0) for p in range(1, M)]
    got, exp = _scan(ctx, oracle, M, 960 + M, plan, None, draft=draft)
    _same(got, exp, 5, 1, 0)
    assert int(got[1][0]) == 1500
    # pre-evaluated end-of-text rows (fp32), and a candidate past the vocabulary (never read)
    draft2 = [0, V + 7] + [400 + p for p in range(2, M)]
    plan2 = [(V - 4, 0, 30.0), (CH + 10, 1, 12.0)]
    got, exp = _scan(ctx, oracle, M, 970 + M, plan2, lm_plant.CHUNK_THRESH, pre=[V - 2, V - 4], draft=draft2)
    assert int(got[1][0]) == V - 4
    (ev, ei, n, act, stp) = exp
    _same(got, exp, n, act, stp)


def test_scan_stopped_chunks_read_no_weights(ctx, oracle):
    """After a stop, the later chunks' launches return before touching their
    rows: rows of chunks 1..4 that would hold every maximum change nothing."""
    say("lm scan stop skips chunks")
    plan = [(5, 0, 25.0), (CH + 1, 0, 60.0), (3 * CH + 2, 0, 70.0)]
    got, exp = _scan(ctx, oracle, 1, 980, plan, lm_plant.CHUNK_THRESH)
    _same(got, exp, 1, 1, 1)
    assert int(got[1][0]) == 5


@pytest.mark.parametrize("case", ["chunk0", "chunk2", "checkpoint3", "all"])
def test_scan_tall_chunks_batch1(ctx, oracle, case):
    """Batch-1 chunks tall enough for the persistent GEMV (12288 rows): each
    chunk's step is applied by the next chunk's launch (or, for the last, by a
    launch of its own), and a step that stops the scan ends that launch before
    it requests weights."""
    V2, CH2 = 60000, 12288  # 5 chunks, the last 10848 rows
    T = lm_plant.CHUNK_THRESH
    say(f"lm scan tall chunks {case}")
    plan0 = [(5, 0, 25.0), (CH2 + 3, 0, 60.0)]  # a larger row in chunk 1 must not be seen after a stop at chunk 0
    if case == "chunk0":
        _same(*_scan(ctx, oracle, 1, 990, plan0, T, V=V2, CH=CH2), 1, 1, 1)
    elif case == "chunk2":
        _same(*_scan(ctx, oracle, 1, 991, [(2 * CH2 + 77, 0, 14.0)], T, V=V2, CH=CH2), 3, 1, 1)
    elif case == "checkpoint3":
        _same(*_scan(ctx, oracle, 1, 992, plan0, T, first_checkpoint=3, V=V2, CH=CH2), 4, 1, 1)
    else:
        got, exp = _scan(ctx, oracle, 1, 993, [(4 * CH2 + 9, 0, 40.0)], None, V=V2, CH=CH2)
        _same(got, exp, 5, 1, 0)
        assert int(got[1][0]) == 4 * CH2 + 9


# ------------------------------------------- the scan behind the final norm
def _scan_rmsnorm(ctx, oracle, M, seed, plan, thresholds, first_checkpoint=0, pre=None, draft=None, V=V, CH=CH):
    """qmm_lm_head_scan_rmsnorm against qmm_rmsnorm_q8k followed by
    qmm_lm_head_scan on its output: (best, id, state) bit-identical, and the
    two-step result against the oracle's scan of that Q8_K row. The plan's
    rows are planted against the normed row."""
    K = 2560
    x = synth.activations(M, K, seed=seed + 1)
    gamma = np.random.default_rng(seed + 2).uniform(0.5, 1.5, K).astype(np.float32)
    xb, gb = ctx.upload(x), ctx.upload(gamma)
    qb = ctx.malloc(ctx.lib.qmm_q8k_bytes(M, K))
    ctx.rmsnorm_q8k(xb, gb, M, K, None, qb)
    ctx.sync()
    q = ctx.read_q8k(qb, M, K)
    w = lm_plant.base_tensor(V + 16, K, seed)
    lm_plant.plant(w, oracle, q, plan, K)
    wb = ctx.weight_upload(w, TYPE_Q6_K, V + 16, K)
    preb = ctx.upload(np.asarray(pre, np.uint32)) if pre is not None else None
    drb = ctx.upload(np.asarray(draft, np.uint32)) if draft is not None else None
    runs = []
    for fused in (False, True):
        bv, bi = ctx.malloc(M * 4), ctx.malloc(M * 4)
        st = ctx.upload(np.full(4, -7, np.int32))
        kw = dict(thresholds=thresholds, first_checkpoint=first_checkpoint, pre_ids=preb,
                  n_pre=0 if pre is None else len(pre), draft_ids=drb, best_val=bv, best_id=bi, scan_state=st)
        if fused:
            ctx.lm_head_scan_rmsnorm(xb, gb, M, K, wb, TYPE_Q6_K, V, CH, **kw)
        else:
            ctx.lm_head_scan(qb, None, M, K, wb, TYPE_Q6_K, V, CH, **kw)
        ctx.sync()
        runs.append((ctx.d2h(bv, np.float32, (M,)), ctx.d2h(bi, np.uint32, (M,)), ctx.d2h(st, np.int32, (4,))))
        for b in (bv, bi, st):
            ctx.free(b)
    exp = oracle.lm_head_scan(q, w, TYPE_Q6_K, V, K, CH, thresholds, first_checkpoint, 1e-3, pre, draft)
    for b in (xb, gb, qb, wb, preb, drb):
        if b is not None:
            ctx.free(b)
    (sv, si, ss), (fv, fi, fs) = runs
    assert np.array_equal(sv.view(np.uint32), fv.view(np.uint32)), (sv, fv)
    assert np.array_equal(si, fi), (si, fi)
    assert np.array_equal(ss, fs), (ss, fs)
    return runs[0], exp


@pytest.mark.parametrize("case", ["chunk0", "chunk2", "checkpoint3", "all", "short_tail", "small_chunks",
                                  "pre_ids", "drafts"])
def test_scan_rmsnorm(ctx, oracle, case):
    """The scan behind its final norm in one call. Batch-1 cases without
    pre-evaluated rows take the norm inside every chunk launch's fill (tall
    chunks, a last chunk of 2944 rows, chunks of 4096 rows); pre-evaluated
    rows and drafts take the norm's own launch first."""
    T = lm_plant.CHUNK_THRESH
    V2, CH2 = 60000, 12288
    say(f"lm scan behind the final norm: {case}")
    if case == "chunk0":
        got, exp = _scan_rmsnorm(ctx, oracle, 1, 1010, [(5, 0, 25.0), (CH2 + 3, 0, 60.0)], T, V=V2, CH=CH2)
        _same(got, exp, 1, 1, 1)
    elif case == "chunk2":
        _same(*_scan_rmsnorm(ctx, oracle, 1, 1011, [(2 * CH2 + 77, 0, 14.0)], T, V=V2, CH=CH2), 3, 1, 1)
    elif case == "checkpoint3":
        got, exp = _scan_rmsnorm(ctx, oracle, 1, 1012, [(5, 0, 25.0)], T, first_checkpoint=3, V=V2, CH=CH2)
        _same(got, exp, 4, 1, 1)
    elif case == "all":
        got, exp = _scan_rmsnorm(ctx, oracle, 1, 1013, [(4 * CH2 + 9, 0, 40.0)], None, V=V2, CH=CH2)
        _same(got, exp, 5, 1, 0)
        assert int(got[1][0]) == 4 * CH2 + 9
    elif case == "short_tail":  # chunk 4 holds 2944 rows, its maximum the last row
        V3 = 4 * CH2 + 2944
        got, exp = _scan_rmsnorm(ctx, oracle, 1, 1014, [(V3 - 1, 0, 9.0)], [30.0] * 4 + [-1e30], V=V3, CH=CH2)
        _same(got, exp, 5, 1, 1)
        assert int(got[1][0]) == V3 - 1
    elif case == "small_chunks":
        _same(*_scan_rmsnorm(ctx, oracle, 1, 1015, [(2 * CH + 77, 0, 14.0)], T), 3, 1, 1)
    elif case == "pre_ids":
        got, exp = _scan_rmsnorm(ctx, oracle, 1, 1016, [(V - 4, 0, 30.0)], T, pre=[V - 2, V - 4])
        assert int(got[1][0]) == V - 4
        _same(got, exp, *exp[2:])
    else:
        M = 3
        plan = [(100, 0, 5.0), (1500, 0, 8.0)] + [(CH + 10 * p, p, 12.0) for p in range(1, M)]
        got, exp = _scan_rmsnorm(ctx, oracle, M, 1017, plan, None, draft=[0, 100, 200])
        _same(got, exp, 5, 1, 0)


def test_scan_in_a_row(ctx, oracle):
    """Batch-1 scans in a row on one context, each the oracle's: a stop after
    chunk 0 (the later launches find the state stopped), all chunks, a stop
    after chunk 2, a checkpoint at every chunk that none meets, chunks of
    4095 and of 1024 rows (20 chunks), and a stop after chunk 0 again: every
    scan seeds its own state, whatever the previous one left."""
    T = lm_plant.CHUNK_THRESH
    V2, CH2 = 60000, 12288
    say("lm scan, scans in a row")
    _same(*_scan(ctx, oracle, 1, 1020, [(5, 0, 25.0), (CH2 + 3, 0, 60.0)], T, V=V2, CH=CH2), 1, 1, 1)
    got, exp = _scan(ctx, oracle, 1, 1021, [(4 * CH2 + 9, 0, 40.0)], None, V=V2, CH=CH2)
    _same(got, exp, 5, 1, 0)
    _same(*_scan(ctx, oracle, 1, 1022, [(2 * CH2 + 77, 0, 14.0)], T, V=V2, CH=CH2), 3, 1, 1)
    got, exp = _scan(ctx, oracle, 1, 1023, [(3 * CH2 + 1, 0, 25.0)], [1e30] * 5, V=V2, CH=CH2)
    _same(got, exp, 5, 1, 0)  # a checkpoint at every chunk, never met
    assert int(got[1][0]) == 3 * CH2 + 1
    _same(*_scan(ctx, oracle, 1, 1024, [(2 * 4095 + 7, 0, 14.0)], T, CH=4095), 3, 1, 1)
    _same(*_scan(ctx, oracle, 1, 1025, [(2 * 1024 + 5, 0, 14.0)], T, CH=1024), 3, 1, 1)
    _same(*_scan(ctx, oracle, 1, 1026, [(5, 0, 25.0)], T, V=V2, CH=CH2), 1, 1, 1)


def test_scan_full_vocabulary_one_launch(ctx, oracle):
    """The engine's LM head at batch 1: 151936 Q6_K rows of K = 2560 in
    chunks of 24832 with chunk_thresh at every chunk (the scan's one launch
    and its final step). A stop after chunk 0 (a larger row in chunk 1 must
    not be taken), after chunk 3 (a row at 12 clears its 11.5), and all
    seven chunks with no threshold met, each against the oracle; the three
    twice on one context (the fold's state is cleared by every scan's last
    step)."""
    Vf, CHf, Kf = 151936, 24832, 2560
    say("lm scan full vocabulary, one launch")
    w0 = lm_plant.base_tensor(Vf, Kf, 1030)
    x = synth.activations(1, Kf, seed=1031)
    q = oracle.quantize_q8k(x)
    qb = ctx.malloc(ctx.lib.qmm_q8k_bytes(1, Kf))
    ctx.write_q8k(qb, *q, x16=oracle.f32_to_fp16(x))
    wb = ctx.malloc(w0.nbytes)
    bv, bi, st = ctx.malloc(4), ctx.malloc(4), ctx.upload(np.full(4, -7, np.int32))
    cases = [("chunk0", [(77, 0, 25.0), (CHf + 5, 0, 60.0)], (1, 1, 1), 77),
             ("chunk3", [(3 * CHf + 11, 0, 12.0)], (4, 1, 1), 3 * CHf + 11),
             ("never", [(6 * CHf + 2, 0, 9.0)], (7, 1, 0), 6 * CHf + 2)]
    for rnd in range(2):
        for name, plan, want, row in cases:
            w = w0.copy()
            lm_plant.plant(w, oracle, q, plan, Kf)
            ctx.h2d(wb, w)
            ctx.lm_head_scan(qb, None, 1, Kf, wb, TYPE_Q6_K, Vf, CHf, thresholds=lm_plant.CHUNK_THRESH, best_val=bv,
                             best_id=bi, scan_state=st)
            ctx.sync()
            got = (ctx.d2h(bv, np.float32, (1,)), ctx.d2h(bi, np.uint32, (1,)), ctx.d2h(st, np.int32, (4,)))
            say(f"  round {rnd} {name}: state {list(got[2])}, best {int(got[1][0])}")
            exp = oracle.lm_head_scan(q, w, TYPE_Q6_K, Vf, Kf, CHf, lm_plant.CHUNK_THRESH)
            _same(got, exp, *want)
            assert int(got[1][0]) == row
    for b in (qb, wb, bv, bi, st):
        ctx.free(b)
