"""The LM-head epilogue on the HIP path: chunked running argmax over fp16
logits and indexed-row evaluation, bit-exact against the oracle (values,
ids and logits), including planted ties across and inside chunks."""
import numpy as np
import pytest

import synth
from gpu_util import check_outputs, say
from oracle import TYPE_Q4_K, TYPE_Q6_K

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
    ctx.eval_rows_argmax(qb, None, M, K, wb, TYPE_Q6_K, idb, len(ids), vb, bv, bi)
    ctx.sync()
    vals, ev, ei = oracle.eval_rows_argmax(q, w, TYPE_Q6_K, K, ids, np.full(M, -1e30, np.float32),
                                           np.zeros(M, np.uint32))
    check_outputs(ctx.d2h(vb, np.float32, (M, len(ids))), vals, "indexed rows")
    assert np.array_equal(ctx.d2h(bv, np.float32, (M,)).view(np.uint32), ev.view(np.uint32))
    assert np.array_equal(ctx.d2h(bi, np.uint32, (M,)), ei)
    for b in (wb, idb, vb, bv, bi, qb):
        ctx.free(b)


@pytest.mark.parametrize("type_id", [TYPE_Q6_K, TYPE_Q4_K])
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
    ctx.eval_rows_argmax(qb, None, 1, K, wb, TYPE_Q6_K, idb, len(ids), None, bv, bi)
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
