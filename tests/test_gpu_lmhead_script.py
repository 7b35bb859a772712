"""The LM-head scan's script-gated exit, expressed with the library's calls
as the engine would: chunk 0 alone (its checkpoint held back), the session
flags from the best tokens on the host, the extended-script rows for the
active positions plus the pruning (a resumed call with no chunks), the
script test and chunk 0's checkpoint on the host, then the remaining chunks
(a resumed call) — compared bit for bit with the oracle's restatement of the
reference's loop (E:9690-9745 at batch 1, E:11107-11262 batched), on
planted logits whose outcome the oracle tests fix."""
import numpy as np
import pytest

import lm_plant
import synth
from gpu_util import say
from oracle import TYPE_Q6_K

pytestmark = pytest.mark.gpu

V, CH, K = 20000, 4096, 2560  # 5 chunks, the last 3616 rows
T = lm_plant.CHUNK_THRESH


def engine_scan(ctx, qb, M, wb, pre, draft, is_cyr, is_cjk, cyr_rows, cjk_rows, has_cyr, has_cjk,
                require_full=False, batch1=False, per_chunk=False):
    """The engine's scan through qmm_lm_head_scan: (best_val, best_id,
    chunks, active, stopped, has_cyr, has_cjk). per_chunk: every chunk after
    chunk 0 in a call of its own, so the session flags see each chunk's best
    tokens (as the engine sets them); else chunks 1.. in one call."""
    fc = 6 if require_full else 0
    bv, bi, st = ctx.malloc(M * 4), ctx.malloc(M * 4), ctx.upload(np.full(4, -7, np.int32))
    preb = ctx.upload(np.asarray(pre, np.uint32)) if pre else None
    drb = ctx.upload(np.asarray(draft, np.uint32)) if draft is not None else None
    bufs = [bv, bi, st, preb, drb]
    common = dict(best_val=bv, best_id=bi, scan_state=st, draft_ids=drb)

    def read():
        ctx.sync()
        return ctx.d2h(bv, np.float32, (M,)), ctx.d2h(bi, np.uint32, (M,)), ctx.d2h(st, np.int32, (4,))

    def flags(ids, n):
        nonlocal has_cyr, has_cjk
        for p in range(n):
            t = int(ids[p])
            has_cyr |= t < V and bool(is_cyr[t])
            has_cjk |= t < V and bool(is_cjk[t])

    # chunk 0 (every position active), its checkpoint held back
    ctx.lm_head_scan(qb, None, M, K, wb, TYPE_Q6_K, V, CH, thresholds=T, first_checkpoint=max(fc, 1), pre_ids=preb,
                     n_pre=len(pre) if pre else 0, chunk_end=1, **common)
    v, i, s = read()
    flags(i, M)
    host_stop = False
    if has_cyr or has_cjk:  # the extended rows of the active scripts, then the pruning
        ext = (list(cyr_rows) if has_cyr else []) + (list(cjk_rows) if has_cjk else [])
        extb = ctx.upload(np.asarray(ext, np.uint32))
        bufs.append(extb)
        ctx.lm_head_scan(qb, None, M, K, wb, TYPE_Q6_K, V, CH, thresholds=T, first_checkpoint=fc, pre_ids=extb,
                         n_pre=len(ext), chunk_begin=1, chunk_end=1, resume=True, **common)
        v, i, s = read()
        act = int(s[1])
        if batch1:
            ok = v[0] >= np.float32(10.5)
        else:
            def in_script(t):
                return t < V and ((has_cyr and is_cyr[t]) or (has_cjk and is_cjk[t]))
            ok = all(v[p] >= np.float32(11.5 if in_script(int(i[p])) else 20.0) for p in range(act))
        host_stop = not require_full and ok
    if not host_stop and not require_full:  # chunk 0's checkpoint
        host_stop = all(v[p] >= np.float32(T[0]) for p in range(int(s[1])))
    if host_stop:
        out = (v, i, 1, int(s[1]), 1)
    else:
        ends = [(c, c + 1) for c in range(1, (V + CH - 1) // CH)] if per_chunk else [(1, 0)]
        for cb, ce in ends:
            before = int(s[1])
            ctx.lm_head_scan(qb, None, M, K, wb, TYPE_Q6_K, V, CH, thresholds=T, first_checkpoint=fc, chunk_begin=cb,
                             chunk_end=ce, resume=True, **common)
            v, i, s = read()
            if per_chunk and int(s[0]) == ce:  # (a stopped scan read nothing more)
                flags(i, before)
            if s[2]:
                break
        if not per_chunk:
            flags(i, int(s[1]))
        out = (v, i, int(s[0]), int(s[1]), int(s[2]))
    for b in bufs:
        if b is not None:
            ctx.free(b)
    return out + (has_cyr, has_cjk)


def _case(ctx, oracle, M, seed, plan, ext_cyr=(), ext_cjk=(), tok_cyr=(), tok_cjk=(), has_cyr=False, has_cjk=False,
          pre=None, draft=None, require_full=False, batch1=False, want=None):
    w = lm_plant.base_tensor(V + 16, K, seed)
    x = synth.activations(M, K, seed=seed + 1)
    q = oracle.quantize_q8k(x)
    lm_plant.plant(w, oracle, q, plan, K)
    is_cyr, is_cjk = np.zeros(V, np.uint8), np.zeros(V, np.uint8)
    is_cyr[list(ext_cyr) + list(tok_cyr)] = 1
    is_cjk[list(ext_cjk) + list(tok_cjk)] = 1
    exp = oracle.lm_head_scan_script(q, w, TYPE_Q6_K, V, K, CH, T, pre_ids=pre, draft_ids=draft, is_cyr=is_cyr,
                                     is_cjk=is_cjk, cyr_rows=list(ext_cyr), cjk_rows=list(ext_cjk), has_cyr=has_cyr,
                                     has_cjk=has_cjk, require_full=require_full, batch1=batch1)
    if want is not None:  # the plan's outcome, on the oracle: (chunks, active, stopped, best id of token 0)
        assert (exp[2], exp[3], exp[4], int(exp[1][0])) == want, exp
    qb = ctx.malloc(ctx.lib.qmm_q8k_bytes(M, K))
    ctx.write_q8k(qb, *q, x16=oracle.f32_to_fp16(x))
    wb = ctx.weight_upload(w, TYPE_Q6_K, V + 16, K)
    for per_chunk in (False, True):
        got = engine_scan(ctx, qb, M, wb, pre, draft, is_cyr, is_cjk, ext_cyr, ext_cjk, has_cyr, has_cjk,
                          require_full, batch1, per_chunk)
        assert np.array_equal(got[0].view(np.uint32), exp[0].view(np.uint32)), (per_chunk, got[0], exp[0])
        assert np.array_equal(got[1], exp[1]), (per_chunk, got[1], exp[1])
        assert got[2:5] == exp[2:5], (per_chunk, got[2:5], exp[2:5])
        if per_chunk or exp[4] and exp[2] == 1:  # every flag (after chunk 0 only, in the one-call form)
            assert got[5:] == exp[5:], (per_chunk, got[5:], exp[5:])
    ctx.free(qb)
    ctx.free(wb)


@pytest.mark.parametrize("batch1", [False, True])
def test_script_exit_after_chunk0(ctx, oracle, batch1):
    say(f"lm scan script exit after chunk 0, batch1={batch1}")
    ext = [3 * CH + 5, 3 * CH + 6]
    # a Cyrillic session: the extended rows give 12 on a Cyrillic token -> the scan ends after chunk 0
    _case(ctx, oracle, 1, 1001, [(3 * CH + 6, 0, 12.0)], ext_cyr=ext, has_cyr=True, batch1=batch1,
          want=(1, 1, 1, 3 * CH + 6))
    # 11: enough for the batch-1 rule (10.5), not for the batched one (11.5): chunk 3's 11.5 is not met
    # either, chunk 4's 10.5 is
    _case(ctx, oracle, 1, 1002, [(3 * CH + 6, 0, 11.0)], ext_cyr=ext, has_cyr=True, batch1=batch1,
          want=(1, 1, 1, 3 * CH + 6) if batch1 else (5, 1, 1, 3 * CH + 6))


def test_script_flag_from_chunk0_and_from_later_chunks(ctx, oracle):
    say("lm scan script flags")
    ext = [4 * CH + 1]
    # chunk 0's best (row 900, 15) is a CJK token: the flag is set, the extended rows run, 15 >= 11.5
    _case(ctx, oracle, 1, 1003, [(900, 0, 15.0), (4 * CH + 1, 0, 11.0)], ext_cjk=ext, tok_cjk=[900],
          want=(1, 1, 1, 900))
    # a Cyrillic best in chunk 2 (14 >= 13.5 stops there): the flag comes from a later chunk
    _case(ctx, oracle, 1, 1004, [(2 * CH + 7, 0, 14.0)], ext_cjk=ext, tok_cyr=[2 * CH + 7], want=(3, 1, 1, 2 * CH + 7))
    # no session script and none found: the plain scan
    _case(ctx, oracle, 1, 1005, [(900, 0, 15.0)], ext_cjk=ext, want=(3, 1, 1, 900))


def test_script_exit_batched_with_pruning(ctx, oracle):
    say("lm scan script rows then pruning M=3")
    ext = [3 * CH + 100]
    plan = [(600, 0, 9.0), (3 * CH + 100, 0, 12.0), (601, 1, 2.0), (CH + 50, 2, 13.0)]
    _case(ctx, oracle, 3, 1006, plan, ext_cyr=ext, tok_cyr=[600], draft=[0, 600, 601], pre=[V - 2],
          want=(1, 1, 1, 3 * CH + 100))
    # required full scan: the extended rows still run, no script exit, no checkpoint before chunk 6
    _case(ctx, oracle, 3, 1007, plan, ext_cyr=ext, tok_cyr=[600], draft=[0, 600, 601], require_full=True,
          want=(5, 1, 0, 3 * CH + 100))
