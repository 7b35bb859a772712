"""F32 / F16 weight rows (sdot_row_f32_batch / _f16_batch, E:3410-3440) and
task groups of several types in one dispatch (the engine's {qkv, gate,
alpha, beta} and {q, k, v} groups, E:7954-7959, E:8110-8114) on the HIP
path, through the C ABI, against the oracle. K-quant outputs must be
bit-exact; F32 / F16 outputs are summed in another order than the
reference's row loop and are held to the stated tolerance."""
import numpy as np
import pytest

import qmm_hip
import synth
from gpu_util import TOL, check_outputs, norm_err, say
from oracle import TYPE_F16, TYPE_F32, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0

pytestmark = pytest.mark.gpu


def _weights(type_id, rows, K, seed):
    if type_id == TYPE_F32:
        return (synth.activations(rows, K, seed=seed) * np.float32(0.05)).view(np.uint8).reshape(-1)
    if type_id == TYPE_F16:
        return (synth.activations(rows, K, seed=seed) * np.float32(0.05)).astype(np.float16).view(np.uint8).reshape(-1)
    return synth.weights(type_id, rows, K, seed=seed)


def _run_group(ctx, oracle, specs, M, K, seed, prequantized=False, residual_on=None):
    """specs: list of (type, rows). One dispatch of all tasks; returns
    [(type, got, expected)] per task."""
    x = synth.activations(M, K, seed=seed)
    ws = [_weights(t, n, K, seed + 10 + i) for i, (t, n) in enumerate(specs)]
    bufs, tasks, otasks = [], [], []
    for i, ((t, n), w) in enumerate(zip(specs, ws)):
        wb = ctx.weight_upload(w, t, n, K)
        yb = ctx.malloc(M * n * 4)
        res = None
        if residual_on == i:
            res = synth.activations(M, n, seed=seed + 99)
            rb = ctx.upload(res)
            bufs.append(rb)
        else:
            rb = None
        bufs += [wb, yb]
        tasks.append(qmm_hip.MatrixTask(wb, t, n, K, yb, n, rb, n))
        od = dict(w=w, type=t, rows=n)
        if res is not None:
            od["residual"] = res
        otasks.append(od)
    xb = ctx.upload(x)
    bufs.append(xb)
    if prequantized:
        need_q80 = any(t == TYPE_Q8_0 for t, _ in specs)
        q = oracle.quantize_q8k(x)
        qb = ctx.malloc(ctx.lib.qmm_q8k_bytes(M, K))
        ctx.write_q8k(qb, *q, x16=oracle.f32_to_fp16(x))
        bufs.append(qb)
        zb = None
        if need_q80:
            z = oracle.quantize_q8_0(x)
            zb = ctx.malloc(ctx.lib.qmm_q8_0_bytes(M, K))
            ctx.write_q80(zb, z[0], z[1])
            bufs.append(zb)
        ctx.gemm_multi_dispatch_prequantized(qb, zb, M, K, tasks)
    else:
        ctx.gemm_multi_dispatch(xb, M, K, tasks)
    ctx.sync()
    got = [ctx.d2h(t.dst, np.float32, (M, t.rows)) for t in tasks]
    exp = oracle.gemm_multi(x, otasks, prequantized=(oracle.quantize_q8k(x), oracle.quantize_q8_0(x))
                            if prequantized else None)
    for b in bufs:
        ctx.free(b)
    return [(t, g, e) for (t, _), g, e in zip(specs, got, exp)]


def _check(results, what):
    for i, (t, g, e) in enumerate(results):
        name = f"{what} task {i} ({qmm_hip.TYPE_NAMES[t]})"
        if t in (TYPE_F32, TYPE_F16):
            err = norm_err(g, e)
            say(f"{name}: normalized max error {err:.2e}")
            assert err <= TOL, f"{name}: {err:.3e} > {TOL}"
        else:
            check_outputs(g, e, name)


@pytest.mark.parametrize("type_id", [TYPE_F32, TYPE_F16])
@pytest.mark.parametrize("M", [1, 8, 70])
@pytest.mark.parametrize("pre", [False, True])
def test_float_rows(ctx, oracle, type_id, M, pre):
    say(f"float rows type={type_id} M={M} prequantized={pre}")
    _check(_run_group(ctx, oracle, [(type_id, 97)], M, 2560, seed=300 + M + type_id, prequantized=pre),
           f"float M={M}")


@pytest.mark.parametrize("M", [1, 8])
def test_engine_linear_attention_group(ctx, oracle, M):
    """{qkv Q5_K 8192, gate Q4_K 4096, alpha F32 32, beta F32 32} x 2560,
    one dispatch (E:7954-7959)."""
    say(f"group qkv/gate/alpha/beta M={M}")
    specs = [(TYPE_Q5_K, 8192), (TYPE_Q4_K, 4096), (TYPE_F32, 32), (TYPE_F32, 32)]
    _check(_run_group(ctx, oracle, specs, M, 2560, seed=310 + M), f"lin-attn M={M}")


@pytest.mark.parametrize("M", [1, 8])
def test_engine_full_attention_group(ctx, oracle, M):
    """{q 8192, k 1024, v 1024} x 2560 of three types, one dispatch
    (E:8110-8114)."""
    say(f"group q/k/v M={M}")
    specs = [(TYPE_Q4_K, 8192), (TYPE_Q6_K, 1024), (TYPE_Q5_K, 1024)]
    _check(_run_group(ctx, oracle, specs, M, 2560, seed=320 + M), f"full-attn M={M}")


@pytest.mark.parametrize("M", [1, 2, 17, 40])
@pytest.mark.parametrize("pre", [False, True])
def test_mixed_groups_small(ctx, oracle, M, pre):
    """Every format in one group (Q8_0 joins the one-launch form at M = 1;
    from M = 2 it runs as a launch of its own), ragged row counts, a residual."""
    say(f"mixed small M={M} prequantized={pre}")
    specs = [(TYPE_Q6_K, 40), (TYPE_Q4_K, 33), (TYPE_F16, 17), (TYPE_Q5_K, 16), (TYPE_Q8_0, 9), (TYPE_F32, 3)]
    _check(_run_group(ctx, oracle, specs, M, 2560, seed=330 + M, prequantized=pre, residual_on=1), f"mixed M={M}")


def test_mixed_group_without_q8_0_at_m64(ctx, oracle):
    say("mixed M=64")
    specs = [(TYPE_Q4_K, 64), (TYPE_Q5_K, 48), (TYPE_Q6_K, 32), (TYPE_F16, 16)]
    _check(_run_group(ctx, oracle, specs, 64, 2560, seed=340), "mixed M=64")


def test_mixed_group_large_k(ctx, oracle):
    """K = 9728 (past the one-launch form's K at M >= 2): per-type launches."""
    say("mixed K=9728")
    specs = [(TYPE_Q6_K, 40), (TYPE_Q4_K, 24), (TYPE_F32, 8)]
    for M in (1, 5):
        _check(_run_group(ctx, oracle, specs, M, 9728, seed=350 + M), f"mixed K=9728 M={M}")


@pytest.mark.parametrize("specs,K,pre", [
    ([(TYPE_Q5_K, 8192), (TYPE_Q4_K, 4096), (TYPE_F32, 32), (TYPE_F32, 32)], 2560, True),
    ([(TYPE_Q5_K, 8192), (TYPE_F32, 32)], 2560, False),
    ([(TYPE_F16, 40), (TYPE_Q4_K, 8192), (TYPE_Q5_K, 2048), (TYPE_Q6_K, 1000)], 3072, False),
    ([(TYPE_Q6_K, 6144), (TYPE_Q4_K, 2048), (TYPE_Q5_K, 8)], 2560, True),
    ([(TYPE_Q5_K, 8192), (TYPE_Q4_K, 4096)], 2560, True),
    ([(TYPE_Q4_K, 3000), (TYPE_Q5_K, 8192), (TYPE_Q4_K, 1111)], 2560, False),
])
def test_mixed_groups_persistent_grid(ctx, oracle, specs, K, pre):
    """Batch-1 groups with enough k-quant row groups for the persistent grid
    (every k-quant task on its own slice of it, F32 / F16 rows one per wave):
    each format's stage-load count, fused and prequantized input, ragged
    row counts, a task smaller than one workgroup's row groups, groups
    without float tasks (the bodies held to three waves per SIMD)."""
    say(f"mixed persistent {[(qmm_hip.TYPE_NAMES[t], n) for t, n in specs]} K={K} prequantized={pre}")
    _check(_run_group(ctx, oracle, specs, 1, K, seed=360 + K + len(specs), prequantized=pre),
           f"mixed persistent K={K}")


@pytest.mark.parametrize("specs,pre", [
    ([(TYPE_Q4_K, 9728), (TYPE_Q4_K, 9728)], False),
    ([(TYPE_Q6_K, 4096), (TYPE_Q6_K, 4096), (TYPE_Q6_K, 1000)], True),
    ([(TYPE_Q5_K, 6144), (TYPE_Q5_K, 1024), (TYPE_Q5_K, 1024)], False),
])
def test_one_format_groups_persistent_grid(ctx, oracle, specs, pre):
    """Batch-1 groups of one k-quant format ({gate, up}, {q, k, v}) on slices
    of one persistent grid, bit-exact against the oracle."""
    say(f"one-format persistent {[(qmm_hip.TYPE_NAMES[t], n) for t, n in specs]} prequantized={pre}")
    _check(_run_group(ctx, oracle, specs, 1, 2560, seed=380 + len(specs), prequantized=pre), "one-format persistent")
