"""RMSNorm -> Q8_K on the HIP path. The sum of squares is a tree on the GPU
and row order in the reference, so y is compared with a tolerance; the
codes are checked by composition (the oracle's quantizer on the GPU's y,
bit-exact), and against the oracle's own codes wherever y agrees."""
import numpy as np
import pytest

from gpu_util import say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,K", [(1, 256), (1, 2560), (4, 4096), (3, 9728), (2, 16384)])
def test_rmsnorm_q8k(ctx, oracle, M, K):
    say(f"rmsnorm_q8k M={M} K={K}")
    g = np.random.default_rng(M * 7 + K)
    x = (g.standard_normal((M, K)) * 3).astype(np.float32)
    if M > 1:
        x[1] *= 1e-3  # mean square near the epsilon
    gamma = g.uniform(0.5, 1.5, K).astype(np.float32)
    xb, gb = ctx.upload(x), ctx.upload(gamma)
    yb = ctx.malloc(M * K * 4)
    q = ctx.malloc(ctx.lib.qmm_q8k_bytes(M, K))
    ctx.rmsnorm_q8k(xb, gb, M, K, yb, q)
    ctx.sync()
    y = ctx.d2h(yb, np.float32, (M, K))
    d, qs, bs = ctx.read_q8k(q, M, K)
    ry, (rd, rqs, rbs) = oracle.rmsnorm_q8k(x, gamma)
    # y: fp16 values; the summation order only moves inv_rms by a few ulps
    assert np.array_equal(y, oracle.fp16_to_f32(oracle.f32_to_fp16(y))), "y must be fp16 values"
    rel = np.abs(y - ry) / np.maximum(np.abs(ry), 6.1e-5)
    assert rel.max() <= 1e-3, rel.max()
    assert np.mean(y != ry) < 0.01
    # codes by composition: bit-exact
    ed, eqs, ebs = oracle.quantize_q8k(y)
    assert np.array_equal(d.view(np.uint32), ed.view(np.uint32))
    assert np.array_equal(qs, eqs) and np.array_equal(bs, ebs)
    assert np.array_equal(ctx.read_q8k_tiles(q, M, K), qs)
    # and equal to the oracle's own codes in every block where y agrees
    same = (y == ry).reshape(M, K // 256, 256).all(axis=2)
    assert np.array_equal(qs.reshape(M, -1, 256)[same], rqs.reshape(M, -1, 256)[same])
    for b in (xb, gb, yb, q):
        ctx.free(b)


def test_rmsnorm_without_y(ctx, oracle):
    M, K = 2, 2560
    x = np.random.default_rng(1).standard_normal((M, K)).astype(np.float32)
    gamma = np.ones(K, np.float32)
    xb, gb = ctx.upload(x), ctx.upload(gamma)
    q = ctx.malloc(ctx.lib.qmm_q8k_bytes(M, K))
    ctx.rmsnorm_q8k(xb, gb, M, K, None, q)
    ctx.sync()
    d, qs, bs = ctx.read_q8k(q, M, K)
    ry, _ = oracle.rmsnorm_q8k(x, gamma)
    ed, eqs, ebs = oracle.quantize_q8k(ry)
    assert np.mean(qs != eqs) < 0.01
    for b in (xb, gb, q):
        ctx.free(b)


def test_rmsnorm_block_mismatch_rate(ctx, oracle):
    """How often the tree-ordered sum of squares changes a Q8_K block against
    the reference's row-ordered sum, at the workload's width (K = 2560) over
    512 rows: the fraction of 256-value blocks whose codes or scale differ
    from the oracle's (the compiled reference's) is printed and bounded."""
    M, K = 512, 2560
    say(f"rmsnorm mismatch rate M={M} K={K}")
    g = np.random.default_rng(2560)
    x = g.standard_normal((M, K)).astype(np.float32)
    gamma = g.uniform(0.5, 1.5, K).astype(np.float32)
    xb, gb = ctx.upload(x), ctx.upload(gamma)
    q = ctx.malloc(ctx.lib.qmm_q8k_bytes(M, K))
    ctx.rmsnorm_q8k(xb, gb, M, K, None, q)
    ctx.sync()
    d, qs, bs = ctx.read_q8k(q, M, K)
    _, (rd, rqs, rbs) = oracle.rmsnorm_q8k(x, gamma)
    nb = K // 256
    code_diff = (qs.reshape(M, nb, 256) != rqs.reshape(M, nb, 256)).any(axis=2)
    scale_diff = d.reshape(M, nb).view(np.uint32) != rd.reshape(M, nb).view(np.uint32)
    blocks = code_diff | scale_diff
    rows = blocks.any(axis=1)
    codes = np.count_nonzero(qs != rqs)
    say(f"rmsnorm K={K}: {np.count_nonzero(blocks)} of {blocks.size} blocks "
        f"({100 * blocks.mean():.2f} %) and {np.count_nonzero(rows)} of {M} rows differ; "
        f"{codes} of {qs.size} codes ({100 * codes / qs.size:.4f} %), each by at most "
        f"{int(np.abs(qs.astype(int) - rqs.astype(int)).max())}")
    assert np.abs(qs.astype(int) - rqs.astype(int)).max() <= 1
    assert blocks.mean() < 0.25
    for b in (xb, gb, q):
        ctx.free(b)
