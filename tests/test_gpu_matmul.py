"""HIP matmul kernels through the C ABI vs the oracle (the reference's
scalar path restated): GEMV (M = 1), MFMA small-M and prefill GEMMs, all four
weight formats, the multi-task dispatcher, residuals, prequantized inputs."""
import numpy as np
import pytest

import qmm_hip
import synth
from gpu_util import check_outputs, say
from oracle import TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0

pytestmark = pytest.mark.gpu
NAMES = {TYPE_Q4_K: "Q4_K", TYPE_Q5_K: "Q5_K", TYPE_Q6_K: "Q6_K", TYPE_Q8_0: "Q8_0"}


def _run(ctx, oracle, type_id, N, K, M, seed, residual=False):
    say(f"{NAMES[type_id]} N={N} K={K} M={M} residual={residual}")
    w = synth.weights(type_id, N, K, seed=seed)
    x = synth.activations(M, K, seed=seed + 1)
    res = synth.activations(M, N, seed=seed + 2) if residual else None
    wb = ctx.weight_upload(w, type_id, N, K)
    y = ctx.gemm(type_id, wb, N, K, x, res)
    ctx.free(wb)
    task = dict(w=w, type=type_id, rows=N)
    if res is not None:
        task["residual"] = res
    ref = oracle.gemm_multi(x, [task])[0]
    check_outputs(y, ref, f"{NAMES[type_id]} N={N} K={K} M={M}")


# ------------------------------------------------------------------ M = 1
@pytest.mark.parametrize("type_id", [TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0])
@pytest.mark.parametrize("N,K", [(1, 256), (7, 512), (64, 2560), (1001, 2560)])
def test_gemv_small_shapes(ctx, oracle, type_id, N, K):
    _run(ctx, oracle, type_id, N, K, 1, seed=N + K + type_id)


def test_gemv_q4k_decode_shape(ctx, oracle):
    _run(ctx, oracle, TYPE_Q4_K, 9728, 2560, 1, seed=1000)


def test_gemv_q6k_lm_head_shape(ctx, oracle):
    _run(ctx, oracle, TYPE_Q6_K, 151936, 2560, 1, seed=1001)


@pytest.mark.parametrize("type_id,N,K,residual", [(TYPE_Q4_K, 60001, 256, True), (TYPE_Q8_0, 50003, 512, False),
                                                  (TYPE_Q6_K, 49157, 768, True), (TYPE_Q5_K, 40007, 512, True)])
def test_gemv_tall_tensors(ctx, oracle, type_id, N, K, residual):
    """Tensors tall enough for the persistent grid (several row groups per
    wave, the next group prefetched), with ragged last groups."""
    _run(ctx, oracle, type_id, N, K, 1, seed=1100 + type_id, residual=residual)


@pytest.mark.parametrize("type_id,N,K,residual", [(TYPE_Q4_K, 9727, 2560, True), (TYPE_Q6_K, 8195, 768, False),
                                                  (TYPE_Q8_0, 8200, 288, True), (TYPE_Q4_K, 8192, 3072, False),
                                                  (TYPE_Q5_K, 8192, 2560, False), (TYPE_Q5_K, 9733, 3072, True)])
def test_gemv_two_group_grid(ctx, oracle, type_id, N, K, residual):
    """The persistent batch-1 grid where no wave has more than two row groups
    (60 % of the waves have a second, prefetched): ragged last groups, groups
    that start 8 B past a 16-B boundary (Q6_K at K = 768, Q8_0 at K = 288),
    K = 3072."""
    _run(ctx, oracle, type_id, N, K, 1, seed=1200 + N + type_id, residual=residual)


@pytest.mark.parametrize("N,K,residual", [(4096, 2560, False), (9731, 2560, True), (8192, 4096, False),
                                          (19456, 2560, True)])
def test_gemv_q8_0_one_row_per_wave(ctx, oracle, N, K, residual):
    """Q8_0 at one token takes one row per wave at every size: the shapes
    that took 2 (from 4096 rows) and 4 (from 8192 rows) before, on the
    persistent grid, with a ragged row count."""
    _run(ctx, oracle, TYPE_Q8_0, N, K, 1, seed=1250 + N, residual=residual)


def test_gemv_two_group_grid_unaligned_base(ctx, oracle):
    """The same grid on a weight pointer 8 B past a 16-B boundary: rows
    1..N of an uploaded N + 1 (840-B Q6_K rows)."""
    N, K = 8192, 1024
    say(f"Q6_K N={N} K={K} M=1 from row 1")
    w = synth.weights(TYPE_Q6_K, N + 1, K, seed=1300)
    rb = qmm_hip.row_bytes(TYPE_Q6_K, K)
    x = synth.activations(1, K, seed=1301)
    wb = ctx.weight_upload(w, TYPE_Q6_K, N + 1, K)
    xb = ctx.upload(x)
    yb = ctx.malloc(N * 4)
    ctx.gemm_multi_dispatch(xb, 1, K, [qmm_hip.MatrixTask(wb.ptr + rb, TYPE_Q6_K, N, K, yb, N)])
    ctx.sync()
    ref = oracle.gemm_multi(x, [dict(w=w[rb:], type=TYPE_Q6_K, rows=N)])[0]
    check_outputs(ctx.d2h(yb, np.float32, (1, N)), ref, "Q6_K from row 1")
    for b in (wb, xb, yb):
        ctx.free(b)


@pytest.mark.parametrize("type_id,N,K", [(TYPE_Q6_K, 2560, 9728), (TYPE_Q5_K, 4096, 2560),
                                         (TYPE_Q8_0, 2560, 2560), (TYPE_Q4_K, 2560, 4096)])
def test_gemv_other_projection_shapes(ctx, oracle, type_id, N, K):
    _run(ctx, oracle, type_id, N, K, 1, seed=N + type_id)


@pytest.mark.parametrize("type_id,N,K,M,residual", [(TYPE_Q4_K, 9728, 2560, 2, False), (TYPE_Q5_K, 300, 4096, 2, True),
                                                    (TYPE_Q6_K, 2560, 9728, 2, True), (TYPE_Q5_K, 4099, 3072, 2, False),
                                                    (TYPE_Q6_K, 30000, 2560, 3, True), (TYPE_Q4_K, 25000, 1024, 4, False),
                                                    (TYPE_Q4_K, 9728, 2560, 3, True), (TYPE_Q5_K, 17000, 4096, 4, False),
                                                    (TYPE_Q6_K, 20000, 2560, 3, True), (TYPE_Q5_K, 8192, 4096, 3, False),
                                                    (TYPE_Q6_K, 151936, 2560, 4, False)])
def test_gemv_two_to_four_tokens(ctx, oracle, type_id, N, K, M, residual):
    """2 tokens, and 3 from 32 up to 96 rows per CU over K <= 4096: the
    batch-1 GEMV's shape with every token's row in LDS (4-, 2- and 1-row
    groups, ragged last group, residual); 4 tokens and 3 on taller tensors
    (the LM head among them) on the MFMA kernels."""
    _run(ctx, oracle, type_id, N, K, M, seed=1900 + N + M, residual=residual)


@pytest.mark.parametrize("type_id,N", [(TYPE_Q5_K, 8192), (TYPE_Q6_K, 12288), (TYPE_Q4_K, 16384)])
def test_gemv_whole_groups_per_wave(ctx, oracle, type_id, N):
    """Batch 1 on 2, 3 or 4 quads of row groups per CU: the persistent grid
    of one, three or two workgroups per CU, every wave taking whole groups."""
    _run(ctx, oracle, type_id, N, 2560, 1, seed=N + 3 * type_id)


@pytest.mark.parametrize("type_id", [TYPE_Q4_K, TYPE_Q6_K])
def test_gemv_residual(ctx, oracle, type_id):
    _run(ctx, oracle, type_id, 300, 2560, 1, seed=5, residual=True)


# ------------------------------------------------------------- M >= 2 MFMA
@pytest.mark.parametrize("type_id", [TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0])
@pytest.mark.parametrize("M", [2, 5, 16, 17, 40, 64])
def test_mfma_small_shapes(ctx, oracle, type_id, M):
    _run(ctx, oracle, type_id, 77, 512, M, seed=M * 13 + type_id)


@pytest.mark.parametrize("type_id,K", [(TYPE_Q6_K, 256), (TYPE_Q6_K, 768), (TYPE_Q8_0, 96), (TYPE_Q8_0, 160)])
@pytest.mark.parametrize("M", [1, 3, 12, 30, 70])
def test_unaligned_tensor_end(ctx, oracle, type_id, K, M):
    """2-B aligned formats whose tensor (and a workgroup's last row) ends
    inside a dword: the last bytes (Q6_K's d) must still be read."""
    _run(ctx, oracle, type_id, 45, K, M, seed=500 + K + M)


@pytest.mark.parametrize("type_id,K,M", [(TYPE_Q6_K, 4096, 8), (TYPE_Q6_K, 9728, 12), (TYPE_Q8_0, 3072, 5),
                                         (TYPE_Q5_K, 2816, 16), (TYPE_Q4_K, 4352, 8)])
def test_mfma_small_m_long_k(ctx, oracle, type_id, K, M):
    """M <= 16 with K past the resident-codes limit (2560): codes stream with
    the weights, chunk by chunk (Q5_K at K = 2816: the part kernel)."""
    _run(ctx, oracle, type_id, 70, K, M, seed=900 + K + M)


@pytest.mark.parametrize("type_id,N,K,M", [(TYPE_Q6_K, 2560, 9728, 64), (TYPE_Q5_K, 300, 4608, 40),
                                           (TYPE_Q4_K, 333, 9728, 17), (TYPE_Q6_K, 200, 3328, 33),
                                           (TYPE_Q8_0, 2560, 2560, 48), (TYPE_Q6_K, 1000, 4096, 9),
                                           (TYPE_Q8_0, 130, 9728, 64)])
def test_mfma_k_split_tiles(ctx, oracle, type_id, N, K, M):
    """9..64 tokens over K > 3072 (and Q8_0 at any K): 16 x 16 tiles whose
    chunks are split over the 4 waves and summed in block order."""
    _run(ctx, oracle, type_id, N, K, M, seed=1700 + K + M)


@pytest.mark.parametrize("type_id,N,K,M", [(TYPE_Q4_K, 9728, 4096, 64), (TYPE_Q6_K, 8192, 4096, 24)])
def test_mfma_wide_tiles_long_k(ctx, oracle, type_id, N, K, M):
    """17..64 tokens over K > 3072 on tensors tall enough to fill the CUs
    with 32 x 32 / 64 x 32 tiles (the K-split tiles are not used there)."""
    _run(ctx, oracle, type_id, N, K, M, seed=1800 + K + M)


@pytest.mark.parametrize("type_id,N,K,M,residual", [(TYPE_Q4_K, 13000, 2560, 8, True), (TYPE_Q5_K, 12400, 1536, 16, False),
                                                    (TYPE_Q5_K, 1000, 2560, 60, True), (TYPE_Q6_K, 2000, 768, 49, False),
                                                    (TYPE_Q5_K, 6144, 2560, 24, False), (TYPE_Q4_K, 9728, 4096, 24, True),
                                                    (TYPE_Q5_K, 6144, 3584, 48, False), (TYPE_Q6_K, 9000, 3328, 64, True),
                                                    (TYPE_Q6_K, 2560, 2560, 24, True), (TYPE_Q6_K, 1024, 2560, 20, False),
                                                    (TYPE_Q6_K, 2050, 2560, 32, False), (TYPE_Q6_K, 3330, 2560, 40, True),
                                                    (TYPE_Q6_K, 2560, 2560, 47, False), (TYPE_Q4_K, 2560, 4096, 60, True),
                                                    (TYPE_Q4_K, 4096, 3328, 52, False), (TYPE_Q6_K, 2560, 4096, 60, True),
                                                    (TYPE_Q6_K, 1024, 3328, 50, False)])
def test_small_m_token_group_bounds(ctx, oracle, type_id, N, K, M, residual):
    """The part kernel where the resident tiles would hold more than three
    per CU (M <= 16), 16-token groups at 49..64 tokens on few row tiles and
    at 17..32 on up to two tiles per CU (Q6_K: up to half a tile per CU,
    else all 32 tokens per workgroup), Q6_K groups of 32 at 33..48 from 3/4
    of a tile per CU, groups of 16 at 49..64 over K > 3072 below 3/4 of a
    tile per CU (Q6_K: up to 1/4), and over K up to 4096 (4 blocks per K part) from 17 tokens
    on tall tensors."""
    _run(ctx, oracle, type_id, N, K, M, seed=4100 + N + M, residual=residual)


@pytest.mark.parametrize("type_id,N,K,M", [(TYPE_Q4_K, 9728, 2560, 8), (TYPE_Q4_K, 12288, 2560, 5),
                                           (TYPE_Q4_K, 8500, 3072, 7), (TYPE_Q4_K, 8211, 768, 6)])
def test_resident_tile_layouts(ctx, oracle, type_id, N, K, M):
    """Q4_K at 8 tokens or fewer on two to three row tiles per CU: three
    16-row tiles resident per workgroup, 12 blocks per row, a partial last
    tile."""
    _run(ctx, oracle, type_id, N, K, M, seed=1500 + N + M)


@pytest.mark.parametrize("type_id,N,K,M", [(TYPE_Q4_K, 6144, 2560, 8), (TYPE_Q6_K, 13000, 1024, 3),
                                           (TYPE_Q5_K, 300, 3072, 16), (TYPE_Q4_K, 4111, 768, 11),
                                           (TYPE_Q6_K, 3000, 2560, 7), (TYPE_Q5_K, 6144, 2560, 12),
                                           (TYPE_Q6_K, 6144, 2560, 16), (TYPE_Q4_K, 9728, 2560, 13)])
def test_part_kernel_small_m_layouts(ctx, oracle, type_id, N, K, M):
    """M <= 16, K <= 3072 outside those: one 16-row tile and 16 tokens per
    workgroup at any tile count, 12 blocks per row, partial last tiles."""
    _run(ctx, oracle, type_id, N, K, M, seed=1500 + N + M)


@pytest.mark.parametrize("type_id,N,K,M,residual", [(TYPE_Q6_K, 1024, 2560, 100, True), (TYPE_Q4_K, 2560, 2560, 80, False),
                                                    (TYPE_Q5_K, 300, 3072, 256, True), (TYPE_Q6_K, 2560, 2560, 192, False),
                                                    (TYPE_Q4_K, 1000, 2560, 65, True), (TYPE_Q5_K, 6144, 2560, 96, False)])
def test_part_kernel_past_64_tokens(ctx, oracle, type_id, N, K, M, residual):
    """65..256 tokens over K <= 3072 on tensors short enough that 32-token
    groups number at most 4.5 workgroups per CU: the part kernel (ragged
    last token group, scales of every token in LDS)."""
    _run(ctx, oracle, type_id, N, K, M, seed=1650 + N + M, residual=residual)


@pytest.mark.parametrize("type_id,N,K,M,residual", [(TYPE_Q4_K, 9728, 4096, 8, True), (TYPE_Q4_K, 19456, 4096, 12, False),
                                                    (TYPE_Q5_K, 2560, 3328, 16, True), (TYPE_Q5_K, 1000, 3584, 3, False),
                                                    (TYPE_Q4_K, 1000, 4096, 9, False), (TYPE_Q5_K, 6144, 4096, 5, True),
                                                    (TYPE_Q5_K, 300, 4096, 40, True), (TYPE_Q4_K, 2560, 4096, 64, False),
                                                    (TYPE_Q5_K, 1024, 3584, 24, False), (TYPE_Q4_K, 4100, 3328, 56, True)])
def test_part_kernel_small_m_long_k(ctx, oracle, type_id, N, K, M, residual):
    """Q4_K / Q5_K up to 64 tokens over 3072 < K <= 4096 at any tile count:
    the part kernel with 4 blocks per K part (13..16 blocks per row), token
    groups, partial last tiles."""
    _run(ctx, oracle, type_id, N, K, M, seed=1600 + N + M, residual=residual)


@pytest.mark.parametrize("M", [8, 16, 32, 48, 64])
def test_tree_verify_q4k(ctx, oracle, M):
    _run(ctx, oracle, TYPE_Q4_K, 9728, 2560, M, seed=2000 + M)


@pytest.mark.parametrize("M", [8, 16, 32, 64])
def test_tree_verify_q5k_qkv(ctx, oracle, M):
    _run(ctx, oracle, TYPE_Q5_K, 4096, 2560, M, seed=2100 + M)


@pytest.mark.parametrize("type_id,N,K,M,residual", [(TYPE_Q4_K, 9728, 2560, 2, False), (TYPE_Q6_K, 6000, 2560, 2, True),
                                                    (TYPE_Q5_K, 333, 4096, 2, False), (TYPE_Q6_K, 2560, 9728, 2, True),
                                                    (TYPE_Q6_K, 24832, 2560, 3, False), (TYPE_Q4_K, 24600, 1024, 4, True)])
def test_few_tokens_fp32_input(ctx, oracle, type_id, N, K, M, residual):
    """2..4 tokens in the batch-1 GEMV's shape on fp32 input: at 2 tokens
    and K <= 4096 the kernel quantizes the tokens' rows in its fill (ragged
    row counts, residuals); past that the quantizer's launch first. Bit-exact
    against the oracle."""
    _run(ctx, oracle, type_id, N, K, M, seed=2400 + N + M, residual=residual)


@pytest.mark.parametrize("type_id,N,K,M,residual", [(TYPE_Q6_K, 3000, 2560, 20, False), (TYPE_Q5_K, 4096, 2560, 33, True),
                                                    (TYPE_Q4_K, 5000, 3072, 29, False), (TYPE_Q6_K, 1000, 1024, 57, True),
                                                    (TYPE_Q4_K, 300, 2560, 47, True), (TYPE_Q5_K, 4000, 768, 64, False)])
def test_part_token_groups(ctx, oracle, type_id, N, K, M, residual):
    """17..64 tokens over K <= 3072: part-kernel workgroups on groups of 16
    or 32 tokens (a last group holding 1..31 of them), or all 32 tokens
    where the row tiles outnumber the CUs."""
    _run(ctx, oracle, type_id, N, K, M, seed=2300 + N + M, residual=residual)


def _extreme_weights(type_id, N, K, seed):
    """Random blocks pushed to the ends of the integer ranges: all 6-bit
    scales and mins 63 (Q4_K / Q5_K) or int8 scales cycling through -128,
    127, -1, 0 (Q6_K), and every third row with all-max or all-zero quants,
    so every weight * scale product reaches its largest magnitude."""
    w = synth.weights(type_id, N, K, seed=seed)
    bb = {TYPE_Q4_K: 144, TYPE_Q5_K: 176, TYPE_Q6_K: 210}[type_id]
    blk = w.reshape(N, -1, bb)
    if type_id == TYPE_Q6_K:
        blk[:, :, 192:208] = np.resize(np.array([-128, 127, -1, 0], np.int8), 16).view(np.uint8)
        blk[0::3, :, 0:192] = 0x00   # q = 0: q - 32 = -32
        blk[1::3, :, 0:192] = 0xFF   # q = 63: q - 32 = 31
    else:
        blk[:, :, 4:16] = 0xFF       # every scale and min 63
        blk[0::3, :, 16:] = 0xFF     # q = 15 (Q4_K) / 31 (Q5_K)
        blk[1::3, :, 16:] = 0x00
    return w


@pytest.mark.parametrize("type_id", [TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K])
@pytest.mark.parametrize("M,K", [(5, 1024), (40, 1024), (512, 1024), (512, 4352), (40, 4352)])
def test_mfma_extreme_scales(ctx, oracle, type_id, M, K):
    """Extreme scales and quants through the MFMA paths (scales folded into
    the weight operand from M > 16; the slab kernels over K > 4096): the
    integer sums stay exact."""
    N = 96
    say(f"extreme scales {NAMES[type_id]} N={N} K={K} M={M}")
    w = _extreme_weights(type_id, N, K, seed=700 + M)
    x = synth.activations(M, K, seed=701)
    x[:, ::7] *= 50.0   # large entries: many codes at +-127
    wb = ctx.weight_upload(w, type_id, N, K)
    y = ctx.gemm(type_id, wb, N, K, x)
    ctx.free(wb)
    ref = oracle.gemm_multi(x, [dict(w=w, type=type_id, rows=N)])[0]
    check_outputs(y, ref, f"extreme {NAMES[type_id]} M={M}")


@pytest.mark.parametrize("type_id", [TYPE_Q4_K, TYPE_Q6_K])
@pytest.mark.parametrize("M", [9, 33])
def test_mfma_residual(ctx, oracle, type_id, M):
    _run(ctx, oracle, type_id, 200, 2560, M, seed=7 + M, residual=True)


@pytest.mark.parametrize("name", ["qkv", "o", "gate", "down", "q8_0"])
def test_prefill_m512_row_subsets(ctx, oracle, name):
    """Full prefill tensors at M = 512 on the GPU; the oracle checks the first
    and last 128 rows (a full check of 512 x 9728 x 2560 on the CPU is slow)."""
    type_id, N, K = synth.PREFILL_LAYER["tensors"][name]
    M = 512
    say(f"prefill {name} {NAMES[type_id]} N={N} K={K} M={M}")
    w = synth.weights(type_id, N, K, seed=3000 + N)
    x = synth.activations(M, K, seed=3001)
    wb = ctx.weight_upload(w, type_id, N, K)
    y = ctx.gemm(type_id, wb, N, K, x)
    ctx.free(wb)
    rb = synth.row_bytes(type_id, K)
    for r0 in (0, N - 128):
        ref = oracle.gemm_multi(x, [dict(w=w[r0 * rb:(r0 + 128) * rb], type=type_id, rows=128)])[0]
        check_outputs(y[:, r0:r0 + 128], ref, f"prefill {name} rows {r0}..{r0 + 128}")


@pytest.mark.parametrize("name", ["qkv", "o", "gate", "down", "q8_0"])
def test_prefill_m512_every_row_tile(ctx, oracle, name):
    """Full prefill tensors at M = 512: one row of every 16-row tile (its
    position in the tile cycling through 0..15), all 512 tokens, against the
    oracle, so every row slab and token group of the grid is checked."""
    type_id, N, K = synth.PREFILL_LAYER["tensors"][name]
    M = 512
    say(f"prefill strided rows {name} {NAMES[type_id]} N={N} K={K} M={M}")
    w = synth.weights(type_id, N, K, seed=3100 + N)
    x = synth.activations(M, K, seed=3101)
    wb = ctx.weight_upload(w, type_id, N, K)
    y = ctx.gemm(type_id, wb, N, K, x)
    ctx.free(wb)
    rb = synth.row_bytes(type_id, K)
    rows = np.array([16 * i + (7 * i) % 16 for i in range(N // 16)])
    sub = w.reshape(N, rb)[rows].reshape(-1)
    ref = oracle.gemm_multi(x, [dict(w=sub, type=type_id, rows=rows.size)])[0]
    check_outputs(y[:, rows], ref, f"prefill {name} strided rows")


@pytest.mark.parametrize("type_id", [TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0])
@pytest.mark.parametrize("N,K,M", [(70, 2560, 65), (201, 1024, 129), (64, 4096, 200), (130, 768, 300),
                                   (70, 4352, 65), (201, 4608, 129), (130, 5120, 300)])
def test_prefill_tails(ctx, oracle, type_id, N, K, M):
    """Partial row slabs and token groups past 64 tokens (N and M not
    multiples of the workgroup tile), several K: the part kernel's 32-token
    groups on these short tensors over K <= 4096, the slab kernels past
    (Q8_0: the tile kernel)."""
    _run(ctx, oracle, type_id, N, K, M, seed=3200 + N + M + type_id)


@pytest.mark.parametrize("M", [65, 100])
def test_prefill_q5k_decoded_slabs_under_128(ctx, oracle, M):
    """Q5_K past 64 tokens on a tensor whose 32-row decoded slabs number at
    least 5/8 of the CUs: the decoded slabs with the tokens padded to 128
    (below that height the packed slabs), with a residual."""
    _run(ctx, oracle, TYPE_Q5_K, 9000, 2560, M, seed=3600 + M, residual=True)


@pytest.mark.parametrize("type_id", [TYPE_Q4_K, TYPE_Q6_K, TYPE_Q8_0])
def test_prefill_residual(ctx, oracle, type_id):
    _run(ctx, oracle, type_id, 150, 2560, 140, seed=3300 + type_id, residual=True)


def test_prefill_task_group(ctx, oracle):
    """gate + up (and a third task) of one type in one call at M = 160: one
    launch over the tasks' concatenated row slabs."""
    K, M = 2560, 160
    say(f"prefill task group M={M}")
    specs = [1000, 333, 64]
    x = synth.activations(M, K, seed=3400)
    ws = [synth.weights(TYPE_Q4_K, n, K, seed=3401 + i) for i, n in enumerate(specs)]
    xb = ctx.upload(x)
    wbs = [ctx.weight_upload(w, TYPE_Q4_K, n, K) for w, n in zip(ws, specs)]
    ybs = [ctx.malloc(M * n * 4) for n in specs]
    tasks = [qmm_hip.MatrixTask(wb, TYPE_Q4_K, n, K, yb, n) for wb, yb, n in zip(wbs, ybs, specs)]
    ctx.gemm_multi_dispatch(xb, M, K, tasks)
    ctx.sync()
    refs = oracle.gemm_multi(x, [dict(w=w, type=TYPE_Q4_K, rows=n) for w, n in zip(ws, specs)])
    for i, (n, yb) in enumerate(zip(specs, ybs)):
        check_outputs(ctx.d2h(yb, np.float32, (M, n)), refs[i], f"group task {i}")
    for b in [xb] + wbs + ybs:
        ctx.free(b)


@pytest.mark.parametrize("M,specs", [(200, (2560, 130, 64)), (400, (2560, 70))])
def test_prefill_q8_0_tile_shapes(ctx, oracle, M, specs):
    """Q8_0 past 64 tokens in task groups: 64 x 16 tiles where the 64 x 32
    tiles would number at most 1.5 per CU (M = 200), else 64 x 32 (M = 400),
    the first task with a residual."""
    K = 2560
    say(f"prefill Q8_0 tiles M={M} tasks={specs}")
    x = synth.activations(M, K, seed=3500 + M)
    ws = [synth.weights(TYPE_Q8_0, n, K, seed=3501 + i) for i, n in enumerate(specs)]
    res = synth.activations(M, specs[0], seed=3510 + M)
    xb = ctx.upload(x)
    rb = ctx.upload(res)
    wbs = [ctx.weight_upload(w, TYPE_Q8_0, n, K) for w, n in zip(ws, specs)]
    ybs = [ctx.malloc(M * n * 4) for n in specs]
    tasks = [qmm_hip.MatrixTask(wb, TYPE_Q8_0, n, K, yb, n, residual=rb if i == 0 else None,
                                res_stride=specs[0] if i == 0 else 0)
             for i, (wb, yb, n) in enumerate(zip(wbs, ybs, specs))]
    ctx.gemm_multi_dispatch(xb, M, K, tasks)
    ctx.sync()
    tdicts = [dict(w=w, type=TYPE_Q8_0, rows=n) for w, n in zip(ws, specs)]
    tdicts[0]["residual"] = res
    refs = oracle.gemm_multi(x, tdicts)
    for i, (n, yb) in enumerate(zip(specs, ybs)):
        check_outputs(ctx.d2h(yb, np.float32, (M, n)), refs[i], f"Q8_0 group task {i}")
    for b in [xb, rb] + wbs + ybs:
        ctx.free(b)


# ---------------------------------------------------------------- dispatch
@pytest.mark.parametrize("M", [1, 6])
def test_multi_task_dispatch_mixed_types(ctx, oracle, M):
    """Four tasks sharing one input (the E:7959 / E:8114 call pattern), one
    with a residual, with Q8_K and Q8_0 activations both needed."""
    K = 2560
    say(f"multi-task dispatch M={M}")
    specs = [(TYPE_Q4_K, 300), (TYPE_Q5_K, 64), (TYPE_Q6_K, 32), (TYPE_Q8_0, 96)]
    x = synth.activations(M, K, seed=9)
    ws = [synth.weights(t, n, K, seed=40 + i) for i, (t, n) in enumerate(specs)]
    res = synth.activations(M, 64, seed=11)
    xb = ctx.upload(x)
    wbs = [ctx.weight_upload(w, t, n, K) for w, (t, n) in zip(ws, specs)]
    ybs = [ctx.malloc(M * n * 4) for _, n in specs]
    rb = ctx.upload(res)
    tasks = [qmm_hip.MatrixTask(wb, t, n, K, yb, n, rb if i == 1 else None, n)
             for i, (wb, yb, (t, n)) in enumerate(zip(wbs, ybs, specs))]
    ctx.gemm_multi_dispatch(xb, M, K, tasks)
    ctx.sync()
    assert [t.start_row for t in tasks] == [0, 300, 364, 396]
    refs = oracle.gemm_multi(x, [dict(w=w, type=t, rows=n, **({"residual": res} if i == 1 else {}))
                                 for i, (w, (t, n)) in enumerate(zip(ws, specs))])
    for i, ((t, n), yb) in enumerate(zip(specs, ybs)):
        check_outputs(ctx.d2h(yb, np.float32, (M, n)), refs[i], f"task {i}")
    for b in [xb, rb] + wbs + ybs:
        ctx.free(b)


def test_prequantized_dispatch_and_strides(ctx, oracle):
    """Oracle-quantized Q8_K activations fed to the prequantized entry point;
    the output written with a row stride wider than the task."""
    M, K, N, ld = 3, 2560, 100, 130
    say("prequantized dispatch")
    x = synth.activations(M, K, seed=12)
    w = synth.weights(TYPE_Q4_K, N, K, seed=13)
    d, qs, bs = oracle.quantize_q8k(x)
    qb = ctx.malloc(ctx.lib.qmm_q8k_bytes(M, K))
    ctx.write_q8k(qb, d, qs, bs)
    wb = ctx.weight_upload(w, TYPE_Q4_K, N, K)
    yb = ctx.malloc(M * ld * 4)
    ctx.h2d(yb, np.full((M, ld), 7.0, np.float32))
    ctx.gemm_multi_dispatch_prequantized(qb, None, M, K, [qmm_hip.MatrixTask(wb, TYPE_Q4_K, N, K, yb, ld)])
    ctx.sync()
    y = ctx.d2h(yb, np.float32, (M, ld))
    ref = oracle.gemm_multi(x, [dict(w=w, type=TYPE_Q4_K, rows=N)], prequantized=((d, qs, bs), None))[0]
    check_outputs(y[:, :N], ref, "prequantized")
    assert np.all(y[:, N:] == 7.0)  # nothing written past the task's rows
    for b in (qb, wb, yb):
        ctx.free(b)


@pytest.mark.parametrize("type_id,specs", [
    (TYPE_Q4_K, [(9000, True), (7001, False), (4003, True)]),
    (TYPE_Q6_K, [(5000, False), (3001, True), (6007, False)]),
])
def test_task_groups_large(ctx, oracle, type_id, specs):
    """Batch-1 task groups of thousands of rows per task (one launch of
    several workgroups per CU), ragged ends and residuals."""
    K = 2560
    say(f"large task group {NAMES[type_id]} {specs}")
    x = synth.activations(1, K, seed=23)
    ws = [synth.weights(type_id, n, K, seed=70 + i) for i, (n, _) in enumerate(specs)]
    ress = [synth.activations(1, n, seed=90 + i) if r else None for i, (n, r) in enumerate(specs)]
    xb = ctx.upload(x)
    wbs = [ctx.weight_upload(w, type_id, n, K) for w, (n, _) in zip(ws, specs)]
    ybs = [ctx.malloc(n * 4) for n, _ in specs]
    rbs = [ctx.upload(r) if r is not None else None for r in ress]
    tasks = [qmm_hip.MatrixTask(wb, type_id, n, K, yb, n, rb, n if rb is not None else 0)
             for wb, yb, rb, (n, _) in zip(wbs, ybs, rbs, specs)]
    ctx.gemm_multi_dispatch(xb, 1, K, tasks)
    ctx.sync()
    refs = oracle.gemm_multi(x, [dict(w=w, type=type_id, rows=n, **({"residual": r} if r is not None else {}))
                                 for w, r, (n, _) in zip(ws, ress, specs)])
    for i, ((n, _), yb) in enumerate(zip(specs, ybs)):
        check_outputs(ctx.d2h(yb, np.float32, (1, n)), refs[i], f"task {i}")
    for b in [xb] + wbs + ybs + [r for r in rbs if r is not None]:
        ctx.free(b)


@pytest.mark.parametrize("M", [1, 6, 40, 70])
def test_task_groups_one_launch(ctx, oracle, M):
    """Many tasks of one type (more than one launch's group of 8), tiny-N tasks
    and residuals interleaved with another type: the E:7954-7959 /
    E:8110-8114 task groups run as one launch per type group."""
    K = 2560
    say(f"task groups M={M}")
    specs = [(TYPE_Q4_K, 96), (TYPE_Q6_K, 40), (TYPE_Q4_K, 32), (TYPE_Q4_K, 1), (TYPE_Q4_K, 300),
             (TYPE_Q4_K, 33), (TYPE_Q6_K, 16), (TYPE_Q4_K, 64), (TYPE_Q4_K, 7), (TYPE_Q4_K, 128),
             (TYPE_Q4_K, 48), (TYPE_Q4_K, 17)]
    x = synth.activations(M, K, seed=19)
    ws = [synth.weights(t, n, K, seed=60 + i) for i, (t, n) in enumerate(specs)]
    ress = [synth.activations(M, n, seed=80 + i) if i % 3 == 1 else None for i, (_, n) in enumerate(specs)]
    xb = ctx.upload(x)
    wbs = [ctx.weight_upload(w, t, n, K) for w, (t, n) in zip(ws, specs)]
    ybs = [ctx.malloc(M * n * 4) for _, n in specs]
    rbs = [ctx.upload(r) if r is not None else None for r in ress]
    tasks = [qmm_hip.MatrixTask(wb, t, n, K, yb, n, rb, n if rb is not None else 0)
             for wb, yb, rb, (t, n) in zip(wbs, ybs, rbs, specs)]
    ctx.gemm_multi_dispatch(xb, M, K, tasks)
    ctx.sync()
    refs = oracle.gemm_multi(x, [dict(w=w, type=t, rows=n, **({"residual": r} if r is not None else {}))
                                 for w, r, (t, n) in zip(ws, ress, specs)])
    for i, ((t, n), yb) in enumerate(zip(specs, ybs)):
        check_outputs(ctx.d2h(yb, np.float32, (M, n)), refs[i], f"task {i}")
    for b in [xb] + wbs + ybs + [r for r in rbs if r is not None]:
        ctx.free(b)


@pytest.mark.parametrize("M,K,specs,residual", [(512, 2560, (9728, 9728), False), (300, 512, (13200, 13107), True)])
def test_prefill_eight_wave_slabs(ctx, oracle, M, K, specs, residual):
    """Task groups with at least four 128 x 64 slabs per CU take the 8-wave
    prefill workgroups: the FFN's gate + up at M = 512, and ragged tasks
    (partial row slabs and token groups, a residual) at M = 300; one row of
    every 16-row tile of each task against the oracle, all tokens."""
    say(f"prefill 8-wave slabs M={M} K={K} tasks={specs}")
    x = synth.activations(M, K, seed=3500 + M)
    xb = ctx.upload(x)
    bufs, tasks, hosts, res_h = [xb], [], [], []
    for i, n in enumerate(specs):
        w = synth.weights(TYPE_Q4_K, n, K, seed=3501 + i + M)
        wb, yb = ctx.weight_upload(w, TYPE_Q4_K, n, K), ctx.malloc(M * n * 4)
        rh = synth.activations(M, n, seed=3520 + i) if residual and i == 1 else None
        rb = ctx.upload(rh) if rh is not None else None
        bufs += [b for b in (wb, yb, rb) if b is not None]
        tasks.append(qmm_hip.MatrixTask(wb, TYPE_Q4_K, n, K, yb, n, residual=rb, res_stride=n if rh is not None else 0))
        hosts.append(w)
        res_h.append(rh)
    ctx.gemm_multi_dispatch(xb, M, K, tasks)
    ctx.sync()
    rbytes = synth.row_bytes(TYPE_Q4_K, K)
    for t, w, rh in zip(tasks, hosts, res_h):
        n = t.rows
        rows = np.array([16 * i + (5 * i) % 16 for i in range(n // 16)] + [n - 1])
        got = ctx.d2h(t.dst, np.float32, (M, n))[:, rows]
        sub = w.reshape(n, rbytes)[rows].reshape(-1)
        ref = oracle.gemm_multi(x, [dict(w=sub, type=TYPE_Q4_K, rows=rows.size)])[0]
        if rh is not None:
            ref = ref + rh[:, rows]
        check_outputs(got, ref, f"8-wave slabs task of {n} rows")
    for b in bufs:
        ctx.free(b)


@pytest.mark.parametrize("type_id,M,K,specs,res_task", [
    (TYPE_Q5_K, 256, 2560, (2048, 512, 528), 1),
    (TYPE_Q5_K, 333, 1024, (4000, 1037), 0),
    (TYPE_Q6_K, 384, 1024, (3000, 450), 1),
    (TYPE_Q6_K, 129, 4352, (2560,), None),
])
def test_prefill_decoded_slab_groups(ctx, oracle, type_id, M, K, specs, res_task):
    """Q5_K / Q6_K from 128 tokens take the decoded-slab workgroups: task
    groups over their concatenated row slabs (partial slabs at each task's
    end), partial token groups, a residual; every row of every task, all
    tokens, against the oracle."""
    say(f"prefill decoded slabs {NAMES[type_id]} M={M} K={K} tasks={specs}")
    x = synth.activations(M, K, seed=3600 + M)
    xb = ctx.upload(x)
    bufs, tasks, hosts, res_h = [xb], [], [], []
    for i, n in enumerate(specs):
        w = synth.weights(type_id, n, K, seed=3601 + i + M)
        wb, yb = ctx.weight_upload(w, type_id, n, K), ctx.malloc(M * n * 4)
        rh = synth.activations(M, n, seed=3620 + i) if res_task == i else None
        rb = ctx.upload(rh) if rh is not None else None
        bufs += [b for b in (wb, yb, rb) if b is not None]
        tasks.append(qmm_hip.MatrixTask(wb, type_id, n, K, yb, n, residual=rb, res_stride=n if rh is not None else 0))
        hosts.append(w)
        res_h.append(rh)
    ctx.gemm_multi_dispatch(xb, M, K, tasks)
    ctx.sync()
    refs = oracle.gemm_multi(x, [dict(w=w, type=type_id, rows=t.rows, **({"residual": rh} if rh is not None else {}))
                                 for t, w, rh in zip(tasks, hosts, res_h)])
    for i, t in enumerate(tasks):
        check_outputs(ctx.d2h(t.dst, np.float32, (M, t.rows)), refs[i], f"decoded slabs task {i}")
    for b in bufs:
        ctx.free(b)


@pytest.mark.parametrize("M,K,specs,res_task", [
    (64, 9728, (2560,), None),
    (48, 4352, (300, 45), 1),
    (33, 9728, (130,), 0),
    (32, 9728, (2560,), None),
    (24, 4352, (300, 45), 1),
    (17, 9728, (130,), 0),
    (20, 4608, (200,), None),
])
def test_small_m_q6k_decoded_slabs_k_split(ctx, oracle, M, K, specs, res_task):
    """Q6_K at 17..64 tokens over K > 4096 (16 x 32 slabs up to 32 tokens,
    16 x 64 past): decoded slabs whose four K groups walk every fourth block
    and meet in block order, steps two deep; task groups, partial row slabs,
    a residual, K not a multiple of 4 blocks (17, 18 and 38 blocks: five
    to ten steps, the transfers issued past the last block reading zeros);
    every row of every task, all tokens, against the oracle."""
    say(f"small-M Q6_K K-split decoded slabs M={M} K={K} tasks={specs}")
    x = synth.activations(M, K, seed=3700 + M)
    xb = ctx.upload(x)
    bufs, tasks, hosts, res_h = [xb], [], [], []
    for i, n in enumerate(specs):
        w = synth.weights(TYPE_Q6_K, n, K, seed=3701 + i + M)
        wb, yb = ctx.weight_upload(w, TYPE_Q6_K, n, K), ctx.malloc(M * n * 4)
        rh = synth.activations(M, n, seed=3720 + i) if res_task == i else None
        rb = ctx.upload(rh) if rh is not None else None
        bufs += [b for b in (wb, yb, rb) if b is not None]
        tasks.append(qmm_hip.MatrixTask(wb, TYPE_Q6_K, n, K, yb, n, residual=rb, res_stride=n if rh is not None else 0))
        hosts.append(w)
        res_h.append(rh)
    ctx.gemm_multi_dispatch(xb, M, K, tasks)
    ctx.sync()
    refs = oracle.gemm_multi(x, [dict(w=w, type=TYPE_Q6_K, rows=t.rows, **({"residual": rh} if rh is not None else {}))
                                 for t, w, rh in zip(tasks, hosts, res_h)])
    for i, t in enumerate(tasks):
        check_outputs(ctx.d2h(t.dst, np.float32, (M, t.rows)), refs[i], f"K-split decoded slabs task {i}")
    for b in bufs:
        ctx.free(b)


@pytest.mark.parametrize("type_id,M,K,specs,res_task", [
    (TYPE_Q4_K, 64, 9728, (2560,), None),
    (TYPE_Q5_K, 48, 8192, (4096,), 0),
    (TYPE_Q4_K, 40, 8448, (3000, 900), 1),
])
def test_small_m_q4k_q5k_decoded_slabs_long_k(ctx, oracle, type_id, M, K, specs, res_task):
    """Q4_K / Q5_K at 33..64 tokens over K >= 8192 where the K-split tiles
    would take more than two per CU: the decoded slabs in four K groups (the
    mins as fp16 sums against fp16 mins), task groups, a residual, K of 33
    blocks; every row of every task, all tokens, against the oracle."""
    say(f"small-M {NAMES[type_id]} K-split decoded slabs M={M} K={K} tasks={specs}")
    x = synth.activations(M, K, seed=3800 + M)
    xb = ctx.upload(x)
    bufs, tasks, hosts, res_h = [xb], [], [], []
    for i, n in enumerate(specs):
        w = synth.weights(type_id, n, K, seed=3801 + i + M)
        wb, yb = ctx.weight_upload(w, type_id, n, K), ctx.malloc(M * n * 4)
        rh = synth.activations(M, n, seed=3820 + i) if res_task == i else None
        rb = ctx.upload(rh) if rh is not None else None
        bufs += [b for b in (wb, yb, rb) if b is not None]
        tasks.append(qmm_hip.MatrixTask(wb, type_id, n, K, yb, n, residual=rb, res_stride=n if rh is not None else 0))
        hosts.append(w)
        res_h.append(rh)
    ctx.gemm_multi_dispatch(xb, M, K, tasks)
    ctx.sync()
    refs = oracle.gemm_multi(x, [dict(w=w, type=type_id, rows=t.rows, **({"residual": rh} if rh is not None else {}))
                                 for t, w, rh in zip(tasks, hosts, res_h)])
    for i, t in enumerate(tasks):
        check_outputs(ctx.d2h(t.dst, np.float32, (M, t.rows)), refs[i], f"long-K decoded slabs task {i}")
    for b in bufs:
        ctx.free(b)


@pytest.mark.parametrize("type_id,M,K,specs,res_task", [
    (TYPE_Q4_K, 8, 2560, (9728,), None),
    (TYPE_Q4_K, 6, 512, (8200, 1000), 1),
    (TYPE_Q4_K, 5, 3072, (9000,), 0),
    (TYPE_Q4_K, 7, 2560, (6000, 4100), 0),
    (TYPE_Q4_K, 16, 512, (4096, 1000), 1),
    (TYPE_Q5_K, 5, 3072, (6144,), None),
    (TYPE_Q5_K, 16, 2560, (4100, 33), 0),
])
def test_resident_tiles_groups(ctx, oracle, type_id, M, K, specs, res_task):
    """Q4_K groups at up to 8 tokens on two to three row tiles per CU take
    the resident-tile kernel (three row tiles per workgroup), the others
    the part kernel (one tile and 16 tokens per workgroup); x with
    codes at +-127 and an all-zero block; every row of every task, all
    tokens, against the oracle. Run three times: an MFMA result read too
    early gave wrong values in random tiles from run to run."""
    say(f"resident tiles {NAMES[type_id]} M={M} K={K} tasks={specs}")
    x = synth.activations(M, K, seed=3800 + M)
    x[:, ::11] *= 30.0  # codes at +-127
    x[1 % M, 256:512] = 0.0  # an all-zero block (d = 0)
    xb = ctx.upload(x)
    bufs, tasks, hosts, res_h = [xb], [], [], []
    for i, n in enumerate(specs):
        w = synth.weights(type_id, n, K, seed=3801 + i + M)
        wb, yb = ctx.weight_upload(w, type_id, n, K), ctx.malloc(M * n * 4)
        rh = synth.activations(M, n, seed=3820 + i) if res_task == i else None
        rb = ctx.upload(rh) if rh is not None else None
        bufs += [b for b in (wb, yb, rb) if b is not None]
        tasks.append(qmm_hip.MatrixTask(wb, type_id, n, K, yb, n, residual=rb, res_stride=n if rh is not None else 0))
        hosts.append(w)
        res_h.append(rh)
    refs = oracle.gemm_multi(x, [dict(w=w, type=type_id, rows=t.rows, **({"residual": rh} if rh is not None else {}))
                                 for t, w, rh in zip(tasks, hosts, res_h)])
    for run in range(3):
        ctx.gemm_multi_dispatch(xb, M, K, tasks)
        ctx.sync()
        for i, t in enumerate(tasks):
            check_outputs(ctx.d2h(t.dst, np.float32, (M, t.rows)), refs[i], f"resident tiles task {i}, run {run}")
    for b in bufs:
        ctx.free(b)
