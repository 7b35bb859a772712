/*
 * ref_harness.c — TEST INFRASTRUCTURE. Compiles the reference engine's own
 * translation unit (src/v182_r22_breakthrough_engine.c, read in place from
 * the reference checkout by oracle/Makefile) for x86 and exports its scalar
 * dequant / quantize / dot functions with plain C signatures, so the tests
 * can check the CPU restatement (qmm_oracle.c) against the real reference
 * and the benchmark can time the reference's own CPU dot path.
 *
 * Build notes (see oracle/Makefile):
 *  - HOST_SYNTAX_CHECK lifts the engine's "arm64 only" #error (E:63-65);
 *    without arm_neon.h every kernel takes its scalar #else branch.
 *  - main (E:12312) and the one non-static bridge engine_exec_block_batch
 *    (E:10891) are renamed to unused static functions, so clang emits only
 *    what the wrappers below reach. That leaves out the dispatcher, whose
 *    Q4_K row kernel sdot_row_q4_k_batch (E:918) exists only under the NEON
 *    guard (E:1951); the Q4_K dot is taken from eval_single_lm_row_dot
 *    (E:10986-11027), the reference's portable Q4_K path.
 *  - fp16 buffers cross the boundary as raw uint16_t bit patterns.
 */
#define main static ref_engine_main_unused
#define engine_exec_block_batch static ref_engine_exec_block_batch_unused
#include "v182_r22_breakthrough_engine.c"
#undef main
#undef engine_exec_block_batch

float ref_fp16_to_f32(uint16_t h) { return fp16_bits_to_f32(h); }

uint16_t ref_f32_to_fp16(float f) {
    __fp16 h = (__fp16)f;
    uint16_t bits;
    memcpy(&bits, &h, 2);
    return bits;
}

void ref_get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    get_scale_min_k4(j, q, d, m);
}

/* One block of the given type -> fp16 bits (E:598-853). */
int ref_dequant_block(uint32_t type, const uint8_t *blk, uint16_t *dst) {
    switch (type) {
        case GGML_TYPE_Q8_0: dequant_block_q8_0(blk, (__fp16 *)dst); return 0;
        case GGML_TYPE_Q4_K: dequant_block_q4_k(blk, (__fp16 *)dst); return 0;
        case GGML_TYPE_Q5_K: dequant_block_q5_k(blk, (__fp16 *)dst); return 0;
        case GGML_TYPE_Q6_K: dequant_block_q6_k(blk, (__fp16 *)dst); return 0;
        default: return -1;
    }
}

/* quantize_row_fp16_to_q8_k (E:925-990) unpacked into d / qs / bsum32 arrays. */
void ref_quantize_row_q8k(const uint16_t *x, int k, float *d, int8_t *qs, int32_t *bsum32) {
    const int nb = k / 256;
    BlockQ8K *y = (BlockQ8K *)calloc((size_t)nb, sizeof(BlockQ8K));
    quantize_row_fp16_to_q8_k((const __fp16 *)x, y, k);
    for (int b = 0; b < nb; ++b) {
        d[b] = y[b].d;
        memcpy(qs + (size_t)b * 256, y[b].qs, 256);
        memcpy(bsum32 + (size_t)b * 8, y[b].bsum32, 8 * sizeof(int32_t));
    }
    free(y);
}

/* quantize_row_fp16_to_q8_0 (E:1016-1064). */
void ref_quantize_row_q8_0(const uint16_t *x, int k, float *d, int8_t *qs) {
    const int nb = k / 32;
    BlockQ8_0_Fast *y = (BlockQ8_0_Fast *)calloc((size_t)nb, sizeof(BlockQ8_0_Fast));
    quantize_row_fp16_to_q8_0((const __fp16 *)x, y, k);
    for (int b = 0; b < nb; ++b) {
        d[b] = y[b].d;
        memcpy(qs + (size_t)b * 32, y[b].qs, 32);
    }
    free(y);
}

int ref_capacity_k(void) { return SDOT_MAX_K; }
int ref_capacity_m(void) { return SDOT_MAX_BATCH; }

static void fill_q8k(QuantizedBatchInput *Q, int M, int K, const float *d, const int8_t *qs,
                     const int32_t *bsum32) {
    const int nb = K / 256;
    for (int m = 0; m < M; ++m)
        for (int b = 0; b < nb; ++b) {
            Q->q8k[m][b].d = d[(size_t)m * nb + b];
            memcpy(Q->q8k[m][b].qs, qs + (size_t)m * K + (size_t)b * 256, 256);
            memcpy(Q->q8k[m][b].bsum32, bsum32 + ((size_t)m * nb + b) * 8, 32);
        }
}

static void fill_q80(QuantizedBatchInput *Q, int M, int K, const float *d, const int8_t *qs) {
    const int nb = K / 32;
    for (int m = 0; m < M; ++m)
        for (int b = 0; b < nb; ++b) {
            Q->q80[m][b].d = d[(size_t)m * nb + b];
            memcpy(Q->q80[m][b].qs, qs + (size_t)m * K + (size_t)b * 32, 32);
        }
}

/* Row dots for M activation rows of one weight row, using
 *  - eval_single_lm_row_dot (E:10986-11105) for Q4_K / Q5_K / Q6_K when
 *    use_batch_kernel == 0,
 *  - sdot_row_q5_k_batch / sdot_row_q6_k_batch / sdot_row_q8_0_batch
 *    (E:3109-3408, scalar branches) when use_batch_kernel != 0.
 * Q8_K activations: d[M][K/256], qs[M][K], bsum32[M][K/32].
 * Q8_0 activations: d[M][K/32], qs[M][K] (bsum32 ignored).
 * Returns -1 outside the reference's static capacity (M <= 32, K <= 9216). */
int ref_dot_rows(uint32_t type, const uint8_t *w_row, int M, int K, const float *d,
                 const int8_t *qs, const int32_t *bsum32, int use_batch_kernel, float *out) {
    if (M < 1 || M > SDOT_MAX_BATCH || K > SDOT_MAX_K) return -1;
    QuantizedBatchInput *Q = (QuantizedBatchInput *)calloc(1, sizeof(QuantizedBatchInput));
    if (!Q) return -1;
    Q->M = M;
    Q->K = K;
    int rc = 0;
    if (type == GGML_TYPE_Q8_0) {
        fill_q80(Q, M, K, d, qs);
        sdot_row_q8_0_batch(w_row, Q, M, K, out);
    } else if (type == GGML_TYPE_Q4_K || type == GGML_TYPE_Q5_K || type == GGML_TYPE_Q6_K) {
        fill_q8k(Q, M, K, d, qs, bsum32);
        if (use_batch_kernel && type == GGML_TYPE_Q5_K) {
            sdot_row_q5_k_batch(w_row, Q, M, K, out);
        } else if (use_batch_kernel && type == GGML_TYPE_Q6_K) {
            sdot_row_q6_k_batch(w_row, Q, M, K, out);
        } else {
            const size_t rb = ggml_row_bytes(type, (size_t)K);
            for (int m = 0; m < M; ++m)
                out[m] = eval_single_lm_row_dot(w_row, type, rb, 0, Q, m, K);
        }
    } else {
        rc = -1;
    }
    free(Q);
    return rc;
}

/* sdot_row_f32_batch / sdot_row_f16_batch (E:3410-3440): one F32 / F16
 * weight row against M fp16 activation rows x16 [M][K] (the dispatcher's
 * x_fp16, E:4206), the row the dispatcher selects at E:3597-3601. */
int ref_dot_rows_float(uint32_t type, const uint8_t *w_row, int M, int K, const uint16_t *x16,
                       float *out) {
    if (M < 1 || M > SDOT_MAX_BATCH) return -1;
    if (type != GGML_TYPE_F32 && type != GGML_TYPE_F16) return -1;
    QuantizedBatchInput *Q = (QuantizedBatchInput *)calloc(1, sizeof(QuantizedBatchInput));
    if (!Q) return -1;
    Q->M = M;
    Q->K = K;
    Q->x_fp16 = (const __fp16 *)x16;
    if (type == GGML_TYPE_F32) sdot_row_f32_batch(w_row, Q, M, K, out);
    else sdot_row_f16_batch(w_row, Q, M, K, out);
    free(Q);
    return 0;
}

/* dequant_contiguous_fast (E:3856-3902) over n_elems values, on the calling
 * thread: the turbo flag selects the serial branch (E:3867), since this
 * harness starts no worker pool. */
int ref_dequant_contiguous(uint32_t type, const uint8_t *src, size_t n_elems, uint16_t *dst) {
    const int saved = Pool.turbo_active;
    Pool.turbo_active = 1;
    dequant_contiguous_fast(src, (__fp16 *)dst, type, n_elems);
    Pool.turbo_active = saved;
    return 0;
}

/* swiglu_chunk_worker (E:4326-4359) on fp16 gate/up [M][N]: gate is
 * overwritten with fp16(silu(g)*u) and the per-256 Q8_K requant (written by
 * the reference into g_sdot_input.q8k) is copied out. */
int ref_swiglu_q8k(uint16_t *gate_inout, const uint16_t *up, int M, int N, float *d,
                   int8_t *qs, int32_t *bsum32) {
    if (M < 1 || M > SDOT_MAX_BATCH || N % 256 || N > SDOT_MAX_K) return -1;
    const int nb = N / 256;
    g_swiglu_work.gate_inout = (__fp16 *)gate_inout;
    g_swiglu_work.up_in = (const __fp16 *)up;
    g_swiglu_work.M = M;
    g_swiglu_work.N = N;
    g_swiglu_work.blocks_per_row = nb;
    g_swiglu_work.total_blocks = M * nb;
    g_swiglu_work.blocks_per_worker = M * nb;
    swiglu_chunk_worker(0);
    for (int m = 0; m < M; ++m)
        for (int b = 0; b < nb; ++b) {
            d[(size_t)m * nb + b] = g_sdot_input.q8k[m][b].d;
            memcpy(qs + (size_t)m * N + (size_t)b * 256, g_sdot_input.q8k[m][b].qs, 256);
            memcpy(bsum32 + ((size_t)m * nb + b) * 8, g_sdot_input.q8k[m][b].bsum32, 32);
        }
    return 0;
}

/* rmsnorm_fp16_rows_fast (E:4264-4314), scalar branch under this build:
 * y rows out, and the Q8_K rows it leaves in g_sdot_input.q8k copied out. */
int ref_rmsnorm_q8k(const uint16_t *x, const uint16_t *gamma, uint16_t *y, int M, int K,
                    float *d, int8_t *qs, int32_t *bsum32) {
    if (M < 1 || M > SDOT_MAX_BATCH || K % 256 || K > SDOT_MAX_K) return -1;
    const int nb = K / 256;
    rmsnorm_fp16_rows_fast((const __fp16 *)x, (const __fp16 *)gamma, (__fp16 *)y, M, K);
    for (int m = 0; m < M; ++m)
        for (int b = 0; b < nb; ++b) {
            d[(size_t)m * nb + b] = g_sdot_input.q8k[m][b].d;
            memcpy(qs + (size_t)m * K + (size_t)b * 256, g_sdot_input.q8k[m][b].qs, 256);
            memcpy(bsum32 + ((size_t)m * nb + b) * 8, g_sdot_input.q8k[m][b].bsum32, 32);
        }
    return 0;
}

/* parse_gguf_file (E:376-413) on an in-memory file: the header values and
 * the tensor table (up to cap entries) copied out. Returns the tensor count,
 * or -1 where the reference rejects the file. */
int ref_gguf_parse(const uint8_t *buf, size_t size, uint64_t *alignment, uint64_t *data_offset,
                   char *names, uint32_t *n_dims, uint64_t *dims, uint32_t *types, uint64_t *rel,
                   uint64_t *abs_off, uint64_t *n_elems, uint64_t *byte_size, int cap) {
    static GgufContext g;
    memset(&g, 0, sizeof(g));
    g.base = buf;
    g.file_size = size;
    g.pos = 0;
    const int ok = parse_gguf_file(&g);
    free(g.vocab_ptrs);
    free(g.vocab_lens);
    if (!ok) return -1;
    *alignment = g.alignment;
    *data_offset = g.data_offset;
    for (int i = 0; i < (int)g.n_tensors && i < cap; ++i) {
        const GgufTensorInfo *t = &g.tensors[i];
        memcpy(names + (size_t)i * 128, t->name, 128);
        n_dims[i] = t->n_dims;
        for (int d = 0; d < 4; ++d) dims[(size_t)i * 4 + d] = t->dims[d];
        types[i] = t->type;
        rel[i] = t->rel_offset;
        abs_off[i] = t->abs_offset;
        n_elems[i] = t->n_elems;
        byte_size[i] = t->byte_size;
    }
    return (int)g.n_tensors;
}

/* ---------------------------------------------------------------------------
 * CPU baseline: the reference's portable batch-1 path for one projection —
 * quantize_row_fp16_to_q8_k of x once, then eval_single_lm_row_dot per
 * weight row — with rows split over `threads` pthreads in grains of
 * SDOT_ROW_GRAIN rows (the reference's row grain, E:866). Runs `iters`
 * passes, pass i on weight replica i mod replicas (replicas copies of the
 * tensor, `stride` bytes apart, so that the weights stream from DRAM rather
 * than the last-level cache), and returns the wall time in seconds
 * (CLOCK_MONOTONIC).
 * ------------------------------------------------------------------------- */
typedef struct {
    const uint8_t *w;
    uint32_t type;
    size_t row_bytes;
    int N, K;
    const QuantizedBatchInput *Q;
    float *y;
    int *cursor;
} BenchShared;

static void *bench_worker(void *arg) {
    BenchShared *s = (BenchShared *)arg;
    for (;;) {
        int r0 = __atomic_fetch_add(s->cursor, SDOT_ROW_GRAIN, __ATOMIC_RELAXED);
        if (r0 >= s->N) break;
        int r1 = r0 + SDOT_ROW_GRAIN;
        if (r1 > s->N) r1 = s->N;
        for (int r = r0; r < r1; ++r)
            s->y[r] = eval_single_lm_row_dot(s->w, s->type, s->row_bytes, (uint32_t)r, s->Q, 0, s->K);
    }
    return NULL;
}

double ref_bench_gemv(uint32_t type, const uint8_t *w, int N, int K, const uint16_t *x_f16,
                      float *y, int threads, int iters, int replicas, size_t stride) {
    if (threads < 1 || threads > 256 || K > SDOT_MAX_K || K % 256 || replicas < 1) return -1.0;
    if (type != GGML_TYPE_Q4_K && type != GGML_TYPE_Q5_K && type != GGML_TYPE_Q6_K) return -1.0;
    QuantizedBatchInput *Q = (QuantizedBatchInput *)calloc(1, sizeof(QuantizedBatchInput));
    if (!Q) return -1.0;
    pthread_t tid[256];
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    for (int it = 0; it < iters; ++it) {
        quantize_row_fp16_to_q8_k((const __fp16 *)x_f16, Q->q8k[0], K);
        Q->M = 1;
        Q->K = K;
        int cursor = 0;
        BenchShared s = {w + (size_t)(it % replicas) * stride, type, ggml_row_bytes(type, (size_t)K), N, K, Q, y,
                         &cursor};
        for (int t = 1; t < threads; ++t) pthread_create(&tid[t], NULL, bench_worker, &s);
        bench_worker(&s);
        for (int t = 1; t < threads; ++t) pthread_join(tid[t], NULL);
    }
    clock_gettime(CLOCK_MONOTONIC, &t1);
    free(Q);
    return (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
}
