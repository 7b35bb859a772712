/*
 * qmm_hip.h — C ABI of the MI355X (gfx950) quantized-weight matmul library.
 *
 * It replaces the quantized CPU compute layer of the reference engine
 * (src/v182_r22_breakthrough_engine.c, cited E:<line>): GGUF-packed
 * Q4_K / Q5_K / Q6_K / Q8_0 weight rows stay in their native block layout in
 * HBM, fp32 activations go in, fp32 outputs come out. Plain C types only:
 * device buffers are `void *` / typed pointers obtained from qmm_malloc (or
 * any HIP allocation on the same device), streams are `void *` hipStream_t.
 *
 * All compute entry points are asynchronous on the context's stream and
 * return a status code (QMM_OK or a QMM_E* value); none fails silently. A
 * context is not thread-safe: use one context per host thread.
 *
 * Numeric contract (fp32 boundary over the reference's fp16 one):
 *  - activations: each fp32 value is rounded to fp16 (round to nearest even)
 *    and then quantized exactly as quantize_row_fp16_to_q8_k (E:925-990) /
 *    quantize_row_fp16_to_q8_0 (E:1016-1064). Inputs must be finite with
 *    |x| < 65520 (the fp16 range).
 *  - dots: exact int32 per block, then the reference's fp32 expression per
 *    block, blocks accumulated in order (eval_single_lm_row_dot
 *    E:10986-11105, sdot_row_q*_batch E:3109-3408); outputs are the fp32
 *    sums the reference casts to fp16 at E:3582-3613.
 *  - F32 / F16 weight rows (sdot_row_f32_batch / _f16_batch, E:3410-3440)
 *    are dotted with the fp16-rounded input in fp32; their sums are added in
 *    a fixed parallel order, not the reference's row order, so they match it
 *    to the stated tolerance (max|d| / max|ref| <= 1e-3), not bit for bit.
 *    Their K must be a multiple of 32 and their rows 16-B aligned.
 */
#ifndef QMM_HIP_H
#define QMM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- status */
#define QMM_OK 0
#define QMM_EINVAL 1  /* null pointer, non-positive size, bad stride */
#define QMM_ETYPE 2   /* ggml type not supported by this path */
#define QMM_ESHAPE 3  /* K not a multiple of the block size, cols != K, ... */
#define QMM_EHIP 4    /* HIP runtime error (message in qmm_last_error) */
#define QMM_ENOMEM 5  /* device allocation failed */
#define QMM_EALIGN 6  /* device pointer misaligned for its format */
#define QMM_ENOTFOUND 7  /* no GGUF tensor of that name */

/* ggml type ids (E:115-120) */
#define QMM_TYPE_F32 0
#define QMM_TYPE_F16 1
#define QMM_TYPE_Q8_0 8
#define QMM_TYPE_Q4_K 12
#define QMM_TYPE_Q5_K 13
#define QMM_TYPE_Q6_K 14

typedef struct qmm_context qmm_context;

/* Matrix task: SdotMatrixTask (E:888-899) with fp32 dst/residual and device
 * pointers. Row r of the task reads w_base + r * row_bytes; output token m,
 * row r goes to dst[m * dst_stride + r] (+ residual[m * res_stride + r]). */
typedef struct {
    const void *w_base;    /* device: rows x row_bytes of packed GGUF blocks */
    uint32_t type;         /* QMM_TYPE_* */
    size_t row_bytes;      /* must equal qmm_row_bytes(type, cols) */
    float *dst;            /* device fp32 [M][dst_stride] */
    size_t dst_stride;     /* >= rows */
    const float *residual; /* device fp32 [M][res_stride], or NULL */
    size_t res_stride;     /* >= rows when residual != NULL */
    int rows;
    int cols;              /* must equal the dispatch K */
    int start_row;         /* written by the dispatcher (concatenated row space) */
} qmm_matrix_task;

/* ------------------------------------------------------------- lifecycle */
/* New context on HIP device `device` with its own (default-priority) stream.
 * Replaces the engine's implicit global state (g_sdot_input E:901, the
 * thread pool E:3442-3855). */
int qmm_init(int device, qmm_context **out_ctx);
int qmm_destroy(qmm_context *ctx);
/* Use an external hipStream_t (NULL restores the context's own stream). */
int qmm_set_stream(qmm_context *ctx, void *hip_stream);
void *qmm_get_stream(qmm_context *ctx);
int qmm_synchronize(qmm_context *ctx);
/* Pre-size the internal activation buffers for M x K dispatches so that
 * later dispatches up to that size allocate nothing (graph capture: a
 * capture that would need a larger buffer fails with QMM_ENOMEM). While
 * instantiated graphs are alive, a call that needs a larger buffer gets a
 * new one and the old one is kept — the graphs go on using it — until the
 * last graph is destroyed (qmm_graph_destroy) or the context is. */
int qmm_reserve(qmm_context *ctx, int max_M, int max_K);
const char *qmm_status_string(int status);
const char *qmm_last_error(const qmm_context *ctx);
/* Device facts: compute units, HBM bytes, gfx arch name. */
int qmm_device_info(qmm_context *ctx, int *cu_count, size_t *hbm_bytes, char *arch,
                    size_t arch_len);

/* ---------------------------------------------------------------- sizes */
/* compute_ggml_bytes / ggml_row_bytes (E:364-374, E:3940-3942); 0 if the
 * type is unsupported or cols is not a multiple of its block size. */
size_t qmm_row_bytes(uint32_t type, int64_t cols);
/* Bytes of a device Q8_K activation buffer for M rows of K values
 * (BlockQ8K E:868-872 as arrays): qs int8[M][K] at 0, d f32[M][K/256] at
 * qmm_q8k_d_offset, bsum32 i32[M][K/32] at qmm_q8k_bsum_offset, and at
 * qmm_q8k_tile_offset the codes again in matrix-core operand order (no
 * counterpart in the reference; read by the M >= 2 kernels): for token tile
 * t (tokens 16t..16t+15), block j and 64-value chunk h, 1 KB at
 * ((t * K/256 + j) * 4 + h) * 1024 whose 16-B slot 16c + n holds token
 * 16t + n's codes at block offsets 64h + 8c..+7 then 64h + 32 + 8c..+7.
 * At qmm_q8k_h_offset: the fp16 values the codes were quantized from,
 * [M][K] (the reference keeps them as x_fp16 beside its quantized input,
 * E:879-886, and dots its F32 / F16 rows with them, E:3410-3440).
 * At qmm_q8k_bh_offset: the sums of 16 codes (the reference's bsums, E:870;
 * exact in fp16) as fp16 in matrix-core operand order (no counterpart; read
 * by the prefill kernels): for token tile t and block j, 512 B at
 * (t * K/256 + j) * 512 whose 8-B slot 16c + n holds token 16t + n's sums of
 * 16-value groups 4c..4c+3.
 * Every producer (qmm_quantize_q8k, qmm_swiglu_q8k, qmm_rmsnorm_q8k)
 * writes all six sections. */
size_t qmm_q8k_bytes(int M, int K);
size_t qmm_q8k_d_offset(int M, int K);
size_t qmm_q8k_bsum_offset(int M, int K);
size_t qmm_q8k_tile_offset(int M, int K);
size_t qmm_q8k_h_offset(int M, int K);
size_t qmm_q8k_bh_offset(int M, int K);
/* Q8_0 activations (BlockQ8_0_Fast E:874-877): qs int8[M][K] at 0,
 * d f32[M][K/32] at qmm_q8_0_d_offset. */
size_t qmm_q8_0_bytes(int M, int K);
size_t qmm_q8_0_d_offset(int M, int K);

/* --------------------------------------------------------------- memory */
int qmm_malloc(qmm_context *ctx, size_t bytes, void **dev_ptr); /* 256-B aligned */
int qmm_free(qmm_context *ctx, void *dev_ptr);
int qmm_memcpy_h2d(qmm_context *ctx, void *dst_dev, const void *src_host, size_t bytes);
int qmm_memcpy_d2h(qmm_context *ctx, void *dst_host, const void *src_dev, size_t bytes);
int qmm_memcpy_d2d(qmm_context *ctx, void *dst_dev, const void *src_dev, size_t bytes);

/* Weight residency: copy rows x qmm_row_bytes(type, cols) bytes of packed
 * GGUF blocks from host memory into a new HBM allocation, unchanged (the
 * reference reads them in place from the GGUF mmap, E:4174-4176, E:12377).
 * Free with qmm_free. */
int qmm_weight_upload(qmm_context *ctx, const void *host_blocks, uint32_t type, int64_t rows,
                      int64_t cols, void **dev_blocks);

/* ------------------------------------------------------------- quantize */
/* quantize_row_fp16_to_q8_k (E:925-990) on M rows of fp32 x [M][K]. */
int qmm_quantize_q8k(qmm_context *ctx, const float *x, int M, int K, void *q8k_out);
/* quantize_row_fp16_to_q8_0 (E:1016-1064). */
int qmm_quantize_q8_0(qmm_context *ctx, const float *x, int M, int K, void *q80_out);
/* swiglu_chunk_worker (E:4326-4359): h = silu(gate) * up in fp32, then the
 * Q8_K quantizer per 256 values; gate/up/h are [M][N]. h_out may be NULL. */
int qmm_swiglu_q8k(qmm_context *ctx, const float *gate, const float *up, int M, int N,
                   float *h_out, void *q8k_out);
/* The FFN block of one layer at batch 1 — the sdot path of E:8287-8296 at
 * M = 1: the {gate, up} task group on the input row (fp32 x, quantized to
 * Q8_K here, or a prequantized Q8_K row: give exactly one), h = silu(gate) *
 * up (swiglu_chunk_worker, E:4349-4357) into h_out (fp32 [N], may be NULL),
 * h's Q8_K, then the down task — its residual included — on that Q8_K.
 * gate and up: N x K, one type, outputs required (the reference keeps both);
 * down: cols = N, any type but Q8_0. N % 256 == 0. Results equal the three
 * steps run as separate calls (qmm_gemm_multi_dispatch, qmm_swiglu_q8k,
 * qmm_gemm_multi_dispatch_prequantized), bit for bit. Two launches where
 * they apply — gate/up Q4_K or Q5_K with K <= 3072 (SwiGLU in the gate/up
 * epilogue), down Q4_K or Q6_K with N <= 12288 on the batch-1 persistent
 * grid (h quantized in its prologue) — else the three steps as separate
 * launches. Uses the context's buffers: qmm_reserve(ctx, 1, N) sizes them
 * for graph capture. */
int qmm_ffn_block(qmm_context *ctx, const float *x, const void *q8k, int K, qmm_matrix_task *gate,
                  qmm_matrix_task *up, qmm_matrix_task *down, float *h_out);
/* The FFN block behind its input norm (E:8287-8296 after the block's
 * rmsnorm_fp16_rows_fast, E:4264-4314): qmm_rmsnorm_q8k of x [K] with gamma,
 * then qmm_ffn_block on that prequantized row, in one call with the same
 * outputs. Where the two-launch form applies the norm runs inside the
 * gate/up launch's activation fill (two launches in all); else the norm's
 * kernel, then the three steps. K % 256 == 0, K <= 16384; x and gamma 16-B
 * aligned. */
int qmm_ffn_block_rmsnorm(qmm_context *ctx, const float *x, const float *gamma, int K, qmm_matrix_task *gate,
                          qmm_matrix_task *up, qmm_matrix_task *down, float *h_out);
/* rmsnorm_fp16_rows_fast (E:4264-4314) with its Q8_K output (E:4303-4305,
 * the producer that sets the prequantized flag, E:4312): per row of x
 * [M][K], y = fp16(x * inv_rms * gamma), inv_rms = 1 / sqrt(mean(x^2) +
 * 1e-6), then the Q8_K quantizer of y; x and gamma are rounded to fp16
 * first. y_out [M][K] may be NULL. K % 256 == 0, K <= 16384. */
int qmm_rmsnorm_q8k(qmm_context *ctx, const float *x, const float *gamma, int M, int K,
                    float *y_out, void *q8k_out);

/* -------------------------------------------------------- LM-head epilogue */
/* One vocabulary chunk of the LM head (run_final_norm_and_lm_head_batch_sdot,
 * E:11150-11184): logits of rows [row_base, row_base + rows) of the tensor
 * (w_rows points at row row_base) for the M prequantized activation rows,
 * then, per token m, the reference's running argmax over the chunk's logits
 * rounded to fp16, in row order with a strictly greater test:
 * (best_val[m], best_id[m]) are read and updated in place (the caller seeds
 * them, e.g. -1e30 / 0, and chains chunks). logits_out [M][rows] receives the
 * fp32 sums, or may be NULL (library scratch). q80 is needed only for Q8_0. */
int qmm_lm_head_argmax(qmm_context *ctx, const void *q8k, const void *q80, int M, int K,
                       const void *w_rows, uint32_t type, int rows, uint32_t row_base,
                       float *logits_out, float *best_val, uint32_t *best_id);
/* Indexed rows (the pre-evaluated candidate / end-of-text rows, E:11141-11148,
 * and the extended-script row lists, exec_cyrillic_lm_work_item E:9473-9579):
 * the fp32 dots of rows row_ids[0..n_ids) (device array) of the tensor at
 * w_tensor (tensor_rows rows), and the running argmax over them in list
 * order, fp32 values, strictly greater; best_id receives row ids. An id at
 * or past tensor_rows is never read: its value is -1e30 (E:11150), so it
 * never replaces a seed of -1e30. vals_out [M][n_ids] may be NULL. */
int qmm_eval_rows_argmax(qmm_context *ctx, const void *q8k, const void *q80, int M, int K,
                         const void *w_tensor, int64_t tensor_rows, uint32_t type,
                         const uint32_t *row_ids, int n_ids, float *vals_out, float *best_val,
                         uint32_t *best_id);

/* The chunked vocabulary scan of run_final_norm_and_lm_head_batch_sdot
 * (E:11107-11262) after its RMSNorm, on the device with no host round trip
 * between chunks. */
typedef struct {
    int chunk_rows;          /* rows per vocabulary chunk (the engine's lm_chunk_rows) */
    const float *thresholds; /* host array: the scan stops after chunk c < n_thresholds when every
                                active position's best is >= thresholds[c] (chunk_thresh,
                                E:11245-11256); NULL / 0 = no early exit */
    int n_thresholds;
    int first_checkpoint;    /* first chunk that may end the scan: 0, or 6 where all 7 chunks are
                                required (g_require_full_7chunks, E:11254) */
    float prune_margin;      /* speculative pruning margin (1e-3f, E:11208) */
    /* A scan in several calls (zero-initialized fields: the whole scan in one call). This call
     * scans chunks [chunk_begin, chunk_end) (chunk_end 0: through the last chunk), so a caller can
     * stop after chunk 0, take the engine's host-side decisions, and continue: the script-gated
     * exit (E:9717-9733 at batch 1, E:11194-11241 batched) needs the token tables on the host
     * between chunk 0 and chunk 1. The call's last chunk always runs its step (argmax update,
     * pruning, its checkpoint test). */
    int chunk_begin;
    int chunk_end;
    int resume;              /* 0: a new scan (best_val / best_id / scan_state seeded as below);
                                nonzero: continue the scan whose best_val / best_id / scan_state
                                an earlier call left (same M, K, tensor, draft_ids): nothing is
                                seeded; pre_ids are evaluated for the active positions only
                                (the extended-script rows, E:11216-11225), then, with drafts,
                                the pruning rule is applied once (E:11226-11231) before the
                                chunks; a stopped scan stays stopped */
} qmm_lm_scan_params;
/* best_val / best_id [M] (device) are seeded with -1e30 / 0 (E:11139-11140);
 * then every position evaluates the rows pre_ids[0..n_pre) (device; the
 * end-of-text rows, E:11143-11146) and, when draft_ids (device [M]) is given,
 * position p < M - 1 its draft candidate draft_ids[p + 1] (-1e30 past the
 * vocabulary, E:11147-11153), fp32 values, strictly greater. Then the
 * vocab_rows rows are scanned in chunks (fp16-rounded logits, strict >,
 * E:11158-11183); after each chunk the first position p whose best is not
 * its draft candidate and beats the candidate's logit by more than the
 * margin ends the active batch at p + 1 (E:11203-11209: later positions are
 * no longer updated), and at a checkpoint the scan stops when every active
 * position's best reaches the chunk's threshold. A chunk after the stop
 * reads no weights. Chunks after which nothing is decided (no checkpoint,
 * no drafts to prune) share one launch with the chunks that follow them, up
 * to the next deciding chunk: the same results, fewer launches. At M = 1
 * with three or more such launches, the first runs alone and all later
 * chunks run as one launch that applies the first's decision before it
 * reads any weight, and whose last workgroup to finish decides the later
 * chunks in order from their bests: the same results (a stop after the first launch
 * reads nothing more; later checkpoints stop nothing in flight).
 * scan_state (device int32[4]) receives: chunks read,
 * active positions, 1 if the scan stopped early, 0. The script-specific
 * extended rows (E:11194-11240) are the caller's: qmm_eval_rows_argmax. */
int qmm_lm_head_scan(qmm_context *ctx, const void *q8k, const void *q80, int M, int K,
                     const void *w_lm, uint32_t type, int vocab_rows,
                     const qmm_lm_scan_params *params, const uint32_t *pre_ids, int n_pre,
                     const uint32_t *draft_ids, float *best_val, uint32_t *best_id,
                     int32_t *scan_state);

/* run_final_norm_and_lm_head_batch_sdot whole: its final RMSNorm of the rows
 * x [M][K] with gamma (rmsnorm_fp16_rows_fast, E:11129), then the scan above
 * on the normed rows — the pair qmm_rmsnorm_q8k + qmm_lm_head_scan in one
 * call, with the same results. At M = 1 with no pre_ids and every chunk
 * launch of a Q4_K / Q5_K / Q6_K tensor on the batch-1 persistent grid,
 * each chunk launch normalizes the row in its activation fill (no launch of
 * the norm's own); otherwise the norm's kernel writes the context's buffers
 * (and, for a Q8_0 tensor, the normed row's Q8_0) first. K % 256 == 0,
 * K <= 16384; x and gamma 16-B aligned. */
int qmm_lm_head_scan_rmsnorm(qmm_context *ctx, const float *x, const float *gamma, int M, int K,
                             const void *w_lm, uint32_t type, int vocab_rows,
                             const qmm_lm_scan_params *params, const uint32_t *pre_ids, int n_pre,
                             const uint32_t *draft_ids, float *best_val, uint32_t *best_id,
                             int32_t *scan_state);

/* -------------------------------------------------------------- dequant */
/* dequant_contiguous_fast (E:3856-3902): rows x cols packed blocks -> fp16
 * bits [rows][cols] (for validation; not on the matmul path). F16 rows are
 * copied, F32 values rounded to fp16 (E:3857-3860, E:3876-3879). */
int qmm_dequantize_f16(qmm_context *ctx, const void *w_blocks, uint32_t type, int64_t rows,
                       int64_t cols, uint16_t *dst);

/* ------------------------------------------------------------- dispatch */
/* sdot_gemm_multi_dispatch (E:4188-4262): quantize x [M][K] once (Q8_K for
 * K-quant tasks, Q8_0 for Q8_0 tasks) into the context's buffers, then run
 * every task on the shared quantized input. */
int qmm_gemm_multi_dispatch(qmm_context *ctx, const float *x, int M, int K,
                            qmm_matrix_task *tasks, int n_tasks);
/* The prequantized form (the engine's g_sdot_input_q8k_prequantized flag,
 * E:4186, E:4207-4208, made explicit): q8k / q80 are device buffers in the
 * layouts above; either may be NULL when no task needs it (F32 / F16 tasks
 * read the fp16 section of q8k). */
int qmm_gemm_multi_dispatch_prequantized(qmm_context *ctx, const void *q8k, const void *q80,
                                         int M, int K, qmm_matrix_task *tasks, int n_tasks);

/* The engine's normed projection: rmsnorm_fp16_rows_fast of x [M][K] with
 * gamma (E:4264-4314, the producer that sets the prequantized flag,
 * E:4303-4312), then sdot_gemm_multi_dispatch on that prequantized input
 * (E:4188-4262, E:4207-4208) — the pair qmm_rmsnorm_q8k +
 * qmm_gemm_multi_dispatch_prequantized in one call, with the same results.
 * At M = 1 with only Q4_K / Q5_K / Q6_K tasks on the batch-1 persistent grid
 * the norm runs inside each workgroup's activation fill (one launch);
 * otherwise the norm's kernel writes the context's buffers (and, for Q8_0
 * tasks, the normed row's Q8_0) and the tasks run on them. K % 256 == 0,
 * K <= 16384; x and gamma 16-B aligned. */
int qmm_gemm_multi_dispatch_rmsnorm(qmm_context *ctx, const float *x, const float *gamma, int M, int K,
                                    qmm_matrix_task *tasks, int n_tasks);

/* qmm_gemm_multi_dispatch that allocates nothing. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Results equal qmm_gemm_multi_dispatch's. At M >= 2 the quantized input
 * goes to a device array of qmm_noalloc_scratch_bytes() (32 MiB) that each
 * GPU holds from qmm_init to the end of the process; a call whose quantized
 * input is larger (qmm_q8k_bytes(M, K) for K-quant / F32 / F16 tasks, plus
 * qmm_q8_0_bytes(M, K) for Q8_0 tasks) fails with QMM_ESHAPE. All calls on
 * one GPU share that array, which keeps the last call's contents: calls that
 * overlap on one GPU (several contexts or streams at once) race. */
int qmm_gemm_multi_dispatch_noalloc(qmm_context *ctx, const float *x, int M, int K,
                                    qmm_matrix_task *tasks, int n_tasks);
size_t qmm_noalloc_scratch_bytes(void);

/* ---------------------------------------------------- graphs and timing */
/* Capture the context stream's work into a HIP graph (hipStreamBeginCapture
 * / hipGraphInstantiate) and replay it; for launch-bound loops. */
int qmm_graph_begin(qmm_context *ctx);
int qmm_graph_end(qmm_context *ctx, void **graph_exec);
int qmm_graph_launch(qmm_context *ctx, void *graph_exec);
/* Waits for the context's stream, then destroys the graph; buffers the
 * context replaced while graphs were alive are freed with the last one. */
int qmm_graph_destroy(qmm_context *ctx, void *graph_exec);
/* The HBM read floor (measurement only; no counterpart in the reference):
 * stream `bytes` from src (16-B aligned) with 16-B non-temporal loads over
 * `workgroups` workgroups of 4 waves, each wave holding loads_per_wave
 * (1, 2, 4 or 8) 1-KB loads in flight; one folded word per workgroup goes
 * to sink[workgroups]. */
int qmm_stream_read(qmm_context *ctx, const void *src, size_t bytes, int workgroups, int loads_per_wave,
                    uint32_t *sink);
/* HIP events on the context stream: begin records, end records and waits,
 * returning the elapsed milliseconds. */
int qmm_timer_begin(qmm_context *ctx);
int qmm_timer_end(qmm_context *ctx, float *ms);

/* ---------------------------------------------------------------- GGUF */
/* GGUF v2/v3 container, memory-mapped read-only (parse_gguf_file E:376-413,
 * GgufTensorInfo E:168-177, find_tensor E:415-420). Host code: needs no GPU.
 * Differences from the reference: tensor bytes outside the file are an
 * error (QMM_ESHAPE), and up to 65536 tensors are accepted (not 512). */
typedef struct qmm_gguf qmm_gguf;
typedef struct {
    char name[128];       /* truncated to 127 bytes, as the reference */
    uint32_t n_dims;      /* 1..4 */
    uint64_t dims[4];     /* dims[0] innermost (= cols of a matrix); unused dims 1 */
    uint32_t type;        /* ggml type id */
    uint64_t rel_offset;  /* from the data section */
    uint64_t abs_offset;  /* from the file start: data_offset + rel_offset */
    uint64_t n_elems;
    uint64_t byte_size;   /* compute_ggml_bytes (E:364-374); 0 for other types */
} qmm_gguf_tensor;

int qmm_gguf_open(const char *path, qmm_gguf **out);
int qmm_gguf_close(qmm_gguf *g);
/* version, alignment (general.alignment or 32), data section offset, tensor count */
int qmm_gguf_header(const qmm_gguf *g, uint32_t *version, uint64_t *alignment, uint64_t *data_offset,
                    int *n_tensors);
int qmm_gguf_tensor_at(const qmm_gguf *g, int i, qmm_gguf_tensor *out);
/* QMM_ENOTFOUND if absent */
int qmm_gguf_find_tensor(const qmm_gguf *g, const char *name, qmm_gguf_tensor *out);
/* host pointer to a tensor's bytes inside the mapping (valid until close) */
const void *qmm_gguf_data(const qmm_gguf *g, const qmm_gguf_tensor *t);
/* residency of one quantized matrix: qmm_weight_upload of its rows
 * (n_elems / dims[0]) x cols (dims[0]); the reference uses the mapped bytes
 * in place (w_base = ctx->base + t->abs_offset, E:4174) */
int qmm_gguf_upload(qmm_context *ctx, const qmm_gguf *g, const char *name, void **dev_blocks,
                    qmm_gguf_tensor *info);

#ifdef __cplusplus
}
#endif

#endif /* QMM_HIP_H */
