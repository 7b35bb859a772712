/*
 * qmm_oracle.h — CPU restatement of the reference engine's quantized-matmul
 * path, used ONLY as test infrastructure (it checks the HIP library's results
 * in the parity tests).  Nothing in the product links or calls
 * this code.
 *
 * Every function follows the scalar (non-NEON) branch of
 * src/v182_r22_breakthrough_engine.c (cited as E:<line>) loop for loop, with
 * the same floating-point operation order, so that when built with
 * -ffp-contract=off its results are bit-identical to the reference's scalar
 * code compiled the same way.
 *
 * fp16 values are passed as raw IEEE binary16 bit patterns (uint16_t): gcc on
 * x86 has no __fp16, so the conversions are restated in qo_fp16_to_f32 /
 * qo_f32_to_fp16 (round-to-nearest-even, as the reference's (__fp16) casts).
 *
 * Q8_K activations are kept as three arrays instead of the reference's
 * BlockQ8K struct (E:868-872):
 *   d[M][K/256] (float), qs[M][K] (int8), bsum32[M][K/32] (int32)
 * Q8_0 activations (BlockQ8_0_Fast, E:874-877):
 *   d[M][K/32] (float), qs[M][K] (int8)
 *
 * Pinning status of each function is listed in the header of qmm_oracle.c.
 */
#ifndef QMM_ORACLE_H
#define QMM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (E:115-120) */
#define QO_TYPE_F32 0
#define QO_TYPE_F16 1
#define QO_TYPE_Q8_0 8
#define QO_TYPE_Q4_K 12
#define QO_TYPE_Q5_K 13
#define QO_TYPE_Q6_K 14

/* fp16 <-> fp32 (E:592-596 and the (__fp16) casts) */
float qo_fp16_to_f32(uint16_t h);
uint16_t qo_f32_to_fp16(float f);
void qo_f32_to_fp16_array(const float *src, uint16_t *dst, size_t n);
void qo_fp16_to_f32_array(const uint16_t *src, float *dst, size_t n);

/* compute_ggml_bytes / ggml_row_bytes (E:364-374, E:3940-3942) */
uint64_t qo_row_bytes(uint32_t type, uint64_t cols);

/* get_scale_min_k4 (E:743-749) */
void qo_get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m);

/* block dequantizers -> fp16 bits (E:598-615, E:673-741, E:758-801, E:803-853) */
void qo_dequant_block_q8_0(const uint8_t *blk, uint16_t *dst);
void qo_dequant_block_q4_k(const uint8_t *blk, uint16_t *dst);
void qo_dequant_block_q5_k(const uint8_t *blk, uint16_t *dst);
void qo_dequant_block_q6_k(const uint8_t *blk, uint16_t *dst);
/* dequant_contiguous_fast over rows x cols (E:3856-3902). Returns 0 on success. */
int qo_dequant_rows(uint32_t type, const uint8_t *src, int64_t rows, int64_t cols,
                    uint16_t *dst);

/* quantize_row_fp16_to_q8_k (E:925-990) on one row of k fp16 values */
void qo_quantize_row_q8k_f16(const uint16_t *x, int k, float *d, int8_t *qs,
                             int32_t *bsum32);
/* quantize_row_fp16_to_q8_0 (E:1016-1064) */
void qo_quantize_row_q8_0_f16(const uint16_t *x, int k, float *d, int8_t *qs);
/* fp32 contract: round each value to fp16 (RNE) and apply the row quantizer.
 * x is [M][K] row-major. */
void qo_quantize_q8k_f32(const float *x, int M, int K, float *d, int8_t *qs,
                         int32_t *bsum32);
void qo_quantize_q8_0_f32(const float *x, int M, int K, float *d, int8_t *qs);

/* Row dot products of one packed weight row against one quantized activation
 * row (eval_single_lm_row_dot E:10986-11105; sdot_row_q5_k/q6_k/q8_0_batch
 * scalar branches E:3193-3230, E:3324-3364, E:3394-3406).
 * For the K-quants: dx = d[m], qs = qs[m], bsum32 = bsum32[m] of a Q8_K row.
 * For Q8_0: dx = the Q8_0 d row, bsum32 unused. */
float qo_dot_row(uint32_t type, const uint8_t *w_row, int K, const float *dx,
                 const int8_t *qs, const int32_t *bsum32);

/* sdot_row_f32_batch / sdot_row_f16_batch (E:3410-3440): one F32 / F16
 * weight row against one fp16 activation row x16 (bits), summed in row
 * order. */
float qo_dot_row_float(uint32_t type, const uint8_t *w_row, int K, const uint16_t *x16);

/* Per-block exact integer partials of a K-quant row dot:
 *   Q4_K/Q5_K: S[b] = sum_j sc_j * dot_j, Mb[b] = sum_j m_j * bsum32_j
 *   Q6_K:      S[b] = sum_s sc_s * dot_s, Mb[b] = 0
 *   Q8_0:      S[b] = dot over the 32-value block, Mb[b] = 0
 * Returns the number of blocks written. */
int qo_block_partials(uint32_t type, const uint8_t *w_row, int K,
                      const int8_t *qs, const int32_t *bsum32, int32_t *S,
                      int32_t *Mb);

/* Matrix task of the reference dispatcher (SdotMatrixTask, E:888-899), with
 * fp32 destination and residual. */
typedef struct {
    const uint8_t *w_base;
    uint32_t type;
    size_t row_bytes;
    float *dst;
    size_t dst_stride;
    const float *residual;
    size_t res_stride;
    int rows;
    int cols;
    int start_row;
} qo_matrix_task;

/* sdot_gemm_multi_dispatch (E:4188-4262) + exec_sdot_job_work_stealing
 * (E:3491-3619): quantize x [M][K] once (Q8_K and/or Q8_0), then for every
 * task row r and token m: dst[m*dst_stride + r] = dot (+ residual).
 * Returns 0, or -1 for an unsupported type / shape. Rows run in parallel
 * (OpenMP); each output is computed by one thread in reference order. */
int qo_gemm_multi(const float *x, int M, int K, qo_matrix_task *tasks, int n_tasks);
/* Same with caller-provided quantized activations (the prequantized path,
 * E:4186, E:4207-4208). q80_d / q80_qs may be NULL when no Q8_0 task; x16
 * (fp16 bits [M][K], the input the engine still passes, E:4206) may be NULL
 * when no F32 / F16 task. */
int qo_gemm_multi_prequantized(const float *q8k_d, const int8_t *q8k_qs,
                               const int32_t *q8k_bsum, const float *q80_d,
                               const int8_t *q80_qs, const uint16_t *x16, int M, int K,
                               qo_matrix_task *tasks, int n_tasks);

/* swiglu_chunk_worker (E:4326-4359) in the fp32 contract: g and u rounded
 * to fp16, h = (g / (1 + expf(-g))) * u in fp32, then the fp32->fp16->Q8_K
 * quantizer per 256-value block. gate/up/h are [M][N]; h may be NULL. */
void qo_swiglu_q8k(const float *gate, const float *up, int M, int N, float *h,
                   float *d, int8_t *qs, int32_t *bsum32);

/* Running argmax over one chunk of logits [M][ldl] (E:11172-11183): row
 * order, fp16-rounded values when round16, strict >; best_* updated in place. */
void qo_chunk_argmax(const float *logits, int M, int rows, size_t ldl, int round16, const uint32_t *ids,
                     uint32_t row_base, float *best_val, uint32_t *best_id);

/* run_final_norm_and_lm_head_batch_sdot's scan after its RMSNorm
 * (E:11138-11256), script-specific rows left out: pre-evaluated rows and
 * draft candidates (fp32), chunks of fp16-rounded logits (strict >), the
 * speculative pruning and the checkpoint thresholds. x* are the Q8_K (or,
 * for Q8_0 weights, Q8_0) activation arrays of M rows; xbs may be NULL for
 * Q8_0. Returns the chunks read (-1 on bad arguments). */
int qo_lm_head_scan(uint32_t type, const uint8_t *w, int vocab_rows, int K, int M, const float *xd,
                    const int8_t *xqs, const int32_t *xbs, int chunk_rows, const float *thresholds,
                    int n_thresholds, int first_checkpoint, float margin, const uint32_t *pre_ids, int n_pre,
                    const uint32_t *draft_ids, float *best_val, uint32_t *best_id, int *active_out,
                    int *stopped_out);

/* The extended-script state of the LM head (E:9690-9733, E:11185-11241):
 * the tokenizer's per-token script flags, each script's extended row list,
 * and the session's sticky flags (read, then updated). */
typedef struct {
    const uint8_t *is_cyr;    /* g_token_is_cyrillic [vocab_rows] */
    const uint8_t *is_cjk;    /* g_token_is_cjk [vocab_rows] */
    const uint32_t *cyr_rows; /* the Cyrillic extended rows, evaluation order */
    int n_cyr;
    const uint32_t *cjk_rows; /* the CJK extended rows */
    int n_cjk;
    int has_cyr, has_cjk;     /* g_session_has_cyrillic / _cjk: in and out */
    int require_full;         /* g_require_full_7chunks: checkpoints from chunk 6, no script exit */
    int batch1;               /* 1: run_final_norm_and_lm_head_pipelined's rule (M = 1, E:9717-9733);
                                 0: run_final_norm_and_lm_head_batch_sdot's (E:11194-11241) */
} qo_script;

/* The whole LM-head scan with its script-gated exit: qo_lm_head_scan's
 * chunk loop (thresholds present stand for the engine's 24832-row
 * chunking: checkpoints at every chunk, from chunk 6 with require_full),
 * plus after each chunk the session flags from the active positions' best
 * tokens, and after chunk 0, when a script is active, its extended rows
 * for the active positions (fp32 values, list order, strict >), then the
 * script exit: batch1, the running best >= 10.5; batched, the pruning
 * again and every active best >= 11.5 when its token is of an active
 * script, else >= 20.0. The batch-1 rule has no pre rows and no drafts
 * (pass none). Returns the chunks read (-1 on bad arguments). */
int qo_lm_head_scan_script(uint32_t type, const uint8_t *w, int vocab_rows, int K, int M, const float *xd,
                           const int8_t *xqs, const int32_t *xbs, int chunk_rows, const float *thresholds,
                           int n_thresholds, float margin, const uint32_t *pre_ids, int n_pre,
                           const uint32_t *draft_ids, qo_script *sc, float *best_val, uint32_t *best_id,
                           int *active_out, int *stopped_out);

/* rmsnorm_fp16_rows_fast (E:4264-4314), scalar branch, on fp16 bits:
 * y [M][K] fp16 bits, then the Q8_K of each y row. K % 256 == 0. */
void qo_rmsnorm_q8k_f16(const uint16_t *x, const uint16_t *gamma, int M, int K, uint16_t *y,
                        float *d, int8_t *qs, int32_t *bsum32);

#ifdef __cplusplus
}
#endif

#endif /* QMM_ORACLE_H */
