/*
 * qmm_oracle.c — CPU restatement of the reference engine's quantized-matmul
 * path.  TEST INFRASTRUCTURE ONLY: the parity tests, the smoke check and the
 * CPU-baseline leg of the benchmark use it to check results; the HIP library
 * never links or calls it.
 *
 * Source followed: src/v182_r22_breakthrough_engine.c (E:<line>), scalar
 * (#else) branches.  Build with -ffp-contract=off so every fp32 operation is
 * rounded exactly where the reference's C source rounds it.
 *
 * How each function is pinned (tests/test_oracle_*.py):
 *   qo_fp16_to_f32 / qo_f32_to_fp16  exhaustive/boundary sweep vs numpy's
 *                                    IEEE float16 conversion, and vs the
 *                                    compiled reference's (__fp16) casts.
 *   qo_get_scale_min_k4, qo_dequant_* golden vectors from the compiled
 *                                    reference + closed-form numpy dequant
 *                                    + special cases (d=0, sc=0, m=63, all
 *                                    code values).
 *   qo_quantize_*                    golden vectors + invariants (|q|<=127,
 *                                    bsum = sum of codes, zero block, single
 *                                    non-zero, RNE ties).
 *   qo_dot_row / qo_block_partials   golden vectors (bit-exact), brute force
 *                                    fp64 sum of dequant(w)*dx*q on tiny K,
 *                                    integer reduction with unit scales.
 *   qo_gemm_multi                    task/row/residual semantics vs per-row
 *                                    qo_dot_row, and vs the compiled
 *                                    reference's dot functions.
 *   qo_swiglu_q8k                    composition: h vs numpy fp64 SiLU*up
 *                                    (tolerance; expf differs between libms),
 *                                    codes vs qo_quantize_q8k_f32(h).
 *   qo_chunk_argmax                  vs a first-maximum / strict-update
 *                                    restatement in numpy on planted ties,
 *                                    NaNs and values equal to the seed.
 *   qo_rmsnorm_q8k_f16               bit-exact vs the compiled reference's
 *                                    rmsnorm_fp16_rows_fast (y and Q8_K);
 *                                    closed forms (constant rows, unit gamma)
 *                                    and fp64 RMS within fp16 rounding.
 */
#include "qmm_oracle.h"

#include <math.h>
#include <string.h>

/* ---------------------------------------------------------------- fp16 -- */

/* (float)(__fp16)bits, E:592-596: exact widening. */
float qo_fp16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    const uint32_t mant = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            /* subnormal: mant * 2^-24, exact in fp32 */
            float v = (float)mant * 5.9604644775390625e-8f;
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (mant << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

/* (__fp16)f: IEEE binary32 -> binary16, round to nearest, ties to even. */
uint16_t qo_f32_to_fp16(float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const uint32_t abs = bits & 0x7fffffffu;
    if (abs > 0x7f800000u) {                 /* NaN: keep it quiet */
        return (uint16_t)(sign | 0x7e00u | ((abs >> 13) & 0x3ffu));
    }
    if (abs >= 0x477ff000u) {                /* >= 65520 rounds to inf */
        return (uint16_t)(sign | 0x7c00u);
    }
    const uint32_t exp = abs >> 23;
    if (exp < 113) {                          /* below 2^-14: subnormal half */
        if (exp < 102) return (uint16_t)sign; /* below 2^-25: rounds to 0 */
        const uint32_t mant = (abs & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - exp;    /* units of 2^-24 */
        uint32_t r = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((exp - 112u) << 10) | ((abs & 0x7fffffu) >> 13);
    const uint32_t rem = abs & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

void qo_f32_to_fp16_array(const float *src, uint16_t *dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = qo_f32_to_fp16(src[i]);
}

void qo_fp16_to_f32_array(const uint16_t *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = qo_fp16_to_f32(src[i]);
}

static inline uint16_t rd16(const uint8_t *p) {
    uint16_t v;
    memcpy(&v, p, 2);
    return v;
}

/* ------------------------------------------------------------ formats -- */

/* compute_ggml_bytes, E:364-374 */
uint64_t qo_row_bytes(uint32_t type, uint64_t cols) {
    switch (type) {
        case QO_TYPE_F32: return cols * 4ull;
        case QO_TYPE_F16: return cols * 2ull;
        case QO_TYPE_Q8_0: return (cols / 32ull) * 34ull;
        case QO_TYPE_Q4_K: return (cols / 256ull) * 144ull;
        case QO_TYPE_Q5_K: return (cols / 256ull) * 176ull;
        case QO_TYPE_Q6_K: return (cols / 256ull) * 210ull;
        default: return 0;
    }
}

/* get_scale_min_k4, E:743-749 */
void qo_get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* ------------------------------------------------------------ dequant -- */

/* dequant_block_q8_0, scalar branch E:613 */
void qo_dequant_block_q8_0(const uint8_t *blk, uint16_t *dst) {
    const float d = qo_fp16_to_f32(rd16(blk));
    const int8_t *qs = (const int8_t *)(blk + 2);
    for (int i = 0; i < 32; ++i) dst[i] = qo_f32_to_fp16(d * (float)qs[i]);
}

/* dequant_block_q6_k, scalar branch E:712-740 */
void qo_dequant_block_q6_k(const uint8_t *blk, uint16_t *dst) {
    const uint8_t *ql = blk;
    const uint8_t *qh = blk + 128;
    const int8_t *sc = (const int8_t *)(blk + 192);
    const float d = qo_fp16_to_f32(rd16(blk + 208));
    for (int half = 0; half < 2; ++half) {
        const uint8_t *ql_p = ql + half * 64;
        const uint8_t *qh_p = qh + half * 32;
        const int8_t *sc_p = sc + half * 8;
        uint16_t *y = dst + half * 128;
        for (int is = 0; is < 2; ++is) {
            const float d_sc0 = d * (float)sc_p[is + 0];
            const float d_sc2 = d * (float)sc_p[is + 2];
            const float d_sc4 = d * (float)sc_p[is + 4];
            const float d_sc6 = d * (float)sc_p[is + 6];
            const int l_base = is * 16;
            for (int l = l_base; l < l_base + 16; ++l) {
                const uint8_t ql0 = ql_p[l], ql1 = ql_p[l + 32], qh0 = qh_p[l];
                const int q1 = (int)((ql0 & 0x0F) | (((qh0 >> 0) & 3) << 4)) - 32;
                const int q2 = (int)((ql1 & 0x0F) | (((qh0 >> 2) & 3) << 4)) - 32;
                const int q3 = (int)((ql0 >> 4) | (((qh0 >> 4) & 3) << 4)) - 32;
                const int q4 = (int)((ql1 >> 4) | (((qh0 >> 6) & 3) << 4)) - 32;
                y[l + 0] = qo_f32_to_fp16(d_sc0 * (float)q1);
                y[l + 32] = qo_f32_to_fp16(d_sc2 * (float)q2);
                y[l + 64] = qo_f32_to_fp16(d_sc4 * (float)q3);
                y[l + 96] = qo_f32_to_fp16(d_sc6 * (float)q4);
            }
        }
    }
}

/* dequant_block_q4_k, scalar branch E:786-800 */
void qo_dequant_block_q4_k(const uint8_t *blk, uint16_t *dst) {
    const float d = qo_fp16_to_f32(rd16(blk));
    const float min = qo_fp16_to_f32(rd16(blk + 2));
    const uint8_t *scales = blk + 4;
    const uint8_t *q = blk + 16;
    int is = 0;
    for (int j = 0; j < 256; j += 64) {
        uint8_t sc, m;
        qo_get_scale_min_k4(is + 0, scales, &sc, &m);
        const float d1 = d * (float)sc, m1 = min * (float)m;
        qo_get_scale_min_k4(is + 1, scales, &sc, &m);
        const float d2 = d * (float)sc, m2 = min * (float)m;
        for (int l = 0; l < 32; ++l) {
            const uint8_t q_v = q[l];
            dst[j + l] = qo_f32_to_fp16(d1 * (float)(q_v & 0x0F) - m1);
            dst[j + 32 + l] = qo_f32_to_fp16(d2 * (float)(q_v >> 4) - m2);
        }
        q += 32;
        is += 2;
    }
}

/* dequant_block_q5_k, scalar branch E:837-852 */
void qo_dequant_block_q5_k(const uint8_t *blk, uint16_t *dst) {
    const float d = qo_fp16_to_f32(rd16(blk));
    const float min = qo_fp16_to_f32(rd16(blk + 2));
    const uint8_t *scales = blk + 4;
    const uint8_t *qh = blk + 16;
    const uint8_t *ql = blk + 48;
    int is = 0;
    uint8_t u1 = 1, u2 = 2;
    for (int j = 0; j < 256; j += 64) {
        uint8_t sc, m;
        qo_get_scale_min_k4(is + 0, scales, &sc, &m);
        const float d1 = d * (float)sc, m1 = min * (float)m;
        qo_get_scale_min_k4(is + 1, scales, &sc, &m);
        const float d2 = d * (float)sc, m2 = min * (float)m;
        for (int l = 0; l < 32; ++l) {
            const uint8_t ql_v = ql[l], qh_v = qh[l];
            dst[j + l] = qo_f32_to_fp16(d1 * (float)((ql_v & 0x0F) + ((qh_v & u1) ? 16 : 0)) - m1);
            dst[j + 32 + l] = qo_f32_to_fp16(d2 * (float)((ql_v >> 4) + ((qh_v & u2) ? 16 : 0)) - m2);
        }
        ql += 32;
        is += 2;
        u1 <<= 2;
        u2 <<= 2;
    }
}

/* dequant_contiguous_fast, E:3856-3902 (single-threaded here): F16 rows are
 * copied (E:3857-3860), F32 values cast to fp16 (E:3876-3879). */
int qo_dequant_rows(uint32_t type, const uint8_t *src, int64_t rows, int64_t cols,
                    uint16_t *dst) {
    if (type == QO_TYPE_F16 || type == QO_TYPE_F32) {
        if (cols <= 0 || rows < 0) return -1;
        const size_t n = (size_t)rows * (size_t)cols;
        if (type == QO_TYPE_F16) {
            memcpy(dst, src, n * 2);
        } else {
            for (size_t i = 0; i < n; ++i) {
                float f;
                memcpy(&f, src + 4 * i, 4);
                dst[i] = qo_f32_to_fp16(f);
            }
        }
        return 0;
    }
    const int64_t qk = (type == QO_TYPE_Q8_0) ? 32 : 256;
    if (cols <= 0 || rows < 0 || cols % qk) return -1;
    const uint64_t bbytes = qo_row_bytes(type, (uint64_t)qk);
    if (bbytes == 0) return -1;
    const int64_t units = rows * (cols / qk);
    for (int64_t b = 0; b < units; ++b) {
        const uint8_t *blk = src + (size_t)b * bbytes;
        uint16_t *y = dst + (size_t)b * (size_t)qk;
        switch (type) {
            case QO_TYPE_Q8_0: qo_dequant_block_q8_0(blk, y); break;
            case QO_TYPE_Q4_K: qo_dequant_block_q4_k(blk, y); break;
            case QO_TYPE_Q5_K: qo_dequant_block_q5_k(blk, y); break;
            case QO_TYPE_Q6_K: qo_dequant_block_q6_k(blk, y); break;
        }
    }
    return 0;
}

/* ---------------------------------------------------------- quantizer -- */

/* quantize_row_fp16_to_q8_k, scalar branches E:941-946 and E:976-988 */
void qo_quantize_row_q8k_f16(const uint16_t *x, int k, float *d, int8_t *qs,
                             int32_t *bsum32) {
    const int nb = k / 256;
    for (int b = 0; b < nb; ++b) {
        const uint16_t *xb = x + (size_t)b * 256;
        float max_abs = 0.0f;
        for (int i = 0; i < 256; ++i) {
            const float v = fabsf(qo_fp16_to_f32(xb[i]));
            if (v > max_abs) max_abs = v;
        }
        int8_t *qb = qs + (size_t)b * 256;
        int32_t *sb = bsum32 + (size_t)b * 8;
        if (max_abs == 0.0f) {
            d[b] = 0.0f;
            memset(qb, 0, 256);
            memset(sb, 0, 8 * sizeof(int32_t));
            continue;
        }
        d[b] = max_abs / 127.0f;
        const float id = 127.0f / max_abs;
        for (int s = 0; s < 8; ++s) {
            int32_t bsum = 0;
            for (int l = 0; l < 32; ++l) {
                int q = (int)lrintf(qo_fp16_to_f32(xb[s * 32 + l]) * id);
                if (q > 127) q = 127;
                if (q < -127) q = -127;
                qb[s * 32 + l] = (int8_t)q;
                bsum += q;
            }
            sb[s] = bsum;
        }
    }
}

/* quantize_row_fp16_to_q8_0, scalar branches E:1030-1035 and E:1056-1062 */
void qo_quantize_row_q8_0_f16(const uint16_t *x, int k, float *d, int8_t *qs) {
    const int nb = k / 32;
    for (int b = 0; b < nb; ++b) {
        const uint16_t *xb = x + (size_t)b * 32;
        float max_abs = 0.0f;
        for (int i = 0; i < 32; ++i) {
            const float v = fabsf(qo_fp16_to_f32(xb[i]));
            if (v > max_abs) max_abs = v;
        }
        int8_t *qb = qs + (size_t)b * 32;
        if (max_abs == 0.0f) {
            d[b] = 0.0f;
            memset(qb, 0, 32);
            continue;
        }
        d[b] = max_abs / 127.0f;
        const float id = 127.0f / max_abs;
        for (int l = 0; l < 32; ++l) {
            int q = (int)lrintf(qo_fp16_to_f32(xb[l]) * id);
            if (q > 127) q = 127;
            if (q < -127) q = -127;
            qb[l] = (int8_t)q;
        }
    }
}

void qo_quantize_q8k_f32(const float *x, int M, int K, float *d, int8_t *qs,
                         int32_t *bsum32) {
    uint16_t h[256];
    const int nb = K / 256;
    for (int m = 0; m < M; ++m) {
        for (int b = 0; b < nb; ++b) {
            const float *xb = x + (size_t)m * K + (size_t)b * 256;
            qo_f32_to_fp16_array(xb, h, 256);
            qo_quantize_row_q8k_f16(h, 256, d + (size_t)m * nb + b,
                                    qs + (size_t)m * K + (size_t)b * 256,
                                    bsum32 + ((size_t)m * nb + b) * 8);
        }
    }
}

void qo_quantize_q8_0_f32(const float *x, int M, int K, float *d, int8_t *qs) {
    uint16_t h[32];
    const int nb = K / 32;
    for (int m = 0; m < M; ++m) {
        for (int b = 0; b < nb; ++b) {
            const float *xb = x + (size_t)m * K + (size_t)b * 32;
            qo_f32_to_fp16_array(xb, h, 32);
            qo_quantize_row_q8_0_f16(h, 32, d + (size_t)m * nb + b,
                                     qs + (size_t)m * K + (size_t)b * 32);
        }
    }
}

/* --------------------------------------------------------------- dots -- */

/* Integer partials of one 256-value Q4_K block (E:11009-11025). */
static void q4k_block_int(const uint8_t *blk, const int8_t *q8, const int32_t *bs,
                          int32_t *S_out, int32_t *Mb_out) {
    const uint8_t *scales = blk + 4;
    const uint8_t *q = blk + 16;
    int32_t sum_sc_dot = 0, sum_m_bsum = 0;
    int is = 0;
    for (int j = 0; j < 256; j += 64) {
        uint8_t sc0, m0, sc1, m1;
        qo_get_scale_min_k4(is + 0, scales, &sc0, &m0);
        qo_get_scale_min_k4(is + 1, scales, &sc1, &m1);
        int32_t dot1 = 0, dot2 = 0;
        for (int l = 0; l < 32; ++l) {
            const uint8_t q_v = q[l];
            dot1 += (int)(q_v & 0x0F) * (int32_t)q8[j + l];
            dot2 += (int)(q_v >> 4) * (int32_t)q8[j + 32 + l];
        }
        sum_sc_dot += (int32_t)sc0 * dot1 + (int32_t)sc1 * dot2;
        sum_m_bsum += (int32_t)m0 * bs[is + 0] + (int32_t)m1 * bs[is + 1];
        q += 32;
        is += 2;
    }
    *S_out = sum_sc_dot;
    *Mb_out = sum_m_bsum;
}

/* Integer partials of one Q5_K block (E:11040-11062). */
static void q5k_block_int(const uint8_t *blk, const int8_t *q8, const int32_t *bs,
                          int32_t *S_out, int32_t *Mb_out) {
    const uint8_t *scales = blk + 4;
    const uint8_t *qh = blk + 16;
    const uint8_t *ql_p = blk + 48;
    int32_t sum_sc_dot = 0, sum_m_bsum = 0;
    int is = 0;
    uint8_t u1 = 1, u2 = 2;
    for (int j = 0; j < 256; j += 64) {
        uint8_t sc0, m0, sc1, m1;
        qo_get_scale_min_k4(is + 0, scales, &sc0, &m0);
        qo_get_scale_min_k4(is + 1, scales, &sc1, &m1);
        int32_t dot1 = 0, dot2 = 0;
        for (int l = 0; l < 32; ++l) {
            const uint8_t ql_v = ql_p[l], qh_v = qh[l];
            const int q1 = (int)(ql_v & 0x0F) + ((qh_v & u1) ? 16 : 0);
            const int q2 = (int)(ql_v >> 4) + ((qh_v & u2) ? 16 : 0);
            dot1 += q1 * (int32_t)q8[j + l];
            dot2 += q2 * (int32_t)q8[j + 32 + l];
        }
        sum_sc_dot += (int32_t)sc0 * dot1 + (int32_t)sc1 * dot2;
        sum_m_bsum += (int32_t)m0 * bs[is + 0] + (int32_t)m1 * bs[is + 1];
        ql_p += 32;
        is += 2;
        u1 <<= 2;
        u2 <<= 2;
    }
    *S_out = sum_sc_dot;
    *Mb_out = sum_m_bsum;
}

/* Integer partial of one Q6_K block (E:11075-11099). */
static int32_t q6k_block_int(const uint8_t *blk, const int8_t *q8) {
    const uint8_t *ql = blk;
    const uint8_t *qh = blk + 128;
    const int8_t *sc = (const int8_t *)(blk + 192);
    int32_t sum_sc_dot = 0;
    for (int half = 0; half < 2; ++half) {
        const uint8_t *ql_p = ql + half * 64;
        const uint8_t *qh_p = qh + half * 32;
        const int8_t *sc_p = sc + half * 8;
        const int8_t *q8_p = q8 + half * 128;
        for (int is = 0; is < 2; ++is) {
            int32_t dot1 = 0, dot2 = 0, dot3 = 0, dot4 = 0;
            const int l_base = is * 16;
            for (int l = l_base; l < l_base + 16; ++l) {
                const uint8_t ql0 = ql_p[l], ql1 = ql_p[l + 32], qh0 = qh_p[l];
                const int q1 = (int)((ql0 & 0x0F) | (((qh0 >> 0) & 3) << 4)) - 32;
                const int q2 = (int)((ql1 & 0x0F) | (((qh0 >> 2) & 3) << 4)) - 32;
                const int q3 = (int)((ql0 >> 4) | (((qh0 >> 4) & 3) << 4)) - 32;
                const int q4 = (int)((ql1 >> 4) | (((qh0 >> 6) & 3) << 4)) - 32;
                dot1 += q1 * (int32_t)q8_p[l + 0];
                dot2 += q2 * (int32_t)q8_p[l + 32];
                dot3 += q3 * (int32_t)q8_p[l + 64];
                dot4 += q4 * (int32_t)q8_p[l + 96];
            }
            sum_sc_dot += (int32_t)sc_p[is + 0] * dot1 + (int32_t)sc_p[is + 2] * dot2 +
                          (int32_t)sc_p[is + 4] * dot3 + (int32_t)sc_p[is + 6] * dot4;
        }
    }
    return sum_sc_dot;
}

/* Integer partial of one Q8_0 block (E:3400-3404). */
static int32_t q80_block_int(const uint8_t *blk, const int8_t *qs_x) {
    const int8_t *qs_w = (const int8_t *)(blk + 2);
    int32_t dot = 0;
    for (int i = 0; i < 32; ++i) dot += (int32_t)qs_w[i] * (int32_t)qs_x[i];
    return dot;
}

float qo_dot_row(uint32_t type, const uint8_t *w_row, int K, const float *dx,
                 const int8_t *qs, const int32_t *bsum32) {
    float acc = 0.0f;
    if (type == QO_TYPE_Q4_K || type == QO_TYPE_Q5_K) {
        /* E:11026 / E:11063: acc += dx * (d * S - min * Mb) */
        const int nb = K / 256;
        const size_t bb = (type == QO_TYPE_Q4_K) ? 144 : 176;
        for (int b = 0; b < nb; ++b) {
            const uint8_t *blk = w_row + (size_t)b * bb;
            const float d = qo_fp16_to_f32(rd16(blk));
            const float min = qo_fp16_to_f32(rd16(blk + 2));
            int32_t S, Mb;
            if (type == QO_TYPE_Q4_K)
                q4k_block_int(blk, qs + (size_t)b * 256, bsum32 + (size_t)b * 8, &S, &Mb);
            else
                q5k_block_int(blk, qs + (size_t)b * 256, bsum32 + (size_t)b * 8, &S, &Mb);
            acc += dx[b] * (d * (float)S - min * (float)Mb);
        }
    } else if (type == QO_TYPE_Q6_K) {
        /* E:11101: acc += (d * dx) * S */
        const int nb = K / 256;
        for (int b = 0; b < nb; ++b) {
            const uint8_t *blk = w_row + (size_t)b * 210;
            const float d = qo_fp16_to_f32(rd16(blk + 208));
            const int32_t S = q6k_block_int(blk, qs + (size_t)b * 256);
            acc += (d * dx[b]) * (float)S;
        }
    } else if (type == QO_TYPE_Q8_0) {
        /* E:3405: out += (d * dx) * dot */
        const int nb = K / 32;
        for (int b = 0; b < nb; ++b) {
            const uint8_t *blk = w_row + (size_t)b * 34;
            const float d = qo_fp16_to_f32(rd16(blk));
            const int32_t dot = q80_block_int(blk, qs + (size_t)b * 32);
            acc += (d * dx[b]) * (float)dot;
        }
    } else {
        return -1e30f; /* E:11104 */
    }
    return acc;
}

/* sdot_row_f32_batch / sdot_row_f16_batch (E:3410-3440) for one activation
 * row: acc += w[i] * (float)x[i] in row order, x the fp16 input. */
float qo_dot_row_float(uint32_t type, const uint8_t *w_row, int K, const uint16_t *x16) {
    float acc = 0.0f;
    if (type == QO_TYPE_F32) {
        for (int i = 0; i < K; ++i) {
            float w;
            memcpy(&w, w_row + 4 * (size_t)i, 4);
            acc += w * qo_fp16_to_f32(x16[i]);
        }
    } else {
        for (int i = 0; i < K; ++i) acc += qo_fp16_to_f32(rd16(w_row + 2 * (size_t)i)) * qo_fp16_to_f32(x16[i]);
    }
    return acc;
}

int qo_block_partials(uint32_t type, const uint8_t *w_row, int K, const int8_t *qs,
                      const int32_t *bsum32, int32_t *S, int32_t *Mb) {
    if (type == QO_TYPE_Q4_K || type == QO_TYPE_Q5_K) {
        const int nb = K / 256;
        const size_t bb = (type == QO_TYPE_Q4_K) ? 144 : 176;
        for (int b = 0; b < nb; ++b) {
            if (type == QO_TYPE_Q4_K)
                q4k_block_int(w_row + b * bb, qs + (size_t)b * 256, bsum32 + (size_t)b * 8,
                              &S[b], &Mb[b]);
            else
                q5k_block_int(w_row + b * bb, qs + (size_t)b * 256, bsum32 + (size_t)b * 8,
                              &S[b], &Mb[b]);
        }
        return nb;
    }
    if (type == QO_TYPE_Q6_K) {
        const int nb = K / 256;
        for (int b = 0; b < nb; ++b) {
            S[b] = q6k_block_int(w_row + (size_t)b * 210, qs + (size_t)b * 256);
            Mb[b] = 0;
        }
        return nb;
    }
    if (type == QO_TYPE_Q8_0) {
        const int nb = K / 32;
        for (int b = 0; b < nb; ++b) {
            S[b] = q80_block_int(w_row + (size_t)b * 34, qs + (size_t)b * 32);
            Mb[b] = 0;
        }
        return nb;
    }
    return 0;
}

/* ----------------------------------------------------------- dispatch -- */

static int is_kquant(uint32_t t) {
    return t == QO_TYPE_Q4_K || t == QO_TYPE_Q5_K || t == QO_TYPE_Q6_K;
}
static int is_float(uint32_t t) { return t == QO_TYPE_F32 || t == QO_TYPE_F16; }

/* exec_sdot_job_work_stealing's row loop (E:3582-3613), fp32 store; F32 /
 * F16 rows read the fp16 input x16 [M][K] (E:3597-3601). */
static void run_tasks(const float *q8k_d, const int8_t *q8k_qs, const int32_t *q8k_bsum,
                      const float *q80_d, const int8_t *q80_qs, const uint16_t *x16, int M, int K,
                      const qo_matrix_task *tasks, int n_tasks, int total_rows) {
    const int nb256 = K / 256, nb32 = K / 32;
#pragma omp parallel for schedule(dynamic, 64)
    for (int r = 0; r < total_rows; ++r) {
        int t = 0;
        while (t < n_tasks && r >= tasks[t].start_row + tasks[t].rows) ++t;
        const qo_matrix_task *T = &tasks[t];
        const int lr = r - T->start_row;
        const uint8_t *w_row = T->w_base + (size_t)lr * T->row_bytes;
        for (int m = 0; m < M; ++m) {
            float s;
            if (is_float(T->type))
                s = qo_dot_row_float(T->type, w_row, K, x16 + (size_t)m * K);
            else if (T->type == QO_TYPE_Q8_0)
                s = qo_dot_row(T->type, w_row, K, q80_d + (size_t)m * nb32,
                               q80_qs + (size_t)m * K, NULL);
            else
                s = qo_dot_row(T->type, w_row, K, q8k_d + (size_t)m * nb256,
                               q8k_qs + (size_t)m * K, q8k_bsum + (size_t)m * nb256 * 8);
            if (T->residual) s = s + T->residual[(size_t)m * T->res_stride + lr];
            T->dst[(size_t)m * T->dst_stride + lr] = s;
        }
    }
}

static int check_tasks(int M, int K, qo_matrix_task *tasks, int n_tasks, int *need_q8k,
                       int *need_q80, int *need_x16, int *total_rows) {
    if (M <= 0 || K <= 0 || n_tasks <= 0 || !tasks) return -1;
    int tr = 0;
    *need_q8k = *need_q80 = *need_x16 = 0;
    for (int t = 0; t < n_tasks; ++t) {
        if (tasks[t].cols != K) return -1;
        if (is_kquant(tasks[t].type)) {
            if (K % 256) return -1;
            *need_q8k = 1;
        } else if (tasks[t].type == QO_TYPE_Q8_0) {
            if (K % 32) return -1;
            *need_q80 = 1;
        } else if (is_float(tasks[t].type)) {
            *need_x16 = 1;
        } else {
            return -1;
        }
        tasks[t].start_row = tr; /* E:4196-4197 */
        tr += tasks[t].rows;
    }
    *total_rows = tr;
    return 0;
}

#include <stdlib.h>

int qo_gemm_multi(const float *x, int M, int K, qo_matrix_task *tasks, int n_tasks) {
    int need_q8k, need_q80, need_x16, total_rows;
    if (check_tasks(M, K, tasks, n_tasks, &need_q8k, &need_q80, &need_x16, &total_rows)) return -1;
    float *kd = NULL, *zd = NULL;
    int8_t *kq = NULL, *zq = NULL;
    int32_t *ks = NULL;
    uint16_t *x16 = NULL;
    if (need_x16) { /* the fp16 input itself, E:4206 */
        x16 = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)M * K);
        qo_f32_to_fp16_array(x, x16, (size_t)M * K);
    }
    if (need_q8k) {
        kd = (float *)malloc(sizeof(float) * (size_t)M * (K / 256));
        kq = (int8_t *)malloc((size_t)M * K);
        ks = (int32_t *)malloc(sizeof(int32_t) * (size_t)M * (K / 32));
        qo_quantize_q8k_f32(x, M, K, kd, kq, ks); /* E:4209-4215 */
    }
    if (need_q80) {
        zd = (float *)malloc(sizeof(float) * (size_t)M * (K / 32));
        zq = (int8_t *)malloc((size_t)M * K);
        qo_quantize_q8_0_f32(x, M, K, zd, zq);
    }
    run_tasks(kd, kq, ks, zd, zq, x16, M, K, tasks, n_tasks, total_rows);
    free(kd); free(kq); free(ks); free(zd); free(zq); free(x16);
    return 0;
}

int qo_gemm_multi_prequantized(const float *q8k_d, const int8_t *q8k_qs,
                               const int32_t *q8k_bsum, const float *q80_d,
                               const int8_t *q80_qs, const uint16_t *x16, int M, int K,
                               qo_matrix_task *tasks, int n_tasks) {
    int need_q8k, need_q80, need_x16, total_rows;
    if (check_tasks(M, K, tasks, n_tasks, &need_q8k, &need_q80, &need_x16, &total_rows)) return -1;
    if (need_q8k && (!q8k_d || !q8k_qs || !q8k_bsum)) return -1;
    if (need_q80 && (!q80_d || !q80_qs)) return -1;
    if (need_x16 && !x16) return -1;
    run_tasks(q8k_d, q8k_qs, q8k_bsum, q80_d, q80_qs, x16, M, K, tasks, n_tasks, total_rows);
    return 0;
}

/* ------------------------------------------------------------- swiglu -- */

/* swiglu_chunk_worker scalar branch, E:4349-4356, then E:4357 requant. Gate
 * and up are fp16 in the reference (the dispatcher's outputs), so each fp32
 * input is rounded to fp16 first (E:4352-4353). */
void qo_swiglu_q8k(const float *gate, const float *up, int M, int N, float *h,
                   float *d, int8_t *qs, int32_t *bsum32) {
    float hb[256];
    const int nb = N / 256;
    for (int m = 0; m < M; ++m) {
        for (int b = 0; b < nb; ++b) {
            const size_t off = (size_t)m * N + (size_t)b * 256;
            for (int i = 0; i < 256; ++i) {
                const float g = qo_fp16_to_f32(qo_f32_to_fp16(gate[off + i]));
                const float u = qo_fp16_to_f32(qo_f32_to_fp16(up[off + i]));
                hb[i] = (g / (1.0f + expf(-g))) * u;
            }
            if (h) memcpy(h + off, hb, sizeof(hb));
            qo_quantize_q8k_f32(hb, 1, 256, d + (size_t)m * nb + b, qs + off,
                                bsum32 + ((size_t)m * nb + b) * 8);
        }
    }
}

/* ------------------------------------------------------------ rmsnorm -- */

/* rmsnorm_fp16_rows_fast scalar branch (E:4292-4302): sum of squares in row
 * order, inv_rms = 1 / sqrtf(sum * (1/K) + 1e-6f), y = fp16(x * inv_rms *
 * gamma), then the row's Q8_K (E:4303-4305). x, gamma, y are fp16 bits. */
void qo_rmsnorm_q8k_f16(const uint16_t *x, const uint16_t *gamma, int M, int K, uint16_t *y,
                        float *d, int8_t *qs, int32_t *bsum32) {
    const float inv_k = 1.0f / (float)K;
    const int nb = K / 256;
    for (int m = 0; m < M; ++m) {
        const uint16_t *xr = x + (size_t)m * K;
        uint16_t *yr = y + (size_t)m * K;
        float sum_sq = 0.0f;
        for (int i = 0; i < K; ++i) {
            const float v = qo_fp16_to_f32(xr[i]);
            sum_sq += v * v;
        }
        const float inv_rms = 1.0f / sqrtf(sum_sq * inv_k + 1.0e-6f);
        for (int i = 0; i < K; ++i)
            yr[i] = qo_f32_to_fp16(qo_fp16_to_f32(xr[i]) * inv_rms * qo_fp16_to_f32(gamma[i]));
        qo_quantize_row_q8k_f16(yr, K, d + (size_t)m * nb, qs + (size_t)m * K,
                                bsum32 + (size_t)m * nb * 8);
    }
}

/* ------------------------------------------------------------- LM head -- */

/* The running argmax of run_final_norm_and_lm_head_batch_sdot over one
 * chunk's logits (E:11172-11183): row order, v = (float)(fp16)logit, replace
 * on v > best only. With round16 = 0, the fp32 form of the indexed-row scans
 * (E:9568-9569). ids (may be NULL) name the rows; else row_base + r. */
void qo_chunk_argmax(const float *logits, int M, int rows, size_t ldl, int round16, const uint32_t *ids,
                     uint32_t row_base, float *best_val, uint32_t *best_id) {
    for (int m = 0; m < M; ++m) {
        float bv = best_val[m];
        uint32_t bi = best_id[m];
        const float *lr = logits + (size_t)m * ldl;
        for (int r = 0; r < rows; ++r) {
            float v = lr[r];
            if (round16) v = qo_fp16_to_f32(qo_f32_to_fp16(v));
            if (v > bv) {
                bv = v;
                bi = ids ? ids[r] : row_base + (uint32_t)r;
            }
        }
        best_val[m] = bv;
        best_id[m] = bi;
    }
}

/* run_final_norm_and_lm_head_batch_sdot after its RMSNorm (E:11138-11256),
 * without the script-specific extended rows: seed (-1e30, 0); the
 * pre-evaluated rows (E:11143-11146) and each position's draft candidate
 * (E:11147-11153) in fp32; then the chunks: fp16-rounded logits, strict >,
 * positions < active only (E:11169-11183); the pruning (E:11203-11209); the
 * checkpoint test (E:11244-11256). Q8_K rows for the K-quants, Q8_0 rows for
 * Q8_0. Returns the number of chunks read; *active_out / *stopped_out get
 * the final active count and whether a checkpoint ended the scan. */
int qo_lm_head_scan(uint32_t type, const uint8_t *w, int vocab_rows, int K, int M, const float *xd,
                    const int8_t *xqs, const int32_t *xbs, int chunk_rows, const float *thresholds,
                    int n_thresholds, int first_checkpoint, float margin, const uint32_t *pre_ids, int n_pre,
                    const uint32_t *draft_ids, float *best_val, uint32_t *best_id, int *active_out,
                    int *stopped_out) {
    const size_t rb = (size_t)qo_row_bytes(type, (uint64_t)K);
    const int nd = (type == QO_TYPE_Q8_0) ? K / 32 : K / 256;
    float cand[4096];
    if (M > 4096 || rb == 0) return -1;
#define QO_DOT(row, p)                                                                                    \
    qo_dot_row(type, w + (size_t)(row) * rb, K, xd + (size_t)(p) * nd, xqs + (size_t)(p) * K,          \
               xbs ? xbs + (size_t)(p) * (K / 32) : NULL)
    for (int p = 0; p < M; ++p) {
        best_val[p] = -1e30f;
        best_id[p] = 0;
    }
    for (int p = 0; p < M; ++p) {
        for (int i = 0; i < n_pre; ++i) {
            const uint32_t id = pre_ids[i];
            const float v = id < (uint32_t)vocab_rows ? QO_DOT(id, p) : -1e30f;
            if (v > best_val[p]) {
                best_val[p] = v;
                best_id[p] = id;
            }
        }
        if (p + 1 < M && draft_ids) {
            const uint32_t cid = draft_ids[p + 1];
            const float vc = cid < (uint32_t)vocab_rows ? QO_DOT(cid, p) : -1e30f;
            cand[p] = vc;
            if (vc > best_val[p]) {
                best_val[p] = vc;
                best_id[p] = cid;
            }
        } else {
            cand[p] = -1e30f;
        }
    }
    int active = M, stopped = 0, c = 0;
    const int nchunks = (vocab_rows + chunk_rows - 1) / chunk_rows;
    for (c = 0; c < nchunks; ++c) {
        const int r0 = c * chunk_rows;
        const int rows = (r0 + chunk_rows > vocab_rows) ? vocab_rows - r0 : chunk_rows;
        for (int p = 0; p < active; ++p)
            for (int r = 0; r < rows; ++r) {
                const float v = qo_fp16_to_f32(qo_f32_to_fp16(QO_DOT(r0 + r, p)));
                if (v > best_val[p]) {
                    best_val[p] = v;
                    best_id[p] = (uint32_t)(r0 + r);
                }
            }
        for (int p = 0; p + 1 < active; ++p) {
            if (draft_ids && best_id[p] != draft_ids[p + 1] && best_val[p] > cand[p] + margin) {
                active = p + 1;
                break;
            }
        }
        const float thresh = (c < n_thresholds) ? thresholds[c] : -1e30f;
        int all_above = 1;
        for (int p = 0; p < active; ++p)
            if (best_val[p] < thresh) {
                all_above = 0;
                break;
            }
        if (n_thresholds > 0 && c >= first_checkpoint && all_above) {
            stopped = 1;
            ++c;
            break;
        }
    }
#undef QO_DOT
    *active_out = active;
    *stopped_out = stopped;
    return c;
}

/* run_final_norm_and_lm_head_batch_sdot (E:11107-11262) whole, script rows
 * included, and at sc->batch1 the batch-1 scan of
 * run_final_norm_and_lm_head_pipelined (E:9675-9744). */
int qo_lm_head_scan_script(uint32_t type, const uint8_t *w, int vocab_rows, int K, int M, const float *xd,
                           const int8_t *xqs, const int32_t *xbs, int chunk_rows, const float *thresholds,
                           int n_thresholds, float margin, const uint32_t *pre_ids, int n_pre,
                           const uint32_t *draft_ids, qo_script *sc, float *best_val, uint32_t *best_id,
                           int *active_out, int *stopped_out) {
    const size_t rb = (size_t)qo_row_bytes(type, (uint64_t)K);
    const int nd = (type == QO_TYPE_Q8_0) ? K / 32 : K / 256;
    float cand[4096];
    if (M > 4096 || rb == 0 || chunk_rows <= 0 || !sc || (sc->batch1 && (M != 1 || n_pre || draft_ids))) return -1;
#define QO_DOT(row, p)                                                                                    \
    qo_dot_row(type, w + (size_t)(row) * rb, K, xd + (size_t)(p) * nd, xqs + (size_t)(p) * K,          \
               xbs ? xbs + (size_t)(p) * (K / 32) : NULL)
    /* seeds, end-of-text rows and draft candidates (E:11133-11155) */
    for (int p = 0; p < M; ++p) {
        best_val[p] = -1e30f;
        best_id[p] = 0;
        cand[p] = -1e30f;
        for (int i = 0; i < n_pre; ++i) {
            const uint32_t id = pre_ids[i];
            const float v = id < (uint32_t)vocab_rows ? QO_DOT(id, p) : -1e30f;
            if (v > best_val[p]) {
                best_val[p] = v;
                best_id[p] = id;
            }
        }
        if (p + 1 < M && draft_ids) {
            const uint32_t cid = draft_ids[p + 1];
            const float vc = cid < (uint32_t)vocab_rows ? QO_DOT(cid, p) : -1e30f;
            cand[p] = vc;
            if (vc > best_val[p]) {
                best_val[p] = vc;
                best_id[p] = cid;
            }
        }
    }
    int active = M, stopped = 0, c = 0;
    const int nchunks = (vocab_rows + chunk_rows - 1) / chunk_rows;
#define QO_PRUNE()                                                                                 \
    for (int p = 0; p + 1 < active; ++p)                                                           \
        if (draft_ids && best_id[p] != draft_ids[p + 1] && best_val[p] > cand[p] + margin) {       \
            active = p + 1;                                                                        \
            break;                                                                                 \
        }
    for (c = 0; c < nchunks; ++c) {
        const int r0 = c * chunk_rows;
        const int rows = (r0 + chunk_rows > vocab_rows) ? vocab_rows - r0 : chunk_rows;
        /* the chunk's fp16 logits, strict > (E:11172-11183, E:9699-9706) */
        for (int p = 0; p < active; ++p)
            for (int r = 0; r < rows; ++r) {
                const float v = qo_fp16_to_f32(qo_f32_to_fp16(QO_DOT(r0 + r, p)));
                if (v > best_val[p]) {
                    best_val[p] = v;
                    best_id[p] = (uint32_t)(r0 + r);
                }
            }
        /* the session's script flags from the best tokens (E:11186-11193, E:9709-9714) */
        for (int p = 0; p < active; ++p) {
            const uint32_t bt = best_id[p];
            if (bt < (uint32_t)vocab_rows && sc->is_cyr && sc->is_cyr[bt]) sc->has_cyr = 1;
            if (bt < (uint32_t)vocab_rows && sc->is_cjk && sc->is_cjk[bt]) sc->has_cjk = 1;
        }
        QO_PRUNE() /* E:11198-11209 */
        /* chunk 0 of the engine's chunking with a script active: its extended rows (E:11211-11241,
           E:9716-9733) */
        if ((sc->has_cyr || sc->has_cjk) && c == 0 && n_thresholds > 0) {
            for (int s = 0; s < 2; ++s) {
                const int on = s == 0 ? sc->has_cyr : sc->has_cjk;
                const uint32_t *ids = s == 0 ? sc->cyr_rows : sc->cjk_rows;
                const int n = s == 0 ? sc->n_cyr : sc->n_cjk;
                if (!on) continue;
                for (int p = 0; p < active; ++p)
                    for (int i = 0; i < n; ++i) {
                        const uint32_t id = ids[i];
                        const float v = id < (uint32_t)vocab_rows ? QO_DOT(id, p) : -1e30f;
                        if (v > best_val[p]) {
                            best_val[p] = v;
                            best_id[p] = id;
                        }
                    }
            }
            if (sc->batch1) {
                if (!sc->require_full && best_val[0] >= 10.5f) { /* E:9731-9733 */
                    stopped = 1;
                    ++c;
                    break;
                }
            } else {
                QO_PRUNE() /* E:11226-11231 */
                int script_ok = 1;
                for (int p = 0; p < active; ++p) { /* E:11232-11238 */
                    const uint32_t bt = best_id[p];
                    const int in_script = bt < (uint32_t)vocab_rows &&
                                          ((sc->has_cyr && sc->is_cyr && sc->is_cyr[bt]) ||
                                           (sc->has_cjk && sc->is_cjk && sc->is_cjk[bt]));
                    const float min_req = in_script ? 11.5f : 20.0f;
                    if (best_val[p] < min_req) {
                        script_ok = 0;
                        break;
                    }
                }
                if (!sc->require_full && script_ok) { /* E:11239-11241 */
                    stopped = 1;
                    ++c;
                    break;
                }
            }
        }
        /* the checkpoint (E:11243-11256, E:9735-9745) */
        const float thresh = (c < n_thresholds) ? thresholds[c] : -1e30f;
        int all_above = 1;
        for (int p = 0; p < active; ++p)
            if (best_val[p] < thresh) {
                all_above = 0;
                break;
            }
        if (n_thresholds > 0 && (!sc->require_full || c >= 6) && all_above) {
            stopped = 1;
            ++c;
            break;
        }
    }
#undef QO_PRUNE
#undef QO_DOT
    *active_out = active;
    *stopped_out = stopped;
    return c;
}
