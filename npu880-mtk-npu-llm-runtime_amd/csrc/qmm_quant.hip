// qmm_quant.hip — activation quantizers (fp32 -> fp16 -> Q8_K / Q8_0), the
// SwiGLU + Q8_K requant producer, and the validation dequantizer.
//
// One wavefront per 256-value block: each lane owns 4 consecutive values
// (one 16-B load), the block amax is a wave max, bsum32 is an 8-lane DPP sum.
// Division and rounding follow the reference exactly: d = amax / 127.0f and
// id = 127.0f / amax correctly rounded, q = rint(x * id) (round to nearest
// even, as lrintf under the default mode), clamp to [-127, 127].
#include "qmm_device.h"

namespace qmm {

// Sections of a Q8_K activation buffer as the producers write them.
struct Q8KOut {
    int8_t *qs;
    float *d;
    int32_t *bs;
    int8_t *qt;
    uint16_t *h;
    uint8_t *bh;
};
__host__ inline Q8KOut q8k_out(void *buf, int M, int K) {
    const Q8KLayout L(M, K);
    uint8_t *b = static_cast<uint8_t *>(buf);
    return {reinterpret_cast<int8_t *>(b), reinterpret_cast<float *>(b + L.d_off),
            reinterpret_cast<int32_t *>(b + L.bs_off), reinterpret_cast<int8_t *>(b + L.tile_off),
            reinterpret_cast<uint16_t *>(b + L.h_off), b + L.bh_off};
}

// Quantize one fp16-rounded 256-value block held 4 values per lane and
// store it as Q8_K block `blk` (flattened over [M][K/256]).
// The codes also go to the tiles section (nb blocks per row), the fp16
// values to the h section, the sums of 16 codes (exact in fp16) to the bh
// section. A null qs, h or bs pointer leaves that section unwritten.
__device__ inline void store_q8k_block(float h0, float h1, float h2, float h3, int lane,
                                       size_t blk, const Q8KOut &o, int nb) {
    int8_t *qs = o.qs, *qt = o.qt;
    float *d = o.d;
    int32_t *bs = o.bs;
    if (o.h) {
        const uint32_t hlo = uint32_t(f32_to_fp16_bits(h0)) | (uint32_t(f32_to_fp16_bits(h1)) << 16);
        const uint32_t hhi = uint32_t(f32_to_fp16_bits(h2)) | (uint32_t(f32_to_fp16_bits(h3)) << 16);
        reinterpret_cast<uint2 *>(o.h + blk * 256)[lane] = make_uint2(hlo, hhi);
    }
    float a = fmaxf(fmaxf(fabsf(h0), fabsf(h1)), fmaxf(fabsf(h2), fabsf(h3)));
    a = wave_max(a);  // E:941-946
    int sum;
    const uint32_t packed = quant4(h0, h1, h2, h3, a, sum);
    if (qs) reinterpret_cast<uint32_t *>(qs + blk * 256)[lane] = packed;
    const int m = int(blk / size_t(nb)), j = int(blk - size_t(m) * size_t(nb));
    *reinterpret_cast<uint32_t *>(qt + q8k_tile_pos(m, j, lane, nb)) = packed;
    sum = group4_sum(sum);  // over 16 values = 4 lanes
    if ((lane & 3) == 0)
        *reinterpret_cast<uint16_t *>(o.bh + q8k_bh_pos(m, j, lane >> 2, nb)) = f32_to_fp16_bits((float)sum);
    sum += dpp_half_mirror(sum);  // bsum32 over 32 values = 8 lanes
    if (bs && (lane & 7) == 0) bs[blk * 8 + (lane >> 3)] = sum;
    if (lane == 0) d[blk] = q8_scale(a);  // E:953
}

// x [M][K] fp32, flattened 256-blocks; one wave per block.
__global__ __launch_bounds__(256) void quantize_q8k_kernel(const float *__restrict__ x,
                                                           size_t nblk, Q8KOut o, int nb) {
    const size_t blk = size_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (blk >= nblk) return;
    const int lane = threadIdx.x & 63;
    const float4 v = reinterpret_cast<const float4 *>(x + blk * 256)[lane];
    store_q8k_block(round_to_fp16(v.x), round_to_fp16(v.y), round_to_fp16(v.z),
                    round_to_fp16(v.w), lane, blk, o, nb);
}

// The same for M >= 16, workgroups placed by token tile: workgroup b runs
// on XCD b mod 8, and the 16 tokens of one token tile (for one quad of
// blocks, a wave per block) are consecutive workgroups of one XCD, so the
// tiles and bh sections' lines, which interleave those 16 tokens, are
// written through one L2 (M = 512, K = 9728: 11.1 -> 9.3 us).
__global__ __launch_bounds__(256) void quantize_q8k_tiled_kernel(const float *__restrict__ x, int M, int nb, int nq,
                                                                 int total, Q8KOut o) {
    const int per = (int(gridDim.x) + 7) / 8;
    const int lin = int(blockIdx.x % 8u) * per + int(blockIdx.x / 8u);
    if (lin >= total) return;
    const int mi = lin & 15, u = lin >> 4;
    const int t = u / nq, q = u - t * nq;
    const int m = 16 * t + mi, j = 4 * q + int(threadIdx.x >> 6);
    if (m >= M || j >= nb) return;
    const int lane = threadIdx.x & 63;
    const size_t blk = size_t(m) * size_t(nb) + size_t(j);
    const float4 v = reinterpret_cast<const float4 *>(x + blk * 256)[lane];
    store_q8k_block(round_to_fp16(v.x), round_to_fp16(v.y), round_to_fp16(v.z), round_to_fp16(v.w), lane, blk, o, nb);
}

// Q8_0: 32-value blocks, 8 lanes each, 8 blocks per wave (flattened).
__global__ __launch_bounds__(256) void quantize_q8_0_kernel(const float *__restrict__ x,
                                                            size_t nblk32,
                                                            int8_t *__restrict__ qs,
                                                            float *__restrict__ d) {
    const size_t wave = size_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const size_t blk = wave * 8 + (lane >> 3);
    if (blk >= nblk32) return;  // whole 8-lane groups drop out together
    const int sub = lane & 7;
    const float4 v = reinterpret_cast<const float4 *>(x + blk * 32)[sub];
    const float h0 = round_to_fp16(v.x), h1 = round_to_fp16(v.y);
    const float h2 = round_to_fp16(v.z), h3 = round_to_fp16(v.w);
    float a = fmaxf(fmaxf(fabsf(h0), fabsf(h1)), fmaxf(fabsf(h2), fabsf(h3)));
    a = group8_max(a);
    int sum;
    const uint32_t packed = quant4(h0, h1, h2, h3, a, sum);
    reinterpret_cast<uint32_t *>(qs + blk * 32)[sub] = packed;
    if (sub == 0) d[blk] = q8_scale(a);
}

// swiglu_chunk_worker (E:4349-4357): h = silu_mul(gate, up) per value, then
// the fp16 round + Q8_K quantizer per 256-value block.
__global__ __launch_bounds__(256) void swiglu_q8k_kernel(const float *__restrict__ gate,
                                                         const float *__restrict__ up,
                                                         size_t nblk, float *__restrict__ h, Q8KOut o, int nb) {
    const size_t blk = size_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (blk >= nblk) return;
    const int lane = threadIdx.x & 63;
    const float4 g = reinterpret_cast<const float4 *>(gate + blk * 256)[lane];
    const float4 u = reinterpret_cast<const float4 *>(up + blk * 256)[lane];
    float4 r;
    r.x = silu_mul(g.x, u.x);
    r.y = silu_mul(g.y, u.y);
    r.z = silu_mul(g.z, u.z);
    r.w = silu_mul(g.w, u.w);
    if (h) reinterpret_cast<float4 *>(h + blk * 256)[lane] = r;
    store_q8k_block(round_to_fp16(r.x), round_to_fp16(r.y), round_to_fp16(r.z),
                    round_to_fp16(r.w), lane, blk, o, nb);
}

// rmsnorm_fp16_rows_fast (E:4264-4314) + its Q8_K (E:4303-4305): one
// workgroup per row. Thread t owns the float4s t + 256 j (values 4t + 1024 j
// .. +3), so wave w holds the 256-value block 4j + w of the row for the
// quantizer. The sum of squares is a tree over threads (not the reference's
// row order: the last bits of inv_rms may differ, so y is compared with a
// tolerance and the codes by composition); inv_rms = 1 / sqrtf(sum * (1/K)
// + 1e-6f) and y = fp16((x * inv_rms) * gamma) as in E:4295-4302.
template <int NJ>
__global__ __launch_bounds__(256) void rmsnorm_q8k_kernel(const float *__restrict__ x,
                                                          const float *__restrict__ gamma, int K,
                                                          float *__restrict__ y, Q8KOut o) {
    __shared__ float part[4];
    const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
    const size_t m = blockIdx.x;
    const float *xr = x + m * size_t(K);
    const int nq = K >> 2;  // float4s in the row
    float4 h[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int q = t + 256 * j;
        const float4 v = q < nq ? reinterpret_cast<const float4 *>(xr)[q] : make_float4(0.f, 0.f, 0.f, 0.f);
        h[j] = make_float4(round_to_fp16(v.x), round_to_fp16(v.y), round_to_fp16(v.z), round_to_fp16(v.w));
    }
    // the sum of squares in the batch-1 activation fill's layout (so the GEMV
    // that normalizes its own input forms the same inv_rms)
    float s = 0.0f;
    const int nc = K >> 8, sub = t & 15;
    for (int c = 4 * wid + ((t >> 4) & 3); c < nc; c += 16) {
        const float4 *q = reinterpret_cast<const float4 *>(xr + c * 256 + 16 * sub);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = q[i];
            s = rms_add4(s, make_float4(round_to_fp16(v.x), round_to_fp16(v.y), round_to_fp16(v.z), round_to_fp16(v.w)));
        }
    }
    const float inv_rms = rms_inv(s, K, part);
    const size_t nbk = size_t(K) >> 8;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int q = t + 256 * j;
        if (4 * (256 * j + 64 * wid) >= K) break;  // whole waves past the row's end
        const float4 g = reinterpret_cast<const float4 *>(gamma)[q];
        float4 r;
        r.x = round_to_fp16(h[j].x * inv_rms * round_to_fp16(g.x));  // E:4301
        r.y = round_to_fp16(h[j].y * inv_rms * round_to_fp16(g.y));
        r.z = round_to_fp16(h[j].z * inv_rms * round_to_fp16(g.z));
        r.w = round_to_fp16(h[j].w * inv_rms * round_to_fp16(g.w));
        if (y) reinterpret_cast<float4 *>(y + m * size_t(K))[q] = r;
        store_q8k_block(r.x, r.y, r.z, r.w, lane, m * nbk + size_t(4 * j + wid), o, int(nbk));
    }
}

// ---------------------------------------------------------------- dequant
// One thread per 32-value group (a K-quant sub-block or a Q8_0 block);
// formulas of dequant_block_q4_k/q5_k/q6_k/q8_0 scalar branches
// (E:786-800, E:837-852, E:712-740, E:613). Validation path only.
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t *__restrict__ w,
                                                      uint32_t type, size_t ngroups,
                                                      uint16_t *__restrict__ dst) {
    const size_t gi = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (gi >= ngroups) return;
    uint16_t *y = dst + gi * 32;
    if (type == kF16) {  // E:3857-3860: a copy
        const uint16_t *src = reinterpret_cast<const uint16_t *>(w) + gi * 32;
        for (int i = 0; i < 32; ++i) y[i] = src[i];
        return;
    }
    if (type == kF32) {  // E:3876-3879: (__fp16) of each value
        const float *src = reinterpret_cast<const float *>(w) + gi * 32;
        for (int i = 0; i < 32; ++i) y[i] = f32_to_fp16_bits(src[i]);
        return;
    }
    if (type == kQ8_0) {
        const uint8_t *blk = w + gi * 34;
        const float dd = fp16_bits_to_f32(uint32_t(blk[0]) | (uint32_t(blk[1]) << 8));
        for (int i = 0; i < 32; ++i) y[i] = f32_to_fp16_bits(dd * (float)(int8_t)blk[2 + i]);
        return;
    }
    const size_t b = gi >> 3;
    const int s = int(gi & 7);  // 32-value group inside the 256 block
    if (type == kQ4_K || type == kQ5_K) {
        const uint8_t *blk = w + b * (type == kQ4_K ? 144 : 176);
        const float dd = fp16_bits_to_f32(uint32_t(blk[0]) | (uint32_t(blk[1]) << 8));
        const float mn = fp16_bits_to_f32(uint32_t(blk[2]) | (uint32_t(blk[3]) << 8));
        uint8_t sc, m;
        const uint8_t *q = blk + 4;
        if (s < 4) {
            sc = q[s] & 63;
            m = q[s + 4] & 63;
        } else {
            sc = (uint8_t)((q[s + 4] & 0x0F) | ((q[s - 4] >> 6) << 4));
            m = (uint8_t)((q[s + 4] >> 4) | ((q[s] >> 6) << 4));
        }
        const float d1 = dd * (float)sc, m1 = mn * (float)m;
        const int j = s >> 1, hi = s & 1;
        if (type == kQ4_K) {
            const uint8_t *qs = blk + 16 + 32 * j;
            for (int l = 0; l < 32; ++l) {
                const int v = hi ? (qs[l] >> 4) : (qs[l] & 0x0F);
                y[l] = f32_to_fp16_bits(d1 * (float)v - m1);
            }
        } else {
            const uint8_t *qh = blk + 16;
            const uint8_t *ql = blk + 48 + 32 * j;
            const uint8_t u = uint8_t(1u << s);
            for (int l = 0; l < 32; ++l) {
                const int v = (hi ? (ql[l] >> 4) : (ql[l] & 0x0F)) + ((qh[l] & u) ? 16 : 0);
                y[l] = f32_to_fp16_bits(d1 * (float)v - m1);
            }
        }
        return;
    }
    // Q6_K: 32-value group s = 32 outputs y[half*128 + 32*i + l], l < 32.
    const uint8_t *blk = w + b * 210;
    const float dd = fp16_bits_to_f32(uint32_t(blk[208]) | (uint32_t(blk[209]) << 8));
    const int half = s >> 2, i = s & 3;
    const uint8_t *ql = blk + half * 64 + ((i & 1) ? 32 : 0);
    const uint8_t *qh = blk + 128 + half * 32;
    const int8_t *sc = reinterpret_cast<const int8_t *>(blk + 192 + half * 8);
    for (int l = 0; l < 32; ++l) {
        const int lo = (i < 2) ? (ql[l] & 0x0F) : (ql[l] >> 4);
        const int q = (lo | (((qh[l] >> (2 * i)) & 3) << 4)) - 32;
        const float dsc = dd * (float)sc[(l >> 4) + 2 * i];
        y[l] = f32_to_fp16_bits(dsc * (float)q);
    }
}

hipError_t launch_quantize_q8k(const float *x, int M, int K, void *out, hipStream_t s, unsigned skip) {
    const size_t nblk = size_t(M) * size_t(K / 256);
    const unsigned grid = unsigned((nblk + 3) / 4);
    Q8KOut o = q8k_out(out, M, K);
    if (skip & kSkipQs) o.qs = nullptr;
    if (skip & kSkipH) o.h = nullptr;
    if (skip & kSkipBs) o.bs = nullptr;
    if (M >= 16) {
        const int nb = K / 256, nq = (nb + 3) / 4, total = ((M + 15) / 16) * nq * 16;
        hipLaunchKernelGGL(quantize_q8k_tiled_kernel, dim3(unsigned((total + 7) / 8 * 8)), dim3(256), 0, s, x, M, nb,
                           nq, total, o);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(quantize_q8k_kernel, dim3(grid), dim3(256), 0, s, x, nblk, o, K / 256);
    return hipGetLastError();
}

hipError_t launch_quantize_q8_0(const float *x, int M, int K, void *out, hipStream_t s) {
    const Q80Layout L(M, K);
    uint8_t *base = static_cast<uint8_t *>(out);
    const size_t nblk = size_t(M) * size_t(K / 32);
    const size_t waves = (nblk + 7) / 8;
    const unsigned grid = unsigned((waves + 3) / 4);
    hipLaunchKernelGGL(quantize_q8_0_kernel, dim3(grid), dim3(256), 0, s, x, nblk,
                       reinterpret_cast<int8_t *>(base), reinterpret_cast<float *>(base + L.d_off));
    return hipGetLastError();
}

hipError_t launch_swiglu_q8k(const float *gate, const float *up, int M, int N, float *h,
                             void *out, hipStream_t s) {
    const size_t nblk = size_t(M) * size_t(N / 256);
    const unsigned grid = unsigned((nblk + 3) / 4);
    hipLaunchKernelGGL(swiglu_q8k_kernel, dim3(grid), dim3(256), 0, s, gate, up, nblk, h, q8k_out(out, M, N),
                       N / 256);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_q8k(const float *x, const float *gamma, int M, int K, float *y,
                              void *out, hipStream_t s) {
    const Q8KOut o = q8k_out(out, M, K);
    const int nj = (K / 4 + 255) / 256;  // float4s per thread
#define QMM_RMS(NJ) \
    hipLaunchKernelGGL(rmsnorm_q8k_kernel<NJ>, dim3(unsigned(M)), dim3(256), 0, s, x, gamma, K, y, o)
    if (nj <= 3) QMM_RMS(3);
    else if (nj <= 4) QMM_RMS(4);
    else if (nj <= 10) QMM_RMS(10);
    else if (nj <= 16) QMM_RMS(16);
    else return hipErrorInvalidValue;
#undef QMM_RMS
    return hipGetLastError();
}

hipError_t launch_dequant_f16(const uint8_t *w, uint32_t type, int64_t rows, int64_t cols,
                              uint16_t *dst, hipStream_t s) {
    const size_t ngroups = size_t(rows) * size_t(cols / 32);
    const unsigned grid = unsigned((ngroups + 255) / 256);
    hipLaunchKernelGGL(dequant_kernel, dim3(grid), dim3(256), 0, s, w, type, ngroups, dst);
    return hipGetLastError();
}

}  // namespace qmm
