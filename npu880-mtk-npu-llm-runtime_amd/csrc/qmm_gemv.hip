// qmm_gemv.hip — batch-1 (M = 1) GEMV over GGUF-packed rows, gfx950.
//
// Work mapping. A wavefront owns R consecutive weight rows; since rows are
// contiguous, its R * nb blocks form one contiguous byte span. Lanes are
// grouped G per block (SLOTS = 64 / G blocks in flight per wave step); each
// lane streams its share of a block straight from HBM (16-B loads for the
// 16-B aligned Q4_K / Q5_K blocks, realigned dword loads for the 2-B aligned
// Q6_K / Q8_0 blocks), unpacks the codes in registers, and forms int32 dot
// partials with v_dot4_i32_i8. The per-block integer partials (S, Mb) are
// summed over the G lanes with DPP — exact and order free — and the block's
// fp32 term is evaluated once with the reference's expression. Block terms
// go to LDS; one lane per row then adds them in block order, the order of
// eval_single_lm_row_dot (E:10986-11105), so the result equals the
// reference's fp32 sum bit for bit.
#include "qmm_device.h"

namespace qmm {

// ----------------------------------------------------------------- Q4_K
// Block (144 B): d f16 @0, dmin f16 @2, scales[12] @4, codes[128] @16.
// Lane k of 8: chunk j = k/2 (64 values), half lh = k%2 -> code bytes
// [16 + 32j + 16lh, +16): low nibbles = values 64j + 16lh + (0..15)
// (sub-block 2j), high nibbles = 64j + 32 + 16lh + (0..15) (sub-block 2j+1).
struct FmtQ4K {
    static constexpr int G = 8, BB = 144, QK = 256;
    struct Raw { uint4 h, c; };
    struct Act { uint4 xl, xh; uint2 bs; float dx; };
    __device__ static Raw load(const uint8_t *blk, int k) {
        return {ld16(blk), ld16(blk + 16 + 16 * k)};
    }
    __device__ static Act load_act(const Q8KView &x, int b, int k) {
        const int j = k >> 1, lh = k & 1;
        const int8_t *xb = x.qs + size_t(b) * 256 + 64 * j + 16 * lh;
        return {ld16(xb), ld16(xb + 32), ld8(x.bs + size_t(b) * 8 + 2 * j), x.d[b]};
    }
    __device__ static float compute(const Raw &r, const Act &a, int k) {
        const int j = k >> 1, lh = k & 1;
        int sc0, m0, sc1, m1;
        scale_min_k4(2 * j, r.h.y, r.h.z, r.h.w, sc0, m0);
        scale_min_k4(2 * j + 1, r.h.y, r.h.z, r.h.w, sc1, m1);
        const uint32_t M4 = 0x0F0F0F0Fu;
        int dot1 = sdot4(int(r.c.x & M4), int(a.xl.x), 0);
        dot1 = sdot4(int(r.c.y & M4), int(a.xl.y), dot1);
        dot1 = sdot4(int(r.c.z & M4), int(a.xl.z), dot1);
        dot1 = sdot4(int(r.c.w & M4), int(a.xl.w), dot1);
        int dot2 = sdot4(int((r.c.x >> 4) & M4), int(a.xh.x), 0);
        dot2 = sdot4(int((r.c.y >> 4) & M4), int(a.xh.y), dot2);
        dot2 = sdot4(int((r.c.z >> 4) & M4), int(a.xh.z), dot2);
        dot2 = sdot4(int((r.c.w >> 4) & M4), int(a.xh.w), dot2);
        int S = __mul24(sc0, dot1) + __mul24(sc1, dot2);
        int Mb = lh ? 0 : __mul24(m0, int(a.bs.x)) + __mul24(m1, int(a.bs.y));
        S = group8_sum(S);
        Mb = group8_sum(Mb);
        const float d = fp16_bits_to_f32(r.h.x & 0xFFFFu);
        const float dmin = fp16_bits_to_f32(r.h.x >> 16);
        return a.dx * (d * (float)S - dmin * (float)Mb);  // E:11026
    }
};

// ----------------------------------------------------------------- Q5_K
// Block (176 B): d @0, dmin @2, scales[12] @4, qh[32] @16, ql[128] @48.
// Lane k: chunk j = k/2, half lh = k%2 -> ql bytes [48 + 32j + 16lh, +16),
// qh bytes [16 + 16lh, +16); high bit of value 64j + l is bit 2j of qh[l],
// of value 64j + 32 + l bit 2j+1.
struct FmtQ5K {
    static constexpr int G = 8, BB = 176, QK = 256;
    struct Raw { uint4 h, qh, ql; };
    using Act = FmtQ4K::Act;
    __device__ static Raw load(const uint8_t *blk, int k) {
        const int j = k >> 1, lh = k & 1;
        return {ld16(blk), ld16(blk + 16 + 16 * lh), ld16(blk + 48 + 32 * j + 16 * lh)};
    }
    __device__ static Act load_act(const Q8KView &x, int b, int k) { return FmtQ4K::load_act(x, b, k); }
    __device__ static float compute(const Raw &r, const Act &a, int k) {
        const int j = k >> 1, lh = k & 1;
        int sc0, m0, sc1, m1;
        scale_min_k4(2 * j, r.h.y, r.h.z, r.h.w, sc0, m0);
        scale_min_k4(2 * j + 1, r.h.y, r.h.z, r.h.w, sc1, m1);
        const uint32_t M4 = 0x0F0F0F0Fu, M1 = 0x01010101u;
        const uint32_t s0 = 2 * j, s1 = 2 * j + 1;
        const uint32_t qlv[4] = {r.ql.x, r.ql.y, r.ql.z, r.ql.w};
        const uint32_t qhv[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
        const uint32_t xl[4] = {a.xl.x, a.xl.y, a.xl.z, a.xl.w};
        const uint32_t xh[4] = {a.xh.x, a.xh.y, a.xh.z, a.xh.w};
        int dot1 = 0, dot2 = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = (qlv[i] & M4) | (((qhv[i] >> s0) & M1) << 4);
            const uint32_t hi = ((qlv[i] >> 4) & M4) | (((qhv[i] >> s1) & M1) << 4);
            dot1 = sdot4(int(lo), int(xl[i]), dot1);
            dot2 = sdot4(int(hi), int(xh[i]), dot2);
        }
        int S = __mul24(sc0, dot1) + __mul24(sc1, dot2);
        int Mb = lh ? 0 : __mul24(m0, int(a.bs.x)) + __mul24(m1, int(a.bs.y));
        S = group8_sum(S);
        Mb = group8_sum(Mb);
        const float d = fp16_bits_to_f32(r.h.x & 0xFFFFu);
        const float dmin = fp16_bits_to_f32(r.h.x >> 16);
        return a.dx * (d * (float)S - dmin * (float)Mb);  // E:11063
    }
};

// ----------------------------------------------------------------- Q6_K
// Block (210 B, 2-B aligned): ql[128] @0, qh[64] @128, int8 sc[16] @192,
// d f16 @208. Lane k: half hf = k/4, l0 = 8 * (k%4), is = (k%4)/2. For
// l in [l0, l0+8): values 128hf + 32i + l (i = 0..3) with scale
// sc[8hf + is + 2i] (E:712-740 / E:11075-11099).
struct FmtQ6K {
    static constexpr int G = 8, BB = 210, QK = 256;
    struct Raw { uint2 a, b, h, s; uint32_t d; };
    struct Act { uint2 x[4]; float dx; };
    __device__ static Raw load(const uint8_t *blk, int k) {
        const int hf = k >> 2, l0 = 8 * (k & 3);
        Raw r;
        r.a = ld8_a2(blk + 64 * hf + l0);
        r.b = ld8_a2(blk + 64 * hf + 32 + l0);
        r.h = ld8_a2(blk + 128 + 32 * hf + l0);
        // the 8 scale bytes of this half, sc[8hf .. 8hf+7]; the lane uses
        // bytes is + {0, 2, 4, 6}
        r.s = ld8_a2(blk + 192 + 8 * hf);
        r.d = ld16b_a2(blk + 208);
        return r;
    }
    __device__ static Act load_act(const Q8KView &x, int b, int k) {
        const int hf = k >> 2, l0 = 8 * (k & 3);
        const int8_t *xb = x.qs + size_t(b) * 256 + 128 * hf + l0;
        return {{ld8(xb), ld8(xb + 32), ld8(xb + 64), ld8(xb + 96)}, x.d[b]};
    }
    __device__ static float compute(const Raw &r, const Act &a, int k) {
        const int is = (k & 3) >> 1;
        const uint32_t M4 = 0x0F0F0F0Fu;
        const uint32_t av[2] = {r.a.x, r.a.y}, bv[2] = {r.b.x, r.b.y}, hv[2] = {r.h.x, r.h.y};
        int dot[4] = {0, 0, 0, 0};
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const uint32_t q1 = (av[w] & M4) | ((hv[w] & 0x03030303u) << 4);
            const uint32_t q2 = (bv[w] & M4) | ((hv[w] & 0x0C0C0C0Cu) << 2);
            const uint32_t q3 = ((av[w] >> 4) & M4) | (hv[w] & 0x30303030u);
            const uint32_t q4 = ((bv[w] >> 4) & M4) | ((hv[w] & 0xC0C0C0C0u) >> 2);
            dot[0] = sdot4(int(sub32_bytes(q1)), int(w ? a.x[0].y : a.x[0].x), dot[0]);
            dot[1] = sdot4(int(sub32_bytes(q2)), int(w ? a.x[1].y : a.x[1].x), dot[1]);
            dot[2] = sdot4(int(sub32_bytes(q3)), int(w ? a.x[2].y : a.x[2].x), dot[2]);
            dot[3] = sdot4(int(sub32_bytes(q4)), int(w ? a.x[3].y : a.x[3].x), dot[3]);
        }
        // sc[8hf + is + 2i], i = 0..3: bytes is, is+2, is+4, is+6 of the 8
        // scale bytes of this half.
        const uint64_t s64 = (uint64_t(r.s.y) << 32) | r.s.x;
        int S = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int sc = int(int8_t(uint8_t(s64 >> (8 * (is + 2 * i)))));
            S += __mul24(sc, dot[i]);
        }
        S = group8_sum(S);
        const float d = fp16_bits_to_f32(r.d);
        return (d * a.dx) * (float)S;  // E:11101
    }
};

// ----------------------------------------------------------------- Q8_0
// Block (34 B, 2-B aligned): d f16 @0, int8 qs[32] @2. Lane k of 4: values
// [8k, 8k+8). Activations are Q8_0 (E:3394-3406).
struct FmtQ80 {
    static constexpr int G = 4, BB = 34, QK = 32;
    struct Raw { uint2 q; uint32_t d; };
    struct Act { uint2 x; float dx; };
    __device__ static Raw load(const uint8_t *blk, int k) { return {ld8_a2(blk + 2 + 8 * k), ld16b_a2(blk)}; }
    __device__ static Act load_act(const Q80View &x, int b, int k) {
        return {ld8(x.qs + size_t(b) * 32 + 8 * k), x.d[b]};
    }
    __device__ static float compute(const Raw &r, const Act &a, int k) {
        (void)k;
        int dot = sdot4(int(r.q.x), int(a.x.x), 0);
        dot = sdot4(int(r.q.y), int(a.x.y), dot);
        dot = group4_sum(dot);
        const float d = fp16_bits_to_f32(r.d);
        return (d * a.dx) * (float)dot;  // E:3405
    }
};

template <class F> struct XViewOf { using T = Q8KView; };
template <> struct XViewOf<FmtQ80> { using T = Q80View; };

// R rows per wave, U wave steps of SLOTS blocks loaded ahead of use.
template <class F, int R, int U>
__global__ __launch_bounds__(256) void gemv_kernel(MatArgs a, typename XViewOf<F>::T x) {
    extern __shared__ float contrib_all[];
    constexpr int G = F::G, SLOTS = 64 / G;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int g = lane / G, k = lane % G;
    const int nb = a.K / F::QK;
    const int row0 = (int(blockIdx.x) * 4 + wid) * R;
    const int nrows = max(0, min(R, a.N - row0));
    const int nblk = nrows * nb;
    float *contrib = contrib_all + wid * R * nb;
    const uint8_t *span = a.w + size_t(max(row0, 0)) * a.row_bytes;

    for (int t0 = 0; t0 < nblk; t0 += SLOTS * U) {
        typename F::Raw raw[U];
        typename F::Act act[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int f = t0 + u * SLOTS + g;
            if (f < nblk) {
                raw[u] = F::load(span + size_t(f) * F::BB, k);
                act[u] = F::load_act(x, f % nb, k);
            } else {
                raw[u] = typename F::Raw{};
                act[u] = typename F::Act{};
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int f = t0 + u * SLOTS + g;
            const float c = F::compute(raw[u], act[u], k);
            if (k == 0 && f < nblk) contrib[f] = c;
        }
    }
    __syncthreads();
    if (lane < nrows) {
        float acc = 0.0f;
        const float *cr = contrib + lane * nb;
        for (int b = 0; b < nb; ++b) acc += cr[b];
        const int row = row0 + lane;
        if (a.res) acc = acc + a.res[row];
        a.y[row] = acc;
    }
}

template <class F, int R, int U>
static hipError_t launch_gemv_t(const MatArgs &a, const typename XViewOf<F>::T &x, hipStream_t s) {
    const int nb = a.K / F::QK;
    const int waves = (a.N + R - 1) / R;
    const unsigned grid = unsigned((waves + 3) / 4);
    const size_t lds = size_t(4) * R * nb * sizeof(float);
    hipLaunchKernelGGL((gemv_kernel<F, R, U>), dim3(grid), dim3(256), lds, s, a, x);
    return hipGetLastError();
}

hipError_t launch_gemv(uint32_t type, const MatArgs &a, const Q8KView &xk, const Q80View &x0,
                       hipStream_t s) {
    switch (type) {
        case kQ4_K: return launch_gemv_t<FmtQ4K, 4, 5>(a, xk, s);
        case kQ5_K: return launch_gemv_t<FmtQ5K, 4, 5>(a, xk, s);
        case kQ6_K: return launch_gemv_t<FmtQ6K, 4, 5>(a, xk, s);
        case kQ8_0: return launch_gemv_t<FmtQ80, 4, 5>(a, x0, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace qmm
