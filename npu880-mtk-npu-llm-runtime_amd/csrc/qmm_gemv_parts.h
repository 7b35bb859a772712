// qmm_gemv_parts.h — the pieces the batch-1 kernels share: the per-format
// block dot products (4 or 8 lanes per block, DPP sums, the reference's
// per-block fp32 expression), the activation fill (fp32 row -> Q8_K / Q8_0
// codes in LDS, or a prequantized row copied in), and the LDS carve-up.
#pragma once
#include "qmm_device.h"

namespace qmm {

// ------------------------------------------------------------ DPP on fp32
template <int CTRL>
__device__ inline float dppf(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// max over each 16-lane row (all 16 lanes active): xor1, xor2, half-mirror, mirror
__device__ inline float row16_max(float v) {
    v = fmaxf(v, dppf<0xB1>(v));
    v = fmaxf(v, dppf<0x4E>(v));
    v = fmaxf(v, dppf<0x141>(v));
    v = fmaxf(v, dppf<0x140>(v));
    return v;
}

// ----------------------------------------------------------------- Q4_K
// Block (144 B): d f16 @0, dmin f16 @2, scales[12] @4, codes[128] @16: code
// bytes [16 + 32j, +32) hold values 64j + (0..31) in their low nibbles
// (sub-block 2j) and 64j + 32 + (0..31) in their high nibbles (sub-block
// 2j+1).
// Q4_K, 4 lanes per block (the form the library launches): lane k owns
// the 64 values of chunk k — code bytes [16 + 32k, +32): low nibbles =
// sub-block 2k, high nibbles = sub-block 2k+1. The wave's span is staged
// through LDS with coalesced 16-B loads (16 blocks per wave step).
// Scales / mins of sub-blocks 2k, 2k+1 (get_scale_min_k4, E:743-749) in the
// two low bytes of SC / MM.
__device__ inline void scale_pair_k4(int k, uint32_t s0, uint32_t s1, uint32_t s2, uint32_t &SC, uint32_t &MM) {
    const uint32_t sh = 16u * uint32_t(k & 1);
    const uint32_t A = s0 >> sh, B = s1 >> sh, C = s2 >> sh;
    const uint32_t sc_lo = A & 0x3F3Fu, m_lo = B & 0x3F3Fu;                  // j < 4
    const uint32_t sc_hi = (C & 0x0F0Fu) | ((A >> 2) & 0x3030u);             // j >= 4
    const uint32_t m_hi = ((C >> 4) & 0x0F0Fu) | ((B >> 2) & 0x3030u);
    SC = (k >= 2) ? sc_hi : sc_lo;
    MM = (k >= 2) ? m_hi : m_lo;
}
struct FmtQ4K4 {
    static constexpr int G = 4, BB = 144, QK = 256;
    static constexpr bool kStaged = true;
    struct Raw { uint4 h, c0, c1; };
    struct Act { uint4 x0, x1, x2, x3; uint2 bs; float dx; };
    __device__ static Raw load(const uint8_t *blk, int k) {  // blk points into the LDS stage
        return {ld16(blk), ld16(blk + 16 + 32 * k), ld16(blk + 32 + 32 * k)};
    }
    __device__ static Act load_act(const LdsAct &x, int b, int k) {
        const int8_t *xb = x.qs + b * 272 + 64 * k;
        return {ld16(xb), ld16(xb + 16), ld16(xb + 32), ld16(xb + 48), ld8(x.bs + b * 8 + 2 * k), x.d[b]};
    }
    __device__ static float compute(const Raw &r, const Act &a, int k) {
        uint32_t SC, MM;
        scale_pair_k4(k, r.h.y, r.h.z, r.h.w, SC, MM);
        const uint32_t M4 = 0x0F0F0F0Fu;
        const uint32_t c[8] = {r.c0.x, r.c0.y, r.c0.z, r.c0.w, r.c1.x, r.c1.y, r.c1.z, r.c1.w};
        const uint32_t xl[8] = {a.x0.x, a.x0.y, a.x0.z, a.x0.w, a.x1.x, a.x1.y, a.x1.z, a.x1.w};
        const uint32_t xh[8] = {a.x2.x, a.x2.y, a.x2.z, a.x2.w, a.x3.x, a.x3.y, a.x3.z, a.x3.w};
        int dot1 = 0, dot2 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            dot1 = sdot4(int(c[i] & M4), int(xl[i]), dot1);
            dot2 = sdot4(int((c[i] >> 4) & M4), int(xh[i]), dot2);
        }
        int S = __mul24(int(SC & 0xFF), dot1) + __mul24(int(SC >> 8), dot2);
        int Mb = __mul24(int(MM & 0xFF), int(a.bs.x)) + __mul24(int(MM >> 8), int(a.bs.y));
        S = group4_sum(S);
        Mb = group4_sum(Mb);
        const float d = fp16_bits_to_f32(r.h.x & 0xFFFFu);
        const float dmin = fp16_bits_to_f32(r.h.x >> 16);
        return a.dx * (d * (float)S - dmin * (float)Mb);  // E:11026
    }
};

// ----------------------------------------------------------------- Q5_K
// Block (176 B): d @0, dmin @2, scales[12] @4, qh[32] @16, ql[128] @48.
// Q5_K, 4 lanes per block (the form the library launches): lane k owns the
// 64 values of chunk k — ql bytes [48 + 32k, +32): low nibbles = sub-block
// 2k, high nibbles = sub-block 2k+1 — and reads the whole qh[32]: the high
// bit of value 64k + l is bit 2k of qh[l], of value 64k + 32 + l bit 2k+1.
// The wave's span is staged through LDS (176-B blocks stay 16-B aligned).
struct FmtQ5K4 {
    static constexpr int G = 4, BB = 176, QK = 256;
    static constexpr bool kStaged = true;
    struct Raw { uint4 h, qh0, qh1, c0, c1; };
    using Act = FmtQ4K4::Act;
    __device__ static Raw load(const uint8_t *blk, int k) {  // blk points into the LDS stage
        return {ld16(blk), ld16(blk + 16), ld16(blk + 32), ld16(blk + 48 + 32 * k), ld16(blk + 64 + 32 * k)};
    }
    __device__ static Act load_act(const LdsAct &x, int b, int k) { return FmtQ4K4::load_act(x, b, k); }
    __device__ static float compute(const Raw &r, const Act &a, int k) {
        uint32_t SC, MM;
        scale_pair_k4(k, r.h.y, r.h.z, r.h.w, SC, MM);
        const uint32_t M4 = 0x0F0F0F0Fu, B4 = 0x10101010u;
        // rotating a qh dword right by 2k - 4 (mod 32) puts bit 2k of each
        // byte at bit 4 and bit 2k + 1 at bit 5; what crosses a byte boundary
        // lands in bits the masks drop
        const uint32_t rot = uint32_t(2 * k - 4) & 31u;
        const uint32_t c[8] = {r.c0.x, r.c0.y, r.c0.z, r.c0.w, r.c1.x, r.c1.y, r.c1.z, r.c1.w};
        const uint32_t qh[8] = {r.qh0.x, r.qh0.y, r.qh0.z, r.qh0.w, r.qh1.x, r.qh1.y, r.qh1.z, r.qh1.w};
        const uint32_t xl[8] = {a.x0.x, a.x0.y, a.x0.z, a.x0.w, a.x1.x, a.x1.y, a.x1.z, a.x1.w};
        const uint32_t xh[8] = {a.x2.x, a.x2.y, a.x2.z, a.x2.w, a.x3.x, a.x3.y, a.x3.z, a.x3.w};
        int dot1 = 0, dot2 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t h = __builtin_amdgcn_alignbit(qh[i], qh[i], rot);
            const uint32_t lo = (c[i] & M4) | (h & B4);
            const uint32_t hi = ((c[i] >> 4) & M4) | ((h >> 1) & B4);
            dot1 = sdot4(int(lo), int(xl[i]), dot1);
            dot2 = sdot4(int(hi), int(xh[i]), dot2);
        }
        int S = __mul24(int(SC & 0xFF), dot1) + __mul24(int(SC >> 8), dot2);
        int Mb = __mul24(int(MM & 0xFF), int(a.bs.x)) + __mul24(int(MM >> 8), int(a.bs.y));
        S = group4_sum(S);
        Mb = group4_sum(Mb);
        const float d = fp16_bits_to_f32(r.h.x & 0xFFFFu);
        const float dmin = fp16_bits_to_f32(r.h.x >> 16);
        return a.dx * (d * (float)S - dmin * (float)Mb);  // E:11063
    }
};

// ----------------------------------------------------------------- Q6_K
// Block (210 B, 2-B aligned): ql[128] @0, qh[64] @128, int8 sc[16] @192,
// d f16 @208 (E:712-740 / E:11075-11099). Read from the LDS stage.
// Q6_K, 4 lanes per block (the form the library launches): lane k takes
// half hf = k / 2 and positions l in [16 (k % 2), +16) of every 32-value run
// i = 0..3 of that half (value 32i + l of the half: ql[64hf + l] low nibble
// for i = 0, ql[64hf + 32 + l] low for i = 1, the high nibbles for i = 2, 3;
// qh[32hf + l] bits 2i, 2i + 1; scale sc[8hf + 2i + k % 2]), so each run
// has one scale per lane. The codes stay unsigned: a run's sum of
// (q - 32) x is sum q x - 32 sum x, both exact int32 dot products.
struct FmtQ6K4 {
    static constexpr int G = 4, BB = 210, QK = 256;
    static constexpr bool kStaged = true;
    struct Raw { uint4 a, b, h; uint2 s; uint32_t d; };
    struct Act { uint4 x[4]; int4 xs; float dx; };  // xs: the lane's four 16-code sums
    // blk points into LDS, 2-B aligned. Every field lies a multiple of 8 B
    // from it, so one misalignment (0 or 2 B) serves all: aligned dword reads
    // (the last one read whatever the misalignment: at most 2 B past the
    // block, inside the stage) and funnel shifts.
    __device__ static Raw load(const uint8_t *blk, int k) {
        const int hf = k >> 1, l0 = 16 * (k & 1);
        const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(blk) & 3);
        const uint32_t *q = reinterpret_cast<const uint32_t *>(blk - sh);
        auto rd16 = [&](int dw) __attribute__((always_inline)) {
            const uint32_t w0 = q[dw], w1 = q[dw + 1], w2 = q[dw + 2], w3 = q[dw + 3], w4 = q[dw + 4];
            return make_uint4(funnel(w1, w0, sh), funnel(w2, w1, sh), funnel(w3, w2, sh), funnel(w4, w3, sh));
        };
        Raw r;
        r.a = rd16(16 * hf + l0 / 4);
        r.b = rd16(16 * hf + 8 + l0 / 4);
        r.h = rd16(32 + 8 * hf + l0 / 4);
        const uint32_t s0 = q[48 + 2 * hf], s1 = q[49 + 2 * hf], s2 = q[50 + 2 * hf];
        r.s = make_uint2(funnel(s1, s0, sh), funnel(s2, s1, sh));  // sc[8hf .. 8hf+7]
        r.d = (q[52] >> (8 * sh)) & 0xFFFFu;
        return r;
    }
    __device__ static Act load_act(const LdsAct &x, int b, int k) {
        const int8_t *xb = x.qs + b * 272 + 128 * (k >> 1) + 16 * (k & 1);
        return {{ld16(xb), ld16(xb + 32), ld16(xb + 64), ld16(xb + 96)},
                *reinterpret_cast<const int4 *>(x.bs16 + 16 * b + 4 * k), x.d[b]};
    }
    __device__ static float compute(const Raw &r, const Act &a, int k) {
        const uint32_t M4 = 0x0F0F0F0Fu;
        const uint32_t av[4] = {r.a.x, r.a.y, r.a.z, r.a.w}, bv[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
        const uint32_t hv[4] = {r.h.x, r.h.y, r.h.z, r.h.w};
        int dot[4] = {0, 0, 0, 0};
        const int xs[4] = {a.xs.x, a.xs.y, a.xs.z, a.xs.w};  // the runs' code sums, from the fill
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t q[4] = {(av[w] & M4) | ((hv[w] & 0x03030303u) << 4),
                                   (bv[w] & M4) | ((hv[w] & 0x0C0C0C0Cu) << 2),
                                   ((av[w] >> 4) & M4) | (hv[w] & 0x30303030u),
                                   ((bv[w] >> 4) & M4) | ((hv[w] & 0xC0C0C0C0u) >> 2)};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t xw = i == 0 ? (w == 0 ? a.x[0].x : w == 1 ? a.x[0].y : w == 2 ? a.x[0].z : a.x[0].w)
                                  : i == 1 ? (w == 0 ? a.x[1].x : w == 1 ? a.x[1].y : w == 2 ? a.x[1].z : a.x[1].w)
                                  : i == 2 ? (w == 0 ? a.x[2].x : w == 1 ? a.x[2].y : w == 2 ? a.x[2].z : a.x[2].w)
                                           : (w == 0 ? a.x[3].x : w == 1 ? a.x[3].y : w == 2 ? a.x[3].z : a.x[3].w);
                dot[i] = sdot4(int(q[i]), int(xw), dot[i]);
            }
        }
        // sc[8hf + 2i + k % 2]: bytes k % 2, 2 + k % 2, 4 + k % 2, 6 + k % 2
        const uint64_t s64 = (uint64_t(r.s.y) << 32) | r.s.x;
        const int is = k & 1;
        int S = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int sc = int(int8_t(uint8_t(s64 >> (8 * (is + 2 * i)))));
            S += __mul24(sc, dot[i] - 32 * xs[i]);
        }
        S = group4_sum(S);
        const float d = fp16_bits_to_f32(r.d);
        return (d * a.dx) * (float)S;  // E:11101
    }
};

// ----------------------------------------------------------------- Q8_0
// Block (34 B, 2-B aligned): d f16 @0, int8 qs[32] @2. Lane k of 4: values
// [8k, 8k+8). Activations are Q8_0 (E:3394-3406). Read from the LDS stage.
struct FmtQ80 {
    static constexpr int G = 4, BB = 34, QK = 32;
    static constexpr bool kStaged = true;
    struct Raw { uint2 q; uint32_t d; };
    struct Act { uint2 x; float dx; };
    // blk in LDS, 2-B aligned (misalignment sh = 0 or 2): the codes at blk + 2 +
    // 8 k start sh ^ 2 bytes into dword 2 k + sh / 2 of blk - sh; the third
    // dword is read whatever the shift (at most 4 B past the block, inside the
    // staged bytes' region)
    __device__ static Raw load(const uint8_t *blk, int k) {
        const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(blk) & 3), s2 = sh ^ 2u;
        const uint32_t *q = reinterpret_cast<const uint32_t *>(blk - sh);
        const uint32_t *p = q + 2 * k + (sh >> 1);
        const uint32_t w0 = p[0], w1 = p[1], w2 = p[2];
        return {make_uint2(funnel(w1, w0, s2), funnel(w2, w1, s2)), (q[0] >> (8 * sh)) & 0xFFFFu};
    }
    __device__ static Act load_act(const LdsAct &x, int b, int k) {
        return {ld8(x.qs + lds_pad(b * 32 + 8 * k)), x.d[b]};
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

template <class F> struct IsQ80 { static constexpr bool v = false; };
template <> struct IsQ80<FmtQ80> { static constexpr bool v = true; };

// ------------------------------------------------------ activation fill
// 16 lanes per 256-value chunk: lane sub of row r in wave w handles values
// 16 * sub .. +16 of chunk c = 16 * round + 4w + r. Round 0 is loaded before
// the weights are requested. A wave whose chunks of a round all lie past the
// row skips that round (x_has): clamped loads would still cost it issue time
// ahead of its weight loads.
struct XPre { float4 v[4]; };

__device__ inline bool x_has(int round, int K) {
    return 16 * round + 4 * int(threadIdx.x >> 6) < ((K + 255) >> 8);
}

__device__ inline int x_chunk(int round, int K) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int nc = (K + 255) >> 8;
    return min(16 * round + 4 * wid + (lane >> 4), nc - 1);
}
// clamped to the last 16 values of x for a partial last Q8_0 chunk; such
// lanes' results are never stored
__device__ inline void x_load(const float *__restrict__ x, int K, int c, XPre &p) {
    const int v0 = min(c * 256 + 16 * int(threadIdx.x & 15), K - 16);
    const float4 *q = reinterpret_cast<const float4 *>(x + v0);
    p.v[0] = q[0];
    p.v[1] = q[1];
    p.v[2] = q[2];
    p.v[3] = q[3];
}

// The batch-1 fill on the row before its RMSNorm (K <= 4096: round 0 holds
// the whole row): the workgroup's sum of squares in the fill's layout
// (rms_inv; duplicates of the last chunk left out), then the lane's values
// become y = fp16((fp16(x) * inv_rms) * fp16(gamma)) (E:4301), the values
// rmsnorm_q8k_kernel forms. gp: the lane's gamma values, loaded as x_load
// loads x. Every wave of the workgroup calls it (a workgroup barrier).
__device__ inline void rms_fill_transform(XPre &xp, const XPre &gp, int K, float *part) {
    const int wid = int(threadIdx.x) >> 6;
    float ss = 0.0f;
    if (x_has(0, K) && 4 * wid + ((int(threadIdx.x) >> 4) & 3) < (K >> 8)) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            ss = rms_add4(ss, make_float4(round_to_fp16(xp.v[i].x), round_to_fp16(xp.v[i].y),
                                          round_to_fp16(xp.v[i].z), round_to_fp16(xp.v[i].w)));
    }
    const float inv_rms = rms_inv(ss, K, part);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        xp.v[i].x = round_to_fp16(round_to_fp16(xp.v[i].x) * inv_rms * round_to_fp16(gp.v[i].x));
        xp.v[i].y = round_to_fp16(round_to_fp16(xp.v[i].y) * inv_rms * round_to_fp16(gp.v[i].y));
        xp.v[i].z = round_to_fp16(round_to_fp16(xp.v[i].z) * inv_rms * round_to_fp16(gp.v[i].z));
        xp.v[i].w = round_to_fp16(round_to_fp16(xp.v[i].w) * inv_rms * round_to_fp16(gp.v[i].w));
    }
}

// Quantize the lane's 16 values of chunk c into the LDS row: Q8_K
// (quantize_row_fp16_to_q8_k, E:925-990) or Q8_0 (E:1016-1064), after
// rounding each value to fp16. `store` is false for clamped duplicates.
// position of the 16-value group at offset o (a multiple of 16) of block b in
// the bs16 row: lane k = 2 (o >> 7) + ((o >> 4) & 1) of a Q6_K block reads
// its four runs (o >> 5) & 3 = 0..3 as one 16-B word at 16 b + 4 k
__device__ inline int bs16_pos(int b, int o) { return 16 * b + 4 * (2 * (o >> 7) + ((o >> 4) & 1)) + ((o >> 5) & 3); }

template <bool Q80, bool BS16 = false>
__device__ inline void x_quant(const XPre &p, int c, int K, bool store, const LdsAct &a) {
    const int sub = threadIdx.x & 15;
    float h[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h[4 * i + 0] = round_to_fp16(p.v[i].x);
        h[4 * i + 1] = round_to_fp16(p.v[i].y);
        h[4 * i + 2] = round_to_fp16(p.v[i].z);
        h[4 * i + 3] = round_to_fp16(p.v[i].w);
    }
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) m = fmaxf(m, fabsf(h[i]));
    // block max: 256 values = the 16-lane row; 32 values (Q8_0) = a lane pair
    const float amax = Q80 ? fmaxf(m, dppf<0xB1>(m)) : row16_max(m);
    int s0, s1, s2, s3;
    uint4 q;
    const float id = q8_inv_scale(amax);
    q.x = quant4_rne(h[0], h[1], h[2], h[3], id, s0);
    q.y = quant4_rne(h[4], h[5], h[6], h[7], id, s1);
    q.z = quant4_rne(h[8], h[9], h[10], h[11], id, s2);
    q.w = quant4_rne(h[12], h[13], h[14], h[15], id, s3);
    int sum = s0 + s1 + s2 + s3;
    const int sum16 = sum;
    sum += __builtin_amdgcn_mov_dpp(sum, 0xB1, 0xF, 0xF, false);  // the 32-value pair
    const int v0 = c * 256 + 16 * sub;
    store = store && v0 < K;
    if (store) {
        if constexpr (BS16) const_cast<int32_t *>(a.bs16)[bs16_pos(c, 16 * sub)] = sum16;
        *reinterpret_cast<uint4 *>(const_cast<int8_t *>(a.qs) + lds_pad(v0)) = q;
        if ((sub & 1) == 0) {
            if constexpr (Q80) {
                const_cast<float *>(a.d)[v0 >> 5] = q8_scale(amax);
            } else {
                const_cast<int32_t *>(a.bs)[v0 >> 5] = sum;
                if (sub == 0) const_cast<float *>(a.d)[c] = q8_scale(amax);
            }
        }
    }
}

template <bool Q80, bool BS16 = false>
__device__ inline void x_fill(const XPre &p0, const float *__restrict__ x, int K, const LdsAct &a) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int nc = (K + 255) >> 8;
    if (x_has(0, K)) x_quant<Q80, BS16>(p0, x_chunk(0, K), K, 4 * wid + (lane >> 4) < nc, a);
    for (int round = 1; 16 * round < nc; ++round) {
        if (!x_has(round, K)) break;
        XPre p;
        const int c = x_chunk(round, K);
        x_load(x, K, c, p);
        x_quant<Q80, BS16>(p, c, K, 16 * round + 4 * wid + (lane >> 4) < nc, a);
    }
}

// fp16 activation row (values already fp16, e.g. SwiGLU's h): the lane's 16
// values of chunk c (clamped as x_load clamps) in two 16-B loads; every
// round is requested before any is quantized. K <= 4096 * kX16Rounds.
constexpr int kX16Rounds = 3;
__device__ inline void x16_load(const uint16_t *__restrict__ x, int K, int c, uint4 (&q)[2]) {
    const int v0 = min(c * 256 + 16 * int(threadIdx.x & 15), K - 16);
    q[0] = ld16(x + v0);
    q[1] = ld16(x + v0 + 8);
}
template <bool Q80, bool BS16 = false>
__device__ inline void x16_fill(const uint4 (&q)[kX16Rounds][2], int K, const LdsAct &a) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int nc = (K + 255) >> 8;
#pragma unroll
    for (int r = 0; r < kX16Rounds; ++r) {
        if (!x_has(r, K)) break;
        XPre p;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t w[4] = {q[r][i].x, q[r][i].y, q[r][i].z, q[r][i].w};
            p.v[2 * i] = make_float4(fp16_bits_to_f32(w[0] & 0xFFFFu), fp16_bits_to_f32(w[0] >> 16),
                                     fp16_bits_to_f32(w[1] & 0xFFFFu), fp16_bits_to_f32(w[1] >> 16));
            p.v[2 * i + 1] = make_float4(fp16_bits_to_f32(w[2] & 0xFFFFu), fp16_bits_to_f32(w[2] >> 16),
                                         fp16_bits_to_f32(w[3] & 0xFFFFu), fp16_bits_to_f32(w[3] >> 16));
        }
        x_quant<Q80, BS16>(p, x_chunk(r, K), K, 16 * r + 4 * wid + (lane >> 4) < nc, a);
    }
}

// Prequantized row: 16-B code chunks, scales and bsum32 per thread.
struct CPre { uint4 q[4]; int32_t bs[2]; float d[2]; };

// BS = false: the 32-code sums are not read (bs may be null)
template <bool Q80, bool BS = true>
__device__ inline void cpre_load(const int8_t *qs, const float *d, const int32_t *bs, int K, CPre &p) {
    const int t = threadIdx.x, t0 = 64 * int(threadIdx.x >> 6);
    const int nq = K >> 4, nd = Q80 ? (K >> 5) : (K >> 8);
    // clamped indices (duplicates are never stored); a load none of whose
    // lanes is in range is not issued (the test is uniform over the wave)
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (t0 + 256 * i < nq) p.q[i] = ld16(qs + 16 * min(t + 256 * i, nq - 1));
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        if constexpr (!Q80 && BS)
            if (t0 + 256 * i < (K >> 5)) p.bs[i] = bs[min(t + 256 * i, (K >> 5) - 1)];
        if (t0 + 256 * i < nd) p.d[i] = d[min(t + 256 * i, nd - 1)];
    }
}

__device__ inline int sum16_codes(uint4 q) {
    return sdot4(int(q.w), 0x01010101, sdot4(int(q.z), 0x01010101, sdot4(int(q.y), 0x01010101, sdot4(int(q.x), 0x01010101, 0))));
}
// BSC: the 32-code sums formed here from the codes (exact integers, the
// quantizer's bsum32) instead of read from the buffer; K <= 16384
template <bool Q80, bool BS16 = false, bool BSC = false>
__device__ inline void cpre_fill(const CPre &p, const int8_t *qs, const float *d, const int32_t *bs,
                                 int K, const LdsAct &a) {
    const int t = threadIdx.x;
    const int nq = K >> 4, nd = Q80 ? (K >> 5) : (K >> 8), nbs = Q80 ? 0 : (K >> 5);
    int8_t *lq = const_cast<int8_t *>(a.qs);
    float *ld = const_cast<float *>(a.d);
    int32_t *lb = const_cast<int32_t *>(a.bs);
    int32_t *l16 = const_cast<int32_t *>(a.bs16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int g = t + 256 * i;
        if (g < nq) {
            *reinterpret_cast<uint4 *>(lq + lds_pad(16 * g)) = p.q[i];
            if constexpr (BS16) l16[bs16_pos(g >> 4, 16 * (g & 15))] = sum16_codes(p.q[i]);
        }
        if constexpr (BSC && !Q80) {
            // codes 16 g .. 16 g + 15 here and 16 (g ^ 1) .. in the lane next door
            const int s16 = g < nq ? sum16_codes(p.q[i]) : 0;
            const int s32 = s16 + dpp_xor1(s16);
            if (g < nq && !(g & 1)) lb[g >> 1] = s32;
        }
    }
    for (int i = t + 1024; i < nq; i += 256) {
        const uint4 q = ld16(qs + 16 * i);
        *reinterpret_cast<uint4 *>(lq + lds_pad(16 * i)) = q;
        if constexpr (BS16) l16[bs16_pos(i >> 4, 16 * (i & 15))] = sum16_codes(q);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        if constexpr (!BSC)
            if (t + 256 * i < nbs) lb[t + 256 * i] = p.bs[i];
        if (t + 256 * i < nd) ld[t + 256 * i] = p.d[i];
    }
    if constexpr (!BSC)
        for (int i = t + 512; i < nbs; i += 256) lb[i] = bs[i];
    for (int i = t + 512; i < nd; i += 256) ld[i] = d[i];
}

// ------------------------------------------------------------ the kernel
constexpr int kGemvR = 4, kGemvU = 5;

// LDS carve-up: padded codes | d | bsum32 (Q8_K only) | bs16 (Q8_K only,
// 16-B aligned) | per-wave block terms and a 64-float dump | per-wave weight
// stage (staged formats)
__host__ __device__ inline size_t gemv_bs16_off(bool q80, int K) {
    const size_t codes = (size_t(lds_pad(K)) + 15) & ~size_t(15);
    const size_t nd = q80 ? size_t(K / 32) : size_t(K / 256);
    const size_t nbs = q80 ? 0 : size_t(K / 32);
    return (codes + 4 * nd + 4 * nbs + 15) & ~size_t(15);
}
__host__ __device__ inline size_t gemv_act_lds_bytes(bool q80, int K) {
    return gemv_bs16_off(q80, K) + (q80 ? 0 : size_t(K / 16) * 4);
}
__device__ inline LdsAct gemv_act_view(uint8_t *lds, bool q80, int K) {
    const size_t codes = (size_t(lds_pad(K)) + 15) & ~size_t(15);
    LdsAct act;
    act.qs = reinterpret_cast<const int8_t *>(lds);
    act.d = reinterpret_cast<const float *>(lds + codes);
    act.bs = reinterpret_cast<const int32_t *>(lds + codes + 4 * (q80 ? K / 32 : K / 256));
    act.bs16 = reinterpret_cast<const int32_t *>(lds + gemv_bs16_off(q80, K));
    return act;
}
template <class F, int U>
__host__ __device__ constexpr int stage_chunks() {  // 16-B loads per lane per batch
    return F::kStaged ? ((64 / F::G) * U * F::BB + 16 + 1023) / 1024 : 0;
}
template <class F, int R, int U>
__host__ __device__ inline size_t gemv_lds_bytes_t(int K) {
    const size_t terms = (size_t(4) * (R * (K / F::QK) + 64) * sizeof(float) + 15) & ~size_t(15);
    return gemv_act_lds_bytes(IsQ80<F>::v, K) + terms + size_t(4) * stage_chunks<F, U>() * 1024;
}

}  // namespace qmm
