// qmm_gemv.hip — batch-1 (M = 1) GEMV over GGUF-packed rows, gfx950.
//
// Work mapping. A wavefront owns R consecutive weight rows; since rows are
// contiguous, its R * nb blocks form one contiguous byte span, processed in
// wave steps of SLOTS = 64 / G blocks (G lanes per block). Each lane unpacks
// its share of a block in registers and forms int32 dot partials with
// v_dot4_i32_i8; the per-block integer partials (S, Mb) are summed over the
// G lanes with DPP — exact and order free — and the block's fp32 term is
// evaluated once with the reference's expression. Block terms go to LDS;
// one lane per row then adds them in block order, the order of
// eval_single_lm_row_dot (E:10986-11105), so the result equals the
// reference's fp32 sum bit for bit.
//
// Weight bytes. Q4_K / Q5_K blocks (144 / 176 B) are 16-B aligned: lanes
// load their pieces straight from HBM with 16-B loads. Q6_K / Q8_0 blocks
// (210 / 34 B) are only 2-B aligned: the wave loads the contiguous bytes of
// U wave steps with 16-B loads into an LDS stage and lanes read their
// pieces from there (two-byte realignment costs LDS reads, not HBM
// transactions).
//
// Activations live in LDS for the whole workgroup. The fp32 input (or the
// prequantized row) is requested first, then the first batch of weights;
// while those are in flight the workgroup quantizes the input to Q8_K /
// Q8_0 itself — 16 lanes per 256 values, DPP reductions, the reference's
// exact arithmetic — so one launch covers quantize + GEMV. Codes are stored
// with 16 B of padding per 256 values so lanes on consecutive blocks hit
// different banks. Vector-memory counters retire in order, so the fill
// waits only for the input loads; the workgroup barrier orders LDS only.
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
// Block (144 B): d f16 @0, dmin f16 @2, scales[12] @4, codes[128] @16.
// Lane k of 8: chunk j = k/2 (64 values), half lh = k%2 -> code bytes
// [16 + 32j + 16lh, +16): low nibbles = values 64j + 16lh + (0..15)
// (sub-block 2j), high nibbles = 64j + 32 + 16lh + (0..15) (sub-block 2j+1).
struct FmtQ4K {
    static constexpr int G = 8, BB = 144, QK = 256;
    static constexpr bool kStaged = false;
    struct Raw { uint4 h, c; };
    struct Act { uint4 xl, xh; uint2 bs; float dx; };
    __device__ static Raw load(const uint8_t *blk, int k) {
        return {ld16_nt(blk), ld16_nt(blk + 16 + 16 * k)};
    }
    __device__ static Act load_act(const LdsAct &x, int b, int k) {
        const int j = k >> 1, lh = k & 1;
        const int8_t *xb = x.qs + b * 272 + 64 * j + 16 * lh;
        return {ld16(xb), ld16(xb + 32), ld8(x.bs + b * 8 + 2 * j), x.d[b]};
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
// Lane k: chunk j = k/2, half lh = k%2 -> ql bytes [48 + 32j + 16lh, +16),
// qh bytes [16 + 16lh, +16); high bit of value 64j + l is bit 2j of qh[l],
// of value 64j + 32 + l bit 2j+1.
struct FmtQ5K {
    static constexpr int G = 8, BB = 176, QK = 256;
    static constexpr bool kStaged = false;
    struct Raw { uint4 h, qh, ql; };
    using Act = FmtQ4K::Act;
    __device__ static Raw load(const uint8_t *blk, int k) {
        const int j = k >> 1, lh = k & 1;
        return {ld16_nt(blk), ld16_nt(blk + 16 + 16 * lh), ld16_nt(blk + 48 + 32 * j + 16 * lh)};
    }
    __device__ static Act load_act(const LdsAct &x, int b, int k) { return FmtQ4K::load_act(x, b, k); }
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

// Prequantized row: 16-B code chunks, scales and bsum32 per thread.
struct CPre { uint4 q[4]; int32_t bs[2]; float d[2]; };

template <bool Q80>
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
        if constexpr (!Q80)
            if (t0 + 256 * i < (K >> 5)) p.bs[i] = bs[min(t + 256 * i, (K >> 5) - 1)];
        if (t0 + 256 * i < nd) p.d[i] = d[min(t + 256 * i, nd - 1)];
    }
}

__device__ inline int sum16_codes(uint4 q) {
    return sdot4(int(q.w), 0x01010101, sdot4(int(q.z), 0x01010101, sdot4(int(q.y), 0x01010101, sdot4(int(q.x), 0x01010101, 0))));
}
template <bool Q80, bool BS16 = false>
__device__ inline void cpre_fill(const CPre &p, const int8_t *qs, const float *d, const int32_t *bs,
                                 int K, const LdsAct &a) {
    const int t = threadIdx.x;
    const int nq = K >> 4, nd = Q80 ? (K >> 5) : (K >> 8), nbs = Q80 ? 0 : (K >> 5);
    int8_t *lq = const_cast<int8_t *>(a.qs);
    float *ld = const_cast<float *>(a.d);
    int32_t *lb = const_cast<int32_t *>(a.bs);
    int32_t *l16 = const_cast<int32_t *>(a.bs16);
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (t + 256 * i < nq) {
            const int g = t + 256 * i;
            *reinterpret_cast<uint4 *>(lq + lds_pad(16 * g)) = p.q[i];
            if constexpr (BS16) l16[bs16_pos(g >> 4, 16 * (g & 15))] = sum16_codes(p.q[i]);
        }
    for (int i = t + 1024; i < nq; i += 256) {
        const uint4 q = ld16(qs + 16 * i);
        *reinterpret_cast<uint4 *>(lq + lds_pad(16 * i)) = q;
        if constexpr (BS16) l16[bs16_pos(i >> 4, 16 * (i & 15))] = sum16_codes(q);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        if (t + 256 * i < nbs) lb[t + 256 * i] = p.bs[i];
        if (t + 256 * i < nd) ld[t + 256 * i] = p.d[i];
    }
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

// R rows per wave, U wave steps of SLOTS blocks per batch.
// FUSED: x32 is quantized in the kernel; otherwise prek / pre0 hold the
// prequantized activation row.
// GRP: several tasks of the type in one launch (a MatGroup argument);
// otherwise one task, passed alone (a smaller argument block).
// NC: 16-B stage loads per lane that a batch needs (at most NST; every
// issued load costs address-unit time even when its lanes are clamped)
// The work of one workgroup (task a, workgroup bx of that task); a device
// function so that a launch of several formats can run it per workgroup.
template <class F, int R, int U, bool FUSED, int NC>
__device__ __attribute__((always_inline)) inline void gemv_wg(const MatArgs &a, int bx, const float *__restrict__ x32,
                                                              const Q8KView &prek, const Q80View &pre0) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int G = F::G, SLOTS = 64 / G, NST = stage_chunks<F, U>();
    constexpr bool q80 = IsQ80<F>::v;
    if (scan_stopped(a.scan)) return;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int g = lane / G, k = lane % G;
    const int K = a.K;
    const int nb = K / F::QK;
    const int row0 = (bx * 4 + wid) * R;
    const int nrows = max(0, min(R, a.N - row0));
    const int nblk = nrows * nb;
    // waves past the last row still issue (discarded) loads of row 0 so the
    // load sequence has no branches
    const uint8_t *span = a.w + size_t(nrows > 0 ? row0 : 0) * a.row_bytes;
    const int flast = max(nblk, 1) - 1;

    const LdsAct act = gemv_act_view(lds, q80, K);
    const size_t act_bytes = gemv_act_lds_bytes(q80, K);
    const size_t terms_bytes = (size_t(4) * (R * nb + 64) * sizeof(float) + 15) & ~size_t(15);
    float *contrib = reinterpret_cast<float *>(lds + act_bytes) + wid * (R * nb + 64);
    float *dump = contrib + R * nb;  // stores of lanes that own no term
    uint8_t *stage = lds + act_bytes + terms_bytes + size_t(wid) * NST * 1024;

    const int8_t *pq = q80 ? pre0.qs : prek.qs;
    const float *pd = q80 ? pre0.d : prek.d;
    const int32_t *pb = prek.bs;

    // Staged formats: the bytes of blocks [t0, t0 + SLOTS*U) of the span, from
    // the 16-B boundary at or below their start; chunk indices are clamped so
    // that every lane issues its loads (duplicates rewrite identical bytes).
    const int span_mis = int(reinterpret_cast<uintptr_t>(span) & 15);
    static_assert(NC <= NST, "stage loads beyond the stage");
    uint4 st[NC > 0 ? NC : 1];
    auto stage_load = [&](int t0) __attribute__((always_inline)) {
        const int nb_batch = max(min(SLOTS * U, nblk - t0), 1);
        const uint8_t *base = span + size_t(t0) * F::BB - span_mis;
        const int nchunks = (span_mis + nb_batch * F::BB + 15) >> 4;
#pragma unroll
        for (int j = 0; j < NC; ++j) st[j] = ld16_nt(base + 16 * min(64 * j + lane, nchunks - 1));
    };
    auto stage_store = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NC; ++j) *reinterpret_cast<uint4 *>(stage + 16 * (64 * j + lane)) = st[j];
    };

    // 1. the activation row into registers
    XPre xp;
    CPre cp;
    if constexpr (FUSED) {
        if (x_has(0, K)) x_load(x32, K, x_chunk(0, K), xp);
    }
    else cpre_load<q80>(pq, pd, pb, K, cp);
    if constexpr (FUSED) wait_vmcnt<0>();  // x before the weights, as in the persistent kernel
    __builtin_amdgcn_sched_barrier(0);  // keep the activation loads first in issue order
    // 2. weights of the first batch
    typename F::Raw raw[U];
    if constexpr (F::kStaged) {
        stage_load(0);
    } else {
#pragma unroll
        for (int u = 0; u < U; ++u) raw[u] = F::load(span + size_t(min(u * SLOTS + g, flast)) * F::BB, k);
    }
    __builtin_amdgcn_sched_barrier(0);
    // 3. activations into LDS while the weights are in flight
    if constexpr (FUSED) x_fill<q80, std::is_same_v<F, FmtQ6K4>>(xp, x32, K, act);
    else cpre_fill<q80, std::is_same_v<F, FmtQ6K4>>(cp, pq, pd, pb, K, act);
    if constexpr (F::kStaged) stage_store();
    lds_barrier();
    // 4. block terms. b = f mod nb advances by SLOTS mod nb per wave step;
    // every lane stores (lanes that own no term into the dump), so the steps
    // are straight-line code the scheduler can overlap.
    const int adv = SLOTS % nb;
    for (int t0 = 0; t0 < nblk; t0 += SLOTS * U) {
        if (t0 > 0) {
            if constexpr (F::kStaged) {
                stage_load(t0);
                // all lanes of this wave are done reading the previous batch
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
                stage_store();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
            } else {
#pragma unroll
                for (int u = 0; u < U; ++u)
                    raw[u] = F::load(span + size_t(min(t0 + u * SLOTS + g, flast)) * F::BB, k);
            }
        }
        int b = (t0 + g) % nb;
        if constexpr (U <= 3) {
            // all steps' operands first (one LDS round trip), then the math
            typename F::Raw rs[U];
            typename F::Act as[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const bool own = t0 + u * SLOTS + g < nblk;
                if constexpr (F::kStaged) rs[u] = F::load(stage + span_mis + (u * SLOTS + g) * F::BB, k);
                else rs[u] = raw[u];
                as[u] = F::load_act(act, own ? b : 0, k);
                b += adv;
                b = b >= nb ? b - nb : b;
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int f = t0 + u * SLOTS + g;
                const float c = F::compute(rs[u], as[u], k);
                *((k == 0 && f < nblk) ? contrib + f : dump + lane) = c;
            }
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int f = t0 + u * SLOTS + g;
                const bool own = f < nblk;
                typename F::Raw r;
                if constexpr (F::kStaged) r = F::load(stage + span_mis + (u * SLOTS + g) * F::BB, k);
                else r = raw[u];
                const float c = F::compute(r, F::load_act(act, own ? b : 0, k), k);
                *((k == 0 && own) ? contrib + f : dump + lane) = c;
                b += adv;
                b = b >= nb ? b - nb : b;
            }
        }
    }
    lds_barrier();
    // 5. per row, blocks in order (eval_single_lm_row_dot's accumulation)
    if (lane < nrows) {
        float acc = 0.0f;
        const float *cr = contrib + lane * nb;
        int b = 0;
        for (; b + 8 <= nb; b += 8) {  // 8 reads in flight, then the adds in order
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = cr[b + i];
#pragma unroll
            for (int i = 0; i < 8; ++i) acc += v[i];
        }
        for (; b < nb; ++b) acc += cr[b];
        const int row = row0 + lane;
        if (a.res) acc = acc + a.res[row];
        a.y[row] = acc;
    }
}

template <class F, int R, int U, bool FUSED, bool GRP, int NC>
__global__ __launch_bounds__(256) void gemv_kernel(std::conditional_t<GRP, MatGroup, MatArgs> grp,
                                                   const float *__restrict__ x32,
                                                   Q8KView prek, Q80View pre0) {
    int bx = int(blockIdx.x);
    if constexpr (GRP) gemv_wg<F, R, U, FUSED, NC>(grp.t[group_task(grp, int(blockIdx.x), bx)], bx, x32, prek, pre0);
    else gemv_wg<F, R, U, FUSED, NC>(grp, bx, x32, prek, pre0);
}

// ------------------------------------------------------- F32 / F16 rows
// sdot_row_f32_batch / sdot_row_f16_batch (E:3410-3440) on the fp16 input
// (x32 rounded to fp16, or the h section of a Q8_K buffer): wave w of
// workgroup bx takes rows (4 bx + w) R .. + R. A lane takes the 16-B pieces
// lane, lane + 64, ... of a row: the wave loads its pieces of the input once
// (NP per lane at a time: all of K = 2560), then streams its rows two at a
// time, every load of both rows issued before any product. Each lane adds
// its products in order, and the wave adds the 64 lane sums by a fixed
// butterfly. The sums' order is not the reference's row order: these
// outputs meet the stated tolerance, not bit equality.
__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
    return v;
}
template <bool F16W, bool FUSED>
__device__ inline void float_x_piece(const float *x32, const uint16_t *xh, int p, float (&xv)[F16W ? 8 : 4]) {
    constexpr int V = F16W ? 8 : 4;
    if constexpr (FUSED) {
#pragma unroll
        for (int h = 0; h < V / 4; ++h) {
            const float4 f = reinterpret_cast<const float4 *>(x32 + V * p)[h];
            xv[4 * h] = round_to_fp16(f.x);
            xv[4 * h + 1] = round_to_fp16(f.y);
            xv[4 * h + 2] = round_to_fp16(f.z);
            xv[4 * h + 3] = round_to_fp16(f.w);
        }
    } else {
        uint32_t hw[V / 2];
        if constexpr (F16W) {
            const uint4 q = ld16(xh + V * p);
            hw[0] = q.x; hw[1] = q.y; hw[2] = q.z; hw[3] = q.w;
        } else {
            const uint2 q = ld8(xh + V * p);
            hw[0] = q.x; hw[1] = q.y;
        }
#pragma unroll
        for (int i = 0; i < V / 2; ++i) {
            xv[2 * i] = fp16_bits_to_f32(hw[i] & 0xFFFFu);
            xv[2 * i + 1] = fp16_bits_to_f32(hw[i] >> 16);
        }
    }
}
template <bool F16W>
__device__ inline float float_piece_dot(const uint4 &wq, const float (&xv)[F16W ? 8 : 4], float acc) {
    const uint32_t ww[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (F16W) {
            const float p0 = fp16_bits_to_f32(ww[i] & 0xFFFFu) * xv[2 * i];  // E:3436 (products rounded, then added)
            acc = acc + p0;
            const float p1 = fp16_bits_to_f32(ww[i] >> 16) * xv[2 * i + 1];
            acc = acc + p1;
        } else {
            const float p0 = __builtin_bit_cast(float, ww[i]) * xv[i];  // E:3420
            acc = acc + p0;
        }
    }
    return acc;
}
template <bool F16W, int R, bool FUSED>
__device__ __attribute__((always_inline)) inline void gemv_float_wg(const MatArgs &a, int bx, const float *x32,
                                                                    const uint16_t *xh) {
    constexpr int V = F16W ? 8 : 4;
    constexpr int NP = F16W ? 5 : 10;  // pieces per lane held at once (K = 2560)
    if (scan_stopped(a.scan)) return;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int npc = a.K / V;            // pieces per row
    const int row0 = (bx * 4 + wid) * R;
    const int nrows = max(0, min(R, a.N - row0));
    if (nrows == 0) return;  // the same in every lane of the wave
    float acc[R];
#pragma unroll
    for (int j = 0; j < R; ++j) acc[j] = 0.0f;
    for (int b0 = 0; b0 < npc; b0 += 64 * NP) {
        float xv[NP][V];
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int p = b0 + lane + 64 * i;
            if (p < npc) float_x_piece<F16W, FUSED>(x32, xh, p, xv[i]);
        }
#pragma unroll
        for (int j = 0; j < R; j += 2) {
            if (j >= nrows) break;  // the same in every lane of the wave
            const bool two = j + 1 < nrows;
            const uint8_t *w0 = a.w + size_t(row0 + j) * a.row_bytes;
            const uint8_t *w1 = a.w + size_t(row0 + (two ? j + 1 : j)) * a.row_bytes;
            uint4 q0[NP], q1[NP];
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const int p = b0 + lane + 64 * i;
                if (p < npc) {
                    q0[i] = ld16_nt(w0 + 16 * size_t(p));
                    if constexpr (R > 1) q1[i] = ld16_nt(w1 + 16 * size_t(p));
                }
            }
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const int p = b0 + lane + 64 * i;
                if (p < npc) {
                    acc[j] = float_piece_dot<F16W>(q0[i], xv[i], acc[j]);
                    if constexpr (R > 1)
                        if (j + 1 < R) acc[j + 1] = float_piece_dot<F16W>(q1[i], xv[i], acc[j + 1]);
                }
            }
        }
    }
#pragma unroll
    for (int j = 0; j < R; ++j) {
        if (j >= nrows) break;
        const float v = wave_sum(acc[j]);
        if (lane == 0) {
            const int row = row0 + j;
            a.y[row] = a.res ? v + a.res[row] : v;
        }
    }
}

// ------------------------------------------------- several formats at once
// A task group whose types differ (the engine's {qkv, gate, alpha, beta} and
// {q, k, v} groups, E:7954-7959, E:8110-8114) in one launch: each workgroup
// runs the body of its own task's format. The dynamic LDS is the largest any
// of the group's formats needs; every workgroup fills its own activations.
template <int R, bool FUSED>
__global__ __launch_bounds__(256) void gemv_mixed_kernel(MatGroup grp, const float *__restrict__ x32, Q8KView prek,
                                                         Q80View pre0) {
    int bx = 0;
    const MatArgs a = grp.t[group_task(grp, int(blockIdx.x), bx)];
    switch (a.type) {
        case kQ4_K: gemv_wg<FmtQ4K4, R, 3, FUSED, stage_chunks<FmtQ4K4, 3>()>(a, bx, x32, prek, pre0); break;
        case kQ5_K: gemv_wg<FmtQ5K, R, kGemvU, FUSED, 0>(a, bx, x32, prek, pre0); break;
        case kQ6_K: gemv_wg<FmtQ6K4, R, 3, FUSED, stage_chunks<FmtQ6K4, 3>()>(a, bx, x32, prek, pre0); break;
        case kQ8_0: gemv_wg<FmtQ80, R, kGemvU, FUSED, stage_chunks<FmtQ80, kGemvU>()>(a, bx, x32, prek, pre0); break;
        // F32 / F16 rows: one row per wave whatever the group's R (their
        // bytes per row are 4-8x a k-quant's; more workgroups share them)
        case kF32: gemv_float_wg<false, 1, FUSED>(a, bx, x32, prek.h); break;
        case kF16: gemv_float_wg<true, 1, FUSED>(a, bx, x32, prek.h); break;
        default: break;
    }
}

// --------------------------------------------- persistent batch-1 kernel
// For one task with many more row groups than workgroups fit at once (the
// LM head). A fixed grid: wave w of workgroup i takes the R-row groups
// (i + j G) * 4 + w, j = 0, 1, ...; the activation row is filled once per
// workgroup, and a wave loads its next group's bytes into registers while it
// computes the current one (one batch per group: R nb <= SLOTS U). After the
// fill the waves never synchronize with each other.
template <class F, int R, int U, bool FUSED, int NC, bool AMAX>
__global__ __launch_bounds__(256) void gemv_persist_kernel(MatArgs a, const float *__restrict__ x32,
                                                           Q8KView prek, Q80View pre0, AmaxOut am) {
    extern __shared__ __align__(16) uint8_t lds[];
    static_assert(F::kStaged, "the persistent kernel stages its rows in LDS");
    constexpr int G = F::G, SLOTS = 64 / G, NST = stage_chunks<F, U>();
    constexpr bool q80 = IsQ80<F>::v;
    if (scan_stopped(a.scan)) return;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int g = lane / G, k = lane % G;
    const int K = a.K, nb = K / F::QK;
    const int ngroups = (a.N + R - 1) / R;

    const LdsAct act = gemv_act_view(lds, q80, K);
    const size_t act_bytes = gemv_act_lds_bytes(q80, K);
    const size_t terms_bytes = (size_t(4) * (R * nb + 64) * sizeof(float) + 15) & ~size_t(15);
    float *contrib = reinterpret_cast<float *>(lds + act_bytes) + wid * (R * nb + 64);
    float *dump = contrib + R * nb;
    uint8_t *stage = lds + act_bytes + terms_bytes + size_t(wid) * NST * 1024;

    const int8_t *pq = q80 ? pre0.qs : prek.qs;
    const float *pd = q80 ? pre0.d : prek.d;
    const int32_t *pb = prek.bs;

    // a group's bytes from the 16-B boundary at or below its first byte;
    // chunk indices clamped so every lane issues its loads
    static_assert(NC <= NST, "stage loads beyond the stage");
    uint4 st[NC];
    auto stage_load = [&](int gr) __attribute__((always_inline)) {
        const int rows = max(0, min(R, a.N - gr * R));
        const uint8_t *span = a.w + size_t(rows > 0 ? gr * R : 0) * a.row_bytes;
        const int mis = int(reinterpret_cast<uintptr_t>(span) & 15);
        const int nchunks = (mis + max(rows * nb, 1) * F::BB + 15) >> 4;
#pragma unroll
        for (int j = 0; j < NC; ++j) st[j] = ld16_nt(span - mis + 16 * min(64 * j + lane, nchunks - 1));
    };

    int gw = int(blockIdx.x) * 4 + wid;
    const int stride = int(gridDim.x) * 4;
    // 0. a scan's step after the previous chunk (the partials are requested
    // ahead of the activations; the decision precedes every weight request,
    // so a chunk the step stops reads no weights)
    Best pb4[4];
    if constexpr (AMAX) {
        if (am.pre.part) {
            const Best *pp = static_cast<const Best *>(am.pre.part);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int e = int(threadIdx.x) + 256 * i;
                pb4[i] = e < am.pre.nparts ? pp[e] : Best{-INFINITY, kNone};
            }
        }
    }
    // 1. the activation row, then the first group's bytes
    XPre xp;
    CPre cp;
    if constexpr (FUSED) {
        if (x_has(0, K)) x_load(x32, K, x_chunk(0, K), xp);
    }
    else cpre_load<q80>(pq, pd, pb, K, cp);
    if constexpr (AMAX) {
        if (am.pre.part) {
            __shared__ Best psh[4];
            __shared__ int pstop;
            Best b = better(better(pb4[0], pb4[1]), better(pb4[2], pb4[3]));  // slices e, e + 256, ... in order
            b = block_best(b, psh);
            const PrevStep &q = am.pre;
            if (threadIdx.x == 0) {
                // the running best of token 0 (E:11177), then the threshold test (E:11248-11256)
                float bv = q.best_val[0];
                uint32_t bi = q.best_id[0];
                const int act = scan_active(q.st, 1);
                if (act > 0 && b.i != kNone && b.v > bv) {
                    bv = b.v;
                    bi = q.row_base + b.i;
                }
                const int stop = q.checkpoint && (act == 0 || !(bv < q.thresh));
                pstop = stop;
                if (blockIdx.x == 0) {
                    q.best_val[0] = bv;
                    q.best_id[0] = bi;
                    q.st[kScanChunks] = q.c + 1;
                    if (stop) q.st[kScanStopped] = 1;
                }
            }
            __syncthreads();
            if (pstop) return;
        }
    }
    // a wave that loads x waits for it before it requests weights (measured:
    // weights first 5.09 us, x first 4.88; all waves held until x is in
    // 5.20): x is the critical path and weight requests slow its arrival
    if constexpr (FUSED) wait_vmcnt<0>();
    __builtin_amdgcn_sched_barrier(0);
    stage_load(min(gw, ngroups - 1));
    __builtin_amdgcn_sched_barrier(0);
    // 2. the activations into LDS, once
    if constexpr (FUSED) x_fill<q80, std::is_same_v<F, FmtQ6K4>>(xp, x32, K, act);
    else cpre_fill<q80, std::is_same_v<F, FmtQ6K4>>(cp, pq, pd, pb, K, act);
    lds_barrier();
    // 3. groups
    const int adv = SLOTS % nb;
    Best wb{-INFINITY, kNone};  // AMAX: the wave's running (max, first row)
    for (; gw < ngroups; gw += stride) {
        const int row0 = gw * R;
        const int nrows = min(R, a.N - row0);
        const int nblk = nrows * nb;
        const int mis = int(reinterpret_cast<uintptr_t>(a.w + size_t(row0) * a.row_bytes) & 15);
        // all lanes of this wave are done with the previous group's stage and terms
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
#pragma unroll
        for (int j = 0; j < NC; ++j) *reinterpret_cast<uint4 *>(stage + 16 * (64 * j + lane)) = st[j];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
        // the next group, in flight during the math (none for a wave's last:
        // a clamped duplicate would cost the address units as much as a new one)
        if (gw + stride < ngroups) stage_load(gw + stride);
        int b = g % nb;
        typename F::Raw rs[U];
        typename F::Act as[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const bool own = u * SLOTS + g < nblk;
            rs[u] = F::load(stage + mis + (u * SLOTS + g) * F::BB, k);
            as[u] = F::load_act(act, own ? b : 0, k);
            b += adv;
            b = b >= nb ? b - nb : b;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int f = u * SLOTS + g;
            const float c = F::compute(rs[u], as[u], k);
            *((k == 0 && f < nblk) ? contrib + f : dump + lane) = c;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
        // per row, blocks in order (eval_single_lm_row_dot's accumulation)
        if (lane < nrows) {
            float acc = 0.0f;
            const float *cr = contrib + lane * nb;
            int bb = 0;
            for (; bb + 8 <= nb; bb += 8) {
                float v[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = cr[bb + i];
#pragma unroll
                for (int i = 0; i < 8; ++i) acc += v[i];
            }
            for (; bb < nb; ++bb) acc += cr[bb];
            const int row = row0 + lane;
            if (a.res) acc = acc + a.res[row];
            if constexpr (AMAX)
                if (am.ids && am.ids[row] >= am.id_limit) acc = -1e30f;  // a row past the tensor (E:11150)
            a.y[row] = acc;
            if constexpr (AMAX) {
                const float v = am.round16 ? round_to_fp16(acc) : acc;  // as the argmax kernels compare
                if (v == v) wb = better(wb, Best{v, uint32_t(row)});
            }
        }
    }
    if constexpr (AMAX) {  // one partial per workgroup (per wave was slower: 4x the partials to combine)
        __shared__ Best wsb[4];
        wb = wave_best(wb);
        if (lane == 0) wsb[wid] = wb;
        __syncthreads();
        if (threadIdx.x == 0) {
            Best r = wsb[0];
            for (int w = 1; w < 4; ++w) r = better(r, wsb[w]);
            static_cast<Best *>(am.part)[blockIdx.x] = r;
        }
    }
}

size_t gemv_lds_bytes(uint32_t type, int K) {
    switch (type) {
        case kQ4_K: return gemv_lds_bytes_t<FmtQ4K4, kGemvR, 3>(K);
        case kQ5_K: return gemv_lds_bytes_t<FmtQ5K, kGemvR, kGemvU>(K);
        case kQ6_K: return gemv_lds_bytes_t<FmtQ6K4, kGemvR, 3>(K);
        case kQ8_0: return gemv_lds_bytes_t<FmtQ80, kGemvR, kGemvU>(K);
        default: return 0;
    }
}

// CUs of the current device (cached per device; concurrent first calls store
// the same value)
static int cu_count() {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}
// Calls launch(std::integral_constant<int, NC>) with the fewest 16-B stage
// loads per lane (NST - 2 .. NST) that cover a batch of `blocks` blocks from
// any 16-B misalignment.
template <class F, int U, class L>
static hipError_t with_stage_chunks(int blocks, L &&launch) {
    constexpr int NST = stage_chunks<F, U>();
    const int need = ((15 + blocks * F::BB + 15) / 16 + 63) / 64;
    if constexpr (NST >= 3)
        if (need <= NST - 2) return launch(std::integral_constant<int, NST - 2>{});
    if constexpr (NST >= 2)
        if (need <= NST - 1) return launch(std::integral_constant<int, NST - 1>{});
    return launch(std::integral_constant<int, NST>{});
}

template <class F, int R, int U, bool AMAX = false>
static hipError_t launch_gemv_persist_t(const MatArgs &a, const float *x32, const Q8KView &xk, const Q80View &x0,
                                        size_t lds, int wgs, hipStream_t s, AmaxOut am = {}) {
    const dim3 grid{unsigned(wgs)};
    return with_stage_chunks<F, U>(R * (a.K / F::QK), [&](auto nc) {
        constexpr int NC = decltype(nc)::value;
        if (x32) hipLaunchKernelGGL((gemv_persist_kernel<F, R, U, true, NC, AMAX>), grid, dim3(256), lds, s, a, x32, xk, x0, am);
        else hipLaunchKernelGGL((gemv_persist_kernel<F, R, U, false, NC, AMAX>), grid, dim3(256), lds, s, a, x32, xk, x0, am);
        return hipGetLastError();
    });
}

// The persistent grid of one task (R = kGemvR) with the running argmax
// fused; NotSupported (nothing launched) where that grid does not apply.
template <class F, int U>
static hipError_t launch_gemv_argmax_t(const MatArgs &a, const Q8KView &xk, const Q80View &x0, bool round16,
                                       const uint32_t *ids, uint32_t id_limit, void *part, int *nparts,
                                       hipStream_t s, const PrevStep &pre) {
    constexpr int R = kGemvR;
    const int nb = a.K / F::QK, cus = cu_count();
    const int wg0 = ((a.N + R - 1) / R + 3) / 4;
    if (a.N < (IsQ80<F>::v ? 8192 : 4096) || R * nb > (64 / F::G) * U || wg0 < 2 * cus) return hipErrorNotSupported;
    const int wgs = min(3 * cus, wg0 * 5 / 8);
    if (wgs > kMaxArgmaxParts || (pre.part && pre.nparts > 1024)) return hipErrorNotSupported;
    *nparts = wgs;
    return launch_gemv_persist_t<F, R, U, true>(a, nullptr, xk, x0, gemv_lds_bytes_t<F, R, U>(a.K), wgs, s,
                                                AmaxOut{part, round16 ? 1 : 0, ids, id_limit, pre});
}

hipError_t launch_gemv_argmax(uint32_t type, const MatArgs &a, const Q8KView &xk, const Q80View &x0, bool round16,
                              const uint32_t *ids, uint32_t id_limit, void *part, int *nparts, hipStream_t s,
                              const PrevStep &pre) {
    switch (type) {
        case kQ4_K: return launch_gemv_argmax_t<FmtQ4K4, 3>(a, xk, x0, round16, ids, id_limit, part, nparts, s, pre);
        case kQ6_K: return launch_gemv_argmax_t<FmtQ6K4, 3>(a, xk, x0, round16, ids, id_limit, part, nparts, s, pre);
        default: return hipErrorNotSupported;  // Q8_0 takes the persistent grid only at K <= 320
    }
}

template <class F, int R, int U>
static hipError_t launch_gemv_t(const MatArgs *tasks, int n, const float *x32, const Q8KView &xk,
                                const Q80View &x0, hipStream_t s) {
    MatGroup g{};
    g.n = n;
    g.wg0[0] = 0;
    for (int i = 0; i < n; ++i) {
        g.t[i] = tasks[i];
        g.wg0[i + 1] = g.wg0[i] + ((tasks[i].N + R - 1) / R + 3) / 4;  // 4 waves of R rows
    }
    const size_t lds = gemv_lds_bytes_t<F, R, U>(tasks[0].K);
    const dim3 grid(unsigned(g.wg0[n]));
    // one task of at least two workgroups' rows per CU: a persistent grid of
    // 5/8 of a workgroup per row group, at most 3 per CU (measured: 380
    // workgroups for 608 groups, 768 for the 9496 of the LM head)
    if constexpr (F::kStaged) {
        const int nb = tasks[0].K / F::QK;
        const int cus = cu_count();
        if (n == 1 && R * nb <= (64 / F::G) * U && g.wg0[1] >= 2 * cus) {
            const int wgs = min(3 * cus, g.wg0[1] * 5 / 8);
            return launch_gemv_persist_t<F, R, U>(tasks[0], x32, xk, x0, lds, wgs, s);
        }
    }
    const int blocks = min(R * (tasks[0].K / F::QK), (64 / F::G) * U);
    return with_stage_chunks<F, U>(blocks, [&](auto nc) {
        constexpr int NC = decltype(nc)::value;
        if (n == 1) {
            if (x32) hipLaunchKernelGGL((gemv_kernel<F, R, U, true, false, NC>), grid, dim3(256), lds, s, g.t[0], x32, xk, x0);
            else hipLaunchKernelGGL((gemv_kernel<F, R, U, false, false, NC>), grid, dim3(256), lds, s, g.t[0], x32, xk, x0);
        } else {
            if (x32) hipLaunchKernelGGL((gemv_kernel<F, R, U, true, true, NC>), grid, dim3(256), lds, s, g, x32, xk, x0);
            else hipLaunchKernelGGL((gemv_kernel<F, R, U, false, true, NC>), grid, dim3(256), lds, s, g, x32, xk, x0);
        }
        return hipGetLastError();
    });
}

// Rows per wave by the launch's total rows and K (measured per shape): the
// k-quants take 4 from 4096 rows, else 2 up to K = 4096, else 1 (the 2560-row
// K = 9728 down projection: 12.4 -> 8.9 us with 1); Q8_0 (34-B blocks, 5
// wave steps per batch) takes 4 from 8192 rows, 2 from 4096, else 1.
template <class F, int U>
static hipError_t launch_gemv_rows(const MatArgs *tasks, int n, const float *x32, const Q8KView &xk,
                                   const Q80View &x0, hipStream_t s) {
    int64_t rows = 0;
    for (int i = 0; i < n; ++i) rows += tasks[i].N;
    const bool q80 = IsQ80<F>::v;
    if (rows >= (q80 ? 8192 : 4096)) return launch_gemv_t<F, kGemvR, U>(tasks, n, x32, xk, x0, s);
    if (q80 ? rows >= 4096 : tasks[0].K <= 4096) return launch_gemv_t<F, 2, U>(tasks, n, x32, xk, x0, s);
    return launch_gemv_t<F, 1, U>(tasks, n, x32, xk, x0, s);
}

// dynamic LDS of one format's body at R rows per wave (F32 / F16: none)
template <int R>
static size_t gemv_wg_lds(uint32_t type, int K) {
    switch (type) {
        case kQ4_K: return gemv_lds_bytes_t<FmtQ4K4, R, 3>(K);
        case kQ5_K: return gemv_lds_bytes_t<FmtQ5K, R, kGemvU>(K);
        case kQ6_K: return gemv_lds_bytes_t<FmtQ6K4, R, 3>(K);
        case kQ8_0: return gemv_lds_bytes_t<FmtQ80, R, kGemvU>(K);
        default: return 0;
    }
}

template <int R>
static hipError_t launch_gemv_mixed_r(const MatArgs *tasks, int n, const float *x32, const Q8KView &xk,
                                      const Q80View &x0, hipStream_t s) {
    MatGroup g{};
    g.n = n;
    g.wg0[0] = 0;
    size_t lds = 0;
    for (int i = 0; i < n; ++i) {
        g.t[i] = tasks[i];
        const int r = (tasks[i].type == kF32 || tasks[i].type == kF16) ? 1 : R;  // rows per wave
        g.wg0[i + 1] = g.wg0[i] + ((tasks[i].N + r - 1) / r + 3) / 4;
        lds = max(lds, gemv_wg_lds<R>(tasks[i].type, tasks[i].K));
    }
    const dim3 grid(unsigned(g.wg0[n]));
    if (x32) hipLaunchKernelGGL((gemv_mixed_kernel<R, true>), grid, dim3(256), lds, s, g, x32, xk, x0);
    else hipLaunchKernelGGL((gemv_mixed_kernel<R, false>), grid, dim3(256), lds, s, g, x32, xk, x0);
    return hipGetLastError();
}

hipError_t launch_gemv_mixed(const MatArgs *tasks, int n, const float *x32, const Q8KView &xk, const Q80View &x0,
                             hipStream_t s) {
    if (n < 1 || n > kMaxGroup) return hipErrorInvalidValue;
    int64_t rows = 0;
    for (int i = 0; i < n; ++i) rows += tasks[i].N;
    // rows per wave as for one k-quant launch of the group's size
    if (rows >= 4096) return launch_gemv_mixed_r<kGemvR>(tasks, n, x32, xk, x0, s);
    if (tasks[0].K <= 4096) return launch_gemv_mixed_r<2>(tasks, n, x32, xk, x0, s);
    return launch_gemv_mixed_r<1>(tasks, n, x32, xk, x0, s);
}

size_t gemv_mixed_lds_bytes(uint32_t type, int K) {
    return max(gemv_wg_lds<kGemvR>(type, K), max(gemv_wg_lds<2>(type, K), gemv_wg_lds<1>(type, K)));
}

hipError_t launch_gemv(uint32_t type, const MatArgs *tasks, int n, const float *x32, const Q8KView &xk,
                       const Q80View &x0, hipStream_t s) {
    if (n < 1 || n > kMaxGroup) return hipErrorInvalidValue;
    switch (type) {
        case kQ4_K: return launch_gemv_rows<FmtQ4K4, 3>(tasks, n, x32, xk, x0, s);
        case kQ5_K: return launch_gemv_rows<FmtQ5K, kGemvU>(tasks, n, x32, xk, x0, s);
        case kQ6_K: return launch_gemv_rows<FmtQ6K4, 3>(tasks, n, x32, xk, x0, s);
        case kQ8_0: return launch_gemv_rows<FmtQ80, kGemvU>(tasks, n, x32, xk, x0, s);
        case kF32:
        case kF16: return launch_gemv_mixed(tasks, n, x32, xk, x0, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace qmm
