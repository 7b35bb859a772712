// qmm_kformats.h — the GGUF k-quant / Q8_0 formats as int8 MFMA operands
// (gfx950), shared by the small-M and prefill GEMM kernels: per-format
// block loads, B-operand unpacking with the unit scales folded in, scale /
// min decoding, and the MFMA wrappers.
#pragma once

#include "qmm_device.h"

namespace qmm {

typedef int int4v __attribute__((ext_vector_type(4)));

__device__ inline int4v mfma16x16x32(uint2 a, uint2 b) {
    const long av = (long)(((uint64_t)a.y << 32) | a.x);
    const long bv = (long)(((uint64_t)b.y << 32) | b.x);
    const int4v z = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bv, z, 0, 0, 0);
}

// ---------------------------------------------------------------- formats
// Each format gives, for lane k-slice c (0..3) of one weight row's block:
//   NU units; B operand (8 int8) and integer scale of unit u; the k offset
//   (inside the block) of the lane's 8 activation values for unit u; and
//   the block's fp32 update.

// Q4_K: unit u = sub-block 2j + h; lane c holds values 64j + 32h + 8c + t.
struct MQ4K {
    static constexpr int NU = 8, QK = 256, BB = 144;
    static constexpr bool kMin = true, kSplit = false;
    struct W { uint4 h; uint2 q[4]; };
    __device__ static W load(const uint8_t *blk, int c) {
        W w;
        w.h = ld16(blk);
#pragma unroll
        for (int j = 0; j < 4; ++j) w.q[j] = ld8(blk + 16 + 32 * j + 8 * c);
        return w;
    }
    __device__ static W load_lds(const uint8_t *blk, int c) { return load(blk, c); }
    __device__ static int koff(int u, int c) { return 64 * (u >> 1) + 32 * (u & 1) + 8 * c; }
    __device__ static uint2 bop(const W &w, int u, int c) {
        (void)c;
        const uint2 q = w.q[u >> 1];
        const int sh = 4 * (u & 1);
        return make_uint2((q.x >> sh) & 0x0F0F0F0Fu, (q.y >> sh) & 0x0F0F0F0Fu);
    }
};

// Q5_K: as Q4_K with the high bit u of qh[8c + t].
struct MQ5K {
    static constexpr int NU = 8, QK = 256, BB = 176;
    static constexpr bool kMin = true, kSplit = false;
    struct W { uint4 h; uint2 qh; uint2 q[4]; };
    __device__ static W load(const uint8_t *blk, int c) {
        W w;
        w.h = ld16(blk);
        w.qh = ld8(blk + 16 + 8 * c);
#pragma unroll
        for (int j = 0; j < 4; ++j) w.q[j] = ld8(blk + 48 + 32 * j + 8 * c);
        return w;
    }
    __device__ static W load_lds(const uint8_t *blk, int c) { return load(blk, c); }
    __device__ static int koff(int u, int c) { return MQ4K::koff(u, c); }
    __device__ static uint2 bop(const W &w, int u, int c) {
        (void)c;
        const uint2 q = w.q[u >> 1];
        const int sh = 4 * (u & 1);
        return make_uint2(((q.x >> sh) & 0x0F0F0F0Fu) | (((w.qh.x >> u) & 0x01010101u) << 4),
                          ((q.y >> sh) & 0x0F0F0F0Fu) | (((w.qh.y >> u) & 0x01010101u) << 4));
    }
};

// Q6_K block constants; the kernels use the folded form MQ6KS below at
// every M (sixteen 16-value scale groups would leave half of each
// 16x16x32 MFMA's k-slices empty).
struct MQ6K {
    static constexpr int NU = 16, QK = 256, BB = 210;
    static constexpr bool kMin = false, kSplit = false;
};

// Q8_0: one unit per 32-value block; lane c holds values 8c + t.
struct MQ80 {
    static constexpr int NU = 1, QK = 32, BB = 34;
    static constexpr bool kMin = false, kSplit = false;
    struct W { uint2 q; uint32_t d; };
    __device__ static W load(const uint8_t *blk, int c) { return {ld8_a2(blk + 2 + 8 * c), ld16b_a2(blk)}; }
    // blk in LDS, 2-B aligned (misalignment sh = 0 or 2): the codes at blk + 2 +
    // 8 c start sh ^ 2 bytes into dword 2 c + sh / 2 of blk - sh; the third
    // dword is read whatever the shift (at most 4 B past the block, inside the
    // staged bytes' region)
    __device__ static W load_lds(const uint8_t *blk, int c) {
        const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(blk) & 3), s2 = sh ^ 2u;
        const uint32_t *q = reinterpret_cast<const uint32_t *>(blk - sh);
        const uint32_t *p = q + 2 * c + (sh >> 1);
        const uint32_t w0 = p[0], w1 = p[1], w2 = p[2];
        return {make_uint2(funnel(w1, w0, s2), funnel(w2, w1, s2)), (q[0] >> (8 * sh)) & 0xFFFFu};
    }
    __device__ static int koff(int u, int c) { (void)u; return 8 * c; }
    __device__ static uint2 bop(const W &w, int u, int c) { (void)u; (void)c; return w.q; }
};

// Q4_K with the unit scales folded into the B operand (token tiles >= 2 per
// wave): sc = 8 sh + sl with sh, sl in 0..7, so q * sh and q * sl (q <= 15)
// are int8 (<= 105) and, byte by byte, one packed 16-bit multiply each (no
// byte product reaches 256). Over one 64-value chunk h (units 2h, 2h+1) a
// v_mfma_i32_16x16x64_i8 chain accumulates sum a*q*sh (D1), sum a*q*sl (D2)
// and sum a*m (Dm, broadcast mins) across the block's 4 chunks, all exact:
// S = 8 D1 + D2, Mb = Dm. A lane's 16 bytes per chunk are values
// 64h + 8c + t (low nibbles, unit 2h) and 64h + 32 + 8c + t (high nibbles,
// unit 2h + 1), t < 8, in both operands.
struct MQ4KS : MQ4K {
    static constexpr bool kSplit = true;
    static constexpr int kShift = 3;  // S = (D1 << 3) + D2
};

// Q5_K with the unit scales folded into the B operand: w = q * sc <= 1953;
// in 16-bit lanes P = w + 128 and w = 256 hi + lo, hi = P's high byte,
// lo = P's low byte xor 0x80 (as for Q6_K below): S = 256 D1 + D2, plus the
// mins chain of Q4_K. Same value placement as Q4_K (the high bit of value
// 64h + 32k + 8c + t is bit 2h + k of qh[8c + t]).
struct MQ5KS : MQ5K {
    static constexpr bool kSplit = true;
    static constexpr int kShift = 8;  // S = (D1 << 8) + D2
};

// Q6_K with the scales folded into the B operand (at every M): w = (q - 32)
// * sc lies in [-4064, 4096]; in 16-bit lanes
// P = w + 128 = q * sc + (128 - 32 sc) (one packed multiply-add), and
// w = 256 hi + lo with hi = the high byte of P (|hi| <= 16) and
// lo = (P mod 256) - 128, i.e. P's low byte xor 0x80: two int8 operands,
// S = 256 D1 + D2 over two K=64 chains, exact.
// Lane group c holds, per half hf, values 32 i + 8 c + t (t < 8) of every
// i = 0..3; chunk h = 2 hf + ip takes i = 2 ip (ql[64 hf + l], nibble 4 ip,
// qh[32 hf + l] bits 4 ip) and i = 2 ip + 1 (ql[64 hf + 32 + l], nibble 4 ip,
// qh bits 4 ip + 2), so the chunk's values are 64 h + 8 c + t and
// 64 h + 32 + 8 c + t as for Q4_K; value 32 i + l of half hf has scale
// sc[8 hf + 2 i + l / 16] with l / 16 = c / 2 (block layout: E:673-700).
struct MQ6KS : MQ6K {
    static constexpr bool kSplit = true;
    static constexpr int kShift = 8;  // S = (D1 << 8) + D2
    struct W { uint2 a[2], b[2], qh[2]; uint2 s0, s1; uint32_t d; };
    // Every field lies a multiple of 8 B from the 2-B aligned block start, so
    // one misalignment (0 or 2 B) serves all: each 8-B field is three dword
    // reads and two funnel shifts, the third dword read whatever the
    // misalignment (at most bytes 208..211 of the block: the staged row
    // holds them).
    __device__ static W load_lds(const uint8_t *blk, int c) {
        const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(blk) & 3);
        const uint32_t *q = reinterpret_cast<const uint32_t *>(blk - sh);
        auto rd8 = [&](int dw) __attribute__((always_inline)) {
            const uint32_t w0 = q[dw], w1 = q[dw + 1], w2 = q[dw + 2];
            return make_uint2(funnel(w1, w0, sh), funnel(w2, w1, sh));
        };
        W w;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            w.a[hf] = rd8(16 * hf + 2 * c);
            w.b[hf] = rd8(16 * hf + 8 + 2 * c);
            w.qh[hf] = rd8(32 + 8 * hf + 2 * c);
        }
        w.s0 = rd8(48);
        w.s1 = rd8(50);
        w.d = (q[52] >> (8 * sh)) & 0xFFFFu;
        return w;
    }
};

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ inline int4v mfma16x16x64(const uint4 &a, const uint4 &b, int4v c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(int4v, a), __builtin_bit_cast(int4v, b), c,
                                                 0, 0, 0);
}
typedef short s16x2 __attribute__((ext_vector_type(2)));
// B operands of one row tile's block: [chunk][high part | low part | mins]
struct SplitB { uint4 b1[4], b2[4], bm[4]; };
// byte b of w in both 16-bit halves / in all four bytes
__device__ inline u16x2 byte_pair(uint32_t w, int b) {
    return __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(0u, w, 0x0C000C00u | (uint32_t(b) * 0x00010001u)));
}
__device__ inline uint32_t byte_bcast(uint32_t w, int b) { return __builtin_amdgcn_perm(0u, w, uint32_t(b) * 0x01010101u); }
__device__ inline uint32_t bytes_times(uint32_t q, u16x2 f) {  // per byte, q_b * f < 256
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, q) * f);
}
// scw / mw: the 8 scales / mins of the block four to a dword (sub-block u is
// byte u & 3 of word u >> 2, as scales_k4_packed gives them); a scale
// s = 8 (s >> 3) + (s & 7) splits into the high and low parts per byte at once
__device__ inline void split_b(const MQ4K::W &w, const uint32_t (&scw)[2], const uint32_t (&mw)[2], SplitB &o) {
    const uint32_t shw[2] = {(scw[0] >> 3) & 0x07070707u, (scw[1] >> 3) & 0x07070707u};
    const uint32_t slw[2] = {scw[0] & 0x07070707u, scw[1] & 0x07070707u};
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        const uint2 q = w.q[h];
        const int d = h >> 1, b0 = 2 * (h & 1), b1 = b0 + 1;  // sub-blocks 2h, 2h + 1
        const uint32_t lo0 = q.x & 0x0F0F0F0Fu, lo1 = q.y & 0x0F0F0F0Fu;
        const uint32_t hi0 = (q.x >> 4) & 0x0F0F0F0Fu, hi1 = (q.y >> 4) & 0x0F0F0F0Fu;
        const u16x2 sh0 = byte_pair(shw[d], b0), sl0 = byte_pair(slw[d], b0);
        const u16x2 sh1 = byte_pair(shw[d], b1), sl1 = byte_pair(slw[d], b1);
        o.b1[h] = make_uint4(bytes_times(lo0, sh0), bytes_times(lo1, sh0), bytes_times(hi0, sh1), bytes_times(hi1, sh1));
        o.b2[h] = make_uint4(bytes_times(lo0, sl0), bytes_times(lo1, sl0), bytes_times(hi0, sl1), bytes_times(hi1, sl1));
        const uint32_t m0 = byte_bcast(mw[d], b0), m1 = byte_bcast(mw[d], b1);
        o.bm[h] = make_uint4(m0, m0, m1, m1);
    }
}

// Four unsigned bytes q (< 64) times one scale: P = q * s + c in 16-bit
// lanes (sp = (s, s), cp = (c, c)); lo gets P's low bytes xor 0x80, hi its
// high bytes, in the order of q's bytes.
__device__ inline void fold4(uint32_t q, u16x2 sp, u16x2 cp, uint32_t &lo, uint32_t &hi) {
    const u16x2 ev = __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(0u, q, 0x0C020C00u));  // bytes 0, 2
    const u16x2 od = __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(0u, q, 0x0C030C01u));  // bytes 1, 3
    const uint32_t pe = __builtin_bit_cast(uint32_t, ev * sp + cp);
    const uint32_t po = __builtin_bit_cast(uint32_t, od * sp + cp);
    lo = __builtin_amdgcn_perm(po, pe, 0x06020400u) ^ 0x80808080u;
    hi = __builtin_amdgcn_perm(po, pe, 0x07030501u);
}

__device__ inline void split_b(const MQ5K::W &w, const uint32_t (&scw)[2], const uint32_t (&mw)[2], SplitB &o) {
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        uint32_t hi[4], lo[4];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int u = 2 * h + k;
            const u16x2 sp = byte_pair(scw[u >> 2], u & 3);
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const uint32_t v = e ? w.q[h].y : w.q[h].x, qv = e ? w.qh.y : w.qh.x;
                const uint32_t q5 = ((v >> (4 * k)) & 0x0F0F0F0Fu) | (((qv >> u) & 0x01010101u) << 4);
                fold4(q5, sp, u16x2{128u, 128u}, lo[2 * k + e], hi[2 * k + e]);
            }
        }
        o.b1[h] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        o.b2[h] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        const uint32_t m0 = byte_bcast(mw[h >> 1], 2 * (h & 1)), m1 = byte_bcast(mw[h >> 1], 2 * (h & 1) + 1);
        o.bm[h] = make_uint4(m0, m0, m1, m1);
    }
}

__device__ inline void split_b(const MQ6KS::W &w, int c, SplitB &o) {
    const int cb = 8 * (c >> 1);  // bit offset of the lane's scale within a byte pair
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        const int hf = h >> 1, ip = h & 1;
        const uint2 sw = hf ? w.s1 : w.s0;
        uint32_t hi[4], lo[4];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int i = 2 * ip + k;
            // sc[8 hf + 2 i + c / 2], sign-extended, in both 16-bit lanes
            const int sc = __builtin_amdgcn_sbfe(int((i & 2) ? sw.y : sw.x), 16 * (i & 1) + cb, 8);
            const u16x2 sp = __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(0u, uint32_t(sc), 0x01000100u));
            const u16x2 cp = sp * u16x2{0xFFE0u, 0xFFE0u} + u16x2{128u, 128u};  // 128 - 32 sc
            const uint2 src = k ? w.b[hf] : w.a[hf];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const uint32_t v = e ? src.y : src.x, qv = e ? w.qh[hf].y : w.qh[hf].x;
                const int hs = 4 * ip + 2 * k;  // qh bits of this i
                const uint32_t q6 = ((v >> (4 * ip)) & 0x0F0F0F0Fu) | (((qv >> hs) & 0x03030303u) << 4);
                fold4(q6, sp, cp, lo[2 * k + e], hi[2 * k + e]);
            }
        }
        o.b1[h] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        o.b2[h] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    }
}

template <class F> struct ActOf { using T = Q8KView; };
template <> struct ActOf<MQ80> { using T = Q80View; };
// the format with the scales folded into the B operand, used from two
// token tiles per wave (M > 16)
template <class F> struct Folded { using T = F; };
template <> struct Folded<MQ4K> { using T = MQ4KS; };
template <> struct Folded<MQ5K> { using T = MQ5KS; };
// formats run with one token tile per wave (M <= 16): the unfolded ones, and
// Q6_K folded
template <class F> constexpr bool kSmallM = !F::kSplit || std::is_same_v<F, MQ6KS>;

// Scales / mins of the lane's row for the current block.
template <class F> struct Scales { int sc[F::NU]; int m[F::NU]; float d, dmin; };

template <class F>
__device__ inline void decode_scales(const typename F::W &w, Scales<F> &s) {
    if constexpr (std::is_same_v<F, MQ6KS>) {  // the scales are folded into the B operand
        s.d = fp16_bits_to_f32(w.d);
        s.dmin = 0.0f;
    } else if constexpr (F::NU == 8) {
#pragma unroll
        for (int u = 0; u < 8; ++u) scale_min_k4(u, w.h.y, w.h.z, w.h.w, s.sc[u], s.m[u]);
        s.d = fp16_bits_to_f32(w.h.x & 0xFFFFu);
        s.dmin = fp16_bits_to_f32(w.h.x >> 16);
    } else {
        s.sc[0] = 1;
        s.m[0] = 0;
        s.d = fp16_bits_to_f32(w.d);
        s.dmin = 0.0f;
    }
}

// Q4_K / Q5_K scales and mins of the 8 sub-blocks from the 12 scale bytes
// (three little-endian dwords s0..s2), four to a dword: sub-block u is byte
// u & 3 of sc[u >> 2] / m[u >> 2] — get_scale_min_k4 (E:743-749) done on
// whole dwords (j < 4: low 6 bits of bytes j, j + 4; j >= 4: the nibbles of
// byte j + 4 under the top 2 bits of bytes j - 4, j).
__device__ inline void scales_k4_packed(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t (&sc)[2], uint32_t (&m)[2]) {
    sc[0] = s0 & 0x3F3F3F3Fu;
    m[0] = s1 & 0x3F3F3F3Fu;
    sc[1] = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
    m[1] = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
}

// a * b + c on 24-bit signed operands (|a|, |b| < 2^23), exact in int32 (the
// compiler may reassociate a sum of such products: integer, so any order
// gives the same sum). Plain code, not inline assembly: b is often an MFMA
// result, and the compiler places the wait states an MFMA result needs before
// its VALU readers only for readers it can see (an inline-assembly reader
// read stale results a few cycles after the MFMA, depending on timing).
__device__ inline int mad_i24(int a, int b, int c) { return c + __mul24(a, b); }

__device__ inline int4v mfma16x16x32_acc(uint2 a, uint2 b, int4v c) {
    const long av = (long)(((uint64_t)a.y << 32) | a.x);
    const long bv = (long)(((uint64_t)b.y << 32) | b.x);
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bv, c, 0, 0, 0);
}

}  // namespace qmm
