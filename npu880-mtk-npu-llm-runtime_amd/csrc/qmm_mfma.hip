// qmm_mfma.hip — small-M (tree-verify, M = 2..64) and prefill (M = 512)
// GEMM over GGUF-packed rows with int8 MFMA, gfx950.
//
// Tile. A wavefront computes 16 weight rows x (16 * TT) tokens with
// v_mfma_i32_16x16x32_i8: A = Q8_K (or Q8_0) activation codes (16 tokens x
// 32 k), B = weight codes unpacked to int8 in registers (32 k x 16 rows).
// Lane l supplies token / weight row l % 16 and the k-slice l / 16 of both
// operands, and receives D[token 4 * (l / 16) + r][row l % 16], r = 0..3, so
// every lane owns one weight row and needs only that row's scales.
//
// One MFMA covers one scale unit of the format (a 32-value sub-block of
// Q4_K / Q5_K, a 16-value group of Q6_K padded with zero weights, a 32-value
// Q8_0 block), so its int32 result is the unit's exact dot; the unit scales,
// the min term and the per-block fp32 expression are applied exactly as the
// reference's scalar kernels do, and blocks are accumulated in order per
// output — the result equals the reference's fp32 sum bit for bit.
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
    static constexpr bool kMin = true;
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
    static constexpr bool kMin = true;
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

// Q6_K: unit u = (hf, i, is) = (u >> 3, (u >> 1) & 3, u & 1), 16 values
// 128hf + 32i + 16is + l, scale sc[8hf + 2i + is]. Lanes c = 0, 1 hold the
// 8 values l = 8c + t; lanes c = 2, 3 supply zero weights.
struct MQ6K {
    static constexpr int NU = 16, QK = 256, BB = 210;
    static constexpr bool kMin = false;
    struct W { uint2 a[4], b[4], qh[4]; uint2 s0, s1; uint32_t d; };
    __device__ static W load(const uint8_t *blk, int c) {
        W w;
        const int c2 = c & 1;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int is = 0; is < 2; ++is) {
                const int p = 2 * hf + is, l = 16 * is + 8 * c2;
                w.a[p] = ld8_a2(blk + 64 * hf + l);
                w.b[p] = ld8_a2(blk + 64 * hf + 32 + l);
                w.qh[p] = ld8_a2(blk + 128 + 32 * hf + l);
            }
        w.s0 = ld8_a2(blk + 192);
        w.s1 = ld8_a2(blk + 200);
        w.d = ld16b_a2(blk + 208);
        return w;
    }
    __device__ static W load_lds(const uint8_t *blk, int c) {
        W w;
        const int c2 = c & 1;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int is = 0; is < 2; ++is) {
                const int p = 2 * hf + is, l = 16 * is + 8 * c2;
                w.a[p] = lds8_a2(blk + 64 * hf + l);
                w.b[p] = lds8_a2(blk + 64 * hf + 32 + l);
                w.qh[p] = lds8_a2(blk + 128 + 32 * hf + l);
            }
        w.s0 = lds8_a2(blk + 192);
        w.s1 = lds8_a2(blk + 200);
        w.d = lds16b_a2(blk + 208);
        return w;
    }
    __device__ static int koff(int u, int c) {
        return 128 * (u >> 3) + 32 * ((u >> 1) & 3) + 16 * (u & 1) + 8 * (c & 1);
    }
    __device__ static uint2 bop(const W &w, int u, int c) {
        if (c >= 2) return make_uint2(0u, 0u);
        const int hf = u >> 3, i = (u >> 1) & 3, is = u & 1, p = 2 * hf + is;
        const uint2 src = (i & 1) ? w.b[p] : w.a[p];
        const int nsh = (i >> 1) * 4;
        const int hsh = 2 * i;
        const uint32_t x = ((src.x >> nsh) & 0x0F0F0F0Fu) | (((w.qh[p].x >> hsh) & 0x03030303u) << 4);
        const uint32_t y = ((src.y >> nsh) & 0x0F0F0F0Fu) | (((w.qh[p].y >> hsh) & 0x03030303u) << 4);
        return make_uint2(sub32_bytes(x), sub32_bytes(y));
    }
    __device__ static int scale(const W &w, int u) {
        const int idx = 8 * (u >> 3) + 2 * ((u >> 1) & 3) + (u & 1);
        const uint2 s = (idx < 8) ? w.s0 : w.s1;
        const uint64_t s64 = (uint64_t(s.y) << 32) | s.x;
        return int(int8_t(uint8_t(s64 >> (8 * (idx & 7)))));
    }
};

// Q8_0: one unit per 32-value block; lane c holds values 8c + t.
struct MQ80 {
    static constexpr int NU = 1, QK = 32, BB = 34;
    static constexpr bool kMin = false;
    struct W { uint2 q; uint32_t d; };
    __device__ static W load(const uint8_t *blk, int c) { return {ld8_a2(blk + 2 + 8 * c), ld16b_a2(blk)}; }
    __device__ static W load_lds(const uint8_t *blk, int c) { return {lds8_a2(blk + 2 + 8 * c), lds16b_a2(blk)}; }
    __device__ static int koff(int u, int c) { (void)u; return 8 * c; }
    __device__ static uint2 bop(const W &w, int u, int c) { (void)u; (void)c; return w.q; }
};

template <class F> struct ActOf { using T = Q8KView; };
template <> struct ActOf<MQ80> { using T = Q80View; };

// Scales / mins of the lane's row for the current block.
template <class F> struct Scales { int sc[F::NU]; int m[F::NU]; float d, dmin; };

template <class F>
__device__ inline void decode_scales(const typename F::W &w, Scales<F> &s) {
    if constexpr (F::NU == 8) {
#pragma unroll
        for (int u = 0; u < 8; ++u) scale_min_k4(u, w.h.y, w.h.z, w.h.w, s.sc[u], s.m[u]);
        s.d = fp16_bits_to_f32(w.h.x & 0xFFFFu);
        s.dmin = fp16_bits_to_f32(w.h.x >> 16);
    } else if constexpr (F::NU == 16) {
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            s.sc[u] = F::scale(w, u);
            s.m[u] = 0;
        }
        s.d = fp16_bits_to_f32(w.d);
        s.dmin = 0.0f;
    } else {
        s.sc[0] = 1;
        s.m[0] = 0;
        s.d = fp16_bits_to_f32(w.d);
        s.dmin = 0.0f;
    }
}

__device__ inline int4v mfma16x16x32_acc(uint2 a, uint2 b, int4v c) {
    const long av = (long)(((uint64_t)a.y << 32) | a.x);
    const long bv = (long)(((uint64_t)b.y << 32) | b.x);
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bv, c, 0, 0, 0);
}

// Workgroup = 16 weight rows x 16*TT tokens; its 4 waves split the K
// blocks (wave w takes blocks w, w+4, ...), each wave keeping PF of its
// blocks' weight bytes in flight. Per group of 4 consecutive blocks every
// wave writes its block's fp32 terms to LDS, and after a barrier each
// output's owner thread adds the 4 terms in block order — the sequential
// accumulation of the reference, so outputs stay bit-identical while the
// K loop runs 4 waves wide.
//
// Per block and token tile: NU MFMAs give the unit dots D_u; S = sum sc_u *
// D_u on the VALU (exact int32). For the formats with mins the min term
// Mb = sum_j m_j * bsum32_j is itself an int8 contraction — sum_k x_k *
// m_{unit(k)} — so it runs on the MFMA unit as one accumulating chain over
// the units with a B operand of broadcast 6-bit mins (exact, no bsum reads).
template <class F, int TT> struct ActBlock {
    uint2 a[TT][F::NU];  // A operands, per token tile and unit
    float dx[TT][4];     // activation scales of the lane's output tokens
};

template <class F, int TT, int PF, int PA>
__global__ __launch_bounds__(256) void mfma_kernel(MatArgs a, typename ActOf<F>::T x) {
    __shared__ float part[4][16 * TT * 16];  // [wave][token * 16 + row]
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int nl = lane & 15, c = lane >> 4;
    const int n0 = int(blockIdx.x) * 16;
    const int m0 = int(blockIdx.y) * 16 * TT;
    const int nload = min(n0 + nl, a.N - 1);
    const int nb = a.K / F::QK;
    const int ngroups = (nb + 3) / 4;
    const uint8_t *wrow = a.w + size_t(nload) * a.row_bytes;

    // A-operand rows of this lane (token m0 + 16t + nl), zero past M; output
    // tokens m0 + 16t + 4c + r for the activation scales
    const int8_t *xa_row[TT];
    bool okA[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        const int tokA = m0 + 16 * t + nl;
        okA[t] = tokA < a.M;
        xa_row[t] = x.qs + size_t(okA[t] ? tokA : 0) * a.K;
    }
    auto load_act = [&](int b, ActBlock<F, TT> &ab) __attribute__((always_inline)) {
        const int bl = min(b, nb - 1);
#pragma unroll
        for (int t = 0; t < TT; ++t) {
#pragma unroll
            for (int u = 0; u < F::NU; ++u)
                ab.a[t][u] = okA[t] ? ld8(xa_row[t] + size_t(bl) * F::QK + F::koff(u, c)) : make_uint2(0u, 0u);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tok = m0 + 16 * t + 4 * c + r;
                ab.dx[t][r] = x.d[size_t(min(tok, a.M - 1)) * nb + bl];
            }
        }
    };

    // weights (PF deep) and activations (PA deep) of this wave's blocks
    // b = wid + 4i, clamped to the last block (never stored past nb)
    typename F::W wq[PF];
    ActBlock<F, TT> aq[PA];
#pragma unroll
    for (int i = 0; i < PF; ++i) wq[i] = F::load(wrow + size_t(min(wid + 4 * i, nb - 1)) * F::BB, c);
#pragma unroll
    for (int i = 0; i < PA; ++i) load_act(wid + 4 * i, aq[i]);

    float acc[TT];
#pragma unroll
    for (int j = 0; j < TT; ++j) acc[j] = 0.0f;

    for (int grp = 0; grp < ngroups; ++grp) {
        const int b = 4 * grp + wid;
        const typename F::W wcur = wq[0];
        const ActBlock<F, TT> acur = aq[0];
#pragma unroll
        for (int i = 0; i + 1 < PF; ++i) wq[i] = wq[i + 1];
        wq[PF - 1] = F::load(wrow + size_t(min(b + 4 * PF, nb - 1)) * F::BB, c);
#pragma unroll
        for (int i = 0; i + 1 < PA; ++i) aq[i] = aq[i + 1];
        load_act(b + 4 * PA, aq[PA - 1]);
        if (b < nb) {
            Scales<F> s;
            decode_scales<F>(wcur, s);
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                int S[4] = {0, 0, 0, 0};
                int4v Mb = {0, 0, 0, 0};
#pragma unroll
                for (int u = 0; u < F::NU; ++u) {
                    const int4v D = mfma16x16x32(acur.a[t][u], F::bop(wcur, u, c));
                    if constexpr (F::kMin) {
                        const uint32_t mb = uint32_t(s.m[u]) * 0x01010101u;
                        Mb = mfma16x16x32_acc(acur.a[t][u], make_uint2(mb, mb), Mb);
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) S[r] += __mul24(s.sc[u], D[r]);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float dx = acur.dx[t][r];
                    float v;
                    if constexpr (F::kMin) v = dx * (s.d * (float)S[r] - s.dmin * (float)Mb[r]);  // E:11026
                    else v = (s.d * dx) * (float)S[r];                                            // E:11101 / E:3405
                    part[wid][(16 * t + 4 * c + r) * 16 + nl] = v;
                }
            }
        }
        lds_barrier();
        // blocks 4grp .. 4grp+3 in order
#pragma unroll
        for (int j = 0; j < TT; ++j) {
            const int o = int(threadIdx.x) + 256 * j;
#pragma unroll
            for (int w = 0; w < 4; ++w)
                if (4 * grp + w < nb) acc[j] += part[w][o];
        }
        lds_barrier();
    }
#pragma unroll
    for (int j = 0; j < TT; ++j) {
        const int o = int(threadIdx.x) + 256 * j;
        const int tok = m0 + (o >> 4), n = n0 + (o & 15);
        if (tok < a.M && n < a.N) {
            float v = acc[j];
            if (a.res) v = v + a.res[size_t(tok) * a.ldr + n];
            a.y[size_t(tok) * a.ldy + n] = v;
        }
    }
}

// ---------------------------------------------------------------- small M
// Workgroup = one 16-row tile x all M <= 64 tokens (TT = ceil(M / 16)
// tiles). K is processed in chunks of KCB blocks. For each chunk the
// workgroup loads the 16 weight-row segments (KCB * BB contiguous bytes
// each) and the token segments (KCB * QK bytes each) with coalesced 16-B
// loads — one chunk ahead, into registers — and stores them to LDS; the 4
// waves share the chunk's (block, token tile) items, read their MFMA
// operands from LDS and write each block's fp32 terms to LDS, where every
// output's owner thread adds them in block order (bit-identical to the
// reference's sequential accumulation).
template <class F, int TT>
struct SmallM {
    static constexpr int TM = 16 * TT;
    // blocks per chunk: about 48 KiB of LDS per workgroup
    static constexpr int per_block = 16 * F::BB + TM * F::QK + TM * 4 + TM * 64;
    static constexpr int KCB0 = (48 * 1024) / per_block;
    static constexpr int KCB = KCB0 < 1 ? 1 : (KCB0 > 32 ? 32 : KCB0);
    static constexpr int WSEG = KCB * F::BB;           // weight bytes per row per chunk
    static constexpr int WCR = (WSEG + 30) / 16;       // 16-B loads per row, any alignment
    static constexpr int WS = WCR * 16 + 16;           // LDS row stride
    static constexpr int ASEG = KCB * F::QK;           // activation bytes per token per chunk
    static constexpr int ACR = ASEG / 16;
    static constexpr int AS = ASEG + 16;               // LDS token stride
    static constexpr int NW = (16 * WCR + 255) / 256;  // loads per thread
    static constexpr int NA = (TM * ACR + 255) / 256;
    static constexpr int ND = (TM * KCB + 255) / 256;
    static constexpr int OFF_A = 16 * WS;
    static constexpr int OFF_D = OFF_A + TM * AS;
    static constexpr int OFF_P = OFF_D + ((TM * KCB * 4 + 15) & ~15);
    static constexpr int LDS = OFF_P + KCB * TM * 16 * 4;
};

template <class F, int TT>
__global__ __launch_bounds__(256) void mfma_small_kernel(MatArgs a, typename ActOf<F>::T x) {
    using C = SmallM<F, TT>;
    extern __shared__ __align__(16) uint8_t lds[];
    uint8_t *lw = lds;
    int8_t *la = reinterpret_cast<int8_t *>(lds + C::OFF_A);
    float *ld = reinterpret_cast<float *>(lds + C::OFF_D);
    float *part = reinterpret_cast<float *>(lds + C::OFF_P);
    const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
    const int nl = lane & 15, cl = lane >> 4;
    const int n0 = int(blockIdx.x) * 16;
    const int K = a.K, nb = K / F::QK;
    const int nchunks = (nb + C::KCB - 1) / C::KCB;

    uint4 rw[C::NW], ra[C::NA];
    float rd[C::ND];
    // chunk ch: weight bytes [ch*KCB*BB, +WSEG) of rows n0..n0+15 (clamped
    // to the last row), token bytes [ch*KCB*QK, +ASEG) of tokens 0..TM-1
    // (clamped to the last token); load indices past the valid bytes repeat
    // the last valid 16 B, which is stored to the same place.
    auto w_src = [&](int ch, int idx, int &dst) __attribute__((always_inline)) -> const uint8_t * {
        const int row = min(idx / C::WCR, 15), piece = idx - row * C::WCR;
        const size_t off = size_t(ch) * C::KCB * F::BB;
        const uint8_t *rp = a.w + size_t(min(n0 + row, a.N - 1)) * a.row_bytes + off;
        const int mis = int(reinterpret_cast<uintptr_t>(rp) & 15);
        const int nbytes = int(min(size_t(C::WSEG), a.row_bytes - off));
        const int pc = min(piece, (mis + nbytes + 15) / 16 - 1);
        dst = row * C::WS + 16 * pc;
        return rp - mis + 16 * pc;
    };
    auto a_src = [&](int ch, int idx, int &dst) __attribute__((always_inline)) -> const int8_t * {
        const int tok = min(idx / C::ACR, C::TM - 1), piece = idx - tok * C::ACR;
        const int off = ch * C::ASEG;
        const int pc = min(piece, min(C::ASEG, K - off) / 16 - 1);
        dst = tok * C::AS + 16 * pc;
        return x.qs + size_t(min(tok, a.M - 1)) * K + off + 16 * pc;
    };
    auto load_chunk = [&](int ch) __attribute__((always_inline)) {
        int dummy;
#pragma unroll
        for (int i = 0; i < C::NW; ++i) rw[i] = ld16_nt(w_src(ch, min(t + 256 * i, 16 * C::WCR - 1), dummy));
#pragma unroll
        for (int i = 0; i < C::NA; ++i) ra[i] = ld16(a_src(ch, min(t + 256 * i, C::TM * C::ACR - 1), dummy));
#pragma unroll
        for (int i = 0; i < C::ND; ++i) {
            const int idx = min(t + 256 * i, C::TM * C::KCB - 1);
            const int tok = idx / C::KCB, j = idx - tok * C::KCB;
            rd[i] = x.d[size_t(min(tok, a.M - 1)) * nb + min(ch * C::KCB + j, nb - 1)];
        }
    };
    auto store_chunk = [&](int ch) __attribute__((always_inline)) {
        int dst;
#pragma unroll
        for (int i = 0; i < C::NW; ++i) {
            const int idx = t + 256 * i;
            (void)w_src(ch, min(idx, 16 * C::WCR - 1), dst);
            if (idx < 16 * C::WCR) *reinterpret_cast<uint4 *>(lw + dst) = rw[i];
        }
#pragma unroll
        for (int i = 0; i < C::NA; ++i) {
            const int idx = t + 256 * i;
            (void)a_src(ch, min(idx, C::TM * C::ACR - 1), dst);
            if (idx < C::TM * C::ACR) *reinterpret_cast<uint4 *>(la + dst) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < C::ND; ++i) {
            const int idx = t + 256 * i;
            if (idx < C::TM * C::KCB) ld[idx] = rd[i];
        }
    };

    float acc[TT];
#pragma unroll
    for (int i = 0; i < TT; ++i) acc[i] = 0.0f;

    load_chunk(0);
    for (int ch = 0; ch < nchunks; ++ch) {
        store_chunk(ch);
        lds_barrier();
        if (ch + 1 < nchunks) load_chunk(ch + 1);
        // the lane's weight row in LDS for this chunk (its 16-B misalignment)
        const size_t off = size_t(ch) * C::KCB * F::BB;
        const int mis = int(reinterpret_cast<uintptr_t>(a.w + size_t(min(n0 + nl, a.N - 1)) * a.row_bytes + off) & 15);
        const uint8_t *wrow = lw + nl * C::WS + mis;
        for (int it = wid; it < C::KCB * TT; it += 4) {
            const int j = it / TT, tt = it - j * TT;
            if (ch * C::KCB + j >= nb) continue;
            const typename F::W wv = F::load_lds(wrow + j * F::BB, cl);
            Scales<F> s;
            decode_scales<F>(wv, s);
            const int8_t *arow = la + (16 * tt + nl) * C::AS + j * F::QK;
            int S[4] = {0, 0, 0, 0};
            int4v Mb = {0, 0, 0, 0};
#pragma unroll
            for (int u = 0; u < F::NU; ++u) {
                const uint2 av = ld8(arow + F::koff(u, cl));
                const int4v D = mfma16x16x32(av, F::bop(wv, u, cl));
                if constexpr (F::kMin) {
                    const uint32_t mb = uint32_t(s.m[u]) * 0x01010101u;
                    Mb = mfma16x16x32_acc(av, make_uint2(mb, mb), Mb);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) S[r] += __mul24(s.sc[u], D[r]);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tok = 16 * tt + 4 * cl + r;
                const float dx = ld[tok * C::KCB + j];
                float v;
                if constexpr (F::kMin) v = dx * (s.d * (float)S[r] - s.dmin * (float)Mb[r]);  // E:11026
                else v = (s.d * dx) * (float)S[r];                                            // E:11101 / E:3405
                part[(j * C::TM + tok) * 16 + nl] = v;
            }
        }
        lds_barrier();
        // this chunk's blocks, in order
#pragma unroll
        for (int i = 0; i < TT; ++i) {
            const int o = t + 256 * i;  // token o / 16, row o % 16
            for (int j = 0; j < C::KCB && ch * C::KCB + j < nb; ++j) acc[i] += part[j * C::TM * 16 + o];
        }
    }
#pragma unroll
    for (int i = 0; i < TT; ++i) {
        const int o = t + 256 * i;
        const int tok = o >> 4, n = n0 + (o & 15);
        if (tok < a.M && n < a.N) {
            float v = acc[i];
            if (a.res) v = v + a.res[size_t(tok) * a.ldr + n];
            a.y[size_t(tok) * a.ldy + n] = v;
        }
    }
}

template <class F, int TT>
static hipError_t launch_small_t(const MatArgs &a, const typename ActOf<F>::T &x, hipStream_t s) {
    using C = SmallM<F, TT>;
    hipLaunchKernelGGL((mfma_small_kernel<F, TT>), dim3(unsigned((a.N + 15) / 16)), dim3(256),
                       size_t(C::LDS), s, a, x);
    return hipGetLastError();
}

template <class F>
static hipError_t launch_small(const MatArgs &a, const typename ActOf<F>::T &x, hipStream_t s) {
    switch ((a.M + 15) / 16) {
        case 1: return launch_small_t<F, 1>(a, x, s);
        case 2: return launch_small_t<F, 2>(a, x, s);
        case 3: return launch_small_t<F, 3>(a, x, s);
        default: return launch_small_t<F, 4>(a, x, s);
    }
}

template <class F, int TT, int PF, int PA>
static hipError_t launch_mfma_t(const MatArgs &a, const typename ActOf<F>::T &x, hipStream_t s) {
    const dim3 grid(unsigned((a.N + 15) / 16), unsigned((a.M + 16 * TT - 1) / (16 * TT)));
    hipLaunchKernelGGL((mfma_kernel<F, TT, PF, PA>), grid, dim3(256), 0, s, a, x);
    return hipGetLastError();
}

template <class F>
static hipError_t launch_mfma_f(const MatArgs &a, const typename ActOf<F>::T &x, hipStream_t s) {
    // large M: 4 token tiles per wave (2 for Q6_K, whose 16 units would spill)
    constexpr int kTT = F::NU > 8 ? 2 : 4;
    if (a.M <= 64) return launch_small<F>(a, x, s);
    return launch_mfma_t<F, kTT, 1, 1>(a, x, s);
}

hipError_t launch_mfma(uint32_t type, const MatArgs &a, const Q8KView &xk, const Q80View &x0,
                       hipStream_t s) {
    switch (type) {
        case kQ4_K: return launch_mfma_f<MQ4K>(a, xk, s);
        case kQ5_K: return launch_mfma_f<MQ5K>(a, xk, s);
        case kQ6_K: return launch_mfma_f<MQ6K>(a, xk, s);
        case kQ8_0: return launch_mfma_f<MQ80>(a, x0, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace qmm
