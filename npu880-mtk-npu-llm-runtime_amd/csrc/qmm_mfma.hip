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
//
// The min term Mb = sum_j m_j * bsum32_j of Q4_K / Q5_K is itself an int8
// contraction, sum_k x_k * m_unit(k), so it runs on the matrix unit as one
// accumulating MFMA chain over the block's units against a B operand of
// broadcast 6-bit mins (exact; equal to the reference's bsum form for every
// Q8_K row whose block sums are the sums of its codes, which the quantizer
// guarantees).
#include "qmm_kformats.h"

namespace qmm {

// ================================================================ tile GEMM
// Workgroup tile = ROWS weight rows x TOK tokens, 4 waves arranged as
// PR row groups x PT token groups x KS K phases; a wave computes WR x WT
// MFMA tiles of 16 x 16 over the blocks j = kp (mod KS) of every chunk.
//
// Operands reach LDS by direct buffer -> LDS transfers (buffer_load ... lds,
// 16 B per lane): no registers, no address clamps. Every transfer goes
// through a buffer descriptor whose range is exactly the workgroup's rows,
// the M tokens' codes or their scales, so a lane past the end reads zeros
// and touches no memory. The K loop walks chunks of KCB blocks through PD
// LDS slots: the transfers of chunk ch + PD - 1 are issued before chunk ch
// is computed, and an explicit vmcnt wait (transfers retire in order)
// releases chunk ch. Every wave issues the same number of transfers per
// chunk (surplus ones target a dump line), so the wait counts are static.
// With KMAX > 0 (small M) the tokens' codes and scales for the whole of
// K <= KMAX are transferred once, ahead of the first chunk, and stay in LDS;
// the slots then carry weights only, so more chunks fit in flight.

template <class F, int WR_, int WT_, int PR_, int PT_, int KS_, int TR_, int PD_, int BUDGET, int KMAX_ = 0>
struct TileCfg {
    static constexpr int WR = WR_, WT = WT_, PR = PR_, PT = PT_, KS = KS_, TR = TR_, PD = PD_;
    static constexpr int KMAX = KMAX_;
    static constexpr bool AR = KMAX > 0;  // codes and scales resident
    static_assert(PR * PT * KS == 4, "4 waves");
    static_assert(TR == 16 || (TR == 8 && WT == 1 && PT == 1), "8 resident tokens: one token tile");
    static constexpr int ROWS = 16 * WR * PR;
    static constexpr int TOK = TR * WT * PT;  // tokens resident per chunk
    static constexpr int wcr(int k) { return ((k * F::BB + 30) / 16) | 1; }  // odd: rows 4 banks apart
    // AT: the codes come from the Q8_K tiles section, already in MFMA operand
    // order (1 KB per 16-token tile, block and 64-value chunk; a lane's 16 B
    // contiguous): one 16-B LDS read per operand, no bank conflicts, no row
    // padding (folded formats with 16-token tiles streamed per chunk)
    static constexpr bool AT = F::kSplit && !AR && TR == 16;
    static constexpr int acr(int k) { return k * F::QK / 16 + 1; }
    static constexpr int nwi(int k) { return (ROWS * wcr(k) + 63) / 64; }
    static constexpr int nai(int k) { return AR ? 0 : AT ? (TOK / 16) * k * (F::QK / 64) : (TOK * acr(k) + 63) / 64; }
    static constexpr int ndi(int k) { return AR ? 0 : (k * TOK + 63) / 64; }
    // resident codes (rows of K / 16 + 1 units of 16 B) and scales ([block][token])
    static constexpr int AR_BYTES = AR ? (TOK * (KMAX / 16 + 1) + 63) / 64 * 1024 : 0;
    static constexpr int DR_BYTES = AR ? (KMAX / F::QK * TOK + 63) / 64 * 256 : 0;
    static constexpr int slot(int k) { return nwi(k) * 1024 + nai(k) * 1024 + ndi(k) * 256; }
    static constexpr int per_wave(int k) { return (nwi(k) + 3) / 4 + (nai(k) + 3) / 4 + (ndi(k) + 3) / 4; }
    static constexpr int part(int k) { return KS > 1 ? k * TOK * ROWS * 4 : 0; }
    static constexpr int total(int k) { return PD * slot(k) + AR_BYTES + DR_BYTES + part(k) + 1024; }
    static constexpr bool fits(int k) { return total(k) <= BUDGET && (PD - 1) * per_wave(k) <= 63; }
    static constexpr int pick() {
        int k = KS;
        while (k + KS <= 16 && fits(k + KS)) k += KS;
        return k;
    }
    static constexpr int KCB = pick();
    static constexpr int WCR = wcr(KCB), ACR = acr(KCB);
    static constexpr int NWI = nwi(KCB), NAI = nai(KCB), NDI = ndi(KCB);
    static constexpr int NWW = (NWI + 3) / 4, NAW = (NAI + 3) / 4, NDW = (NDI + 3) / 4;
    static constexpr int L = NWW + NAW + NDW;  // transfers per wave per chunk
    static constexpr int OFF_A = NWI * 1024, OFF_D = OFF_A + NAI * 1024, SLOT = slot(KCB);
    static constexpr int OFF_AR = PD * SLOT, OFF_DR = OFF_AR + AR_BYTES;
    static constexpr int OFF_P = OFF_DR + DR_BYTES, OFF_DUMP = OFF_P + part(KCB), LDS = total(KCB);
    static_assert(fits(KCB), "tile does not fit the LDS budget");
    static_assert(KS == 1 || TOK * ROWS <= 4 * 256, "K-split tiles: at most 4 outputs per thread");
};

template <class C, class F>
__global__ __launch_bounds__(256) void tile_kernel(MatGroup grp, typename ActOf<F>::T x) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int WR = C::WR, WT = C::WT, KS = C::KS, TR = C::TR, KCB = C::KCB;
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nl = lane & 15, cl = lane >> 4;
    const int kp = wid % KS, pt = (wid / KS) % C::PT, pr = wid / (KS * C::PT);
    int bx;
    const MatArgs a = grp.t[group_task(grp, int(blockIdx.x), bx)];
    if (scan_stopped(a.scan)) return;
    const int n0 = bx * C::ROWS, m0 = int(blockIdx.y) * C::TOK;
    const int K = a.K, nb = K / F::QK;
    const int nchunks = (nb + KCB - 1) / KCB;
    const int acr_rt = C::AR ? K / 16 + 1 : C::ACR;  // codes row stride, 16-B units

    // descriptors: this workgroup's rows (from the 16-B boundary at or below
    // the first), the M tokens' codes, their block scales
    const uintptr_t wstart = reinterpret_cast<uintptr_t>(a.w) + size_t(n0) * a.row_bytes;
    const uint32_t bl = uint32_t(wstart & 15);
    const int rows_valid = min(C::ROWS, a.N - n0);
    // (the range is rounded up to whole 16-B granules: the range check is per
    // dword, and a 2-B aligned format's last bytes may share one with the end)
    const v4i32 rw = buf_rsrc(reinterpret_cast<const void *>(wstart - bl),
                              (bl + uint32_t(rows_valid) * uint32_t(a.row_bytes) + 15u) & ~15u);
    v4i32 ra;  // the codes: [M][K], or the tiles section of ceil(M / 16) * 16 tokens
    if constexpr (C::AT) ra = buf_rsrc(x.qt, uint32_t((a.M + 15) & ~15) * uint32_t(K));
    else ra = buf_rsrc(x.qs, uint32_t(a.M) * uint32_t(K));
    const v4i32 rd = buf_rsrc(x.d, uint32_t(a.M) * uint32_t(nb) * 4u);
    const uint32_t lds0 = lds_addr(lds);

    // per-lane transfer offsets (chunk 0); lanes past a region's pieces get kFar
    uint32_t wo[C::NWW], wp[C::NWW], ao[C::NAW > 0 ? C::NAW : 1], dof[C::NDW > 0 ? C::NDW : 1];
#pragma unroll
    for (int s = 0; s < C::NWW; ++s) {
        const int p = (s * 4 + wid) * 64 + lane;
        const int row = p / C::WCR, pc = p - row * C::WCR;
        wo[s] = row < C::ROWS ? uint32_t(row) * uint32_t(a.row_bytes) + bl : kFar;
        wp[s] = 16u * uint32_t(pc);
    }
#pragma unroll
    for (int s = 0; s < C::NAW; ++s) {
        if constexpr (C::AT) {  // transfer i: token tile i / 4 KCB, block (i / 4) mod KCB, chunk i mod 4
            const int i = s * 4 + wid, tt = i / (4 * KCB), j = (i >> 2) % KCB, h = i & 3;
            ao[s] = i < C::NAI ? ((uint32_t(m0 / 16 + tt) * uint32_t(nb) + uint32_t(j)) * 4u + uint32_t(h)) * 1024u +
                                     16u * uint32_t(lane)
                               : kFar;
        } else {
            const int p = (s * 4 + wid) * 64 + lane;
            const int tok = p / C::ACR, pc = p - tok * C::ACR;
            ao[s] = tok < C::TOK ? uint32_t(m0 + tok) * uint32_t(K) + 16u * uint32_t(pc) : kFar;
        }
    }
#pragma unroll
    for (int s = 0; s < C::NDW; ++s) {
        const int p = (s * 4 + wid) * 64 + lane;
        const int j = p / C::TOK, tok = p - j * C::TOK;
        dof[s] = j < KCB ? (uint32_t(m0 + tok) * uint32_t(nb) + uint32_t(j)) * 4u : kFar;
    }
    // issue chunk ch into slot sl; a chunk past the end reads nothing
    auto issue = [&](int ch, int sl) __attribute__((always_inline)) {
        const bool live = ch < nchunks;
        const uint32_t base = lds0 + uint32_t(sl * C::SLOT), dump = lds0 + uint32_t(C::OFF_DUMP);
        const uint32_t cw = uint32_t(ch) * uint32_t(KCB * F::BB);
        const uint32_t ca = uint32_t(ch) * uint32_t(KCB * (C::AT ? 4096 : F::QK));  // 4 KB per block and token tile
        const uint32_t cd = uint32_t(ch) * uint32_t(KCB) * 4u;
#pragma unroll
        for (int s = 0; s < C::NWW; ++s) {
            const int i = s * 4 + wid;
            const uint32_t v = ((wo[s] + cw) & ~15u) + wp[s];
            dma16(rw, live ? v : kFar, i < C::NWI ? base + uint32_t(i * 1024) : dump);
        }
#pragma unroll
        for (int s = 0; s < C::NAW; ++s) {
            const int i = s * 4 + wid;
            dma16(ra, live ? ao[s] + ca : kFar, i < C::NAI ? base + uint32_t(C::OFF_A + i * 1024) : dump);
        }
#pragma unroll
        for (int s = 0; s < C::NDW; ++s) {
            const int i = s * 4 + wid;
            dma4(rd, live ? dof[s] + cd : kFar, i < C::NDI ? base + uint32_t(C::OFF_D + i * 256) : dump);
        }
    };

    float acc[WR][WT][4];
#pragma unroll
    for (int wr = 0; wr < WR; ++wr)
#pragma unroll
        for (int wt = 0; wt < WT; ++wt)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[wr][wt][r] = 0.0f;
    float *part = reinterpret_cast<float *>(lds + C::OFF_P);
    float *dump4 = reinterpret_cast<float *>(lds + C::OFF_DUMP);

    // one chunk: wait for it, compute its blocks of this wave's phase
    auto step = [&](int ch, int sl) __attribute__((always_inline)) {
        issue(ch + C::PD - 1, (sl + C::PD - 1) % C::PD);
        wait_vmcnt<(C::PD - 1) * C::L>();
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t *ws = lds + sl * C::SLOT;
        const int8_t *as = reinterpret_cast<const int8_t *>(C::AR ? lds + C::OFF_AR : ws + C::OFF_A);
        const float *ds = reinterpret_cast<const float *>(C::AR ? lds + C::OFF_DR : ws + C::OFF_D);
        const uint32_t cw = uint32_t(ch) * uint32_t(KCB * F::BB);
#pragma unroll
        for (int jj = 0; jj < KCB / KS; ++jj) {
            const int j = jj * KS + kp;
            // (one block per chunk: every chunk walked is inside K)
            const bool valid = KCB == 1 || ch * KCB + j < nb;
            // one K phase: a block past K adds nothing, skipped (the test is the
            // same in every lane); K-split terms of every block are summed
            if constexpr (KS == 1)
                if (!valid) continue;
            // block index into the codes and scales: of the chunk's slot, or of
            // the resident arrays (block 0 stands in for blocks past K)
            const int jr = C::AR ? (valid ? ch * KCB + j : 0) : j;
#pragma unroll
            for (int wr = 0; wr < WR; ++wr) {
                const int rl = (pr * WR + wr) * 16 + nl;  // lane's weight row in the tile
                const int mis = int((uint32_t(rl) * uint32_t(a.row_bytes) + bl + cw) & 15u);
                const typename F::W wv = F::load_lds(ws + rl * (C::WCR * 16) + mis + j * F::BB, cl);
                Scales<F> sc;
                decode_scales<F>(wv, sc);
                // a block past the end of K holds stale bytes: its d, dmin and
                // dx are zeroed, its term is a signed zero, the sums are
                // unchanged (a sum starting at +0 is never -0)
                const float d = valid ? sc.d : 0.0f, dmin = valid ? sc.dmin : 0.0f;
                [[maybe_unused]] SplitB sb;
                if constexpr (F::kSplit) {
                    if constexpr (F::kMin) {
                uint32_t scp[2], mp[2];
                scales_k4_packed(wv.h.y, wv.h.z, wv.h.w, scp, mp);
                split_b(wv, scp, mp, sb);
            }
                    else split_b(wv, cl, sb);
                }
#pragma unroll
                for (int wt = 0; wt < WT; ++wt) {
                    const int tl = (pt * WT + wt) * TR + (nl & (TR - 1));  // lane's A token
                    const int8_t *arow = as + tl * (acr_rt * 16) + jr * F::QK;
                    int S[4] = {0, 0, 0, 0};
                    int4v Mb = {0, 0, 0, 0};
                    if constexpr (F::kSplit) {
                        int4v D1 = {0, 0, 0, 0}, D2 = {0, 0, 0, 0};
#pragma unroll
                        for (int h = 0; h < 4; ++h) {
                            uint4 av;
                            if constexpr (C::AT) {
                                av = ld16(as + (((pt * WT + wt) * KCB + j) * 4 + h) * 1024 + 16 * lane);
                            } else {
                                const uint2 a0 = ld8(arow + 64 * h + 8 * cl), a1 = ld8(arow + 64 * h + 32 + 8 * cl);
                                av = make_uint4(a0.x, a0.y, a1.x, a1.y);
                            }
                            D1 = mfma16x16x64(av, sb.b1[h], D1);
                            D2 = mfma16x16x64(av, sb.b2[h], D2);
                            if constexpr (F::kMin) Mb = mfma16x16x64(av, sb.bm[h], Mb);
                        }
#pragma unroll
                        for (int r = 0; r < 4; ++r) S[r] = (D1[r] << F::kShift) + D2[r];
                    } else {
#pragma unroll
                        for (int u = 0; u < F::NU; ++u) {
                            const uint2 av = ld8(arow + F::koff(u, cl));
                            const int4v D = mfma16x16x32(av, F::bop(wv, u, cl));
                            if constexpr (F::kMin) {
                                const uint32_t mb = __builtin_amdgcn_perm(0u, uint32_t(sc.m[u]), 0u);  // byte broadcast
                                Mb = mfma16x16x32_acc(av, make_uint2(mb, mb), Mb);
                            }
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                if constexpr (F::NU == 1) S[r] = D[r];  // Q8_0: the unit scale is 1
                                else S[r] += __mul24(sc.sc[u], D[r]);
                            }
                        }
                    }
                    // dx of output tokens 4 cl + r of this token tile (tokens
                    // past TR read neighbouring scales; their outputs are not kept)
                    const float4 dx4 = *reinterpret_cast<const float4 *>(ds + jr * C::TOK + (pt * WT + wt) * TR + 4 * cl);
                    const float dxr[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float dx = valid ? dxr[r] : 0.0f;
                        float v;
                        if constexpr (F::kMin) v = dx * (d * (float)S[r] - dmin * (float)Mb[r]);  // E:11026
                        else v = (d * dx) * (float)S[r];                                        // E:11101 / E:3405
                        if constexpr (KS == 1) {
                            acc[wr][wt][r] += v;
                        } else {
                            const int tok = (pt * WT + wt) * TR + 4 * cl + r;
                            float *dst = tok < (pt * WT + wt + 1) * TR
                                             ? part + (j * C::TOK + tok) * C::ROWS + rl
                                             : dump4 + lane;
                            *dst = v;
                        }
                    }
                }
            }
        }
        if constexpr (KS > 1) {
            wait_lgkm0();
            __builtin_amdgcn_s_barrier();
            // outputs (token o / ROWS, row o % ROWS): this chunk's blocks in order
#pragma unroll
            for (int q = 0; q < (C::TOK * C::ROWS + 255) / 256; ++q) {
                const int o = int(threadIdx.x) + 256 * q;
                if (o < C::TOK * C::ROWS) {
                    float s = acc[0][0][q & 3];
                    for (int j = 0; j < KCB; ++j) s += part[j * C::TOK * C::ROWS + o];
                    acc[0][0][q & 3] = s;
                }
            }
        }
        wait_lgkm0();
        __builtin_amdgcn_s_barrier();  // every wave is done with slot sl
    };

    // resident codes (row stride K / 16 + 1 units) and scales, once, ahead of
    // every chunk: the first chunk's wait covers them
    if constexpr (C::AR) {
        const int nar = (C::TOK * acr_rt + 63) / 64;
        for (int i = wid; i < nar; i += 4) {
            const int p = i * 64 + lane;
            const int tok = p / acr_rt, pc = p - tok * acr_rt;
            dma16(ra, tok < C::TOK ? uint32_t(m0 + tok) * uint32_t(K) + 16u * uint32_t(pc) : kFar,
                  lds0 + uint32_t(C::OFF_AR + i * 1024));
        }
        const int ndr = (nb * C::TOK + 63) / 64;
        for (int i = wid; i < ndr; i += 4) {
            const int e = i * 64 + lane;
            const int j = e / C::TOK, tok = e - j * C::TOK;
            dma4(rd, j < nb ? (uint32_t(m0 + tok) * uint32_t(nb) + uint32_t(j)) * 4u : kFar,
                 lds0 + uint32_t(C::OFF_DR + i * 256));
        }
    }
#pragma unroll
    for (int p = 0; p + 1 < C::PD; ++p) issue(p, p);
    int ch = 0;
    for (; ch + C::PD <= nchunks; ch += C::PD)
#pragma unroll
        for (int q = 0; q < C::PD; ++q) step(ch + q, q);
    for (int q = 0; ch < nchunks; ++ch, ++q) step(ch, q);
    wait_vmcnt<0>();  // the tail's transfers (zeros into a free slot) land before the workgroup ends

    if constexpr (KS == 1) {
#pragma unroll
        for (int wr = 0; wr < WR; ++wr) {
            const int n = n0 + (pr * WR + wr) * 16 + nl;
            if (n >= a.N) continue;
#pragma unroll
            for (int wt = 0; wt < WT; ++wt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    // with 8-token tiles, columns 8..15 of the MFMA tile are the
                    // next token group's (computed on neighbouring scales): not kept
                    if (4 * cl + r >= TR) continue;
                    const int tok = m0 + (pt * WT + wt) * TR + 4 * cl + r;
                    if (tok >= a.M) continue;
                    float v = acc[wr][wt][r];
                    if (a.res) v = v + a.res[size_t(tok) * a.ldr + n];
                    a.y[size_t(tok) * a.ldy + n] = v;
                }
        }
    } else {
#pragma unroll
        for (int q = 0; q < (C::TOK * C::ROWS + 255) / 256; ++q) {
            const int o = int(threadIdx.x) + 256 * q;
            const int tok = m0 + o / C::ROWS, n = n0 + o % C::ROWS;
            if (o < C::TOK * C::ROWS && tok < a.M && n < a.N) {
                float v = acc[0][0][q & 3];
                if (a.res) v = v + a.res[size_t(tok) * a.ldr + n];
                a.y[size_t(tok) * a.ldy + n] = v;
            }
        }
    }
}

// ====================================================== resident-tile GEMM
// Small M (up to 16 * TT tokens) of a k-quant over K <= NBK * 4 * 256: one
// workgroup per CU owns RT <= RTM consecutive 16-row tiles (of the group's
// concatenated row tiles) and every token, with one wave per (tile, K part):
// wave (rt, kp) computes tile rt over the kp-th of 4 contiguous parts of the
// K blocks. At start the waves move the M x K codes (rows padded by 16 B)
// and the M x nb block scales into LDS (1-KB buffer -> LDS transfers, each
// code fetched once per CU), then each wave its own part of its tile's 16
// rows, so every byte is in flight at once and a wave starts computing as
// soon as its own transfers land. A lane keeps one fp32 term per output and
// block; a chain through LDS hands the running sum of part kp - 1 to part
// kp, which adds its terms in block order, so every output is the
// reference's block-ordered fp32 sum.
struct ResArgs {
    int tiles;                // row tiles of the group
    int acr;                  // codes row stride in LDS, 16-B units (K / 16 + 1)
    int off_a, off_d, off_t;  // LDS offsets of the codes, the scales, the terms
    int lds;                  // LDS bytes
};

template <class F, int NBK>
struct ResPart {
    // row stride in 16-B units: a part's bytes from the 16-B boundary at or
    // below its start; odd, so the 16 rows start 4 banks apart
    static constexpr int RU = ((15 + NBK * F::BB + 15) / 16) | 1;
    static constexpr int NI = (16 * RU + 63) / 64;  // transfers (KB) per wave
};

template <class F, int TT, int NBK, int RTM>
__global__ __launch_bounds__(256 * RTM) void res_kernel(MatGroup grp, Q8KView x, ResArgs ra) {
    using P = ResPart<F, NBK>;
    constexpr int W = 4 * RTM;
    extern __shared__ __align__(16) uint8_t lds[];
    if (scan_stopped(grp.t[0].scan)) return;  // (every task of a group shares the scan)
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rt = wid % RTM, kp = wid / RTM;
    const int nl = lane & 15, cl = lane >> 4;
    const int G = int(gridDim.x);
    const int t0 = int(blockIdx.x) * ra.tiles / G, nrt = (int(blockIdx.x) + 1) * ra.tiles / G - t0;
    const int M = grp.t[0].M, K = grp.t[0].K, nb = K / 256;
    const uint32_t lds0 = lds_addr(lds);

    // codes and scales, dealt out to the waves in turn
    const int ncode = (M * ra.acr + 63) / 64, nscale = (M * nb + 63) / 64;
    const v4i32 ra_q = buf_rsrc(x.qs, uint32_t(M) * uint32_t(K));
    const v4i32 ra_d = buf_rsrc(x.d, uint32_t(M) * uint32_t(nb) * 4u);
    for (int q = wid; q < ncode + nscale; q += W) {
        if (q < ncode) {
            const int g = q * 64 + lane;
            const int tok = g / ra.acr, u = g - tok * ra.acr;
            dma16(ra_q, (tok < M && 16 * u < K) ? uint32_t(tok) * uint32_t(K) + 16u * uint32_t(u) : kFar,
                  lds0 + uint32_t(ra.off_a + q * 1024));
        } else {
            const int e = (q - ncode) * 64 + lane;
            dma4(ra_d, e < M * nb ? 4u * uint32_t(e) : kFar, lds0 + uint32_t(ra.off_d + (q - ncode) * 256));
        }
    }
    // this wave's part of its tile's rows (P::NI transfers by every wave;
    // rows past N, bytes past the tile and waves without a tile or blocks
    // read zeros)
    const int j0 = kp * nb / 4, nbk = (kp + 1) * nb / 4 - j0;
    const bool live = rt < nrt;
    int bx = 0;
    const MatArgs a = grp.t[group_task(grp, t0 + (live ? rt : 0), bx)];
    const int n0 = bx * 16;
    const uintptr_t wstart = reinterpret_cast<uintptr_t>(a.w) + size_t(n0) * a.row_bytes;
    const uint32_t bl = uint32_t(wstart & 15);
    const v4i32 rw = buf_rsrc(reinterpret_cast<const void *>(wstart - bl),
                              (bl + uint32_t(min(16, a.N - n0)) * uint32_t(a.row_bytes) + 15u) & ~15u);
    uint8_t *ws = lds + wid * (P::NI * 1024);
    const uint32_t part0 = bl + uint32_t(j0) * uint32_t(F::BB);  // part start in row 0, from the 16-B base
#pragma unroll
    for (int i = 0; i < P::NI; ++i) {
        const int p = i * 64 + lane;
        const int row = p / P::RU, u = p - row * P::RU;
        const uint32_t o = ((uint32_t(row) * uint32_t(a.row_bytes) + part0) & ~15u) + 16u * uint32_t(u);
        dma16(rw, (live && nbk > 0 && row < 16) ? o : kFar, lds_addr(ws) + uint32_t(i * 1024));
    }
    wait_vmcnt<P::NI>();              // this wave's codes and scales
    __builtin_amdgcn_s_barrier();     // everyone's
    wait_vmcnt<0>();                  // this wave's rows
    const uint8_t *wrow = ws + nl * (P::RU * 16) + int((uint32_t(nl) * uint32_t(a.row_bytes) + part0) & 15u);
    const int8_t *acode = reinterpret_cast<const int8_t *>(lds + ra.off_a) + 8 * cl;
    // scales of the lane's output tokens 16t + 4c + r at block j0
    const float *dxp[TT][4];
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            dxp[t][r] = reinterpret_cast<const float *>(lds + ra.off_d) + min(16 * t + 4 * cl + r, M - 1) * nb + j0;

    float term[NBK][TT][4];
    static_for<0, NBK>([&](auto JB) __attribute__((always_inline)) {
        constexpr int jb = decltype(JB)::value;
#pragma unroll
        for (int t = 0; t < TT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) term[jb][t][r] = 0.0f;
        if (!live || jb >= nbk) return;
        const int j = j0 + jb;
        const typename F::W wv = F::load_lds(wrow + jb * F::BB, cl);
        Scales<F> sc;
        decode_scales<F>(wv, sc);
        [[maybe_unused]] SplitB sb;
        [[maybe_unused]] uint32_t scw[2], mw[2];
        if constexpr (F::kSplit) {
            if constexpr (F::kMin) {
                uint32_t scp[2], mp[2];
                scales_k4_packed(wv.h.y, wv.h.z, wv.h.w, scp, mp);
                split_b(wv, scp, mp, sb);
            }
            else split_b(wv, cl, sb);
        } else {
            scales_k4_packed(wv.h.y, wv.h.z, wv.h.w, scw, mw);
        }
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            // the lane's A token (tokens past M repeat token M - 1; their
            // outputs are not kept); chunk h: values 64h + 8c + t, 64h + 32 + 8c + t
            const int8_t *arow = acode + min(16 * t + nl, M - 1) * (ra.acr * 16) + 256 * j;
            uint4 av[4];
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const uint2 lo = ld8(arow + 64 * h), hi = ld8(arow + 64 * h + 32);
                av[h] = make_uint4(lo.x, lo.y, hi.x, hi.y);
            }
            int S[4] = {0, 0, 0, 0};
            int4v Mb = {0, 0, 0, 0};
            if constexpr (F::kSplit) {
                int4v D1 = {0, 0, 0, 0}, D2 = {0, 0, 0, 0};
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    D1 = mfma16x16x64(av[h], sb.b1[h], D1);
                    D2 = mfma16x16x64(av[h], sb.b2[h], D2);
                    if constexpr (F::kMin) Mb = mfma16x16x64(av[h], sb.bm[h], Mb);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) S[r] = (D1[r] << F::kShift) + D2[r];
            } else {
                // Q4_K / Q5_K: one 16x16x32 MFMA per sub-block, its scale
                // applied in int32; the mins of sub-blocks 2h, 2h + 1 as
                // one 16x16x64 MFMA against broadcast bytes
                int4v D[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const uint4 &q = av[u >> 1];
                    const uint2 au = (u & 1) ? make_uint2(q.z, q.w) : make_uint2(q.x, q.y);
                    D[u] = mfma16x16x32(au, F::bop(wv, u, cl));
                }
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    const uint32_t m0 = __builtin_amdgcn_perm(0u, mw[h >> 1], 0x01010101u * uint32_t(2 * h & 3));
                    const uint32_t m1 = __builtin_amdgcn_perm(0u, mw[h >> 1], 0x01010101u * uint32_t((2 * h + 1) & 3));
                    Mb = mfma16x16x64(av[h], make_uint4(m0, m0, m1, m1), Mb);
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int su = int(__builtin_amdgcn_ubfe(scw[u >> 2], 8 * (u & 3), 8));
#pragma unroll
                    for (int r = 0; r < 4; ++r) S[r] = mad_i24(su, D[u][r], S[r]);  // |D| <= 32 * 31 * 127
                }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float dx = dxp[t][r][jb];
                if constexpr (F::kMin) term[jb][t][r] = dx * (sc.d * (float)S[r] - sc.dmin * (float)Mb[r]);  // E:11026
                else term[jb][t][r] = (sc.d * dx) * (float)S[r];                                          // E:11101 / E:3405
            }
        }
    });

    // the terms go to this wave's own (spent) weight region as
    // [block][token tile][r][lane]; after one barrier wave (rt, kp) sums
    // output r = kp of each token tile of tile rt over the 4 parts' blocks,
    // in block order
    static_assert(NBK * TT <= P::NI, "terms fit the wave's region");
    float *mine = reinterpret_cast<float *>(ws);
    if (live) {
#pragma unroll
        for (int jb = 0; jb < NBK; ++jb)
#pragma unroll
            for (int t = 0; t < TT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (jb < nbk) mine[((jb * TT + t) * 4 + r) * 64 + lane] = term[jb][t][r];
    }
    lds_barrier();
    if (live) {
        const int n = n0 + nl;
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            float x4[4][NBK];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const float *src = reinterpret_cast<const float *>(lds + (p * RTM + rt) * (P::NI * 1024));
#pragma unroll
                for (int jb = 0; jb < NBK; ++jb) x4[p][jb] = src[((jb * TT + t) * 4 + kp) * 64 + lane];
            }
            float v = 0.0f;
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const int nbp = (p + 1) * nb / 4 - p * nb / 4;
#pragma unroll
                for (int jb = 0; jb < NBK; ++jb)
                    if (jb < nbp) v = v + x4[p][jb];
            }
            const int tok = 16 * t + 4 * cl + kp;
            if (tok < M && n < a.N) {
                if (a.res) v = v + a.res[size_t(tok) * a.ldr + n];
                a.y[size_t(tok) * a.ldy + n] = v;
            }
        }
    }
}

// ============================================== one tile, codes in registers
// Up to 16 * TT tokens (TT <= 4) of a k-quant over K <= NBK * 4 * 256: a
// workgroup owns one 16-row tile and every token, one wave per K part.
// Wave kp moves its part of the 16 rows into LDS, the token scales arrive
// in LDS (then transposed to [block][token]), and the part's codes for
// every token load straight into registers from the tiles section of the
// Q8_K buffer (1 KB per wave load); each block's weights are decoded once
// for all tokens. The fp32 terms of the 4 parts then meet in LDS, and each
// wave sums a quarter of the outputs over all blocks in block order, so
// every output is the reference's block-ordered fp32 sum.
template <class F, int TT, int NBK>
struct PartCfg {
    using P = ResPart<F, NBK>;
    // terms of a wave, [block][token tile][r][lane] floats: in its own
    // (spent) part region when they fit, else in a region of their own
    static constexpr bool kOwn = NBK * TT <= P::NI;
    static constexpr int TERMS = kOwn ? 0 : 4 * NBK * TT * 1024;
};

template <class F, int TT, int NBK>
__device__ __attribute__((always_inline)) inline void part_wg(const MatArgs &a, int bx, const Q8KView &x,
                                                              const ResArgs &ra, int m0 = 0) {
    using C = PartCfg<F, TT, NBK>;
    using P = typename C::P;
    extern __shared__ __align__(16) uint8_t lds[];
    if (scan_stopped(a.scan)) return;
    const int lane = threadIdx.x & 63;
    const int kp = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nl = lane & 15, cl = lane >> 4;
    const int n0 = bx * 16, M = a.M, K = a.K, nb = K / 256;
    const int j0 = kp * nb / 4, nbk = (kp + 1) * nb / 4 - j0;
    const uint32_t lds0 = lds_addr(lds);

    // this wave's part of the tile's rows (rows past N and bytes past the
    // tile read zeros), then the token scales (dealt out to the waves)
    const uintptr_t wstart = reinterpret_cast<uintptr_t>(a.w) + size_t(n0) * a.row_bytes;
    const uint32_t bl = uint32_t(wstart & 15);
    const v4i32 rw = buf_rsrc(reinterpret_cast<const void *>(wstart - bl),
                              (bl + uint32_t(min(16, a.N - n0)) * uint32_t(a.row_bytes) + 15u) & ~15u);
    const uint32_t part0 = bl + uint32_t(j0) * uint32_t(F::BB);  // part start in row 0, from the 16-B base
    uint8_t *ws = lds + kp * (P::NI * 1024);
#pragma unroll
    for (int i = 0; i < P::NI; ++i) {
        const int p = i * 64 + lane;
        const int row = p / P::RU, u = p - row * P::RU;
        const uint32_t o = ((uint32_t(row) * uint32_t(a.row_bytes) + part0) & ~15u) + 16u * uint32_t(u);
        dma16(rw, (nbk > 0 && row < 16) ? o : kFar, lds_addr(ws) + uint32_t(i * 1024));
    }
    const int nscale = (M * nb + 63) / 64;
    const v4i32 ra_d = buf_rsrc(x.d, uint32_t(M) * uint32_t(nb) * 4u);
    for (int q = kp; q < nscale; q += 4) {
        const int e = q * 64 + lane;
        dma4(ra_d, e < M * nb ? 4u * uint32_t(e) : kFar, lds0 + uint32_t(ra.off_d + q * 256));
    }
    // The codes load into registers last: the compiler's own waits for them
    // count only its own loads, and every transfer above is older, so they
    // are exact (codes issued first would make its wait for the last code
    // also wait for every younger transfer). The wait before the barrier
    // leaves the NBK * TT * 4 code loads in flight (vmcnt retires in order,
    // so every transfer has landed): block 0's products start while the
    // later blocks' codes arrive (Q4_K 9728 x 2560, M = 8 / 48: 7.93 / 12.77
    // -> 7.78 / 12.21 us).
    // Blocks past the part repeat its last block; token slots past M hold
    // stray codes whose outputs are not kept (token tiles past the tiles
    // section's last repeat it).
    const int tlast = (M + 15) / 16 - 1;
    uint4 av[NBK][TT][4];
#pragma unroll
    for (int jb = 0; jb < NBK; ++jb) {
        const int j = j0 + min(jb, max(nbk - 1, 0));
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            const size_t tt = size_t(min(m0 / 16 + t, tlast));
#pragma unroll
            for (int h = 0; h < 4; ++h)
                av[jb][t][h] = ld16(x.qt + ((tt * size_t(nb) + size_t(j)) * 4 + size_t(h)) * 1024 + 16 * lane);
        }
    }
    asm volatile("" ::: "memory");    // every code load issued above this point
    wait_vmcnt<NBK * TT * 4>();       // this wave's transfers
    __builtin_amdgcn_s_barrier();     // everyone's scales
    // scales of tokens m0 .. m0 + 63 transposed to [block][64 tokens]
    // (tokens past M repeat M - 1), so a lane reads its 4 tokens' scales of
    // a block as one float4
    float *dxt = reinterpret_cast<float *>(lds + ra.off_d + (M * nb + 63) / 64 * 256);
    for (int e = int(threadIdx.x); e < nb * 64; e += 256) {
        const int j = e >> 6, tok = e & 63;
        dxt[e] = reinterpret_cast<const float *>(lds + ra.off_d)[min(m0 + tok, M - 1) * nb + j];
    }
    lds_barrier();

    const uint8_t *wrow = ws + nl * (P::RU * 16) + int((uint32_t(nl) * uint32_t(a.row_bytes) + part0) & 15u);
    float term[NBK][TT][4];
#pragma unroll
    for (int jb = 0; jb < NBK; ++jb) {
#pragma unroll
        for (int t = 0; t < TT; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q) term[jb][t][q] = 0.0f;
        if (jb >= nbk) continue;
        const int j = j0 + jb;
        const typename F::W wv = F::load_lds(wrow + jb * F::BB, cl);
        Scales<F> sc;
        decode_scales<F>(wv, sc);
        [[maybe_unused]] SplitB sb;
        [[maybe_unused]] uint32_t scw[2], mw[2];
        if constexpr (F::kSplit) {
            if constexpr (F::kMin) {
                uint32_t scp[2], mp[2];
                scales_k4_packed(wv.h.y, wv.h.z, wv.h.w, scp, mp);
                split_b(wv, scp, mp, sb);
            }
            else split_b(wv, cl, sb);
        } else {
            scales_k4_packed(wv.h.y, wv.h.z, wv.h.w, scw, mw);
        }
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            int S[4] = {0, 0, 0, 0};
            int4v Mb = {0, 0, 0, 0};
            if constexpr (F::kSplit) {
                int4v D1 = {0, 0, 0, 0}, D2 = {0, 0, 0, 0};
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    D1 = mfma16x16x64(av[jb][t][h], sb.b1[h], D1);
                    D2 = mfma16x16x64(av[jb][t][h], sb.b2[h], D2);
                    if constexpr (F::kMin) Mb = mfma16x16x64(av[jb][t][h], sb.bm[h], Mb);
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) S[q] = (D1[q] << F::kShift) + D2[q];
            } else {
                // Q4_K / Q5_K: one 16x16x32 MFMA per sub-block, its scale
                // applied in int32; the mins of sub-blocks 2h, 2h + 1 as
                // one 16x16x64 MFMA against broadcast bytes
                int4v D[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const uint4 &qv = av[jb][t][u >> 1];
                    const uint2 au = (u & 1) ? make_uint2(qv.z, qv.w) : make_uint2(qv.x, qv.y);
                    D[u] = mfma16x16x32(au, F::bop(wv, u, cl));
                }
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    const uint32_t m0 = __builtin_amdgcn_perm(0u, mw[h >> 1], 0x01010101u * uint32_t(2 * h & 3));
                    const uint32_t m1 = __builtin_amdgcn_perm(0u, mw[h >> 1], 0x01010101u * uint32_t((2 * h + 1) & 3));
                    Mb = mfma16x16x64(av[jb][t][h], make_uint4(m0, m0, m1, m1), Mb);
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int su = int(__builtin_amdgcn_ubfe(scw[u >> 2], 8 * (u & 3), 8));
#pragma unroll
                    for (int q = 0; q < 4; ++q) S[q] += __mul24(su, D[u][q]);
                }
            }
            const float4 dx4 = *reinterpret_cast<const float4 *>(dxt + j * 64 + 16 * t + 4 * cl);
            const float dxr[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float dx = dxr[q];
                if constexpr (F::kMin) term[jb][t][q] = dx * (sc.d * (float)S[q] - sc.dmin * (float)Mb[q]);  // E:11026
                else term[jb][t][q] = (sc.d * dx) * (float)S[q];                                          // E:11101 / E:3405
            }
        }
    }

    // the terms meet in LDS; wave kp then sums output r = kp of each token
    // tile over the 4 parts' blocks, in block order
    auto terms_of = [&](int p) __attribute__((always_inline)) {
        return reinterpret_cast<float *>(C::kOwn ? lds + p * (P::NI * 1024) : lds + ra.off_t + p * (NBK * TT * 1024));
    };
    float *mine = terms_of(kp);
#pragma unroll
    for (int jb = 0; jb < NBK; ++jb)
#pragma unroll
        for (int t = 0; t < TT; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (jb < nbk) mine[((jb * TT + t) * 4 + q) * 64 + lane] = term[jb][t][q];
    lds_barrier();
    const int n = n0 + nl;
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        float xs[4][NBK];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const float *src = terms_of(p);
#pragma unroll
            for (int jb = 0; jb < NBK; ++jb) xs[p][jb] = src[((jb * TT + t) * 4 + kp) * 64 + lane];
        }
        float v = 0.0f;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int nbp = (p + 1) * nb / 4 - p * nb / 4;
#pragma unroll
            for (int jb = 0; jb < NBK; ++jb)
                if (jb < nbp) v = v + xs[p][jb];
        }
        const int tok = m0 + 16 * t + 4 * cl + kp;
        if (tok < M && n < a.N) {
            if (a.res) v = v + a.res[size_t(tok) * a.ldr + n];
            a.y[size_t(tok) * a.ldy + n] = v;
        }
    }
}

// workgroup (bx, by): row tile bx, tokens 16 TT by ..
template <class F, int TT, int NBK>
__global__ __launch_bounds__(256) void part_kernel(MatGroup grp, Q8KView x, ResArgs ra) {
    int bx = 0;
    const MatArgs a = grp.t[group_task(grp, int(blockIdx.x), bx)];
    part_wg<F, TT, NBK>(a, bx, x, ra, int(blockIdx.y) * 16 * TT);
}

// ================================================== F32 / F16 weight rows
// sdot_row_f32_batch / sdot_row_f16_batch (E:3410-3440) for M >= 2: the
// fp16 input (the h section of the Q8_K buffer) against 16 weight rows per
// wave on the matrix unit, fp32 accumulation — F16 rows by
// v_mfma_f32_16x16x32_f16 (products of fp16 values are exact in fp32), F32
// rows by v_mfma_f32_16x16x4_f32 on the input widened to fp32. Lane l
// supplies token / row l % 16 and k-slice l / 16 (F32: the four k of a
// 16-B piece go to four successive MFMAs, a k permutation shared by both
// operands) and receives D[token 4 (l / 16) + r][row l % 16]. The sums'
// order is not the reference's row order: within the stated tolerance, not
// bit-exact. Rows past N and tokens past M repeat the last one (their
// outputs are not kept), so every load stays inside the buffers.
typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8v __attribute__((ext_vector_type(8)));
template <bool F16W>
__device__ inline f32x4v float_tile(const MatArgs &a, int n0, int m0, int k0, int k1, const uint16_t *xh,
                                    f32x4v acc) {
    const int lane = threadIdx.x & 63, nl = lane & 15, cl = lane >> 4;
    const uint8_t *wr = a.w + size_t(min(n0 + nl, a.N - 1)) * a.row_bytes;
    const uint16_t *xr = xh + size_t(min(m0 + nl, a.M - 1)) * size_t(a.K);
    constexpr int KQ = F16W ? 32 : 16;  // k per step of the 4 lane groups
    constexpr int U = 8;                // steps whose loads are issued together
    auto step = [&](const uint4 &wq, const uint4 &xq) __attribute__((always_inline)) {
        if constexpr (F16W) {
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8v, xq), __builtin_bit_cast(f16x8v, wq),
                                                         acc, 0, 0, 0);
        } else {
            const float xv[4] = {fp16_bits_to_f32(xq.x & 0xFFFFu), fp16_bits_to_f32(xq.x >> 16),
                                 fp16_bits_to_f32(xq.y & 0xFFFFu), fp16_bits_to_f32(xq.y >> 16)};
            const uint32_t wv[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[i], __builtin_bit_cast(float, wv[i]), acc, 0, 0, 0);
        }
    };
    auto load = [&](int k, uint4 &wq, uint4 &xq) __attribute__((always_inline)) {
        if constexpr (F16W) {
            wq = ld16_nt(wr + 2 * size_t(k + 8 * cl));
            xq = ld16(xr + k + 8 * cl);
        } else {
            wq = ld16_nt(wr + 4 * size_t(k + 4 * cl));
            const uint2 h = ld8(xr + k + 4 * cl);
            xq = make_uint4(h.x, h.y, 0u, 0u);
        }
    };
    int k = k0;
    for (; k + U * KQ <= k1; k += U * KQ) {
        uint4 wq[U], xq[U];
#pragma unroll
        for (int u = 0; u < U; ++u) load(k + u * KQ, wq[u], xq[u]);
#pragma unroll
        for (int u = 0; u < U; ++u) step(wq[u], xq[u]);
    }
    for (; k < k1; k += KQ) {
        uint4 wq, xq;
        load(k, wq, xq);
        step(wq, xq);
    }
    return acc;
}

// An F32 / F16 task in the part kernel's shape: one 16-row tile and the
// 16 TT tokens from m0, wave kp taking the kp-th quarter of K; the four
// quarters' sums meet in LDS and are added in quarter order, as the k-quant
// parts are. Token tiles past M are skipped.
template <bool F16W, int TT>
__device__ __attribute__((always_inline)) inline void part_float_wg(const MatArgs &a, int bx, const Q8KView &x,
                                                                    int m0 = 0) {
    extern __shared__ __align__(16) uint8_t lds[];
    if (scan_stopped(a.scan)) return;
    const int lane = threadIdx.x & 63, nl = lane & 15, cl = lane >> 4;
    const int kp = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = bx * 16;
    constexpr int KQ = F16W ? 32 : 16;  // values per k step of the 4 lane groups
    const int steps = a.K / KQ;
    const int k0 = (kp * steps / 4) * KQ, k1 = ((kp + 1) * steps / 4) * KQ;
    float *terms = reinterpret_cast<float *>(lds);  // [part][token tile][r][lane]
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        if (m0 + 16 * t >= a.M) break;  // the same in every lane
        f32x4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
        acc = float_tile<F16W>(a, n0, m0 + 16 * t, k0, k1, x.h, acc);
#pragma unroll
        for (int r = 0; r < 4; ++r) terms[((kp * TT + t) * 4 + r) * 64 + lane] = acc[r];
    }
    lds_barrier();
    const int n = n0 + nl;
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        if (m0 + 16 * t >= a.M) break;
        float v = 0.0f;
#pragma unroll
        for (int p = 0; p < 4; ++p) v = v + terms[((p * TT + t) * 4 + kp) * 64 + lane];
        const int tok = m0 + 16 * t + 4 * cl + kp;
        if (tok < a.M && n < a.N) {
            if (a.res) v = v + a.res[size_t(tok) * a.ldr + n];
            a.y[size_t(tok) * a.ldy + n] = v;
        }
    }
}

// One F32 / F16 task (or several of one type) for M >= 2: workgroup (bx, by)
// owns rows 16 bx .. +15 and tokens 64 by .. +63 over all of K.
template <bool F16W>
__global__ __launch_bounds__(256) void float_tile_kernel(MatGroup grp, Q8KView x) {
    int bx = 0;
    const MatArgs a = grp.t[group_task(grp, int(blockIdx.x), bx)];
    part_float_wg<F16W, 4>(a, bx, x, int(blockIdx.y) * 64);
}

// ================================================ several formats at once
// A task group whose types differ (E:7954-7959, E:8110-8114) in one launch
// for 2 <= M <= 64 and K <= 3072: every workgroup is one 16-row tile of its
// task and runs that format's part-kernel body (the k-quants folded from
// two token tiles, as a single-format launch does). ra[f] holds format f's
// LDS offsets (f = kMixQ4K ..); the launch's LDS is the largest of them.
constexpr int kMixQ4K = 0, kMixQ5K = 1, kMixQ6K = 2, kMixF32 = 3, kMixF16 = 4, kMixFormats = 5;
struct MixArgs {
    ResArgs ra[kMixFormats];
};
__host__ __device__ inline int mix_format(uint32_t type) {
    return type == kQ4_K ? kMixQ4K : type == kQ5_K ? kMixQ5K : type == kQ6_K ? kMixQ6K : type == kF32 ? kMixF32 : kMixF16;
}

template <int TT>
__global__ __launch_bounds__(256) void part_mixed_kernel(MatGroup grp, Q8KView x, MixArgs mx) {
    int bx = 0;
    const MatArgs a = grp.t[group_task(grp, int(blockIdx.x), bx)];
    using Q4 = std::conditional_t<(TT > 1), MQ4KS, MQ4K>;
    using Q5 = std::conditional_t<(TT > 1), MQ5KS, MQ5K>;
    switch (a.type) {
        case kQ4_K: part_wg<Q4, TT, 3>(a, bx, x, mx.ra[kMixQ4K]); break;
        case kQ5_K: part_wg<Q5, TT, 3>(a, bx, x, mx.ra[kMixQ5K]); break;
        case kQ6_K: part_wg<MQ6KS, TT, 3>(a, bx, x, mx.ra[kMixQ6K]); break;
        case kF32: part_float_wg<false, TT>(a, bx, x); break;
        case kF16: part_float_wg<true, TT>(a, bx, x); break;
        default: break;
    }
}

int mfma_cu_count();

// Resident-tile launch if the tiles, codes and scales fit one CU's LDS;
// returns hipErrorNotSupported (nothing launched) otherwise.
template <class F, int TT, int NBK, int RTM>
static hipError_t launch_res_r(const MatArgs *tasks, int n, const Q8KView &x, int tiles, hipStream_t s) {
    using P = ResPart<F, NBK>;
    const MatArgs &a = tasks[0];
    const int nb = a.K / 256;
    if (nb > 4 * NBK) return hipErrorNotSupported;
    ResArgs ra{};
    ra.tiles = tiles;
    ra.acr = a.K / 16 + 1;
    ra.off_a = 4 * RTM * P::NI * 1024;
    ra.off_d = ra.off_a + (a.M * ra.acr + 63) / 64 * 1024;
    ra.lds = ra.off_d + (a.M * nb + 63) / 64 * 256;
    const size_t lds = size_t(ra.lds);
    if (lds > 160 * 1024) return hipErrorNotSupported;
    MatGroup g{};
    g.n = n;
    g.wg0[0] = 0;
    for (int i = 0; i < n; ++i) {
        g.t[i] = tasks[i];
        g.wg0[i + 1] = g.wg0[i] + (tasks[i].N + 15) / 16;
    }
    // at most RTM tiles per workgroup, and one workgroup per CU while the
    // tiles last
    const unsigned grid = unsigned(max((tiles + RTM - 1) / RTM, min(tiles, mfma_cu_count())));
    hipLaunchKernelGGL((res_kernel<F, TT, NBK, RTM>), dim3(grid), dim3(256 * RTM), lds, s, g, x, ra);
    return hipGetLastError();
}

// Part-kernel launch if the parts, scales and terms fit one CU's LDS;
// returns hipErrorNotSupported (nothing launched) otherwise. One tile and
// one group of 16 TT tokens per workgroup (grid rows: the token groups).
// Up to 32 tokens a workgroup needs few enough registers for three per CU,
// so any number of tiles runs as one wave of workgroups; past 32 tokens
// (three or four token tiles, as the mixed-group kernel uses) only one fits
// a CU, and the tiles must not outnumber the CUs.
// LDS offsets of the part-kernel body of format F for (M, K)
template <class F, int TT, int NBK = 3>
static ResArgs part_args(int M, int K) {
    using C = PartCfg<F, TT, NBK>;
    using P = typename C::P;
    const int nb = K / 256;
    ResArgs ra{};
    ra.off_d = 4 * P::NI * 1024;
    ra.off_t = ra.off_d + (M * nb + 63) / 64 * 256 + nb * 64 * 4;
    ra.lds = ra.off_t + C::TERMS;
    return ra;
}

template <class F, int TT, int NBK>
static hipError_t launch_part_n(const MatArgs *tasks, int n, const Q8KView &x, hipStream_t s) {
    const MatArgs &a = tasks[0];
    const int nb = a.K / 256;
    int tiles = 0;
    for (int i = 0; i < n; ++i) tiles += (tasks[i].N + 15) / 16;
    if (nb > 4 * NBK || !x.qt || (TT > 2 && tiles > mfma_cu_count())) return hipErrorNotSupported;
    ResArgs ra = part_args<F, TT, NBK>(a.M, a.K);
    ra.tiles = tiles;
    if (ra.lds > 160 * 1024) return hipErrorNotSupported;
    MatGroup g{};
    g.n = n;
    g.wg0[0] = 0;
    for (int i = 0; i < n; ++i) {
        g.t[i] = tasks[i];
        g.wg0[i + 1] = g.wg0[i] + (tasks[i].N + 15) / 16;
    }
    const dim3 grid(unsigned(tiles), unsigned((a.M + 16 * TT - 1) / (16 * TT)));
    hipLaunchKernelGGL((part_kernel<F, TT, NBK>), grid, dim3(256), size_t(ra.lds), s, g, x, ra);
    return hipGetLastError();
}

// up to 3 blocks per K part (K <= 3072), else 4 (K <= 4096)
template <class F, int TT>
static hipError_t launch_part(const MatArgs *tasks, int n, const Q8KView &x, hipStream_t s) {
    if (tasks[0].K <= 3072) return launch_part_n<F, TT, 3>(tasks, n, x, s);
    return launch_part_n<F, TT, 4>(tasks, n, x, s);
}

static int group_tiles(const MatArgs *tasks, int n) {
    int tiles = 0;
    for (int i = 0; i < n; ++i) tiles += (tasks[i].N + 15) / 16;
    return tiles;
}

// The resident tiles three to a workgroup, where the row tiles number more
// than two and at most three per CU; hipErrorNotSupported (nothing
// launched) elsewhere.
template <class F, int TT>
static hipError_t launch_res(const MatArgs *tasks, int n, const Q8KView &x, hipStream_t s) {
    const int tiles = group_tiles(tasks, n), cus = mfma_cu_count();
    if (tiles <= 2 * cus || tiles > 3 * cus) return hipErrorNotSupported;
    return launch_res_r<F, TT, 3, 3>(tasks, n, x, tiles, s);
}

template <class C, class F>
static hipError_t launch_tile_t(const MatArgs *tasks, int n, const typename ActOf<F>::T &x, hipStream_t s) {
    if constexpr (C::AT)
        if (!x.qt) return hipErrorInvalidValue;  // the codes are read from the tiles section
    MatGroup g{};
    g.n = n;
    g.wg0[0] = 0;
    for (int i = 0; i < n; ++i) {
        g.t[i] = tasks[i];
        g.wg0[i + 1] = g.wg0[i] + (tasks[i].N + C::ROWS - 1) / C::ROWS;
    }
    const dim3 grid(unsigned(g.wg0[n]), unsigned((tasks[0].M + C::TOK - 1) / C::TOK));
    hipLaunchKernelGGL((tile_kernel<C, F>), grid, dim3(256), size_t(C::LDS), s, g, x);
    return hipGetLastError();
}

// the prefill kernel (qmm_slab.hip); hipErrorNotSupported where it does not apply
template <class F>
hipError_t launch_slab(const MatArgs *tasks, int n, const typename ActOf<F>::T &x, hipStream_t s);

template <class F>
static hipError_t launch_tile(const MatArgs *tasks, int n, const typename ActOf<F>::T &x, hipStream_t s) {
    const MatArgs &a = tasks[0];
    if constexpr (std::is_same_v<F, MQ4K> || std::is_same_v<F, MQ5K> || std::is_same_v<F, MQ6KS>) {
        // (Q6_K at 17..64 tokens over K > 4096, Q4_K / Q5_K at 33..64 over
        // K >= 8192: the decoded slabs split over K, where the launcher
        // takes them; Q6_K over K <= 4096 measured faster on the part kernel:
        // 9728 x 3584 at M = 48 / 64 31.3 / 32.4 -> 22.0 / 22.5 us, 1024 x
        // 3328 at M = 24 / 64 10.9 / 12.4 -> 7.3 / 7.3)
        // past 64 tokens over K <= 4096, the part kernel's 32-token groups
        // where they number at most 4.5 workgroups per CU (over K > 3072: 3):
        // the slabs' 64- and 128-token tiles leave most CUs idle on short
        // tensors (Q6_K 1024 x 2560 at M = 80..128: 11.6 -> 6.8 us, Q4_K
        // 2560 x 2560 at M = 80 / 128 11.3 / 11.4 -> 7.3 / 8.8, Q5_K 6144 x
        // 2560 at M = 96 16.2 -> 14.5, Q5_K 1024 x 4096 at M = 80 17.5 ->
        // 8.1; 9728 x 2560 at M = 80 14.8 against 17.1 keeps the slabs, Q6_K
        // 4096 x 4096 at M = 128 16.8 against 19.6)
        const int pwg = group_tiles(tasks, n) * ((a.M + 31) / 32), pcus = mfma_cu_count();
        if (a.M > 64 && a.K <= 4096 && (a.K <= 3072 ? 2 * pwg <= 9 * pcus : pwg <= 3 * pcus)) {
            const hipError_t e = launch_part<typename Folded<F>::T, 2>(tasks, n, x, s);
            if (e != hipErrorNotSupported) return e;
        }
        if (a.M > 64 || (a.M > 16 && a.K > 4096 && (std::is_same_v<F, MQ6KS> || (a.M > 32 && a.K >= 8192)))) {
            const hipError_t e = launch_slab<typename Folded<F>::T>(tasks, n, x, s);
            if (e != hipErrorNotSupported) return e;
        }
    }
    // buffer offsets are 32-bit with kFar past every range (the tiles section
    // holds ceil(M / 16) * 16 tokens)
    if (size_t((a.M + 15) & ~15) * size_t(a.K) >= (size_t(1) << 31)) return hipErrorInvalidValue;
    using G = typename Folded<F>::T;
    // 9..64 tokens over K > 3072, and Q8_0 at any K: 16-row x 16-token tiles,
    // each chunk's 4 blocks split over the 4 waves, two workgroups per CU,
    // where the configurations below would leave CUs idle: at 9..16 tokens
    // always, at 17..32 where the 32 x 32 tiles number fewer than the CUs,
    // at 33..64 where the 64 x 32 tiles number fewer than 5/8 of them.
    // Measured: Q6_K 2560 x 9728 at M = 16 / 32 / 64 13.2 / 18.7 / 27.0 us
    // against 22.6 / 29.1 / 44.7; Q8_0 2560 x 2560 10.5 / 12.1 / 17.0 against
    // 15.7 / 20.8 / 22.7; on taller tensors (Q4_K / Q6_K 9728 x 4096, Q8_0
    // 6144 x 2560) faster at M = 16 (12.0 / 14.9 / 13.3 against 13.6 / 16.5 /
    // 15.1), slower at M = 64 (27.9 / 36.4 / 27.5 against 21.8 / 28.9 / 23.0)
    // (Q4_K / Q5_K over K <= 4096 take the part kernel below: 4096 x 4096
    // at M = 24 / 40 / 64 8.3 / 10.9 / 13.0 -> 7.6 / 9.0 / 10.0 us, 2560 x
    // 3584 8.9 / 9.3 / 12.4 -> 7.3 / 7.4 / 10.0, Q5_K 1024 x 4096 6.7 -> 6.1)
    // (and Q6_K from 17 tokens over K <= 4096: 2560 x 4096 at M = 24 / 48
    // 10.4 / 12.0 -> 8.5 / 9.9 us, 4096 x 4096 at M = 24 10.8 -> 9.4)
    constexpr bool kQ45 = std::is_same_v<F, MQ4K> || std::is_same_v<F, MQ5K>;
    constexpr bool kPart = kQ45 || std::is_same_v<F, MQ6KS>;
    if (a.M > 8 && a.M <= 64 && (a.K > 3072 || std::is_same_v<G, MQ80>) &&
        !(kPart && a.K <= 4096 && (kQ45 || a.M > 16))) {
        int wg = 0;  // workgroups of the configuration below
        for (int i = 0; i < n; ++i)
            wg += a.M <= 32 ? (tasks[i].N + 31) / 32 : (tasks[i].N + 63) / 64 * ((a.M + 31) / 32);
        const int cus = mfma_cu_count();
        if (a.M <= 16 || (a.M <= 32 ? wg < cus : 8 * wg < 5 * cus))
            return launch_tile_t<TileCfg<G, 1, 1, 1, 1, 4, 16, 2, 100 * 1024>, G>(tasks, n, x, s);
    }
    // up to 64 tokens over K <= 3072: the resident-tile and part kernels.
    // Past 16 tokens the part kernel's workgroups each take a group of 16
    // or 32 tokens (a grid row per group): at 17..32 tokens groups of 16
    // where the row tiles are at most two per CU (else all 32 tokens per
    // workgroup), at 33..48 groups of 16, at 49..64 groups of 32 (of 16
    // where those would leave half the CUs idle). Measured (Q4_K 9728 x
    // 2560 / Q5_K 4096 x 2560, M = 24, 40, 48, 64): 10.22 / 6.60, 13.37 /
    // 7.79, 12.93 / 7.87, 14.02 / 8.70 us against one workgroup per row
    // tile (Q4_K past 32 tokens: the 64 x 32 tiles) 10.22 / 7.28, 14.90 /
    // 8.33, 14.94 / 8.28, 15.32 / 9.27; from a sweep of six tensors at
    // M = 5..64: Q4_K 19456 x 2560 at M = 5..16 13.5..14.4 -> 11.0..11.1
    // (one tile per workgroup past three tiles per CU), Q5_K 6144 x 2560 at
    // M = 24 / 32 9.3 -> 8.1 / 8.3, Q5_K 1024 x 2560 at M = 64 6.8 -> 5.3.
    if constexpr (std::is_same_v<F, MQ4K> || std::is_same_v<F, MQ5K> || std::is_same_v<F, MQ6KS>) {
        hipError_t e = hipErrorNotSupported;
        // (K up to 4096: from 17 tokens on the tensors the K-split tiles
        // above leave — Q4_K 9728 x 4096 at M = 24 / 48 / 64 16.0 / 21.6 /
        // 21.8 -> 14.4 / 18.2 / 20.3 us against the chunked tiles, 6144 x
        // 3584 at M = 48 14.3 -> 12.1 — and Q4_K / Q5_K at every M <= 64:
        // Q4_K 9728 x 4096 at M = 8 / 16 10.4 / 12.0 -> 10.2 / 10.2 us,
        // 19456 x 4096 at M = 12 18.3 -> 14.3, 2560 x 4096 at M = 8 6.65 ->
        // 5.83, Q5_K 2560 x 3328 at M = 8 / 16 6.81 / 6.88 -> 6.05 / 6.02,
        // against the 8-token and the K-split tiles; Q6_K measured slower
        // at 8 tokens, 4096 x 4096 7.8 -> 8.2)
        if (a.K <= 3072 || (a.K <= 4096 && (a.M > 16 || kQ45))) {
            const int tiles = group_tiles(tasks, n), cus = mfma_cu_count();
            if (a.M <= 16) {
                // one tile per workgroup, but for Q4_K at 8 tokens or fewer
                // on more than two row tiles per CU (up to three): there the
                // resident tiles, three per workgroup, measure level or
                // faster (9728 x 2560 at M = 5: 7.97 -> 7.78 us); elsewhere
                // the part kernel is faster (Q5_K / Q6_K 6144 x 2560 at
                // M = 16: 7.57 / 9.02 -> 6.90 / 8.18 us)
                if (std::is_same_v<F, MQ4K> && a.M <= 8) e = launch_res<F, 1>(tasks, n, x, s);
                if (e == hipErrorNotSupported) e = launch_part<F, 1>(tasks, n, x, s);
            } else if (a.M <= 32) {
                // Q6_K (the costlier unpacking) takes all 32 tokens per
                // workgroup from more than half a tile per CU (2560 x 2560
                // at M = 24: 7.32 -> 6.99 us, 1024 x 2560: 5.99 against 6.75)
                const bool g16 = tiles <= 2 * cus && !(std::is_same_v<F, MQ6KS> && 2 * tiles > cus);
                e = g16 ? launch_part<F, 1>(tasks, n, x, s) : launch_part<G, 2>(tasks, n, x, s);
            } else if (a.M <= 48) {
                // groups of 16; Q6_K groups of 32 from 3/4 of a tile per CU
                // (6144 x 2560 at M = 40: 13.1 -> 11.4 us, 3328 x 2560 9.3 ->
                // 8.6; 2560 x 2560 7.6 against 8.1)
                const bool g32 = std::is_same_v<F, MQ6KS> && 4 * tiles > 3 * cus;
                e = g32 ? launch_part<G, 2>(tasks, n, x, s) : launch_part<F, 1>(tasks, n, x, s);
            } else if (a.M <= 64) {
                // groups of 32 from half a tile per CU, over K > 3072 (4
                // blocks per K part) from 3/4 (Q4_K 2560 x 4096 at M = 64:
                // 8.8 against 9.4 us; 4096 x 4096 9.8 against 11.1), Q6_K
                // there past 1/4 (2560 x 4096: 13.1 -> 11.4 us, 2048 x 3584
                // 9.0 -> 8.3; 1024 x 3328 7.3 against 8.4)
                const bool q6 = std::is_same_v<F, MQ6KS>;
                const bool g16 = a.K > 3072 ? (q6 ? 4 * tiles <= cus : 4 * tiles < 3 * cus) : 2 * tiles < cus;
                e = g16 ? launch_part<F, 1>(tasks, n, x, s) : launch_part<G, 2>(tasks, n, x, s);
            }
        }
        if (e != hipErrorNotSupported) return e;
    }
    //                          WR WT PR PT KS TR PD  LDS budget
    if constexpr (kSmallM<F>) {
        // codes resident for K <= 2560 (the hidden size of the workload)
        if (a.M <= 8 && a.K <= 2560)
            return launch_tile_t<TileCfg<F, 1, 1, 1, 1, 4, 8, 2, 53 * 1024, 2560>, F>(tasks, n, x, s);
        if (a.M <= 8) return launch_tile_t<TileCfg<F, 1, 1, 1, 1, 4, 8, 2, 52 * 1024>, F>(tasks, n, x, s);
        if (a.M <= 16 && a.K <= 2560)
            return launch_tile_t<TileCfg<F, 1, 1, 2, 1, 2, 16, 2, 80 * 1024, 2560>, F>(tasks, n, x, s);
        if (a.M <= 16) return launch_tile_t<TileCfg<F, 1, 1, 2, 1, 2, 16, 2, 56 * 1024>, F>(tasks, n, x, s);
    }
    if constexpr (!std::is_same_v<G, F>) {
        return launch_tile<G>(tasks, n, x, s);
    } else {
        if (a.M <= 32) return launch_tile_t<TileCfg<F, 1, 2, 2, 1, 2, 16, 2, 80 * 1024>, F>(tasks, n, x, s);
        // 64 rows x 32 tokens: half the activation re-reads of 32-row tiles
        if (a.M <= 64) return launch_tile_t<TileCfg<F, 1, 2, 4, 1, 1, 16, 2, 53 * 1024>, F>(tasks, n, x, s);
        // folded formats: one row tile decoded per wave, shared by 4 (Q6_K: 3)
        // token tiles
        if constexpr (F::kSplit && F::NU > 8)
            return launch_tile_t<TileCfg<F, 1, 3, 4, 1, 1, 16, 2, 76 * 1024>, F>(tasks, n, x, s);
        else if constexpr (F::kSplit)
            return launch_tile_t<TileCfg<F, 1, 4, 4, 1, 1, 16, 2, 76 * 1024>, F>(tasks, n, x, s);
        else {  // Q8_0: a fp32 term per 32 values; smaller tiles, 3 workgroups per CU
            // 64 x 32 tiles; 64 x 16 where the 64 x 32 tiles number at most 1.5
            // per CU (2560 x 2560 at M = 65 / 128 / 256: 20.4 / 20.5 / 23.4 ->
            // 15.0 / 16.9 / 20.4 us; 6144 x 2560 at M = 128: 24.0 -> 21.6; at
            // 1.56 per CU and above slower: 2560 x 2560 at M = 320 23.7 -> 29.2)
            int wg = 0;
            for (int i = 0; i < n; ++i) wg += (tasks[i].N + 63) / 64 * ((a.M + 31) / 32);
            if (2 * wg <= 3 * mfma_cu_count())
                return launch_tile_t<TileCfg<F, 1, 1, 4, 1, 1, 16, 2, 52 * 1024>, F>(tasks, n, x, s);
            return launch_tile_t<TileCfg<F, 1, 2, 4, 1, 1, 16, 2, 52 * 1024>, F>(tasks, n, x, s);
        }
    }
}

template <int TT>
static hipError_t launch_part_mixed_t(const MatArgs *tasks, int n, const Q8KView &x, hipStream_t s) {
    const int M = tasks[0].M, K = tasks[0].K;
    using Q4 = std::conditional_t<(TT > 1), MQ4KS, MQ4K>;
    using Q5 = std::conditional_t<(TT > 1), MQ5KS, MQ5K>;
    MixArgs mx{};
    mx.ra[kMixQ4K] = part_args<Q4, TT>(M, K);
    mx.ra[kMixQ5K] = part_args<Q5, TT>(M, K);
    mx.ra[kMixQ6K] = part_args<MQ6KS, TT>(M, K);
    mx.ra[kMixF32].lds = mx.ra[kMixF16].lds = 4 * TT * 1024;
    MatGroup g{};
    g.n = n;
    g.wg0[0] = 0;
    int lds = 0;
    for (int i = 0; i < n; ++i) {
        g.t[i] = tasks[i];
        g.wg0[i + 1] = g.wg0[i] + (tasks[i].N + 15) / 16;
        lds = max(lds, mx.ra[mix_format(tasks[i].type)].lds);
    }
    if (lds > 160 * 1024) return hipErrorNotSupported;
    hipLaunchKernelGGL((part_mixed_kernel<TT>), dim3(unsigned(g.wg0[n])), dim3(256), size_t(lds), s, g, x, mx);
    return hipGetLastError();
}

// Several types in one launch (k-quants, F32, F16; 2 <= M <= 64, K <= 3072,
// K % 256 == 0, no Q8_0); hipErrorNotSupported (nothing launched) otherwise.
// Past 32 tokens a workgroup needs a CU to itself, so the tiles must not
// outnumber the CUs.
hipError_t launch_mfma_mixed(const MatArgs *tasks, int n, const Q8KView &x, hipStream_t s) {
    if (n < 1 || n > kMaxGroup) return hipErrorInvalidValue;
    const int M = tasks[0].M, K = tasks[0].K;
    if (M < 2 || M > 64 || K > 3072 || K % 256 || !x.qt || !x.h) return hipErrorNotSupported;
    int tiles = 0;
    for (int i = 0; i < n; ++i) {
        if (tasks[i].type == kQ8_0) return hipErrorNotSupported;
        tiles += (tasks[i].N + 15) / 16;
    }
    if (M <= 16) return launch_part_mixed_t<1>(tasks, n, x, s);
    if (M <= 32) return launch_part_mixed_t<2>(tasks, n, x, s);
    if (tiles > mfma_cu_count()) return hipErrorNotSupported;
    if (M <= 48) return launch_part_mixed_t<3>(tasks, n, x, s);
    return launch_part_mixed_t<4>(tasks, n, x, s);
}

// F32 / F16 tasks of one type, M >= 2 (any K with K % 32 == 0 for F16,
// K % 16 == 0 for F32)
static hipError_t launch_float(uint32_t type, const MatArgs *tasks, int n, const Q8KView &x, hipStream_t s) {
    if (!x.h) return hipErrorInvalidValue;
    MatGroup g{};
    g.n = n;
    g.wg0[0] = 0;
    for (int i = 0; i < n; ++i) {
        g.t[i] = tasks[i];
        g.wg0[i + 1] = g.wg0[i] + (tasks[i].N + 15) / 16;
    }
    const dim3 grid(unsigned(g.wg0[n]), unsigned((tasks[0].M + 63) / 64));
    const size_t lds = 4 * 4 * 1024;  // the four parts' sums of 4 token tiles
    if (type == kF16) hipLaunchKernelGGL((float_tile_kernel<true>), grid, dim3(256), lds, s, g, x);
    else hipLaunchKernelGGL((float_tile_kernel<false>), grid, dim3(256), lds, s, g, x);
    return hipGetLastError();
}

int mfma_cu_count() {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int c = 0;
        cus[dev] = (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && c > 0) ? c : 256;
    }
    return cus[dev];
}

// 2 tokens always; 3 from 32 up to 96 rows per CU over K <= 4096 (Q4_K
// 19456 x 2560: 10.4 against 10.8 us, 9728 x 2560: 7.1 against 7.7). At 4
// tokens, and at 3 on taller tensors, the MFMA kernels measure faster since
// the part kernel issues its codes ahead of its first block (Q6_K 151936 x
// 2560 at M = 3 / 4: 80.8 / 92.7 -> 74.5 / 77.3 us, Q4_K 25000 x 1024 at
// M = 4: 13.0 -> 8.8, Q4_K 19456 x 2560 at M = 4: 11.7 -> 10.8).
bool gemv_mt_shape(const MatArgs &a) {
    const int cus = mfma_cu_count();
    if (a.M == 2) return true;
    return a.M == 3 && a.K <= 4096 && a.N >= 32 * cus && a.N < 96 * cus;
}

hipError_t launch_mfma(uint32_t type, const MatArgs *tasks, int n, const Q8KView &xk, const Q80View &x0,
                       hipStream_t s) {
    if (n < 1 || n > kMaxGroup) return hipErrorInvalidValue;
    // one k-quant task at 2 tokens, or at 3..4 on a tensor tall enough that
    // the MFMA kernels need several rounds of workgroups: the batch-1 GEMV's
    // shape (measured, M = 2: Q4_K 9728 x 2560 7.75 -> 6.16 us, Q6_K 2560 x
    // 9728 13.57 -> 9.00, Q6_K 151936 x 2560 111 -> 62; M = 4: Q6_K 151936 x
    // 2560 111 -> 93, while Q4_K 9728 x 2560 went 7.73 -> 8.58)
    if (n == 1 && gemv_mt_shape(tasks[0])) {
        const hipError_t e = launch_gemv_mt(type, tasks, n, xk, s);
        if (e != hipErrorNotSupported) return e;
    }
    switch (type) {
        case kQ4_K: return launch_tile<MQ4K>(tasks, n, xk, s);
        case kQ5_K: return launch_tile<MQ5K>(tasks, n, xk, s);
        case kQ6_K: return launch_tile<MQ6KS>(tasks, n, xk, s);
        case kQ8_0: return launch_tile<MQ80>(tasks, n, x0, s);
        case kF32:
        case kF16: return launch_float(type, tasks, n, xk, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace qmm
