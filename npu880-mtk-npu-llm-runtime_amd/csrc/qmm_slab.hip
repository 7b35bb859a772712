// qmm_slab.hip — prefill GEMM (M > 64 tokens) over GGUF-packed k-quant rows
// (Q4_K, Q5_K, Q6_K) with int8 MFMA, gfx950.
//
// Workgroup = NW (4 or 8) waves on a slab of R = 16 RW PR weight rows x
// T = 16 TW PT tokens; wave (pr, pt) owns RW row tiles x TW token tiles of
// 16 x 16. The K
// loop walks one 256-value block at a time through PD LDS stages, each filled by direct buffer -> LDS
// transfers (buffer_load ... lds): the slab's packed weight rows, the
// tokens' codes from the tiles section of the activation buffer (already in
// MFMA operand order), their fp16 sums of 16 codes (bh section) and their
// block scales. A wave unpacks each of its row tiles once per step into
// registers (the unit scales folded into two int8 B operands, as the small-M
// kernels do) and reuses it for all TW token tiles, so the unpacking is paid
// once per 16 TW tokens.
//
// Per 16 x 16 tile and block: S = 8 D1 + D2 (Q4_K) or 256 D1 + D2 (Q5_K,
// Q6_K) from two v_mfma_i32_16x16x64_i8 chains over the block's four 64-value
// chunks; the Q4_K / Q5_K min term Mb = sum_u m_u bsum32_u from one
// v_mfma_f32_16x16x16_f16 of the 16 sums of 16 codes (|sum| <= 2032) against
// the mins (<= 63), both exact in fp16, every product and partial sum an
// integer below 2^24, so the fp32 result is Mb exactly, in any summation
// order. The per-block fp32 update is the reference's expression, blocks in
// order, so every output equals the reference's fp32 sum bit for bit:
//   Q4_K / Q5_K: acc += dx * (d * (float)S - dmin * (float)Mb)   (E:11026, E:11063)
//   Q6_K:        acc += (d * dx) * (float)S                      (E:11101)
//
// Workgroups are numbered so that the ones sharing a row slab run together on
// one XCD (workgroup b runs on XCD b mod 8): that XCD's L2 then serves the
// slab's weights to every token group after the first read from HBM.
#include "qmm_kformats.h"

namespace qmm {

typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

template <class F, int RW_, int TW_, int PR_, int PD_, int NW_ = 4, int WPS_ = 1>
struct SlabCfg {
    static constexpr int NW = NW_;    // waves per workgroup
    static constexpr int WPS = WPS_;  // waves per SIMD the registers must allow (launch bound)
    static constexpr int RW = RW_, TW = TW_, PR = PR_, PT = NW_ / PR_, PD = PD_;
    static_assert(PR * PT == NW, "PR x PT waves");
    static constexpr bool MIN = F::kMin;
    static constexpr int R = 16 * RW * PR;  // weight rows per workgroup
    static constexpr int T = 16 * TW * PT;  // tokens per workgroup
    static constexpr int SB = F::BB;  // weight bytes per row and step
    // rows of Q4_K / Q5_K start 16-B aligned (the launcher checks):
    // a step's bytes are whole 16-B units; Q6_K's 210-B blocks take the 16-B
    // aligned span around them (at most 14 B of lead-in, 4 B read past).
    static constexpr bool ALIGNED = SB % 16 == 0;
    static constexpr int WCR = (ALIGNED ? SB / 16 : (SB + 30) / 16) | 1;  // 16-B units per row, odd
    static constexpr int NWI = (R * WCR + 63) / 64;       // weight transfers (1 KB each)
    static constexpr int NAI = (T / 16) * 4;              // code transfers (4 KB per token tile)
    static constexpr int NBI = MIN ? (T / 16 * 32 + 63) / 64 : 0;  // bh transfers (512 B per token tile)
    static constexpr int NDI = (T + 63) / 64;                        // scales (4-B transfers)
    static constexpr int NWW = (NWI + NW - 1) / NW, NAW = NAI / NW, NBW = (NBI + NW - 1) / NW,
                         NDW = (NDI + NW - 1) / NW;
    static constexpr int L = NWW + NAW + NBW + NDW;       // transfers per wave and step
    static constexpr int OFF_A = NWI * 1024;
    static constexpr int OFF_B = OFF_A + NAI * 1024;
    static constexpr int OFF_D = OFF_B + NBI * 1024;
    static constexpr int STAGE = OFF_D + NDI * 256;
    static constexpr int OFF_DUMP = PD * STAGE, LDS = OFF_DUMP + 1024;
    static_assert(NAI % NW == 0, "code transfers: a multiple of the waves");
    static_assert((PD - 2) * L <= 63, "vmcnt range");
    static_assert(LDS <= 160 * 1024, "LDS");
};

// B operands of one row tile for one block
struct SlabB {
    uint4 b1[4], b2[4];
    half4v mh;  // mins of the lane's groups (Q4_K / Q5_K)
    float d, dmin;
};

// the 4 mins (as fp16) a lane supplies for groups 4c .. 4c + 3: units 2c, 2c,
// 2c + 1, 2c + 1 (mw: the 8 mins four to a dword)
__device__ inline half4v mins_f16(const uint32_t (&mw)[2], int c) {
    // (a mask select: an index would put mw in scratch memory)
    const uint32_t sel = 0u - uint32_t((c >> 1) & 1);
    const uint32_t w = (mw[0] & ~sel) | (mw[1] & sel);
    const int b0 = 2 * (c & 1);
    const half2v bias = {(_Float16)1024.0f, (_Float16)1024.0f};
    // 0x6400 | m is the fp16 value 1024 + m (m < 64): subtract 1024, exactly
    const half2v lo = __builtin_bit_cast(half2v, __builtin_bit_cast(uint32_t, byte_pair(w, b0)) | 0x64006400u) - bias;
    const half2v hi =
        __builtin_bit_cast(half2v, __builtin_bit_cast(uint32_t, byte_pair(w, b0 + 1)) | 0x64006400u) - bias;
    return half4v{lo.x, lo.y, hi.x, hi.y};
}

template <class F>
__device__ inline void slab_unpack(const uint8_t *blk, int c, SlabB &o) {
    if constexpr (std::is_same_v<F, MQ6KS>) {
        const MQ6KS::W w = MQ6KS::load_lds(blk, c);
        SplitB sb;
        split_b(w, c, sb);
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            o.b1[h] = sb.b1[h];
            o.b2[h] = sb.b2[h];
        }
        o.d = fp16_bits_to_f32(w.d);
        o.dmin = 0.0f;
    } else {  // Q4_K / Q5_K folded
        const typename F::W w = F::load_lds(blk, c);
        uint32_t scp[2], mp[2];
        scales_k4_packed(w.h.y, w.h.z, w.h.w, scp, mp);
        SplitB sb;
        split_b(w, scp, mp, sb);
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            o.b1[h] = sb.b1[h];
            o.b2[h] = sb.b2[h];
        }
        o.mh = mins_f16(mp, c);
        o.d = fp16_bits_to_f32(w.h.x & 0xFFFFu);
        o.dmin = fp16_bits_to_f32(w.h.x >> 16);
    }
}

template <class C, class F>
__global__ __launch_bounds__(64 * C::NW, C::WPS) void slab_kernel(MatGroup grp, typename ActOf<F>::T x, int ntg) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int RW = C::RW, TW = C::TW;
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nl = lane & 15, cl = lane >> 4;
    const int pt = wid % C::PT, pr = wid / C::PT;

    // workgroup -> (row slab, token group): consecutive slots of one XCD
    // take the token groups of one slab
    const int G = grp.wg0[grp.n] * ntg;
    const int per = (G + 7) / 8;
    const int lin = int(blockIdx.x % 8u) * per + int(blockIdx.x / 8u);
    if (lin >= G) return;
    const int rg = lin / ntg, tg = lin - rg * ntg;
    int bx;
    const MatArgs a = grp.t[group_task(grp, rg, bx)];
    if (scan_stopped(a.scan)) return;
    const int n0 = bx * C::R, m0 = tg * C::T;
    const int K = a.K;
    const int nsteps = K / 256;
    const int nbk = K / 256;  // blocks per activation row

    // descriptors: the slab's rows (from the 16-B boundary at or below the
    // first), the codes, sums and scales of the tokens
    const uintptr_t wstart = reinterpret_cast<uintptr_t>(a.w) + size_t(n0) * a.row_bytes;
    const uint32_t bl = uint32_t(wstart & 15);
    const int rows_valid = min(C::R, a.N - n0);
    const v4i32 rw = buf_rsrc(reinterpret_cast<const void *>(wstart - bl),
                              (bl + uint32_t(rows_valid) * uint32_t(a.row_bytes) + 15u) & ~15u);
    const uint32_t mpad = uint32_t((a.M + 15) & ~15);
    const v4i32 ra = buf_rsrc(x.qt, mpad * uint32_t(K));
    v4i32 rb = ra;
    if constexpr (C::MIN) rb = buf_rsrc(x.bh, mpad * uint32_t(K / 8));
    const v4i32 rd = buf_rsrc(x.d, uint32_t(a.M) * uint32_t(nbk) * 4u);
    const uint32_t lds0 = lds_addr(lds);

    // per-lane source offsets of step 0 (lanes past a region's data get
    // kFar); the step's own offset is a uniform soffset, and a step past the
    // end adds the region's whole range, so it reads zeros
    uint32_t wo[C::NWW], wp[C::NWW], ao[C::NAW], bo[C::NBW > 0 ? C::NBW : 1], dof[C::NDW];
#pragma unroll
    for (int s = 0; s < C::NWW; ++s) {  // unit pc of row `row`: 16 B from the 16-B boundary at or below its step bytes
        const int p = (s * C::NW + wid) * 64 + lane;
        const int row = p / C::WCR, pc = p - row * C::WCR;
        wo[s] = row < C::R ? uint32_t(row) * uint32_t(a.row_bytes) + bl : kFar;
        wp[s] = 16u * uint32_t(pc);
        if constexpr (C::ALIGNED) wo[s] = row < C::R ? wo[s] + wp[s] : kFar;  // bl = 0: every step starts 16-B aligned
    }
#pragma unroll
    for (int s = 0; s < C::NAW; ++s) {
        const int i = s * C::NW + wid, tt = i >> 2, h = i & 3;  // token tile, 1-KB quarter
        const uint32_t tile = uint32_t(m0 / 16 + tt);
        ao[s] = (tile * uint32_t(nbk)) * 4096u + 1024u * uint32_t(h) + 16u * uint32_t(lane);
    }
#pragma unroll
    for (int s = 0; s < C::NBW; ++s) {
        const int p = (s * C::NW + wid) * 64 + lane, tt = p >> 5, q = p & 31;
        bo[s] = tt < C::T / 16 ? (uint32_t(m0 / 16 + tt) * uint32_t(nbk)) * 512u + 16u * uint32_t(q) : kFar;
    }
#pragma unroll
    for (int s = 0; s < C::NDW; ++s) {
        const int p = (s * C::NW + wid) * 64 + lane;
        dof[s] = p < C::T ? uint32_t(m0 + p) * uint32_t(nbk) * 4u : kFar;
    }
    const uint32_t wrange = uint32_t(rw.z), arange = uint32_t(ra.z), brange = uint32_t(rb.z), drange = uint32_t(rd.z);
    // the transfers of step st into stage sg (every wave issues L per step)
    auto issue = [&](int st, int sg) __attribute__((always_inline)) {
        const bool live = st < nsteps;
        const uint32_t base = lds0 + uint32_t(sg * C::STAGE), dump = lds0 + uint32_t(C::OFF_DUMP);
#pragma unroll
        for (int s = 0; s < C::NWW; ++s) {
            const int i = s * C::NW + wid;
            const uint32_t dst = i < C::NWI ? base + uint32_t(i * 1024) : dump;
            if constexpr (C::ALIGNED) {
                dma16s(rw, wo[s], live ? uint32_t(st) * uint32_t(C::SB) : wrange, dst);
            } else {
                const uint32_t v = ((wo[s] + uint32_t(st) * uint32_t(C::SB)) & ~15u) + wp[s];
                dma16s(rw, wo[s] != kFar ? v : kFar, live ? 0u : wrange, dst);
            }
        }
#pragma unroll
        for (int s = 0; s < C::NAW; ++s)
            dma16s(ra, ao[s], live ? uint32_t(st) * 4096u : arange,
                   base + uint32_t(C::OFF_A + (s * C::NW + wid) * 1024));
#pragma unroll
        for (int s = 0; s < C::NBW; ++s) {
            const int i = s * C::NW + wid;
            dma16s(rb, bo[s], live ? uint32_t(st) * 512u : brange, i < C::NBI ? base + uint32_t(C::OFF_B + i * 1024) : dump);
        }
#pragma unroll
        for (int s = 0; s < C::NDW; ++s) {
            const int i = s * C::NW + wid;
            dma4s(rd, dof[s], live ? uint32_t(st) * 4u : drange, i < C::NDI ? base + uint32_t(C::OFF_D + i * 256) : dump);
        }
    };

    float acc[RW][TW][4];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int t = 0; t < TW; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[r][t][q] = 0.0f;

#pragma unroll
    for (int p = 0; p + 1 < C::PD; ++p) issue(p, p);
    for (int st = 0; st < nsteps; ++st) {
        const int sg = st % C::PD;
        wait_vmcnt<(C::PD - 2) * C::L>();  // this wave's transfers of step st have landed
        __builtin_amdgcn_s_barrier();       // every wave's have; stage (st - 1) is free
        __builtin_amdgcn_sched_barrier(0);
        issue(st + C::PD - 1, (st + C::PD - 1) % C::PD);
        const uint8_t *sbase = lds + sg * C::STAGE;
        const uint8_t *sa = sbase + C::OFF_A;
        const float *sd = reinterpret_cast<const float *>(sbase + C::OFF_D);
        SlabB B[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            const int rl = (pr * RW + r) * 16 + nl;  // lane's row in the slab
            const uint32_t mis = C::ALIGNED ? 0u : (uint32_t(rl) * uint32_t(a.row_bytes) + bl + uint32_t(st) * uint32_t(C::SB)) & 15u;
            slab_unpack<F>(sbase + rl * (C::WCR * 16) + mis, cl, B[r]);
        }
        {
            // tile u: codes and sums loaded two tiles ahead, dx one ahead; the
            // MFMAs of tile t + 1 are issued before tile t's fp32 update, so
            // the matrix core runs while the update's VALU work issues
            uint4 av[2][4];
            half4v bh[2];
            float4 dx[2];
            int4v D1[2][RW], D2[2][RW];
            f32x4v Mb[2][RW];
            auto load_a = [&](int t, int buf) __attribute__((always_inline)) {
                const int tt = pt * TW + t;
#pragma unroll
                for (int h = 0; h < 4; ++h) av[buf][h] = ld16(sa + (tt * 4 + h) * 1024 + 16 * lane);
                if constexpr (C::MIN) bh[buf] = __builtin_bit_cast(half4v, ld8(sbase + C::OFF_B + tt * 512 + 8 * lane));
            };
            auto load_d = [&](int t, int buf) __attribute__((always_inline)) {
                dx[buf] = *reinterpret_cast<const float4 *>(sd + (pt * TW + t) * 16 + 4 * cl);
            };
            auto mm = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
                for (int r = 0; r < RW; ++r) {
                    int4v d1 = {0, 0, 0, 0}, d2 = {0, 0, 0, 0};
#pragma unroll
                    for (int h = 0; h < 4; ++h) {
                        d1 = mfma16x16x64(av[buf][h], B[r].b1[h], d1);
                        d2 = mfma16x16x64(av[buf][h], B[r].b2[h], d2);
                    }
                    D1[buf][r] = d1;
                    D2[buf][r] = d2;
                    f32x4v m = {0.0f, 0.0f, 0.0f, 0.0f};
                    if constexpr (C::MIN) m = __builtin_amdgcn_mfma_f32_16x16x16f16(bh[buf], B[r].mh, m, 0, 0, 0);
                    Mb[buf][r] = m;
                }
            };
            auto epi = [&](int t, int buf) __attribute__((always_inline)) {
                const float dxq[4] = {dx[buf].x, dx[buf].y, dx[buf].z, dx[buf].w};
#pragma unroll
                for (int r = 0; r < RW; ++r)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int S = (D1[buf][r][q] << F::kShift) + D2[buf][r][q];
                        if constexpr (C::MIN)
                            acc[r][t][q] += dxq[q] * (B[r].d * (float)S - B[r].dmin * Mb[buf][r][q]);  // E:11026 / E:11063
                        else
                            acc[r][t][q] += (B[r].d * dxq[q]) * (float)S;  // E:11101
                    }
            };
            load_a(0, 0);
            load_d(0, 0);
            if (TW > 1) load_a(1, 1);
            mm(0);
#pragma unroll
            for (int t = 0; t < TW; ++t) {
                if (t + 1 < TW) {
                    mm((t + 1) & 1);
                    load_d(t + 1, (t + 1) & 1);
                }
                if (t + 2 < TW) load_a(t + 2, t & 1);
                epi(t, t & 1);
                if (t + 1 < TW) {
#pragma unroll
                    for (int i = 0; i < (C::MIN ? 9 : 8) * RW; ++i) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA of tile t + 1
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read of tile t + 2
                        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // three VALU of tile t's update
                    }
                }
            }
        }
    }
    wait_vmcnt<0>();  // the tail's transfers (zeros into a free stage) land before the workgroup ends

#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const int n = n0 + (pr * RW + r) * 16 + nl;
        if (n >= a.N) continue;
#pragma unroll
        for (int t = 0; t < TW; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int tok = m0 + (pt * TW + t) * 16 + 4 * cl + q;
                if (tok >= a.M) continue;
                float v = acc[r][t][q];
                if (a.res) v = v + a.res[size_t(tok) * a.ldr + n];
                a.y[size_t(tok) * a.ldy + n] = v;
            }
    }
}

// ------------------------------------------------------------ decoded slabs
// Prefill GEMM with each weight block decoded once per workgroup into int8
// MFMA tiles in LDS. The slab's RT row tiles are staged packed (buffer -> LDS
// transfers, PD stages, two blocks ahead); after block j's MFMAs the waves
// decode block j + 1 into the other of two decoded buffers (per row tile:
// the two folded int8 planes of each 64-value chunk in MFMA B-operand order,
// the mins as fp16, d and dmin per row), each wave HC of the slab's 4 RT
// chunks. Every wave owns TW token tiles: their codes and sums are loaded
// from the activation buffer into registers (the codes of block j + 1 once
// block j's last MFMAs are issued), their block scales staged once per
// workgroup in LDS; it reads the decoded B operands of all RT row tiles. A
// block's decoding is thus paid once per 16 NW TW tokens, where the slab
// kernel pays it once per wave's 16 TW. One barrier per block. Per 16 x 16
// tile and block the integer sums and the fp32 update are the slab kernel's.
// With KS > 1 (few tokens, long K) the waves form KS groups that walk the
// blocks g, g + KS, ... side by side, each with its own stages and decoded
// buffers; each step every group writes its fp32 terms to LDS and group 0
// adds the step's KS terms in block order behind the barrier, so every sum
// is still the reference's, in its order.
// Step s waits for its own wave's loads, then the barrier. Plain form: every
// load issued before (the weights of step s + 1 and the codes of step s, both
// issued one step earlier), so a step lasts at least one memory round trip.
// DEEP form: the weights are issued three steps ahead and the codes and sums
// two (a second register set of codes), every wave issues the same LPS loads
// per step (past the last block they read zeros), and step s waits until only
// the previous step's LPS are outstanding: two steps per round trip.

template <class F, int RT_, int NW_, int TW_, int WPS_ = 2, int PD_ = 3, int KS_ = 1, bool DEEP_ = false>
struct DsCfg {
    static constexpr int RT = RT_, NW = NW_, TW = TW_, PD = PD_, WPS = WPS_;
    static constexpr bool DEEP = DEEP_;
    // KS > 1: the waves form KS groups; group g takes blocks g, g + KS, ...
    // (its own stages and decoded buffers), and group 0 adds the groups'
    // fp32 terms of each KS blocks in block order (through LDS)
    static constexpr int KS = KS_, NWG = NW_ / KS_;
    static_assert(NWG * KS == NW, "KS groups of waves");
    static constexpr bool MIN = F::kMin;
    static constexpr int R = 16 * RT, T = 16 * NWG * TW;
    static constexpr int SB = F::BB;
    static constexpr bool ALIGNED = SB % 16 == 0;
    static constexpr int WCR = (ALIGNED ? SB / 16 : (SB + 30) / 16) | 1;  // 16-B units per staged row, odd
    static constexpr int NWI = (R * WCR + 63) / 64;                       // weight transfers (1 KB) per block
    static constexpr int NWW = (NWI + NWG - 1) / NWG;                     // of them per wave of a group
    static constexpr int PS = NWI * 1024;                                 // one packed stage
    static constexpr int LPS = NWW + 4 * TW + (F::kMin ? TW : 0);         // loads per wave and step (DEEP)
    static_assert(!DEEP || LPS <= 63, "vmcnt range");
    static constexpr int HC = 4 * RT / NWG;                               // chunks a wave decodes per block
    static_assert(HC >= 1 && 4 * RT % NWG == 0, "chunks per wave");
    // decoded row tile: planes [chunk][high | low] (1 KB each), mins (512 B), (d, dmin) per row
    static constexpr int OB_M = 8192, OB_D = MIN ? 8704 : 8192, RTB = OB_D + 128;
    static constexpr int DB = RT * RTB;  // a group's decoded buffer (two per group, as static arrays)
    // dynamic LDS: packed stages [group][PD] | a scratch KB | the groups'
    // terms [2][KS][NWG][RT][TW][64 lanes] float4 (group 0's are written and
    // never read: a store without a branch on the group between the MFMAs and
    // their epilogue) | the tokens' block scales [T][nbk]
    static constexpr int OFF_DUMP = KS * PD * PS, OFF_TM = OFF_DUMP + 1024;
    static constexpr int TMB = KS > 1 ? KS * NWG * RT * TW * 1024 : 0;  // one terms buffer
    static constexpr int OFF_DX = OFF_TM + 2 * TMB;
    static constexpr int lds_bytes(int nbk) { return OFF_DX + (T * nbk * 4 + 1023) / 1024 * 1024; }
    static_assert(PD >= 3, "a block is staged two steps ahead of its use");
};

// B operands of chunk h (0..3) of a block for lane k-slice c: the high and low
// folded planes (the layout of split_b)
template <class F>
__device__ inline void ds_fold(const uint8_t *blk, int c, int h, uint4 &o1, uint4 &o2) {
    if constexpr (std::is_same_v<F, MQ6KS>) {
        const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(blk) & 3);
        const uint32_t *q = reinterpret_cast<const uint32_t *>(blk - sh);
        auto rd8 = [&](int dw) __attribute__((always_inline)) {
            const uint32_t w0 = q[dw], w1 = q[dw + 1], w2 = q[dw + 2];
            return make_uint2(funnel(w1, w0, sh), funnel(w2, w1, sh));
        };
        const int hf = h >> 1, ip = h & 1;
        const uint2 wa = rd8(16 * hf + 2 * c), wb = rd8(16 * hf + 8 + 2 * c), wq = rd8(32 + 8 * hf + 2 * c);
        const uint2 sw = rd8(48 + 2 * hf);
        const int cb = 8 * (c >> 1);
        uint32_t hi[4], lo[4];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int i = 2 * ip + k;
            const int sc = __builtin_amdgcn_sbfe(int((i & 2) ? sw.y : sw.x), 16 * (i & 1) + cb, 8);
            const u16x2 sp = __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(0u, uint32_t(sc), 0x01000100u));
            const u16x2 cp = sp * u16x2{0xFFE0u, 0xFFE0u} + u16x2{128u, 128u};  // 128 - 32 sc
            const uint2 src = k ? wb : wa;
            const int hs = 4 * ip + 2 * k;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const uint32_t v = e ? src.y : src.x, qv = e ? wq.y : wq.x;
                const uint32_t q6 = ((v >> (4 * ip)) & 0x0F0F0F0Fu) | (((qv >> hs) & 0x03030303u) << 4);
                fold4(q6, sp, cp, lo[2 * k + e], hi[2 * k + e]);
            }
        }
        o1 = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        o2 = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    } else {
        const uint4 hd = ld16(blk);
        uint32_t scp[2], mp[2];
        scales_k4_packed(hd.y, hd.z, hd.w, scp, mp);
        const uint32_t scw = (h >> 1) ? scp[1] : scp[0];  // sub-blocks 2h, 2h + 1: bytes 2 (h & 1), + 1
        const int b0 = 2 * (h & 1);
        if constexpr (std::is_same_v<F, MQ4KS>) {
            const uint2 q = ld8(blk + 16 + 32 * h + 8 * c);
            const uint32_t shw = (scw >> 3) & 0x07070707u, slw = scw & 0x07070707u;
            const uint32_t lo0 = q.x & 0x0F0F0F0Fu, lo1 = q.y & 0x0F0F0F0Fu;
            const uint32_t hi0 = (q.x >> 4) & 0x0F0F0F0Fu, hi1 = (q.y >> 4) & 0x0F0F0F0Fu;
            const u16x2 sh0 = byte_pair(shw, b0), sl0 = byte_pair(slw, b0);
            const u16x2 sh1 = byte_pair(shw, b0 + 1), sl1 = byte_pair(slw, b0 + 1);
            o1 = make_uint4(bytes_times(lo0, sh0), bytes_times(lo1, sh0), bytes_times(hi0, sh1), bytes_times(hi1, sh1));
            o2 = make_uint4(bytes_times(lo0, sl0), bytes_times(lo1, sl0), bytes_times(hi0, sl1), bytes_times(hi1, sl1));
        } else {  // Q5_K
            const uint2 qh = ld8(blk + 16 + 8 * c);
            const uint2 q = ld8(blk + 48 + 32 * h + 8 * c);
            uint32_t hi[4], lo[4];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int u = 2 * h + k;
                const u16x2 sp = byte_pair(scw, b0 + k);
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const uint32_t v = e ? q.y : q.x, qv = e ? qh.y : qh.x;
                    const uint32_t q5 = ((v >> (4 * k)) & 0x0F0F0F0Fu) | (((qv >> u) & 0x01010101u) << 4);
                    fold4(q5, sp, u16x2{128u, 128u}, lo[2 * k + e], hi[2 * k + e]);
                }
            }
            o1 = make_uint4(hi[0], hi[1], hi[2], hi[3]);
            o2 = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        }
    }
}

// the row's d, dmin and the lane's mins (fp16, as mins_f16) of a block
template <class F>
__device__ inline void ds_row(const uint8_t *blk, int c, half4v &mh, float &d, float &dmin) {
    if constexpr (std::is_same_v<F, MQ6KS>) {
        const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(blk) & 3);
        const uint32_t *q = reinterpret_cast<const uint32_t *>(blk - sh);
        d = fp16_bits_to_f32((q[52] >> (8 * sh)) & 0xFFFFu);
        dmin = 0.0f;
        mh = half4v{0, 0, 0, 0};
    } else {
        const uint4 hd = ld16(blk);
        uint32_t scp[2], mp[2];
        scales_k4_packed(hd.y, hd.z, hd.w, scp, mp);
        mh = mins_f16(mp, c);
        d = fp16_bits_to_f32(hd.x & 0xFFFFu);
        dmin = fp16_bits_to_f32(hd.x >> 16);
    }
}

template <class C, class F>
__global__ __launch_bounds__(64 * C::NW, C::WPS) void dslab_kernel(MatGroup grp, Q8KView x, int ntg) {
    extern __shared__ __align__(16) uint8_t lds[];
    // the decoded buffers as two static arrays: the compiler then knows that
    // a block's decoding (into one) and the previous block's reads (of the
    // other) are independent and interleaves them
    __shared__ __align__(16) uint8_t dbuf0[C::KS * C::DB], dbuf1[C::KS * C::DB];
    constexpr int RT = C::RT, TW = C::TW, KS = C::KS;
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = wid / C::NWG, lw = wid - g * C::NWG;  // K group, wave in the group
    const int nl = lane & 15, cl = lane >> 4;

    // workgroup -> (row slab, token group): consecutive slots of one XCD
    // take the token groups of one slab
    const int G = grp.wg0[grp.n] * ntg;
    const int per = (G + 7) / 8;
    const int lin = int(blockIdx.x % 8u) * per + int(blockIdx.x / 8u);
    if (lin >= G) return;
    const int rg = lin / ntg, tg = lin - rg * ntg;
    int bx;
    const MatArgs a = grp.t[group_task(grp, rg, bx)];
    if (scan_stopped(a.scan)) return;
    const int n0 = bx * C::R, m0 = tg * C::T;
    const int K = a.K;
    const int nbk = K / 256;
    const int nsteps = (nbk + KS - 1) / KS;  // group g's block at step s: s KS + g

    const uintptr_t wstart = reinterpret_cast<uintptr_t>(a.w) + size_t(n0) * a.row_bytes;
    const uint32_t bl = uint32_t(wstart & 15);
    const int rows_valid = min(C::R, a.N - n0);
    const v4i32 rw = buf_rsrc(reinterpret_cast<const void *>(wstart - bl),
                              (bl + uint32_t(rows_valid) * uint32_t(a.row_bytes) + 15u) & ~15u);
    const int ntile = (a.M + 15) / 16;
    auto rsrc = [](const void *p, uint32_t bytes) __attribute__((always_inline)) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), short(0), int(bytes), 0x00020000);
    };
    const __amdgpu_buffer_rsrc_t ra = rsrc(x.qt, uint32_t(ntile) * 16u * uint32_t(K));
    const __amdgpu_buffer_rsrc_t rb = rsrc(C::MIN ? static_cast<const void *>(x.bh) : static_cast<const void *>(x.qt),
                                           C::MIN ? uint32_t(ntile) * 16u * uint32_t(K / 8) : 0u);
    const uint32_t lds0 = lds_addr(lds);

    // weight transfers of the group's block: unit pc of staged row `row` (as
    // the slab kernel)
    uint32_t wo[C::NWW], wp[C::NWW];
#pragma unroll
    for (int s = 0; s < C::NWW; ++s) {
        const int p = (s * C::NWG + lw) * 64 + lane;
        const int row = p / C::WCR, pc = p - row * C::WCR;
        wo[s] = row < C::R ? uint32_t(row) * uint32_t(a.row_bytes) + bl : kFar;
        wp[s] = 16u * uint32_t(pc);
        if constexpr (C::ALIGNED) wo[s] = row < C::R ? wo[s] + wp[s] : kFar;
    }
    // (a block past the row reads zeros: the whole range as the uniform offset)
    const uint32_t wrange = uint32_t(rw.z);
    auto stage_of = [&](int s) __attribute__((always_inline)) { return (g * C::PD + s % C::PD) * C::PS; };
    auto issue_w = [&](int s) __attribute__((always_inline)) {
        const int j = s * KS + g;
        const bool live = j < nbk;
        const uint32_t base = lds0 + uint32_t(stage_of(s)), dump = lds0 + uint32_t(C::OFF_DUMP);
#pragma unroll
        for (int t = 0; t < C::NWW; ++t) {
            const int i = t * C::NWG + lw;
            const uint32_t dst = i < C::NWI ? base + uint32_t(i * 1024) : dump;
            if constexpr (C::ALIGNED) {
                dma16s(rw, wo[t], live ? uint32_t(j) * uint32_t(C::SB) : wrange, dst);
            } else {
                const uint32_t v = ((wo[t] + uint32_t(j) * uint32_t(C::SB)) & ~15u) + wp[t];
                dma16s(rw, wo[t] != kFar ? v : kFar, live ? 0u : wrange, dst);
            }
        }
    };

    // the wave's token tiles: codes (4 KB per tile and block), sums of 16
    // codes (512 B); tiles past the input read zeros
    uint32_t ao[TW], bo[TW];
#pragma unroll
    for (int t = 0; t < TW; ++t) {
        const int tile = m0 / 16 + lw * TW + t;
        const bool in = tile < ntile;
        ao[t] = in ? uint32_t(tile) * uint32_t(nbk) * 4096u + 16u * uint32_t(lane) : kFar;
        bo[t] = in ? uint32_t(tile) * uint32_t(nbk) * 512u + 8u * uint32_t(lane) : kFar;
    }
    // the codes of one block (two with DEEP; reloaded once the block's MFMAs
    // are issued); the sums of two
    constexpr bool DEEP = C::DEEP;
    uint4 A[DEEP ? 2 : 1][TW][4];
    half4v BH[2][TW];
    auto load_codes = [&](auto Q, int s) __attribute__((always_inline)) {
        constexpr int q = decltype(Q)::value;
        const uint32_t j = uint32_t(s * KS + g);
#pragma unroll
        for (int t = 0; t < TW; ++t)
#pragma unroll
            for (int h = 0; h < 4; ++h)
                A[q][t][h] = __builtin_bit_cast(
                    uint4, __builtin_amdgcn_raw_buffer_load_b128(ra, ao[t] + 1024u * uint32_t(h), j * 4096u, 0));
    };
    auto load_sums = [&](auto P, int s) __attribute__((always_inline)) {
        constexpr int p = decltype(P)::value;
        if constexpr (C::MIN) {
            const uint32_t j = uint32_t(s * KS + g);
#pragma unroll
            for (int t = 0; t < TW; ++t)
                BH[p][t] = __builtin_bit_cast(half4v, __builtin_amdgcn_raw_buffer_load_b64(rb, bo[t], j * 512u, 0));
        }
    };
    // the scales of the workgroup's tokens, [T][nbk] (contiguous in the
    // activation buffer; tokens past the input read zeros), staged once
    const float *sdx = reinterpret_cast<const float *>(lds + C::OFF_DX);
    {
        const v4i32 rdd = buf_rsrc(x.d, uint32_t(a.M) * uint32_t(nbk) * 4u);
        const int n16 = (C::T * nbk * 4 + 1023) / 1024;  // 1-KB transfers
        for (int i = wid; i < n16; i += C::NW)
            dma16s(rdd, uint32_t(i * 1024 + 16 * lane), uint32_t(m0) * uint32_t(nbk) * 4u,
                   lds0 + uint32_t(C::OFF_DX + i * 1024));
    }

    // decoding: wave lw of group g takes chunks [h0, h0 + HC) of row tile rt
    // of the group's block
    const int dchunk = lw * C::HC, drt = dchunk >> 2, dh0 = dchunk & 3;
    auto decode = [&](auto P, int s) __attribute__((always_inline)) {
        const int j = s * KS + g;
        const uint8_t *stage = lds + stage_of(s);
        uint8_t *db = (decltype(P)::value ? dbuf1 : dbuf0) + g * C::DB + drt * C::RTB;
        const int rl = drt * 16 + nl;
        const uint32_t mis =
            C::ALIGNED ? 0u : (uint32_t(rl) * uint32_t(a.row_bytes) + bl + uint32_t(j) * uint32_t(C::SB)) & 15u;
        const uint8_t *blk = stage + rl * (C::WCR * 16) + mis;
#pragma unroll
        for (int i = 0; i < C::HC; ++i) {
            const int h = dh0 + i;
            uint4 o1, o2;
            ds_fold<F>(blk, cl, h, o1, o2);
            *reinterpret_cast<uint4 *>(db + (2 * h) * 1024 + 16 * lane) = o1;
            *reinterpret_cast<uint4 *>(db + (2 * h + 1) * 1024 + 16 * lane) = o2;
        }
        // the row scales: by the wave holding the row tile's chunk 0; without
        // mins by every wave and lane (the same value to the same word), so
        // the decoding has no branch to schedule around
        if (!C::MIN || dh0 == 0) {
            half4v mh;
            float d, dmin;
            ds_row<F>(blk, cl, mh, d, dmin);
            if constexpr (C::MIN) *reinterpret_cast<half4v *>(db + C::OB_M + 8 * lane) = mh;
            if (!C::MIN || cl == 0) *reinterpret_cast<float2 *>(db + C::OB_D + 8 * nl) = make_float2(d, dmin);
        }
    };

    float acc[RT][TW][4];
    [[maybe_unused]] float d0[RT][TW][4];  // group 0's terms of the last step, added behind the previous step's
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int t = 0; t < TW; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[r][t][q] = d0[r][t][q] = 0.0f;
    // the terms of group gg (>= 1) of the wave's tiles in terms buffer b
    auto term_slot = [&](int b, int gg, int r, int t) __attribute__((always_inline)) {
        return reinterpret_cast<float4 *>(lds + C::OFF_TM + b * C::TMB) +
               (((gg * C::NWG + lw) * RT + r) * TW + t) * 64 + lane;
    };
    // group 0: step s's blocks in order (its own terms, then those of the
    // groups whose block is inside K), published by the barrier after them
    auto add_step = [&](int s) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < RT; ++r)
#pragma unroll
            for (int t = 0; t < TW; ++t) {
                float v[4] = {d0[r][t][0], d0[r][t][1], d0[r][t][2], d0[r][t][3]};
#pragma unroll
                for (int q = 0; q < 4; ++q) acc[r][t][q] += v[q];
                for (int gg = 1; gg < KS && s * KS + gg < nbk; ++gg) {
                    const float4 w = *term_slot(s & 1, gg, r, t);
                    acc[r][t][0] += w.x;
                    acc[r][t][1] += w.y;
                    acc[r][t][2] += w.z;
                    acc[r][t][3] += w.w;
                }
            }
    };

    // step s: the group's block j = s KS + g: A[ap] its codes, BH[P] its
    // sums, the group's decoded buffer (s & 1) its B operands (published by
    // the barrier); stage (s + 1) % PD has landed. MORE: step s + 1 exists
    // (its weights are decoded here, after this step's reads of the decoded
    // buffer; plain form: its activations are loaded here too)
    using T0c = std::integral_constant<int, 0>;
    auto step = [&](auto P, int s, auto MORE) __attribute__((always_inline)) {
        constexpr int p = decltype(P)::value;
        constexpr int ap = DEEP ? p : 0;  // the code registers of this step
        using AP = std::integral_constant<int, ap>;
        constexpr bool more = decltype(MORE)::value;
        const int j = s * KS + g;
        // plain: this wave's transfers of step s + 1 and activations of step s;
        // DEEP: all but the previous step's LPS loads (the transfers of step
        // s + 1 and the activations of step s were issued two steps ago)
        wait_vmcnt<DEEP ? C::LPS : 0>();
        lds_barrier();  // every wave's, and step s decoded; decoded buffers (s + 1) & 1 free, and the
                        // stage written next ((s + 2) % PD plain, s % PD DEEP)
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (DEEP) {
            issue_w(s + 3);  // zeros past the last block
        } else if constexpr (more) {
            issue_w(s + 2);  // zeros past the last block
            load_sums(std::integral_constant<int, p ^ 1>{}, s + 1);
        }
        if constexpr (KS > 1)
            if (g == 0 && s > 0) add_step(s - 1);
        const uint8_t *db = (p ? dbuf1 : dbuf0) + g * C::DB;
        // DEEP: a group's block past K is computed too (zeros staged, its term
        // never added: group 0's block is inside K, add_step skips the rest),
        // so no load sits behind a branch (the compiler would wait for it to
        // copy registers where the paths join)
        if (KS == 1 || DEEP || j < nbk) {
            const int jd = min(j, nbk - 1);  // (a DEEP block past K reads block nbk - 1's scales)
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                const uint8_t *dr = db + r * C::RTB;
                uint4 bb[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) bb[i] = ld16(dr + i * 1024 + 16 * lane);
                const float2 dd = *reinterpret_cast<const float2 *>(dr + C::OB_D + 8 * nl);
                half4v mh;
                if constexpr (C::MIN) mh = *reinterpret_cast<const half4v *>(dr + C::OB_M + 8 * lane);
                int4v D1[TW], D2[TW];
#pragma unroll
                for (int t = 0; t < TW; ++t) {
                    D1[t] = int4v{0, 0, 0, 0};
                    D2[t] = int4v{0, 0, 0, 0};
                }
#pragma unroll
                for (int h = 0; h < 4; ++h)
#pragma unroll
                    for (int t = 0; t < TW; ++t) {
                        D1[t] = mfma16x16x64(A[ap][t][h], bb[2 * h], D1[t]);
                        D2[t] = mfma16x16x64(A[ap][t][h], bb[2 * h + 1], D2[t]);
                    }
                // once the block's last MFMAs have their operands: the next
                // codes, then the next block's decoding (independent of the
                // MFMAs in flight, ahead of the epilogue that waits for them)
                if (r == RT - 1) {
                    if constexpr (DEEP) load_codes(AP{}, s + 2);
                    else if constexpr (more) load_codes(T0c{}, s + 1);
                    if constexpr (more) decode(std::integral_constant<int, p ^ 1>{}, s + 1);
                }
                f32x4v Mb[TW];
                if constexpr (C::MIN) {
#pragma unroll
                    for (int t = 0; t < TW; ++t)
                        Mb[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(BH[p][t], mh, f32x4v{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0,
                                                                      0);
                    if constexpr (DEEP)
                        if (r == RT - 1) load_sums(P, s + 2);
                }
#pragma unroll
                for (int t = 0; t < TW; ++t) {
                    float v[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int S = (D1[t][q] << F::kShift) + D2[t][q];
                        const float dx = sdx[((lw * TW + t) * 16 + 4 * cl + q) * nbk + jd];
                        if constexpr (C::MIN)
                            v[q] = dx * (dd.x * (float)S - dd.y * Mb[t][q]);  // E:11026 / E:11063
                        else
                            v[q] = (dd.x * dx) * (float)S;  // E:11101
                    }
                    if constexpr (KS == 1) {
#pragma unroll
                        for (int q = 0; q < 4; ++q) acc[r][t][q] += v[q];
                    } else {
#pragma unroll
                        for (int q = 0; q < 4; ++q) d0[r][t][q] = v[q];
                        *term_slot(s & 1, g, r, t) = make_float4(v[0], v[1], v[2], v[3]);
                    }
                }
            }
        } else if constexpr (more) {
            load_codes(T0c{}, s + 1);
            decode(std::integral_constant<int, p ^ 1>{}, s + 1);
        }
    };

    // prologue: the groups' first two (DEEP: three) blocks staged, their
    // first (two) blocks' activations, the first block decoded
    if constexpr (DEEP) {
        issue_w(0);
        issue_w(1);
        load_codes(T0c{}, 0);
        load_sums(T0c{}, 0);
        load_codes(std::integral_constant<int, 1>{}, 1);
        load_sums(std::integral_constant<int, 1>{}, 1);
        issue_w(2);
        wait_vmcnt<C::NWW>();  // all but the third block's transfers
    } else {
        issue_w(0);
        if (nsteps > 1) issue_w(1);
        load_codes(T0c{}, 0);
        load_sums(T0c{}, 0);
        wait_vmcnt<0>();
    }
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
    decode(std::integral_constant<int, 0>{}, 0);
    using T0 = std::integral_constant<int, 0>;
    using T1 = std::integral_constant<int, 1>;
    using Yes = std::true_type;
    using No = std::false_type;
    int s = 0;
    for (; s + 2 < nsteps; s += 2) {
        step(T0{}, s, Yes{});
        step(T1{}, s + 1, Yes{});
    }
    if (s + 1 < nsteps) {
        step(T0{}, s, Yes{});
        step(T1{}, s + 1, No{});
    } else {
        step(T0{}, s, No{});
    }
    wait_vmcnt<0>();
    if constexpr (KS > 1) {  // the last step's terms
        lds_barrier();
        if (g != 0) return;
        add_step(nsteps - 1);
    }

#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const int n = n0 + r * 16 + nl;
        if (n >= a.N) continue;
#pragma unroll
        for (int t = 0; t < TW; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int tok = m0 + (lw * TW + t) * 16 + 4 * cl + q;
                if (tok >= a.M) continue;
                float v = acc[r][t][q];
                if (a.res) v = v + a.res[size_t(tok) * a.ldr + n];
                a.y[size_t(tok) * a.ldy + n] = v;
            }
    }
}

template <class C, class F>
static hipError_t launch_dslab_t(const MatArgs *tasks, int n, const Q8KView &x, hipStream_t s) {
    MatGroup g{};
    g.n = n;
    g.wg0[0] = 0;
    for (int i = 0; i < n; ++i) {
        g.t[i] = tasks[i];
        g.wg0[i + 1] = g.wg0[i] + (tasks[i].N + C::R - 1) / C::R;
    }
    const int ntg = (tasks[0].M + C::T - 1) / C::T;
    const int G = g.wg0[n] * ntg;
    const unsigned grid = unsigned((G + 7) / 8 * 8);
    const int lds = C::lds_bytes(tasks[0].K / 256);
    if (lds + 2 * C::KS * C::DB > 160 * 1024) return hipErrorNotSupported;
    hipLaunchKernelGGL((dslab_kernel<C, F>), dim3(grid), dim3(64 * C::NW), size_t(lds), s, g, x, ntg);
    return hipGetLastError();
}

template <class C, class F>
static hipError_t launch_slab_t(const MatArgs *tasks, int n, const typename ActOf<F>::T &x, hipStream_t s) {
    MatGroup g{};
    g.n = n;
    g.wg0[0] = 0;
    for (int i = 0; i < n; ++i) {
        g.t[i] = tasks[i];
        g.wg0[i + 1] = g.wg0[i] + (tasks[i].N + C::R - 1) / C::R;
    }
    const int ntg = (tasks[0].M + C::T - 1) / C::T;
    const int G = g.wg0[n] * ntg;
    const unsigned grid = unsigned((G + 7) / 8 * 8);
    hipLaunchKernelGGL((slab_kernel<C, F>), dim3(grid), dim3(64 * C::NW), size_t(C::LDS), s, g, x, ntg);
    return hipGetLastError();
}

int mfma_cu_count();

// hipErrorNotSupported (nothing launched) where the slab kernels do not
// apply: K not a multiple of 256, operand sections missing, rows of an
// aligned format not 16-B aligned, offsets past the 32-bit buffer range, 64
// tokens or fewer other than Q6_K, or a decoded slab's LDS over the CU's.
template <class F>
hipError_t launch_slab(const MatArgs *tasks, int n, const typename ActOf<F>::T &x, hipStream_t s) {
    const MatArgs &a = tasks[0];
    if (a.K % 256 || !x.qt) return hipErrorNotSupported;
    if constexpr (F::kMin)
        if (!x.bh) return hipErrorNotSupported;
    if (size_t((a.M + 15) & ~15) * size_t(a.K) >= (size_t(1) << 31)) return hipErrorNotSupported;
    constexpr bool aligned = F::BB % 16 == 0;
    for (int i = 0; i < n; ++i) {
        if (aligned && ((reinterpret_cast<uintptr_t>(tasks[i].w) | tasks[i].row_bytes) & 15)) return hipErrorNotSupported;
        if (size_t(tasks[i].N) * tasks[i].row_bytes + 16 >= (size_t(1) << 31)) return hipErrorNotSupported;
    }
    // Packed slabs (the shape is chosen at the end): 128 rows x 64 tokens in
    // 8 waves, two per CU (2 x 74 KB of LDS, <= 128 VGPRs), so four waves per
    // SIMD and the 64 tokens' codes staged once per 128 rows (gate + up 2 x
    // 9728 x 2560 at M = 512: 87.5 -> 79.1 us); 64 x 64 (two per CU); 64 x 32
    // (three or four per CU: O 2560 x 4096 at M = 512: 28.5 -> 23.9 us).
    // Measured slower at M = 512: 128 x 128 in 8 waves, 128 x 32 in 8 waves,
    // 32 x 128, 32 x 64, 64 x 16, 32 x 32, three stages, and two row tiles
    // per wave.
    // Q6_K at 33..64 tokens: decoded slabs of 16 rows x 64 tokens in 16
    // waves, four K groups of four, steps two deep (down 2560 x 9728 at M =
    // 48 / 64: 20.1 / 20.8 us; one deep 21.9 / 22.2; 23 / 27.1 for the 16 x 16
    // K-split tiles, which decode each block once per 16 tokens). At 17..32
    // tokens, where the row tiles are no more than the CUs, 16 x 32 in 8 waves
    // (M = 24 / 32: 17.3 / 17.3 us against 18.7 / 18.6 on the K-split tiles).
    // At 9..16 tokens (16.9 against 13.2 us) slower than the small-M kernels.
    // Q4_K / Q5_K at 33..64 tokens over K >= 8192 where the 16 x 16 K-split
    // tiles would take more than two per CU (Q4_K 4096 x 9728 at M = 48 / 64:
    // 21.6 / 26.2 -> 18.3 / 19.1 us, 2560 x 9728 at M = 64: 21.1 -> 18.9);
    // over K = 4096, or within two per CU, the tiles stay (2560 x 9728 at
    // M = 48: 15.5 against 18.0 us decoded).
    if (a.M <= 64) {
        if constexpr (!std::is_same_v<F, MQ6KS>) {
            int tiles = 0;
            for (int i = 0; i < n; ++i) tiles += (tasks[i].N + 15) / 16;
            const int cus = mfma_cu_count();
            if (a.M > 32 && a.K >= 8192 && tiles <= cus && tiles * ((a.M + 15) / 16) > 2 * cus)
                return launch_dslab_t<DsCfg<F, 1, 16, 1, 4, 3, 4, true>, F>(tasks, n, x, s);
        }
        if constexpr (std::is_same_v<F, MQ6KS>) {
            if (a.M > 32) return launch_dslab_t<DsCfg<F, 1, 16, 1, 4, 3, 4, true>, F>(tasks, n, x, s);
            int tiles = 0;
            for (int i = 0; i < n; ++i) tiles += (tasks[i].N + 15) / 16;
            if (a.M > 16 && tiles <= mfma_cu_count())
                return launch_dslab_t<DsCfg<F, 1, 8, 1, 4, 3, 4, true>, F>(tasks, n, x, s);
        }
        return hipErrorNotSupported;
    }
    // Q6_K / Q5_K from 128 tokens: decoded slabs (their decoding is costly
    // next to the epilogue). Measured at M = 128 / 200 / 300 / 512 / 1024:
    // down 2560 x 9728 (16 rows x 128 tokens) 34.4 / 42.6 / 43.5 / 58.4 /
    // 103.8 us against 39.0 / 56.6 / 57.5 / 77.8 / 126.3 (slab kernel); QKV
    // 6144 x 2560 (32 x 128) 16.8 / 22.5 / 33.1 / 33.9 / 59.0 against 18.7 /
    // 24.0 / 31.2 / 37.2 / 63.1. Q4_K stays on the slab kernel (gate + up and
    // O at M = 512: 86.5 and 29.0 us against 78.9 and 28.0): its epilogue
    // outweighs its decoding, and the slab kernel fits more waves per SIMD.
    // Q6_K from 65 tokens (the tokens padded to 128): faster than the packed
    // slabs at every height measured (down 2560 x 9728 at M = 65..127 38.6 ->
    // 33.1 us; 1024 x 9728 38.6 -> 32.7, 1024 x 2560 12.9 -> 11.6, 4096 x
    // 2560 13.0 -> 11.9 at M = 65..512). Q5_K where its workgroups number at
    // least 5/8 of the CUs (QKV 6144 x 2560 at M = 65..127 17.4 -> 16.1 us;
    // 4096 x 2560 at M = 128 12.8 against 16.2, 1024 x 2560 12.3 against 15.8
    // on the packed slabs: there they stay).
    if constexpr (std::is_same_v<F, MQ6KS> || std::is_same_v<F, MQ5KS>) {
        int wgs = 0;
        for (int i = 0; i < n; ++i) wgs += (tasks[i].N + 31) / 32;
        if (std::is_same_v<F, MQ6KS> || 8 * wgs * ((a.M + 127) / 128) >= 5 * mfma_cu_count()) {
            hipError_t e = hipErrorNotSupported;
            if constexpr (std::is_same_v<F, MQ6KS>) e = launch_dslab_t<DsCfg<F, 1, 4, 2>, F>(tasks, n, x, s);
            if constexpr (std::is_same_v<F, MQ5KS>) e = launch_dslab_t<DsCfg<F, 2, 4, 2>, F>(tasks, n, x, s);
            if (e != hipErrorNotSupported) return e;
        }
    }
    int slabs = 0, slabs128 = 0;
    for (int i = 0; i < n; ++i) {
        slabs += (tasks[i].N + 63) / 64;
        slabs128 += (tasks[i].N + 127) / 128;
    }
    const int tg64 = (a.M + 63) / 64, cus = mfma_cu_count();
    const int w128 = slabs128 * tg64, w64 = slabs * tg64;  // workgroups of the 128 x 64 / 64 x 64 shapes
    // 128 x 64 in 8 waves where those workgroups number at least 1.5 per CU;
    // 64 x 64 where they make one round of two per CU (1.75..2 per CU); else
    // 64 x 32. Measured (Q4_K, M = 65..512, K = 2560, kernel alone): 19456
    // rows at M = 65 / 128 / 384 32.5 / 33.5 / 72.5 -> 23.0 / 30.0 / 59.8 us,
    // 9728 rows at M = 256 33.2 -> 28.0, 6144 rows at M = 384 32.2 -> 27.0;
    // M = 512 of gate + up and O unchanged (128 x 64 and 64 x 32).
    //                                                         RW TW PR PD NW WPS
    if (2 * w128 >= 3 * cus) return launch_slab_t<SlabCfg<F, 1, 4, 8, 2, 8, 4>, F>(tasks, n, x, s);
    if (4 * w64 >= 7 * cus && w64 <= 2 * cus) return launch_slab_t<SlabCfg<F, 1, 4, 4, 2>, F>(tasks, n, x, s);
    return launch_slab_t<SlabCfg<F, 1, 2, 4, 2>, F>(tasks, n, x, s);
}

template hipError_t launch_slab<MQ4KS>(const MatArgs *, int, const Q8KView &, hipStream_t);
template hipError_t launch_slab<MQ5KS>(const MatArgs *, int, const Q8KView &, hipStream_t);
template hipError_t launch_slab<MQ6KS>(const MatArgs *, int, const Q8KView &, hipStream_t);

}  // namespace qmm
