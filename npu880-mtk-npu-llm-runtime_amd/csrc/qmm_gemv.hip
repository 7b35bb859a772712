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
// Weight bytes. Every format is staged: the wave loads the contiguous bytes
// of U wave steps with 16-B loads into an LDS stage and lanes read their
// pieces from there, so each byte moves in a full 16-B transaction whatever
// the block's alignment (Q4_K / Q5_K blocks of 144 / 176 B are 16-B aligned;
// Q6_K / Q8_0 blocks of 210 / 34 B only 2-B aligned: two-byte realignment
// costs LDS reads, not HBM transactions).
//
// Activations live in LDS for the whole workgroup. The fp32 input (or the
// prequantized row) is requested first, then the first batch of weights;
// while those are in flight the workgroup quantizes the input to Q8_K /
// Q8_0 itself — 16 lanes per 256 values, DPP reductions, the reference's
// exact arithmetic — so one launch covers quantize + GEMV. Codes are stored
// with 16 B of padding per 256 values so lanes on consecutive blocks hit
// different banks. Vector-memory counters retire in order, so the fill
// waits only for the input loads; the workgroup barrier orders LDS only.
#include <mutex>

#include "qmm_gemv_parts.h"

namespace qmm {

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
    // 4a. rows whose blocks fit one batch, 4 lanes per block (R = 1, 2 or 4
    // rows of GPR = 16 / R lane groups): the row's lane groups take its
    // blocks in runs of bpg = ceil(nb / GPR) <= U and sum them in order
    // along the groups in registers, as the persistent kernel does (slots
    // past the row's blocks add +0.0, which changes no sum)
    constexpr bool CHAIN = F::kStaged && G == 4 && SLOTS % R == 0 && U <= 3;
    constexpr int GPR = CHAIN ? SLOTS / R : 1;
    if constexpr (CHAIN) {
        if (nb <= GPR * U) {
            const int r = g / GPR, q = g % GPR, bpg = (nb + GPR - 1) / GPR;
            typename F::Raw rs[U];
            typename F::Act as[U];
            bool own[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int b = q * bpg + u;
                own[u] = u < bpg && b < nb && r < nrows;
                rs[u] = F::load(stage + span_mis + (own[u] ? r * nb + b : 0) * F::BB, k);
                as[u] = F::load_act(act, own[u] ? b : 0, k);
            }
            float c[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const float v = F::compute(rs[u], as[u], k);
                c[u] = own[u] ? v : 0.0f;
            }
            float acc = 0.0f;
#pragma unroll
            for (int h = 0; h < GPR; ++h) {  // each group takes its left neighbour's sum; q = 0 starts at +0.0
                float t = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, acc), 0x114,
                                                                                0xF, 0xF, true));
                if constexpr (GPR > 4) {
                    const float up = __builtin_bit_cast(
                        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, acc), 0x142, 0xF, 0xF, true));
                    t = q == 0 ? 0.0f : (q & 3) == 0 ? up : t;
                }
#pragma unroll
                for (int u = 0; u < U; ++u) t = t + c[u];
                acc = t;
            }
            if (q == GPR - 1 && k == 0 && r < nrows) {
                const int row = row0 + r;
                if (a.res) acc = acc + a.res[row];
                a.y[row] = acc;
            }
            return;  // (nb is the task's: every wave of the workgroup returns here)
        }
    }
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
    // Every load is unconditional, at the piece index clamped into the row,
    // and a piece past the row's end leaves the sums as they were; all of a
    // row's loads are issued before the first product. (Loads behind a
    // branch, or scheduled next to their use, each waited for their own HBM
    // round trip: 7 us for 64 rows of 2560.)
    for (int b0 = 0; b0 < npc; b0 += 64 * NP) {
        float xv[NP][V];
#pragma unroll
        for (int i = 0; i < NP; ++i) float_x_piece<F16W, FUSED>(x32, xh, min(b0 + lane + 64 * i, npc - 1), xv[i]);
#pragma unroll
        for (int j = 0; j < R; j += 2) {
            if (j >= nrows) break;  // the same in every lane of the wave
            const bool two = j + 1 < nrows;
            const uint8_t *w0 = a.w + size_t(row0 + j) * a.row_bytes;
            const uint8_t *w1 = a.w + size_t(row0 + (two ? j + 1 : j)) * a.row_bytes;
            uint4 q0[NP], q1[NP];
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const size_t pc = size_t(min(b0 + lane + 64 * i, npc - 1));
                q0[i] = ld16_nt(w0 + 16 * pc);
                if constexpr (R > 1) q1[i] = ld16_nt(w1 + 16 * pc);
            }
            __builtin_amdgcn_sched_barrier(0);  // all loads in flight before the first use
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const bool in = b0 + lane + 64 * i < npc;
                const float s0 = float_piece_dot<F16W>(q0[i], xv[i], acc[j]);
                acc[j] = in ? s0 : acc[j];
                if constexpr (R > 1)
                    if (j + 1 < R) {
                        const float s1 = float_piece_dot<F16W>(q1[i], xv[i], acc[j + 1]);
                        acc[j + 1] = in ? s1 : acc[j + 1];
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
        case kQ5_K: gemv_wg<FmtQ5K4, R, 3, FUSED, stage_chunks<FmtQ5K4, 3>()>(a, bx, x32, prek, pre0); break;
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
// X16: x32 holds an fp16 row (reinterpreted), quantized in the kernel.
// The body of one workgroup of the persistent grid: workgroup wgi of the
// nwg that share the task's row groups. RMS (with FUSED, K <= 4096): x32 is
// the row before its RMSNorm, gamma the norm's weights; the workgroup forms
// the normed fp16 row (rmsnorm_fp16_rows_fast, E:4264-4314, the same values
// as rmsnorm_q8k_kernel) and quantizes that.
// ------------------------------------- the chunk scan's fold (SCAN mode)
// the largest key over the wave (returned in every lane): DPP row shifts
// within each 16-lane row, then the row broadcasts, the result in lane 63
__device__ inline unsigned long long wave_max_key(unsigned long long k) {
    uint32_t hi = uint32_t(k >> 32), lo = uint32_t(k);
    auto step = [&](auto ctrl, auto rows) __attribute__((always_inline)) {
        constexpr int C = decltype(ctrl)::value, RM = decltype(rows)::value;
        // lanes with no source (or outside the row mask) see the key 0, the smallest
        const uint32_t h2 = uint32_t(__builtin_amdgcn_update_dpp(0, int(hi), C, RM, 0xF, false));
        const uint32_t l2 = uint32_t(__builtin_amdgcn_update_dpp(0, int(lo), C, RM, 0xF, false));
        const bool take = h2 > hi || (h2 == hi && l2 > lo);
        hi = take ? h2 : hi;
        lo = take ? l2 : lo;
    };
    using std::integral_constant;
    step(integral_constant<int, 0x111>{}, integral_constant<int, 0xF>{});  // row_shr:1
    step(integral_constant<int, 0x112>{}, integral_constant<int, 0xF>{});  // row_shr:2
    step(integral_constant<int, 0x114>{}, integral_constant<int, 0xF>{});  // row_shr:4
    step(integral_constant<int, 0x118>{}, integral_constant<int, 0xF>{});  // row_shr:8
    step(integral_constant<int, 0x142>{}, integral_constant<int, 0xA>{});  // row_bcast:15 into rows 1, 3
    step(integral_constant<int, 0x143>{}, integral_constant<int, 0xC>{});  // row_bcast:31 into rows 2, 3
    hi = uint32_t(__builtin_amdgcn_readlane(int(hi), 63));
    lo = uint32_t(__builtin_amdgcn_readlane(int(lo), 63));
    return (static_cast<unsigned long long>(hi) << 32) | lo;
}

template <class F, int R, int U, bool FUSED, int NC, bool AMAX, bool X16 = false, bool RMS = false, bool SCAN = false>
__device__ __attribute__((always_inline)) inline void gemv_persist_wg(MatArgs a, const float *__restrict__ x32,
                                                                      Q8KView prek, Q80View pre0, AmaxOut am,
                                                                      int wgi, int nwg,
                                                                      const float *__restrict__ gamma = nullptr,
                                                                      const ScanPlan *sp = nullptr) {
    static_assert(!RMS || (FUSED && !X16), "the RMSNorm fill takes an fp32 row");
    static_assert(!(SCAN && AMAX), "the scan folds its chunk bests instead of writing partials");
    constexpr bool STEP = AMAX || SCAN;  // a scan chunk's launch: the previous chunk's step first
    extern __shared__ __align__(16) uint8_t lds[];
    static_assert(F::kStaged, "the persistent kernel stages its rows in LDS");
    constexpr int G = F::G, SLOTS = 64 / G, NST = stage_chunks<F, U>();
    constexpr bool q80 = IsQ80<F>::v;
    if (scan_stopped(a.scan)) return;
    const int lane = threadIdx.x & 63, wid = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
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

    // a group's bytes from the 16-B boundary at or below its first byte,
    // through a descriptor that ends with the group (rounded up to a 16-B
    // granule: the range check is per dword, and a granule never crosses a
    // page): lanes past the end read zeros and request no memory. The group
    // index is wave-uniform, so its address is scalar arithmetic and every
    // lane's offset is fixed.
    static_assert(NC <= NST, "stage loads beyond the stage");
    uint4 st[NC];
    auto stage_load = [&](int gr) __attribute__((always_inline)) {
        const int rows = max(0, min(R, a.N - gr * R));
        const uint8_t *span = a.w + size_t(rows > 0 ? gr * R : 0) * a.row_bytes;
        const int mis = int(reinterpret_cast<uintptr_t>(span) & 15);
        const int bytes = (mis + max(rows * nb, 1) * F::BB + 15) & ~15;
        const __amdgpu_buffer_rsrc_t rs =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(span - mis), short(0), bytes, 0x00020000);
#pragma unroll
        for (int j = 0; j < NC; ++j)
            st[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, uint32_t(16 * (64 * j + lane)), 0, kNonTemporal));
    };

    int gw = wgi * 4 + wid;
    const int stride = nwg * 4;
    // 0. a scan's step after the previous chunk (the partials are requested
    // ahead of the activations; the decision precedes every weight request,
    // so a chunk the step stops reads no weights). The scan's first launch
    // at batch 1 seeds its state instead (E:11138-11141): nothing in this
    // launch reads it, the next launch does.
    Best pb4[4];
    if constexpr (STEP) {
        if (am.pre.init && wgi == 0 && threadIdx.x == 0) {
            am.pre.best_val[0] = -1e30f;
            am.pre.best_id[0] = 0;
            am.pre.st[kScanChunks] = 0;
            am.pre.st[kScanActive] = 1;
            am.pre.st[kScanStopped] = 0;
            am.pre.st[kScanPad] = 0;
        }
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
    uint4 x16q[X16 ? kX16Rounds : 1][2];
    if constexpr (X16) {
        const uint16_t *x16 = reinterpret_cast<const uint16_t *>(x32);
#pragma unroll
        for (int r = 0; r < kX16Rounds; ++r)
            if (x_has(r, K)) x16_load(x16, K, x_chunk(r, K), x16q[r]);
    } else if constexpr (FUSED) {
        if (x_has(0, K)) x_load(x32, K, x_chunk(0, K), xp);
    }
    else cpre_load<q80>(pq, pd, pb, K, cp);
    // RMS: the norm's weights, in the fill's order
    [[maybe_unused]] XPre gp;
    if constexpr (RMS)
        if (x_has(0, K)) x_load(gamma, K, x_chunk(0, K), gp);
    if constexpr (STEP) {
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
                if (wgi == 0) {
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
    if constexpr (FUSED || X16) wait_vmcnt<0>();
    __builtin_amdgcn_sched_barrier(0);
    stage_load(min(gw, ngroups - 1));
    __builtin_amdgcn_sched_barrier(0);
    // 2. the activations into LDS, once
    if constexpr (RMS) {
        __shared__ float rms_part[4];
        rms_fill_transform(xp, gp, K, rms_part);
    }
    if constexpr (X16) x16_fill<q80, std::is_same_v<F, FmtQ6K4>>(x16q, K, act);
    else if constexpr (FUSED) x_fill<q80, std::is_same_v<F, FmtQ6K4>>(xp, x32, K, act);
    else cpre_fill<q80, std::is_same_v<F, FmtQ6K4>>(cp, pq, pd, pb, K, act);
    // SCAN: the workgroup's per-chunk best
    [[maybe_unused]] __shared__ unsigned long long lkey[SCAN ? kFoldChunks : 1];
    if constexpr (SCAN)
        if (threadIdx.x < kFoldChunks) lkey[threadIdx.x] = 0ull;
    lds_barrier();
    // 3. groups. With 4 lanes per block (R = 1, 2 or 4 rows of 16 / R lane
    // groups each), a row's GPR lane groups take its blocks in consecutive
    // runs of bpg = ceil(nb / GPR) <= U, and the row sum (blocks in order,
    // eval_single_lm_row_dot's accumulation) runs along them in registers:
    // group q adds its run to the sum group q - 1 passes it, in GPR steps.
    // The sum moves 4 lanes up within a 16-lane DPP row (row_shr:4) and from
    // a row's lane 15 into the next row (row_bcast:15). Slots past the row's
    // blocks add +0.0, which leaves every sum unchanged (none is -0.0: each
    // starts from +0.0). Other formats: the block terms meet in LDS and one
    // lane per row sums them.
    constexpr bool CHAIN = G == 4 && SLOTS % R == 0;
    constexpr int GPR = CHAIN ? SLOTS / R : 1;
    const int bpg = (nb + GPR - 1) / GPR;
    [[maybe_unused]] const int adv = SLOTS % nb;
    Best wb{-INFINITY, kNone};  // AMAX: the wave's running (max, first row); SCAN: of the current chunk
    [[maybe_unused]] int ccur = 0;
    // SCAN: this wave's contribution to chunk c (its best over its rows of
    // the chunk, or nothing), into the workgroup's best of the chunk in LDS
    [[maybe_unused]] auto contribute = [&](int c) __attribute__((always_inline)) {
        const unsigned long long k = wave_max_key(best_key(wb));
        if (lane == 0) (void)__hip_atomic_fetch_max(&lkey[c], k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        wb = Best{-INFINITY, kNone};
    };
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
        if constexpr (SCAN) {  // entering a later chunk: the chunks left behind (while the next bytes travel)
            const int cg = gw / sp->chunk_groups;
            while (ccur < cg) contribute(ccur++);
        }
        float acc = 0.0f;
        int orow = lane;  // the row (of the group) this lane's acc belongs to
        bool wr = lane < nrows;
        if constexpr (CHAIN) {
            const int r = g / GPR, q = g % GPR;  // row, its lane group's place in the row
            typename F::Raw rs[U];
            typename F::Act as[U];
            bool own[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int b = q * bpg + u;  // the row's blocks in runs of bpg
                own[u] = u < bpg && b < nb && r < nrows;
                rs[u] = F::load(stage + mis + (own[u] ? r * nb + b : 0) * F::BB, k);
                as[u] = F::load_act(act, own[u] ? b : 0, k);
            }
            float c[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const float v = F::compute(rs[u], as[u], k);
                c[u] = own[u] ? v : 0.0f;
            }
            // after step h the groups q <= h hold their sums through their
            // runs (each group takes its left neighbour's sum; groups q = 0
            // start from +0.0)
            float sacc = 0.0f;
#pragma unroll
            for (int h = 0; h < GPR; ++h) {
                float t = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sacc), 0x114,
                                                                                0xF, 0xF, true));
                if constexpr (GPR > 4) {
                    const float up = __builtin_bit_cast(
                        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sacc), 0x142, 0xF, 0xF, true));
                    t = q == 0 ? 0.0f : (q & 3) == 0 ? up : t;
                }
#pragma unroll
                for (int u = 0; u < U; ++u) t = t + c[u];
                sacc = t;
            }
            acc = sacc;
            orow = r;
            wr = q == GPR - 1 && k == 0 && r < nrows;
        } else {
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
            }
        }
        if (wr) {
            const int row = row0 + orow;
            if (a.res) acc = acc + a.res[row];
            if constexpr (AMAX)
                if (am.ids && am.ids[row] >= am.id_limit) acc = -1e30f;  // a row past the tensor (E:11150)
            if constexpr (!SCAN) a.y[row] = acc;
            if constexpr (AMAX || SCAN) {
                const float v = am.round16 ? round_to_fp16(acc) : acc;  // as the argmax kernels compare
                if (v == v) wb = better(wb, Best{v, uint32_t(row)});
            }
        }
    }
    if constexpr (SCAN) {
        while (ccur < sp->nch) contribute(ccur++);
        // one thread folds the workgroup's chunk bests into word wgi % 16 of
        // each chunk (device-scope maxima, performed where every XCD's
        // atomics meet), waits until they are done, and counts the workgroup
        // in on the arrival word; workgroup 0 first releases its state
        // writes (the one L2 write-back of the launch: one per workgroup
        // measured 17 us slower). The workgroup that completes the count
        // takes the launch's final step. (A workgroup that returned above
        // found the scan stopped, as every workgroup of the launch then does:
        // nothing counts, and nothing is left to decide.)
        __syncthreads();
        __shared__ int last;
        if (threadIdx.x == 0) {
            for (int c = 0; c < sp->nch; ++c)
                (void)__hip_atomic_fetch_max(&sp->fold->wd[wgi % kFoldWords][c].key, lkey[c], __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
            if (wgi == 0) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
            else wait_vmcnt<0>();
            last = __hip_atomic_fetch_add(&sp->fold->arrived, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                   unsigned(nwg - 1);
        }
        __syncthreads();
        if (last) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            scan_fold_decide(*sp);
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
            static_cast<Best *>(am.part)[wgi] = r;
        }
    }
}

template <class F, int R, int U, bool FUSED, int NC, bool AMAX, bool X16 = false>
__global__ __launch_bounds__(256) void gemv_persist_kernel(MatArgs a, const float *__restrict__ x32,
                                                           Q8KView prek, Q80View pre0, AmaxOut am) {
    gemv_persist_wg<F, R, U, FUSED, NC, AMAX, X16>(a, x32, prek, pre0, am, int(blockIdx.x), int(gridDim.x));
}

// ------------------------------ several formats on one persistent grid
// A batch-1 task group of several k-quant formats (with F32 / F16 tasks
// beside them) in one launch, the k-quant tasks on the persistent grid:
// task t owns the workgroups grp.wg0[t] .. grp.wg0[t + 1] - 1, which share
// its row groups exactly as the one-task persistent kernel's grid does
// (the slices are in proportion to the tasks' row groups); every workgroup
// fills its own activations. F32 / F16 tasks keep one row per wave. The
// stage loads per lane are the format's largest count less D (the launcher
// takes the largest D that still covers every task's row groups). Each
// output equals the one-task launch's, bit for bit.
// RMS: x32 is the row before its RMSNorm (gamma: the norm's weights), every
// task a k-quant one; each workgroup normalizes the row itself.
// OCC: waves per SIMD the registers are held to (3: <= 168 VGPRs).
template <bool FUSED, int D, bool RMS = false, int OCC = 1>
__global__ __launch_bounds__(256, OCC) void gemv_mixed_persist_kernel(MatGroup grp, const float *__restrict__ x32,
                                                                 Q8KView prek, Q80View pre0,
                                                                 const float *__restrict__ gamma) {
    int bx = 0;
    const int t = group_task(grp, int(blockIdx.x), bx);
    const MatArgs a = grp.t[t];
    const int nwg = grp.wg0[t + 1] - grp.wg0[t];
    constexpr int N4 = stage_chunks<FmtQ4K4, 3>() - D, N5 = stage_chunks<FmtQ5K4, 3>() - D;
    constexpr int N6 = stage_chunks<FmtQ6K4, 3>() - D;
    switch (a.type) {
        case kQ4_K:
            gemv_persist_wg<FmtQ4K4, kGemvR, 3, FUSED, N4, false, false, RMS>(a, x32, prek, pre0, AmaxOut{}, bx, nwg, gamma);
            break;
        case kQ5_K:
            gemv_persist_wg<FmtQ5K4, kGemvR, 3, FUSED, N5, false, false, RMS>(a, x32, prek, pre0, AmaxOut{}, bx, nwg, gamma);
            break;
        case kQ6_K:
            gemv_persist_wg<FmtQ6K4, kGemvR, 3, FUSED, N6, false, false, RMS>(a, x32, prek, pre0, AmaxOut{}, bx, nwg, gamma);
            break;
        case kF32:
            if constexpr (!RMS) gemv_float_wg<false, 1, FUSED>(a, bx, x32, prek.h);
            break;
        case kF16:
            if constexpr (!RMS) gemv_float_wg<true, 1, FUSED>(a, bx, x32, prek.h);
            break;
        default: break;
    }
}

template <class F> struct FmtTag { using type = F; };

// One task on the row before its RMSNorm: the one-task persistent grid with
// the norm in its fill, the task's arguments passed directly (no group
// table to resolve before the first activation load).
template <class F, int NC>
__global__ __launch_bounds__(256) void gemv_persist_rms_kernel(MatArgs a, const float *__restrict__ x32,
                                                               const float *__restrict__ gamma) {
    gemv_persist_wg<F, kGemvR, 3, true, NC, false, false, true>(a, x32, Q8KView{}, Q80View{}, AmaxOut{},
                                                               int(blockIdx.x), int(gridDim.x), gamma);
}

// The running argmax GEMV on the row before its RMSNorm (the LM head behind
// the final norm, run_final_norm_and_lm_head_batch_sdot): every workgroup
// normalizes and quantizes the row in its fill, as gemv_persist_rms_kernel.
template <class F, int NC>
__global__ __launch_bounds__(256) void gemv_argmax_rms_kernel(MatArgs a, const float *__restrict__ x32,
                                                              const float *__restrict__ gamma, AmaxOut am) {
    gemv_persist_wg<F, kGemvR, 3, true, NC, true, false, true>(a, x32, Q8KView{}, Q80View{}, am, int(blockIdx.x),
                                                              int(gridDim.x), gamma);
}

// The batch-1 chunk scan's later chunks in one launch: the persistent
// argmax GEMV over all the launch's chunks, the previous chunk's step first
// (pre), each wave folding its chunk bests as it moves on (SCAN mode
// above); a prequantized row, or (RMS) the row before its norm.
// (three waves per SIMD: the persistent grid puts up to three workgroups on a CU)
template <class F, int NC, bool RMS>
__global__ __launch_bounds__(256, 3) void gemv_scan_kernel(MatArgs a, const float *__restrict__ x32,
                                                        const float *__restrict__ gamma, Q8KView prek, ScanPlan sp,
                                                        PrevStep pre) {
    AmaxOut am{};
    am.round16 = 1;  // chunk logits compare as fp16 (E:11175)
    am.pre = pre;
    gemv_persist_wg<F, kGemvR, 3, RMS, NC, false, false, RMS, true>(a, x32, prek, Q80View{}, am, int(blockIdx.x),
                                                                    int(gridDim.x), gamma, &sp);
}

// ------------------------------------------- 2..4 tokens, batch-1 shape
// The persistent kernel's structure for 2 <= M <= MT <= 4 tokens on a
// prequantized input (the codes and scales of the Q8_K buffer; the 32-code
// sums are formed from the codes, so the buffer's bsum32 section is not
// read): every token's row is filled into LDS once per workgroup, and each
// wave's row groups are
// staged and unpacked once for all tokens; per token the lane groups form
// the block terms (the batch-1 expression) and sum them in block order
// along each row's lane groups in registers. Each output equals the batch-1
// GEMV of its token, bit for bit. 4 lanes per block, R = 1, 2 or 4.
// FUSED: x32 holds the tokens' fp32 rows, which every workgroup quantizes
// into its LDS rows itself (the batch-1 fill per token: the quantizer's
// launch saved); the rows are requested before the weights.
template <class F, int R, int U, int NC, int MT, bool FUSED = false>
__global__ __launch_bounds__(256) void gemv_mt_kernel(MatArgs a, Q8KView prek, const float *__restrict__ x32) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int G = F::G, SLOTS = 64 / G, GPR = SLOTS / R;
    static_assert(G == 4 && SLOTS % R == 0 && F::kStaged, "4 lanes per block, whole rows per DPP rows");
    if (scan_stopped(a.scan)) return;
    const int lane = threadIdx.x & 63, wid = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    const int g = lane / G, k = lane % G;
    const int K = a.K, nb = K / F::QK, M = a.M;
    const int ngroups = (a.N + R - 1) / R;
    const size_t act_bytes = gemv_act_lds_bytes(false, K);
    uint8_t *stage = lds + MT * act_bytes + size_t(wid) * NC * 1024;

    uint4 st[NC];
    auto stage_load = [&](int gr) __attribute__((always_inline)) {
        const int rows = max(0, min(R, a.N - gr * R));
        const uint8_t *span = a.w + size_t(rows > 0 ? gr * R : 0) * a.row_bytes;
        const int mis = int(reinterpret_cast<uintptr_t>(span) & 15);
        const int bytes = (mis + max(rows * nb, 1) * F::BB + 15) & ~15;
        const __amdgpu_buffer_rsrc_t rs =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(span - mis), short(0), bytes, 0x00020000);
#pragma unroll
        for (int j = 0; j < NC; ++j)
            st[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, uint32_t(16 * (64 * j + lane)), 0, kNonTemporal));
    };

    // 1. the tokens' rows requested, then the first group's bytes; the rows into LDS
    int gw = int(blockIdx.x) * 4 + wid;
    const int stride = int(gridDim.x) * 4;
    if constexpr (FUSED) {
        XPre xp[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t)
            if (t < M && x_has(0, K)) x_load(x32 + size_t(t) * K, K, x_chunk(0, K), xp[t]);
        wait_vmcnt<0>();  // the rows before the weights (as the batch-1 fill)
        __builtin_amdgcn_sched_barrier(0);
        stage_load(min(gw, ngroups - 1));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < MT; ++t)
            if (t < M)
                x_fill<false, std::is_same_v<F, FmtQ6K4>>(xp[t], x32 + size_t(t) * K, K,
                                                          gemv_act_view(lds + t * act_bytes, false, K));
    } else {
        CPre cp[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t)
            if (t < M)
                cpre_load<false, false>(prek.qs + size_t(t) * K, prek.d + size_t(t) * nb, nullptr, K, cp[t]);
        __builtin_amdgcn_sched_barrier(0);
        stage_load(min(gw, ngroups - 1));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < MT; ++t)
            if (t < M)
                cpre_fill<false, std::is_same_v<F, FmtQ6K4>, true>(cp[t], prek.qs + size_t(t) * K,
                                                                    prek.d + size_t(t) * nb, nullptr, K,
                                                                    gemv_act_view(lds + t * act_bytes, false, K));
    }
    lds_barrier();

    // 2. groups (as the batch-1 persistent kernel's register row sums)
    const int bpg = (nb + GPR - 1) / GPR;
    const int r = g / GPR, q = g % GPR;
    for (; gw < ngroups; gw += stride) {
        const int row0 = gw * R;
        const int nrows = min(R, a.N - row0);
        const int mis = int(reinterpret_cast<uintptr_t>(a.w + size_t(row0) * a.row_bytes) & 15);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
#pragma unroll
        for (int j = 0; j < NC; ++j) *reinterpret_cast<uint4 *>(stage + 16 * (64 * j + lane)) = st[j];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
        if (gw + stride < ngroups) stage_load(gw + stride);
        typename F::Raw rs[U];
        bool own[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int b = q * bpg + u;
            own[u] = u < bpg && b < nb && r < nrows;
            rs[u] = F::load(stage + mis + (own[u] ? r * nb + b : 0) * F::BB, k);
        }
        const bool wr = q == GPR - 1 && k == 0 && r < nrows;
        const int row = row0 + r;
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            if (t >= M) break;  // the same in every lane
            const LdsAct act = gemv_act_view(lds + t * act_bytes, false, K);
            float c[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int b = q * bpg + u;
                const float v = F::compute(rs[u], F::load_act(act, own[u] ? b : 0, k), k);
                c[u] = own[u] ? v : 0.0f;
            }
            float acc = 0.0f;
#pragma unroll
            for (int h = 0; h < GPR; ++h) {  // each group takes its left neighbour's sum; q = 0 starts at +0.0
                float s = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, acc), 0x114,
                                                                                0xF, 0xF, true));
                if constexpr (GPR > 4) {
                    const float up = __builtin_bit_cast(
                        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, acc), 0x142, 0xF, 0xF, true));
                    s = q == 0 ? 0.0f : (q & 3) == 0 ? up : s;
                }
#pragma unroll
                for (int u = 0; u < U; ++u) s = s + c[u];
                acc = s;
            }
            if (wr) {
                if (a.res) acc = acc + a.res[size_t(t) * a.ldr + row];
                a.y[size_t(t) * a.ldy + row] = acc;
            }
        }
    }
}


size_t gemv_lds_bytes(uint32_t type, int K) {
    switch (type) {
        case kQ4_K: return gemv_lds_bytes_t<FmtQ4K4, kGemvR, 3>(K);
        case kQ5_K: return gemv_lds_bytes_t<FmtQ5K4, kGemvR, 3>(K);
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
// Workgroups of kernel fn (256 threads, lds bytes of dynamic LDS) resident
// on one CU at once, from the runtime's occupancy query, remembered per
// device, kernel and LDS size; 0 where the query fails.
static int resident_per_cu(const void *fn, size_t lds) {
    struct Entry { int dev; const void *fn; size_t lds; int n; };
    static std::mutex mu;
    static Entry seen[64];
    static int nseen = 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    {
        std::lock_guard<std::mutex> lock(mu);
        for (int i = 0; i < nseen; ++i)
            if (seen[i].dev == dev && seen[i].fn == fn && seen[i].lds == lds) return seen[i].n;
    }
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, 256, lds) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (nseen < 64) seen[nseen++] = Entry{dev, fn, lds, n};
    return n;
}

// Workgroups of the persistent batch-1 grid for `quads` (four row groups
// each, one per wave): where the quads are exactly 2, 3 or 4 per CU, a whole
// number of workgroups per CU whose waves take a whole number of groups each
// (measured, K = 2560: 8192 rows on one workgroup per CU, Q4_K / Q5_K / Q6_K
// 4.65 / 5.40 / 6.80 -> 4.34 / 4.82 / 5.98 us; 12288 rows on three, 5.72 /
// 6.85 / 8.63 -> 5.50 / 6.45 / 7.70; 16384 rows on two, Q4_K / Q6_K 6.79 /
// 10.15 -> 6.19 / 9.19); otherwise 5/8 of a workgroup per quad, at most
// three per CU (380 workgroups for the 608 quads of 9728 rows, 768 for the
// LM head's 9496)
static int persist_grid(int quads, int cus) {
    if (quads == 2 * cus) return cus;
    if (quads == 3 * cus) return 3 * cus;
    if (quads == 4 * cus) return 2 * cus;
    return min(3 * cus, quads * 5 / 8);
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

template <class F, int R, int U, bool AMAX = false, bool X16 = false>
static hipError_t launch_gemv_persist_t(const MatArgs &a, const float *x32, const Q8KView &xk, const Q80View &x0,
                                        size_t lds, int wgs, hipStream_t s, AmaxOut am = {}) {
    const dim3 grid{unsigned(wgs)};
    return with_stage_chunks<F, U>(R * (a.K / F::QK), [&](auto nc) {
        constexpr int NC = decltype(nc)::value;
        if constexpr (X16) {
            hipLaunchKernelGGL((gemv_persist_kernel<F, R, U, true, NC, AMAX, true>), grid, dim3(256), lds, s, a, x32, xk, x0, am);
            return hipGetLastError();
        }
        if (x32) hipLaunchKernelGGL((gemv_persist_kernel<F, R, U, true, NC, AMAX>), grid, dim3(256), lds, s, a, x32, xk, x0, am);
        else hipLaunchKernelGGL((gemv_persist_kernel<F, R, U, false, NC, AMAX>), grid, dim3(256), lds, s, a, x32, xk, x0, am);
        return hipGetLastError();
    });
}

// The persistent grid of one task (R = kGemvR) with the running argmax
// fused; NotSupported (nothing launched) where that grid does not apply.
// Below two workgroups per CU the grid is one workgroup per four row groups
// (each wave's first group is its only one; the waves past the last group
// stage the last group's bytes and hold no rows). gamma: x32 is the row
// before its RMSNorm, normalized and quantized in every workgroup's fill.
template <class F, int U>
static hipError_t launch_gemv_argmax_t(const MatArgs &a, const Q8KView &xk, const Q80View &x0, bool round16,
                                       const uint32_t *ids, uint32_t id_limit, void *part, int *nparts,
                                       hipStream_t s, const PrevStep &pre, bool launch, const float *x32,
                                       const float *gamma) {
    constexpr int R = kGemvR;
    const int nb = a.K / F::QK, cus = cu_count();
    const int wg0 = ((a.N + R - 1) / R + 3) / 4;
    if (R * nb > (64 / F::G) * U || (gamma && !x32)) return hipErrorNotSupported;
    const int wgs = wg0 < 2 * cus ? wg0 : persist_grid(wg0, cus);
    if (wgs > kMaxArgmaxParts || (pre.part && pre.nparts > 1024)) return hipErrorNotSupported;
    *nparts = wgs;
    if (!launch) return hipSuccess;
    const AmaxOut am{part, round16 ? 1 : 0, ids, id_limit, pre};
    const size_t lds = gemv_lds_bytes_t<F, R, U>(a.K);
    if (gamma)
        return with_stage_chunks<F, U>(R * nb, [&](auto nc) {
            constexpr int NC = decltype(nc)::value;
            hipLaunchKernelGGL((gemv_argmax_rms_kernel<F, NC>), dim3(unsigned(wgs)), dim3(256), lds, s, a, x32, gamma,
                               am);
            return hipGetLastError();
        });
    return launch_gemv_persist_t<F, R, U, true>(a, nullptr, xk, x0, lds, wgs, s, am);
}

// The one-launch scan over the persistent grid of launch_gemv_argmax;
// NotSupported (nothing launched) where that grid does not apply or the
// chunks do not fall on whole quads of row groups. launch = false: the check
// alone.
static_assert(kScanRows == kGemvR, "the scan's chunks are counted in the persistent grid's row groups");
template <class F>
static hipError_t launch_gemv_scan_t(const MatArgs &a, const Q8KView &xk, const float *x32, const float *gamma,
                                     const ScanPlan &sp, const PrevStep &pre, bool launch, hipStream_t s) {
    constexpr int R = kGemvR, U = 3;
    const int nb = a.K / F::QK, cus = cu_count();
    const int wg0 = ((a.N + R - 1) / R + 3) / 4;
    if (R * nb > (64 / F::G) * U || (gamma && !x32) || (!gamma && !xk.qs)) return hipErrorNotSupported;
    if (sp.nch < 1 || sp.nch > kFoldChunks || sp.chunk_groups <= 0 || sp.chunk_groups % 4) return hipErrorNotSupported;
    const int wgs = wg0 < 2 * cus ? wg0 : persist_grid(wg0, cus);
    if (pre.part && pre.nparts > 1024) return hipErrorNotSupported;  // (the step reads at most 1024 partials)
    if (!launch) return hipSuccess;
    const size_t lds = gemv_lds_bytes_t<F, R, U>(a.K);
    return with_stage_chunks<F, U>(R * nb, [&](auto nc) {
        constexpr int NC = decltype(nc)::value;
        if (gamma)
            hipLaunchKernelGGL((gemv_scan_kernel<F, NC, true>), dim3(unsigned(wgs)), dim3(256), lds, s, a, x32, gamma,
                               xk, sp, pre);
        else
            hipLaunchKernelGGL((gemv_scan_kernel<F, NC, false>), dim3(unsigned(wgs)), dim3(256), lds, s, a, x32, gamma,
                               xk, sp, pre);
        return hipGetLastError();
    });
}

hipError_t launch_gemv_scan(uint32_t type, const MatArgs &a, const Q8KView &xk, const float *x32, const float *gamma,
                            const ScanPlan &plan, const PrevStep &pre, bool launch, hipStream_t s) {
    switch (type) {
        case kQ4_K: return launch_gemv_scan_t<FmtQ4K4>(a, xk, x32, gamma, plan, pre, launch, s);
        case kQ5_K: return launch_gemv_scan_t<FmtQ5K4>(a, xk, x32, gamma, plan, pre, launch, s);
        case kQ6_K: return launch_gemv_scan_t<FmtQ6K4>(a, xk, x32, gamma, plan, pre, launch, s);
        default: return hipErrorNotSupported;
    }
}

hipError_t launch_gemv_argmax(uint32_t type, const MatArgs &a, const Q8KView &xk, const Q80View &x0, bool round16,
                              const uint32_t *ids, uint32_t id_limit, void *part, int *nparts, hipStream_t s,
                              const PrevStep &pre, bool launch, const float *x32, const float *gamma) {
    switch (type) {
        case kQ4_K:
            return launch_gemv_argmax_t<FmtQ4K4, 3>(a, xk, x0, round16, ids, id_limit, part, nparts, s, pre, launch, x32,
                                                    gamma);
        case kQ5_K:
            return launch_gemv_argmax_t<FmtQ5K4, 3>(a, xk, x0, round16, ids, id_limit, part, nparts, s, pre, launch, x32,
                                                    gamma);
        case kQ6_K:
            return launch_gemv_argmax_t<FmtQ6K4, 3>(a, xk, x0, round16, ids, id_limit, part, nparts, s, pre, launch, x32,
                                                    gamma);
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
    // one task of at least two workgroups' rows per CU: the persistent grid
    if constexpr (F::kStaged) {
        const int nb = tasks[0].K / F::QK;
        const int cus = cu_count();
        if (n == 1 && R * nb <= (64 / F::G) * U && g.wg0[1] >= 2 * cus) {
            const int wgs = persist_grid(g.wg0[1], cus);
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

static hipError_t launch_gemv_mixed_persist(const MatArgs *tasks, int n, const float *x32, const Q8KView &xk,
                                            const Q80View &x0, hipStream_t s, const float *gamma = nullptr);

// Rows per wave by the launch's total rows and K (measured per shape): the
// k-quants take 4 from 4096 rows, else 2 up to K = 4096, else 1 (the 2560-row
// K = 9728 down projection: 12.4 -> 8.9 us with 1); Q8_0 (34-B blocks, 5
// wave steps per batch) takes 1 at every size (4096x2560: 6.3 -> 4.9 us,
// 9728x2560: 9.9 -> 7.9, 19456x2560: 14.0 -> 13.2, 8192x4096: 14.3 -> 13.4
// against the 2 / 4 rows it took from 4096 / 8192 rows).
template <class F, int U>
static hipError_t launch_gemv_rows(const MatArgs *tasks, int n, const float *x32, const Q8KView &xk,
                                   const Q80View &x0, hipStream_t s) {
    // several k-quant tasks of one format: each on its own slice of one
    // persistent grid, where their row groups are enough for it
    if constexpr (!IsQ80<F>::v)
        if (n > 1)
            if (const hipError_t e = launch_gemv_mixed_persist(tasks, n, x32, xk, x0, s); e != hipErrorNotSupported)
                return e;
    int64_t rows = 0;
    for (int i = 0; i < n; ++i) rows += tasks[i].N;
    if constexpr (!IsQ80<F>::v) {
        if (rows >= 4096) return launch_gemv_t<F, kGemvR, U>(tasks, n, x32, xk, x0, s);
        if (tasks[0].K <= 4096) return launch_gemv_t<F, 2, U>(tasks, n, x32, xk, x0, s);
    }
    return launch_gemv_t<F, 1, U>(tasks, n, x32, xk, x0, s);
}

// dynamic LDS of one format's body at R rows per wave (F32 / F16: none)
template <int R>
static size_t gemv_wg_lds(uint32_t type, int K) {
    switch (type) {
        case kQ4_K: return gemv_lds_bytes_t<FmtQ4K4, R, 3>(K);
        case kQ5_K: return gemv_lds_bytes_t<FmtQ5K4, R, 3>(K);
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

// A mixed group on the persistent grid (gemv_mixed_persist_kernel): its
// k-quant tasks (Q4_K / Q5_K / Q6_K, R = kGemvR rows per group within one
// batch) hold at least two workgroups' row groups per CU in all; the grid is
// the one-task kernel's for that many row groups, dealt to the k-quant tasks
// in proportion to their row groups. hipErrorNotSupported (nothing launched)
// where that does not apply.
static hipError_t launch_gemv_mixed_persist(const MatArgs *tasks, int n, const float *x32, const Q8KView &xk,
                                            const Q80View &x0, hipStream_t s, const float *gamma) {
    const int K = tasks[0].K, nb = K / 256, cus = cu_count();
    if (K % 256 || kGemvR * nb > 16 * 3) return hipErrorNotSupported;
    const bool rms = gamma != nullptr;  // (K <= 3072 here: the fill's sum of squares covers it)
    if (rms && !x32) return hipErrorNotSupported;
    int quads[kMaxGroup] = {}, total = 0, d = 2, fw = 0;
    size_t lds = 0;
    for (int i = 0; i < n; ++i) {
        const uint32_t ty = tasks[i].type;
        if (ty == kF32 || ty == kF16) {
            if (rms) return hipErrorNotSupported;
            fw += (tasks[i].N + 3) / 4;  // one row per wave
            continue;
        }
        int bb, nst;
        switch (ty) {
            case kQ4_K: bb = FmtQ4K4::BB; nst = stage_chunks<FmtQ4K4, 3>(); lds = max(lds, gemv_lds_bytes_t<FmtQ4K4, kGemvR, 3>(K)); break;
            case kQ5_K: bb = FmtQ5K4::BB; nst = stage_chunks<FmtQ5K4, 3>(); lds = max(lds, gemv_lds_bytes_t<FmtQ5K4, kGemvR, 3>(K)); break;
            case kQ6_K: bb = FmtQ6K4::BB; nst = stage_chunks<FmtQ6K4, 3>(); lds = max(lds, gemv_lds_bytes_t<FmtQ6K4, kGemvR, 3>(K)); break;
            default: return hipErrorNotSupported;
        }
        // 16-B stage loads per lane a group needs from any misalignment (as with_stage_chunks)
        const int need = ((15 + kGemvR * nb * bb + 15) / 16 + 63) / 64;
        d = min(d, nst - need);
        quads[i] = ((tasks[i].N + kGemvR - 1) / kGemvR + 3) / 4;
        total += quads[i];
    }
    if (total < 2 * cus || d < 0) return hipErrorNotSupported;
    // The merged bodies hold more registers than any one-format kernel: the
    // grid is the one-task grid, but never more than the workgroups resident
    // at once (a one-format kernel per group measured no faster).
    uint32_t one = 0;
    for (int i = 0; i < n && fw == 0; ++i) {
        if (one == 0) one = tasks[i].type;
        else if (tasks[i].type != one) one = ~0u;
    }
    if (fw > 0) one = ~0u;
    const int dd = min(d, 2);
    auto run = [&](auto kern) -> hipError_t {
        const int per_cu = resident_per_cu(reinterpret_cast<const void *>(kern), lds);
        if (per_cu < 1) return hipErrorNotSupported;
        const int G = min(persist_grid(total, cus), max(cus, per_cu * cus - fw));
        MatGroup g{};
        g.n = n;
        g.wg0[0] = 0;
        int cum = 0;
        for (int i = 0; i < n; ++i) {
            g.t[i] = tasks[i];
            int w;
            if (quads[i] == 0) {
                w = (tasks[i].N + 3) / 4;
            } else {
                w = max(1, int(int64_t(G) * (cum + quads[i]) / total - int64_t(G) * cum / total));
                cum += quads[i];
            }
            g.wg0[i + 1] = g.wg0[i] + w;
        }
        hipLaunchKernelGGL(kern, dim3(unsigned(g.wg0[n])), dim3(256), lds, s, g, x32, xk, x0, gamma);
        return hipGetLastError();
    };
    // one task of one format on the row before its norm: its arguments
    // passed directly, at stage-load count NST - D
    auto one_task = [&](auto fmt) -> hipError_t {
        using F = typename decltype(fmt)::type;
        constexpr int NST = stage_chunks<F, 3>();
        auto go1 = [&](auto kern) -> hipError_t {
            const int per_cu = resident_per_cu(reinterpret_cast<const void *>(kern), lds);
            if (per_cu < 1) return hipErrorNotSupported;
            const int G = min(persist_grid(total, cus), per_cu * cus);
            hipLaunchKernelGGL(kern, dim3(unsigned(G)), dim3(256), lds, s, tasks[0], x32, gamma);
            return hipGetLastError();
        };
        if (dd == 2) return go1(gemv_persist_rms_kernel<F, NST - 2>);
        if (dd == 1) return go1(gemv_persist_rms_kernel<F, NST - 1>);
        return go1(gemv_persist_rms_kernel<F, NST>);
    };
    if (rms && n == 1) {
        switch (one) {
            case kQ4_K: return one_task(FmtTag<FmtQ4K4>{});
            case kQ5_K: return one_task(FmtTag<FmtQ5K4>{});
            case kQ6_K: return one_task(FmtTag<FmtQ6K4>{});
            default: break;
        }
    }
    // At D = 1 without F32 / F16 tasks the merged bodies are held to three
    // waves per SIMD (168 VGPRs, no spills; at D = 2 they fit anyway), so the
    // grid reaches three workgroups per CU: one format's {gate, up} Q4_K
    // 2 x 9728 x 2560 7.71 -> 7.15 us, {Q5_K 8192, Q4_K 4096} 6.42 -> 6.28 us.
    // With float tasks the k-quant grid then loses their workgroups' share
    // of the CUs (the {Q5_K 8192, Q4_K 4096, F32, F32} group 6.40 -> 6.82
    // us): the unconstrained bodies there.
    const bool occ3 = fw == 0;
    if (rms) {
        if (dd == 2) return run(gemv_mixed_persist_kernel<true, 2, true>);
        if (dd == 1) return run(gemv_mixed_persist_kernel<true, 1, true, 3>);
        return run(gemv_mixed_persist_kernel<true, 0, true>);
    }
    if (x32) {
        if (dd == 2) return run(gemv_mixed_persist_kernel<true, 2>);
        if (dd == 1) return occ3 ? run(gemv_mixed_persist_kernel<true, 1, false, 3>) : run(gemv_mixed_persist_kernel<true, 1>);
        return run(gemv_mixed_persist_kernel<true, 0>);
    }
    if (dd == 2) return run(gemv_mixed_persist_kernel<false, 2>);
    if (dd == 1) return occ3 ? run(gemv_mixed_persist_kernel<false, 1, false, 3>) : run(gemv_mixed_persist_kernel<false, 1>);
    return run(gemv_mixed_persist_kernel<false, 0>);
}

hipError_t launch_gemv_mixed(const MatArgs *tasks, int n, const float *x32, const Q8KView &xk, const Q80View &x0,
                             hipStream_t s) {
    if (n < 1 || n > kMaxGroup) return hipErrorInvalidValue;
    if (const hipError_t e = launch_gemv_mixed_persist(tasks, n, x32, xk, x0, s); e != hipErrorNotSupported) return e;
    int64_t rows = 0;
    for (int i = 0; i < n; ++i) rows += tasks[i].N;
    // rows per wave as for one k-quant launch of the group's size
    if (rows >= 4096) return launch_gemv_mixed_r<kGemvR>(tasks, n, x32, xk, x0, s);
    if (tasks[0].K <= 4096) return launch_gemv_mixed_r<2>(tasks, n, x32, xk, x0, s);
    return launch_gemv_mixed_r<1>(tasks, n, x32, xk, x0, s);
}

// A batch-1 group (one task or several) of k-quant tasks on the row before
// its RMSNorm: the norm fused into every workgroup's activation fill, on the
// persistent slices; hipErrorNotSupported (nothing launched) where those do
// not apply (the caller then runs the norm's own kernel and the group on
// its Q8_K buffer).
hipError_t launch_gemv_rms(const MatArgs *tasks, int n, const float *x32, const float *gamma, hipStream_t s) {
    if (n < 1 || n > kMaxGroup || !x32 || !gamma) return hipErrorNotSupported;
    return launch_gemv_mixed_persist(tasks, n, x32, Q8KView{}, Q80View{}, s, gamma);
}

size_t gemv_mixed_lds_bytes(uint32_t type, int K) {
    return max(gemv_wg_lds<kGemvR>(type, K), max(gemv_wg_lds<2>(type, K), gemv_wg_lds<1>(type, K)));
}

// One task on an fp16 activation row: the persistent grid of launch_gemv_t
// with its rows per wave, or hipErrorNotSupported (nothing launched; with
// launch = false, only the answer).
template <class F, int U>
static hipError_t launch_gemv_x16_t(const MatArgs &a, const uint16_t *x16, hipStream_t s, bool launch) {
    const int nb = a.K / F::QK;
    const int R = a.N >= 4096 ? kGemvR : a.K <= 4096 ? 2 : 1;  // as launch_gemv_rows
    const int wg = ((a.N + R - 1) / R + 3) / 4;
    const int cus = cu_count();
    if (a.K % 256 || a.K > 4096 * kX16Rounds || R * nb > (64 / F::G) * U || wg < 2 * cus) return hipErrorNotSupported;
    if (!launch) return hipSuccess;
    const int wgs = persist_grid(wg, cus);
    const float *xp = reinterpret_cast<const float *>(x16);
    switch (R) {
        case kGemvR: return launch_gemv_persist_t<F, kGemvR, U, false, true>(a, xp, {}, {}, gemv_lds_bytes_t<F, kGemvR, U>(a.K), wgs, s);
        case 2: return launch_gemv_persist_t<F, 2, U, false, true>(a, xp, {}, {}, gemv_lds_bytes_t<F, 2, U>(a.K), wgs, s);
        default: return launch_gemv_persist_t<F, 1, U, false, true>(a, xp, {}, {}, gemv_lds_bytes_t<F, 1, U>(a.K), wgs, s);
    }
}

hipError_t launch_gemv_x16(uint32_t type, const MatArgs &a, const uint16_t *x16, hipStream_t s, bool launch) {
    switch (type) {
        case kQ4_K: return launch_gemv_x16_t<FmtQ4K4, 3>(a, x16, s, launch);
        case kQ5_K: return launch_gemv_x16_t<FmtQ5K4, 3>(a, x16, s, launch);
        case kQ6_K: return launch_gemv_x16_t<FmtQ6K4, 3>(a, x16, s, launch);
        default: return hipErrorNotSupported;
    }
}

hipError_t launch_gemv(uint32_t type, const MatArgs *tasks, int n, const float *x32, const Q8KView &xk,
                       const Q80View &x0, hipStream_t s) {
    if (n < 1 || n > kMaxGroup) return hipErrorInvalidValue;
    switch (type) {
        case kQ4_K: return launch_gemv_rows<FmtQ4K4, 3>(tasks, n, x32, xk, x0, s);
        case kQ5_K: return launch_gemv_rows<FmtQ5K4, 3>(tasks, n, x32, xk, x0, s);
        case kQ6_K: return launch_gemv_rows<FmtQ6K4, 3>(tasks, n, x32, xk, x0, s);
        case kQ8_0: return launch_gemv_rows<FmtQ80, kGemvU>(tasks, n, x32, xk, x0, s);
        case kF32:
        case kF16: return launch_gemv_mixed(tasks, n, x32, xk, x0, s);
        default: return hipErrorInvalidValue;
    }
}

template <class F, int R, int U, int MT>
static hipError_t launch_gemv_mt_r(const MatArgs &a, const Q8KView &xk, const float *x32, hipStream_t s) {
    const int nb = a.K / F::QK;
    if (R * nb > (64 / F::G) * U) return hipErrorNotSupported;
    const int cus = cu_count();
    const int quads = ((a.N + R - 1) / R + 3) / 4;
    const int wgs = quads >= 2 * cus ? persist_grid(quads, cus) : quads;
    const size_t lds = MT * gemv_act_lds_bytes(false, a.K) + size_t(4) * stage_chunks<F, U>() * 1024;
    if (lds > 160 * 1024) return hipErrorNotSupported;
    return with_stage_chunks<F, U>(R * nb, [&](auto nc) {
        constexpr int NC = decltype(nc)::value;
        if constexpr (MT == 2) {  // (the fused fill is taken at 2 tokens only)
            if (x32) {
                hipLaunchKernelGGL((gemv_mt_kernel<F, R, U, NC, MT, true>), dim3(unsigned(wgs)), dim3(256), lds, s, a,
                                   xk, x32);
                return hipGetLastError();
            }
        }
        hipLaunchKernelGGL((gemv_mt_kernel<F, R, U, NC, MT>), dim3(unsigned(wgs)), dim3(256), lds, s, a, xk, x32);
        return hipGetLastError();
    });
}

template <class F, int U>
static hipError_t launch_gemv_mt_t(const MatArgs &a, const Q8KView &xk, const float *x32, hipStream_t s) {
    // rows per wave as for a batch-1 launch of the same tensor
    const int R = a.N >= 4096 ? kGemvR : a.K <= 4096 ? 2 : 1;
    if (a.M <= 2) {
        if (R == kGemvR) return launch_gemv_mt_r<F, kGemvR, U, 2>(a, xk, x32, s);
        if (R == 2) return launch_gemv_mt_r<F, 2, U, 2>(a, xk, x32, s);
        return launch_gemv_mt_r<F, 1, U, 2>(a, xk, x32, s);
    }
    if (R == kGemvR) return launch_gemv_mt_r<F, kGemvR, U, 4>(a, xk, x32, s);
    if (R == 2) return launch_gemv_mt_r<F, 2, U, 4>(a, xk, x32, s);
    return launch_gemv_mt_r<F, 1, U, 4>(a, xk, x32, s);
}

hipError_t launch_gemv_mt(uint32_t type, const MatArgs *tasks, int n, const Q8KView &xk, hipStream_t s,
                          const float *x32) {
    const MatArgs &a = tasks[0];
    if (n != 1 || a.M < 2 || a.M > 4 || a.K % 256 || a.K > 16384) return hipErrorNotSupported;
    if (!x32 && (!xk.qs || !xk.d)) return hipErrorNotSupported;
    // the fill quantizes the rows where that beats the quantizer's launch:
    // 2 tokens, one fill round (K <= 4096), at most four quads of row groups
    // per CU (measured: Q4_K 9728 x 2560 8.49 -> 6.57 us; slower at K = 9728,
    // Q6_K 2560 x 9728 11.3 -> 12.4, and on the 151936-row LM head, 60.6 ->
    // 66.3; even at 3..4 tokens)
    if (x32) {
        const int R = a.N >= 4096 ? kGemvR : a.K <= 4096 ? 2 : 1;
        if (a.M != 2 || a.K > 4096 || ((a.N + R - 1) / R + 3) / 4 > 4 * cu_count()) return hipErrorNotSupported;
    }
    switch (type) {
        case kQ4_K: return launch_gemv_mt_t<FmtQ4K4, 3>(a, xk, x32, s);
        case kQ5_K: return launch_gemv_mt_t<FmtQ5K4, 3>(a, xk, x32, s);
        case kQ6_K: return launch_gemv_mt_t<FmtQ6K4, 3>(a, xk, x32, s);
        default: return hipErrorNotSupported;
    }
}

}  // namespace qmm
