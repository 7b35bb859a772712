// qmm_ffn.hip — the FFN block of one layer at batch 1 in two launches, gfx950.
//
// The reference's CPU path for the block (E:8287-8296) is three steps: the
// {gate, up} task group on the normed input row, swiglu_fp16_rows_fast (h =
// silu(gate) * up and h's Q8_K, E:4326-4378), and the down task with its
// residual on that Q8_K. Here:
//
//  1. gate/up (this file): a persistent grid whose waves take groups of two
//     row pairs — gate rows 2p, 2p + 1 and the same up rows, one contiguous
//     span of each, staged through LDS — with the lanes, per-block
//     expression and in-order block sums of the batch-1 GEMV. Each group's
//     epilogue writes gate and up, h = silu(g) * u, and h rounded to fp16
//     (the quantizer's input): the SwiGLU step costs no launch of its own.
//  2. down: the batch-1 persistent GEMV on that fp16 row, which quantizes it
//     to Q8_K in LDS (the reference's quantizer) while the first weights
//     are in flight.
// The launch boundary orders h's writes before its reads. Every output
// equals the three separate steps' bit for bit: the same block terms,
// summed in the same order, and the same Q8_K codes of h.
#include "qmm_gemv_parts.h"

namespace qmm {

namespace {

constexpr int kRP = 2;  // row pairs per gate/up group (4 rows)
constexpr int kU = 3;   // wave steps of 16 blocks per batch: 48 blocks

// LDS: x codes | per-wave stage
__host__ __device__ inline size_t gate_up_lds_bytes(int K, int nc) {
    return gemv_act_lds_bytes(false, K) + size_t(4) * nc * 1024;
}

__device__ inline void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

}  // namespace

// FG: the gate/up format (FmtQ4K4 or FmtQ5K4, 4 lanes per block); FUSED:
// x32 is quantized here, otherwise prek holds the prequantized input row.
// NC: 16-B stage loads per lane of a group.
// RMS (with FUSED, K <= 4096): x32 is the row before its RMSNorm, a.gamma
// the norm's weights; the workgroup forms the normed row in its fill.
template <class FG, bool FUSED, int NC, bool RMS = false>
__global__ __launch_bounds__(256) void ffn_gate_up_kernel(FfnArgs a, const float *__restrict__ x32, Q8KView prek) {
    static_assert(!RMS || FUSED, "the RMSNorm fill takes the fp32 row");
    extern __shared__ __align__(16) uint8_t lds[];
    static_assert(FG::G == 4, "a row's lane groups fill one 16-lane DPP row");
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int g = lane / FG::G, k = lane % FG::G;
    const int K = a.K, F = a.F, nb = K / 256;
    const int ngroups = (F + kRP - 1) / kRP;

    const LdsAct act = gemv_act_view(lds, false, K);
    const size_t act_b = gemv_act_lds_bytes(false, K);
    uint8_t *stage = lds + act_b + size_t(wid) * NC * 1024;

    // a group's bytes: the gate span, then the up span (both 16-B aligned;
    // chunk indices clamped so every lane issues its loads)
    uint4 st[NC];
    auto stage_load = [&](int gp) __attribute__((always_inline)) {
        const int rows = min(kRP, F - gp * kRP);
        const int half = rows * (a.rb1 >> 4);
        const uint8_t *sg = a.wg + size_t(gp) * kRP * a.rb1;
        const uint8_t *su = a.wu + size_t(gp) * kRP * a.rb1;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int c = min(64 * j + lane, 2 * half - 1);
            st[j] = ld16_nt(c < half ? sg + 16 * c : su + 16 * (c - half));
        }
    };

    // 1. the input row, then the first group's bytes; the input into LDS
    int gw = int(blockIdx.x) * 4 + wid;
    const int stride = int(gridDim.x) * 4;
    XPre xp;
    CPre cp;
    [[maybe_unused]] XPre gp;
    if constexpr (FUSED) {
        if (x_has(0, K)) x_load(x32, K, x_chunk(0, K), xp);
        if constexpr (RMS)
            if (x_has(0, K)) x_load(a.gamma, K, x_chunk(0, K), gp);
    } else {
        cpre_load<false>(prek.qs, prek.d, prek.bs, K, cp);
    }
    if constexpr (FUSED) wait_vmcnt<0>();  // x before the weights (as in the persistent GEMV)
    __builtin_amdgcn_sched_barrier(0);
    if (gw < ngroups) stage_load(gw);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (RMS) {
        __shared__ float rms_part[4];
        rms_fill_transform(xp, gp, K, rms_part);
    }
    if constexpr (FUSED) x_fill<false, false>(xp, x32, K, act);
    else cpre_fill<false, false>(cp, prek.qs, prek.d, prek.bs, K, act);
    lds_barrier();

    // 2. groups; each step requests the next group's bytes first. The
    // group's 4 rows (r = 0, 1: gate rows 2p, 2p + 1; r = 2, 3: the same up
    // rows) take 4 lane groups each (16 lanes, one DPP row): lane group q of
    // row r computes the row's blocks q bpg .. q bpg + bpg - 1, and the row
    // sum runs along the 4 groups in registers, blocks in order
    // (eval_single_lm_row_dot's accumulation): group q adds its run to the
    // sum group q - 1 passes it. Slots past the row's blocks add +0.0, which
    // leaves every sum unchanged (none is -0.0: each starts from +0.0).
    // Row r's sum ends in lane 16 r + 12.
    const int bpg = (nb + 3) / 4;  // <= kU (K <= 3072)
    const int r = g / 4, q = g % 4;
    for (; gw < ngroups; gw += stride) {
        const int rows = min(kRP, F - gw * kRP);
        const bool rown = (r & 1) < rows;
        const int srow = r < kRP ? r : rows + (r - kRP);  // the row's place in the stage
        wave_lds_fence();
#pragma unroll
        for (int j = 0; j < NC; ++j) *reinterpret_cast<uint4 *>(stage + 16 * (64 * j + lane)) = st[j];
        wave_lds_fence();
        if (gw + stride < ngroups) stage_load(gw + stride);
        typename FG::Raw rs[kU];
        typename FG::Act as[kU];
        bool own[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int b = q * bpg + u;
            own[u] = u < bpg && b < nb && rown;
            rs[u] = FG::load(stage + (own[u] ? srow * nb + b : 0) * FG::BB, k);
            as[u] = FG::load_act(act, own[u] ? b : 0, k);
        }
        float c[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const float v = FG::compute(rs[u], as[u], k);
            c[u] = own[u] ? v : 0.0f;
        }
        float acc = 0.0f;
#pragma unroll
        for (int h = 0; h < 4; ++h) {  // row_shr:4 gives groups q = 0 a +0.0 start
            float t = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, acc), 0x114, 0xF,
                                                                            0xF, true));
#pragma unroll
            for (int u = 0; u < kU; ++u) t = t + c[u];
            acc = t;
        }
        const float upv = __shfl(acc, lane + 32);  // lane 16 r + 12: up row r - 2 + 2 = r + 2's sum
        const float hv = silu_mul(acc, upv);       // (meaningful in the gate lanes 12, 28)
        const float hv1 = __shfl(hv, lane + 16);   // lane 12: gate row 1's h
        if (q == 3 && k == 0 && rown) {
            const bool gate = r < kRP;
            const int row = gw * kRP + (r & 1);
            float *dst = gate ? a.g : a.u;
            if (dst) dst[row] = acc;
            if (gate && a.h_out) a.h_out[row] = hv;
        }
        if (lane == 12)  // the group's two h rows in fp16 (F is even: whole pairs)
            a.hx[gw] = uint32_t(f32_to_fp16_bits(hv)) | (uint32_t(f32_to_fp16_bits(hv1)) << 16);
    }
}

namespace {

int cus_of_device() {
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

template <class FG, bool FUSED, int NC, bool RMS = false>
hipError_t launch_gate_up_t(const FfnArgs &a, const float *x32, const Q8KView &xk, hipStream_t s) {
    const int ngroups = (a.F + kRP - 1) / kRP;
    const int quads = (ngroups + 3) / 4;
    // a persistent grid as the batch-1 GEMV's: 5/8 of a workgroup per four
    // groups, at most two per CU (measured on the 9728 x 2560 pair: 512
    // workgroups 15.9 us, 760 16.1, 1024 16.7, 384 17.2)
    const int cus = cus_of_device();
    const int wgs = max(1, min(2 * cus, quads * 5 / 8));
    hipLaunchKernelGGL((ffn_gate_up_kernel<FG, FUSED, NC, RMS>), dim3(unsigned(wgs)), dim3(256), gate_up_lds_bytes(a.K, NC),
                       s, a, x32, xk);
    return hipGetLastError();
}

// the stage loads per lane a group needs (whole 16-B units, both spans): 6
// for Q4_K at K = 2560, 7 for Q5_K (or Q4_K at K = 3072), 9 for Q5_K at 3072
template <class FG>
hipError_t launch_gate_up_f(const FfnArgs &a, const float *x32, const Q8KView &xk, hipStream_t s) {
    const int need = (2 * kRP * (a.K / 256) * FG::BB + 1023) / 1024;
    if (a.gamma) {  // (K <= 3072: round 0 of the fill holds the whole row)
        if (!x32) return hipErrorNotSupported;
        if (need <= 6) return launch_gate_up_t<FG, true, 6, true>(a, x32, xk, s);
        if (need <= 7) return launch_gate_up_t<FG, true, 7, true>(a, x32, xk, s);
        return launch_gate_up_t<FG, true, 9, true>(a, x32, xk, s);
    }
    if (x32) {
        if (need <= 6) return launch_gate_up_t<FG, true, 6>(a, x32, xk, s);
        if (need <= 7) return launch_gate_up_t<FG, true, 7>(a, x32, xk, s);
        return launch_gate_up_t<FG, true, 9>(a, x32, xk, s);
    }
    if (need <= 6) return launch_gate_up_t<FG, false, 6>(a, x32, xk, s);
    if (need <= 7) return launch_gate_up_t<FG, false, 7>(a, x32, xk, s);
    return launch_gate_up_t<FG, false, 9>(a, x32, xk, s);
}

}  // namespace

hipError_t launch_ffn_gate_up(const FfnArgs &a, const float *x32, const Q8KView &xk, hipStream_t s) {
    if (a.K % 256 || a.K > 3072 || a.F % 256 || a.F <= 0 || a.rb1 % 16 || !a.hx) return hipErrorNotSupported;
    if (!x32 && (!xk.qs || !xk.d || !xk.bs)) return hipErrorNotSupported;
    if (a.type == kQ4_K) return launch_gate_up_f<FmtQ4K4>(a, x32, xk, s);
    if (a.type == kQ5_K) return launch_gate_up_f<FmtQ5K4>(a, x32, xk, s);
    return hipErrorNotSupported;
}

}  // namespace qmm
