// qmm_device.h — device-side helpers shared by the gfx950 kernels, and the
// launcher interface between the kernel files and the C ABI (qmm_api.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include <type_traits>

namespace qmm {

// ggml type ids (E:115-120)
constexpr uint32_t kF32 = 0;
constexpr uint32_t kF16 = 1;
constexpr uint32_t kQ8_0 = 8;
constexpr uint32_t kQ4_K = 12;
constexpr uint32_t kQ5_K = 13;
constexpr uint32_t kQ6_K = 14;

__host__ __device__ inline size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

// Q8_K activation buffer layout (all sections 256-B aligned):
//   qs int8[M][K] | d f32[M][K/256] | bsum32 i32[M][K/32] | tiles | h fp16[M][K] | bh
// tiles: the codes again, in the order of an MFMA operand: for token tile t
// (tokens 16t .. 16t + 15), 256-value block j and 64-value chunk h, 1 KB at
// ((t * K/256 + j) * 4 + h) * 1024 whose 16-B slot 16c + n (c < 4, n < 16)
// holds token 16t + n's codes at block offsets 64h + 8c .. +7, then
// 64h + 32 + 8c .. +7 (slots of tokens past M are not written).
// h: the fp16 values the codes were quantized from (the reference keeps them
// beside its quantized input as x_fp16, E:879-886; its F32 / F16 rows are
// dotted with them, E:3410-3440).
// bh: the sums of 16 codes (the reference's bsums, E:870, |sum| <= 2032, so
// exact in fp16) as fp16, in the order of a 16x16x16 fp16 MFMA operand: for
// token tile t and block j, 512 B at (t * K/256 + j) * 512 whose 8-B slot
// 16c + n holds token 16t + n's sums of groups 4c .. 4c + 3.
struct Q8KLayout {
    size_t d_off, bs_off, tile_off, h_off, bh_off, total;
    __host__ __device__ Q8KLayout(int M, int K) {
        const size_t mk = size_t(M) * size_t(K);
        const size_t mt = size_t((M + 15) / 16) * 16;
        d_off = align256(mk);
        bs_off = align256(d_off + 4 * size_t(M) * size_t(K / 256));
        tile_off = align256(bs_off + 4 * size_t(M) * size_t(K / 32));
        h_off = align256(tile_off + mt * size_t(K));
        bh_off = align256(h_off + 2 * mk);
        total = align256(bh_off + mt * size_t(K / 8));
    }
};
// byte offset in the tiles section of the 4 codes of token m at values
// 4i .. 4i + 3 of block j (nb blocks per row)
__host__ __device__ inline size_t q8k_tile_pos(int m, int j, int i, int nb) {
    const int h = i >> 4, kk = 4 * (i & 15);
    const int c = (kk & 31) >> 3, byte = (kk & 7) + ((kk & 32) >> 2);
    return ((size_t(m >> 4) * size_t(nb) + size_t(j)) * 4 + size_t(h)) * 1024 + size_t(16 * (16 * c + (m & 15)) + byte);
}
// byte offset in the bh section of token m's sum of group g (< 16) of block j
__host__ __device__ inline size_t q8k_bh_pos(int m, int j, int g, int nb) {
    return (size_t(m >> 4) * size_t(nb) + size_t(j)) * 512 + size_t(8 * (16 * (g >> 2) + (m & 15)) + 2 * (g & 3));
}
// Q8_0 activation buffer layout: qs int8[M][K] | d f32[M][K/32]
struct Q80Layout {
    size_t d_off, total;
    __host__ __device__ Q80Layout(int M, int K) {
        d_off = align256(size_t(M) * size_t(K));
        total = align256(d_off + 4 * size_t(M) * size_t(K / 32));
    }
};

// Activation views handed to the matmul kernels.
struct Q8KView {
    const int8_t *qs;   // [M][K]
    const float *d;     // [M][K/256]
    const int32_t *bs;  // [M][K/32]
    const int8_t *qt;   // the tiles section
    const uint16_t *h;  // fp16 values [M][K]
    const uint16_t *bh; // fp16 sums of 16 codes, MFMA operand order
};
struct Q80View {
    const int8_t *qs;  // [M][K]
    const float *d;    // [M][K/32]
};

// LDS-resident activation row of the GEMV: codes padded by 16 B per 256
// values (lds_pad), d per block, bsum32 per 32 values (Q8_K only).
struct LdsAct {
    const int8_t *qs;
    const float *d;
    const int32_t *bs;
    const int32_t *bs16;  // Q8_K: sums of 16 codes, [block][run order of the Q6_K lanes]
};
__host__ __device__ inline int lds_pad(int v) { return v + ((v >> 8) << 4); }

// State of a chunked LM-head scan (int32 words in device memory): chunks
// read, active_batch_len (E:11160), stopped (the checkpoint test passed).
constexpr int kScanChunks = 0, kScanActive = 1, kScanStopped = 2, kScanPad = 3, kScanWords = 4;

// One matmul launch: a task after validation.
struct MatArgs {
    const uint8_t *w;  // packed rows
    uint32_t type;     // ggml type id (kernels of one format ignore it)
    size_t row_bytes;
    int N;             // rows
    int K;             // cols
    int M;             // tokens
    float *y;          // [M][ldy]
    size_t ldy;
    const float *res;  // [M][ldr] or nullptr
    size_t ldr;
    const int32_t *scan = nullptr;  // a scan's state: the launch does nothing once it has stopped
};

// Several tasks of one type in one launch (the dispatcher's task groups,
// E:7954-7959, E:8110-8114): task i owns workgroups [wg0[i], wg0[i+1]) of
// the grid's x dimension; all tasks share K, M and the activations.
constexpr int kMaxGroup = 8;
struct MatGroup {
    MatArgs t[kMaxGroup];
    int wg0[kMaxGroup + 1];
    int n;
};
// the task of workgroup bx (uniform), and bx relative to that task
__device__ inline int group_task(const MatGroup &g, int bx, int &local) {
    int i = 0;
    while (i + 1 < g.n && bx >= g.wg0[i + 1]) ++i;
    local = bx - g.wg0[i];
    return i;
}

// Launchers (return hipSuccess or the launch error).
// sections a Q8_K producer may leave unwritten (the dispatcher's own buffer,
// where no kernel of the call reads them): the codes [M][K], the h values,
// the bsum32 array
constexpr unsigned kSkipQs = 1, kSkipH = 2, kSkipBs = 4;
hipError_t launch_quantize_q8k(const float *x, int M, int K, void *out, hipStream_t s, unsigned skip = 0);
hipError_t launch_quantize_q8_0(const float *x, int M, int K, void *out, hipStream_t s);
hipError_t launch_swiglu_q8k(const float *gate, const float *up, int M, int N, float *h,
                             void *out, hipStream_t s);
hipError_t launch_rmsnorm_q8k(const float *x, const float *gamma, int M, int K, float *y,
                              void *out, hipStream_t s);
// LM-head epilogue (qmm_lmhead.hip). ids: list positions name rows ids[i]
// (NULL: row_base + i), ids at or past id_limit count as -1e30; st: a
// scan's state or NULL.
size_t argmax_scratch_bytes(int M, int rows);
hipError_t launch_argmax(float *logits, int M, int rows, size_t ldl, bool round16, const uint32_t *ids,
                         uint32_t id_limit, uint32_t row_base, float *best_val, uint32_t *best_id, void *scratch,
                         const int32_t *st, hipStream_t s);
hipError_t launch_gather_rows(const uint8_t *w, size_t row_bytes, const uint32_t *ids, uint32_t id_limit, int n,
                              uint8_t *dst, const int32_t *st, hipStream_t s);
hipError_t launch_scan_init(int M, float *best_val, uint32_t *best_id, float *cand, int32_t *st, hipStream_t s);
hipError_t launch_scan_cand(int M, const float *vals, const uint32_t *draft, uint32_t vocab, float *best_val,
                            uint32_t *best_id, float *cand, hipStream_t s);
// one chunk of a scan: what its final step needs
struct ScanStep {
    const float *cand;     // each position's candidate logit
    const uint32_t *draft; // draft ids or NULL
    float margin, thresh;
    bool checkpoint;
    int c;
};
// after chunk c: the argmax update of the active tokens from their partials
// (nslices per token), then pruning and the checkpoint test
hipError_t launch_scan_final(const void *part, int nslices, uint32_t row_base, float *best_val, uint32_t *best_id,
                             const float *cand, const uint32_t *draft, float margin, float thresh, bool checkpoint,
                             int c, int32_t *st, hipStream_t s);
hipError_t launch_argmax_partials(float *logits, int M, int rows, size_t ldl, void *scratch, const int32_t *st,
                                  hipStream_t s);
int argmax_slices(int rows);
hipError_t launch_dequant_f16(const uint8_t *w, uint32_t type, int64_t rows, int64_t cols,
                              uint16_t *dst, hipStream_t s);
// the streaming-read floor (qmm_stream.hip): loads_per_wave in {1, 2, 4, 8}
hipError_t launch_stream_read(const void *src, size_t bytes, int workgroups, int loads_per_wave, uint32_t *sink,
                              hipStream_t s);
// M = 1 GEMV. x32 != nullptr: fp32 activations quantized inside the kernel;
// otherwise xk / x0 hold the prequantized row.
hipError_t launch_gemv(uint32_t type, const MatArgs *tasks, int n, const float *x32, const Q8KView &xk,
                       const Q80View &x0, hipStream_t s);
// dynamic LDS bytes the GEMV needs for K (must stay <= 64 KiB)
size_t gemv_lds_bytes(uint32_t type, int K);
// M = 1, tasks of several types (and F32 / F16 tasks) in one launch; each
// workgroup runs its own task's format. Its LDS need per type and K:
hipError_t launch_gemv_mixed(const MatArgs *tasks, int n, const float *x32, const Q8KView &xk, const Q80View &x0,
                             hipStream_t s);
// batch-1 k-quant group on the row before its RMSNorm, the norm fused into
// the activation fill; hipErrorNotSupported (nothing launched) where it does
// not apply
hipError_t launch_gemv_rms(const MatArgs *tasks, int n, const float *x32, const float *gamma, hipStream_t s);
size_t gemv_mixed_lds_bytes(uint32_t type, int K);
// M = 1 GEMV of one task with the LM head's running (max, argmax) fused into
// its persistent grid: each workgroup writes one partial (value, row) to part
// (round16: values rounded to fp16 first); *nparts receives their number
// (<= kMaxArgmaxParts) for launch_argmax_final. hipErrorNotSupported, with
// nothing launched, where that grid does not apply.
constexpr int kMaxArgmaxParts = 4096;
// A batch-1 scan's step after the previous chunk, applied at the start of the
// next chunk's launch instead of by a launch of its own: that chunk's
// partials, its first row and its threshold test. Every workgroup reads the
// partials and reaches the same decision; workgroup 0 writes the state.
struct PrevStep {
    const void *part;  // nullptr: none
    int nparts;
    uint32_t row_base;
    float thresh;
    int checkpoint, c;
    float *best_val;
    uint32_t *best_id;
    int32_t *st;
    int init = 0;  // the scan's first launch at batch 1: workgroup 0 seeds the best and the state
};
struct AmaxOut {
    void *part;
    int round16;
    const uint32_t *ids;  // the rows' ids (NULL: contiguous rows); ids >= id_limit count as -1e30
    uint32_t id_limit;
    PrevStep pre;
};
// The batch-1 chunk scan's later chunks in one launch (qmm_lm_head_scan at
// M = 1 with checkpoints): chunk 0 runs as its own launch, whose step the
// later chunks' launch applies first (every workgroup, from chunk 0's
// partials, before any weight request: a stop there ends the scan at
// once); then each wave contributes its best over its rows of every later
// chunk (a DPP max over the wave, an LDS max over the workgroup, one
// device-scope max per workgroup and chunk into one of 16 words, none of
// them waited for), and the last workgroup to finish decides those chunks
// in order from the word keys (scan_fold_decide, after the workgroups have
// counted themselves in on the arrival word): the chunks after chunk 0 are
// all read, their decisions taken at the end. Cleared (scan_fold_clear_kernel)
// before first use and by every final step for the next scan.
constexpr int kFoldChunks = 64;  // chunks per launch at most
constexpr int kFoldWords = 16;   // words per chunk
constexpr int kScanRows = 4;     // rows per row group of the batch-1 persistent grid (kGemvR)
// a key on a 256-B line of its own (the device's atomics serialize per line)
struct FoldWord {
    unsigned long long key;  // best key (best_key) of the word's workgroups
    unsigned int pad[62];
};
struct ScanFold {
    FoldWord wd[kFoldWords][kFoldChunks];  // word w of chunk c; a chunk's words 16 KB apart
    unsigned int arrived;                  // workgroups of the launch done (on a line of its own)
    unsigned int apad[63];
};
struct ScanPlan {
    ScanFold *fold;
    int nch;                   // chunks of the launch
    int chunk_groups;          // row groups per chunk
    uint32_t row_base;         // the launch's first row in the tensor (row ids of the result)
    unsigned long long ckpt;   // bit c: chunk c is a checkpoint
    float thresh[kFoldChunks];
    float *best_val;
    uint32_t *best_id;
    int32_t *st;
    int c0;                    // the launch's first chunk in the scan (the state's chunk count)
};
hipError_t launch_gemv_scan(uint32_t type, const MatArgs &a, const Q8KView &xk, const float *x32, const float *gamma,
                            const ScanPlan &plan, const PrevStep &pre, bool launch, hipStream_t s);
hipError_t launch_scan_fold_clear(ScanFold *fold, hipStream_t s);
hipError_t launch_gemv_argmax(uint32_t type, const MatArgs &a, const Q8KView &xk, const Q80View &x0, bool round16,
                              const uint32_t *ids, uint32_t id_limit, void *part, int *nparts, hipStream_t s,
                              const PrevStep &pre = PrevStep{}, bool launch = true, const float *x32 = nullptr,
                              const float *gamma = nullptr);
hipError_t launch_argmax_final(const void *part, int nparts, const uint32_t *ids, uint32_t row_base,
                               float *best_val, uint32_t *best_id, const int32_t *st, hipStream_t s);
hipError_t launch_mfma(uint32_t type, const MatArgs *tasks, int n, const Q8KView &xk, const Q80View &x0,
                       hipStream_t s);
// M >= 2, tasks of several types (k-quants, F32, F16) in one launch;
// hipErrorNotSupported (nothing launched) outside 2 <= M <= 64, K <= 3072,
// K % 256 == 0, or with a Q8_0 task.
hipError_t launch_mfma_mixed(const MatArgs *tasks, int n, const Q8KView &x, hipStream_t s);

// The FFN block's gate/up launch at batch 1 (qmm_ffn.hip): gate and up (F
// x K, Q4_K) on one input row, with SwiGLU's h written in fp32 (h_out, may
// be null) and rounded to fp16 (hx) for the down projection's launch
// (launch_gemv_x16). hipErrorNotSupported (nothing launched) unless K % 256
// == 0, K <= 3072, F % 256 == 0, 16-B aligned rows.
struct FfnArgs {
    const uint8_t *wg, *wu;
    float *g, *u;      // gate / up outputs (either may be null)
    float *h_out;      // h (fp32 [F]) or null
    uint32_t *hx;      // h rounded to fp16, two rows per word ([F / 2])
    int K, F;
    int rb1;           // row bytes of gate / up
    uint32_t type;     // gate / up format: kQ4_K or kQ5_K
    const float *gamma = nullptr;  // the input norm's weights: x is the row before its RMSNorm
};
hipError_t launch_ffn_gate_up(const FfnArgs &a, const float *x32, const Q8KView &xk, hipStream_t s);
// M = 1 GEMV of one task on an fp16 activation row x16 (16-B aligned, K %
// 256 == 0, K <= 12288), quantized to Q8_K (or Q8_0) in the kernel: Q4_K /
// Q6_K on the persistent grid, else hipErrorNotSupported (nothing
// launched). launch = false: only whether it applies.
hipError_t launch_gemv_x16(uint32_t type, const MatArgs &a, const uint16_t *x16, hipStream_t s, bool launch = true);
// 2 <= M <= 4 tokens of one Q4_K / Q5_K / Q6_K task on a prequantized input
// (its codes, scales and 32-code sums) in the batch-1 GEMV's shape, else
// hipErrorNotSupported (nothing launched)
// one task at 2 tokens, or at 3..4 on a tensor tall enough that the MFMA
// kernels need several rounds of workgroups: the batch-1 GEMV's shape
bool gemv_mt_shape(const MatArgs &a);
// x32 non-null: the tokens' fp32 rows, quantized in the kernel's fill (xk unused)
hipError_t launch_gemv_mt(uint32_t type, const MatArgs *tasks, int n, const Q8KView &xk, hipStream_t s,
                          const float *x32 = nullptr);

#if defined(__HIP_DEVICE_COMPILE__) || defined(__HIPCC__)

// ------------------------------------------------------------ fp16 helpers
__device__ inline float fp16_bits_to_f32(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}
// fp32 -> fp16 (round to nearest even, v_cvt_f16_f32) -> fp32
__device__ inline float round_to_fp16(float x) { return (float)(_Float16)x; }
// swiglu_chunk_worker (E:4349-4357): gate and up are the dispatcher's fp16
// outputs in the reference, so each fp32 input is rounded to fp16 first
// (E:4352-4353); h = (g / (1 + expf(-g))) * u in fp32 (E:4355). The caller
// rounds h to fp16 before its Q8_K quantizer.
__device__ inline float silu_mul(float g, float u) {
    g = round_to_fp16(g);
    u = round_to_fp16(u);
    return (g / (1.0f + expf(-g))) * u;  // E:4355
}
__device__ inline uint16_t f32_to_fp16_bits(float x) {
    return __builtin_bit_cast(uint16_t, (_Float16)x);
}

// ------------------------------------------------------------ int helpers
__device__ inline int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }
__device__ inline uint32_t funnel(uint32_t hi, uint32_t lo, uint32_t byte_shift) {
    return __builtin_amdgcn_alignbyte(hi, lo, byte_shift);
}

// ------------------------------------------------------- cross-lane sums
// DPP sums inside aligned lane groups. All lanes of the group must be active.
__device__ inline int dpp_xor1(int v) { return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false); }
__device__ inline int dpp_xor2(int v) { return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false); }
__device__ inline int dpp_half_mirror(int v) { return __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, false); }
__device__ inline int group4_sum(int v) {
    v += dpp_xor1(v);
    v += dpp_xor2(v);
    return v;
}
__device__ inline int group8_sum(int v) {
    v = group4_sum(v);
    v += dpp_half_mirror(v);
    return v;
}

// --------------------------------------------------------- global loads
typedef uint32_t v4u32 __attribute__((ext_vector_type(4)));
// 16 B load of an address that is 16-B aligned.
__device__ inline uint4 ld16(const void *p) { return *reinterpret_cast<const uint4 *>(p); }
// cache policy of a buffer load: non-temporal (streaming, read once)
constexpr int kNonTemporal = 2;
// streaming (non-temporal) 16 B load: weights are read exactly once
__device__ inline uint4 ld16_nt(const void *p) {
    const v4u32 v = __builtin_nontemporal_load(reinterpret_cast<const v4u32 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Workgroup barrier that orders LDS only: waits for this wave's LDS
// accesses (not its outstanding global loads) before s_barrier.
__device__ inline void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
// RMSNorm's scale of one row (rmsnorm_fp16_rows_fast, E:4264-4314) in a
// 256-thread workgroup, in the batch-1 activation fill's layout: thread t of
// wave w, 16-lane row r = (t / 16) % 4 and lane sub = t % 16 adds the squares
// of the fp16-rounded values 16 sub .. 16 sub + 15 of the row's 256-value
// chunks 16 i + 4 w + r (i = 0, 1, ... while inside the row) in order into s;
// the wave adds the 64 sums by a fixed butterfly, and the four wave sums meet
// as (w0 + w1) + (w2 + w3); inv_rms = 1 / sqrtf(sum * (1 / K) + 1e-6f)
// (E:4295). part: 4 floats of LDS. Every workgroup that calls it on the same
// row gets the same value (not the reference's row-ordered sum: its last bits
// may differ).
__device__ inline float rms_add4(float s, float4 h) {
    s += h.x * h.x;
    s += h.y * h.y;
    s += h.z * h.z;
    s += h.w * h.w;
    return s;
}
__device__ inline float rms_inv(float s, int K, float *part) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    lds_barrier();
    const float sum_sq = (part[0] + part[1]) + (part[2] + part[3]);
    const float inv_k = 1.0f / (float)K;
    return 1.0f / sqrtf(sum_sq * inv_k + 1.0e-6f);  // E:4295
}
__device__ inline uint2 ld8(const void *p) { return *reinterpret_cast<const uint2 *>(p); }
// 8 bytes starting at a 2-B aligned address: the aligned dwords that hold
// them, then a funnel shift by the misalignment. Every dword read contains
// at least one requested byte, so the read never leaves the pages of the
// requested range.
// (The aligned address is formed by pointer arithmetic on p, not through an
// integer, so the compiler keeps the global address space: global_load, not
// flat_load.)
__device__ inline uint2 ld8_a2(const uint8_t *p) {
    const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(p) & 3);
    const uint32_t *q = reinterpret_cast<const uint32_t *>(p - sh);
    const uint32_t w0 = __builtin_nontemporal_load(q), w1 = __builtin_nontemporal_load(q + 1);
    const uint32_t w2 = __builtin_nontemporal_load(q + (sh ? 2 : 1));
    return make_uint2(funnel(w1, w0, sh), funnel(w2, w1, sh));
}
// the 16-bit value at a 2-B aligned address
__device__ inline uint32_t ld16b_a2(const uint8_t *p) {
    const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(p) & 3);
    const uint32_t w = __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p - sh));
    return (w >> (sh * 8)) & 0xFFFFu;
}

// ------------------------------------------------- running (max, argmax)
// (value, row) with kNone for empty; better(a, b) takes b when a is empty,
// b is larger, or b is equal and at an earlier row — so any reduction order
// gives the first row holding the maximum, as a scan in row order would
struct Best {
    float v;
    uint32_t i;
};
constexpr uint32_t kNone = 0xFFFFFFFFu;
__device__ inline Best better(Best a, Best b) {
    if (b.i == kNone) return a;
    if (a.i == kNone || b.v > a.v || (b.v == a.v && b.i < a.i)) return b;
    return a;
}
__device__ inline Best wave_best(Best b) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        Best o;
        o.v = __shfl_xor(b.v, off, 64);
        o.i = uint32_t(__shfl_xor(int(b.i), off, 64));
        b = better(b, o);
    }
    return b;
}

// A Best as a 64-bit key whose unsigned order is better()'s: the value's
// bits in an order-preserving form above, the row's complement below (an
// earlier row wins a tie); 0 is the empty Best. NaN never enters.
__device__ inline unsigned long long best_key(Best b) {
    if (b.i == kNone) return 0ull;
    uint32_t u = __builtin_bit_cast(uint32_t, b.v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (static_cast<unsigned long long>(u) << 32) | (0xFFFFFFFFu - b.i);
}
__device__ inline Best key_best(unsigned long long k) {
    if (k == 0ull) return Best{-INFINITY, kNone};
    uint32_t u = uint32_t(k >> 32);
    u = (u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u;
    return Best{__builtin_bit_cast(float, u), 0xFFFFFFFFu - uint32_t(k & 0xFFFFFFFFu)};
}

// a scan that has stopped (uniform: every thread reads the same word)
__device__ inline bool scan_stopped(const int32_t *st) {
    return st && __builtin_amdgcn_readfirstlane(st[kScanStopped]) != 0;
}
__device__ inline int scan_active(const int32_t *st, int M) {
    return st ? __builtin_amdgcn_readfirstlane(st[kScanActive]) : M;
}
// the fold's keys and arrival count to zero (one workgroup)
__device__ inline void fold_clear(ScanFold *f) {
    for (int i = int(threadIdx.x); i < kFoldWords * kFoldChunks; i += int(blockDim.x))
        __hip_atomic_store(&f->wd[i / kFoldChunks][i % kFoldChunks].key, 0ull, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    if (threadIdx.x == 0) __hip_atomic_store(&f->arrived, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The later chunks' last step (one 256-thread workgroup, every word key of
// the launch performed): from the running best chunk 0's step left, the
// chunks in order — each chunk's best is the largest of its word keys,
// taken when strictly greater (E:11177) — to the first checkpoint whose
// threshold the running best reaches (E:11248-11256); then the best, the
// state, and the keys and arrival count cleared for the next scan.
__device__ inline void scan_fold_decide(const ScanPlan &sp) {
    ScanFold *f = sp.fold;
    __shared__ unsigned long long ck[kFoldChunks];
    if (threadIdx.x < kFoldChunks) ck[threadIdx.x] = 0ull;
    __syncthreads();
    // every word key read at once, one per thread, folded per chunk in LDS
    for (int i = int(threadIdx.x); i < kFoldWords * sp.nch; i += int(blockDim.x))
        (void)__hip_atomic_fetch_max(&ck[i % sp.nch],
                                     __hip_atomic_load(&f->wd[i / sp.nch][i % sp.nch].key, __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT),
                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __syncthreads();
    if (threadIdx.x == 0) {
        float rv = sp.best_val[0];
        uint32_t ri = sp.best_id[0];
        int c = 0, stop = 0;
        for (; c < sp.nch; ++c) {
            const Best cb = key_best(ck[c]);
            if (cb.i != kNone && cb.v > rv) {
                rv = cb.v;
                ri = sp.row_base + cb.i;
            }
            if (((sp.ckpt >> c) & 1ull) && !(rv < sp.thresh[c])) {
                stop = 1;
                ++c;
                break;
            }
        }
        sp.best_val[0] = rv;
        sp.best_id[0] = ri;
        sp.st[kScanChunks] = sp.c0 + c;
        sp.st[kScanActive] = 1;
        sp.st[kScanStopped] = stop;
        sp.st[kScanPad] = 0;
    }
    __syncthreads();  // (the keys are read above before they are cleared)
    fold_clear(f);
}

// the best of a 256-thread workgroup (sh: 4 entries of LDS)
__device__ inline Best block_best(Best b, Best *sh) {
    b = wave_best(b);
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    if (lane == 0) sh[wid] = b;
    __syncthreads();
    Best r = sh[0];
    for (int w = 1; w < 4; ++w) r = better(r, sh[w]);
    return r;
}

// ------------------------------------------------------ Q8 quantization
// Q8_K / Q8_0 codes of fp16-rounded values (quantize_row_fp16_to_q8_k
// E:947-988): id = 127 / amax, correctly rounded, computed once per block;
// q = rint(x * id) (round to nearest even, as lrintf in the default mode),
// clamped to [-127, 127]. An all-zero block (E:947-952) takes id = 0, which
// gives the same all-zero codes.
__device__ inline float q8_inv_scale(float amax) { return amax == 0.0f ? 0.0f : 127.0f / amax; }
// 4 values at a given id: the packed int8 codes and their sum
__device__ inline uint32_t quant4_id(float h0, float h1, float h2, float h3, float id, int &sum) {
    int q[4];
    const float h[4] = {h0, h1, h2, h3};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int v = (int)rintf(h[i] * id);  // E:979
        v = v > 127 ? 127 : v;
        v = v < -127 ? -127 : v;
        q[i] = v;
    }
    sum = q[0] + q[1] + q[2] + q[3];
    const uint32_t lo = __builtin_amdgcn_perm(uint32_t(q[1]), uint32_t(q[0]), 0x0C0C0400u);  // q0, q1 low bytes
    const uint32_t hi = __builtin_amdgcn_perm(uint32_t(q[3]), uint32_t(q[2]), 0x04000C0Cu);  // q2, q3 low bytes
    return lo | hi;
}
// The same codes with the rounding done by an fp32 add: for |p| < 2^22,
// p + 1.5 * 2^23 lies where the fp32 spacing is 1, so the add rounds p to an
// integer, to nearest even (the default mode), and the code is the low byte
// of the sum's bits. With |x| <= amax, |x * id| <= 127 (1 + 2^-24)^2 < 127.5:
// the clamp never binds, and x * id is NaN (code 0, as the conversion of NaN
// gives) only for a block holding an infinity or a NaN.
__device__ inline uint32_t quant4_rne(float h0, float h1, float h2, float h3, float id, int &sum) {
    constexpr float kMagic = 12582912.0f;  // 1.5 * 2^23
    const uint32_t y0 = __builtin_bit_cast(uint32_t, h0 * id + kMagic);  // E:979 (separate mul and add)
    const uint32_t y1 = __builtin_bit_cast(uint32_t, h1 * id + kMagic);
    const uint32_t y2 = __builtin_bit_cast(uint32_t, h2 * id + kMagic);
    const uint32_t y3 = __builtin_bit_cast(uint32_t, h3 * id + kMagic);
    const uint32_t q = __builtin_amdgcn_perm(y1, y0, 0x0C0C0400u) | __builtin_amdgcn_perm(y3, y2, 0x04000C0Cu);
    sum = __builtin_amdgcn_sdot4(int(q), 0x01010101, 0, false);
    return q;
}
__device__ inline uint32_t quant4(float h0, float h1, float h2, float h3, float amax, int &sum) {
    return quant4_id(h0, h1, h2, h3, q8_inv_scale(amax), sum);
}
// d = amax / 127 (E:953), 0 for an all-zero block
__device__ inline float q8_scale(float amax) { return amax == 0.0f ? 0.0f : amax / 127.0f; }

__device__ inline float wave_max(float a) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) a = fmaxf(a, __shfl_xor(a, off));
    return a;
}
__device__ inline float group8_max(float a) {
    a = fmaxf(a, __shfl_xor(a, 1));
    a = fmaxf(a, __shfl_xor(a, 2));
    a = fmaxf(a, __shfl_xor(a, 4));
    return a;
}

// get_scale_min_k4 (E:743-749) for sub-block j given the 12 scale bytes
// as three little-endian dwords s0, s1, s2.
__device__ inline uint32_t byte_of(uint32_t s0, uint32_t s1, uint32_t s2, int i) {
    const uint32_t w = (i < 4) ? s0 : ((i < 8) ? s1 : s2);
    return (w >> ((i & 3) * 8)) & 0xFFu;
}
__device__ inline void scale_min_k4(int j, uint32_t s0, uint32_t s1, uint32_t s2, int &sc, int &m) {
    if (j < 4) {
        sc = int(byte_of(s0, s1, s2, j) & 63u);
        m = int(byte_of(s0, s1, s2, j + 4) & 63u);
    } else {
        const uint32_t qj4 = byte_of(s0, s1, s2, j + 4);
        sc = int((qj4 & 0x0Fu) | ((byte_of(s0, s1, s2, j - 4) >> 6) << 4));
        m = int((qj4 >> 4) | ((byte_of(s0, s1, s2, j) >> 6) << 4));
    }
}

#endif  // device compile

// ------------------------------------------------ direct buffer -> LDS transfers
// Operands reach LDS by buffer_load ... lds (16 or 4 B per lane, lane l's
// bytes land at the LDS base + l * size): no registers, no address
// clamps, since every transfer goes through a buffer descriptor whose
// range ends exactly at the data (a lane past it reads zeros and touches
// no memory). Transfers retire in order, so a kernel releases a chunk with
// one static vmcnt wait.
//
// The transfers are written as inline assembly: the compiler tracks the
// builtin form as an LDS store and answers every later LDS read with a
// full vmcnt(0) wait (it cannot tell the slots apart), which would wait for
// the chunk still in flight. The kernel orders them itself with explicit
// vmcnt waits and barriers; inside the asm, M0 (the LDS destination) is set
// and given its one wait state.
typedef int v4i32 __attribute__((ext_vector_type(4)));

// buffer descriptor: base, stride 0, num_records bytes, raw 32-bit dwords
__device__ inline v4i32 buf_rsrc(const void *p, uint32_t bytes) {
    const uint64_t b = reinterpret_cast<uint64_t>(p);
    v4i32 r;
    r.x = __builtin_amdgcn_readfirstlane(int(uint32_t(b)));
    r.y = __builtin_amdgcn_readfirstlane(int(uint32_t(b >> 32) & 0xFFFFu));
    r.z = __builtin_amdgcn_readfirstlane(int(bytes));
    r.w = 0x00020000;
    return r;
}
__device__ inline uint32_t lds_addr(const void *p) {
    return __builtin_amdgcn_readfirstlane(
        uint32_t(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void *)p)));
}
// M0 is reserved to the compiler, which uses it in these kernels for nothing
// else (no LDS transfers of its own, no message or interpolation ops).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// lane l's 16 B at byte offset voff of the buffer land at LDS byte address lds + 16 l
__device__ inline void dma16(const v4i32 &r, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %2, 0 offen lds"
                 : : "v"(voff), "s"(lds), "s"(r) : "memory", "m0");
}
// lane l's 4 B land at lds + 4 l
__device__ inline void dma4(const v4i32 &r, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dword %0, %2, 0 offen lds"
                 : : "v"(voff), "s"(lds), "s"(r) : "memory", "m0");
}
// the same with a uniform byte offset soff added to every lane's voff
__device__ inline void dma16s(const v4i32 &r, uint32_t voff, uint32_t soff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %2, %3 offen lds"
                 : : "v"(voff), "s"(lds), "s"(r), "s"(soff) : "memory", "m0");
}
__device__ inline void dma4s(const v4i32 &r, uint32_t voff, uint32_t soff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dword %0, %2, %3 offen lds"
                 : : "v"(voff), "s"(lds), "s"(r), "s"(soff) : "memory", "m0");
}
#pragma clang diagnostic pop
// s_waitcnt vmcnt(N) (lgkmcnt and expcnt not waited on)
template <int N> __device__ inline void wait_vmcnt() {
    static_assert(N >= 0 && N <= 63, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
__device__ inline void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }  // lgkmcnt(0) only

constexpr uint32_t kFar = 0x80000000u;  // a byte offset past every descriptor's range

// fn(integral_constant<int, I>) for I = B .. E-1, unrolled at compile time
template <int B, int E, class Fn>
__device__ inline __attribute__((always_inline)) void static_for(Fn &&fn) {
    if constexpr (B < E) {
        fn(std::integral_constant<int, B>{});
        static_for<B + 1, E>(fn);
    }
}

}  // namespace qmm
