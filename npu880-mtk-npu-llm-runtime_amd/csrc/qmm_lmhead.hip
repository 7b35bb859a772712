// qmm_lmhead.hip — the LM-head epilogue: running (max, argmax) per token over
// a chunk of vocabulary rows, the row gather for evaluating an indexed set of
// rows (candidate / extended-script rows), and the device-side control of the
// chunked vocabulary scan (early exit, speculative pruning).
//
// The reference scans a chunk's logits in row order and replaces its running
// best only on a strictly greater value (E:11172-11183), so the winner is the
// first row holding the chunk maximum, and a value equal to the running best
// never replaces it. In parallel: every workgroup reduces a slice to
// (value, first index) — a value that compares false both ways (NaN) is never
// taken — and one workgroup per token combines the slices in order and then
// applies the strict comparison against the running best.
//
// Scan control. Every launch of a chunk reads the scan's device state first
// and returns at once when the scan has stopped; after each chunk one
// single-thread launch applies the reference's rules (E:11203-11256), so the
// host enqueues every chunk up front and never waits between chunks.
#include "qmm_device.h"

namespace qmm {

// slice s of token m: rows [s * SLICE, (s + 1) * SLICE) of logits[m][.]
constexpr int kSlice = 1024;

// Position i of an indexed list names row ids[i]; a row past the tensor
// (ids[i] >= id_limit) has the value -1e30 (E:11150), written back to the
// logits so that the caller's values show it too.
template <bool ROUND16>
__global__ __launch_bounds__(256) void argmax_partial_kernel(float *__restrict__ logits, int rows, size_t ldl,
                                                             Best *__restrict__ part, int nslices,
                                                             const uint32_t *__restrict__ ids, uint32_t id_limit,
                                                             const int32_t *__restrict__ st) {
    __shared__ Best sh[4];
    if (scan_stopped(st)) return;
    const int s = blockIdx.x, m = blockIdx.y;
    float *lr = logits + size_t(m) * ldl;
    const int r0 = s * kSlice, r1 = min(rows, r0 + kSlice);
    Best b{-INFINITY, kNone};
    for (int r = r0 + int(threadIdx.x); r < r1; r += 256) {  // increasing r: ties keep the first
        float v = lr[r];
        if (ids && ids[r] >= id_limit) {
            v = -1e30f;
            lr[r] = v;
        }
        if (ROUND16) v = round_to_fp16(v);  // the reference compares fp16 logits (E:11175)
        if (v == v) b = better(b, Best{v, uint32_t(r)});
    }
    b = block_best(b, sh);
    if (threadIdx.x == 0) part[size_t(m) * nslices + s] = b;
}

// combine token m's slices in order, then the strict update of the running
// best; ids[i] names list position i (NULL: row_base + i). Tokens at or past
// the scan's active count keep their best (E:11169: only active_batch_len
// positions are updated).
__global__ __launch_bounds__(256) void argmax_final_kernel(const Best *__restrict__ part, int nslices,
                                                           const uint32_t *__restrict__ ids, uint32_t row_base,
                                                           float *__restrict__ best_val,
                                                           uint32_t *__restrict__ best_id,
                                                           const int32_t *__restrict__ st) {
    __shared__ Best sh[4];
    const int m = blockIdx.x;
    if (scan_stopped(st) || m >= scan_active(st, int(gridDim.x))) return;
    Best b{-INFINITY, kNone};
    for (int s = int(threadIdx.x); s < nslices; s += 256) b = better(b, part[size_t(m) * nslices + s]);
    b = block_best(b, sh);
    if (threadIdx.x == 0 && b.i != kNone && b.v > best_val[m]) {  // E:11177: v > best_v
        best_val[m] = b.v;
        best_id[m] = ids ? ids[b.i] : row_base + b.i;
    }
}

// rows ids[0..n) of a tensor of id_limit rows -> n contiguous rows (2-B
// units: every row length of the supported types is even); a row past the
// tensor is never read: zeros stand in for it (its value is set to -1e30
// afterwards)
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint8_t *__restrict__ w, size_t row_bytes,
                                                          const uint32_t *__restrict__ ids, uint32_t id_limit,
                                                          uint8_t *__restrict__ dst, const int32_t *__restrict__ st) {
    if (scan_stopped(st)) return;
    const size_t i = blockIdx.x;
    const uint32_t id = ids[i];
    uint16_t *out = reinterpret_cast<uint16_t *>(dst + i * row_bytes);
    if (id >= id_limit) {
        for (size_t k = threadIdx.x; k < row_bytes / 2; k += 256) out[k] = 0;
        return;
    }
    const uint16_t *src = reinterpret_cast<const uint16_t *>(w + size_t(id) * row_bytes);
    for (size_t k = threadIdx.x; k < row_bytes / 2; k += 256) out[k] = src[k];
}

// ------------------------------------------------------ scan of the chunks
// Start of a scan (E:11138-11141): best = (-1e30, 0) per token, every token
// active, no chunk read, candidate logits -1e30.
__global__ void scan_init_kernel(int M, float *best_val, uint32_t *best_id, float *cand, int32_t *st) {
    for (int p = int(threadIdx.x); p < M; p += int(blockDim.x)) {
        best_val[p] = -1e30f;
        best_id[p] = 0;
        cand[p] = -1e30f;
    }
    if (threadIdx.x == 0) {
        st[kScanChunks] = 0;
        st[kScanActive] = M;
        st[kScanStopped] = 0;
        st[kScanPad] = 0;
    }
}

// The draft candidates (E:11147-11153): token p < M - 1 evaluates row
// draft[p + 1]; vals [M][M - 1] holds every token's dot with every gathered
// candidate row (column q = row draft[q + 1]), of which token p's own is
// column p: -1e30 for a row past the vocabulary, then the strict update.
__global__ void scan_cand_kernel(int M, const float *vals, const uint32_t *draft, uint32_t vocab, float *best_val,
                                 uint32_t *best_id, float *cand) {
    for (int p = int(threadIdx.x); p + 1 < M; p += int(blockDim.x)) {
        const uint32_t cid = draft[p + 1];
        const float vc = cid < vocab ? vals[size_t(p) * size_t(M - 1) + p] : -1e30f;
        cand[p] = vc;
        if (vc > best_val[p]) {
            best_val[p] = vc;
            best_id[p] = cid;
        }
    }
}

// After chunk c of a scan (one workgroup): the running argmax update of every
// active token from its nslices partials (as argmax_final_kernel), then, by
// one thread, the reference's rules (E:11203-11256): positions whose best
// already beats their draft candidate by the margin end the active batch,
// and at a checkpoint the scan stops when every active token's best reaches
// the chunk's threshold. A stopped scan changes nothing.
__global__ __launch_bounds__(256) void scan_final_kernel(const Best *__restrict__ part, int nslices, uint32_t row_base,
                                                         float *__restrict__ best_val, uint32_t *__restrict__ best_id,
                                                         const float *__restrict__ cand,
                                                         const uint32_t *__restrict__ draft, float margin,
                                                         float thresh, int checkpoint, int c, int32_t *st) {
    __shared__ Best sh[4];
    if (scan_stopped(st)) return;
    int active = scan_active(st, 0);
    for (int m = 0; m < active; ++m) {
        Best b{-INFINITY, kNone};
        for (int s = int(threadIdx.x); s < nslices; s += 256) b = better(b, part[size_t(m) * nslices + s]);
        b = block_best(b, sh);
        if (threadIdx.x == 0 && b.i != kNone && b.v > best_val[m]) {  // E:11177
            best_val[m] = b.v;
            best_id[m] = row_base + b.i;
        }
        __syncthreads();  // (sh is reused by the next token)
    }
    if (threadIdx.x != 0) return;
    st[kScanChunks] = c + 1;
    if (draft) {
        for (int p = 0; p + 1 < active; ++p) {
            if (best_id[p] != draft[p + 1] && best_val[p] > cand[p] + margin) {  // E:11207-11208
                active = p + 1;
                break;
            }
        }
        st[kScanActive] = active;
    }
    int all_above = 1;
    for (int p = 0; p < active; ++p)
        if (best_val[p] < thresh) {  // E:11248
            all_above = 0;
            break;
        }
    if (checkpoint && all_above) st[kScanStopped] = 1;  // E:11254-11256
}

__global__ __launch_bounds__(256) void scan_fold_clear_kernel(ScanFold *f) { fold_clear(f); }

hipError_t launch_scan_fold_clear(ScanFold *fold, hipStream_t s) {
    hipLaunchKernelGGL(scan_fold_clear_kernel, dim3(1), dim3(256), 0, s, fold);
    return hipGetLastError();
}

size_t argmax_scratch_bytes(int M, int rows) {
    return size_t(M) * size_t((rows + kSlice - 1) / kSlice) * sizeof(Best);
}

hipError_t launch_argmax(float *logits, int M, int rows, size_t ldl, bool round16, const uint32_t *ids,
                         uint32_t id_limit, uint32_t row_base, float *best_val, uint32_t *best_id, void *scratch,
                         const int32_t *st, hipStream_t s) {
    const int nslices = (rows + kSlice - 1) / kSlice;
    Best *part = static_cast<Best *>(scratch);
    const dim3 g{unsigned(nslices), unsigned(M), 1u};
    if (round16)
        hipLaunchKernelGGL(argmax_partial_kernel<true>, g, dim3(256), 0, s, logits, rows, ldl, part, nslices, ids,
                           id_limit, st);
    else
        hipLaunchKernelGGL(argmax_partial_kernel<false>, g, dim3(256), 0, s, logits, rows, ldl, part, nslices, ids,
                           id_limit, st);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(unsigned(M)), dim3(256), 0, s, part, nslices, ids, row_base,
                       best_val, best_id, st);
    return hipGetLastError();
}

// one token: combine nparts partials in order, then the strict update
hipError_t launch_argmax_final(const void *part, int nparts, const uint32_t *ids, uint32_t row_base,
                               float *best_val, uint32_t *best_id, const int32_t *st, hipStream_t s) {
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(256), 0, s, static_cast<const Best *>(part), nparts, ids,
                       row_base, best_val, best_id, st);
    return hipGetLastError();
}

hipError_t launch_gather_rows(const uint8_t *w, size_t row_bytes, const uint32_t *ids, uint32_t id_limit, int n,
                              uint8_t *dst, const int32_t *st, hipStream_t s) {
    hipLaunchKernelGGL(gather_rows_kernel, dim3(unsigned(n)), dim3(256), 0, s, w, row_bytes, ids, id_limit, dst, st);
    return hipGetLastError();
}

hipError_t launch_scan_init(int M, float *best_val, uint32_t *best_id, float *cand, int32_t *st, hipStream_t s) {
    hipLaunchKernelGGL(scan_init_kernel, dim3(1), dim3(64), 0, s, M, best_val, best_id, cand, st);
    return hipGetLastError();
}

hipError_t launch_scan_cand(int M, const float *vals, const uint32_t *draft, uint32_t vocab, float *best_val,
                            uint32_t *best_id, float *cand, hipStream_t s) {
    hipLaunchKernelGGL(scan_cand_kernel, dim3(1), dim3(64), 0, s, M, vals, draft, vocab, best_val, best_id, cand);
    return hipGetLastError();
}

hipError_t launch_scan_final(const void *part, int nslices, uint32_t row_base, float *best_val, uint32_t *best_id,
                             const float *cand, const uint32_t *draft, float margin, float thresh, bool checkpoint,
                             int c, int32_t *st, hipStream_t s) {
    hipLaunchKernelGGL(scan_final_kernel, dim3(1), dim3(256), 0, s, static_cast<const Best *>(part), nslices, row_base,
                       best_val, best_id, cand, draft, margin, thresh, checkpoint ? 1 : 0, c, st);
    return hipGetLastError();
}

// partials of the non-fused path for a scan: per 1024-row slice and token
hipError_t launch_argmax_partials(float *logits, int M, int rows, size_t ldl, void *scratch, const int32_t *st,
                                  hipStream_t s) {
    const int nslices = (rows + kSlice - 1) / kSlice;
    const dim3 g{unsigned(nslices), unsigned(M), 1u};
    hipLaunchKernelGGL(argmax_partial_kernel<true>, g, dim3(256), 0, s, logits, rows, ldl, static_cast<Best *>(scratch),
                       nslices, nullptr, 0u, st);
    return hipGetLastError();
}
int argmax_slices(int rows) { return (rows + kSlice - 1) / kSlice; }

}  // namespace qmm
