// qmm_lmhead.hip — the LM-head epilogue: running (max, argmax) per token over
// a chunk of vocabulary rows, and the row gather for evaluating an indexed
// set of rows (candidate / extended-script rows).
//
// The reference scans a chunk's logits in row order and replaces its running
// best only on a strictly greater value (E:11172-11183), so the winner is the
// first row holding the chunk maximum, and a value equal to the running best
// never replaces it. In parallel: every workgroup reduces a slice to
// (value, first index) — a value that compares false both ways (NaN) is never
// taken — and one workgroup per token combines the slices in order and then
// applies the strict comparison against the running best.
#include "qmm_device.h"

namespace qmm {


__device__ inline Best block_best(Best b, Best *sh) {
    b = wave_best(b);
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    if (lane == 0) sh[wid] = b;
    __syncthreads();
    Best r = sh[0];
    for (int w = 1; w < 4; ++w) r = better(r, sh[w]);
    return r;
}

// slice s of token m: rows [s * SLICE, (s + 1) * SLICE) of logits[m][.]
constexpr int kSlice = 1024;

template <bool ROUND16>
__global__ __launch_bounds__(256) void argmax_partial_kernel(const float *__restrict__ logits, int rows,
                                                             size_t ldl, Best *__restrict__ part,
                                                             int nslices) {
    __shared__ Best sh[4];
    const int s = blockIdx.x, m = blockIdx.y;
    const float *lr = logits + size_t(m) * ldl;
    const int r0 = s * kSlice, r1 = min(rows, r0 + kSlice);
    Best b{-INFINITY, kNone};
    for (int r = r0 + int(threadIdx.x); r < r1; r += 256) {  // increasing r: ties keep the first
        float v = lr[r];
        if (ROUND16) v = round_to_fp16(v);  // the reference compares fp16 logits (E:11175)
        if (v == v) b = better(b, Best{v, uint32_t(r)});
    }
    b = block_best(b, sh);
    if (threadIdx.x == 0) part[size_t(m) * nslices + s] = b;
}

// combine token m's slices in order, then the strict update of the running
// best; ids[i] names list position i (NULL: row_base + i)
__global__ __launch_bounds__(256) void argmax_final_kernel(const Best *__restrict__ part, int nslices,
                                                           const uint32_t *__restrict__ ids, uint32_t row_base,
                                                           float *__restrict__ best_val,
                                                           uint32_t *__restrict__ best_id) {
    __shared__ Best sh[4];
    const int m = blockIdx.x;
    Best b{-INFINITY, kNone};
    for (int s = int(threadIdx.x); s < nslices; s += 256) b = better(b, part[size_t(m) * nslices + s]);
    b = block_best(b, sh);
    if (threadIdx.x == 0 && b.i != kNone && b.v > best_val[m]) {  // E:11177: v > best_v
        best_val[m] = b.v;
        best_id[m] = ids ? ids[b.i] : row_base + b.i;
    }
}

// rows ids[0..n) of a tensor -> n contiguous rows (2-B units: every row
// length of the supported types is even)
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint8_t *__restrict__ w, size_t row_bytes,
                                                          const uint32_t *__restrict__ ids,
                                                          uint8_t *__restrict__ dst) {
    const size_t i = blockIdx.x;
    const uint16_t *src = reinterpret_cast<const uint16_t *>(w + size_t(ids[i]) * row_bytes);
    uint16_t *out = reinterpret_cast<uint16_t *>(dst + i * row_bytes);
    for (size_t k = threadIdx.x; k < row_bytes / 2; k += 256) out[k] = src[k];
}

size_t argmax_scratch_bytes(int M, int rows) {
    return size_t(M) * size_t((rows + kSlice - 1) / kSlice) * sizeof(Best);
}

hipError_t launch_argmax(const float *logits, int M, int rows, size_t ldl, bool round16,
                         const uint32_t *ids, uint32_t row_base, float *best_val, uint32_t *best_id,
                         void *scratch, hipStream_t s) {
    const int nslices = (rows + kSlice - 1) / kSlice;
    Best *part = static_cast<Best *>(scratch);
    const dim3 g{unsigned(nslices), unsigned(M), 1u};
    if (round16)
        hipLaunchKernelGGL(argmax_partial_kernel<true>, g, dim3(256), 0, s, logits, rows, ldl, part, nslices);
    else
        hipLaunchKernelGGL(argmax_partial_kernel<false>, g, dim3(256), 0, s, logits, rows, ldl, part, nslices);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(unsigned(M)), dim3(256), 0, s, part, nslices, ids, row_base,
                       best_val, best_id);
    return hipGetLastError();
}

// one token: combine nparts partials in order, then the strict update
hipError_t launch_argmax_final(const void *part, int nparts, const uint32_t *ids, uint32_t row_base,
                               float *best_val, uint32_t *best_id, hipStream_t s) {
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(256), 0, s, static_cast<const Best *>(part), nparts, ids,
                       row_base, best_val, best_id);
    return hipGetLastError();
}

hipError_t launch_gather_rows(const uint8_t *w, size_t row_bytes, const uint32_t *ids, int n, uint8_t *dst,
                              hipStream_t s) {
    hipLaunchKernelGGL(gather_rows_kernel, dim3(unsigned(n)), dim3(256), 0, s, w, row_bytes, ids, dst);
    return hipGetLastError();
}

}  // namespace qmm
