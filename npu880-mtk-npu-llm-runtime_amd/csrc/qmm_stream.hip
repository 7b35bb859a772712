// qmm_stream.hip — the HBM read floor the batch-1 GEMV is measured against:
// a kernel that only streams bytes in with 16-B non-temporal loads (no
// counterpart in the reference; it is measurement, not part of the matmul).
//
// Workgroup i of G owns the byte span [i * span, (i + 1) * span) (span =
// bytes / G rounded up to 1 KB); each of its 4 waves loads 1-KB pieces
// wave, wave + 4, ... of the span, all of a wave's loads issued before any
// is used. The loaded words are folded into one word per workgroup (written
// to sink[i]) so that no load is dead.
#include "qmm_device.h"

namespace qmm {

template <int NL>
__global__ __launch_bounds__(256) void stream_read_kernel(const uint8_t *__restrict__ src, size_t bytes,
                                                          size_t span, uint32_t *__restrict__ sink) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const size_t b0 = size_t(blockIdx.x) * span;
    const size_t b1 = b0 + span < bytes ? b0 + span : bytes;
    uint32_t acc = 0;
    for (size_t p = b0 + size_t(wid) * 1024; p < b1; p += size_t(NL) * 4096) {
        uint4 v[NL];
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const size_t q = p + size_t(j) * 4096 + 16 * size_t(lane);
            v[j] = q + 16 <= b1 ? ld16_nt(src + q) : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int j = 0; j < NL; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc ^= uint32_t(__shfl_xor(int(acc), off, 64));
    __shared__ uint32_t part[4];
    if (lane == 0) part[wid] = acc;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

hipError_t launch_stream_read(const void *src, size_t bytes, int workgroups, int loads_per_wave, uint32_t *sink,
                              hipStream_t s) {
    const size_t span = ((bytes + size_t(workgroups) - 1) / size_t(workgroups) + 1023) & ~size_t(1023);
    const uint8_t *p = static_cast<const uint8_t *>(src);
    switch (loads_per_wave) {
        case 1: hipLaunchKernelGGL(stream_read_kernel<1>, dim3(unsigned(workgroups)), dim3(256), 0, s, p, bytes, span, sink); break;
        case 2: hipLaunchKernelGGL(stream_read_kernel<2>, dim3(unsigned(workgroups)), dim3(256), 0, s, p, bytes, span, sink); break;
        case 4: hipLaunchKernelGGL(stream_read_kernel<4>, dim3(unsigned(workgroups)), dim3(256), 0, s, p, bytes, span, sink); break;
        case 8: hipLaunchKernelGGL(stream_read_kernel<8>, dim3(unsigned(workgroups)), dim3(256), 0, s, p, bytes, span, sink); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace qmm
