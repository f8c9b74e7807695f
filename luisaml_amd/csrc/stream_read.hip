// stream_read.hip -- a read-only streaming kernel: the HBM read floor that
// the bandwidth-bound small-M GEMM is measured against (the same bytes with
// no arithmetic and no output stream).  Each thread keeps four independent
// 16-byte loads in flight per iteration of a grid-stride loop and folds them
// into one word, which is stored only when it equals a fixed constant: the
// loads cannot be removed, and the kernel writes (almost) nothing.
#include "lcml_internal.hpp"

namespace lcml {
namespace {

constexpr int kThreads = 256, kUnroll = 4;

__global__ __launch_bounds__(kThreads) void k_stream_read(const uint4 *__restrict__ p, int64_t n16,
                                                          uint32_t *sink) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    uint32_t acc = 0;
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    for (; i + (kUnroll - 1) * stride < n16; i += kUnroll * stride) {
        uint4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) v[u] = p[i + u * stride];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += stride) {
        const uint4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;
}

}  // namespace

hipError_t launch_stream_read(const void *p, int64_t bytes, int workgroups, uint32_t *sink, hipStream_t s) {
    hipLaunchKernelGGL(k_stream_read, dim3(workgroups), dim3(kThreads), 0, s, static_cast<const uint4 *>(p),
                       bytes / 16, sink);
    return hipGetLastError();
}

}  // namespace lcml
