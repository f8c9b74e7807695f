// pack.hip -- load-time weight packing into 64-column panels of 16-byte
// k-chunks (the operand-chunk order of the gfx950 FP8 MFMAs) and its inverse.
//
// Packed byte (k, n) of a logical [K, N] weight:
//   ((n / 64) * (Kp / 16) + k / 16) * 1024 + (n % 64) * 16 + k % 16,
// Kp = K rounded up to 128, N rounded up to 64, padding zero.
// One thread owns one 16-byte unit of the packed array, so the packed side
// is written (read) as one contiguous 1 KB run per wavefront.
#include "lcml_internal.hpp"

namespace lcml {
namespace {

typedef uint32_t u4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void k_pack(const uint8_t *__restrict__ w, int64_t K, int64_t N,
                                              int w_is_nk, int64_t KC, int64_t units,
                                              uint8_t *__restrict__ packed) {
    int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (u >= units) return;
    int64_t col = u & 63, c = (u >> 6) % KC, panel = (u >> 6) / KC;
    int64_t n = panel * 64 + col, k0 = c * 16;
    uint8_t b[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        int64_t k = k0 + j;
        bool ok = n < N && k < K;
        b[j] = ok ? (w_is_nk ? w[n * K + k] : w[k * N + n]) : (uint8_t)0;
    }
    u4 out;
    out.x = b[0] | (b[1] << 8) | (b[2] << 16) | ((uint32_t)b[3] << 24);
    out.y = b[4] | (b[5] << 8) | (b[6] << 16) | ((uint32_t)b[7] << 24);
    out.z = b[8] | (b[9] << 8) | (b[10] << 16) | ((uint32_t)b[11] << 24);
    out.w = b[12] | (b[13] << 8) | (b[14] << 16) | ((uint32_t)b[15] << 24);
    *reinterpret_cast<u4 *>(packed + u * 16) = out;
}

__global__ __launch_bounds__(256) void k_unpack(const uint8_t *__restrict__ packed, int64_t K,
                                                int64_t N, int w_is_nk, int64_t KC, int64_t units,
                                                uint8_t *__restrict__ w) {
    int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (u >= units) return;
    int64_t col = u & 63, c = (u >> 6) % KC, panel = (u >> 6) / KC;
    int64_t n = panel * 64 + col, k0 = c * 16;
    if (n >= N) return;
    u4 in = *reinterpret_cast<const u4 *>(packed + u * 16);
    uint32_t words[4] = {in.x, in.y, in.z, in.w};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        int64_t k = k0 + j;
        if (k < K) {
            uint8_t v = (uint8_t)(words[j >> 2] >> (8 * (j & 3)));
            if (w_is_nk) w[n * K + k] = v;
            else w[k * N + n] = v;
        }
    }
}

}  // namespace

hipError_t launch_pack_weight(const uint8_t *w, int64_t K, int64_t N, int w_is_nk,
                              uint8_t *packed, hipStream_t s) {
    int64_t Kp = pad_to(K, kPackK), Np = pad_to(N, kPanelCols);
    int64_t units = Np * Kp / 16;
    hipLaunchKernelGGL(k_pack, dim3((unsigned)((units + 255) / 256)), dim3(256), 0, s, w, K, N,
                       w_is_nk, Kp / 16, units, packed);
    return hipGetLastError();
}

hipError_t launch_unpack_weight(const uint8_t *packed, int64_t K, int64_t N, int w_is_nk,
                                uint8_t *w, hipStream_t s) {
    int64_t Kp = pad_to(K, kPackK), Np = pad_to(N, kPanelCols);
    int64_t units = Np * Kp / 16;
    hipLaunchKernelGGL(k_unpack, dim3((unsigned)((units + 255) / 256)), dim3(256), 0, s, packed, K,
                       N, w_is_nk, Kp / 16, units, w);
    return hipGetLastError();
}

}  // namespace lcml
