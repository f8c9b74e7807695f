// conv.hip -- the data-layout kernels around the implicit-im2col FP8 conv:
//   * QuantizeLinear of an NCHW fp32 activation straight into the NHWC E4M3
//     layout the conv GEMM reads (per-tensor scale, static or from a reduced
//     amax), through an LDS transpose so both the fp32 reads (along W) and
//     the byte writes (along C) are contiguous;
//   * load-time packing of E4M3 conv weights [Cout][Cin][KH][KW] into the
//     packed-panel GEMM layout with K ordered (kh, kw, c) and N = Cout.
#include "lcml_internal.hpp"

namespace lcml {
namespace {

constexpr int kTile = 64;  // 64 channels x 64 pixels of one image row per workgroup
constexpr int kThreads = 256;

// grid: (Nb*H, ceil(W/64), ceil(C/64)); requires C % 4 == 0 (4-byte stores)
template <bool FROM_AMAX>
__global__ __launch_bounds__(kThreads) void k_quantize_nchw_to_nhwc(const float *__restrict__ x,
                                                                    uint8_t *__restrict__ y, int C, int H, int W,
                                                                    const float *__restrict__ scale,
                                                                    const uint32_t *__restrict__ amax_bits,
                                                                    float *__restrict__ scale_out) {
    __shared__ uint8_t tile[kTile][kTile + 4];  // [pixel][channel]
    const int w0 = blockIdx.y * kTile, c0 = blockIdx.z * kTile;
    const int n = blockIdx.x / H, h = blockIdx.x - n * H;
    const float s = FROM_AMAX ? scale_from_amax_bits(*amax_bits) : scale[0];
    if (FROM_AMAX && scale_out && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 && threadIdx.x == 0)
        *scale_out = s;
    const Recip d = make_recip(s);
    const int64_t plane = (int64_t)H * W;
    // read: 64 channel rows x 64 pixels, contiguous along W
    for (int idx = threadIdx.x; idx < kTile * kTile; idx += kThreads) {
        const int c = idx / kTile, w = idx - c * kTile;
        uint32_t code = 0;
        if (c0 + c < C && w0 + w < W) {
            const float v = x[((int64_t)n * C + c0 + c) * plane + (int64_t)h * W + w0 + w];
            code = e4m3x2_hw(div_by(v, d), 0.0f) & 0xffu;
        }
        tile[w][c] = (uint8_t)code;
    }
    __syncthreads();
    // write: per pixel 64 contiguous channel bytes, 4 per thread
    uint8_t *yrow = y + (((int64_t)n * H + h) * W) * C;
    for (int idx = threadIdx.x; idx < kTile * (kTile / 4); idx += kThreads) {
        const int w = idx / (kTile / 4), c4 = (idx - w * (kTile / 4)) * 4;
        if (w0 + w < W && c0 + c4 < C) {
            const uint32_t v = (uint32_t)tile[w][c4] | ((uint32_t)tile[w][c4 + 1] << 8) |
                               ((uint32_t)tile[w][c4 + 2] << 16) | ((uint32_t)tile[w][c4 + 3] << 24);
            *reinterpret_cast<uint32_t *>(yrow + (int64_t)(w0 + w) * C + c0 + c4) = v;
        }
    }
}

// One thread per 16-byte unit of the packed matrices (16 consecutive k of
// one column n of one group's GEMM weight): k = (kh*KW + kw)*Cin + c gathers
// W[grp*Mg + n][c][kh][kw]; k >= K and n >= Mg are zero.
__global__ void k_pack_conv_weight(const uint8_t *__restrict__ w, int Mg, int Cin, int KH, int KW,
                                   uint8_t *__restrict__ packed, int64_t KC, int64_t units_g, int64_t units) {
    const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= units) return;
    const int64_t grp = u / units_g, ul = u - grp * units_g;
    // packed byte (k, n) sits at ((n/64)*KC + k/16)*1024 + (n%64)*16 + k%16
    const int64_t blk = ul / 64, col = ul - blk * 64;  // 1 KB block = 64 columns x 16 k
    const int64_t panel = blk / KC, kc = blk - panel * KC;
    const int64_t n = panel * 64 + col;
    const int64_t K = (int64_t)KH * KW * Cin;
    uint32_t out[4] = {0u, 0u, 0u, 0u};
    if (n < Mg) {
        const int64_t co = grp * Mg + n;
        for (int j = 0; j < 16; ++j) {
            const int64_t k = kc * 16 + j;
            if (k >= K) break;
            const int64_t tap = k / Cin, c = k - tap * Cin;
            const int64_t kh = tap / KW, kw = tap - kh * KW;
            const uint32_t b = w[((co * Cin + c) * KH + kh) * KW + kw];
            out[j >> 2] |= b << (8 * (j & 3));
        }
    }
    uint32_t *dst = reinterpret_cast<uint32_t *>(packed + u * 16);
    dst[0] = out[0]; dst[1] = out[1]; dst[2] = out[2]; dst[3] = out[3];
}

}  // namespace

hipError_t launch_quantize_nhwc(const float *x, uint8_t *y, int64_t Nb, int C, int H, int W, const float *scale,
                                const uint32_t *amax_bits, float *scale_out, hipStream_t s) {
    dim3 grid((unsigned)(Nb * H), (unsigned)((W + kTile - 1) / kTile), (unsigned)((C + kTile - 1) / kTile));
    if (amax_bits)
        hipLaunchKernelGGL(k_quantize_nchw_to_nhwc<true>, grid, dim3(kThreads), 0, s, x, y, C, H, W, scale,
                           amax_bits, scale_out);
    else
        hipLaunchKernelGGL(k_quantize_nchw_to_nhwc<false>, grid, dim3(kThreads), 0, s, x, y, C, H, W, scale,
                           amax_bits, scale_out);
    return hipGetLastError();
}

hipError_t launch_pack_conv_weight(const uint8_t *w, int Cout, int Cin_g, int KH, int KW, int group, uint8_t *packed,
                                   hipStream_t s) {
    const int Mg = Cout / group;
    const int64_t K = (int64_t)KH * KW * Cin_g;
    const int64_t KC = pad_to(K, kPackK) / 16, npanels = pad_to(Mg, kPanelCols) / 64;
    const int64_t units_g = npanels * KC * 64, units = units_g * group;
    hipLaunchKernelGGL(k_pack_conv_weight, dim3((unsigned)((units + 255) / 256)), dim3(256), 0, s, w, Mg, Cin_g, KH,
                       KW, packed, KC, units_g, units);
    return hipGetLastError();
}

}  // namespace lcml
