// conv.hip -- the data-layout kernels around the implicit-im2col FP8 conv:
//   * QuantizeLinear of an NCHW fp32 activation straight into the NHWC E4M3
//     layout the conv GEMM reads (per-tensor scale, static or from partial
//     maxima), through an LDS transpose so both the fp32 reads (along H*W)
//     and the byte writes (along C) are contiguous and 16 bytes wide;
//   * load-time packing of E4M3 conv weights [Cout][Cin][KH][KW] into the
//     packed-panel GEMM layout with K ordered (kh, kw, c) and N = Cout.
#include "lcml_internal.hpp"

namespace lcml {
namespace {

constexpr int kPix = 64;   // pixels of the flattened H*W plane per workgroup
constexpr int kPQ = kPix / 4;  // pixel quads per tile
constexpr int kThreads = 256;

typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

// NCHW fp32 -> NHWC E4M3: per image a [C][H*W] -> [H*W][C] transpose with the
// quantiser in between.  Workgroup tile: kPix consecutive pixels x CT
// channels.  Thread t owns pixel quad t % kPQ and channel quads
// t / kPQ + (kThreads / kPQ) j: it reads four
// channel rows x four pixels (one float4 per row when VEC, i.e. H*W % 4 == 0
// and x 16-byte aligned), quantises them, and writes four 32-bit words (one
// pixel's four channels each) into the LDS tile [pixel][channel]; the tile
// then leaves as 16-byte pieces of each pixel's channel run (STORE16: C % 16
// == 0 and y 16-byte aligned; else 32-bit stores, C % 4 == 0).  The x loads
// are issued before the scale is known, so with a dynamic scale the
// reduction of the partial maxima overlaps them.
// grid: (Nb * ceil(HW/kPix), ceil(C/CT))
template <int CT, bool FROM_AMAX, bool VEC, bool STORE16>
__global__ __launch_bounds__(kThreads) void k_quantize_nchw_to_nhwc(const float *__restrict__ x,
                                                                    uint8_t *__restrict__ y, int C, int64_t HW,
                                                                    int tiles_p, const float *__restrict__ scale,
                                                                    const uint32_t *__restrict__ part, int npart,
                                                                    float *__restrict__ scale_out) {
    constexpr int CQP = kThreads / kPQ;  // channel quads per pass
    constexpr int J = CT / 4 / CQP;      // passes
    static_assert(J >= 1 && J * CQP * 4 == CT && (kPix * CT / 16) % kThreads == 0, "tile shape");
    constexpr int PITCH = CT / 4 + 1;   // LDS words per pixel row (odd: writes spread over all banks)
    __shared__ uint32_t tile[kPix * PITCH];
    __shared__ float red[kThreads / 64];
    const int n = blockIdx.x / tiles_p;
    const int64_t p0 = (int64_t)(blockIdx.x - n * tiles_p) * kPix;
    const int c0 = blockIdx.y * CT;
    const int pq = threadIdx.x % kPQ;
    const int64_t p = p0 + 4 * pq;
    const float *xn = x + (int64_t)n * C * HW;
    f4 v[J][4];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int c = c0 + 4 * (threadIdx.x / kPQ + CQP * j);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[j][i] = f4{0.f, 0.f, 0.f, 0.f};
            if (c < C) {  // C % 4 == 0: a channel quad is whole
                const float *row = xn + (int64_t)(c + i) * HW + p;
                if (VEC) {
                    if (p < HW) v[j][i] = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(row));
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (p + e < HW) v[j][i][e] = row[e];
                }
            }
        }
    }
    float s;
    if (FROM_AMAX) {
        s = scale_from_partials<kThreads>(part, npart, red);
        if (scale_out && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *scale_out = s;
    } else {
        s = scale[0];
    }
    const Recip d = make_recip(s);
    auto encode = [&](auto fast) {  // the scale's range test is uniform: one branch
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int cq = threadIdx.x / kPQ + CQP * j;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                tile[(4 * pq + e) * PITCH + cq] =
                    quantize4_t<decltype(fast)::value>(v[j][0][e], v[j][1][e], v[j][2][e], v[j][3][e], d);
        }
    };
    if (d.fast)
        encode(std::true_type{});
    else
        encode(std::false_type{});
    __syncthreads();
    constexpr int CHUNKS = CT / 16;  // 16-byte pieces per pixel
    uint8_t *yn = y + (int64_t)n * HW * C;
#pragma unroll
    for (int k0 = 0; k0 < kPix * CHUNKS; k0 += kThreads) {
        const int k = k0 + threadIdx.x;
        const int pp = k / CHUNKS, ch = k - pp * CHUNKS;
        const int64_t pix = p0 + pp;
        const int cc = c0 + 16 * ch;
        if (pix >= HW || cc >= C) continue;
        const uint32_t *src = &tile[pp * PITCH + 4 * ch];
        uint8_t *dst = yn + pix * C + cc;
        if (STORE16) {
            const u4 w = {src[0], src[1], src[2], src[3]};
            *reinterpret_cast<u4 *>(dst) = w;
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (cc + 4 * q < C) reinterpret_cast<uint32_t *>(dst)[q] = src[q];
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

template <int CT, bool FROM_AMAX>
void launch_nhwc_ct(const float *x, uint8_t *y, int64_t Nb, int C, int64_t HW, bool vec, bool store16,
                    const float *scale, const uint32_t *part, int npart, float *scale_out, hipStream_t s) {
    const int tiles_p = (int)((HW + kPix - 1) / kPix);
    dim3 grid((unsigned)(Nb * tiles_p), (unsigned)((C + CT - 1) / CT));
#define LCML_NHWC(V, S)                                                                                          \
    hipLaunchKernelGGL((k_quantize_nchw_to_nhwc<CT, FROM_AMAX, V, S>), grid, dim3(kThreads), 0, s, x, y, C, HW, \
                       tiles_p, scale, part, npart, scale_out)
    if (vec) {
        if (store16) LCML_NHWC(true, true); else LCML_NHWC(true, false);
    } else {
        if (store16) LCML_NHWC(false, true); else LCML_NHWC(false, false);
    }
#undef LCML_NHWC
}

template <bool FROM_AMAX>
void launch_nhwc(const float *x, uint8_t *y, int64_t Nb, int C, int64_t HW, const float *scale, const uint32_t *part,
                 int npart, float *scale_out, hipStream_t s) {
    const bool vec = HW % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    const bool store16 = C % 16 == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
    if (C % 128 == 0)
        launch_nhwc_ct<128, FROM_AMAX>(x, y, Nb, C, HW, vec, store16, scale, part, npart, scale_out, s);
    else
        launch_nhwc_ct<64, FROM_AMAX>(x, y, Nb, C, HW, vec, store16, scale, part, npart, scale_out, s);
}

}  // namespace

hipError_t launch_quantize_nhwc(const float *x, uint8_t *y, int64_t Nb, int C, int H, int W, const float *scale,
                                const uint32_t *part, int npart, float *scale_out, hipStream_t s) {
    const int64_t HW = (int64_t)H * W;
    if (part)
        launch_nhwc<true>(x, y, Nb, C, HW, scale, part, npart, scale_out, s);
    else
        launch_nhwc<false>(x, y, Nb, C, HW, scale, nullptr, 0, nullptr, s);
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
