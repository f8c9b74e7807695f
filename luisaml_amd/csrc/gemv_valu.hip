// gemv_valu.hip -- small-M FP8-weight linear on the vector ALUs (no MFMA).
//
// Lane l of a wavefront owns output column (panel*64 + l).  In the packed
// layout the 64 columns of a panel store each 16-byte k-chunk side by side,
// so one 128-bit load per lane streams 1 KB of contiguous weights per
// wavefront instruction.  The 16 weights are decoded with v_cvt_pk_f32_fp8
// and folded into per-row fp32 fma chains; the activations are wave-uniform
// and are read through the scalar data cache (constant address space), so
// they occupy SGPR operands instead of VGPRs or LDS bandwidth.  The
// wavefronts of a workgroup split K (16 ways for fp32 activations, 4 for
// E4M3) and sum the partial columns through LDS (a cross-wavefront
// reduction; no cross-lane reduction is needed since a lane owns its
// column).  The K split is what keeps the per-wavefront chain of dependent
// loads short: with four ways, the first layer of the 784-256-128-10 MLP
// (batch 64) took 12 us, latency-bound on 14 chunks per wavefront.
//
// Activations are either fp32 (W8A32: DequantizeLinear(W) -> Gemm with
// unquantised inputs) or E4M3 (W8A8, decoded per chunk).
#include "lcml_internal.hpp"

namespace lcml {
namespace {

// wavefronts per workgroup, which split K: 16 for fp32 activations (113
// VGPRs), 4 for E4M3 ones (their decode needs more registers)
template <bool FP8>
constexpr int kVW = FP8 ? 4 : 16;

typedef float f2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(4))) float cfloat;
typedef const __attribute__((address_space(4))) uint32_t cu32;

struct ValuArgs {
    int64_t M, N, K;
    const void *a;
    int64_t lda;  // elements
    const uint8_t *bp;
    int64_t KC;
    Epilogue e;
};

__device__ inline void decode16(u4 w, float *f) {
    uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        f2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)words[q], false);
        f2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)words[q], true);
        f[q * 4 + 0] = lo.x; f[q * 4 + 1] = lo.y; f[q * 4 + 2] = hi.x; f[q * 4 + 3] = hi.y;
    }
}

// 16 uniform activation values of row m, k-chunk c (zero beyond K) of the
// activations act, row stride lda elements.
template <bool FP8>
__device__ inline void load_act16(const void *act, int64_t lda, int K, int64_t m, int64_t c, float *a) {
    const int64_t k0 = c * 16;
    if (FP8) {
        const uint8_t *row = static_cast<const uint8_t *>(act) + m * lda;
        if (k0 + 16 <= K) {
            cu32 *p = (cu32 *)(uintptr_t)(row + k0);
            u4 w = {p[0], p[1], p[2], p[3]};
            decode16(w, a);
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                f2 v = __builtin_amdgcn_cvt_pk_f32_fp8(k0 + j < K ? (int)row[k0 + j] : 0, false);
                a[j] = v.x;
            }
        }
    } else {
        const float *row = static_cast<const float *>(act) + m * lda;
        if (k0 + 16 <= K) {
            cfloat *p = (cfloat *)(uintptr_t)(row + k0);
#pragma unroll
            for (int j = 0; j < 16; ++j) a[j] = p[j];
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) a[j] = k0 + j < K ? row[k0 + j] : 0.0f;
        }
    }
}

// VMB rows per workgroup (1, 2 or 4; launch_valu chooses).  The values the
// first loads depend on come as leading scalar arguments (the activations
// and their row stride, the packed weights, M, K, the k-chunks per panel),
// and this file is compiled with -amdgpu-kernarg-preload-count=6: they
// arrive in SGPRs at wave start, so the first weight and activation loads
// wait for no kernel-argument fetch.  The struct's copies are not read.
template <bool FP8, int VMB>
__global__ __launch_bounds__(kVW<FP8> * 64) void k_gemv_valu(const void *act, const uint8_t *bp, int64_t lda, int M,
                                                              int K, int kc, ValuArgs g) {
    constexpr int VW = kVW<FP8>;
    static_assert(VMB <= VW, "one wavefront finalises one row");
    __shared__ float red[VW][VMB][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int panel = blockIdx.x;
    const int m0 = (int)blockIdx.y * VMB;
    const int rows = min(VMB, M - m0);
    // this wavefront's k-chunks (kc < 2^27: unsigned, so the divisions are shifts)
    const int c_begin = (int)((uint32_t)(kc * wave) / VW), c_end = (int)((uint32_t)(kc * (wave + 1)) / VW);
    // chunks wholly beyond K hold zero weights; skip them
    const int c_live = (K + 15) / 16;
    const int c_stop = c_end < c_live ? c_end : c_live;

    const uint8_t *wp = bp + (size_t)panel * (size_t)kc * 1024 + lane * 16;
    float acc[VMB];
#pragma unroll
    for (int r = 0; r < VMB; ++r) acc[r] = 0.0f;

    constexpr int U = 4;
    for (int c0 = c_begin; c0 < c_stop; c0 += U) {
        u4 w[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
            w[u] = c0 + u < c_stop
                       ? __builtin_nontemporal_load(reinterpret_cast<const u4 *>(wp + (size_t)(c0 + u) * 1024))
                       : u4{0, 0, 0, 0};
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (c0 + u >= c_stop) break;
            float wf[16];
            decode16(w[u], wf);
#pragma unroll
            for (int r = 0; r < VMB; ++r) {
                if (r >= rows) break;
                float a[16];
                load_act16<FP8>(act, lda, K, m0 + r, c0 + u, a);
#pragma unroll
                for (int j = 0; j < 16; ++j) acc[r] = fmaf(a[j], wf[j], acc[r]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < VMB; ++r) red[wave][r][lane] = acc[r];
    __syncthreads();

    const Epilogue &e = g.e;
    const float a_s = e.a_scale ? e.a_scale[0] : 1.0f;
    const int64_t col = (int64_t)panel * 64 + lane;
    // wave w < VMB finalises row w of the block
    if (wave < VMB && wave < rows && col < e.N) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < VW; ++w) v += red[w][wave][lane];
        const int64_t row = (int64_t)m0 + wave;
        epi_store(e, row, col, epi_value(e, epi_scale(e, a_s, col), row, col, v));
    }
}

template <bool FP8>
hipError_t launch_valu(int64_t M, int64_t N, int64_t K, const void *a, int64_t lda, const uint8_t *bp,
                       const Epilogue &e, hipStream_t s) {
    // the kernel's leading arguments M, K and the k-chunks are 32-bit
    if (M >= ((int64_t)1 << 31) || K >= ((int64_t)1 << 31) - kPackK) return hipErrorInvalidValue;
    ValuArgs g;
    g.M = M; g.N = N; g.K = K; g.a = a; g.lda = lda; g.bp = bp;
    g.KC = pad_to(K, kPackK) / 16;
    g.e = e;
    int64_t npanels = pad_to(N, kPanelCols) / 64;
    // Rows per workgroup: the largest of 4, 2, 1 whose grid still gives every
    // CU a workgroup (every row group re-reads its weight panel, so fewer
    // rows per workgroup only pay where they fill otherwise idle CUs).  On
    // the 784-256-128-10 MLP at batch 64 the three layers run 64/32/16
    // workgroups with 4 rows each: 17.4 us per forward (graph), 10.1 us with
    // one row each (bit-identical: a row's sums do not depend on the grouping).
    constexpr int64_t kFill = 256;
    const int vmb = npanels * ((M + 3) / 4) >= kFill ? 4 : npanels * ((M + 1) / 2) >= kFill ? 2 : 1;
    dim3 grid((unsigned)npanels, (unsigned)((M + vmb - 1) / vmb));
#define LCML_VALU_LEAD g.a, g.bp, g.lda, (int)g.M, (int)g.K, (int)g.KC, g
    if (vmb == 4)
        hipLaunchKernelGGL((k_gemv_valu<FP8, 4>), grid, dim3(kVW<FP8> * 64), 0, s, LCML_VALU_LEAD);
    else if (vmb == 2)
        hipLaunchKernelGGL((k_gemv_valu<FP8, 2>), grid, dim3(kVW<FP8> * 64), 0, s, LCML_VALU_LEAD);
    else
        hipLaunchKernelGGL((k_gemv_valu<FP8, 1>), grid, dim3(kVW<FP8> * 64), 0, s, LCML_VALU_LEAD);
#undef LCML_VALU_LEAD
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemv_valu_f32(int64_t M, int64_t N, int64_t K, const float *a, int64_t lda,
                                const uint8_t *bp, const Epilogue &e, hipStream_t s) {
    return launch_valu<false>(M, N, K, a, lda, bp, e, s);
}

hipError_t launch_gemv_valu_fp8(int64_t M, int64_t N, int64_t K, const uint8_t *a, int64_t lda,
                                const uint8_t *bp, const Epilogue &e, hipStream_t s) {
    return launch_valu<true>(M, N, K, a, lda, bp, e, s);
}

}  // namespace lcml
