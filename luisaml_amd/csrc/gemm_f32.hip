// gemm_f32.hip -- plain fp32 Gemm and elementwise activations, used by the
// operator layer for graphs that are not (or cannot be) fused into the FP8
// path: an fp32 Gemm/MatMul, a standalone Relu/Gelu.
//
// The Gemm keeps the reference's arithmetic exactly: every output is one
// sequential fma chain over k from 0 (src/onnx/operators/gemm.cpp:155-162),
// then alpha, then beta*C with the reference broadcast, then the activation.
// 64x64 output tile per 256-thread workgroup, 4x4 outputs per thread, K
// staged through LDS 16 at a time (the chain order over k is unchanged).
#include "lcml_internal.hpp"

namespace lcml {
namespace {

constexpr int TM = 64, TN = 64, TK = 16;

__global__ __launch_bounds__(256) void k_sgemm(int64_t M, int64_t N, int64_t K, const float *__restrict__ A,
                                               int64_t lda, int transA, const float *__restrict__ B, int64_t ldb,
                                               int transB, Epilogue e) {
    __shared__ float sa[TK][TM + 1];
    __shared__ float sb[TK][TN + 1];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int64_t m0 = (int64_t)blockIdx.y * TM, n0 = (int64_t)blockIdx.x * TN;
    float acc[4][4] = {};
    for (int64_t k0 = 0; k0 < K; k0 += TK) {
        for (int i = threadIdx.x; i < TK * TM; i += 256) {
            const int kk = i / TM, mm = i % TM;
            const int64_t m = m0 + mm, k = k0 + kk;
            sa[kk][mm] = (m < M && k < K) ? (transA ? A[k * lda + m] : A[m * lda + k]) : 0.0f;
        }
        for (int i = threadIdx.x; i < TK * TN; i += 256) {
            const int kk = i / TN, nn = i % TN;
            const int64_t n = n0 + nn, k = k0 + kk;
            sb[kk][nn] = (n < N && k < K) ? (transB ? B[n * ldb + k] : B[k * ldb + n]) : 0.0f;
        }
        __syncthreads();
        const int kmax = (int)((K - k0) < TK ? (K - k0) : TK);
        for (int kk = 0; kk < kmax; ++kk)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(sa[kk][ty * 4 + i], sb[kk][tx * 4 + j], acc[i][j]);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t m = m0 + ty * 4 + i;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t n = n0 + tx * 4 + j;
            if (n < N) epi_store(e, m, n, epi_value(e, 1.0f, m, n, acc[i][j]));
        }
    }
}

__global__ __launch_bounds__(256) void k_activation(const float *__restrict__ x, float *__restrict__ y, int64_t n,
                                                    int act) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        y[i] = apply_act(x[i], act);
}

// Direct fp32 NCHW convolution, one thread per output element, one fma
// chain per output in the reference Conv's reduction order (kh, kw, then the
// group's input channels; conv.cpp:143-192, whose 4-wide partial sums differ
// from this chain only in fp32 rounding), begin pads only (conv.cpp:121),
// dilation, groups, bias, activation.
__global__ __launch_bounds__(256) void k_conv2d_f32(const float *__restrict__ x, const float *__restrict__ w,
                                                    const float *__restrict__ bias, float *__restrict__ y, int C,
                                                    int H, int W, int Cout, int KH, int KW, int sh, int sw, int ph,
                                                    int pw, int dh, int dw, int group, int OH, int OW, int act,
                                                    int64_t total) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int ow = (int)(i % OW);
    const int oh = (int)((i / OW) % OH);
    const int co = (int)((i / ((int64_t)OW * OH)) % Cout);
    const int64_t n = i / ((int64_t)OW * OH * Cout);
    const int cg = C / group, mg = Cout / group, g = co / mg;
    const float *xn = x + (n * C + (int64_t)g * cg) * H * W;
    const float *wc = w + (int64_t)co * cg * KH * KW;
    float sum = 0.0f;
    for (int kh = 0; kh < KH; ++kh) {
        const int ih = oh * sh + kh * dh - ph;
        if ((unsigned)ih >= (unsigned)H) continue;
        for (int kw = 0; kw < KW; ++kw) {
            const int iw = ow * sw + kw * dw - pw;
            if ((unsigned)iw >= (unsigned)W) continue;
            for (int c = 0; c < cg; ++c)
                sum = fmaf(xn[((int64_t)c * H + ih) * W + iw], wc[((int64_t)c * KH + kh) * KW + kw], sum);
        }
    }
    if (bias) sum += bias[co];
    y[i] = apply_act(sum, act);
}

}  // namespace

hipError_t launch_conv2d_f32(const float *x, const float *w, const float *bias, float *y, int64_t Nb, int C, int H,
                             int W, int Cout, int KH, int KW, int sh, int sw, int ph, int pw, int dh, int dw,
                             int group, int OH, int OW, int act, hipStream_t s) {
    const int64_t total = Nb * Cout * OH * OW;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(k_conv2d_f32, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, x, w, bias, y, C, H, W,
                       Cout, KH, KW, sh, sw, ph, pw, dh, dw, group, OH, OW, act, total);
    return hipGetLastError();
}

hipError_t launch_sgemm(int64_t M, int64_t N, int64_t K, const float *A, int64_t lda, int transA, const float *B,
                        int64_t ldb, int transB, const Epilogue &e, hipStream_t s) {
    dim3 grid((unsigned)((N + TN - 1) / TN), (unsigned)((M + TM - 1) / TM));
    hipLaunchKernelGGL(k_sgemm, grid, dim3(256), 0, s, M, N, K, A, lda, transA, B, ldb, transB, e);
    return hipGetLastError();
}

hipError_t launch_activation(const float *x, float *y, int64_t n, int act, hipStream_t s) {
    int64_t g = (n + 255) / 256;
    g = g < 1 ? 1 : (g > 4096 ? 4096 : g);
    hipLaunchKernelGGL(k_activation, dim3((unsigned)g), dim3(256), 0, s, x, y, n, act);
    return hipGetLastError();
}

}  // namespace lcml
