// lcml_internal.hpp -- launchers implemented in the .hip files and called by
// the C ABI (capi.hip).  Each returns hipSuccess or the launch error.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lcml_device.hpp"

#include <atomic>

namespace lcml {

hipError_t launch_quantize(const float *x, uint8_t *y, int64_t outer, int64_t axis_len,
                           int64_t inner, const float *scale, hipStream_t s);
hipError_t launch_dequantize(const uint8_t *x, float *y, int64_t outer, int64_t axis_len,
                             int64_t inner, const float *scale, hipStream_t s);
// amax into a zero-initialised uint word (atomic max on fp32 bits)
hipError_t launch_amax(const float *x, int64_t n, uint32_t *amax_bits, hipStream_t s);
// partial maxima (at most kMaxAmaxPartials words at part); *npart = count
constexpr int kMaxAmaxPartials = 1024;
hipError_t launch_amax_partials(const float *x, int64_t n, uint32_t *part, int *npart, hipStream_t s);
// the number of partials launch_amax_partials writes for n elements
int amax_partials_count(int64_t n);
// the encode half of a dynamic quantisation, from npart partial maxima
// (fp32 bits of max |x| over parts covering x) already computed
hipError_t launch_quantize_dynamic_parts(const float *x, uint8_t *y, int64_t n, const uint32_t *part, int npart,
                                         float *scale_out, hipStream_t s);
hipError_t launch_quantize_dynamic(const float *x, uint8_t *y, int64_t n, float *scale_out,
                                   uint32_t *work, hipStream_t s);
hipError_t launch_amax_to_float(const uint32_t *amax_bits, float *out, hipStream_t s);
hipError_t launch_fill_u32(uint32_t *p, uint32_t v, int64_t n, hipStream_t s);

hipError_t launch_pack_weight(const uint8_t *w, int64_t K, int64_t N, int w_is_nk,
                              uint8_t *packed, hipStream_t s);
hipError_t launch_unpack_weight(const uint8_t *packed, int64_t K, int64_t N, int w_is_nk,
                                uint8_t *w, hipStream_t s);

// exact: bf16 MFMAs on widened E4M3 (fp32-accurate); else native FP8 MFMAs
// small_tiles: 128x128 workgroup tiles instead of 256x256
hipError_t launch_gemm_mfma(int64_t M, int64_t N, int64_t K, const uint8_t *a, int64_t lda,
                            const uint8_t *bp, const Epilogue &e, bool exact, hipStream_t s,
                            bool small_tiles = false);
// workgroups of a non-persistent tile GEMM launch (one per tile): with
// e.amax_part set, the number of partial maxima it writes
int64_t gemm_mfma_workgroups(int64_t M, int64_t N, bool small_tiles);
// implicit-im2col FP8 convolution on the MFMA tile kernel: x_nhwc E4M3
// [Nb][H][W][C] ((C/group) % 16 == 0), bp = conv weights packed per group
// with K = (kh, kw, c), output NCHW [Nb][Cout][OH][OW] through the epilogue
// (y, y_bf16; ldy unused; the epilogue's N is Cout/group and its per-channel
// scale and bias pointers cover all Cout channels)
hipError_t launch_conv_mfma(const uint8_t *x_nhwc, int64_t Nb, int C, int H, int W, const uint8_t *bp, int Cout,
                            int KH, int KW, int sh, int sw, int ph, int pw, int dh, int dw, int group, int OH, int OW,
                            const Epilogue &e, bool exact, hipStream_t s,
                            bool small_tiles = false);
// NCHW fp32 -> NHWC E4M3 with a per-tensor scale: scale[0], or amax/448 from
// npart partial maxima when part is given (then written to scale_out if
// non-null)
hipError_t launch_quantize_nhwc(const float *x, uint8_t *y, int64_t Nb, int C, int H, int W, const float *scale,
                                const uint32_t *part, int npart, float *scale_out, hipStream_t s);
// per group g: the packed GEMM weight of W[g*Cout/group ..][Cin_g][KH][KW],
// blocks of packed_weight_bytes(KH*KW*Cin_g, Cout/group) one after another
hipError_t launch_pack_conv_weight(const uint8_t *w, int Cout, int Cin_g, int KH, int KW, int group, uint8_t *packed,
                                   hipStream_t s);
hipError_t launch_gemm_skinny(int64_t M, int64_t N, int64_t K, const uint8_t *a, int64_t lda,
                              const uint8_t *bp, const Epilogue &e, bool exact, hipStream_t s);
// the skinny kernel's 16-row blocks per workgroup (1, 2 or 4) for an M x N
// output over K, and its modelled time in units of one 4-block workgroup's run
int skinny_row_blocks(int64_t M, int64_t N, int64_t K, double *cost);
// fused DynamicQuantizeLinear + skinny GEMM (fp32 activations, M <= 16):
// LDS use is skinny_dynamic_lds_bytes(M, K) <= kSkinnyDynLdsMax
constexpr int64_t kSkinnyDynLdsMax = 128 * 1024 - 32 * 1024;
int64_t skinny_dynamic_lds_bytes(int64_t M, int64_t K);
hipError_t launch_gemm_skinny_dynamic(int64_t M, int64_t N, int64_t K, const float *x, int64_t ldx,
                                      const uint8_t *bp, const Epilogue &e, float *scale_out, bool exact,
                                      hipStream_t s);
hipError_t launch_gemv_valu_f32(int64_t M, int64_t N, int64_t K, const float *a, int64_t lda,
                                const uint8_t *bp, const Epilogue &e, hipStream_t s);
hipError_t launch_gemv_valu_fp8(int64_t M, int64_t N, int64_t K, const uint8_t *a, int64_t lda,
                                const uint8_t *bp, const Epilogue &e, hipStream_t s);

hipError_t launch_sgemm(int64_t M, int64_t N, int64_t K, const float *A, int64_t lda, int transA, const float *B,
                        int64_t ldb, int transB, const Epilogue &e, hipStream_t s);
hipError_t launch_conv2d_f32(const float *x, const float *w, const float *bias, float *y, int64_t Nb, int C, int H,
                             int W, int Cout, int KH, int KW, int sh, int sw, int ph, int pw, int dh, int dw,
                             int group, int OH, int OW, int act, hipStream_t s);
hipError_t launch_activation(const float *x, float *y, int64_t n, int act, hipStream_t s);

// element formats of the fp8 data-type kernels (the ONNX type numbers)
constexpr int kFmtFloat = 1, kFmtE4M3 = 17, kFmtE5M2 = 19;
hipError_t launch_cast(const void *x, int x_fmt, void *y, int y_fmt, int64_t n, hipStream_t s);
hipError_t launch_quantize_e5m2(const float *x, uint8_t *y, int64_t outer, int64_t axis_len, int64_t inner,
                                const float *scale, bool saturate, hipStream_t s);
hipError_t launch_dequantize_e5m2(const uint8_t *x, float *y, int64_t outer, int64_t axis_len, int64_t inner,
                                  const float *scale, hipStream_t s);
// y = a OP b with numpy broadcasting: out_dims[ndim], element strides of a
// and b per output dim (0 where broadcast); ndim <= kMaxBcastDims
constexpr int kMaxBcastDims = 8;
struct BcastGeom {
    int ndim;
    int64_t dims[kMaxBcastDims], sa[kMaxBcastDims], sb[kMaxBcastDims];
};
hipError_t launch_fp8_binary(int op, int fmt, const void *a, const void *b, void *y, int64_t n, bool same_shape,
                             const BcastGeom &g, hipStream_t s);

// read-only stream over bytes (% 16 == 0) of 16-byte aligned p with
// `workgroups` workgroups of 256 threads; sink: one word, written only when
// the fold of the data equals a fixed constant
hipError_t launch_stream_read(const void *p, int64_t bytes, int workgroups, uint32_t *sink, hipStream_t s);

// A kernel's dynamic-LDS limit (hipFuncSetAttribute) is per device: set it
// once per (kernel, device), tracked in `done` (bit d = device d; devices past
// 63 set it on every call).  The call is idempotent, so two threads racing on
// the first launch both succeed.
inline hipError_t ensure_dynamic_lds(const void *fn, int bytes, std::atomic<uint64_t> &done) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return err;
    const uint64_t bit = dev < 64 ? (uint64_t)1 << dev : 0;
    if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
    err = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (err == hipSuccess && bit) done.fetch_or(bit, std::memory_order_release);
    return err;
}

}  // namespace lcml
