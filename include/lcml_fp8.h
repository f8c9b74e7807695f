/*
 * lcml_fp8.h -- C ABI of the MI355X (gfx950) FP8 quantized-linear library
 * (liblcml_fp8.so).
 *
 * This is the drop-in boundary below the C++ operator registry
 * (luisaml_amd/host): the reference ONNX runtime's Gemm / MatMul / Cast /
 * QuantizeLinear / DequantizeLinear operators call into it.  Plain pointers
 * and sizes only: every tensor argument is a DEVICE pointer, every `stream`
 * is a hipStream_t passed as void* (NULL = the default stream).  Calls are
 * asynchronous and stream-ordered; none synchronises the host.
 *
 * Status codes: 0 on success, negative on failure; the message of the last
 * failure on the calling thread is returned by lcml_fp8_last_error().
 *
 * Data conventions
 *   E4M3: OCP float8 E4M3FN, one byte per element, dense, row-major in ONNX
 *         shape order (reference include/onnx/dynamic_array/fp8_data.h:25-43).
 *   Encoder: the reference's saturating round-to-nearest-even
 *         FP8E4M3FN::from_float (include/onnx/fp_quantized.h:149-223):
 *         NaN -> 0x7f, +-0 -> 0x00, |x| > 448 or inf -> sign|0x7e,
 *         otherwise RNE, underflow keeps the sign (0x80).
 *   Decoder: FP8E4M3FN::to_float (fp_quantized.h:226-249); 0x7f/0xff = NaN.
 *   Packed weights: see lcml_fp8_pack_weight.
 */
#ifndef LCML_FP8_H
#define LCML_FP8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define LCML_API __attribute__((visibility("default")))
#else
#define LCML_API
#endif

/* 2: LCML_FP8_DYNAMIC_WORKSPACE_BYTES grew from 256 to 4096 */
#define LCML_FP8_ABI_VERSION 2

/* status codes */
#define LCML_OK 0
#define LCML_ERR_INVALID_ARG (-1)
#define LCML_ERR_UNSUPPORTED (-2)
#define LCML_ERR_HIP (-3)

/* element type codes: the ONNX TensorProto.DataType numbers
 * (reference include/onnx/onnx.h:31-60) */
#define LCML_DTYPE_FLOAT 1
#define LCML_DTYPE_BFLOAT16 16
#define LCML_DTYPE_FLOAT8E4M3FN 17
#define LCML_DTYPE_FLOAT8E5M2 19

/* fused epilogue activations */
#define LCML_ACT_NONE 0
#define LCML_ACT_RELU 1      /* Relu, src/onnx/operators/unary.cpp:85 */
#define LCML_ACT_GELU_ERF 2  /* Gelu approximate="none", gelu.cpp:122-126 */
#define LCML_ACT_GELU_TANH 3 /* Gelu approximate="tanh", gelu.cpp:84-91 */

/* kernel selection for the GEMM entry points.
 * MFMA / SKINNY / VALU meet the reference tolerance (fp32-accurate
 * accumulation; only the summation order differs).  The *_FP8 kernels run
 * gfx950's native FP8 MFMAs at twice the matrix-core rate, but those
 * instructions drop product bits more than ~2^13 below the largest product
 * of each block (relative Frobenius error ~1.4e-5 on N(0,1) data, above the
 * 1e-5 bar), so AUTO never picks them.  AUTO_FP8 is the opt-in: AUTO's
 * choice of tiling, run with the native FP8 twin of that kernel (SKINNY ->
 * SKINNY_FP8, MFMA -> MFMA_FP8, MFMA_128 -> MFMA_128_FP8), for callers that
 * accept the FP8-MFMA precision for twice the large-GEMM rate.  It has no
 * counterpart in the reference, whose Gemm runs fp32 fma chains. */
#define LCML_KERNEL_AUTO 0
#define LCML_KERNEL_MFMA 1       /* 256x256 LDS double-buffered tiles, E4M3 widened to bf16 MFMA */
#define LCML_KERNEL_SKINNY 2     /* small-M: weights streamed to registers, bf16 16x16x32 MFMA */
#define LCML_KERNEL_VALU 3       /* small-M: 128-bit weight streaming, VALU fma, no MFMA */
#define LCML_KERNEL_MFMA_FP8 4   /* as MFMA with v_mfma_f32_32x32x64_f8f6f4 */
#define LCML_KERNEL_SKINNY_FP8 5 /* as SKINNY with v_mfma_f32_16x16x128_f8f6f4 */
#define LCML_KERNEL_MFMA_128 6   /* as MFMA with 128x128 tiles (mid-size GEMMs) */
#define LCML_KERNEL_MFMA_128_FP8 7 /* as MFMA_128 with v_mfma_f32_32x32x64_f8f6f4 */
#define LCML_KERNEL_AUTO_FP8 8   /* AUTO's tiling with the native FP8 MFMA kernels (opt-in) */

/* Message of the last failed call on this thread ("" if none). */
LCML_API const char *lcml_fp8_last_error(void);

/* Names of the kernels this thread launched since the previous call, comma
 * separated in launch order ("gemm_skinny_dynamic", "quantize_dynamic,
 * gemm_mfma_256", ...; entry points that launch fixed kernels are named
 * after themselves), then the record is cleared.  The string stays valid
 * until the thread's next call of this function.  No counterpart in the
 * reference (whose GPU code has no C ABI); the operator layer's execution
 * log (NetworkInstance::enable_logging) reads it per node. */
LCML_API const char *lcml_fp8_kernel_trace(void);

/* LCML_FP8_ABI_VERSION of the loaded library. */
LCML_API int lcml_fp8_abi_version(void);

/*
 * QuantizeLinear, float -> E4M3 (ONNX opset 21, saturate=1, zero point 0):
 *   y[i] = from_float(x[i] / y_scale[a(i)])   (IEEE fp32 divide, bit-exact)
 * The tensor is viewed as [outer, axis_len, inner]; y_scale holds axis_len
 * entries (axis_len == 1: per-tensor scale).
 * Replaces the reference's only float->fp8 conversion, Cast(to=FLOAT8E4M3FN)
 * (src/onnx/operators/cast.cpp:63-67), and adds the QuantizeLinear op that
 * its loader rejects (src/onnx/onnx.cpp:228-229).
 */
LCML_API int lcml_fp8_quantize(const float *x, uint8_t *y, int64_t outer, int64_t axis_len,
                      int64_t inner, const float *y_scale, void *stream);

/*
 * DequantizeLinear, E4M3 -> float:  y[i] = to_float(x[i]) * x_scale[a(i)]
 * (one fp32 multiply, bit-exact).  Same [outer, axis_len, inner] view.
 * Replaces Cast(fp8 -> float) (cast.cpp:44-48) followed by Mul by the scale
 * (src/onnx/operators/binary.cpp:347).
 */
LCML_API int lcml_fp8_dequantize(const uint8_t *x, float *y, int64_t outer, int64_t axis_len,
                        int64_t inner, const float *x_scale, void *stream);

/*
 * Dynamic per-tensor quantisation:  amax = max |x| over non-NaN elements,
 * scale = amax / 448 (1.0 when that is not a positive finite number),
 * y = from_float(x / scale).  Writes the scale to *scale_out (device).
 * workspace: device memory of LCML_FP8_DYNAMIC_WORKSPACE_BYTES (per-workgroup
 * partial maxima, written before they are read: it needs no clearing); may
 * be NULL when n <= LCML_FP8_DYNAMIC_SMALL_MAX (one-launch path).
 * The reference has no dynamic quantiser; its nearest composition would be
 * Abs -> ReduceMax (src/onnx/operators/reduce.cpp:417-459) -> Div -> Cast.
 */
#define LCML_FP8_DYNAMIC_WORKSPACE_BYTES 4096
#define LCML_FP8_DYNAMIC_SMALL_MAX 65536
LCML_API int lcml_fp8_quantize_dynamic(const float *x, uint8_t *y, int64_t n, float *scale_out,
                              void *workspace, void *stream);

/* amax of x over non-NaN elements into *amax_out (device); 0 for n == 0. */
LCML_API int lcml_fp8_amax(const float *x, int64_t n, float *amax_out, void *stream);

/*
 * Weight packing (load time).  The packed layout is "64-column panels of
 * 16-byte k-chunks":  byte (k, n) of the logical [K, N] weight sits at
 *     ((n / 64) * (Kp / 16) + k / 16) * 1024 + (n % 64) * 16 + k % 16
 * with Kp = K rounded up to 128 and N rounded up to 64, padding zero-filled.
 * Every 16-byte unit is one lane's operand chunk of a gfx950 FP8 MFMA
 * (32x32x64 and 16x16x128), so a wavefront's fragment read is
 * lane-contiguous and a column's k-run streams as 128-bit loads.
 * w is [K, N] row-major (MatMul B) when w_is_nk == 0, or [N, K] row-major
 * (Gemm transB=1, the torch Linear layout) when w_is_nk == 1.
 * Replaces the dense FP8 weight binding of
 * src/onnx/network_instance.cpp:215-232 (4-byte padded dense u8).
 */
LCML_API int64_t lcml_fp8_packed_weight_bytes(int64_t K, int64_t N);
LCML_API int lcml_fp8_pack_weight(const uint8_t *w, int64_t K, int64_t N, int w_is_nk, uint8_t *packed,
                         void *stream);
LCML_API int lcml_fp8_unpack_weight(const uint8_t *packed, int64_t K, int64_t N, int w_is_nk,
                           uint8_t *w, void *stream);

/*
 * FP8 GEMM with fused epilogue (W8A8):
 *   acc[m,n] = sum_k to_float(a[m,k]) * to_float(B[k,n])        (fp32)
 *   y[m,n]   = act( alpha * acc * a_scale[0] * b_scale[n|0] + beta * C )
 * a: E4M3 [M, K] row-major with row pitch lda bytes (lda % 16 == 0, a 16-byte
 *    aligned; K % 16 == 0).
 * b_packed: from lcml_fp8_pack_weight (K, N).
 * b_scale: N entries if b_scale_per_channel, else 1.
 * C (optional, may be NULL): fp32 with the reference Gemm broadcast rules
 *    (gemm.cpp:81-103): c_ndim 0 or [1] -> scalar; 1-D of length N -> per
 *    column, other 1-D -> per row; 2-D [c_dim0, c_dim1] with size-1 dims
 *    broadcast.
 * y: y_dtype LCML_DTYPE_FLOAT or LCML_DTYPE_BFLOAT16 (round to nearest
 *    even), row pitch ldy elements.
 * kernel: LCML_KERNEL_* (AUTO picks SKINNY for M <= 16 and MFMA when the
 *    256x256 grid has at least 256 tiles; in between, the cheapest of
 *    SKINNY, MFMA_128 and MFMA by a measured cost model).
 * Replaces the per-thread fma loop nest of Gemm::apply (gemm.cpp:27-325) and
 * MatMul (src/onnx/operators/mat_mul.cpp:51-186) for the DQ->Gemm pattern.
 */
LCML_API int lcml_fp8_gemm(int64_t M, int64_t N, int64_t K, const uint8_t *a, int64_t lda,
                  const float *a_scale, const uint8_t *b_packed, const float *b_scale,
                  int b_scale_per_channel, float alpha, const float *c, int c_ndim,
                  int64_t c_dim0, int64_t c_dim1, float beta, int act, void *y, int y_dtype,
                  int64_t ldy, int kernel, void *stream);

/*
 * Linear with dynamic per-tensor activation quantisation, one call:
 *   s = amax(x) / 448 (1 when that is not a positive finite number),
 *   Y = act( alpha * (DQ(Q(x, s)) x DQ(W)) + beta * C )
 * i.e. DynamicQuantizeLinear(x) -> DequantizeLinear -> Gemm/MatMul with the
 * packed E4M3 weight and its scales, bit-identical to
 * lcml_fp8_quantize_dynamic followed by lcml_fp8_gemm.
 * x: fp32 [M, K] row-major, row pitch ldx elements.
 * With kernel LCML_KERNEL_SKINNY or SKINNY_FP8, M <= 16, x 16-byte aligned,
 * ldx % 4 == 0 and M * (K rounded up to 128, + 16) <= 96 KiB, one fused
 * kernel quantises x on the fly and needs no workspace; LCML_KERNEL_AUTO
 * fuses under the same conditions when also M * K <= 16384 (each workgroup
 * of the fused kernel encodes all of x).  Otherwise x must be
 * contiguous (ldx == K) and the call quantises into `workspace`
 * (lcml_fp8_gemm_dynamic_workspace_bytes(M, K, kernel) bytes) and runs the
 * GEMM selected by `kernel`.  The size query assumes a 16-byte aligned x:
 * where it returns 0 but x is not 16-byte aligned, the call takes the
 * two-step path and needs lcml_fp8_gemm_dynamic_workspace_bytes(M, K,
 * LCML_KERNEL_MFMA) bytes (a smaller workspace is rejected before any
 * launch).
 * x_scale_out: optional device float that receives s.
 * Epilogue arguments and y as for lcml_fp8_gemm.
 * The reference has no dynamic quantiser; this replaces the composition
 * Abs -> ReduceMax (src/onnx/operators/reduce.cpp:417-459) -> Div -> Cast
 * (src/onnx/operators/cast.cpp:63-67) feeding Gemm (gemm.cpp:27-325).
 */
LCML_API int64_t lcml_fp8_gemm_dynamic_workspace_bytes(int64_t M, int64_t K, int kernel);
LCML_API int lcml_fp8_gemm_dynamic(int64_t M, int64_t N, int64_t K, const float *x, int64_t ldx,
                          const uint8_t *b_packed, const float *b_scale, int b_scale_per_channel,
                          float alpha, const float *c, int c_ndim, int64_t c_dim0, int64_t c_dim1,
                          float beta, int act, void *y, int y_dtype, int64_t ldy, float *x_scale_out,
                          void *workspace, int64_t workspace_bytes, int kernel, void *stream);

/*
 * lcml_fp8_gemm_dynamic for a chain of dynamically quantised linears (the
 * fp32 output of one is the next one's input, as the up-projection's GELU
 * output feeds the down-projection): the amax pass over an activation moves
 * into the epilogue that produces it.  No counterpart in the reference
 * (whose composition recomputes ReduceMax over each input).  Arguments as
 * for lcml_fp8_gemm_dynamic, plus:
 * y_amax_part (optional): receives partial maxima of y, *y_amax_npart words
 *   (written by the call, on the host), each the fp32 bits of max |y| over a
 *   part of y (NaN skipped), the parts covering y; y must then be fp32 and
 *   dense (ldy == N) and the buffer hold y_amax_capacity >=
 *   lcml_fp8_amax_parts_max(M, N) words.  The tile kernels write them from
 *   their epilogue (one per workgroup); the other kernels are followed by
 *   an amax pass over y.
 * x_amax_part, x_amax_npart (optional): such partials of x (e.g. a previous
 *   call's y_amax_part): the dynamic scale is amax/448 of their maximum,
 *   computed without a pass over x (the fused small-M kernel still reduces
 *   x itself; the maximum, and so every result, is the same).
 * The results (y, x_scale_out) equal lcml_fp8_gemm_dynamic's bit for bit.
 */
LCML_API int64_t lcml_fp8_amax_parts_max(int64_t M, int64_t N);
LCML_API int lcml_fp8_gemm_dynamic_ex(int64_t M, int64_t N, int64_t K, const float *x, int64_t ldx,
                                      const uint8_t *b_packed, const float *b_scale, int b_scale_per_channel,
                                      float alpha, const float *c, int c_ndim, int64_t c_dim0, int64_t c_dim1,
                                      float beta, int act, void *y, int y_dtype, int64_t ldy, float *x_scale_out,
                                      const uint32_t *x_amax_part, int x_amax_npart, uint32_t *y_amax_part,
                                      int64_t y_amax_capacity, int *y_amax_npart, void *workspace,
                                      int64_t workspace_bytes, int kernel, void *stream);

/*
 * lcml_fp8_gemm_dynamic without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * that forbid allocation, harnesses that count allocations).  No counterpart
 * in the reference.  Same arguments, semantics and results (bit for bit) as
 * lcml_fp8_gemm_dynamic with the workspace arguments removed; where that call
 * would use its workspace (the two-step quantise + GEMM path), this one uses
 * a device array of LCML_FP8_NOALLOC_SCRATCH_BYTES that the library holds on
 * each device it runs on, from the library's load until the process ends.
 * M * K above LCML_FP8_NOALLOC_MAX_ELEMS is rejected with
 * LCML_ERR_UNSUPPORTED before anything runs.  The call allocates nothing and
 * needs no clearing of the array (every byte it reads there it wrote first
 * in the same call); calls that overlap on one device share the array and
 * race, so issue them on one stream (or order them) per device.
 */
#define LCML_FP8_NOALLOC_MAX_ELEMS 16777216
#define LCML_FP8_NOALLOC_SCRATCH_BYTES (LCML_FP8_NOALLOC_MAX_ELEMS + LCML_FP8_DYNAMIC_WORKSPACE_BYTES + 256)
LCML_API int lcml_fp8_gemm_dynamic_noalloc(int64_t M, int64_t N, int64_t K, const float *x, int64_t ldx,
                                           const uint8_t *b_packed, const float *b_scale, int b_scale_per_channel,
                                           float alpha, const float *c, int c_ndim, int64_t c_dim0, int64_t c_dim1,
                                           float beta, int act, void *y, int y_dtype, int64_t ldy,
                                           float *x_scale_out, int kernel, void *stream);

/*
 * QuantizeLinear of an NCHW fp32 activation [n, c, h, w] with one per-tensor
 * scale, written in NHWC order (y[n][h][w][c], E4M3) for lcml_fp8_conv2d.
 * y_scale: device float; NULL selects the dynamic scale amax/448 (1 when
 *   that is not a positive finite number), written to scale_out (required)
 *   and computed with `workspace` (LCML_FP8_DYNAMIC_WORKSPACE_BYTES).
 * c % 4 == 0.  Same codes as lcml_fp8_quantize on the same values (the
 * reference encoder of fp_quantized.h:149-223 on x / scale); only the order
 * of the output bytes differs.
 */
LCML_API int lcml_fp8_quantize_nhwc(const float *x, uint8_t *y, int64_t n, int64_t c, int64_t h, int64_t w,
                           const float *y_scale, float *scale_out, void *workspace, void *stream);

/*
 * Conv weights: E4M3 [cout][cin/group][kh][kw] (ONNX Conv W layout, dense)
 * packed for lcml_fp8_conv2d.  For each group g (output channels
 * g*cout/group ..), the GEMM weight with reduction index
 * k = (kh*KW + kw)*cin_g + c (the reference Conv's loop order kh, kw, then
 * channels, src/onnx/operators/conv.cpp:143-192) and cout/group columns, in
 * the lcml_fp8_pack_weight panel layout; the groups' blocks follow one
 * another.  Size: lcml_fp8_packed_conv_weight_bytes(...) =
 * group * lcml_fp8_packed_weight_bytes(kh*kw*cin_g, cout/group).
 * cin_g = input channels per group.
 */
LCML_API int64_t lcml_fp8_packed_conv_weight_bytes(int64_t cout, int64_t cin_g, int64_t kh, int64_t kw,
                                          int64_t group);
LCML_API int lcml_fp8_pack_conv_weight(const uint8_t *w, int64_t cout, int64_t cin_g, int64_t kh, int64_t kw,
                              int64_t group, uint8_t *packed, void *stream);

/*
 * 2-D convolution with E4M3 input and weights, fp32 accumulation, as an
 * implicit-im2col GEMM on the matrix cores (no im2col buffer):
 *   y[n][co][oh][ow] = act( x_scale * w_scale[co|0] *
 *        sum_{kh,kw,c} x[n][oh*sh - ph + kh*dh][ow*sw - pw + kw*dw][c] * w[co][c][kh][kw]
 *        + bias[co] )
 * with out-of-range input positions contributing zero.  pad_h/pad_w are the
 * BEGIN pads (the reference applies only those, conv.cpp:121; end pads only
 * enter through the output size oh x ow, which the caller passes).
 * x_nhwc: lcml_fp8_quantize_nhwc output; group divides c and cout, and
 * (c/group) % 16 == 0 (group g reads channels g*c/group .. and writes output
 * channels g*cout/group .., conv.cpp:139,158).
 * w_packed: lcml_fp8_pack_conv_weight output.  bias: cout floats or NULL.
 * y: NCHW [n][cout][oh][ow], y_dtype LCML_DTYPE_FLOAT or BFLOAT16.
 * kernel: LCML_KERNEL_AUTO / MFMA / MFMA_128 (exact bf16 matrix cores,
 *    256x256 or 128x128 tiles) or MFMA_FP8 / MFMA_128_FP8 / AUTO_FP8; AUTO
 *    takes the 128x128 tiles when the 256x256 grid (times the groups) is
 *    small, AUTO_FP8 the same tiles with the native FP8 MFMAs.
 * Replaces Conv::apply (src/onnx/operators/conv.cpp:115-207) for the
 * DQ(x), DQ(W) -> Conv [-> Relu/Gelu] pattern.
 */
LCML_API int lcml_fp8_conv2d(const uint8_t *x_nhwc, const float *x_scale, int64_t n, int64_t c, int64_t h,
                    int64_t w, const uint8_t *w_packed, const float *w_scale, int w_scale_per_channel,
                    int64_t cout, int64_t kh, int64_t kw, int64_t stride_h, int64_t stride_w, int64_t pad_h,
                    int64_t pad_w, int64_t dil_h, int64_t dil_w, int64_t group, int64_t oh, int64_t ow,
                    const float *bias, int act, void *y, int y_dtype, int kernel, void *stream);

/*
 * W8A32 linear: fp32 activations times packed E4M3 weights, same epilogue:
 *   y[m,n] = act( alpha * (sum_k a[m,k] * to_float(B[k,n])) * b_scale[n|0]
 *                 + beta * C )
 * a: fp32 [M, K] row-major, row pitch lda elements (lda % 4 == 0).
 * This is the reference graph DequantizeLinear(W) -> Gemm with unquantised
 * activations (the 3-layer MLP).  Runs the VALU kernel (no MFMA).
 */
LCML_API int lcml_fp8_gemm_w8a32(int64_t M, int64_t N, int64_t K, const float *a, int64_t lda,
                        const uint8_t *b_packed, const float *b_scale, int b_scale_per_channel,
                        float alpha, const float *c, int c_ndim, int64_t c_dim0,
                        int64_t c_dim1, float beta, int act, void *y, int y_dtype, int64_t ldy,
                        void *stream);

/*
 * Plain fp32 Gemm for graphs that stay in fp32 (no FP8 pattern to fuse):
 * Y = act(alpha * op(A) op(B) + beta * C), op = transpose when trans_*;
 * every output is one sequential fma chain over k from 0, exactly the
 * reference's scalar Gemm order (src/onnx/operators/gemm.cpp:155-162).
 * a: [M,K] (or [K,M] when trans_a) with row pitch lda; b: [K,N] (or [N,K]
 * when trans_b) with row pitch ldb; C and y as in lcml_fp8_gemm.
 */
/*
 * Plain fp32 2-D convolution for graphs that stay in fp32 (the reference
 * Conv::apply, src/onnx/operators/conv.cpp:115-207): x NCHW, w
 * [cout][c/group][kh][kw], bias (cout floats or NULL), y NCHW fp32
 * [n][cout][oh][ow]; begin pads, strides, dilations, groups; one sequential
 * fma chain per output over (kh, kw, channel).
 */
LCML_API int lcml_fp8_conv2d_f32(const float *x, const float *w, const float *bias, float *y, int64_t n, int64_t c,
                        int64_t h, int64_t wd, int64_t cout, int64_t kh, int64_t kw, int64_t stride_h,
                        int64_t stride_w, int64_t pad_h, int64_t pad_w, int64_t dil_h, int64_t dil_w,
                        int64_t group, int64_t oh, int64_t ow, int act, void *stream);

LCML_API int lcml_fp8_sgemm(int64_t M, int64_t N, int64_t K, const float *a, int64_t lda, int trans_a,
                            const float *b, int64_t ldb, int trans_b, float alpha, const float *c, int c_ndim,
                            int64_t c_dim0, int64_t c_dim1, float beta, int act, void *y, int y_dtype,
                            int64_t ldy, void *stream);

/*
 * Elementwise fp32 activation y = act(x) for an unfused Relu
 * (src/onnx/operators/unary.cpp:85) or Gelu (src/onnx/operators/gelu.cpp:
 * 84-91, 122-126); act is LCML_ACT_*.  y may equal x.
 */
LCML_API int lcml_fp8_activation(const float *x, float *y, int64_t n, int act, void *stream);

/*
 * Cast between LCML_DTYPE_FLOAT, FLOAT8E4M3FN and FLOAT8E5M2 (n elements;
 * x and y may not overlap unless equal in size per element and identical).
 * float -> fp8: the reference's CPU encoders, FP8E4M3FN::from_float
 * (saturating to +-448) and FP8E5M2::from_float (|x| > 57344 -> +-inf),
 * include/onnx/fp_quantized.h:149-223, 272-346; fp8 -> float: to_float
 * (226-249, 350-377); fp8 -> fp8 through the exact float value.  Replaces
 * Cast::apply's fp8 branches (src/onnx/operators/cast.cpp:39-77), whose
 * float -> fp8 direction goes through half first; `saturate` is not an
 * argument because that op reads it only for float -> int (cast.cpp:86-98).
 */
LCML_API int lcml_fp8_cast(const void *x, int x_dtype, void *y, int y_dtype, int64_t n, void *stream);

/*
 * QuantizeLinear / DequantizeLinear with a FLOAT8E5M2 tensor (ONNX opset 21,
 * zero point 0), same [outer, axis_len, inner] view as lcml_fp8_quantize:
 *   y = from_float_e5m2(x / y_scale) (IEEE fp32 divide), where saturate = 1
 *       first clamps |x / y_scale| > 57344 (inf included) to +-57344 and
 *       saturate = 0 keeps the encoder's +-inf;
 *   y = to_float_e5m2(x) * x_scale.
 * No counterpart in the reference (its loader rejects both ops,
 * src/onnx/onnx.cpp:228-229); the numeric core is FP8E5M2.
 */
LCML_API int lcml_fp8_quantize_e5m2(const float *x, uint8_t *y, int64_t outer, int64_t axis_len, int64_t inner,
                                    const float *y_scale, int saturate, void *stream);
LCML_API int lcml_fp8_dequantize_e5m2(const uint8_t *x, float *y, int64_t outer, int64_t axis_len,
                                      int64_t inner, const float *x_scale, void *stream);

/*
 * Elementwise binary op, y = a OP b, with numpy broadcasting (shapes are
 * right-aligned, size-1 dimensions broadcast; y_shape must be the
 * broadcast shape; at most 8 dimensions; shapes are HOST arrays, data
 * device pointers).  dtype: LCML_DTYPE_FLOAT (the op in fp32),
 * FLOAT8E4M3FN or FLOAT8E5M2 (all three tensors of that type): as the
 * reference's Binary ops on quantised tensors
 * (src/onnx/operators/binary.cpp:184-285), both operands are decoded, the
 * op is rounded to half precision (the reference computes in half) and the
 * result is encoded with the format's from_float.
 * Replaces Add / Sub / Mul / Div (binary.cpp:335-345) on the fp8 path.
 */
#define LCML_BINARY_ADD 0
#define LCML_BINARY_SUB 1
#define LCML_BINARY_MUL 2
#define LCML_BINARY_DIV 3
LCML_API int lcml_fp8_binary(int op, int dtype, const void *a, const int64_t *a_shape, int a_ndim, const void *b,
                             const int64_t *b_shape, int b_ndim, void *y, const int64_t *y_shape, int y_ndim,
                             void *stream);

/*
 * Measurement aid, no counterpart in the reference: reads `bytes` bytes
 * (a multiple of 16) at 16-byte aligned device pointer p with `workgroups`
 * workgroups of 512 threads, each streaming one contiguous, equal share
 * (below 2 GiB) with non-temporal loads, and does nothing else (`sink`: one
 * device word, written only when a fold of the data equals a fixed
 * constant).  Its time
 * over a buffer is the HBM read floor that the bandwidth-bound small-M GEMM
 * (which reads the same weight bytes once) is compared with.
 */
LCML_API int lcml_fp8_stream_read(const void *p, int64_t bytes, int workgroups, uint32_t *sink, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* LCML_FP8_H */
