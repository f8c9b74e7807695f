// capi.hip -- the extern "C" boundary (include/lcml_fp8.h): argument
// validation, kernel selection and error reporting.  No entry point
// synchronises the host or allocates device memory.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>

#include "../../include/lcml_fp8.h"
#include "lcml_internal.hpp"

namespace {

thread_local char g_err[512] = "";
// names of the kernels launched on this thread since the last
// lcml_fp8_kernel_trace() call, comma separated (truncated when full)
thread_local char g_trace[1024] = "";
thread_local char g_trace_out[1024] = "";
thread_local size_t g_trace_len = 0;

void note(const char *label) {
    const size_t n = strlen(label), sep = g_trace_len ? 2 : 0;
    if (g_trace_len + sep + n + 1 > sizeof(g_trace)) return;
    if (sep) memcpy(g_trace + g_trace_len, ", ", 2);
    memcpy(g_trace + g_trace_len + sep, label, n + 1);
    g_trace_len += sep + n;
}

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

// a launch's status; on success the launch is noted in the kernel trace
// under `label` (the entry point's name when none is given)
int hip_status(hipError_t err, const char *what, const char *label = nullptr) {
    if (err == hipSuccess) {
        note(label ? label : what);
        return LCML_OK;
    }
    return fail(LCML_ERR_HIP, "%s: %s", what, hipGetErrorString(err));
}

bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int check_view(int64_t outer, int64_t axis_len, int64_t inner, const char *fn) {
    if (outer < 0 || axis_len < 1 || inner < 0)
        return fail(LCML_ERR_INVALID_ARG, "%s: invalid view [outer=%lld, axis_len=%lld, inner=%lld]", fn,
                    (long long)outer, (long long)axis_len, (long long)inner);
    return LCML_OK;
}

// Shared validation of the GEMM epilogue arguments.
int make_epilogue(lcml::Epilogue &e, const char *fn, int64_t M, int64_t N, const float *a_scale,
                  const float *b_scale, int per_channel, float alpha, const float *c, int c_ndim,
                  int64_t c0, int64_t c1, float beta, int act, void *y, int y_dtype, int64_t ldy,
                  bool scales_optional = false) {
    if (!b_scale && !scales_optional) return fail(LCML_ERR_INVALID_ARG, "%s: b_scale is NULL", fn);
    if (!y && M > 0 && N > 0) return fail(LCML_ERR_INVALID_ARG, "%s: y is NULL", fn);
    if (y_dtype != LCML_DTYPE_FLOAT && y_dtype != LCML_DTYPE_BFLOAT16)
        return fail(LCML_ERR_UNSUPPORTED, "%s: output dtype %d (FLOAT=1 or BFLOAT16=16 supported)", fn, y_dtype);
    if (ldy < N) return fail(LCML_ERR_INVALID_ARG, "%s: ldy=%lld < N=%lld", fn, (long long)ldy, (long long)N);
    if (act < LCML_ACT_NONE || act > LCML_ACT_GELU_TANH)
        return fail(LCML_ERR_UNSUPPORTED, "%s: activation %d", fn, act);
    const bool has_c = c != nullptr && beta != 0.0f;
    if (has_c) {
        if (c_ndim < 0 || c_ndim > 2) return fail(LCML_ERR_INVALID_ARG, "%s: C ndim %d", fn, c_ndim);
        if (c_ndim == 1 && !(c0 == 1 || c0 == N || c0 == M))
            return fail(LCML_ERR_INVALID_ARG, "%s: 1-D C of length %lld broadcasts to neither N nor M", fn,
                        (long long)c0);
        if (c_ndim == 2 && (!(c0 == 1 || c0 == M) || !(c1 == 1 || c1 == N)))
            return fail(LCML_ERR_INVALID_ARG, "%s: C shape [%lld, %lld] does not broadcast to [%lld, %lld]",
                        fn, (long long)c0, (long long)c1, (long long)M, (long long)N);
    }
    e.a_scale = a_scale;
    e.b_scale = b_scale;
    e.b_per_channel = per_channel ? 1 : 0;
    e.alpha = alpha;
    e.c = has_c ? c : nullptr;
    e.c_ndim = c_ndim;
    e.c0 = c0;
    e.c1 = c1;
    e.beta = beta;
    e.act = act;
    e.y = y;
    e.y_bf16 = y_dtype == LCML_DTYPE_BFLOAT16;
    e.ldy = ldy;
    e.M = M;
    e.N = N;
    e.amax_part = nullptr;
    return LCML_OK;
}

}  // namespace

extern "C" {

const char *lcml_fp8_last_error(void) { return g_err; }

const char *lcml_fp8_kernel_trace(void) {
    memcpy(g_trace_out, g_trace, g_trace_len + 1);
    g_trace[0] = 0;
    g_trace_len = 0;
    return g_trace_out;
}

int lcml_fp8_abi_version(void) { return LCML_FP8_ABI_VERSION; }

int lcml_fp8_quantize(const float *x, uint8_t *y, int64_t outer, int64_t axis_len, int64_t inner,
                      const float *y_scale, void *stream) {
    if (int rc = check_view(outer, axis_len, inner, "lcml_fp8_quantize")) return rc;
    if (outer * axis_len * inner == 0) return LCML_OK;
    if (!x || !y || !y_scale) return fail(LCML_ERR_INVALID_ARG, "lcml_fp8_quantize: NULL pointer");
    return hip_status(lcml::launch_quantize(x, y, outer, axis_len, inner, y_scale, (hipStream_t)stream),
                      "lcml_fp8_quantize");
}

int lcml_fp8_dequantize(const uint8_t *x, float *y, int64_t outer, int64_t axis_len, int64_t inner,
                        const float *x_scale, void *stream) {
    if (int rc = check_view(outer, axis_len, inner, "lcml_fp8_dequantize")) return rc;
    if (outer * axis_len * inner == 0) return LCML_OK;
    if (!x || !y || !x_scale) return fail(LCML_ERR_INVALID_ARG, "lcml_fp8_dequantize: NULL pointer");
    return hip_status(lcml::launch_dequantize(x, y, outer, axis_len, inner, x_scale, (hipStream_t)stream),
                      "lcml_fp8_dequantize");
}

int lcml_fp8_quantize_dynamic(const float *x, uint8_t *y, int64_t n, float *scale_out, void *workspace,
                              void *stream) {
    if (n < 0) return fail(LCML_ERR_INVALID_ARG, "lcml_fp8_quantize_dynamic: n < 0");
    if (!scale_out) return fail(LCML_ERR_INVALID_ARG, "lcml_fp8_quantize_dynamic: scale_out is NULL");
    if (n > 0 && (!x || !y)) return fail(LCML_ERR_INVALID_ARG, "lcml_fp8_quantize_dynamic: NULL pointer");
    if (n > LCML_FP8_DYNAMIC_SMALL_MAX && !workspace)
        return fail(LCML_ERR_INVALID_ARG,
                    "lcml_fp8_quantize_dynamic: n=%lld needs a workspace of %d bytes", (long long)n,
                    LCML_FP8_DYNAMIC_WORKSPACE_BYTES);
    return hip_status(lcml::launch_quantize_dynamic(x, y, n, scale_out, static_cast<uint32_t *>(workspace),
                                                    (hipStream_t)stream),
                      "lcml_fp8_quantize_dynamic");
}

int lcml_fp8_amax(const float *x, int64_t n, float *amax_out, void *stream) {
    if (n < 0 || !amax_out || (n > 0 && !x)) return fail(LCML_ERR_INVALID_ARG, "lcml_fp8_amax: bad argument");
    // The amax word is amax_out itself (fp32 bits of a non-negative float).
    hipStream_t s = (hipStream_t)stream;
    uint32_t *word = reinterpret_cast<uint32_t *>(amax_out);
    hipError_t err = lcml::launch_fill_u32(word, 0u, 1, s);
    if (err == hipSuccess && n > 0) err = lcml::launch_amax(x, n, word, s);
    return hip_status(err, "lcml_fp8_amax");
}

int64_t lcml_fp8_packed_weight_bytes(int64_t K, int64_t N) {
    if (K <= 0 || N <= 0) return 0;
    return lcml::pad_to(K, lcml::kPackK) * lcml::pad_to(N, lcml::kPanelCols);
}

int lcml_fp8_pack_weight(const uint8_t *w, int64_t K, int64_t N, int w_is_nk, uint8_t *packed,
                         void *stream) {
    if (K <= 0 || N <= 0 || !w || !packed)
        return fail(LCML_ERR_INVALID_ARG, "lcml_fp8_pack_weight: bad argument (K=%lld N=%lld)", (long long)K,
                    (long long)N);
    if (!aligned(packed, 16)) return fail(LCML_ERR_INVALID_ARG, "lcml_fp8_pack_weight: packed not 16-byte aligned");
    return hip_status(lcml::launch_pack_weight(w, K, N, w_is_nk, packed, (hipStream_t)stream),
                      "lcml_fp8_pack_weight");
}

int lcml_fp8_unpack_weight(const uint8_t *packed, int64_t K, int64_t N, int w_is_nk, uint8_t *w,
                           void *stream) {
    if (K <= 0 || N <= 0 || !w || !packed)
        return fail(LCML_ERR_INVALID_ARG, "lcml_fp8_unpack_weight: bad argument");
    if (!aligned(packed, 16)) return fail(LCML_ERR_INVALID_ARG, "lcml_fp8_unpack_weight: packed not 16-byte aligned");
    return hip_status(lcml::launch_unpack_weight(packed, K, N, w_is_nk, w, (hipStream_t)stream),
                      "lcml_fp8_unpack_weight");
}

namespace {
// AUTO's kernel for an M x N x K GEMM.  All times grow about linearly in K;
// in units of one skinny workgroup with 4 row blocks (19 us at K = 4096,
// 38 us at K = 11008), measured on 4096x11008, 11008x4096 and 4096x4096:
//   * 256x256 tiles: one round of up to 256 tiles takes 4.5 units;
//   * 128x128 tiles: 2.2 units per 256 tiles (two workgroups share a CU);
//   * the skinny kernel: lcml::skinny_row_blocks.
// M <= 16 always takes the skinny kernel; a 256x256 grid of at least 256
// tiles keeps the 256x256 kernel.  Examples: 4096x11008 at M = 512: 128x128
// tiles 64 us against 83 (skinny) and 93 (256x256); 4096x4096 at M = 1024:
// 46 us against 66 and 91; 11008x4096 at M = 512: skinny 73 us against 91.
// the native-FP8 kernel of the same tiling (LCML_KERNEL_AUTO_FP8)
int fp8_twin(int kernel) {
    switch (kernel) {
    case LCML_KERNEL_MFMA: return LCML_KERNEL_MFMA_FP8;
    case LCML_KERNEL_MFMA_128: return LCML_KERNEL_MFMA_128_FP8;
    case LCML_KERNEL_SKINNY: return LCML_KERNEL_SKINNY_FP8;
    default: return kernel;
    }
}

// the kernel trace's name of a resolved GEMM kernel choice
const char *kernel_label(int kernel) {
    switch (kernel) {
    case LCML_KERNEL_MFMA: return "gemm_mfma_256";
    case LCML_KERNEL_MFMA_FP8: return "gemm_mfma_256_fp8";
    case LCML_KERNEL_MFMA_128: return "gemm_mfma_128";
    case LCML_KERNEL_MFMA_128_FP8: return "gemm_mfma_128_fp8";
    case LCML_KERNEL_SKINNY: return "gemm_skinny";
    case LCML_KERNEL_SKINNY_FP8: return "gemm_skinny_fp8";
    case LCML_KERNEL_VALU: return "gemv_valu";
    default: return "gemm";
    }
}

int auto_gemm_kernel(int64_t M, int64_t N, int64_t K) {
    if (M <= 16) return LCML_KERNEL_SKINNY;
    const int64_t tiles = (M + 255) / 256 * ((N + 255) / 256);
    if (tiles >= 256) return LCML_KERNEL_MFMA;
    double skinny = 0;
    lcml::skinny_row_blocks(M, N, K, &skinny);
    const double t128 = (double)((M + 127) / 128 * ((N + 127) / 128));
    const double small = 2.2 * (t128 > 256 ? t128 / 256 : 1.0);
    if (skinny <= small && skinny < 4.5) return LCML_KERNEL_SKINNY;
    return small < 4.5 ? LCML_KERNEL_MFMA_128 : LCML_KERNEL_MFMA;
}
}  // namespace

namespace {
// Amax partials of y (optional, y_amax_part non-null): the caller checked
// y is fp32, dense (ldy == N) and the buffer holds lcml_fp8_amax_parts_max
// words; *y_amax_npart receives the count written.
struct YAmax {
    uint32_t *part = nullptr;
    int *npart = nullptr;
};

// lcml_fp8_gemm with an optional amax-partials output
int gemm_core(const char *fn, int64_t M, int64_t N, int64_t K, const uint8_t *a, int64_t lda, const float *a_scale,
              const uint8_t *b_packed, const float *b_scale, int b_scale_per_channel, float alpha, const float *c,
              int c_ndim, int64_t c_dim0, int64_t c_dim1, float beta, int act, void *y, int y_dtype, int64_t ldy,
              int kernel, void *stream, YAmax ya) {
    if (M < 0 || N <= 0 || K <= 0) return fail(LCML_ERR_INVALID_ARG, "%s: M=%lld N=%lld K=%lld", fn,
                                               (long long)M, (long long)N, (long long)K);
    lcml::Epilogue e;
    if (int rc = make_epilogue(e, fn, M, N, a_scale, b_scale, b_scale_per_channel, alpha, c, c_ndim, c_dim0,
                               c_dim1, beta, act, y, y_dtype, ldy))
        return rc;
    if (M == 0) {
        if (ya.npart) *ya.npart = 0;
        return LCML_OK;
    }
    if (!a || !b_packed) return fail(LCML_ERR_INVALID_ARG, "%s: NULL operand", fn);
    if (K % 16 != 0) return fail(LCML_ERR_UNSUPPORTED, "%s: K=%lld is not a multiple of 16", fn, (long long)K);
    if (lda < K || lda % 16 != 0 || !aligned(a, 16))
        return fail(LCML_ERR_INVALID_ARG, "%s: a must be 16-byte aligned with lda >= K, lda %% 16 == 0", fn);
    if (!aligned(b_packed, 16)) return fail(LCML_ERR_INVALID_ARG, "%s: b_packed not 16-byte aligned", fn);
    hipStream_t s = (hipStream_t)stream;
    if (kernel == LCML_KERNEL_AUTO) kernel = auto_gemm_kernel(M, N, K);
    if (kernel == LCML_KERNEL_AUTO_FP8) kernel = fp8_twin(auto_gemm_kernel(M, N, K));
    hipError_t err;
    const char *label = kernel_label(kernel);
    switch (kernel) {
    case LCML_KERNEL_MFMA:
    case LCML_KERNEL_MFMA_FP8:
    case LCML_KERNEL_MFMA_128:
    case LCML_KERNEL_MFMA_128_FP8:
        // buffer offsets are 32-bit with 0x80000000 as the out-of-range marker
        if ((M - 1) * lda + K >= (int64_t)0x80000000 || lcml_fp8_packed_weight_bytes(K, N) >= (int64_t)0x80000000)
            return fail(LCML_ERR_UNSUPPORTED, "%s: operand larger than 2 GiB for the MFMA kernel", fn);
        if ((M + 127) / 128 * ((N + 127) / 128) >= (int64_t)0x80000000)
            return fail(LCML_ERR_UNSUPPORTED, "%s: M=%lld N=%lld exceeds the tile grid", fn, (long long)M, (long long)N);
        if (ya.part) {  // the tile kernels write one partial per workgroup
            e.amax_part = ya.part;
            *ya.npart = (int)lcml::gemm_mfma_workgroups(
                M, N, kernel == LCML_KERNEL_MFMA_128 || kernel == LCML_KERNEL_MFMA_128_FP8);
        }
        err = lcml::launch_gemm_mfma(M, N, K, a, lda, b_packed, e,
                                     kernel == LCML_KERNEL_MFMA || kernel == LCML_KERNEL_MFMA_128, s,
                                     kernel == LCML_KERNEL_MFMA_128 || kernel == LCML_KERNEL_MFMA_128_FP8);
        if (ya.part) label = kernel == LCML_KERNEL_MFMA_128 || kernel == LCML_KERNEL_MFMA_128_FP8
                                 ? (kernel == LCML_KERNEL_MFMA_128 ? "gemm_mfma_128_amax" : "gemm_mfma_128_fp8_amax")
                                 : (kernel == LCML_KERNEL_MFMA ? "gemm_mfma_256_amax" : "gemm_mfma_256_fp8_amax");
        ya.part = nullptr;  // written
        break;
    case LCML_KERNEL_SKINNY:
    case LCML_KERNEL_SKINNY_FP8:
        // buffer extents are 32-bit: the activations and one weight panel
        if ((M - 1) * lda + K >= (int64_t)0x80000000 || lcml::pad_to(K, lcml::kPackK) * 64 >= (int64_t)0x80000000)
            return fail(LCML_ERR_UNSUPPORTED, "%s: operand larger than 2 GiB for the skinny kernel", fn);
        if ((M + 63) / 64 * ((N + 63) / 64) >= (int64_t)0x80000000)
            return fail(LCML_ERR_UNSUPPORTED, "%s: M=%lld N=%lld exceeds the skinny kernel's grid", fn, (long long)M,
                        (long long)N);
        err = lcml::launch_gemm_skinny(M, N, K, a, lda, b_packed, e, kernel == LCML_KERNEL_SKINNY, s);
        break;
    case LCML_KERNEL_VALU: err = lcml::launch_gemv_valu_fp8(M, N, K, a, lda, b_packed, e, s); break;
    default: return fail(LCML_ERR_INVALID_ARG, "%s: unknown kernel %d", fn, kernel);
    }
    if (int rc = hip_status(err, fn, label)) return rc;
    if (ya.part)  // kernels without the epilogue partials: an amax pass over y
        return hip_status(lcml::launch_amax_partials(static_cast<const float *>(y), M * N, ya.part, ya.npart, s),
                          fn, "amax_partials");
    return LCML_OK;
}
}  // namespace

int lcml_fp8_gemm(int64_t M, int64_t N, int64_t K, const uint8_t *a, int64_t lda, const float *a_scale,
                  const uint8_t *b_packed, const float *b_scale, int b_scale_per_channel, float alpha,
                  const float *c, int c_ndim, int64_t c_dim0, int64_t c_dim1, float beta, int act, void *y,
                  int y_dtype, int64_t ldy, int kernel, void *stream) {
    return gemm_core("lcml_fp8_gemm", M, N, K, a, lda, a_scale, b_packed, b_scale, b_scale_per_channel, alpha, c,
                     c_ndim, c_dim0, c_dim1, beta, act, y, y_dtype, ldy, kernel, stream, YAmax{});
}

int64_t lcml_fp8_amax_parts_max(int64_t M, int64_t N) {
    if (M <= 0 || N <= 0) return 0;
    const int64_t tiles = lcml::gemm_mfma_workgroups(M, N, true);  // 128x128 tiles: the most workgroups
    const int64_t pass = lcml::amax_partials_count(M * N);
    return tiles > pass ? tiles : pass;
}

namespace {
// The fused kernel applies when the quantised activations fit its LDS copy.
// Every workgroup of it reads and encodes all M*K activations; on the
// 4096x11008 linear that redundant pass beats the separate quantise launch
// up to M = 4 (13.9 us against 15.6 us; at M = 8 it loses, 18.6 against
// 16 us), so AUTO fuses while M*K <= 16384.
constexpr int64_t kAutoFuseMaxElems = 16384;
bool dynamic_fusable(int64_t M, int64_t K, const float *x, int64_t ldx, int kernel) {
    const bool fits = M <= 16 && lcml::skinny_dynamic_lds_bytes(M, K) <= lcml::kSkinnyDynLdsMax &&
                      (!x || aligned(x, 16)) && ldx % 4 == 0 && ((M - 1) * ldx + K) * 4 < (int64_t)0x80000000;
    if (kernel == LCML_KERNEL_AUTO || kernel == LCML_KERNEL_AUTO_FP8) return fits && M * K <= kAutoFuseMaxElems;
    return fits && (kernel == LCML_KERNEL_SKINNY || kernel == LCML_KERNEL_SKINNY_FP8);
}
int64_t pad256(int64_t n) { return (n + 255) / 256 * 256; }
static_assert(LCML_FP8_DYNAMIC_WORKSPACE_BYTES >= lcml::kMaxAmaxPartials * 4, "workspace holds the partial maxima");
// quantised activations, the partial maxima, the scale (when not returned)
int64_t two_step_workspace_bytes(int64_t M, int64_t K) { return pad256(M * K) + LCML_FP8_DYNAMIC_WORKSPACE_BYTES + 256; }
}  // namespace

int64_t lcml_fp8_gemm_dynamic_workspace_bytes(int64_t M, int64_t K, int kernel) {
    if (M <= 0 || K <= 0) return 0;
    if (dynamic_fusable(M, K, nullptr, K, kernel)) return 0;
    return two_step_workspace_bytes(M, K);
}

}  // extern "C"

namespace {
// lcml_fp8_gemm_dynamic with the workspace resolved by the caller: the
// caller's buffer, or the no-allocation entry point's device array.
// x partial maxima given (x_amax_part, x_amax_npart > 0): the two-step path
// encodes from them instead of an amax pass over x (the fused small-M
// kernel computes the same maximum itself)
struct XAmax {
    const uint32_t *part = nullptr;
    int npart = 0;
};

int gemm_dynamic_impl(const char *fn, int64_t M, int64_t N, int64_t K, const float *x, int64_t ldx,
                      const uint8_t *b_packed, const float *b_scale, int b_scale_per_channel, float alpha,
                      const float *c, int c_ndim, int64_t c_dim0, int64_t c_dim1, float beta, int act, void *y,
                      int y_dtype, int64_t ldy, float *x_scale_out, void *workspace, int64_t workspace_bytes,
                      int kernel, void *stream, XAmax xa = XAmax{}, YAmax ya = YAmax{}) {
    if (M < 0 || N <= 0 || K <= 0) return fail(LCML_ERR_INVALID_ARG, "%s: M=%lld N=%lld K=%lld", fn,
                                               (long long)M, (long long)N, (long long)K);
    lcml::Epilogue e;
    if (int rc = make_epilogue(e, fn, M, N, nullptr, b_scale, b_scale_per_channel, alpha, c, c_ndim, c_dim0,
                               c_dim1, beta, act, y, y_dtype, ldy))
        return rc;
    if (M == 0) {
        if (ya.npart) *ya.npart = 0;
        return LCML_OK;
    }
    if (!x || !b_packed) return fail(LCML_ERR_INVALID_ARG, "%s: NULL operand", fn);
    if (K % 16 != 0) return fail(LCML_ERR_UNSUPPORTED, "%s: K=%lld is not a multiple of 16", fn, (long long)K);
    if (ldx < K) return fail(LCML_ERR_INVALID_ARG, "%s: ldx=%lld < K=%lld", fn, (long long)ldx, (long long)K);
    if (!aligned(b_packed, 16)) return fail(LCML_ERR_INVALID_ARG, "%s: b_packed not 16-byte aligned", fn);
    hipStream_t s = (hipStream_t)stream;
    if (dynamic_fusable(M, K, x, ldx, kernel)) {
        if (int rc = hip_status(lcml::launch_gemm_skinny_dynamic(M, N, K, x, ldx, b_packed, e, x_scale_out,
                                                                 kernel != LCML_KERNEL_SKINNY_FP8 &&
                                                                     kernel != LCML_KERNEL_AUTO_FP8,
                                                                 s),
                                fn,
                                kernel == LCML_KERNEL_SKINNY_FP8 || kernel == LCML_KERNEL_AUTO_FP8
                                    ? "gemm_skinny_dynamic_fp8"
                                    : "gemm_skinny_dynamic"))
            return rc;
        if (ya.part)
            return hip_status(lcml::launch_amax_partials(static_cast<const float *>(y), M * N, ya.part, ya.npart, s),
                              fn, "amax_partials");
        return LCML_OK;
    }
    // two-step path: quantise into the workspace, then the selected GEMM.
    // The size is that of this path whatever the size query said: the query
    // cannot see x, and a misaligned x takes this path where an aligned one
    // would have fused.
    if (ldx != K) return fail(LCML_ERR_UNSUPPORTED, "%s: x must be contiguous (ldx == K) for M=%lld", fn, (long long)M);
    const int64_t need = two_step_workspace_bytes(M, K);
    if (!workspace || workspace_bytes < need || !aligned(workspace, 256))
        return fail(LCML_ERR_INVALID_ARG, "%s: needs a 256-byte aligned workspace of %lld bytes", fn,
                    (long long)need);
    uint8_t *ws = static_cast<uint8_t *>(workspace);
    uint8_t *q = ws;
    uint32_t *part = reinterpret_cast<uint32_t *>(ws + pad256(M * K));
    float *scale = x_scale_out ? x_scale_out : reinterpret_cast<float *>(ws + pad256(M * K) + LCML_FP8_DYNAMIC_WORKSPACE_BYTES);
    hipError_t err = xa.part ? lcml::launch_quantize_dynamic_parts(x, q, M * K, xa.part, xa.npart, scale, s)
                             : lcml::launch_quantize_dynamic(x, q, M * K, scale, part, s);
    if (int rc = hip_status(err, fn, xa.part ? "quantize_dynamic_parts" : "quantize_dynamic")) return rc;
    return gemm_core(fn, M, N, K, q, K, scale, b_packed, b_scale, b_scale_per_channel, alpha, c, c_ndim, c_dim0,
                     c_dim1, beta, act, y, y_dtype, ldy, kernel, stream, ya);
}

// The no-allocation variant's workspace: one array per device, in device
// memory from the moment the library's code object is loaded on that device
// until the process ends.  `scratch` names a host-side shadow of it; its
// device address comes from hipGetSymbolAddress, resolved once per device
// (with that device current) and kept in scratch_addr.  Calls that overlap
// on one device share it and race.
constexpr int64_t kNoAllocScratchBytes = LCML_FP8_NOALLOC_SCRATCH_BYTES;
static_assert(kNoAllocScratchBytes >= LCML_FP8_NOALLOC_MAX_ELEMS + LCML_FP8_DYNAMIC_WORKSPACE_BYTES + 256,
              "scratch holds the two-step workspace of the largest accepted M*K");
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
std::atomic<void *> scratch_addr[kMaxDevices];

int noalloc_scratch(const char *fn, void **out) {
    int dev = 0;
    if (hipError_t err = hipGetDevice(&dev); err != hipSuccess) return hip_status(err, fn);
    if (dev < 0 || dev >= kMaxDevices) return fail(LCML_ERR_UNSUPPORTED, "%s: device %d (at most %d)", fn, dev, kMaxDevices);
    void *p = scratch_addr[dev].load(std::memory_order_acquire);
    if (!p) {
        // the same address on every call: threads racing here store equal values
        if (hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)); err != hipSuccess)
            return hip_status(err, fn);
        if (!p) return fail(LCML_ERR_HIP, "%s: no device address for the scratch array", fn);
        scratch_addr[dev].store(p, std::memory_order_release);
    }
    *out = p;
    return LCML_OK;
}
}  // namespace

extern "C" {

int lcml_fp8_gemm_dynamic(int64_t M, int64_t N, int64_t K, const float *x, int64_t ldx, const uint8_t *b_packed,
                          const float *b_scale, int b_scale_per_channel, float alpha, const float *c, int c_ndim,
                          int64_t c_dim0, int64_t c_dim1, float beta, int act, void *y, int y_dtype, int64_t ldy,
                          float *x_scale_out, void *workspace, int64_t workspace_bytes, int kernel, void *stream) {
    return gemm_dynamic_impl("lcml_fp8_gemm_dynamic", M, N, K, x, ldx, b_packed, b_scale, b_scale_per_channel, alpha,
                             c, c_ndim, c_dim0, c_dim1, beta, act, y, y_dtype, ldy, x_scale_out, workspace,
                             workspace_bytes, kernel, stream);
}

int lcml_fp8_gemm_dynamic_ex(int64_t M, int64_t N, int64_t K, const float *x, int64_t ldx, const uint8_t *b_packed,
                             const float *b_scale, int b_scale_per_channel, float alpha, const float *c, int c_ndim,
                             int64_t c_dim0, int64_t c_dim1, float beta, int act, void *y, int y_dtype, int64_t ldy,
                             float *x_scale_out, const uint32_t *x_amax_part, int x_amax_npart, uint32_t *y_amax_part,
                             int64_t y_amax_capacity, int *y_amax_npart, void *workspace, int64_t workspace_bytes,
                             int kernel, void *stream) {
    const char *fn = "lcml_fp8_gemm_dynamic_ex";
    XAmax xa;
    if (x_amax_part) {
        if (x_amax_npart < 1) return fail(LCML_ERR_INVALID_ARG, "%s: x_amax_npart=%d", fn, x_amax_npart);
        xa.part = x_amax_part;
        xa.npart = x_amax_npart;
    }
    YAmax ya;
    if (y_amax_part) {
        if (y_dtype != LCML_DTYPE_FLOAT || ldy != N)
            return fail(LCML_ERR_UNSUPPORTED, "%s: amax partials of y need a dense fp32 y (ldy == N)", fn);
        if (!y_amax_npart) return fail(LCML_ERR_INVALID_ARG, "%s: y_amax_npart is NULL", fn);
        if (y_amax_capacity < lcml_fp8_amax_parts_max(M, N))
            return fail(LCML_ERR_INVALID_ARG, "%s: y_amax_capacity=%lld < lcml_fp8_amax_parts_max=%lld", fn,
                        (long long)y_amax_capacity, (long long)lcml_fp8_amax_parts_max(M, N));
        ya.part = y_amax_part;
        ya.npart = y_amax_npart;
    }
    return gemm_dynamic_impl(fn, M, N, K, x, ldx, b_packed, b_scale, b_scale_per_channel, alpha, c, c_ndim, c_dim0,
                             c_dim1, beta, act, y, y_dtype, ldy, x_scale_out, workspace, workspace_bytes, kernel,
                             stream, xa, ya);
}

int lcml_fp8_gemm_dynamic_noalloc(int64_t M, int64_t N, int64_t K, const float *x, int64_t ldx,
                                  const uint8_t *b_packed, const float *b_scale, int b_scale_per_channel, float alpha,
                                  const float *c, int c_ndim, int64_t c_dim0, int64_t c_dim1, float beta, int act,
                                  void *y, int y_dtype, int64_t ldy, float *x_scale_out, int kernel, void *stream) {
    const char *fn = "lcml_fp8_gemm_dynamic_noalloc";
    if (M > 0 && K > 0 && M * K > LCML_FP8_NOALLOC_MAX_ELEMS)
        return fail(LCML_ERR_UNSUPPORTED, "%s: M*K=%lld exceeds the no-allocation limit of %lld elements", fn,
                    (long long)(M * K), (long long)LCML_FP8_NOALLOC_MAX_ELEMS);
    if (M < 0 || N <= 0 || K <= 0) return fail(LCML_ERR_INVALID_ARG, "%s: M=%lld N=%lld K=%lld", fn,
                                               (long long)M, (long long)N, (long long)K);
    if (M == 0) return gemm_dynamic_impl(fn, M, N, K, x, ldx, b_packed, b_scale, b_scale_per_channel, alpha, c,
                                         c_ndim, c_dim0, c_dim1, beta, act, y, y_dtype, ldy, x_scale_out, nullptr, 0,
                                         kernel, stream);
    void *ws = nullptr;
    if (int rc = noalloc_scratch(fn, &ws)) return rc;
    return gemm_dynamic_impl(fn, M, N, K, x, ldx, b_packed, b_scale, b_scale_per_channel, alpha, c, c_ndim, c_dim0,
                             c_dim1, beta, act, y, y_dtype, ldy, x_scale_out, ws, kNoAllocScratchBytes, kernel,
                             stream);
}

int lcml_fp8_quantize_nhwc(const float *x, uint8_t *y, int64_t n, int64_t c, int64_t h, int64_t w,
                           const float *y_scale, float *scale_out, void *workspace, void *stream) {
    const char *fn = "lcml_fp8_quantize_nhwc";
    if (n < 0 || c <= 0 || h <= 0 || w <= 0) return fail(LCML_ERR_INVALID_ARG, "%s: bad shape", fn);
    if (c % 4 != 0) return fail(LCML_ERR_UNSUPPORTED, "%s: c=%lld is not a multiple of 4", fn, (long long)c);
    if (n * c * h * w >= (int64_t)1 << 31 || n * h >= ((int64_t)1 << 31))
        return fail(LCML_ERR_UNSUPPORTED, "%s: tensor too large", fn);
    if (n == 0) return LCML_OK;
    if (!x || !y) return fail(LCML_ERR_INVALID_ARG, "%s: NULL pointer", fn);
    if (!aligned(y, 4)) return fail(LCML_ERR_INVALID_ARG, "%s: y must be 4-byte aligned", fn);
    hipStream_t s = (hipStream_t)stream;
    if (y_scale)
        return hip_status(lcml::launch_quantize_nhwc(x, y, n, (int)c, (int)h, (int)w, y_scale, nullptr, 0, nullptr, s),
                          fn);
    if (!scale_out || !workspace)
        return fail(LCML_ERR_INVALID_ARG, "%s: the dynamic scale needs scale_out and a workspace", fn);
    uint32_t *part = static_cast<uint32_t *>(workspace);
    int npart = 0;
    hipError_t err = lcml::launch_amax_partials(x, n * c * h * w, part, &npart, s);
    if (err == hipSuccess)
        err = lcml::launch_quantize_nhwc(x, y, n, (int)c, (int)h, (int)w, nullptr, part, npart, scale_out, s);
    return hip_status(err, fn);
}

int64_t lcml_fp8_packed_conv_weight_bytes(int64_t cout, int64_t cin_g, int64_t kh, int64_t kw, int64_t group) {
    if (cout <= 0 || cin_g <= 0 || kh <= 0 || kw <= 0 || group <= 0 || cout % group != 0) return 0;
    return group * lcml_fp8_packed_weight_bytes(kh * kw * cin_g, cout / group);
}

int lcml_fp8_pack_conv_weight(const uint8_t *w, int64_t cout, int64_t cin_g, int64_t kh, int64_t kw, int64_t group,
                              uint8_t *packed, void *stream) {
    const char *fn = "lcml_fp8_pack_conv_weight";
    if (cout <= 0 || cin_g <= 0 || kh <= 0 || kw <= 0 || group <= 0 || cout % group != 0)
        return fail(LCML_ERR_INVALID_ARG, "%s: bad shape or group", fn);
    if (!w || !packed) return fail(LCML_ERR_INVALID_ARG, "%s: NULL pointer", fn);
    if (!aligned(packed, 16)) return fail(LCML_ERR_INVALID_ARG, "%s: packed not 16-byte aligned", fn);
    if (lcml_fp8_packed_conv_weight_bytes(cout, cin_g, kh, kw, group) >= (int64_t)1 << 31)
        return fail(LCML_ERR_UNSUPPORTED, "%s: packed weight larger than 2 GiB", fn);
    return hip_status(lcml::launch_pack_conv_weight(w, (int)cout, (int)cin_g, (int)kh, (int)kw, (int)group, packed,
                                                    (hipStream_t)stream),
                      fn);
}

int lcml_fp8_conv2d(const uint8_t *x_nhwc, const float *x_scale, int64_t n, int64_t c, int64_t h, int64_t w,
                    const uint8_t *w_packed, const float *w_scale, int w_scale_per_channel, int64_t cout, int64_t kh,
                    int64_t kw, int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w, int64_t dil_h,
                    int64_t dil_w, int64_t group, int64_t oh, int64_t ow, const float *bias, int act, void *y,
                    int y_dtype, int kernel, void *stream) {
    const char *fn = "lcml_fp8_conv2d";
    if (n < 0 || c <= 0 || h <= 0 || w <= 0 || cout <= 0 || kh <= 0 || kw <= 0 || oh <= 0 || ow <= 0)
        return fail(LCML_ERR_INVALID_ARG, "%s: bad shape", fn);
    if (stride_h <= 0 || stride_w <= 0 || dil_h <= 0 || dil_w <= 0 || pad_h < 0 || pad_w < 0)
        return fail(LCML_ERR_INVALID_ARG, "%s: strides and dilations must be >= 1, pads >= 0", fn);
    if (group <= 0 || c % group != 0 || cout % group != 0)
        return fail(LCML_ERR_INVALID_ARG, "%s: group=%lld must divide c=%lld and cout=%lld", fn, (long long)group,
                    (long long)c, (long long)cout);
    if ((c / group) % 16 != 0)
        return fail(LCML_ERR_UNSUPPORTED, "%s: channels per group (%lld) not a multiple of 16", fn,
                    (long long)(c / group));
    const int64_t M = n * oh * ow;
    if (n * h * w * c >= (int64_t)1 << 31 || M >= (int64_t)1 << 31 ||
        lcml_fp8_packed_conv_weight_bytes(cout, c / group, kh, kw, group) >= (int64_t)1 << 31)
        return fail(LCML_ERR_UNSUPPORTED, "%s: operand larger than 2 GiB", fn);
    if (kernel == LCML_KERNEL_AUTO || kernel == LCML_KERNEL_AUTO_FP8) {
        // as auto_gemm_kernel without the skinny kernel; groups add grid rows
        const int64_t N = cout / group;
        const double big = (double)((M + 255) / 256 * ((N + 255) / 256) * group);
        const double t128 = (double)((M + 127) / 128 * ((N + 127) / 128) * group);
        const double small = 2.2 * (t128 > 256 ? t128 / 256 : 1.0);
        const int tiles = big < 256 && small < 4.5 ? LCML_KERNEL_MFMA_128 : LCML_KERNEL_MFMA;
        kernel = kernel == LCML_KERNEL_AUTO_FP8 ? fp8_twin(tiles) : tiles;
    }
    if (kernel != LCML_KERNEL_MFMA && kernel != LCML_KERNEL_MFMA_FP8 && kernel != LCML_KERNEL_MFMA_128 &&
        kernel != LCML_KERNEL_MFMA_128_FP8)
        return fail(LCML_ERR_UNSUPPORTED, "%s: kernel %d (AUTO, AUTO_FP8 or one of the MFMA tile kernels)", fn,
                    kernel);
    lcml::Epilogue e;
    if (int rc = make_epilogue(e, fn, M, cout, x_scale, w_scale, w_scale_per_channel, 1.0f, bias, 1, cout, 0, 1.0f,
                               act, y, y_dtype, cout))
        return rc;
    // per group: N = cout/group columns; the scale and bias pointers are
    // advanced to the group's channels in the kernel
    e.N = cout / group;
    e.c0 = cout / group;
    if (n == 0) return LCML_OK;
    if (!x_nhwc || !w_packed) return fail(LCML_ERR_INVALID_ARG, "%s: NULL operand", fn);
    if (!aligned(x_nhwc, 16) || !aligned(w_packed, 16))
        return fail(LCML_ERR_INVALID_ARG, "%s: x_nhwc and w_packed must be 16-byte aligned", fn);
    return hip_status(lcml::launch_conv_mfma(x_nhwc, n, (int)c, (int)h, (int)w, w_packed, (int)cout, (int)kh, (int)kw,
                                             (int)stride_h, (int)stride_w, (int)pad_h, (int)pad_w, (int)dil_h,
                                             (int)dil_w, (int)group, (int)oh, (int)ow, e,
                                             kernel == LCML_KERNEL_MFMA || kernel == LCML_KERNEL_MFMA_128,
                                             (hipStream_t)stream,
                                             kernel == LCML_KERNEL_MFMA_128 || kernel == LCML_KERNEL_MFMA_128_FP8),
                      fn,
                      kernel == LCML_KERNEL_MFMA       ? "conv_mfma_256"
                      : kernel == LCML_KERNEL_MFMA_FP8 ? "conv_mfma_256_fp8"
                      : kernel == LCML_KERNEL_MFMA_128 ? "conv_mfma_128"
                                                       : "conv_mfma_128_fp8");
}

int lcml_fp8_gemm_w8a32(int64_t M, int64_t N, int64_t K, const float *a, int64_t lda, const uint8_t *b_packed,
                        const float *b_scale, int b_scale_per_channel, float alpha, const float *c, int c_ndim,
                        int64_t c_dim0, int64_t c_dim1, float beta, int act, void *y, int y_dtype, int64_t ldy,
                        void *stream) {
    const char *fn = "lcml_fp8_gemm_w8a32";
    if (M < 0 || N <= 0 || K <= 0) return fail(LCML_ERR_INVALID_ARG, "%s: M=%lld N=%lld K=%lld", fn,
                                               (long long)M, (long long)N, (long long)K);
    lcml::Epilogue e;
    if (int rc = make_epilogue(e, fn, M, N, nullptr, b_scale, b_scale_per_channel, alpha, c, c_ndim, c_dim0,
                               c_dim1, beta, act, y, y_dtype, ldy))
        return rc;
    if (M == 0) return LCML_OK;
    if (!a || !b_packed) return fail(LCML_ERR_INVALID_ARG, "%s: NULL operand", fn);
    if (lda < K || !aligned(a, 4)) return fail(LCML_ERR_INVALID_ARG, "%s: lda < K or a misaligned", fn);
    if (!aligned(b_packed, 16)) return fail(LCML_ERR_INVALID_ARG, "%s: b_packed not 16-byte aligned", fn);
    return hip_status(lcml::launch_gemv_valu_f32(M, N, K, a, lda, b_packed, e, (hipStream_t)stream), fn);
}

int lcml_fp8_conv2d_f32(const float *x, const float *w, const float *bias, float *y, int64_t n, int64_t c, int64_t h,
                        int64_t wd, int64_t cout, int64_t kh, int64_t kw, int64_t stride_h, int64_t stride_w,
                        int64_t pad_h, int64_t pad_w, int64_t dil_h, int64_t dil_w, int64_t group, int64_t oh,
                        int64_t ow, int act, void *stream) {
    const char *fn = "lcml_fp8_conv2d_f32";
    if (n < 0 || c <= 0 || h <= 0 || wd <= 0 || cout <= 0 || kh <= 0 || kw <= 0 || oh <= 0 || ow <= 0 ||
        group <= 0 || c % group != 0 || cout % group != 0)
        return fail(LCML_ERR_INVALID_ARG, "%s: bad shape or group", fn);
    if (stride_h <= 0 || stride_w <= 0 || dil_h <= 0 || dil_w <= 0 || pad_h < 0 || pad_w < 0)
        return fail(LCML_ERR_INVALID_ARG, "%s: strides and dilations must be >= 1, pads >= 0", fn);
    if (act < LCML_ACT_NONE || act > LCML_ACT_GELU_TANH) return fail(LCML_ERR_UNSUPPORTED, "%s: activation %d", fn, act);
    if (n == 0) return LCML_OK;
    if (!x || !w || !y) return fail(LCML_ERR_INVALID_ARG, "%s: NULL pointer", fn);
    if (n * cout * oh * ow >= (int64_t)1 << 40) return fail(LCML_ERR_UNSUPPORTED, "%s: output too large", fn);
    return hip_status(lcml::launch_conv2d_f32(x, w, bias, y, n, (int)c, (int)h, (int)wd, (int)cout, (int)kh, (int)kw,
                                              (int)stride_h, (int)stride_w, (int)pad_h, (int)pad_w, (int)dil_h,
                                              (int)dil_w, (int)group, (int)oh, (int)ow, act, (hipStream_t)stream),
                      fn);
}

int lcml_fp8_sgemm(int64_t M, int64_t N, int64_t K, const float *a, int64_t lda, int trans_a, const float *b,
                   int64_t ldb, int trans_b, float alpha, const float *c, int c_ndim, int64_t c_dim0,
                   int64_t c_dim1, float beta, int act, void *y, int y_dtype, int64_t ldy, void *stream) {
    const char *fn = "lcml_fp8_sgemm";
    if (M < 0 || N <= 0 || K <= 0) return fail(LCML_ERR_INVALID_ARG, "%s: M=%lld N=%lld K=%lld", fn,
                                               (long long)M, (long long)N, (long long)K);
    lcml::Epilogue e;
    if (int rc = make_epilogue(e, fn, M, N, nullptr, nullptr, 0, alpha, c, c_ndim, c_dim0, c_dim1, beta, act, y,
                               y_dtype, ldy, true))
        return rc;
    if (M == 0) return LCML_OK;
    if (!a || !b) return fail(LCML_ERR_INVALID_ARG, "%s: NULL operand", fn);
    if (lda < (trans_a ? M : K) || ldb < (trans_b ? K : N))
        return fail(LCML_ERR_INVALID_ARG, "%s: leading dimension too small", fn);
    return hip_status(lcml::launch_sgemm(M, N, K, a, lda, trans_a, b, ldb, trans_b, e, (hipStream_t)stream), fn);
}

int lcml_fp8_activation(const float *x, float *y, int64_t n, int act, void *stream) {
    if (n < 0 || act < LCML_ACT_NONE || act > LCML_ACT_GELU_TANH)
        return fail(LCML_ERR_INVALID_ARG, "lcml_fp8_activation: n=%lld act=%d", (long long)n, act);
    if (n == 0) return LCML_OK;
    if (!x || !y) return fail(LCML_ERR_INVALID_ARG, "lcml_fp8_activation: NULL pointer");
    return hip_status(lcml::launch_activation(x, y, n, act, (hipStream_t)stream), "lcml_fp8_activation");
}

int lcml_fp8_stream_read(const void *p, int64_t bytes, int workgroups, uint32_t *sink, void *stream) {
    const char *fn = "lcml_fp8_stream_read";
    if (bytes < 0 || bytes % 16 != 0 || workgroups < 1 || workgroups > (1 << 20))
        return fail(LCML_ERR_INVALID_ARG, "%s: bytes=%lld (multiple of 16) workgroups=%d", fn, (long long)bytes,
                    workgroups);
    if (bytes == 0) return LCML_OK;
    if (!p || !sink || !aligned(p, 16)) return fail(LCML_ERR_INVALID_ARG, "%s: p must be 16-byte aligned, sink set", fn);
    if ((bytes / 16 + workgroups - 1) / workgroups >= ((int64_t)1 << 27))
        return fail(LCML_ERR_UNSUPPORTED, "%s: a workgroup's share of %lld bytes over %d workgroups exceeds 2 GiB", fn,
                    (long long)bytes, workgroups);
    return hip_status(lcml::launch_stream_read(p, bytes, workgroups, sink, (hipStream_t)stream), fn);
}

namespace {
bool fp8_dtype_ok(int dt) {
    return dt == LCML_DTYPE_FLOAT || dt == LCML_DTYPE_FLOAT8E4M3FN || dt == LCML_DTYPE_FLOAT8E5M2;
}
}  // namespace

int lcml_fp8_cast(const void *x, int x_dtype, void *y, int y_dtype, int64_t n, void *stream) {
    const char *fn = "lcml_fp8_cast";
    if (n < 0) return fail(LCML_ERR_INVALID_ARG, "%s: n < 0", fn);
    if (!fp8_dtype_ok(x_dtype) || !fp8_dtype_ok(y_dtype))
        return fail(LCML_ERR_UNSUPPORTED, "%s: dtypes %d -> %d (FLOAT, FLOAT8E4M3FN, FLOAT8E5M2 only)", fn, x_dtype,
                    y_dtype);
    if (n == 0) return LCML_OK;
    if (!x || !y) return fail(LCML_ERR_INVALID_ARG, "%s: NULL pointer", fn);
    if (x_dtype == LCML_DTYPE_FLOAT ? !aligned(x, 4) : false) return fail(LCML_ERR_INVALID_ARG, "%s: x misaligned", fn);
    if (y_dtype == LCML_DTYPE_FLOAT ? !aligned(y, 4) : false) return fail(LCML_ERR_INVALID_ARG, "%s: y misaligned", fn);
    return hip_status(lcml::launch_cast(x, x_dtype, y, y_dtype, n, (hipStream_t)stream), fn);
}

int lcml_fp8_quantize_e5m2(const float *x, uint8_t *y, int64_t outer, int64_t axis_len, int64_t inner,
                           const float *y_scale, int saturate, void *stream) {
    if (int rc = check_view(outer, axis_len, inner, "lcml_fp8_quantize_e5m2")) return rc;
    if (outer * axis_len * inner == 0) return LCML_OK;
    if (!x || !y || !y_scale) return fail(LCML_ERR_INVALID_ARG, "lcml_fp8_quantize_e5m2: NULL pointer");
    if (saturate != 0 && saturate != 1) return fail(LCML_ERR_INVALID_ARG, "lcml_fp8_quantize_e5m2: saturate %d", saturate);
    return hip_status(lcml::launch_quantize_e5m2(x, y, outer, axis_len, inner, y_scale, saturate == 1,
                                                 (hipStream_t)stream),
                      "lcml_fp8_quantize_e5m2");
}

int lcml_fp8_dequantize_e5m2(const uint8_t *x, float *y, int64_t outer, int64_t axis_len, int64_t inner,
                             const float *x_scale, void *stream) {
    if (int rc = check_view(outer, axis_len, inner, "lcml_fp8_dequantize_e5m2")) return rc;
    if (outer * axis_len * inner == 0) return LCML_OK;
    if (!x || !y || !x_scale) return fail(LCML_ERR_INVALID_ARG, "lcml_fp8_dequantize_e5m2: NULL pointer");
    return hip_status(lcml::launch_dequantize_e5m2(x, y, outer, axis_len, inner, x_scale, (hipStream_t)stream),
                      "lcml_fp8_dequantize_e5m2");
}

int lcml_fp8_binary(int op, int dtype, const void *a, const int64_t *a_shape, int a_ndim, const void *b,
                    const int64_t *b_shape, int b_ndim, void *y, const int64_t *y_shape, int y_ndim, void *stream) {
    const char *fn = "lcml_fp8_binary";
    if (op < LCML_BINARY_ADD || op > LCML_BINARY_DIV) return fail(LCML_ERR_INVALID_ARG, "%s: op %d", fn, op);
    if (!fp8_dtype_ok(dtype)) return fail(LCML_ERR_UNSUPPORTED, "%s: dtype %d", fn, dtype);
    if (a_ndim < 0 || b_ndim < 0 || y_ndim < 0 || y_ndim > lcml::kMaxBcastDims || a_ndim > y_ndim || b_ndim > y_ndim)
        return fail(LCML_ERR_INVALID_ARG, "%s: ranks a=%d b=%d y=%d (at most %d, y the largest)", fn, a_ndim, b_ndim,
                    y_ndim, lcml::kMaxBcastDims);
    if ((a_ndim && !a_shape) || (b_ndim && !b_shape) || (y_ndim && !y_shape))
        return fail(LCML_ERR_INVALID_ARG, "%s: NULL shape", fn);
    // numpy broadcasting, right-aligned; element strides of a and b per output dim
    lcml::BcastGeom g{};
    g.ndim = y_ndim;
    int64_t n = 1, acc_a = 1, acc_b = 1;
    bool same = a_ndim == y_ndim && b_ndim == y_ndim;
    for (int d = y_ndim - 1; d >= 0; --d) {
        const int da = d - (y_ndim - a_ndim), db = d - (y_ndim - b_ndim);
        const int64_t ea = da >= 0 ? a_shape[da] : 1, eb = db >= 0 ? b_shape[db] : 1, ey = y_shape[d];
        if (ea < 0 || eb < 0 || ey < 0) return fail(LCML_ERR_INVALID_ARG, "%s: negative dimension", fn);
        const int64_t want = ea == 1 ? eb : (eb == 1 || eb == ea ? ea : -1);
        if (want < 0 || want != ey)
            return fail(LCML_ERR_INVALID_ARG, "%s: dim %d: a %lld, b %lld do not broadcast to y %lld", fn, d,
                        (long long)ea, (long long)eb, (long long)ey);
        same = same && ea == ey && eb == ey;
        g.dims[d] = ey;
        g.sa[d] = ea == 1 ? 0 : acc_a;
        g.sb[d] = eb == 1 ? 0 : acc_b;
        acc_a *= ea;
        acc_b *= eb;
        if (ey && n > ((int64_t)1 << 40) / ey) return fail(LCML_ERR_UNSUPPORTED, "%s: tensor too large", fn);
        n *= ey;
    }
    if (n == 0) return LCML_OK;
    if (!a || !b || !y) return fail(LCML_ERR_INVALID_ARG, "%s: NULL pointer", fn);
    if (dtype == LCML_DTYPE_FLOAT && (!aligned(a, 4) || !aligned(b, 4) || !aligned(y, 4)))
        return fail(LCML_ERR_INVALID_ARG, "%s: fp32 tensors must be 4-byte aligned", fn);
    return hip_status(lcml::launch_fp8_binary(op, dtype, a, b, y, n, same, g, (hipStream_t)stream), fn);
}

}  // extern "C"
