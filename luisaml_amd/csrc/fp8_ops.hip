// fp8_ops.hip -- the FP8 data-type surface around the linear path:
//   * Cast between FLOAT, FLOAT8E4M3FN and FLOAT8E5M2 with the reference's
//     CPU codecs (FP8E4M3FN / FP8E5M2 from_float / to_float,
//     include/onnx/fp_quantized.h:149-249, 272-377), bit for bit;
//   * QuantizeLinear / DequantizeLinear with FLOAT8E5M2 tensors;
//   * elementwise Add / Sub / Mul / Div with numpy broadcasting on FLOAT and
//     on fp8 tensors.  For fp8 the reference's Binary ops
//     (src/onnx/operators/binary.cpp:184-285) decode both operands to half
//     (exact for every fp8 value), run the op in half and encode the half
//     result; here the op runs in fp32 and is rounded once to half, which
//     gives the same half (24 >= 2*11 + 2 bits, so the double rounding is
//     innocuous for +, -, *, /), and the encode is the CPU from_float.
// All of these are HBM-bound streaming kernels: 4 elements per thread.
#include "lcml_internal.hpp"

namespace lcml {
namespace {

constexpr int kThreads = 256;
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));

// four codes of one fp8 word -> four floats (OCP E4M3FN / E5M2 decode: the
// reference's to_float on every code, NaN codes -> NaN, inf codes -> inf)
template <int FMT>
__device__ inline f4 decode4(uint32_t w) {
    f2 lo, hi;
    if constexpr (FMT == kFmtE4M3) {
        lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
        hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
    } else {
        lo = __builtin_amdgcn_cvt_pk_f32_bf8((int)w, false);
        hi = __builtin_amdgcn_cvt_pk_f32_bf8((int)w, true);
    }
    return f4{lo.x, lo.y, hi.x, hi.y};
}

template <int FMT>
__device__ inline uint32_t encode4(f4 v) {
    if constexpr (FMT == kFmtE4M3)
        return e4m3x2_hw(v.x, v.y) | (e4m3x2_hw(v.z, v.w) << 16);
    else
        return e5m2x2_hw(v.x, v.y) | (e5m2x2_hw(v.z, v.w) << 16);
}

template <int FMT>
__device__ inline float load1(const void *p, int64_t i) {
    if constexpr (FMT == kFmtFloat)
        return static_cast<const float *>(p)[i];
    else
        return decode4<FMT>(static_cast<const uint8_t *>(p)[i]).x;
}

template <int FMT>
__device__ inline f4 load4(const void *p, int64_t i4) {
    if constexpr (FMT == kFmtFloat)
        return reinterpret_cast<const f4 *>(p)[i4];
    else
        return decode4<FMT>(reinterpret_cast<const uint32_t *>(p)[i4]);
}

template <int FMT>
__device__ inline void store1(void *p, int64_t i, float v) {
    if constexpr (FMT == kFmtFloat)
        static_cast<float *>(p)[i] = v;
    else
        static_cast<uint8_t *>(p)[i] = (uint8_t)(encode4<FMT>(f4{v, 0.f, 0.f, 0.f}) & 0xffu);
}

template <int FMT>
__device__ inline void store4(void *p, int64_t i4, f4 v) {
    if constexpr (FMT == kFmtFloat)
        reinterpret_cast<f4 *>(p)[i4] = v;
    else
        reinterpret_cast<uint32_t *>(p)[i4] = encode4<FMT>(v);
}

// Cast: decode then encode.  n4 groups of four (aligned), then the tail.
template <int SRC, int DST>
__global__ __launch_bounds__(kThreads) void k_cast(const void *__restrict__ x, void *__restrict__ y, int64_t n,
                                                   int64_t n4) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n4; i += stride)
        store4<DST>(y, i, load4<SRC>(x, i));
    for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
        store1<DST>(y, i, load1<SRC>(x, i));
}

// E5M2 QuantizeLinear: from_float(x / s) (exact quotient, as the E4M3
// quantiser), with saturate = clamp |x / s| > 57344 (inf included) to
// +-57344 first.  One scale per element index (outer, axis_len, inner).
template <bool SAT>
__device__ inline float e5m2_sat(float q) {
    if (SAT && fabsf(q) > 57344.0f) q = q < 0.0f ? -57344.0f : 57344.0f;  // NaN compares false
    return q;
}

template <bool SAT>
__global__ __launch_bounds__(kThreads) void k_quantize_e5m2(const float *__restrict__ x, uint8_t *__restrict__ y,
                                                            int64_t n, int64_t n4, int64_t axis_len, int64_t inner,
                                                            const float *__restrict__ scale) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    const Recip d_tensor = make_recip(scale[0]);
    // groups of four share one scale when axis_len == 1 or inner % 4 == 0
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n4; i += stride) {
        const Recip d = axis_len == 1 ? d_tensor : make_recip(scale[((i * 4) / inner) % axis_len]);
        const f4 v = reinterpret_cast<const f4 *>(x)[i];
        const f4 q = {e5m2_sat<SAT>(div_by(v.x, d)), e5m2_sat<SAT>(div_by(v.y, d)), e5m2_sat<SAT>(div_by(v.z, d)),
                      e5m2_sat<SAT>(div_by(v.w, d))};
        reinterpret_cast<uint32_t *>(y)[i] = encode4<kFmtE5M2>(q);
    }
    for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
        const float s = scale[axis_len == 1 ? 0 : (i / inner) % axis_len];
        y[i] = (uint8_t)(encode4<kFmtE5M2>(f4{e5m2_sat<SAT>(__fdiv_rn(x[i], s)), 0.f, 0.f, 0.f}) & 0xffu);
    }
}

__global__ __launch_bounds__(kThreads) void k_dequantize_e5m2(const uint8_t *__restrict__ x, float *__restrict__ y,
                                                              int64_t n, int64_t n4, int64_t axis_len, int64_t inner,
                                                              const float *__restrict__ scale) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n4; i += stride) {
        const float s = scale[axis_len == 1 ? 0 : ((i * 4) / inner) % axis_len];
        const f4 v = decode4<kFmtE5M2>(reinterpret_cast<const uint32_t *>(x)[i]);
        reinterpret_cast<f4 *>(y)[i] = f4{v.x * s, v.y * s, v.z * s, v.w * s};
    }
    for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
        const float s = scale[axis_len == 1 ? 0 : (i / inner) % axis_len];
        y[i] = decode4<kFmtE5M2>(x[i]).x * s;
    }
}

// Binary ops.  FLOAT: the op in fp32.  fp8: the op in fp32 on the decoded
// values, rounded once to half (v_cvt_f16_f32, nearest even, overflow to
// inf), then encoded.
template <int OP>
__device__ inline float bin_op(float a, float b) {
    if constexpr (OP == 0) return a + b;
    else if constexpr (OP == 1) return a - b;
    else if constexpr (OP == 2) return a * b;
    else return a / b;  // IEEE division
}

template <int FMT, int OP>
__device__ inline float bin_value(float a, float b) {
    const float r = bin_op<OP>(a, b);
    if constexpr (FMT == kFmtFloat) return r;
    else return (float)(_Float16)r;
}

template <int FMT, int OP>
__global__ __launch_bounds__(kThreads) void k_binary_same(const void *__restrict__ a, const void *__restrict__ b,
                                                          void *__restrict__ y, int64_t n, int64_t n4) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n4; i += stride) {
        const f4 va = load4<FMT>(a, i), vb = load4<FMT>(b, i);
        store4<FMT>(y, i, f4{bin_value<FMT, OP>(va.x, vb.x), bin_value<FMT, OP>(va.y, vb.y),
                             bin_value<FMT, OP>(va.z, vb.z), bin_value<FMT, OP>(va.w, vb.w)});
    }
    for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
        store1<FMT>(y, i, bin_value<FMT, OP>(load1<FMT>(a, i), load1<FMT>(b, i)));
}

template <int FMT, int OP>
__global__ __launch_bounds__(kThreads) void k_binary_bcast(const void *__restrict__ a, const void *__restrict__ b,
                                                           void *__restrict__ y, int64_t n, BcastGeom g) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
        int64_t r = i, ia = 0, ib = 0;
        for (int d = g.ndim - 1; d >= 0; --d) {
            const int64_t q = r / g.dims[d], c = r - q * g.dims[d];
            r = q;
            ia += c * g.sa[d];
            ib += c * g.sb[d];
        }
        store1<FMT>(y, i, bin_value<FMT, OP>(load1<FMT>(a, ia), load1<FMT>(b, ib)));
    }
}

int grid_for(int64_t items) {
    int64_t g = (items + kThreads - 1) / kThreads;
    return (int)(g < 1 ? 1 : (g > 8192 ? 8192 : g));
}

bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }
int fmt_bytes(int fmt) { return fmt == kFmtFloat ? 4 : 1; }

template <int SRC>
hipError_t cast_from(const void *x, void *y, int y_fmt, int64_t n, int64_t n4, hipStream_t s) {
    const dim3 grid(grid_for(n4 ? n4 : n)), block(kThreads);
    switch (y_fmt) {
    case kFmtFloat: hipLaunchKernelGGL((k_cast<SRC, kFmtFloat>), grid, block, 0, s, x, y, n, n4); break;
    case kFmtE4M3: hipLaunchKernelGGL((k_cast<SRC, kFmtE4M3>), grid, block, 0, s, x, y, n, n4); break;
    default: hipLaunchKernelGGL((k_cast<SRC, kFmtE5M2>), grid, block, 0, s, x, y, n, n4); break;
    }
    return hipGetLastError();
}

template <int FMT>
hipError_t binary_fmt(int op, const void *a, const void *b, void *y, int64_t n, bool same, const BcastGeom &g,
                      hipStream_t s) {
    const int bytes = fmt_bytes(FMT);
    const int64_t n4 = (same && aligned(a, 4 * bytes) && aligned(b, 4 * bytes) && aligned(y, 4 * bytes)) ? n / 4 : 0;
    const dim3 grid(grid_for(same ? (n4 ? n4 : n) : n)), block(kThreads);
#define LCML_BIN(OPC)                                                                                   \
    if (same)                                                                                          \
        hipLaunchKernelGGL((k_binary_same<FMT, OPC>), grid, block, 0, s, a, b, y, n, n4);               \
    else                                                                                               \
        hipLaunchKernelGGL((k_binary_bcast<FMT, OPC>), grid, block, 0, s, a, b, y, n, g)
    switch (op) {
    case 0: LCML_BIN(0); break;
    case 1: LCML_BIN(1); break;
    case 2: LCML_BIN(2); break;
    default: LCML_BIN(3); break;
    }
#undef LCML_BIN
    return hipGetLastError();
}

}  // namespace

hipError_t launch_cast(const void *x, int x_fmt, void *y, int y_fmt, int64_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const int64_t n4 = (aligned(x, 4 * fmt_bytes(x_fmt)) && aligned(y, 4 * fmt_bytes(y_fmt))) ? n / 4 : 0;
    switch (x_fmt) {
    case kFmtFloat: return cast_from<kFmtFloat>(x, y, y_fmt, n, n4, s);
    case kFmtE4M3: return cast_from<kFmtE4M3>(x, y, y_fmt, n, n4, s);
    default: return cast_from<kFmtE5M2>(x, y, y_fmt, n, n4, s);
    }
}

hipError_t launch_quantize_e5m2(const float *x, uint8_t *y, int64_t outer, int64_t axis_len, int64_t inner,
                                const float *scale, bool saturate, hipStream_t s) {
    const int64_t n = outer * axis_len * inner;
    if (n == 0) return hipSuccess;
    const bool quad = axis_len == 1 || inner % 4 == 0;
    const int64_t n4 = (quad && aligned(x, 16) && aligned(y, 4)) ? n / 4 : 0;
    const dim3 grid(grid_for(n4 ? n4 : n)), block(kThreads);
    if (saturate)
        hipLaunchKernelGGL(k_quantize_e5m2<true>, grid, block, 0, s, x, y, n, n4, axis_len, inner, scale);
    else
        hipLaunchKernelGGL(k_quantize_e5m2<false>, grid, block, 0, s, x, y, n, n4, axis_len, inner, scale);
    return hipGetLastError();
}

hipError_t launch_dequantize_e5m2(const uint8_t *x, float *y, int64_t outer, int64_t axis_len, int64_t inner,
                                  const float *scale, hipStream_t s) {
    const int64_t n = outer * axis_len * inner;
    if (n == 0) return hipSuccess;
    const bool quad = axis_len == 1 || inner % 4 == 0;
    const int64_t n4 = (quad && aligned(x, 4) && aligned(y, 16)) ? n / 4 : 0;
    hipLaunchKernelGGL(k_dequantize_e5m2, dim3(grid_for(n4 ? n4 : n)), dim3(kThreads), 0, s, x, y, n, n4, axis_len,
                       inner, scale);
    return hipGetLastError();
}

hipError_t launch_fp8_binary(int op, int fmt, const void *a, const void *b, void *y, int64_t n, bool same_shape,
                             const BcastGeom &g, hipStream_t s) {
    if (n == 0) return hipSuccess;
    switch (fmt) {
    case kFmtFloat: return binary_fmt<kFmtFloat>(op, a, b, y, n, same_shape, g, s);
    case kFmtE4M3: return binary_fmt<kFmtE4M3>(op, a, b, y, n, same_shape, g, s);
    default: return binary_fmt<kFmtE5M2>(op, a, b, y, n, same_shape, g, s);
    }
}

}  // namespace lcml
