// quantize.hip -- QuantizeLinear / DequantizeLinear / amax kernels (gfx950).
//
// All three are HBM-bound streaming kernels (4 B in + 1 B out per element
// for quantize, 1 B in + 4 B out for dequantize).  The vector paths move one
// float4 <-> one 32-bit code word per lane per instruction, so a wavefront
// instruction touches 1 KB (fp32 side) or 256 B (fp8 side) of contiguous
// memory, with eight such float4s per thread in flight.
#include "lcml_internal.hpp"

namespace lcml {
namespace {

constexpr int kThreads = 256;

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

// four elements of one per-tensor scale (reciprocal division + hardware
// conversion, both exact stand-ins for the reference's x / s and encoder)
__device__ inline uint32_t enc4(f4 v, const Recip &d) { return quantize4(v.x, v.y, v.z, v.w, d); }


// Vector path, per-tensor or per-axis with inner % 4 == 0 (one scale per
// float4); requires x 16-byte and y 4-byte aligned.  Each thread encodes kU
// float4s per pass, taken kThreads apart so that every load instruction of a
// wavefront reads 1 KB and every store writes 256 contiguous bytes (kU = 4
// measured a little faster than 8 or 16 on 16M-45M element tensors).  The first pass's loads are issued before
// the scale is known (with a dynamic scale, its reduction from the partial
// maxima overlaps them) and each later pass's before the previous pass's
// stores.
constexpr int kU = 4;

template <bool FROM_AMAX>
__global__ __launch_bounds__(kThreads) void k_quantize_vec(const float *__restrict__ x,
                                                           uint8_t *__restrict__ y, int64_t n4,
                                                           int64_t axis_len, int64_t inner,
                                                           const float *__restrict__ scale,
                                                           const uint32_t *__restrict__ part, int npart,
                                                           float *__restrict__ scale_out) {
    __shared__ float red[kThreads / 64];
    const f4 *x4 = reinterpret_cast<const f4 *>(x);
    uint32_t *y4 = reinterpret_cast<uint32_t *>(y);
    const int64_t stride = (int64_t)gridDim.x * kThreads * kU;
    int64_t i0 = (int64_t)blockIdx.x * kThreads * kU + threadIdx.x;
    f4 v[kU];
    auto load = [&](int64_t b) {
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int64_t i = b + (int64_t)u * kThreads;
            v[u] = i < n4 ? __builtin_nontemporal_load(x4 + i) : f4{0.f, 0.f, 0.f, 0.f};
        }
    };
    load(i0);
    float s_tensor = 1.0f;
    if (FROM_AMAX) {
        s_tensor = scale_from_partials<kThreads>(part, npart, red);
        if (scale_out && blockIdx.x == 0 && threadIdx.x == 0) *scale_out = s_tensor;
    } else if (axis_len == 1) {
        s_tensor = scale[0];
    }
    const Recip d_tensor = make_recip(s_tensor);
    // per-tensor: the scale's range test is uniform, one branch outside the
    // loop; per-axis: a scale (and its test) per float4
    auto run = [&](auto mode) {
        constexpr int MODE = decltype(mode)::value;  // 0: per-axis, 1: tensor fast, 2: tensor IEEE
        for (; i0 < n4; i0 += stride) {
            uint32_t code[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                const int64_t i = i0 + (int64_t)u * kThreads;
                if constexpr (MODE == 0)
                    code[u] = enc4(v[u], make_recip(scale[((i * 4) / inner) % axis_len]));
                else
                    code[u] = quantize4_t<MODE == 1>(v[u].x, v[u].y, v[u].z, v[u].w, d_tensor);
            }
            if (i0 + stride < n4) load(i0 + stride);
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                const int64_t i = i0 + (int64_t)u * kThreads;
                if (i < n4) y4[i] = code[u];
            }
        }
    };
    if (!FROM_AMAX && axis_len != 1)
        run(std::integral_constant<int, 0>{});
    else if (d_tensor.fast)
        run(std::integral_constant<int, 1>{});
    else
        run(std::integral_constant<int, 2>{});
}

// Scalar path: any alignment, any per-axis layout, and the vector tail.
template <bool FROM_AMAX>
__global__ __launch_bounds__(kThreads) void k_quantize_scalar(const float *__restrict__ x,
                                                              uint8_t *__restrict__ y, int64_t begin,
                                                              int64_t n, int64_t axis_len, int64_t inner,
                                                              const float *__restrict__ scale,
                                                              const uint32_t *__restrict__ part, int npart,
                                                              float *__restrict__ scale_out) {
    __shared__ float red[kThreads / 64];
    int64_t stride = (int64_t)gridDim.x * kThreads;
    float s_amax = FROM_AMAX ? scale_from_partials<kThreads>(part, npart, red) : 0.0f;
    if (FROM_AMAX && scale_out && blockIdx.x == 0 && threadIdx.x == 0) *scale_out = s_amax;
    for (int64_t i = begin + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
        float s = FROM_AMAX ? s_amax : scale[axis_len == 1 ? 0 : (i / inner) % axis_len];
        y[i] = (uint8_t)e4m3_encode(__fdiv_rn(x[i], s));
    }
}

// DequantizeLinear: y = to_float(q) * s.  v_cvt_pk_f32_fp8 decodes OCP
// E4M3FN, which is the reference's to_float on every code (0x7f/0xff -> NaN,
// 0x80 -> -0.0, subnormals m*2^-9).
__device__ inline void dec4(uint32_t w, float s, f4 &o) {
    f2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
    f2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
    o.x = lo.x * s; o.y = lo.y * s; o.z = hi.x * s; o.w = hi.y * s;
}

// Same shape as k_quantize_vec with kUd 32-bit code words per thread,
// kThreads apart; requires q 4-byte and y 16-byte aligned, inner % 4 == 0
// per axis.
constexpr int kUd = 8;

__global__ __launch_bounds__(kThreads) void k_dequantize_vec(const uint8_t *__restrict__ q,
                                                             float *__restrict__ y, int64_t n4,
                                                             int64_t axis_len, int64_t inner,
                                                             const float *__restrict__ scale) {
    const uint32_t *q4 = reinterpret_cast<const uint32_t *>(q);
    f4 *y4 = reinterpret_cast<f4 *>(y);
    const float s_tensor = axis_len == 1 ? scale[0] : 0.0f;
    const int64_t stride = (int64_t)gridDim.x * kThreads * kUd;
    for (int64_t i0 = (int64_t)blockIdx.x * kThreads * kUd + threadIdx.x; i0 < n4; i0 += stride) {
        uint32_t w[kUd];
#pragma unroll
        for (int u = 0; u < kUd; ++u) {
            const int64_t i = i0 + (int64_t)u * kThreads;
            w[u] = i < n4 ? __builtin_nontemporal_load(q4 + i) : 0u;
        }
#pragma unroll
        for (int u = 0; u < kUd; ++u) {
            const int64_t i = i0 + (int64_t)u * kThreads;
            const float sc = axis_len == 1 ? s_tensor : scale[((i * 4) / inner) % axis_len];
            f4 o;
            dec4(w[u], sc, o);
            if (i < n4) y4[i] = o;
        }
    }
}

__global__ __launch_bounds__(kThreads) void k_dequantize_scalar(const uint8_t *__restrict__ q,
                                                                float *__restrict__ y, int64_t begin,
                                                                int64_t n, int64_t axis_len, int64_t inner,
                                                                const float *__restrict__ scale) {
    int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = begin + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
        float s = scale[axis_len == 1 ? 0 : (i / inner) % axis_len];
        f2 v = __builtin_amdgcn_cvt_pk_f32_fp8((int)q[i], false);
        y[i] = v.x * s;
    }
}

// max |x| over non-NaN elements of one thread's values
__device__ inline float absmax_acc(float m, float v) {
    float a = fabsf(v);
    return a > m ? a : m;  // NaN compares false and is skipped
}

constexpr int kAmaxThreads = 512;
constexpr int kAmaxU = 8;

// this workgroup's max |x| over its grid-stride share (8 float4 loads in
// flight per thread); every thread gets the result
__device__ inline float wg_amax(const float *__restrict__ x, int64_t n, float *red) {
    float m = 0.0f;
    bool vec = (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    const int64_t nv = vec ? n / 4 : 0;
    const f4 *x4 = reinterpret_cast<const f4 *>(x);
    const int64_t stride = (int64_t)gridDim.x * kAmaxThreads * kAmaxU;
    for (int64_t i0 = (int64_t)blockIdx.x * kAmaxThreads * kAmaxU + threadIdx.x; i0 < nv; i0 += stride) {
        f4 v[kAmaxU];
#pragma unroll
        for (int u = 0; u < kAmaxU; ++u) {
            const int64_t i = i0 + (int64_t)u * kAmaxThreads;
            // plain loads (not non-temporal): a dynamic quantisation's
            // encode pass re-reads x at once, last-read chunks first
            // (k_quantize_after_amax), and finds them in its XCD's L2
            v[u] = i < nv ? x4[i] : f4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < kAmaxU; ++u) {
            m = absmax_acc(m, v[u].x); m = absmax_acc(m, v[u].y);
            m = absmax_acc(m, v[u].z); m = absmax_acc(m, v[u].w);
        }
    }
    for (int64_t i = nv * 4 + (int64_t)blockIdx.x * kAmaxThreads + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kAmaxThreads)
        m = absmax_acc(m, x[i]);
    return block_max<kAmaxThreads>(m, red);
}

// amax into one word: one atomic max per workgroup on the fp32 bits
// (non-negative floats order like their unsigned bit patterns); the grid is
// capped at 256 workgroups so the same-address atomics stay few.
__global__ __launch_bounds__(kAmaxThreads) void k_amax(const float *__restrict__ x, int64_t n,
                                                       uint32_t *__restrict__ amax_bits) {
    __shared__ float red[kAmaxThreads / 64];
    const float m = wg_amax(x, n, red);
    if (threadIdx.x == 0) atomicMax(amax_bits, f32_bits(m));
}

// Partial maxima: workgroup b stores its maximum (fp32 bits) in part[b].
// Every entry is written, so the buffer needs no clearing and no atomics are
// involved; the consumer reduces the gridDim.x entries itself
// (scale_from_partials).
__global__ __launch_bounds__(kAmaxThreads) void k_amax_partials(const float *__restrict__ x, int64_t n,
                                                                uint32_t *__restrict__ part) {
    __shared__ float red[kAmaxThreads / 64];
    const float m = wg_amax(x, n, red);
    if (threadIdx.x == 0) part[blockIdx.x] = f32_bits(m);
}

// The encode pass of a dynamic quantisation right after k_amax_partials, on
// the same grid: workgroup b encodes the chunks of x that workgroup b of the
// amax pass read (same XCD, same L2), last-read chunk first, so the tail of
// x that is still in the L2s is read from there before it is evicted
// (4096x4096: 29.5 -> 26.6 us for both passes, 4096x11008: 67.8 -> 62.6 us,
// bit-identical).  Each workgroup reduces the partial maxima to the scale
// while its first loads are in flight.  Requires x 16-byte and y 4-byte
// aligned, n % 4 == 0 (nv = n / 4 float4 groups).
__global__ __launch_bounds__(kAmaxThreads) void k_quantize_after_amax(const float *__restrict__ x,
                                                                     uint8_t *__restrict__ y, int64_t nv,
                                                                     const uint32_t *__restrict__ part, int npart,
                                                                     float *__restrict__ scale_out) {
    __shared__ float red[kAmaxThreads / 64];
    const f4 *x4 = reinterpret_cast<const f4 *>(x);
    uint32_t *y4 = reinterpret_cast<uint32_t *>(y);
    const int64_t stride = (int64_t)gridDim.x * kAmaxThreads * kAmaxU;
    const int64_t first = (int64_t)blockIdx.x * kAmaxThreads * kAmaxU + threadIdx.x;
    // this thread's last chunk of the amax pass's grid-stride walk (-1: none)
    int64_t i0 = first < nv ? first + ((nv - 1 - first) / stride) * stride : -1;
    f4 v[kAmaxU];
    auto load = [&](int64_t b) {
#pragma unroll
        for (int u = 0; u < kAmaxU; ++u) {
            const int64_t i = b + (int64_t)u * kAmaxThreads;
            v[u] = b >= 0 && i < nv ? x4[i] : f4{0.f, 0.f, 0.f, 0.f};
        }
    };
    load(i0);
    const float s_tensor = scale_from_partials<kAmaxThreads>(part, npart, red);
    if (scale_out && blockIdx.x == 0 && threadIdx.x == 0) *scale_out = s_tensor;
    const Recip d = make_recip(s_tensor);
    // the scale's range test is uniform: one branch outside the loop
    auto run = [&](auto fast) {
        for (; i0 >= 0; i0 -= stride) {
            uint32_t code[kAmaxU];
#pragma unroll
            for (int u = 0; u < kAmaxU; ++u)
                code[u] = quantize4_t<decltype(fast)::value>(v[u].x, v[u].y, v[u].z, v[u].w, d);
            if (i0 - stride >= 0) load(i0 - stride);
#pragma unroll
            for (int u = 0; u < kAmaxU; ++u) {
                const int64_t i = i0 + (int64_t)u * kAmaxThreads;
                if (i < nv) y4[i] = code[u];
            }
        }
    };
    if (d.fast)
        run(std::true_type{});
    else
        run(std::false_type{});
}

__global__ void k_fill_u32(uint32_t *p, uint32_t v, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ void k_amax_to_float(const uint32_t *amax_bits, float *out) {
    if (threadIdx.x == 0) *out = bits_f32(*amax_bits);
}

// Dynamic quantisation of a small tensor in ONE launch with no workspace:
// each of the P = ceil(n/4096) workgroups loads the whole tensor (float4
// loads, L2-resident after the first workgroup touches it) and reduces its
// amax, then encodes only its own 4096-element slice from the registers it
// already holds, so the encode work is spread over P CUs and x is read once
// per workgroup.
constexpr int kSmallThreads = 1024;
constexpr int64_t kSmallMax = 65536;
constexpr int kRedThreads = 1024;

__global__ __launch_bounds__(kRedThreads) void k_quantize_dynamic_spread(
    const float *__restrict__ x, uint8_t *__restrict__ y, int64_t n4, float *__restrict__ scale_out) {
    __shared__ float red[kRedThreads / 64];
    const f4 *x4 = reinterpret_cast<const f4 *>(x);
    float m = 0.0f;
    // 1024 threads x 16 float4 = the whole (at most 64K-element) tensor in
    // one round trip; thread t holds float4 t + 1024*u in v[u]
    constexpr int U = 16;
    f4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t i = threadIdx.x + (int64_t)u * kRedThreads;
        v[u] = i < n4 ? x4[i] : f4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        m = absmax_acc(m, v[u].x); m = absmax_acc(m, v[u].y);
        m = absmax_acc(m, v[u].z); m = absmax_acc(m, v[u].w);
    }
    m = block_max<kRedThreads>(m, red);
    const float s = scale_from_amax_bits(f32_bits(m));
    const Recip d = make_recip(s);
    // workgroup b encodes float4s b*1024 + t, which thread t already holds
    // in v[b]: no second read of x
    f4 mine = v[0];
#pragma unroll
    for (int u = 1; u < U; ++u)
        if ((int)blockIdx.x == u) mine = v[u];
    const int64_t i = (int64_t)blockIdx.x * kRedThreads + threadIdx.x;
    if (i < n4) reinterpret_cast<uint32_t *>(y)[i] = enc4(mine, d);
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = s;
}

// Scalar fallback (unaligned pointers or n % 4 != 0): amax pass, then an
// encode pass that re-reads x.
__global__ __launch_bounds__(kSmallThreads) void k_quantize_dynamic_small(
    const float *__restrict__ x, uint8_t *__restrict__ y, int64_t n, float *__restrict__ scale_out) {
    __shared__ float red[kSmallThreads / 64];
    float m = 0.0f;
    for (int64_t i = threadIdx.x; i < n; i += kSmallThreads) m = absmax_acc(m, x[i]);
    m = block_max<kSmallThreads>(m, red);
    const float s = scale_from_amax_bits(f32_bits(m));
    for (int64_t i = threadIdx.x; i < n; i += kSmallThreads) y[i] = (uint8_t)e4m3_encode(__fdiv_rn(x[i], s));
    if (threadIdx.x == 0) *scale_out = s;
}

int grid_for(int64_t work_items, int64_t cap = 4096) {
    int64_t g = (work_items + kThreads - 1) / kThreads;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (int)g;
}

// workgroups for the vector kernels: u float4 / code words per thread per
// pass, at most 4096 workgroups (grid-stride beyond)
int grid_vec(int64_t n4, int u) {
    int64_t g = (n4 + (int64_t)kThreads * u - 1) / ((int64_t)kThreads * u);
    return (int)(g < 1 ? 1 : (g > 4096 ? 4096 : g));
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
bool aligned4(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 3) == 0; }

}  // namespace

hipError_t launch_quantize(const float *x, uint8_t *y, int64_t outer, int64_t axis_len,
                           int64_t inner, const float *scale, hipStream_t s) {
    int64_t n = outer * axis_len * inner;
    if (n == 0) return hipSuccess;
    const bool quad_uniform = axis_len == 1 || inner % 4 == 0;
    const int64_t n4 = (aligned16(x) && aligned4(y) && quad_uniform) ? n / 4 : 0;
    if (n4)
        hipLaunchKernelGGL(k_quantize_vec<false>, dim3(grid_vec(n4, kU)), dim3(kThreads), 0, s, x, y, n4, axis_len,
                           inner, scale, nullptr, 0, nullptr);
    if (n4 * 4 < n)
        hipLaunchKernelGGL(k_quantize_scalar<false>, dim3(grid_for(n - n4 * 4)), dim3(kThreads), 0, s, x, y,
                           n4 * 4, n, axis_len, inner, scale, nullptr, 0, nullptr);
    return hipGetLastError();
}

hipError_t launch_dequantize(const uint8_t *x, float *y, int64_t outer, int64_t axis_len,
                             int64_t inner, const float *scale, hipStream_t s) {
    int64_t n = outer * axis_len * inner;
    if (n == 0) return hipSuccess;
    const bool quad_uniform = axis_len == 1 || inner % 4 == 0;
    const int64_t n4 = (aligned4(x) && aligned16(y) && quad_uniform) ? n / 4 : 0;
    if (n4)
        hipLaunchKernelGGL(k_dequantize_vec, dim3(grid_vec(n4, kUd)), dim3(kThreads), 0, s, x, y, n4, axis_len, inner,
                           scale);
    if (n4 * 4 < n)
        hipLaunchKernelGGL(k_dequantize_scalar, dim3(grid_for(n - n4 * 4)), dim3(kThreads), 0, s, x, y, n4 * 4, n,
                           axis_len, inner, scale);
    return hipGetLastError();
}

hipError_t launch_fill_u32(uint32_t *p, uint32_t v, int64_t n, hipStream_t s) {
    hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, v, n);
    return hipGetLastError();
}

hipError_t launch_amax(const float *x, int64_t n, uint32_t *amax_bits, hipStream_t s) {
    int64_t g = (n / 4 + (int64_t)kAmaxThreads * kAmaxU - 1) / ((int64_t)kAmaxThreads * kAmaxU);
    g = g < 1 ? 1 : (g > 256 ? 256 : g);
    hipLaunchKernelGGL(k_amax, dim3((unsigned)g), dim3(kAmaxThreads), 0, s, x, n, amax_bits);
    return hipGetLastError();
}

int amax_partials_count(int64_t n) {
    // one workgroup per CU at most (grid-stride beyond), which measured
    // faster than 512 or 1024 workgroups on 16M-45M element tensors
    constexpr int64_t kGrid = 256;
    static_assert(kGrid <= kMaxAmaxPartials, "partials fit the workspace");
    int64_t g = (n / 4 + (int64_t)kAmaxThreads * kAmaxU - 1) / ((int64_t)kAmaxThreads * kAmaxU);
    return (int)(g < 1 ? 1 : (g > kGrid ? kGrid : g));
}

hipError_t launch_amax_partials(const float *x, int64_t n, uint32_t *part, int *npart, hipStream_t s) {
    const int64_t g = amax_partials_count(n);
    *npart = (int)g;
    hipLaunchKernelGGL(k_amax_partials, dim3((unsigned)g), dim3(kAmaxThreads), 0, s, x, n, part);
    return hipGetLastError();
}

hipError_t launch_amax_to_float(const uint32_t *amax_bits, float *out, hipStream_t s) {
    hipLaunchKernelGGL(k_amax_to_float, dim3(1), dim3(64), 0, s, amax_bits, out);
    return hipGetLastError();
}

// Dynamic per-tensor quantisation.  Small tensors: one workgroup, one launch.
// Larger: partial maxima into `work` (kMaxAmaxPartials words), then the
// encode, whose every workgroup reduces them to the scale.
hipError_t launch_quantize_dynamic(const float *x, uint8_t *y, int64_t n, float *scale_out,
                                   uint32_t *work, hipStream_t s) {
    if (n <= kSmallMax) {
        if (n % 4 == 0 && aligned16(x) && (reinterpret_cast<uintptr_t>(y) & 3) == 0) {
            // one float4 per thread in the encode pass: ceil(n4 / 1024) <= 16 workgroups
            const int64_t n4 = n / 4;
            int p = (int)((n4 + kRedThreads - 1) / kRedThreads);
            p = p < 1 ? 1 : p;
            hipLaunchKernelGGL(k_quantize_dynamic_spread, dim3(p), dim3(kRedThreads), 0, s, x, y, n4, scale_out);
        } else
            hipLaunchKernelGGL(k_quantize_dynamic_small, dim3(1), dim3(kSmallThreads), 0, s, x, y, n,
                               scale_out);
        return hipGetLastError();
    }
    // two launches: partial maxima into `work`, then the encode kernel(s),
    // each workgroup of which reduces the partials to the scale
    int npart = 0;
    hipError_t err = launch_amax_partials(x, n, work, &npart, s);
    if (err != hipSuccess) return err;
    if (n % 4 == 0 && aligned16(x) && aligned4(y)) {
        hipLaunchKernelGGL(k_quantize_after_amax, dim3((unsigned)npart), dim3(kAmaxThreads), 0, s, x, y, n / 4, work,
                           npart, scale_out);
        return hipGetLastError();
    }
    return launch_quantize_dynamic_parts(x, y, n, work, npart, scale_out, s);
}

hipError_t launch_quantize_dynamic_parts(const float *x, uint8_t *y, int64_t n, const uint32_t *part, int npart,
                                         float *scale_out, hipStream_t s) {
    const int64_t n4 = (aligned16(x) && aligned4(y)) ? n / 4 : 0;
    if (n4)
        hipLaunchKernelGGL(k_quantize_vec<true>, dim3(grid_vec(n4, kU)), dim3(kThreads), 0, s, x, y, n4, (int64_t)1,
                           n, nullptr, part, npart, scale_out);
    if (n4 * 4 < n)
        hipLaunchKernelGGL(k_quantize_scalar<true>, dim3(grid_for(n - n4 * 4)), dim3(kThreads), 0, s, x, y,
                           n4 * 4, n, (int64_t)1, n, nullptr, part, npart, n4 ? nullptr : scale_out);
    return hipGetLastError();
}

}  // namespace lcml
