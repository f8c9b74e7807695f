// quantize.hip -- QuantizeLinear / DequantizeLinear / amax kernels (gfx950).
//
// All three are HBM-bound streaming kernels (4 B in + 1 B out per element
// for quantize, 1 B in + 4 B out for dequantize).  Each thread moves 16
// elements: four 128-bit fp32 loads and one 128-bit fp8 store (or the
// reverse), so every wavefront instruction touches 1 KB (fp8 side) or 4 KB
// (fp32 side) of contiguous memory.
#include "lcml_internal.hpp"

namespace lcml {
namespace {

constexpr int kThreads = 256;
constexpr int kVec = 16;  // elements per thread per step

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

// four elements of one per-tensor scale (reciprocal division + hardware
// conversion, both exact stand-ins for the reference's x / s and encoder)
__device__ inline uint32_t enc4(f4 v, const Recip &d) { return quantize4(v.x, v.y, v.z, v.w, d); }


// Per-tensor (or per-axis with a 16-element-uniform scale index) vector path.
// grid-stride over 16-element groups; requires x, y 16-byte aligned.
template <bool FROM_AMAX>
__global__ __launch_bounds__(kThreads) void k_quantize_vec(const float *__restrict__ x,
                                                           uint8_t *__restrict__ y, int64_t ngroups,
                                                           int64_t axis_len, int64_t inner,
                                                           const float *__restrict__ scale,
                                                           const uint32_t *__restrict__ amax_bits) {
    float s_tensor = 1.0f;
    if (FROM_AMAX) s_tensor = scale_from_amax_bits(*amax_bits);
    else if (axis_len == 1) s_tensor = scale[0];
    const Recip d_tensor = make_recip(s_tensor);
    int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t g = (int64_t)blockIdx.x * kThreads + threadIdx.x; g < ngroups; g += stride) {
        // per-axis: one scale per 16-element group (inner % 16 == 0)
        const Recip d = (!FROM_AMAX && axis_len != 1) ? make_recip(scale[((g * kVec) / inner) % axis_len]) : d_tensor;
        const f4 *xp = reinterpret_cast<const f4 *>(x + g * kVec);
        f4 v0 = __builtin_nontemporal_load(xp + 0), v1 = __builtin_nontemporal_load(xp + 1);
        f4 v2 = __builtin_nontemporal_load(xp + 2), v3 = __builtin_nontemporal_load(xp + 3);
        u4 out = {enc4(v0, d), enc4(v1, d), enc4(v2, d), enc4(v3, d)};
        *reinterpret_cast<u4 *>(y + g * kVec) = out;
    }
}

// Scalar path: any alignment, any per-axis layout, and the vector tail.
template <bool FROM_AMAX>
__global__ __launch_bounds__(kThreads) void k_quantize_scalar(const float *__restrict__ x,
                                                              uint8_t *__restrict__ y, int64_t begin,
                                                              int64_t n, int64_t axis_len, int64_t inner,
                                                              const float *__restrict__ scale,
                                                              const uint32_t *__restrict__ amax_bits) {
    int64_t stride = (int64_t)gridDim.x * kThreads;
    float s_amax = FROM_AMAX ? scale_from_amax_bits(*amax_bits) : 0.0f;
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

__global__ __launch_bounds__(kThreads) void k_dequantize_vec(const uint8_t *__restrict__ q,
                                                             float *__restrict__ y, int64_t ngroups,
                                                             int64_t axis_len, int64_t inner,
                                                             const float *__restrict__ scale) {
    float s_tensor = axis_len == 1 ? scale[0] : 0.0f;
    int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t g = (int64_t)blockIdx.x * kThreads + threadIdx.x; g < ngroups; g += stride) {
        float s = axis_len == 1 ? s_tensor : scale[((g * kVec) / inner) % axis_len];
        u4 w = __builtin_nontemporal_load(reinterpret_cast<const u4 *>(q + g * kVec));
        f4 o0, o1, o2, o3;
        dec4(w.x, s, o0); dec4(w.y, s, o1); dec4(w.z, s, o2); dec4(w.w, s, o3);
        f4 *yp = reinterpret_cast<f4 *>(y + g * kVec);
        yp[0] = o0; yp[1] = o1; yp[2] = o2; yp[3] = o3;
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

__device__ inline float wave_max(float m) {
    for (int off = 32; off > 0; off >>= 1) {
        float o = __shfl_xor(m, off, 64);
        m = o > m ? o : m;
    }
    return m;
}

template <int THREADS>
__device__ inline float block_max(float m, float *red) {
    m = wave_max(m);
    int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = m;
    __syncthreads();
    if (wave == 0) {
        m = lane < THREADS / 64 ? red[lane] : 0.0f;
        m = wave_max(m);
        if (lane == 0) red[0] = m;
    }
    __syncthreads();
    m = red[0];
    __syncthreads();
    return m;
}

// amax: each block reduces its grid-stride share (8 float4 loads in flight
// per thread), then one atomic max on the fp32 bits (non-negative floats
// order like their unsigned bit patterns).  The grid is capped at 256
// workgroups so the same-address atomics stay few.
constexpr int kAmaxThreads = 512;
constexpr int kAmaxU = 8;

__global__ __launch_bounds__(kAmaxThreads) void k_amax(const float *__restrict__ x, int64_t n,
                                                       uint32_t *__restrict__ amax_bits) {
    __shared__ float red[kAmaxThreads / 64];
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
            v[u] = i < nv ? __builtin_nontemporal_load(x4 + i) : f4{0.f, 0.f, 0.f, 0.f};
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
    m = block_max<kAmaxThreads>(m, red);
    if (threadIdx.x == 0) atomicMax(amax_bits, f32_bits(m));
}

__global__ void k_fill_u32(uint32_t *p, uint32_t v, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ void k_amax_finalize(const uint32_t *amax_bits, float *scale_out) {
    if (threadIdx.x == 0) *scale_out = scale_from_amax_bits(*amax_bits);
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

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

hipError_t launch_quantize(const float *x, uint8_t *y, int64_t outer, int64_t axis_len,
                           int64_t inner, const float *scale, hipStream_t s) {
    int64_t n = outer * axis_len * inner;
    if (n == 0) return hipSuccess;
    bool group_uniform = axis_len == 1 || inner % kVec == 0;
    int64_t ngroups = (aligned16(x) && aligned16(y) && group_uniform) ? n / kVec : 0;
    if (ngroups)
        hipLaunchKernelGGL(k_quantize_vec<false>, dim3(grid_for(ngroups)), dim3(kThreads), 0, s, x, y,
                           ngroups, axis_len, inner, scale, nullptr);
    if (ngroups * kVec < n)
        hipLaunchKernelGGL(k_quantize_scalar<false>, dim3(grid_for(n - ngroups * kVec)), dim3(kThreads),
                           0, s, x, y, ngroups * kVec, n, axis_len, inner, scale, nullptr);
    return hipGetLastError();
}

hipError_t launch_dequantize(const uint8_t *x, float *y, int64_t outer, int64_t axis_len,
                             int64_t inner, const float *scale, hipStream_t s) {
    int64_t n = outer * axis_len * inner;
    if (n == 0) return hipSuccess;
    bool group_uniform = axis_len == 1 || inner % kVec == 0;
    int64_t ngroups = (aligned16(x) && aligned16(y) && group_uniform) ? n / kVec : 0;
    if (ngroups)
        hipLaunchKernelGGL(k_dequantize_vec, dim3(grid_for(ngroups)), dim3(kThreads), 0, s, x, y,
                           ngroups, axis_len, inner, scale);
    if (ngroups * kVec < n)
        hipLaunchKernelGGL(k_dequantize_scalar, dim3(grid_for(n - ngroups * kVec)), dim3(kThreads), 0,
                           s, x, y, ngroups * kVec, n, axis_len, inner, scale);
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

hipError_t launch_amax_to_float(const uint32_t *amax_bits, float *out, hipStream_t s) {
    hipLaunchKernelGGL(k_amax_to_float, dim3(1), dim3(64), 0, s, amax_bits, out);
    return hipGetLastError();
}

// Dynamic per-tensor quantisation.  Small tensors: one workgroup, one launch.
// Larger: zero the amax word, reduce, encode, then write the scale; `work`
// is one device uint32 of scratch (the caller's scale_out is not reused for
// it because the encode kernel reads the amax while running).
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
    hipError_t err = launch_fill_u32(work, 0u, 1, s);
    if (err != hipSuccess) return err;
    err = launch_amax(x, n, work, s);
    if (err != hipSuccess) return err;
    int64_t ngroups = (aligned16(x) && aligned16(y)) ? n / kVec : 0;
    if (ngroups)
        hipLaunchKernelGGL(k_quantize_vec<true>, dim3(grid_for(ngroups)), dim3(kThreads), 0, s, x, y,
                           ngroups, (int64_t)1, n, nullptr, work);
    if (ngroups * kVec < n)
        hipLaunchKernelGGL(k_quantize_scalar<true>, dim3(grid_for(n - ngroups * kVec)), dim3(kThreads),
                           0, s, x, y, ngroups * kVec, n, (int64_t)1, n, nullptr, work);
    hipLaunchKernelGGL(k_amax_finalize, dim3(1), dim3(64), 0, s, work, scale_out);
    return hipGetLastError();
}

}  // namespace lcml
