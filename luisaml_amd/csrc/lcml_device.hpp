// lcml_device.hpp -- scalar helpers shared by the gfx950 kernels and the
// host-side launch code: the E4M3 encoder, bf16 rounding, the epilogue
// activations and the epilogue parameter block.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace lcml {

__host__ __device__ inline uint32_t f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }
__host__ __device__ inline float bits_f32(uint32_t u) { return __builtin_bit_cast(float, u); }

// fp32 -> E4M3FN with the reference encoder's exact behaviour
// (FP8E4M3FN::from_float, include/onnx/fp_quantized.h:149-223):
//   NaN -> 0x7f; +-0 -> 0x00; |x| > 448 or inf -> sign|0x7e;
//   otherwise round to nearest even; a result of zero keeps the sign (0x80).
// Written on the fp32 bit pattern (integer shifts, no frexp/floor), which is
// the same rounding: the 24-bit significand is shifted right by 20 bits for
// normal E4M3 results and by 141-e bits for subnormal ones, the remainder is
// compared with the halfway point, and a carry out of the 3-bit mantissa
// increments the exponent field through the integer add.
__host__ __device__ inline uint32_t e4m3_encode(float x) {
    uint32_t u = f32_bits(x);
    uint32_t s = (u >> 24) & 0x80u;
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return 0x7fu;      // NaN, sign ignored
    if (a > 0x43e00000u) return s | 0x7eu;  // > 448 and inf saturate
    if (a <= 0x3a800000u)                   // |x| <= 2^-10 rounds to zero
        return a == 0 ? 0u : s;             // -0.0 -> 0x00, tiny -> signed 0
    uint32_t e = a >> 23;                   // 117 .. 135
    uint32_t mant = (a & 0x7fffffu) | 0x800000u;
    uint32_t shift = e >= 121u ? 20u : 141u - e;
    uint32_t q = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    q += (rem > half || (rem == half && (q & 1u))) ? 1u : 0u;
    uint32_t code = e >= 121u ? ((e - 121u) << 3) + q : q;
    if (code > 0x7eu) code = 0x7eu;
    return code == 0 ? s : (s | code);
}

// Two fp32 -> E4M3FN codes (a in bits 0-7, b in bits 8-15) through the
// hardware conversion v_cvt_pk_fp8_f32 (round to nearest even into OCP
// E4M3FN), with the reference encoder's special cases put around it:
//   * clamping to +-448 first gives its saturation of |x| > 448 and of +-inf
//     (every finite value above 448 encodes to 0x7e, as does 448 itself);
//   * adding +0.0 turns -0.0 into +0.0 (the reference encodes both zeros as
//     0x00, while a nonzero value that underflows keeps its sign: 0x80);
//   * NaN is patched to 0x7f.
// Equal to e4m3_encode on all 2^32 fp32 inputs (checked exhaustively on
// gfx950 against the integer encoder above).
__device__ inline uint32_t e4m3x2_hw(float a, float b) {
    const float ca = __builtin_amdgcn_fmed3f(a + 0.0f, -448.0f, 448.0f);
    const float cb = __builtin_amdgcn_fmed3f(b + 0.0f, -448.0f, 448.0f);
    uint32_t v = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(ca, cb, 0, false) & 0xffffu;
    if (a != a) v = (v & 0xff00u) | 0x7fu;
    if (b != b) v = (v & 0x00ffu) | 0x7f00u;
    return v;
}

// Two fp32 values -> two E5M2 codes in bytes 0..1, as the reference's
// FP8E5M2::from_float (include/onnx/fp_quantized.h:272-346): NaN -> 0x7f,
// +-0 -> 0x00, |v| > 57344 and +-inf -> sign|0x7c (infinity: this encoder
// does not saturate), otherwise round to nearest even with signed underflow.
// The rounding is v_cvt_pk_bf8_f32 (OCP E5M2) on v + 0.0, which turns -0
// into +0; NaN and the overflow range are selected explicitly.
__device__ inline uint32_t e5m2_fix(float v, uint32_t hw) {
    if (v != v) return 0x7fu;
    if (fabsf(v) > 57344.0f) return v < 0.0f ? 0xfcu : 0x7cu;
    return hw;
}

__device__ inline uint32_t e5m2x2_hw(float a, float b) {
    const uint32_t v = (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(a + 0.0f, b + 0.0f, 0, false);
    return e5m2_fix(a, v & 0xffu) | (e5m2_fix(b, (v >> 8) & 0xffu) << 8);
}

// Division by a scale that is fixed for many elements, rounded exactly like
// IEEE x / s.  With r = RN(1/s), q0 = RN(x*r) is within one ulp of x/s and
// one Newton correction q = RN(q0 + RN(x - q0*s)*r) (the residual is exact
// under fma) is the correctly rounded quotient (Markstein's theorem), as long
// as nothing underflows.  Guards:
//   * s outside [2^-60, 2^40] (1/s near the ends of the exponent range):
//     plain IEEE division throughout;
//   * 0 < |q0| < 2^-100 (the residual may be subnormal): IEEE division for
//     that element; the quotient only decides between +-0 there;
//   * q0 = +-inf (x/s beyond the fp32 range): q0 itself;
//   * x = +-0 gives +0 (-0 / s would be -0; both encode to 0x00) and NaN
//     stays NaN, which is all the encoder needs.
// Checked on gfx950 against __fdiv_rn for 184 scales spread over the fast
// range, each against all 2^32 fp32 x: every quotient with |q| >= 2^-11 (the
// smallest magnitude the E4M3 encoding depends on) agrees bit for bit, and
// all E4M3 encodings agree.
struct Recip {
    float s, r;
    bool fast;
};

__device__ inline Recip make_recip(float s) {
    Recip d;
    d.s = s;
    d.r = __fdiv_rn(1.0f, s);
    d.fast = s >= 0x1p-60f && s <= 0x1p40f;
    return d;
}

// x / s for d.fast scales.  The IEEE fallback for a tiny q0 sits under a
// wavefront-uniform branch (ballot) that the empty volatile asm keeps the
// compiler from if-converting (it would otherwise run the division sequence
// for every element and select), so the common case costs three VALU
// operations and a few compares.
__device__ inline float div_fast(float x, const Recip &d) {
    const float q0 = x * d.r;
    float q = fmaf(fmaf(-q0, d.s, x), d.r, q0);
    const bool tiny = q0 != 0.0f && fabsf(q0) < 0x1p-100f;
    if (__builtin_amdgcn_ballot_w64(tiny) != 0) {
        asm volatile("");
        if (tiny) q = __fdiv_rn(x, d.s);
    }
    if (fabsf(q0) == __builtin_inff()) q = q0;
    return q;
}

__device__ inline float div_by(float x, const Recip &d) { return d.fast ? div_fast(x, d) : __fdiv_rn(x, d.s); }

// a / 448 as div_fast's corrected product with r = RN(1/448): equal to the
// IEEE quotient for every a in [2^-100, FLT_MAX], checked on all of them
// (tests/test_oracle_codec.py, host build of this function)
__host__ __device__ inline float div448_corrected(float a) {
    constexpr float r = 1.0f / 448.0f;
    const float q0 = a * r;
    return fmaf(fmaf(-q0, 448.0f, a), r, q0);
}

// dynamic per-tensor scale from the fp32 bits of amax = max |x| over the
// non-NaN elements: amax / 448, or 1 when that is not a positive finite
// number.  On the critical path of the dynamic quantisers, so the quotient
// is div448_corrected where that is exact; zero, tiny amax and inf take the
// division.
__device__ inline float scale_from_amax_bits(uint32_t bits) {
    const float a = bits_f32(bits);
    float s = a >= 0x1p-100f && a <= 0x1.fffffep127f ? div448_corrected(a) : __fdiv_rn(a, 448.0f);
    if (!(s > 0.0f) || __builtin_isinf(s)) s = 1.0f;
    return s;
}

// max over a wavefront / a workgroup of THREADS threads (red: THREADS/64
// floats of LDS) of values m >= 0 (maxima of |x| with NaN skipped); every
// thread gets the result.  For m >= 0 the max of the bit patterns is the max
// of the values: within each 16-lane row by DPP shifts (lane 15 of a row ends
// with the row's max; lanes shifted in from outside the row read 0), then the
// four rows' lanes 15 by readlane.  A few VALU cycles, where a __shfl_xor
// ladder is six LDS permute round trips.
__device__ inline float wave_max(float m) {
    int b = __builtin_bit_cast(int, m);
    b = max(b, __builtin_amdgcn_update_dpp(0, b, 0x111, 0xf, 0xf, true));  // row_shr:1
    b = max(b, __builtin_amdgcn_update_dpp(0, b, 0x112, 0xf, 0xf, true));  // row_shr:2
    b = max(b, __builtin_amdgcn_update_dpp(0, b, 0x114, 0xf, 0xf, true));  // row_shr:4
    b = max(b, __builtin_amdgcn_update_dpp(0, b, 0x118, 0xf, 0xf, true));  // row_shr:8
    const int r0 = __builtin_amdgcn_readlane(b, 15), r1 = __builtin_amdgcn_readlane(b, 31);
    const int r2 = __builtin_amdgcn_readlane(b, 47), r3 = __builtin_amdgcn_readlane(b, 63);
    return __builtin_bit_cast(float, max(max(r0, r1), max(r2, r3)));
}

// (wavefront 0 reduces the wavefront maxima and broadcasts the result through
// red[0]: every thread reading all THREADS/64 of them after one barrier
// measured 0.2 us slower in the small quantise launches)
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

// the dynamic scale from npart partial maxima (fp32 bits of non-negative
// floats, one per workgroup of the amax pass); called by whole workgroups
template <int THREADS>
__device__ inline float scale_from_partials(const uint32_t *part, int npart, float *red) {
    float m = 0.0f;
    for (int i = threadIdx.x; i < npart; i += THREADS) {
        const float v = bits_f32(part[i]);
        m = v > m ? v : m;
    }
    return scale_from_amax_bits(f32_bits(block_max<THREADS>(m, red)));
}

// four consecutive elements quantised with one scale -> four packed codes;
// quantize4_t<FAST> is for loops that test d.fast once outside
template <bool FAST>
__device__ inline uint32_t quantize4_t(float a, float b, float c, float e, const Recip &d) {
    if constexpr (FAST)
        return e4m3x2_hw(div_fast(a, d), div_fast(b, d)) | (e4m3x2_hw(div_fast(c, d), div_fast(e, d)) << 16);
    else
        return e4m3x2_hw(__fdiv_rn(a, d.s), __fdiv_rn(b, d.s)) | (e4m3x2_hw(__fdiv_rn(c, d.s), __fdiv_rn(e, d.s)) << 16);
}

// quantize4_t<true> for inputs known to hold no NaN and no +-inf (a
// workgroup-uniform fact, e.g. from the amax pass) and |x| <= amax with
// s = amax/448 in the fast range: every quotient is finite (|q0| stays
// about 448), so the infinity pass-through of div_fast and the NaN patch of
// e4m3x2_hw never apply; the clamp to +-448 (a quotient may round just past
// it) and the +0.0 (the reference encodes -0 as 0x00) stay.  The
// tiny-quotient fallback is the same as div_fast's, tested once for the four
// values.  Bit-identical to quantize4_t<true> on such inputs.
__device__ inline uint32_t quantize4_clean(float a, float b, float c, float e, const Recip &d) {
    const float q0a = a * d.r, q0b = b * d.r, q0c = c * d.r, q0e = e * d.r;
    float qa = fmaf(fmaf(-q0a, d.s, a), d.r, q0a), qb = fmaf(fmaf(-q0b, d.s, b), d.r, q0b);
    float qc = fmaf(fmaf(-q0c, d.s, c), d.r, q0c), qe = fmaf(fmaf(-q0e, d.s, e), d.r, q0e);
    const bool ta = q0a != 0.0f && fabsf(q0a) < 0x1p-100f, tb = q0b != 0.0f && fabsf(q0b) < 0x1p-100f;
    const bool tc = q0c != 0.0f && fabsf(q0c) < 0x1p-100f, te = q0e != 0.0f && fabsf(q0e) < 0x1p-100f;
    if (__builtin_amdgcn_ballot_w64(ta || tb || tc || te) != 0) {
        asm volatile("");
        if (ta) qa = __fdiv_rn(a, d.s);
        if (tb) qb = __fdiv_rn(b, d.s);
        if (tc) qc = __fdiv_rn(c, d.s);
        if (te) qe = __fdiv_rn(e, d.s);
    }
    auto clamp = [](float q) { return __builtin_amdgcn_fmed3f(q + 0.0f, -448.0f, 448.0f); };
    const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(clamp(qa), clamp(qb), 0, false);
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(clamp(qc), clamp(qe), lo, true);
}

__device__ inline uint32_t quantize4(float a, float b, float c, float e, const Recip &d) {
    return d.fast ? quantize4_t<true>(a, b, c, e, d) : quantize4_t<false>(a, b, c, e, d);
}

// fp32 -> bf16 bits, round to nearest even; NaN stays a quiet NaN.
__host__ __device__ inline uint16_t bf16_rne(float f) {
    uint32_t u = f32_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Abramowitz & Stegun 7.1.26 erf, as in the reference
// (include/onnx/operators/common.h:176-195).
// The reciprocal and the exponential use the hardware approximations
// (v_rcp_f32, v_exp_f32; a few ulp), which keeps GELU epilogues cheap; the
// formula's own error (|err| <= 1.5e-7) is of the same order.
__device__ inline float as_erf(float x) {
    float ax = fabsf(x);
    float t = __builtin_amdgcn_rcpf(1.0f + 0.3275911f * ax);
    float poly = t * (0.254829592f +
                      t * (-0.284496736f + t * (1.421413741f + t * (-1.453152027f + t * 1.061405429f))));
    float r = 1.0f - poly * __expf(-ax * ax);
    return x < 0.0f ? -r : r;
}

enum Act : int { ACT_NONE = 0, ACT_RELU = 1, ACT_GELU_ERF = 2, ACT_GELU_TANH = 3 };

__device__ inline float apply_act(float v, int act) {
    if (act == ACT_RELU) return v > 0.0f ? v : 0.0f;  // max(0, x), unary.cpp:85
    if (act == ACT_GELU_ERF)                           // gelu.cpp:122-126
        return v * 0.5f * (1.0f + as_erf(v * 0.70710678f));
    if (act == ACT_GELU_TANH) {                        // gelu.cpp:84-91
        float inner = 0.79788456f * fmaf(0.044715f * v * v, v, v);
        return v * 0.5f * (1.0f + tanhf(inner));
    }
    return v;
}

// Epilogue of every GEMM kernel:
//   y[m,n] = act(alpha * acc * a_scale * b_scale[n|0] + beta * C[bcast(m,n)])
struct Epilogue {
    const float *a_scale;  // device, 1 entry, or nullptr (= 1)
    const float *b_scale;  // device, 1 or N entries, or nullptr (= 1)
    int b_per_channel;
    float alpha;
    const float *c;  // nullptr: no C
    int c_ndim;
    int64_t c0, c1;
    float beta;
    int act;
    void *y;
    int y_bf16;
    int64_t ldy;
    int64_t M, N;
    // the tile kernels' AMAX instantiation: one word per workgroup, the fp32
    // bits of max |y| over the elements it stores (NaN skipped), the input
    // of the next dynamic quantisation of y; nullptr elsewhere
    uint32_t *amax_part;
};

// Bias under the reference Gemm broadcast rules (gemm.cpp:84-97).
__device__ inline float epi_c(const Epilogue &e, int64_t m, int64_t n) {
    if (e.c_ndim == 0 || (e.c_ndim == 1 && e.c0 == 1)) return e.c[0];
    if (e.c_ndim == 1) return e.c0 == e.N ? e.c[n] : e.c[m];
    int64_t ci = e.c0 == 1 ? 0 : m, cj = e.c1 == 1 ? 0 : n;
    return e.c[ci * e.c1 + cj];
}

__device__ inline float epi_value(const Epilogue &e, float scale_n, int64_t m, int64_t n, float acc) {
    float v = acc * scale_n;
    if (e.alpha != 1.0f) v *= e.alpha;
    if (e.c) v = e.beta == 1.0f ? v + epi_c(e, m, n) : v + e.beta * epi_c(e, m, n);
    return apply_act(v, e.act);
}

// True when C's broadcast value does not depend on the row m (a bias over
// N, or a scalar), so an epilogue with a fixed column per lane reads it once.
__device__ inline bool epi_c_row_invariant(const Epilogue &e) {
    if (e.c_ndim == 0 || (e.c_ndim == 1 && (e.c0 == 1 || e.c0 == e.N))) return true;
    return e.c_ndim == 2 && e.c0 == 1;
}

// epi_value with C's element already read (cv; ignored without C): the same
// operations in the same order
__device__ inline float epi_value_cv(const Epilogue &e, float scale_n, float cv, float acc) {
    float v = acc * scale_n;
    if (e.alpha != 1.0f) v *= e.alpha;
    if (e.c) v = e.beta == 1.0f ? v + cv : v + e.beta * cv;
    return apply_act(v, e.act);
}

// a_scale * b_scale[n] for column n.
__device__ inline float epi_scale(const Epilogue &e, float a_s, int64_t n) {
    float bs = e.b_scale ? (e.b_per_channel ? e.b_scale[n] : e.b_scale[0]) : 1.0f;
    return a_s * bs;
}

__device__ inline void epi_store(const Epilogue &e, int64_t m, int64_t n, float v) {
    if (e.y_bf16)
        reinterpret_cast<uint16_t *>(e.y)[m * e.ldy + n] = bf16_rne(v);
    else
        reinterpret_cast<float *>(e.y)[m * e.ldy + n] = v;
}

// columns n and n + 1 of row m in one store (n even, ldy even: the pair is
// 4- or 8-byte aligned)
__device__ inline void epi_store2(const Epilogue &e, int64_t m, int64_t n, float v0, float v1) {
    if (e.y_bf16)
        reinterpret_cast<uint32_t *>(e.y)[(m * e.ldy + n) >> 1] = (uint32_t)bf16_rne(v0) | ((uint32_t)bf16_rne(v1) << 16);
    else
        reinterpret_cast<float2 *>(e.y)[(m * e.ldy + n) >> 1] = float2{v0, v1};
}

// E4M3 -> bf16 (exact: every E4M3 value is a bf16 value; 0x7f/0xff -> NaN)
// for 8 consecutive bytes (two dwords) with v_cvt_scalef32_pk_bf16_fp8 at
// scale 1.0, giving one 8-element operand of the bf16 MFMAs.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ inline bf16x8 e4m3x8_to_bf16(uint32_t w0, uint32_t w1) {
    bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w0, 1.0f, false);
    bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w0, 1.0f, true);
    bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w1, 1.0f, false);
    bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w1, 1.0f, true);
    return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// Packed weight geometry (see lcml_fp8_pack_weight in include/lcml_fp8.h).
__host__ __device__ inline int64_t pad_to(int64_t x, int64_t m) { return (x + m - 1) / m * m; }
constexpr int kPanelCols = 64;   // columns per panel
constexpr int kChunk = 16;       // bytes per k-chunk
constexpr int kPackK = 128;      // K padding of packed weights

}  // namespace lcml
