/*
 * lcml_oracle.c -- CPU oracle for the FP8 (E4M3 / E5M2) quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file restates, on the CPU, the arithmetic
 * of the reference ONNX runtime (LuisaGroup/LuisaML) that the HIP library in
 * luisaml_amd/ replaces.  It is what parity is judged against and the timed CPU
 * baseline; it is never linked into, loaded by or called from the product
 * library.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.
 *
 * What each function follows (reference paths are relative to the reference
 * repository root):
 *   orc_e4m3_from_float   include/onnx/fp_quantized.h:149-223  (line by line)
 *   orc_e4m3_to_float     include/onnx/fp_quantized.h:226-249  (line by line)
 *   orc_e4m3_spec_encode  closed-form specification of the above (independent
 *                         nearest-grid search); pins orc_e4m3_from_float over
 *                         all 2^32 fp32 bit patterns.
 *   orc_dequantize        DequantizeLinear = Cast(fp8->f32) then Mul by the
 *                         scale: src/onnx/operators/cast.cpp:44-48 and
 *                         src/onnx/operators/binary.cpp:347 (one fp32 multiply)
 *   orc_quantize          QuantizeLinear (ONNX opset 21, float8 target,
 *                         saturate=1, zero point 0): from_float(x / scale)
 *                         with an IEEE fp32 divide.  No counterpart in the
 *                         reference (its graph loader rejects the op,
 *                         src/onnx/onnx.cpp:228-229); the numeric core is
 *                         orc_e4m3_from_float.
 *   orc_gemm              src/onnx/operators/gemm.cpp:27-325: per-output
 *                         sequential fma chain over k (155-162), alpha applied
 *                         to the dot (106-110), then beta*C with the reference
 *                         broadcast rules (81-103).
 *   orc_relu              src/onnx/operators/unary.cpp:85
 *   orc_gelu_erf          src/onnx/operators/gelu.cpp:122-126 with the A&S erf
 *                         of include/onnx/operators/common.h:176-195
 *   orc_gelu_tanh         src/onnx/operators/gelu.cpp:84-91
 *   orc_conv2d            src/onnx/operators/conv.cpp:115-207 (direct NCHW
 *                         loop, begin pads, dilation, groups, bias), fp32
 *                         accumulate (the QDQ composition, not the reference's
 *                         half accumulation for fp8 inputs at conv.cpp:67-70)
 *   orc_bf16_rne          closed form: fp32 -> bf16 round to nearest even,
 *                         NaN kept quiet.  No counterpart in the reference.
 *   orc_e5m2_from_float   include/onnx/fp_quantized.h:272-346  (line by line)
 *   orc_e5m2_to_float     include/onnx/fp_quantized.h:350-377  (line by line)
 *   orc_e5m2_spec_encode  closed-form specification of the above; pins it over
 *                         all 2^32 fp32 bit patterns.
 *   orc_half_round        IEEE binary16 round to nearest even (subnormals,
 *                         overflow to inf): the precision of the reference's
 *                         DSL arithmetic on decoded fp8 values (its decoders
 *                         return half, fp_quantized.h:610, 721).
 *   orc_fp8_binary        src/onnx/operators/binary.cpp:184-285 (quantised
 *                         Add/Sub/Mul/Div: decode both operands to half, the
 *                         op in half, encode) and 59-182 (numpy broadcasting);
 *                         the encode is the CPU from_float of the half value.
 *   orc_quantize_e5m2 / orc_dequantize_e5m2
 *                         QuantizeLinear / DequantizeLinear with a
 *                         FLOAT8E5M2 target (ONNX opset 21): from_float(x / s)
 *                         with saturate=1 clamping |x / s| > 57344 (inf
 *                         included) to +-57344; to_float(q) * s.
 *
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off -fopenmp -mavx2 -mfma).
 * -ffp-contract=off keeps every multiply and add separately rounded except
 * where fmaf / _mm256_fmadd_ps is written explicitly, as the reference's
 * fma() is.
 */
#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_API __attribute__((visibility("default")))

static int g_threads = 0; /* 0 = OpenMP default */

ORC_API void orc_set_threads(int n) { g_threads = n; }
ORC_API int orc_get_threads(void) {
    return g_threads > 0 ? g_threads : omp_get_max_threads();
}

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------------ */
/* E4M3FN codec                                                             */
/* ------------------------------------------------------------------------ */

/* Restatement of FP8E4M3FN::from_float, fp_quantized.h:149-223. */
ORC_API uint8_t orc_e4m3_from_float(float v) {
    const int kMantBits = 3, kBias = 7, kInfNanExp = 15;
    const uint8_t kMantMask = 0x07, kSignMask = 0x80;
    if (isnan(v)) return 0x7f;                 /* 151-154 */
    if (v == 0.0f) return 0;                   /* 155-158 (-0.0 -> 0x00) */
    uint32_t sign = 0;
    if (v < 0.0f) { sign = 1; v = -v; }        /* 159-163 */
    const float max_finite = 448.0f;
    if (v > max_finite) return sign ? 0xfe : 0x7e; /* 166-171 */
    int32_t exp;
    float mant = frexpf(v, &exp);              /* 174-178 */
    mant *= 2.0f;
    exp -= 1;
    int32_t e = exp + kBias;                   /* 180 */
    if (e <= 0) {                              /* 181-191 */
        if (e < -kMantBits) return sign ? kSignMask : 0;
        int32_t shift = 1 - e;
        mant = mant / (float)(1 << shift);
        e = 0;
    }
    float mant_q = floorf(mant * (float)(1 << kMantBits)); /* 193-196 */
    float frac = mant * (float)(1 << kMantBits) - mant_q;
    uint8_t m = (uint8_t)((uint8_t)mant_q & kMantMask);
    if (frac > 0.5f || (frac == 0.5f && (m & 1))) { /* 198-205 */
        m += 1;
        if (m > kMantMask) { m = 0; e += 1; }
    }
    if (e >= kInfNanExp) {                     /* 207-213 */
        e = kInfNanExp;
        if (m >= kMantMask) m = kMantMask - 1;
    }
    if (e == 0 && m == 0) return sign ? kSignMask : 0; /* 216-218 */
    return (uint8_t)((sign ? kSignMask : 0) | (uint8_t)(e << kMantBits) | m); /* 221 */
}

/* Restatement of FP8E4M3FN::to_float, fp_quantized.h:226-249. */
ORC_API float orc_e4m3_to_float(uint8_t bits) {
    uint8_t sign = (bits & 0x80) >> 7;
    uint8_t e = (bits >> 3) & 15;
    uint8_t m = bits & 7;
    if (e == 0 && m == 0) return sign ? -0.0f : 0.0f;
    if (e == 15 && m == 7) return u2f(0x7fc00000u); /* quiet NaN */
    float value;
    if (e == 0)
        value = (float)m / (float)(1 << 3) * powf(2.0f, (float)(1 - 7));
    else
        value = (1.0f + (float)m / (float)(1 << 3)) * powf(2.0f, (float)(e - 7));
    return sign ? -value : value;
}

/*
 * Closed-form specification of the encoder, written independently of the
 * frexp/floor algorithm above:
 *   NaN -> 0x7f;  +-0 -> 0x00;  |x| > 448 (incl. inf) -> sign|0x7e;
 *   otherwise the E4M3FN grid point nearest to |x| (exact comparison in
 *   double), ties to the even code; a zero result keeps the sign (0x80).
 */
static double g_grid[127]; /* positive finite codes 0x00..0x7e */
static int g_grid_ready = 0;
static void grid_init(void) {
    if (g_grid_ready) return;
    for (int c = 0; c < 127; ++c) {
        int e = c >> 3, m = c & 7;
        g_grid[c] = e == 0 ? ldexp((double)m, -9) : ldexp(1.0 + m / 8.0, e - 7);
    }
    g_grid_ready = 1;
}

ORC_API uint8_t orc_e4m3_spec_encode(float x) {
    uint32_t u = f2u(x);
    uint32_t s = u >> 31, a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return 0x7f;
    if (a == 0) return 0x00;
    double v = (double)u2f(a);
    if (v > 448.0) return (uint8_t)((s << 7) | 0x7e);
    grid_init();
    int lo = 0, hi = 126; /* g_grid[lo] <= v <= g_grid[hi] */
    while (hi - lo > 1) {
        int mid = (lo + hi) / 2;
        if (g_grid[mid] <= v) lo = mid; else hi = mid;
    }
    int c;
    double dlo = v - g_grid[lo], dhi = g_grid[hi] - v;
    if (dlo < dhi) c = lo;
    else if (dhi < dlo) c = hi;
    else c = (lo & 1) ? hi : lo;
    if (c == 0) return (uint8_t)(s << 7);
    return (uint8_t)((s << 7) | c);
}

/* out[i] = from_float(as_float(first + i)), i < count.  Used by the
 * exhaustive sweeps. */
ORC_API void orc_e4m3_encode_bits(uint32_t first, uint64_t count, uint8_t *out) {
    int nt = orc_get_threads();
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t i = 0; i < (int64_t)count; ++i)
        out[i] = orc_e4m3_from_float(u2f(first + (uint32_t)i));
}

/* Compare the restatement with the closed-form spec over the fp32 bit
 * patterns [first, first+count).  Returns the number of mismatches and the
 * lowest mismatching pattern in *first_bad (unchanged when none). */
ORC_API uint64_t orc_e4m3_sweep_vs_spec(uint32_t first, uint64_t count, uint32_t *first_bad) {
    grid_init();
    uint64_t bad = 0;
    uint32_t lowest = 0xffffffffu;
    int nt = orc_get_threads();
#pragma omp parallel for num_threads(nt) schedule(static) reduction(+ : bad) reduction(min : lowest)
    for (int64_t i = 0; i < (int64_t)count; ++i) {
        uint32_t b = first + (uint32_t)i;
        float x = u2f(b);
        if (orc_e4m3_from_float(x) != orc_e4m3_spec_encode(x)) {
            ++bad;
            if (b < lowest) lowest = b;
        }
    }
    if (bad && first_bad) *first_bad = lowest;
    return bad;
}

/* Round-trip sweep: count codes c with from_float(to_float(c)) != c for
 * finite codes (0x80 maps to 0x00 by the -0.0 rule; NaN codes map to 0x7f). */
ORC_API void orc_e4m3_decode_table(float *out256) {
    for (int c = 0; c < 256; ++c) out256[c] = orc_e4m3_to_float((uint8_t)c);
}

/* fp32 -> bf16, round to nearest even; NaN stays NaN (quiet bit forced). */
ORC_API uint16_t orc_bf16_rne(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

ORC_API void orc_bf16_rne_array(const float *x, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_bf16_rne(x[i]);
}

/* ------------------------------------------------------------------------ */
/* QuantizeLinear / DequantizeLinear                                        */
/* ------------------------------------------------------------------------ */

/*
 * Tensor viewed as [outer, axis_len, inner]; scale has axis_len entries
 * (axis_len == 1: per-tensor).  ONNX opset-21 semantics for float8 targets.
 */
ORC_API void orc_quantize(const float *x, uint8_t *y, int64_t outer, int64_t axis_len,
                          int64_t inner, const float *scale) {
    int nt = orc_get_threads();
#pragma omp parallel for num_threads(nt) schedule(static) collapse(2)
    for (int64_t o = 0; o < outer; ++o)
        for (int64_t a = 0; a < axis_len; ++a) {
            float s = scale[a];
            const float *xp = x + (o * axis_len + a) * inner;
            uint8_t *yp = y + (o * axis_len + a) * inner;
            for (int64_t i = 0; i < inner; ++i) yp[i] = orc_e4m3_from_float(xp[i] / s);
        }
}

ORC_API void orc_dequantize(const uint8_t *q, float *y, int64_t outer, int64_t axis_len,
                            int64_t inner, const float *scale) {
    int nt = orc_get_threads();
#pragma omp parallel for num_threads(nt) schedule(static) collapse(2)
    for (int64_t o = 0; o < outer; ++o)
        for (int64_t a = 0; a < axis_len; ++a) {
            float s = scale[a];
            const uint8_t *qp = q + (o * axis_len + a) * inner;
            float *yp = y + (o * axis_len + a) * inner;
            for (int64_t i = 0; i < inner; ++i) yp[i] = orc_e4m3_to_float(qp[i]) * s;
        }
}

/* max |x| over non-NaN elements (0 for an empty or all-NaN tensor). */
ORC_API float orc_amax(const float *x, int64_t n) {
    float m = 0.0f;
    int nt = orc_get_threads();
#pragma omp parallel for num_threads(nt) schedule(static) reduction(max : m)
    for (int64_t i = 0; i < n; ++i) {
        float a = fabsf(x[i]);
        if (a > m) m = a; /* NaN compares false */
    }
    return m;
}

/*
 * Dynamic E4M3 scale from an amax: amax / 448 when that quotient is a
 * positive finite number, else 1.0 (all-zero, all-NaN or inf-bearing input,
 * or an amax so small the quotient underflows to 0).
 */
ORC_API float orc_scale_from_amax(float amax) {
    float s = amax / 448.0f;
    if (!(s > 0.0f) || isinf(s)) s = 1.0f;
    return s;
}

/* Per-slice amax for per-axis scales: tensor [outer, axis_len, inner]. */
ORC_API void orc_amax_axis(const float *x, int64_t outer, int64_t axis_len, int64_t inner,
                           float *amax_out) {
    for (int64_t a = 0; a < axis_len; ++a) amax_out[a] = 0.0f;
    for (int64_t o = 0; o < outer; ++o)
        for (int64_t a = 0; a < axis_len; ++a) {
            const float *xp = x + (o * axis_len + a) * inner;
            float m = amax_out[a];
            for (int64_t i = 0; i < inner; ++i) {
                float v = fabsf(xp[i]);
                if (v > m) m = v;
            }
            amax_out[a] = m;
        }
}

/* ------------------------------------------------------------------------ */
/* Activations                                                              */
/* ------------------------------------------------------------------------ */

ORC_API float orc_relu(float x) { return x > 0.0f ? x : 0.0f; } /* max(T{0}, x) */

/* A&S 7.1.26 erf, common.h:176-195 (scalar branch). */
static float as_erf(float x) {
    float ax = fabsf(x);
    float t = 1.0f / (1.0f + 0.3275911f * ax);
    float poly = t * (0.254829592f +
                      t * (-0.284496736f + t * (1.421413741f + t * (-1.453152027f + t * 1.061405429f))));
    float result = 1.0f - poly * expf(-ax * ax);
    return x < 0.0f ? -result : result;
}

ORC_API float orc_gelu_erf(float x) { return x * 0.5f * (1.0f + as_erf(x * 0.70710678f)); }

ORC_API float orc_gelu_tanh(float x) {
    float x2 = x * x;
    float inner = 0.79788456f * fmaf(0.044715f * x2, x, x);
    return x * 0.5f * (1.0f + tanhf(inner));
}

enum { ORC_ACT_NONE = 0, ORC_ACT_RELU = 1, ORC_ACT_GELU_ERF = 2, ORC_ACT_GELU_TANH = 3 };

static inline float apply_act(float v, int act) {
    switch (act) {
    case ORC_ACT_RELU: return orc_relu(v);
    case ORC_ACT_GELU_ERF: return orc_gelu_erf(v);
    case ORC_ACT_GELU_TANH: return orc_gelu_tanh(v);
    default: return v;
    }
}

ORC_API void orc_activation(const float *x, float *y, int64_t n, int act) {
    for (int64_t i = 0; i < n; ++i) y[i] = apply_act(x[i], act);
}

/* ------------------------------------------------------------------------ */
/* Gemm                                                                     */
/* ------------------------------------------------------------------------ */

/* Bias value for output (m, n) under the reference broadcast rules,
 * gemm.cpp:84-97.  c_ndim < 0 means "no C". */
static inline float c_value(const float *C, int c_ndim, int64_t c0, int64_t c1, int64_t N,
                            int64_t m, int64_t n) {
    if (c_ndim == 0 || (c_ndim == 1 && c0 == 1)) return C[0];
    if (c_ndim == 1) return c0 == N ? C[n] : C[m];
    int64_t ci = c0 == 1 ? 0 : m, cj = c1 == 1 ? 0 : n;
    return C[ci * c1 + cj];
}

#define MR 6
#define NR 16

/*
 * Y[M,N] = act(alpha * op(A) op(B) + beta * C).
 * op(A) is A [M,K] (transA=0) or A^T of a [K,M] array; op(B) is B [K,N]
 * (transB=0) or B^T of an [N,K] array.  Each output is one sequential fma
 * chain over k = 0..K-1 starting from 0 (gemm.cpp:155-162); the loop nest is
 * tiled over (m, n) only, so that order is kept for every output.
 */
ORC_API void orc_gemm(int64_t M, int64_t N, int64_t K, const float *A, int transA,
                      const float *B, int transB, float alpha, float beta, const float *C,
                      int c_ndim, int64_t c0, int64_t c1, int act, float *Y) {
    int nt = orc_get_threads();
    int64_t mp = (M + MR - 1) / MR, np_ = (N + NR - 1) / NR;
    /* Pack: Ap[mp][k][MR], Bp[np][k][NR], zero padded. */
    size_t abytes = ((size_t)(mp * K * MR) * sizeof(float) + 127) & ~(size_t)63;
    size_t bbytes = ((size_t)(np_ * K * NR) * sizeof(float) + 127) & ~(size_t)63;
    float *Ap = (float *)aligned_alloc(64, abytes);
    float *Bp = (float *)aligned_alloc(64, bbytes);
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t p = 0; p < mp; ++p)
        for (int64_t k = 0; k < K; ++k)
            for (int r = 0; r < MR; ++r) {
                int64_t m = p * MR + r;
                Ap[(p * K + k) * MR + r] =
                    m < M ? (transA ? A[k * M + m] : A[m * K + k]) : 0.0f;
            }
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t p = 0; p < np_; ++p)
        for (int64_t k = 0; k < K; ++k)
            for (int c = 0; c < NR; ++c) {
                int64_t n = p * NR + c;
                Bp[(p * K + k) * NR + c] =
                    n < N ? (transB ? B[n * K + k] : B[k * N + n]) : 0.0f;
            }
    int has_alpha = alpha != 1.0f;
    int has_C = C != NULL && c_ndim >= 0 && beta != 0.0f;
    int beta_is_one = beta == 1.0f;
#pragma omp parallel for num_threads(nt) schedule(dynamic, 1) collapse(2)
    for (int64_t pi = 0; pi < mp; ++pi)
        for (int64_t pj = 0; pj < np_; ++pj) {
            const float *ap = Ap + pi * K * MR;
            const float *bp = Bp + pj * K * NR;
            __m256 acc[MR][2];
            for (int r = 0; r < MR; ++r) acc[r][0] = acc[r][1] = _mm256_setzero_ps();
            for (int64_t k = 0; k < K; ++k) {
                __m256 b0 = _mm256_load_ps(bp + k * NR);
                __m256 b1 = _mm256_load_ps(bp + k * NR + 8);
                for (int r = 0; r < MR; ++r) {
                    __m256 a = _mm256_broadcast_ss(ap + k * MR + r);
                    acc[r][0] = _mm256_fmadd_ps(a, b0, acc[r][0]);
                    acc[r][1] = _mm256_fmadd_ps(a, b1, acc[r][1]);
                }
            }
            float tile[MR][NR];
            for (int r = 0; r < MR; ++r) {
                _mm256_storeu_ps(&tile[r][0], acc[r][0]);
                _mm256_storeu_ps(&tile[r][8], acc[r][1]);
            }
            for (int r = 0; r < MR; ++r) {
                int64_t m = pi * MR + r;
                if (m >= M) break;
                for (int c = 0; c < NR; ++c) {
                    int64_t n = pj * NR + c;
                    if (n >= N) break;
                    float sum = tile[r][c];
                    if (has_alpha) sum *= alpha;
                    if (has_C) {
                        float cv = c_value(C, c_ndim, c0, c1, N, m, n);
                        if (beta_is_one) sum += cv;
                        else sum += beta * cv;
                    }
                    Y[m * N + n] = apply_act(sum, act);
                }
            }
        }
    free(Ap);
    free(Bp);
}

/*
 * Tolerance scale for output (m,n): sum_k |a_mk b_kn| (+ |beta C| when C is
 * present), accumulated in double.  Same operand conventions as orc_gemm.
 */
ORC_API void orc_gemm_abs_bound(int64_t M, int64_t N, int64_t K, const float *A, int transA,
                                const float *B, int transB, float alpha, float beta,
                                const float *C, int c_ndim, int64_t c0, int64_t c1,
                                double *bound) {
    int nt = orc_get_threads();
    int has_C = C != NULL && c_ndim >= 0 && beta != 0.0f;
#pragma omp parallel for num_threads(nt) schedule(dynamic, 4)
    for (int64_t m = 0; m < M; ++m) {
        double *row = bound + m * N;
        for (int64_t n = 0; n < N; ++n) row[n] = 0.0;
        for (int64_t k = 0; k < K; ++k) {
            double a = fabs((double)(transA ? A[k * M + m] : A[m * K + k]));
            if (a == 0.0) continue;
            if (transB) {
                for (int64_t n = 0; n < N; ++n) row[n] += a * fabs((double)B[n * K + k]);
            } else {
                const float *br = B + k * N;
                for (int64_t n = 0; n < N; ++n) row[n] += a * fabs((double)br[n]);
            }
        }
        for (int64_t n = 0; n < N; ++n) {
            row[n] *= fabs((double)alpha);
            if (has_C) row[n] += fabs((double)beta * c_value(C, c_ndim, c0, c1, N, m, n));
        }
    }
}

/* Plain double-precision product, for brute-force checks on tiny shapes. */
ORC_API void orc_gemm_f64(int64_t M, int64_t N, int64_t K, const float *A, const float *B,
                          double *Y) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            double s = 0.0;
            for (int64_t k = 0; k < K; ++k) s += (double)A[m * K + k] * (double)B[k * N + n];
            Y[m * N + n] = s;
        }
}

/* ------------------------------------------------------------------------ */
/* Conv 2-D (NCHW), conv.cpp:115-207 semantics, fp32 accumulate             */
/* ------------------------------------------------------------------------ */

ORC_API void orc_conv2d(const float *X, const float *W, const float *bias, float *Y,
                        int64_t N, int64_t C, int64_t H, int64_t Wd, int64_t M, int64_t kH,
                        int64_t kW, int64_t sH, int64_t sW, int64_t pH, int64_t pW, int64_t dH,
                        int64_t dW, int64_t group, int64_t oH, int64_t oW, int act) {
    int nt = orc_get_threads();
    int64_t Cg = C / group, Mg = M / group;
#pragma omp parallel for num_threads(nt) schedule(dynamic, 1) collapse(2)
    for (int64_t n = 0; n < N; ++n)
        for (int64_t m = 0; m < M; ++m) {
            int64_t g = m / Mg;
            for (int64_t oh = 0; oh < oH; ++oh)
                for (int64_t ow = 0; ow < oW; ++ow) {
                    float sum = 0.0f;
                    for (int64_t kh = 0; kh < kH; ++kh)
                        for (int64_t kw = 0; kw < kW; ++kw) {
                            int64_t ih = oh * sH + kh * dH - pH;
                            int64_t iw = ow * sW + kw * dW - pW;
                            if (ih < 0 || ih >= H || iw < 0 || iw >= Wd) continue;
                            for (int64_t c = 0; c < Cg; ++c) {
                                float xv = X[((n * C + g * Cg + c) * H + ih) * Wd + iw];
                                float wv = W[((m * Cg + c) * kH + kh) * kW + kw];
                                sum = fmaf(xv, wv, sum);
                            }
                        }
                    if (bias) sum += bias[m];
                    Y[((n * M + m) * oH + oh) * oW + ow] = apply_act(sum, act);
                }
        }
}

/* ------------------------------------------------------------------------ */
/* E5M2 codec                                                               */
/* ------------------------------------------------------------------------ */

/* Restatement of FP8E5M2::from_float, fp_quantized.h:272-346.  Unlike the
 * E4M3 encoder it does not saturate: |v| > 57344 and +-inf give +-inf. */
ORC_API uint8_t orc_e5m2_from_float(float v) {
    const int kMantBits = 2, kBias = 15, kInfNanExp = 31;
    const uint8_t kMantMask = 0x03, kSignMask = 0x80;
    if (isnan(v)) return 0x7f;                        /* 274-277 */
    if (isinf(v)) return v < 0.0f ? 0xfc : 0x7c;      /* 278-281 */
    if (v == 0.0f) return 0;                          /* 282-285 (-0.0 -> 0x00) */
    uint32_t sign = 0;
    if (v < 0.0f) { sign = 1; v = -v; }               /* 286-290 */
    const float max_finite = 57344.0f;
    if (v > max_finite) return sign ? 0xfc : 0x7c;    /* 292-297 */
    int32_t exp;
    float mant = frexpf(v, &exp);                     /* 299-304 */
    mant *= 2.0f;
    exp -= 1;
    int32_t e = exp + kBias;                          /* 306 */
    if (e <= 0) {                                     /* 307-317 */
        if (e < -kMantBits) return sign ? kSignMask : 0;
        int32_t shift = 1 - e;
        mant = mant / (float)(1 << shift);
        e = 0;
    }
    float mant_q = floorf(mant * (float)(1 << kMantBits)); /* 319-322 */
    float frac = mant * (float)(1 << kMantBits) - mant_q;
    uint8_t m = (uint8_t)((uint8_t)mant_q & kMantMask);
    if (frac > 0.5f || (frac == 0.5f && (m & 1))) {   /* 324-331 */
        m += 1;
        if (m > kMantMask) { m = 0; e += 1; }
    }
    if (e >= kInfNanExp) { e = kInfNanExp; m = 0; }   /* 333-337 */
    if (e == 0 && m == 0) return sign ? kSignMask : 0; /* 339-343 */
    return (uint8_t)((sign ? kSignMask : 0) | (uint8_t)(e << kMantBits) | m);
}

/* Restatement of FP8E5M2::to_float, fp_quantized.h:350-377. */
ORC_API float orc_e5m2_to_float(uint8_t bits) {
    uint8_t sign = (bits & 0x80) >> 7;
    uint8_t e = (bits >> 2) & 31;
    uint8_t m = bits & 3;
    if (e == 0 && m == 0) return sign ? -0.0f : 0.0f;
    if (e == 31 && m == 0) return sign ? -INFINITY : INFINITY;
    if (e == 31) return u2f(0x7fc00000u); /* quiet NaN */
    float value;
    if (e == 0)
        value = (float)m / (float)(1 << 2) * powf(2.0f, (float)(1 - 15));
    else
        value = (1.0f + (float)m / (float)(1 << 2)) * powf(2.0f, (float)(e - 15));
    return sign ? -value : value;
}

/*
 * Closed-form specification of the E5M2 encoder, independent of the
 * frexp/floor algorithm:
 *   NaN -> 0x7f;  +-0 -> 0x00;  |x| > 57344 (incl. inf) -> sign|0x7c;
 *   otherwise the E5M2 grid point nearest to |x|, ties to the even code;
 *   a zero result keeps the sign (0x80).
 */
static double g_grid5[124]; /* positive finite codes 0x00..0x7b */
static int g_grid5_ready = 0;
static void grid5_init(void) {
    if (g_grid5_ready) return;
    for (int c = 0; c < 124; ++c) {
        int e = c >> 2, m = c & 3;
        g_grid5[c] = e == 0 ? ldexp((double)m, -16) : ldexp(1.0 + m / 4.0, e - 15);
    }
    g_grid5_ready = 1;
}

ORC_API uint8_t orc_e5m2_spec_encode(float x) {
    uint32_t u = f2u(x);
    uint32_t s = u >> 31, a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return 0x7f;
    if (a == 0) return 0x00;
    double v = (double)u2f(a);
    if (v > 57344.0) return (uint8_t)((s << 7) | 0x7c);
    grid5_init();
    int lo = 0, hi = 123;
    while (hi - lo > 1) {
        int mid = (lo + hi) / 2;
        if (g_grid5[mid] <= v) lo = mid; else hi = mid;
    }
    int c;
    double dlo = v - g_grid5[lo], dhi = g_grid5[hi] - v;
    if (dlo < dhi) c = lo;
    else if (dhi < dlo) c = hi;
    else c = (lo & 1) ? hi : lo;
    if (c == 0) return (uint8_t)(s << 7);
    return (uint8_t)((s << 7) | c);
}

ORC_API void orc_e5m2_encode_bits(uint32_t first, uint64_t count, uint8_t *out) {
    int nt = orc_get_threads();
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t i = 0; i < (int64_t)count; ++i)
        out[i] = orc_e5m2_from_float(u2f(first + (uint32_t)i));
}

ORC_API uint64_t orc_e5m2_sweep_vs_spec(uint32_t first, uint64_t count, uint32_t *first_bad) {
    grid5_init();
    uint64_t bad = 0;
    uint32_t lowest = 0xffffffffu;
    int nt = orc_get_threads();
#pragma omp parallel for num_threads(nt) schedule(static) reduction(+ : bad) reduction(min : lowest)
    for (int64_t i = 0; i < (int64_t)count; ++i) {
        uint32_t b = first + (uint32_t)i;
        float x = u2f(b);
        if (orc_e5m2_from_float(x) != orc_e5m2_spec_encode(x)) {
            ++bad;
            if (b < lowest) lowest = b;
        }
    }
    if (bad && first_bad) *first_bad = lowest;
    return bad;
}

ORC_API void orc_e5m2_decode_table(float *out256) {
    for (int c = 0; c < 256; ++c) out256[c] = orc_e5m2_to_float((uint8_t)c);
}

/* x rounded once to IEEE binary16 (nearest, ties to even; subnormals with
 * quantum 2^-24; |x| >= 65520 -> inf), returned as float (exact). */
ORC_API float orc_half_round(double x) {
    if (isnan(x)) return u2f(0x7fc00000u);
    if (isinf(x)) return (float)x;
    double a = fabs(x);
    if (a >= 65520.0) return x < 0 ? -INFINITY : INFINITY;
    if (a == 0.0) return (float)x;
    int e;
    frexp(a, &e);                 /* a = f * 2^e, f in [0.5, 1) */
    int q = e - 1 - 10;           /* quantum exponent for 11 significant bits */
    if (q < -24) q = -24;         /* subnormal quantum */
    double r = rint(ldexp(a, -q)); /* default rounding mode: nearest, ties to even */
    r = ldexp(r, q);
    return (float)(x < 0 ? -r : r);
}

ORC_API void orc_half_round_array(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_half_round((double)x[i]);
}

/* dtype codes: the ONNX TensorProto numbers */
#define ORC_FLOAT 1
#define ORC_E4M3 17
#define ORC_E5M2 19

static inline float dec_any(const void *p, int64_t i, int dtype) {
    if (dtype == ORC_FLOAT) return ((const float *)p)[i];
    uint8_t c = ((const uint8_t *)p)[i];
    return dtype == ORC_E4M3 ? orc_e4m3_to_float(c) : orc_e5m2_to_float(c);
}

/*
 * Elementwise Add(0) / Sub(1) / Mul(2) / Div(3) with numpy broadcasting
 * (shapes right-aligned, size-1 dims broadcast; binary.cpp:59-182).
 * FLOAT: the op in fp32.  E4M3 / E5M2 (binary.cpp:184-285): both operands
 * decoded (to half in the reference; every fp8 value is exact there), the
 * op rounded to half, then the CPU encoder of the same format.
 */
ORC_API void orc_fp8_binary(int op, int dtype, const void *a, const int64_t *a_shape, int a_ndim, const void *b,
                            const int64_t *b_shape, int b_ndim, void *y, const int64_t *y_shape, int y_ndim) {
    int64_t sa[8], sb[8], n = 1;
    for (int d = y_ndim - 1, acc_a = 1, acc_b = 1; d >= 0; --d) {
        int da = d - (y_ndim - a_ndim), db = d - (y_ndim - b_ndim);
        int64_t ea = da >= 0 ? a_shape[da] : 1, eb = db >= 0 ? b_shape[db] : 1;
        sa[d] = ea == 1 ? 0 : acc_a;
        sb[d] = eb == 1 ? 0 : acc_b;
        acc_a *= (int)ea;
        acc_b *= (int)eb;
    }
    for (int d = 0; d < y_ndim; ++d) n *= y_shape[d];
    for (int64_t i = 0; i < n; ++i) {
        int64_t r = i, ia = 0, ib = 0;
        for (int d = y_ndim - 1; d >= 0; --d) {
            int64_t c = r % y_shape[d];
            r /= y_shape[d];
            ia += c * sa[d];
            ib += c * sb[d];
        }
        float va = dec_any(a, ia, dtype), vb = dec_any(b, ib, dtype);
        if (dtype == ORC_FLOAT) {
            float v = op == 0 ? va + vb : op == 1 ? va - vb : op == 2 ? va * vb : va / vb;
            ((float *)y)[i] = v;
        } else {
            double dv = op == 0 ? (double)va + vb : op == 1 ? (double)va - vb : op == 2 ? (double)va * vb
                                                                            : (double)va / vb;
            float h = orc_half_round(dv);
            ((uint8_t *)y)[i] = dtype == ORC_E4M3 ? orc_e4m3_from_float(h) : orc_e5m2_from_float(h);
        }
    }
}

/* QuantizeLinear / DequantizeLinear with a FLOAT8E5M2 tensor. */
ORC_API void orc_quantize_e5m2(const float *x, uint8_t *y, int64_t outer, int64_t axis_len, int64_t inner,
                               const float *scale, int saturate) {
    for (int64_t o = 0; o < outer; ++o)
        for (int64_t a = 0; a < axis_len; ++a) {
            const float s = scale[axis_len == 1 ? 0 : a];
            for (int64_t i = 0; i < inner; ++i) {
                const int64_t k = (o * axis_len + a) * inner + i;
                float q = x[k] / s;
                if (saturate && !isnan(q) && fabsf(q) > 57344.0f) q = q < 0 ? -57344.0f : 57344.0f;
                y[k] = orc_e5m2_from_float(q);
            }
        }
}

ORC_API void orc_dequantize_e5m2(const uint8_t *q, float *y, int64_t outer, int64_t axis_len, int64_t inner,
                                 const float *scale) {
    for (int64_t o = 0; o < outer; ++o)
        for (int64_t a = 0; a < axis_len; ++a) {
            const float s = scale[axis_len == 1 ? 0 : a];
            for (int64_t i = 0; i < inner; ++i) {
                const int64_t k = (o * axis_len + a) * inner + i;
                y[k] = orc_e5m2_to_float(q[k]) * s;
            }
        }
}
