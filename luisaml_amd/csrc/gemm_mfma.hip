// gemm_mfma.hip -- large-M FP8 GEMM (and the implicit-im2col conv) on gfx950
// matrix cores.
//
// Y[M,N] = epilogue( A[M,K] (E4M3, row-major) x B[K,N] (E4M3, packed panels) )
//
// Three workgroup layouts, K step 64 (BK):
//   * 256x256 tiles, 512 threads = 8 wavefronts laid out 2 (M) x 4 (N), each
//     owning 128x64 = 4x2 blocks of 32x32 fp32 accumulators; two wavefronts
//     per SIMD; a 4-stage LDS ring (LCML_GEMM_STAGES).  fp32 outputs, grids of
//     one tile column and the conv.
//   * 256x256 tiles, 256 threads = 2x2 wavefronts of 128x128 (4x4 blocks, the
//     256 accumulators per lane in AGPRs), one wavefront per SIMD, a 5-stage
//     ring and an explicitly placed step schedule.  bf16 outputs on grids of
//     more than one tile column.
//   * 128x128 tiles, 256 threads = 2x2 wavefronts of 64x64, two workgroups
//     per CU, for mid-size GEMMs whose 256x256 grid would leave CUs idle.
//
// Two instantiations share everything but the matrix-core instruction:
//   EXACT (default): the E4M3 fragments read from LDS are widened to bf16 in
//     registers (v_cvt_scalef32_pk_bf16_fp8, exact) and multiplied with
//     v_mfma_f32_32x32x16_bf16, which accumulates at fp32 accuracy.  Every
//     product of two E4M3 values is exact in fp32, so the result differs from
//     the fp32 reference only by summation order.
//   native FP8: v_mfma_f32_32x32x64_f8f6f4 directly on the E4M3 bytes.  Twice
//     the matrix-core rate, but gfx950's FP8 MFMAs drop product bits more than
//     about 2^13 below the largest product of each block (measured: relative
//     Frobenius error ~1.4e-5 on N(0,1) data), so it is an opt-in kernel.
// Every layout sums each output's products in the same order, so all of them
// give bit-identical results.
//
// Each LDS stage holds one 64-k step: A (BM x 64 B) then B (BN x 64 B), 32 KB
// for a 256x256 tile.  Tiles move global -> LDS with buffer_load_dwordx4 ...
// lds (no staging registers): each wavefront instruction deposits one
// contiguous 1 KB block, and lanes whose offset is out of range (rows >= M,
// k >= K, panels beyond N) deposit zeros.  While the matrix cores work on one
// stage, the following K steps stream into the others; one barrier per step.
//
// LDS layouts (bank-conflict free for 16-lane groups of ds_read_b128 on the
// 64-bank gfx950 LDS):
//   A: row-major [rows][64 B]; the 16-byte chunk c of row r is stored at
//      chunk position c ^ ((r >> 2) & 3).  A 1 KB load block is 16 rows;
//      lane l fills position l%4 of row l/4, so it fetches logical chunk
//      (l%4) ^ ((row >> 2) & 3) -- each 4-lane group still reads one
//      contiguous 64 B row segment.
//   B: the packed global layout verbatim, [panels][4 k-chunks][64 cols][16 B].
// MFMA operand chunks: lane l of a 32x32x64 fragment holds row/column l%32
// and k = (l/32)*32 + 0..31, i.e. two consecutive 16-byte k-chunks.
//
// Workgroup -> tile map: consecutive workgroup ids land on different XCDs
// (id % 8), so ids are first regrouped so that each XCD works on one
// contiguous range of tiles, and tiles are ordered in groups of 8 tile-rows
// so that the tiles resident at one time on an XCD share A rows and B
// columns in that XCD's L2.
#include "lcml_internal.hpp"

namespace lcml {
namespace {

#ifndef LCML_GEMM_WAVES_M
#define LCML_GEMM_WAVES_M 2
#endif
#ifndef LCML_GEMM_WAVES_N
#define LCML_GEMM_WAVES_N 4
#endif

#ifndef LCML_GEMM_STAGES
#define LCML_GEMM_STAGES 4
#endif
#ifndef LCML_GEMM_WG_PER_CU
#define LCML_GEMM_WG_PER_CU 1  // occupancy the register budget is sized for
#endif
constexpr int BK = 64;                    // K per pipeline step
constexpr int NSTAGE = LCML_GEMM_STAGES;  // LDS ring depth: NSTAGE-1 steps of loads in flight
constexpr int CPR = BK / 16;              // 16-byte chunks per A row per step
constexpr int GROUP_M = 8;
constexpr int EP_PITCH = 36;   // CONV epilogue staging row pitch (floats): 16-byte rows with 4 floats of padding, b128 reads conflict-free
constexpr int EP2_PITCH = 72;  // row-major epilogue staging row pitch (floats)

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf2 __attribute__((ext_vector_type(2)));

// Tile geometry: WAVES_M x WAVES_N wavefronts, each owning WM x WN blocks of
// 32x32 outputs: 256x256 tiles of 2x4 wavefronts of 128x64 or of 2x2
// wavefronts of 128x128 (one wavefront per SIMD, a five-stage ring), and
// 128x128 tiles of 2x2 wavefronts of 64x64.
template <int WAVES_M, int WAVES_N, int WM, int WN>
struct Tile {
    static constexpr int NW = WAVES_M * WAVES_N, NT = NW * 64;
    static constexpr bool ONE_PER_SIMD = NW == 4 && WM == 4 && WN == 4;
    static constexpr int NST = ONE_PER_SIMD ? 5 : NSTAGE;  // LDS ring depth
    static constexpr int BM = WAVES_M * WM * 32, BN = WAVES_N * WN * 32;
    static constexpr int A_BYTES = BM * BK, B_BYTES = BN * BK, STAGE = A_BYTES + B_BYTES;
    static constexpr int A_BLK = A_BYTES / 1024 / NW, B_BLK = B_BYTES / 1024 / NW;  // 1 KB load blocks per wavefront
    static constexpr int LOADS = A_BLK + B_BLK;  // load instructions per wavefront per step
    // row-major epilogue pass height: all WM*32 rows of a wavefront where the
    // staging of every wavefront fits the LDS (the one-wavefront-per-SIMD
    // layout: two passes of 128 rows instead of four of 64, half the
    // barriers; +1.4% at 8192^3 native FP8, +0.5% exact), else 64
    static constexpr int EP_ROWS = NW * WM * 32 * EP2_PITCH * 4 <= 160 * 1024 ? WM * 32 : 64;
    static constexpr int EP_BYTES =
        NW * (WM * 32 * EP_PITCH > EP_ROWS * EP2_PITCH ? WM * 32 * EP_PITCH : EP_ROWS * EP2_PITCH) * 4;
    static constexpr int LDS_BYTES = NST * STAGE > EP_BYTES ? NST * STAGE : EP_BYTES;
    static_assert(BM % 64 == 0 && BN % 64 == 0 && (A_BYTES / 1024) % NW == 0 && (B_BYTES / 1024) % NW == 0,
                  "tile shape");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
    static_assert(NST >= 3 && (NST - 2) * LOADS <= 63, "pipeline depth");
};

// Implicit-im2col convolution geometry (CONV instantiation).  A is the
// quantised input in NHWC order, so the GEMM row m = (n, oh, ow) and the
// reduction index k = (kh, kw, c) — the reference's loop order (kh, kw, then
// channels, conv.cpp:143-192) — address the bytes
//   X[n][oh*sh - ph + kh*dh][ow*sw - pw + kw*dw][c]
// and taps that fall into the padding read zeros (the reference's unsigned
// bounds check, conv.cpp:145-148; begin pads only, conv.cpp:121).  The
// output goes to NCHW: Y[n][co][oh][ow].
// With groups, workgroup row blockIdx.y = g runs the GEMM of group g: input
// channels g*Cg .. (g+1)*Cg-1, output channels g*N .. (g+1)*N-1 (N = Cout /
// group), weights = the g-th packed block.
struct ConvGeom {
    int H, W, Cg, Ctot, CoutTot, OH, OW, KH, KW, sh, sw, ph, pw, dh, dw;
};

struct GemmArgs {
    ConvGeom cv;
    int64_t M, N, K;
    const uint8_t *a;
    int64_t lda;
    const uint8_t *bp;
    int64_t KC;       // k-chunks per packed panel (Kp / 16)
    int64_t npanels;  // packed panels (Np / 64)
    uint32_t a_bytes, b_bytes;  // buffer extents for range checking
    int tiles_m, tiles_n;
    int nk;           // K steps of 128
    // row slices of the 2x4 layout (slice_rows: 0 for none, else a multiple
    // of 32 below BM).  slice_cols == 0 (a grid of one tile column): ids
    // 0 .. slice_first-1 are whole BM-row tiles, the ids after them slices of
    // slice_rows rows below those.  slice_cols > 0: the first slice_first =
    // slice_cols * tiles_m ids are the whole tiles of the first slice_cols
    // tile columns, the ids after them slices of slice_rows rows of the
    // other columns, ceil(M / slice_rows) per column.
    int slice_first, slice_rows, slice_cols;
    Epilogue e;
};

typedef __attribute__((address_space(3))) void lds_void;
constexpr uint32_t OOB = 0x80000000u;  // offset past every buffer extent

__device__ inline v8i join(u4 lo, u4 hi) {
    v8i r;
    r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
    r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
    return r;
}

// A rows in LDS: chunk c of row r at chunk position c ^ swz(r); the 16 rows
// of a ds_read_b128 lane group then cover all 16 16-byte bank slots of the
// 64-bank LDS (BK=128: 2 rows per 256 B; BK=64: 4 rows per 256 B).
__device__ inline int a_swz(int r) { return (r / (256 / BK)) & (CPR - 1); }
__device__ inline int a_lds_off(int r, int c) { return r * BK + ((c ^ a_swz(r)) << 4); }

// One 64-row pass of the row-major epilogue with the uniform choices made at
// compile time (activation, C, output type), so that its loop is
// straight-line: lane l writes columns col and col + 1 of rows row0 + 2q
// (q < 32) from the staged sums at src, computing epi_value_cv's value
// (acc * scale * alpha, + beta * C, activation; the multiply by alpha = 1 is
// exact).  bf16 pairs are packed by v_cvt_pk_bf16_f32, which rounds to
// nearest even exactly as bf16_rne does (checked over all 2^32 fp32 inputs).
// Every store is a buffer store, and the hardware drops those past the
// buffer's extent: a row past M lies past num_records = M * ldy elements, and
// a lane whose columns lie past N, or a pass that starts past M, carries an
// offset past it.  The caller keeps (M + 64) * ldy elements below 2^31 bytes,
// so neither a pass that starts before M (rows up to M + 62) nor OOB plus 31
// row steps of a pass past M wraps 32 bits.
// With every CU busy, the general path (uniform tests on every element,
// software rounding) took ~19 us for a 256x256 tile's bf16 epilogue, this one
// ~4.5 us (fp32: ~8 us); on the 4096-row transformer linears that is 6-7% of
// the exact kernel's time and 15-18% of the native FP8 one's.
// Rows from rows_end on (M, or the end of the wavefront's rows in a row
// slice, whose rows after it are another slice's) are dropped as rows past M
// are: the buffer's extent ends there.
// AMAX: m accumulates max |value| over the in-range elements written (rows
// below rows_end, columns below N; NaN compares false and is skipped).
template <int ACT, bool HAS_C, bool BF16, bool AMAX = false>
__device__ __forceinline__ void epi_rows(const Epilogue &e, const float *src, int64_t row0, int64_t col, bool cols_ok,
                                         float sc0, float sc1, float cb0, float cb1, float &m, bool c1_ok,
                                         int64_t rows_end) {
    // every operation rounds on its own, as in epi_value_cv (where alpha is
    // applied under a runtime test, so nothing fuses across it): no FMA
#pragma clang fp contract(off)
    constexpr uint32_t ES = BF16 ? 2 : 4;
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(e.y, 0, (int)(rows_end * e.ldy * ES), 0x00020000);
    const uint32_t step = (uint32_t)(2 * e.ldy * ES);
    uint32_t off = cols_ok && row0 < rows_end ? (uint32_t)((row0 * e.ldy + col) * ES) : OOB;
    const float alpha = e.alpha;
#pragma unroll 8
    for (int q = 0; q < 32; ++q, off += step) {
        const f2 a = *reinterpret_cast<const f2 *>(src + 2 * q * EP2_PITCH);
        float v0 = a.x * sc0 * alpha, v1 = a.y * sc1 * alpha;
        if constexpr (HAS_C) {
            v0 += cb0;
            v1 += cb1;
        }
        v0 = apply_act(v0, ACT);
        v1 = apply_act(v1, ACT);
        if constexpr (AMAX) {
            const bool r_ok = row0 + 2 * q < rows_end;
            const float a0 = fabsf(v0), a1 = fabsf(v1);
            m = r_ok && cols_ok && a0 > m ? a0 : m;
            m = r_ok && c1_ok && a1 > m ? a1 : m;
        }
        if constexpr (BF16) {
            const f2 v = {v0, v1};
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf2)), r, off,
                                                  0, 0);
        } else {
            const f2 v = {v0, v1};
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2, v), r, off, 0, 0);
        }
    }
}

// The NCHW epilogue's column loop with the same compile-time choices (ACT < 0:
// the activation taken from e.act at run time): lane l writes its output
// pixel of columns colb .. colb + ncol - 1 (address p for column colb,
// `step` elements per column), the column's scale and beta * C taken from
// lane c of sc_l and cb_l.
template <int ACT, bool HAS_C, bool BF16>
__device__ __forceinline__ void epi_cols(const Epilogue &e, const float *srow, void *p, int64_t step, int ncol,
                                         int sc_l, int cb_l) {
#pragma clang fp contract(off)  // as in epi_rows
    const float alpha = e.alpha;
    auto put = [&](int c, float acc) {
        float v = acc * __builtin_bit_cast(float, __builtin_amdgcn_readlane(sc_l, c)) * alpha;
        if constexpr (HAS_C) v += __builtin_bit_cast(float, __builtin_amdgcn_readlane(cb_l, c));
        v = apply_act(v, ACT < 0 ? e.act : ACT);
        if constexpr (BF16) {
            const f2 vv = {v, 0.0f};
            reinterpret_cast<uint16_t *>(p)[c * step] =
                (uint16_t)(__builtin_bit_cast(uint32_t, __builtin_convertvector(vv, bf2)) & 0xffffu);
        } else {
            reinterpret_cast<float *>(p)[c * step] = v;
        }
    };
    if (ncol == 32) {
        // a whole block: four staged columns per 16-byte read, the next read
        // issued before the current four are stored (the read past the last
        // group lands in the row's padding), so an LDS round trip is paid
        // once per four columns and overlapped.  Rolled: unrolling all 32
        // columns of every specialisation doubled the kernel's code and made
        // the whole conv 40% slower.
        f4 a = *reinterpret_cast<const f4 *>(srow);
#pragma unroll 1
        for (int q = 0; q < 8; ++q) {
            const f4 next = *reinterpret_cast<const f4 *>(srow + 4 * q + 4);
            put(4 * q, a.x);
            put(4 * q + 1, a.y);
            put(4 * q + 2, a.z);
            put(4 * q + 3, a.w);
            a = next;
        }
    } else {
        // a rolled loop: v_readlane is convergent, so the compiler does not
        // unroll around it; the stores do not wait, so several are in flight
        for (int c = 0; c < ncol; ++c) put(c, srow[c]);
    }
}

// The lane index, computed where it is used (v_mbcnt): the volatile asm
// cannot be hoisted, so the persistent kernel's code between tiles holds no
// per-lane value through the main loop, whose registers are all taken.
__device__ __forceinline__ int lane_here() {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
}

// Direct-store epilogue of the persistent one-wavefront-per-SIMD GEMM (bf16
// output, no LDS).  Its MFMAs run with the operands swapped (the B block
// first), so of a 32x32 block a lane holds one output row, m = lane % 32,
// at columns 8*(r/4) + 4*(lane/32) + r%4 for accumulator r.  Each value
// gets epi_value_cv's operations in its order (acc * scale * alpha, + beta
// * C, the activation; no contraction); pairs are rounded to bf16 by
// v_cvt_pk_bf16_f32, and one v_permlane32_swap per two pairs trades the
// column groups 8g+4.. (upper lanes) and 8(g+1).. (lower lanes), after
// which lane l holds 8 consecutive columns 16h + 8*(l/32) of its row.  Per
// pass of 32 rows x 64 columns these 16-byte pieces go to the wavefront's
// part of a free LDS stage and come back as whole 128-byte row segments,
// 8 rows per buffer store: full cache lines, where storing the pieces
// straight from the registers (32 rows x 32 bytes per store) measured 4-5%
// slower at 8192^3.  Rows past M and columns past N carry an out-of-range
// offset (the caller
// guarantees N % 8 == 0, ldy % 8 == 0, a 16-byte aligned y, M * ldy * 2 <
// 2^31 bytes, and a C that does not vary over rows).  mr0 / nc0: the
// wavefront's first output row and column.
// The uniform inputs of epi_direct_bf16, read once per kernel: the
// per-tensor scale product and a scalar C (reads inside the tile loop would
// be vector loads waiting on every load in flight).
struct DirectUniforms {
    float a_s, s_uni, c_uni;
    bool pc, c_vec;
};

// (each value passed through v_readfirstlane: uniform, so it lives in a
// scalar register rather than taking one of the main loop's vector ones)
__device__ inline float uniform_f(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x)));
}

__device__ inline DirectUniforms direct_uniforms(const Epilogue &e) {
    DirectUniforms u;
    u.a_s = uniform_f(e.a_scale ? e.a_scale[0] : 1.0f);
    u.pc = e.b_scale && e.b_per_channel;
    u.s_uni = uniform_f(e.b_scale && !u.pc ? u.a_s * e.b_scale[0] : u.a_s);  // epi_scale of a per-tensor scale
    // C over N (a vector) or one value: the row-invariant broadcasts of epi_c
    u.c_vec = e.c && !(e.c_ndim == 0 || (e.c_ndim == 1 && e.c0 == 1) || (e.c_ndim == 2 && e.c1 == 1));
    u.c_uni = uniform_f(e.c && !u.c_vec ? e.c[0] : 0.0f);
    return u;
}

// Row pitch (bytes) of the epilogue's per-wavefront LDS staging: 32 rows of
// 64 bf16 columns plus 16 bytes, so the 16 rows of a ds_write_b128 lane group
// fall on distinct 16-byte bank slots (9 slots per row, odd).
constexpr int EPD_PITCH = 144;
// a wavefront's part of the free ring stage: the staging rows, then its 128
// columns' scales and C (512 bytes each, each the first half of a 1 KB
// global->LDS load whose upper lanes load nothing)
constexpr int EPD_SCALE = 32 * EPD_PITCH, EPD_C = EPD_SCALE + 1024, EPD_BYTES = EPD_C + 1024;

// ALPHA1: alpha == 1, whose multiply is exact and left out
template <int ACT, bool HAS_C, bool ALPHA1>
__device__ __forceinline__ void epi_direct_bf16(const Epilogue &e, const DirectUniforms &u, const v16f (&acc)[4][4],
                                                int mr0, int nc0, uint8_t *lds) {
#pragma clang fp contract(off)
    const int lane = lane_here();
    // 32-bit offsets: the launcher keeps M * ldy * 2 below 2^31
    const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(e.y, 0, (int)(e.M * e.ldy * 2), 0x00020000);
    const float a_s = u.a_s, s_uni = u.s_uni, c_uni = u.c_uni;
    const bool pc = u.pc, c_vec = u.c_vec;
    const float alpha = e.alpha, beta = e.beta;
    const bool upper = lane >= 32;
    const int M = (int)e.M, N = (int)e.N;
    const uint32_t ldy2 = (uint32_t)e.ldy * 2u;
    auto val = [&](float a, float s, float c) {
        float v = a * s;
        if constexpr (!ALPHA1) v *= alpha;
        if constexpr (HAS_C) v += c;
        return apply_act(v, ACT);
    };
    // column j*32 + 8g + 4*(lane/32) + q's scale and beta * C; per-channel
    // scales and a C over N come from the copies that the tile's last step
    // loaded into LDS (waited for by the caller)
    // (read unconditionally, all reads issued before any use; the choices
    // are selects, not branches)
    auto coef = [&](int j, f4 (&sc)[4], f4 (&cb)[4]) {
        f4 bs[4], cv[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int col = j * 32 + 8 * g + 4 * upper;  // within the wavefront's 128 columns
            bs[g] = *reinterpret_cast<const f4 *>(lds + EPD_SCALE + col * 4);
            if constexpr (HAS_C) cv[g] = *reinterpret_cast<const f4 *>(lds + EPD_C + col * 4);
        }
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                sc[g][q] = pc ? a_s * bs[g][q] : s_uni;
                if constexpr (HAS_C) {
                    const float c = c_vec ? cv[g][q] : c_uni;
                    cb[g][q] = beta == 1.0f ? c : beta * c;
                }
            }
    };
    // Passes of 32 rows x 64 columns, blocks (i, 2jp) and (i, 2jp + 1),
    // software-pipelined: a pass's values are computed while the previous
    // pass's read-back is in flight, then that read-back is stored, this
    // pass written and read back (LDS runs a wavefront's operations in
    // order, so the writes follow the previous reads).
    u4 rb[4];
    int pm = 0, pn = 0;  // the previous pass's first row and column
    auto store_prev = [&]() {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int m = pm + rr * 8 + (lane >> 3), n = pn + (lane & 7) * 8;
            const uint32_t off = m < M && n < N ? (uint32_t)m * ldy2 + (uint32_t)n * 2u : OOB;
            __builtin_amdgcn_raw_buffer_store_b128(rb[rr], ry, off, 0, 0);
        }
    };
#pragma unroll
    for (int jp = 0; jp < 2; ++jp) {
        f4 sc[2][4], cb[2][4];
        coef(2 * jp, sc[0], cb[0]);
        coef(2 * jp + 1, sc[1], cb[1]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            u4 pk[2][2];
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    uint32_t px[2], py[2];
#pragma unroll
                    for (int k = 0; k < 2; ++k) {
                        // x: column group g = 2h, y: g = 2h + 1; values q = 2k, 2k + 1
                        const v16f &a = acc[i][2 * jp + jj];
                        const f4 &sx = sc[jj][2 * h], &sy = sc[jj][2 * h + 1];
                        const f4 &cx = cb[jj][2 * h], &cy = cb[jj][2 * h + 1];
                        const f2 vx = {val(a[8 * h + 2 * k], sx[2 * k], cx[2 * k]),
                                       val(a[8 * h + 2 * k + 1], sx[2 * k + 1], cx[2 * k + 1])};
                        const f2 vy = {val(a[8 * h + 4 + 2 * k], sy[2 * k], cy[2 * k]),
                                       val(a[8 * h + 4 + 2 * k + 1], sy[2 * k + 1], cy[2 * k + 1])};
                        const uint32_t bx = __builtin_bit_cast(uint32_t, __builtin_convertvector(vx, bf2));
                        const uint32_t by = __builtin_bit_cast(uint32_t, __builtin_convertvector(vy, bf2));
                        const auto sw = __builtin_amdgcn_permlane32_swap(bx, by, false, false);
                        px[k] = sw[0];
                        py[k] = sw[1];
                    }
                    pk[jj][h] = u4{px[0], px[1], py[0], py[1]};
                }
            if (jp > 0 || i > 0) store_prev();
            // row lane % 32, columns jj*32 + 16h + 8*(lane/32) .. + 7 of the pass
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    *reinterpret_cast<u4 *>(lds + (lane & 31) * EPD_PITCH + (jj * 32 + 16 * h + 8 * upper) * 2) =
                        pk[jj][h];
            // back as whole rows: 8 lanes per 128-byte row, 8 rows per store
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
                rb[rr] = *reinterpret_cast<const u4 *>(lds + (rr * 8 + (lane >> 3)) * EPD_PITCH + (lane & 7) * 16);
            pm = mr0 + i * 32;
            pn = nc0 + jp * 64;
        }
    }
    store_prev();
}

// Scheduling pattern for one step of the native FP8 loop: the NL
// global->LDS loads first (the LDS reads may not pass them: the compiler
// cannot tell the loads' LDS writes from the reads' addresses), then NM
// MFMAs, each followed by its share of the next step's NR LDS fragment reads,
// the reads spread over all but the last TAIL MFMAs, which cover the latency
// of the final reads before the next barrier's wait.  Against the same loop
// with the reads issued as one burst (the LDS command FIFO filled, stalling
// the in-order issue of the MFMAs behind them): +3-4% at 8192^3 and on the
// M=4096 linears, bit-identical.
template <int NM, int NR, int NL, int TAIL = 4, int R = 0>
__device__ __forceinline__ void sched_interleave() {
    if constexpr (R == 0) __builtin_amdgcn_sched_group_barrier(0x020, NL, 0);  // global->LDS loads
    if constexpr (R < NM) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        constexpr int NMR = NM > TAIL ? NM - TAIL : NM;  // MFMAs that take reads
        constexpr int rd = R < NMR ? (NR * (R + 1)) / NMR - (NR * R) / NMR : 0;
        if constexpr (rd > 0) __builtin_amdgcn_sched_group_barrier(0x100, rd, 0);  // LDS reads
        sched_interleave<NM, NR, NL, TAIL, R + 1>();
    }
}

// One 16-byte-per-lane global->LDS load.  A device function of its own: the
// same builtin called from a lambda inside the one-wavefront-per-SIMD loop
// made clang drop that kernel's host-side launch stub without a diagnostic.
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t r, uint8_t *lds, uint32_t off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds, 16, off, 0, 0, 0);
}

template <int WAVES_M, int WAVES_N, int WM, int WN, bool EXACT, bool CONV, bool PP, bool DIRECT = false,
          bool AMAX = false>
__global__ __launch_bounds__(WAVES_M *WAVES_N * 64, LCML_GEMM_WG_PER_CU) void k_gemm_mfma(GemmArgs g) {
    using T = Tile<WAVES_M, WAVES_N, WM, WN>;
    constexpr int NSTAGE = T::NST;
    static_assert(!DIRECT || (T::ONE_PER_SIMD && !CONV && !PP), "the persistent direct-store loop is the one-wavefront-per-SIMD GEMM's");
    static_assert(!AMAX || (!CONV && !DIRECT), "amax partials: the row-major staged epilogue");
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;

    // ---- tile selection -------------------------------------------------
    // Workgroup id -> tile: ids regrouped so that each XCD (id % 8) owns a
    // contiguous range of tiles, walked in groups of GROUP_M tile-rows.  The
    // persistent kernel walks ids blockIdx.x, + gridDim.x, ... (gridDim.x a
    // multiple of 8 whenever it is below the tile count, so every id of one
    // workgroup stays on its XCD's range).
    const int ntiles = g.tiles_m * g.tiles_n;
    // (over a grid of tm x tn tiles: the whole grid, or the whole-tile
    // columns of a sliced one)
    auto tile_origin_in = [&](int t, int tm, int tn, int64_t &om0, int64_t &on0) {
        const int nt = tm * tn;
        if ((nt & 7) == 0) t = (t & 7) * (nt >> 3) + (t >> 3);
        const int per_group = GROUP_M * tn;
        const int group = t / per_group;
        const int first_m = group * GROUP_M;
        const int gsize = min(tm - first_m, GROUP_M);
        om0 = (int64_t)(first_m + (t % per_group) % gsize) * T::BM;
        on0 = (int64_t)((t % per_group) / gsize) * T::BN;
    };
    auto tile_origin = [&](int t, int64_t &om0, int64_t &on0) { tile_origin_in(t, g.tiles_m, g.tiles_n, om0, on0); };
    int64_t m0, n0;
    tile_origin(blockIdx.x, m0, n0);
    // Row slices (SLICE, when the launcher sets them): workgroup t below
    // slice_first takes rows t*BM .. (the ids in order: the first round of
    // workgroups fills every CU with whole tiles), a later one slice_rows
    // rows after them.  A tile of L 32-row blocks gives wave row 0 the first
    // ceil(L/2) blocks and wave row 1 the rest (4 and 4 in a whole tile), so
    // the two wavefronts that share a SIMD split a slice's blocks evenly;
    // each wavefront's loop runs MFMAs for its own blocks only.
    constexpr bool SLICE = WAVES_M == 2 && WM == 4 && !T::ONE_PER_SIMD;
    int tile_rows = T::BM;
    if constexpr (SLICE)
        if (g.slice_rows) {
            // within each part, ids regrouped so that each XCD (id % 8)
            // takes one contiguous range, as tile_origin does (with
            // slice_first a multiple of 8, id % 8 = part id % 8)
            const int t = (int)blockIdx.x, first = g.slice_first;
            const bool whole = t < first;
            const int s = whole ? t : t - first, cnt = whole ? first : (int)gridDim.x - first;
            const int q = cnt >> 3, r = cnt & 7, x = s & 7;
            const int idx = x * q + (x < r ? x : r) + (s >> 3);
            // (the conv slices one tile column only)
            if (CONV || g.slice_cols == 0) {  // one tile column: whole row tiles, then slices below them
                m0 = whole ? (int64_t)idx * T::BM : (int64_t)first * T::BM + (int64_t)idx * g.slice_rows;
                n0 = 0;
            } else if (whole) {  // the whole-tile columns, walked as an unsliced grid of them
                tile_origin_in(t, g.tiles_m, g.slice_cols, m0, n0);
            } else {  // the other columns, each cut into slices
                const int spc = (int)((g.M + g.slice_rows - 1) / g.slice_rows);
                m0 = (int64_t)(idx % spc) * g.slice_rows;
                n0 = (int64_t)(g.slice_cols + idx / spc) * T::BN;
            }
            tile_rows = whole ? T::BM : g.slice_rows;
        }
    const int live0 = (tile_rows / 32 + 1) / 2;  // 32-row blocks of wave row 0 (WM in a whole tile)
    // this wavefront's blocks and first row in the tile (wave-uniform)
    const int wlive = SLICE ? __builtin_amdgcn_readfirstlane(wm ? tile_rows / 32 - live0 : live0) : WM;
    const int wrow0 = SLICE ? __builtin_amdgcn_readfirstlane(wm ? live0 * 32 : 0) : wm * WM * 32;

    // ---- global -> LDS block assignment ----------------------------------
    // A: 1 KB block b holds rows (1024/BK)*b ..; B: block b holds panel b/CPR,
    // k-chunk b%CPR of the step.
    const __amdgpu_buffer_rsrc_t a_rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void *)g.a, 0, (int)g.a_bytes, 0x00020000);
    const int grp = CONV ? (int)blockIdx.y : 0;  // CONV: convolution group
    const __amdgpu_buffer_rsrc_t b_rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void *)(g.bp + (size_t)grp * g.b_bytes), 0, (int)g.b_bytes, 0x00020000);
    uint32_t a_off[T::A_BLK];
    // the lane's 16-byte k-chunk within a step's 64 bytes: the same for every
    // A block (the chunk swizzle of row (wave*A_BLK + i)*16 + lane/4 depends
    // only on (lane/16) % 4)
    int a_kc = 0;
    uint32_t a_klim[CONV ? 1 : T::A_BLK];  // K for rows in range, 0 for rows past M
    uint32_t b_off[T::B_BLK];
    int a_ih0[CONV ? T::A_BLK : 1], a_iw0[CONV ? T::A_BLK : 1];  // CONV: top-left input pixel of the row
    // CONV: where the lane's chunk of the next step to issue lies in (kh, kw,
    // c), the same for every block
    int a_c = 0, a_kw = 0, a_kh = 0;
    // the load offsets of the tile at (m0, n0); valid = false: every load
    // out of range (a persistent workgroup past its last tile)
    // (ln, wv: the lane and wavefront index; the persistent kernel passes a
    // lane index computed on the spot, so that nothing per lane is held
    // through its main loop for this)
    auto setup_offsets = [&](int64_t m0, int64_t n0, bool valid, int ln, int wv) {
        const int lane = ln, wave = wv;
#pragma unroll
    for (int i = 0; i < T::A_BLK; ++i) {
        const int r = (wave * T::A_BLK + i) * (1024 / BK) + lane / CPR;
        const int c = (lane % CPR) ^ a_swz(r);
        if (i == 0) a_kc = c * 16;
        if constexpr (CONV) {
            // a_off = the row's image base n*H*W*C; rows past M (or past a
            // slice's rows) get an input pixel that is out of range for
            // every tap
            const ConvGeom &cv = g.cv;
            const int64_t m = m0 + r;
            const uint32_t ohw = (uint32_t)(cv.OH * cv.OW);
            const uint32_t mm = m < g.M ? (uint32_t)m : 0u;
            const uint32_t n = mm / ohw, pix = mm - n * ohw, oh = pix / (uint32_t)cv.OW, ow = pix - oh * (uint32_t)cv.OW;
            a_off[i] = n * (uint32_t)(cv.H * cv.W * cv.Ctot) + (uint32_t)(grp * cv.Cg);
            a_ih0[i] = r < tile_rows && m < g.M ? (int)oh * cv.sh - cv.ph : -(1 << 30);
            a_iw0[i] = (int)ow * cv.sw - cv.pw;
        } else {
            // 32-bit: the host keeps (M - 1) * lda + K below 2^31
            const bool in = r < tile_rows && (int)m0 + r < (int)g.M;
            a_off[i] = valid && in ? ((uint32_t)m0 + (uint32_t)r) * (uint32_t)g.lda + (uint32_t)(c * 16) : OOB;
            a_klim[i] = in ? (uint32_t)g.K : 0u;
        }
    }
    if constexpr (CONV) {
        // step 0 starts at k = a_kc < 64; a_kc may still exceed C (C >= 16),
        // so normalise once
        int cc = a_kc, kw = 0, kh = 0;
        while (cc >= g.cv.Cg) {
            cc -= g.cv.Cg;
            if (++kw == g.cv.KW) { kw = 0; ++kh; }
        }
        a_c = cc; a_kw = kw; a_kh = kh;
    }
#pragma unroll
    for (int i = 0; i < T::B_BLK; ++i) {
        const int b = wave * T::B_BLK + i;
        const int64_t panel = (n0 >> 6) + b / CPR;
        b_off[i] = valid && panel < g.npanels ? (uint32_t)((panel * g.KC + b % CPR) * 1024 + lane * 16) : OOB;
    }
    };
    setup_offsets(m0, n0, true, lane, wave);
    auto issue_tile = [&](int kt, int stage) {
        uint8_t *sa = smem + stage * T::STAGE;
        const uint32_t kbyte = (uint32_t)kt * BK;
        // CONV: k = kbyte + chunk -> (kh, kw, c), tracked incrementally:
        // steps are issued in order, each advancing k by BK; C % 16 == 0
        // keeps every 16-byte chunk inside one tap
        // (CONV: k < K exactly when the chunk's tap row kh is below KH)
        const bool k_ok = CONV ? a_kh < g.cv.KH : (int64_t)(kbyte + (uint32_t)a_kc) < g.K;
        const int dih = CONV ? a_kh * g.cv.dh : 0, diw = CONV ? a_kw * g.cv.dw : 0;
#pragma unroll
        for (int i = 0; i < T::A_BLK; ++i) {
            uint32_t off;
            if constexpr (CONV) {
                const ConvGeom &cv = g.cv;
                const int ih = a_ih0[i] + dih, iw = a_iw0[i] + diw;
                const bool ok = k_ok && (uint32_t)ih < (uint32_t)cv.H && (uint32_t)iw < (uint32_t)cv.W;
                off = ok ? a_off[i] + ((uint32_t)ih * (uint32_t)cv.W + (uint32_t)iw) * (uint32_t)cv.Ctot +
                               (uint32_t)a_c
                         : OOB;
            } else {
                off = kbyte + (uint32_t)a_kc < a_klim[i] ? a_off[i] + kbyte : OOB;
            }
            __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, (lds_void *)(sa + (wave * T::A_BLK + i) * 1024), 16,
                                                     off, 0, 0, 0);
        }
        if constexpr (CONV) {
            a_c += BK;
            while (a_c >= g.cv.Cg) {
                a_c -= g.cv.Cg;
                if (++a_kw == g.cv.KW) { a_kw = 0; ++a_kh; }
            }
        }
#pragma unroll
        for (int i = 0; i < T::B_BLK; ++i) {
            // steps past the end (the pipeline tail) still issue their loads,
            // so that every step counts the same loads for the vmcnt waits,
            // but out of range: zeros into a stage that is never read again,
            // no memory traffic
            const uint32_t off = b_off[i] != OOB && kt < g.nk ? b_off[i] + (uint32_t)kt * CPR * 1024 : OOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                b_rsrc, (lds_void *)(sa + T::A_BYTES + (wave * T::B_BLK + i) * 1024), 16, off, 0, 0, 0);
        }
    };

    v16f acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int kgrp = (lane >> 5) * 2;  // first k-chunk of this lane within a 64-k block
    const int a_r0 = wrow0 + (lane & 31);
    int b_off_lds[WN];
#pragma unroll
    for (int j = 0; j < WN; ++j) {
        const int col = wn * WN * 32 + j * 32;  // first column of this 32-column block in the tile
        b_off_lds[j] = (col >> 6) * (CPR * 1024) + ((col & 63) + (lane & 31)) * 16;
    }

    // Ring of NSTAGE LDS stages of one 64-k step each; every step issues
    // exactly LOADS loads per wavefront (past-the-end steps load zeros or
    // unused bytes into stages nobody reads).  The sync of step kt waits
    // until tile kt+1 has landed (at most (NSTAGE-3)*LOADS loads of this
    // wavefront outstanding), drains this wavefront's LDS reads (lgkmcnt(0),
    // a wait the compiler sees), and barriers: after it every wavefront's
    // share of tile kt+1 is visible and tile kt-1 is consumed everywhere, so
    // its stage takes the prefetch of tile kt+NSTAGE-1.  The vmcnt wait is
    // written out because the compiler's own accounting would wait for every
    // load; sched_barrier(0) keeps LDS reads and MFMAs on their side of it.
    auto step_sync = [&](auto outstanding) {
        if constexpr (!EXACT) __builtin_amdgcn_sched_barrier(0);  // the step's MFMAs stay above the barrier
        __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));  // lgkmcnt(0)
        asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(decltype(outstanding)::value) : "memory");
        __builtin_amdgcn_sched_barrier(0);
    };
    using Steady = std::integral_constant<int, (NSTAGE - 3) * T::LOADS>;
    using First = std::integral_constant<int, (NSTAGE - 2) * T::LOADS>;
    const uint8_t *stage0 = smem;
    auto stage_a = [&](int kt) { return stage0 + (kt % NSTAGE) * T::STAGE; };
    // one 16-byte k-chunk (chunk index c of the step) of every A and B block
    // (the first NA of the A blocks: a wavefront's live ones)
    auto read_chunk = [&](u4 (&fa)[WM], u4 (&fb)[WN], int kt, int c, auto na) {
        const uint8_t *sa = stage_a(kt), *sb = sa + T::A_BYTES;
#pragma unroll
        for (int j = 0; j < WN; ++j) fb[j] = *reinterpret_cast<const u4 *>(sb + b_off_lds[j] + c * 1024);
        // rows a_r0 + 32i share one chunk swizzle (a_swz depends on r/4 mod
        // 4), so the blocks lie 32*BK bytes apart from one per-lane base
        const uint8_t *pa = sa + a_lds_off(a_r0, c);
#pragma unroll
        for (int i = 0; i < decltype(na)::value; ++i) fa[i] = *reinterpret_cast<const u4 *>(pa + i * 32 * BK);
    };

#pragma unroll
    for (int p = 0; p < NSTAGE - 1; ++p) issue_tile(p, p);
    step_sync(First{});  // tile 0

    if constexpr (!CONV && T::ONE_PER_SIMD) {
        // One wavefront per SIMD (2x2 wavefronts of 128x128): a step reads
        // 64 KB of fragments from the LDS instead of the 2x4 layout's 96 KB,
        // and the exact instantiation widens 128 instead of 192 fragment
        // values per lane and SIMD.  Nothing shares a SIMD with the
        // wavefront, so each step's instructions are placed explicitly
        // (sched_barrier between groups): 2 MFMAs, the barrier, then the
        // next step's 16 fragment reads and this wavefront's 8 loads of step
        // kt+NSTAGE-1 (whose stage was last read two steps ago) spread
        // between the MFMAs.  A 5-stage ring keeps 2.5 steps of loads in
        // flight.  Load offsets and the LDS destination (M0) are plain adds,
        // the k-range test only in the steps whose loads reach past K.
        // Against the 2x4 layout on MI355X (bit-identical results): 8192^3
        // +5-7% native FP8, +3% exact; the M = 4096 O- and down-projections
        // +3-4% FP8, +2-3% exact; QKV +1%.  With an fp32 output (the 128x128
        // wavefront tiles' epilogue on 4 wavefronts costs more than the loop
        // gains) and on grids of one tile column it loses 3-6%; those keep
        // the 2x4 layout.
        constexpr int NF = WM + WN;
        static_assert(NF == 8 && T::LOADS == 8 && NSTAGE >= 4,
                      "schedule: 16 chunk reads of 4+4 fragments, 8 loads spread over the MFMAs after the barrier");
        u4 f0[NF][2], f1[NF][2];  // raw E4M3 fragments [A0..A3, B0..B3][16-byte chunk]
        // The 16 chunk reads of a step, q = 0..15 in the order the first
        // MFMAs of a step use them: A0, B0..B3, A1..A3 (two chunks each).
        // Three per-lane bases and compile-time offsets address them: the A
        // row blocks a_r0 + 32i share one swizzle (a_swz depends on r/4 mod
        // 4), so they lie 32*BK bytes apart; B's 32-column block j of this
        // wavefront's 128 columns sits (j/2) panels and (j%2)*32 columns past
        // block 0.
        int ra0 = a_lds_off(a_r0, kgrp), ra1 = a_lds_off(a_r0, kgrp + 1);
        int rb = T::A_BYTES + b_off_lds[0] + kgrp * 1024;
        // the same bases from a lane index computed on the spot (the
        // persistent kernel recomputes them after each tile's epilogue
        // instead of holding them through it)
        auto frag_bases = [&](int ln, int wv) {
            const int kg = (ln >> 5) * 2, r0 = (wv / WAVES_N) * WM * 32 + (ln & 31);
            const int col = (wv % WAVES_N) * WN * 32;
            ra0 = a_lds_off(r0, kg);
            ra1 = a_lds_off(r0, kg + 1);
            rb = T::A_BYTES + (col >> 6) * (CPR * 1024) + ((col & 63) + (ln & 31)) * 16 + kg * 1024;
        };
        auto frag = [&](u4 (&f)[NF][2], int q) -> u4 & {
            const int blk = q >> 1;
            return f[blk == 0 ? 0 : blk <= 4 ? WM + blk - 1 : blk - 4][q & 1];
        };
        const int wave_u = __builtin_amdgcn_readfirstlane(wave);
        auto read = [&](u4 (&f)[NF][2], const uint8_t *st, int q) {
            const int blk = q >> 1, c = q & 1;
            const uint8_t *p = blk >= 1 && blk <= 4
                                   ? st + rb + ((blk - 1) >> 1) * (CPR * 1024) + ((blk - 1) & 1) * 512 + c * 1024
                                   : st + (c ? ra1 : ra0) + (blk == 0 ? 0 : (blk - 4) * 32 * BK);
            frag(f, q) = *reinterpret_cast<const u4 *>(p);
        };
        // load l (A blocks, then B) of step lt into the stage at `lst`
        // DIRECT (persistent walk): the workgroup's next tile, whose first
        // NSTAGE-1 steps the last steps of the current tile load
        int tb = blockIdx.x;
        int64_t nm0 = 0, nn0 = 0;
        bool has_next = false;
        auto load = [&](uint8_t *lst, int lt, int l, bool checked) {
            // DIRECT: steps past the tile's end are the next tile's first
            // ones, and by then a_off / b_off are the next tile's (switched
            // before the first step that loads them)
            if constexpr (DIRECT)
                if (checked && lt >= g.nk) lt -= g.nk;
            const uint32_t kbyte = (uint32_t)lt * BK;
            if (l < T::A_BLK) {
                // rows past M carry OOB, and OOB + kbyte stays out of range;
                // the lane's k-chunk a_kc is the same for every row block
                // (a_swz of row (wave*A_BLK + l)*16 + lane/4 is (lane/16) % 4)
                uint32_t off = a_off[l] + kbyte;
                if (checked) off = kbyte + (uint32_t)a_kc < (uint32_t)g.K ? off : OOB;
                lds_load16(a_rsrc, lst + (wave_u * T::A_BLK + l) * 1024, off);
            } else {
                // past the last step (checked steps only): out of range, as in issue_tile
                const uint32_t boff = b_off[l - T::A_BLK] + (uint32_t)lt * CPR * 1024;
                lds_load16(b_rsrc, lst + T::A_BYTES + (wave_u * T::B_BLK + l - T::A_BLK) * 1024,
                           checked && lt >= g.nk ? OOB : boff);
            }
        };
        auto sync_step = [&]() {
            __builtin_amdgcn_sched_barrier(0);
            asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(Steady::value) : "memory");
            __builtin_amdgcn_sched_barrier(0);
        };
        // exact: the widened 16-k substeps, converted one substep ahead
        bf16x8 cv0[EXACT ? NF : 1], cv1[EXACT ? NF : 1];
        auto conv = [&](bf16x8 (&o)[EXACT ? NF : 1], const u4 (&f)[NF][2], int sub, int x) {
            const u4 &w = f[x][sub >> 1];
            o[x] = (sub & 1) ? e4m3x8_to_bf16(w.z, w.w) : e4m3x8_to_bf16(w.x, w.y);
        };
        // rso: stage offset of step kt+1 (read), lso: of step kt+NSTAGE-1 (loaded)
        // DIRECT: the tile's last step also loads, ahead of its ring loads,
        // this wavefront's 128 columns of per-channel scales and of a C over
        // N into its part of the free ring stage (that of the step itself:
        // the stage before rso), for the epilogue, which waits for them
        // with vmcnt(LOADS).  Lanes 0-31 load 16 bytes each; the rest, and
        // everything when there is nothing to load, read out of range.
        const __amdgpu_buffer_rsrc_t sc_rsrc = __builtin_amdgcn_make_buffer_rsrc(
            (void *)g.e.b_scale, 0, g.e.b_scale && g.e.b_per_channel ? (int)(g.e.N * 4) : 0, 0x00020000);
        const bool c_over_n = g.e.c && !(g.e.c_ndim == 0 || (g.e.c_ndim == 1 && g.e.c0 == 1) ||
                                         (g.e.c_ndim == 2 && g.e.c1 == 1));
        const __amdgpu_buffer_rsrc_t c_rsrc =
            __builtin_amdgcn_make_buffer_rsrc((void *)g.e.c, 0, c_over_n ? (int)(g.e.N * 4) : 0, 0x00020000);
        auto load_coef = [&](int rso_now) {
            if constexpr (DIRECT) {
                uint8_t *dst = smem + (rso_now >= T::STAGE ? rso_now - T::STAGE : (NSTAGE - 1) * T::STAGE) +
                               wave_u * EPD_BYTES;
                const int ln = lane_here();
                const int col = (int)n0 + (wave_u % WAVES_N) * WN * 32 + 4 * ln;
                const uint32_t off = ln < 32 && col < (int)g.N ? (uint32_t)col * 4u : OOB;
                lds_load16(sc_rsrc, dst + EPD_SCALE, off);
                lds_load16(c_rsrc, dst + EPD_C, off);
            }
        };
        // first (DIRECT): the tile's first step, whose MFMAs start from zero
        // instead of the accumulators
        const v16f vzero = {};
        // last (DIRECT): a tile's last step, which reads no fragments of the
        // next step (they are read after the tile's epilogue, so that they
        // are not held through it)
        auto step = [&](u4 (&fc)[NF][2], u4 (&fn)[NF][2], int kt, int rso, int lso, bool checked,
                        auto first, auto last) {
            constexpr bool FIRST = decltype(first)::value, LAST = decltype(last)::value;
            const uint8_t *rst = stage0 + rso;
            uint8_t *lst = smem + lso;
            const int lt = kt + NSTAGE - 1;
            // DIRECT: the fragment bases are recomputed at every step, so
            // that no per-lane value is held through the tile epilogues
            if constexpr (DIRECT) frag_bases(lane_here(), wave_u);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (EXACT) {
                // 4 substeps of 16 bf16 MFMAs; each substep widens the next
                // one's fragments (two conversions per MFMA), the last one
                // the next step's first substep
                // DIRECT: operands swapped (B block first), so that a lane's
                // accumulators hold one output row (epi_direct_bf16)
                auto mma = [&](const bf16x8 (&o)[NF], int b, auto zero_c) {
                    const int i = b / WN, j = b % WN;
                    const v16f &c = decltype(zero_c)::value ? vzero : acc[i][j];
                    if constexpr (DIRECT)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(o[WM + j], o[i], c, 0, 0, 0);
                    else
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(o[i], o[WM + j], c, 0, 0, 0);
                };
                using Acc = std::false_type;
                // DIRECT: a tile's first step widens its own first substep
                // (nothing converted is held through the loop's back edge)
                if constexpr (DIRECT && FIRST) {
                    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));  // lgkmcnt(0): fc landed
#pragma unroll
                    for (int x = 0; x < NF; ++x) conv(cv0, fc, 0, x);
                    __builtin_amdgcn_sched_barrier(0);
                }
                // substep 0: the barrier after 2 MFMAs, then 14 reads
#pragma unroll
                for (int b = 0; b < 16; ++b) {
                    mma(cv0, b, std::integral_constant<bool, FIRST>{});
                    if ((b & 1) == 0) conv(cv1, fc, 1, b >> 1);
                    if (!LAST && b >= 2) read(fn, rst, b - 2);
                    __builtin_amdgcn_sched_barrier(0);
                    if (b == 1) sync_step();
                }
                // substep 1: the last 2 reads, the 8 loads
#pragma unroll
                for (int b = 0; b < 16; ++b) {
                    mma(cv1, b, Acc{});
                    if ((b & 1) == 0) conv(cv0, fc, 2, b >> 1);
                    if (!LAST && b < 2) read(fn, rst, 14 + b);
                    if (LAST && b == 2) load_coef(rso);
                    // the 8 loads one per 4 MFMAs over substeps 1 and 2: in
                    // a burst, the four wavefronts' loads fill the TA's
                    // command FIFO and a stalled load holds up the MFMAs
                    // issued after it (+0.7% at 8192^3)
                    if ((b & 3) == 3) load(lst, lt, b >> 2, checked);
                    __builtin_amdgcn_sched_barrier(0);
                }
#pragma unroll
                for (int b = 0; b < 16; ++b) {
                    mma(cv0, b, Acc{});
                    if ((b & 1) == 0) conv(cv1, fc, 3, b >> 1);
                    if ((b & 3) == 3) load(lst, lt, 4 + (b >> 2), checked);
                    __builtin_amdgcn_sched_barrier(0);
                }
                __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));  // lgkmcnt(0): fn landed
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int b = 0; b < 16; ++b) {
                    mma(cv1, b, Acc{});
                    if (!LAST && (b & 1) == 0) conv(cv0, fn, 0, b >> 1);
                    __builtin_amdgcn_sched_barrier(0);
                }
            } else {
                // 16 FP8 MFMAs: reads two per MFMA on the 8 after the
                // barrier, the 8 loads on the last 6
                auto mma = [&](int b) {
                    const int i = b / WN, j = b % WN;
                    const v16f &c = FIRST ? vzero : acc[i][j];
                    if constexpr (DIRECT)  // operands swapped, as in the exact loop
                        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                            join(fc[WM + j][0], fc[WM + j][1]), join(fc[i][0], fc[i][1]), c, 0, 0, 0, 0, 0, 0);
                    else
                        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                            join(fc[i][0], fc[i][1]), join(fc[WM + j][0], fc[WM + j][1]), c, 0, 0, 0, 0, 0, 0);
                };
                __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));  // lgkmcnt(0): fc landed
                mma(0);
                mma(1);
                sync_step();
                // the loads spread over all 14 MFMAs after the barrier (load
                // l on the MFMA after ceil(14*l/8) - 1 of them): in a burst
                // on the last six, the four wavefronts' loads fill the TA's
                // command FIFO and a stalled load holds up the MFMAs issued
                // after it (+1% at 8192^3)
                int l = 0;
#pragma unroll
                for (int b = 2; b < 16; ++b) {
                    mma(b);
                    if (b < 10 && !LAST) {
                        read(fn, rst, 2 * (b - 2));
                        read(fn, rst, 2 * (b - 2) + 1);
                    }
                    if (LAST && b == 2) load_coef(rso);
#pragma unroll
                    for (int n = ((b - 1) * T::LOADS + 13) / 14 - l; n > 0; --n, ++l) load(lst, lt, l, checked);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        };
#pragma unroll
        for (int q = 0; q < 16; ++q) read(f0, stage_a(0), q);
        if constexpr (EXACT && !DIRECT) {  // DIRECT: the first step converts
            __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));  // lgkmcnt(0)
#pragma unroll
            for (int x = 0; x < NF; ++x) conv(cv0, f0, 0, x);
        }
        int rso = T::STAGE, lso = (NSTAGE - 1) * T::STAGE;
        auto adv = [&]() {
            rso = rso + T::STAGE == NSTAGE * T::STAGE ? 0 : rso + T::STAGE;
            lso = lso + T::STAGE == NSTAGE * T::STAGE ? 0 : lso + T::STAGE;
        };
        // steps whose loads (of step kt+NSTAGE-1) lie inside K need no k test
        const int nfull = (int)(g.K / BK);
        const int l1 = (nfull - (NSTAGE - 1) > 0 ? nfull - (NSTAGE - 1) : 0) & ~1;
        using No = std::false_type;
        if constexpr (DIRECT) {
            // Persistent walk over tiles tb = blockIdx.x, + gridDim.x, ...:
            // the ring runs on across tile boundaries (the last steps of a
            // tile load the next tile's first ones, and its last step reads
            // the next tile's first fragments), and each tile's epilogue
            // stores straight from the accumulators, so nothing of the LDS
            // is needed between tiles and the next tile's loads are in
            // flight meanwhile.  The first step of a tile starts its MFMAs
            // from zero.  nk is even, so every tile starts on f0.
            auto find_next = [&]() {
                has_next = tb + (int)gridDim.x < ntiles;
                if (has_next) tile_origin(tb + (int)gridDim.x, nm0, nn0);
            };
            find_next();
            const DirectUniforms du = direct_uniforms(g.e);
            // wavefront-uniform (scalar) row and column offsets of this wavefront
            const int mr0 = (wave_u / WAVES_N) * WM * 32, nc0 = (wave_u % WAVES_N) * WN * 32;
            using Yes = std::true_type;
            static_assert(NSTAGE == 5, "the offset switch sits four steps before a tile's end");
            static_assert(T::NW * EPD_BYTES <= T::STAGE, "the epilogue staging fits one ring stage");
            static_assert(T::LOADS <= 63, "vmcnt field");
            // from step nk - 4 on, the steps load the next tile's first ones
            auto switch_offsets = [&]() { setup_offsets(nm0, nn0, has_next, lane_here(), wave_u); };
            for (;;) {
                // nk >= 4 (the launcher's condition) and even: a first pair,
                // the middle pairs, the offset switch, the last two pairs
                if (g.nk == 4) switch_offsets();
                step(f0, f1, 0, rso, lso, true, Yes{}, No{}); adv();
                step(f1, f0, 1, rso, lso, true, No{}, No{}); adv();
                if (g.nk > 4) {
                    for (int kt = 2; kt < l1; kt += 2) {
                        step(f0, f1, kt, rso, lso, false, No{}, No{}); adv();
                        step(f1, f0, kt + 1, rso, lso, false, No{}, No{}); adv();
                    }
                    for (int kt = l1 > 2 ? l1 : 2; kt < g.nk - 4; kt += 2) {
                        step(f0, f1, kt, rso, lso, true, No{}, No{}); adv();
                        step(f1, f0, kt + 1, rso, lso, true, No{}, No{}); adv();
                    }
                    switch_offsets();
                    step(f0, f1, g.nk - 4, rso, lso, true, No{}, No{}); adv();
                    step(f1, f0, g.nk - 3, rso, lso, true, No{}, No{}); adv();
                }
                step(f0, f1, g.nk - 2, rso, lso, true, No{}, No{}); adv();
                step(f1, f0, g.nk - 1, rso, lso, true, No{}, Yes{}); adv();
                __builtin_amdgcn_sched_barrier(0);
                const Epilogue &e = g.e;
                // the ring stage of this tile's last step: its fragments were
                // read in the step before, every wavefront is past that
                // step's barrier, and the next loads into it follow the next
                // step's barrier
                uint8_t *est = smem + (rso >= 2 * T::STAGE ? rso - 2 * T::STAGE : rso + (NSTAGE - 2) * T::STAGE) +
                               wave_u * EPD_BYTES;
                // the coefficient loads landed: only the last step's ring
                // loads, issued after them, may still be in flight
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(T::LOADS) : "memory");
                const int mt = (int)m0 + mr0, nt = (int)n0 + nc0;
                if (e.alpha == 1.0f) {
                    if (e.c) epi_direct_bf16<ACT_NONE, true, true>(e, du, acc, mt, nt, est);
                    else epi_direct_bf16<ACT_NONE, false, true>(e, du, acc, mt, nt, est);
                } else {
                    if (e.c) epi_direct_bf16<ACT_NONE, true, false>(e, du, acc, mt, nt, est);
                    else epi_direct_bf16<ACT_NONE, false, false>(e, du, acc, mt, nt, est);
                }
                __builtin_amdgcn_sched_barrier(0);
                if (!has_next) break;
                tb += (int)gridDim.x;
                m0 = nm0;
                n0 = nn0;
                find_next();
                // the next tile's first fragments: step 0's stage, the one
                // before rso (it landed by the last step's barrier, and no
                // load targets it before the next step's barrier)
                frag_bases(lane_here(), wave_u);  // for the reads below
                const uint8_t *st0 = stage0 + (rso == 0 ? (NSTAGE - 1) * T::STAGE : rso - T::STAGE);
#pragma unroll
                for (int q = 0; q < 16; ++q) read(f0, st0, q);
            }
        } else {
            for (int kt = 0; kt < l1; kt += 2) {
                step(f0, f1, kt, rso, lso, false, No{}, No{}); adv();
                step(f1, f0, kt + 1, rso, lso, false, No{}, No{}); adv();
            }
            for (int kt = l1; kt < g.nk; kt += 2) {
                step(f0, f1, kt, rso, lso, true, No{}, No{}); adv();
                step(f1, f0, kt + 1, rso, lso, true, No{}, No{}); adv();
            }
        }
    } else {
    // the loops of the 2x4 and 128x128 layouts for LV live 32-row blocks
    // of this wavefront (WM, but fewer in a slice): the others take no
    // fragment reads, conversions or MFMAs
    auto tile_loop = [&](auto lv) {
    constexpr int LV = decltype(lv)::value;
    using NA = std::integral_constant<int, LV>;
    if constexpr (PP) {
        // Ping-pong: the two wavefronts on each SIMD (row halves wm = 0 and
        // wm = 1; wavefront w runs on SIMD w % 4) take turns.  A phase ends
        // at a workgroup barrier; in each phase one group issues its share of
        // a tile's global->LDS loads and reads its fragments of the next
        // step from LDS (the memory phase) while the other group only issues
        // matrix-core instructions on fragments it already holds (the
        // compute phase), so the SIMD's MFMA pipe is fed from registers
        // while the LDS serves the other wavefront.  Group 1 runs one phase
        // behind group 0 (one extra barrier at its start, one at group 0's
        // end: both execute 2*nk + 1 barriers).
        //   phase 2m:   group 0 memory (step m),  group 1 compute (step m-1)
        //   phase 2m+1: group 0 compute (step m), group 1 memory (step m)
        // Memory phase of step m: issue tile m+NSTAGE-1 into the stage of
        // tile m-1 (read by both groups in phases 2m-2 and 2m-1, whose reads
        // completed before those phases' barriers), read tile m, wait for
        // the reads (lgkmcnt(0)).  Every phase ends with vmcnt((NSTAGE-2) *
        // LOADS): a wavefront that has issued tiles up to m+NSTAGE-1 then
        // holds tiles <= m+1, so at the barrier closing phase 2m+1 every
        // wavefront's share of tile m+1 has landed, before group 0 reads it
        // in phase 2m+2.
        const bool second = wm != 0;  // wavefront-uniform
        auto phase_end = [&](bool lds_reads) {
            // nothing of the phase may sink below its barrier (MFMAs do not
            // touch memory, so the asm's memory clobber alone does not hold them)
            __builtin_amdgcn_sched_barrier(0);
            if (lds_reads) __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));  // lgkmcnt(0)
            asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(First::value) : "memory");
            __builtin_amdgcn_sched_barrier(0);
        };
        u4 fa[WM][2], fb[WN][2];
        if (second) {
            asm volatile("s_barrier" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
        }
        for (int m = 0; m < g.nk; ++m) {
            issue_tile(m + NSTAGE - 1, (m + NSTAGE - 1) % NSTAGE);
            {
                u4 ta[WM], tb[WN];
                read_chunk(ta, tb, m, kgrp, NA{});
#pragma unroll
                for (int i = 0; i < LV; ++i) fa[i][0] = ta[i];
#pragma unroll
                for (int j = 0; j < WN; ++j) fb[j][0] = tb[j];
                read_chunk(ta, tb, m, kgrp + 1, NA{});
#pragma unroll
                for (int i = 0; i < LV; ++i) fa[i][1] = ta[i];
#pragma unroll
                for (int j = 0; j < WN; ++j) fb[j][1] = tb[j];
            }
            phase_end(true);
            if constexpr (EXACT) {
#pragma unroll
                for (int c = 0; c < 2; ++c)
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        bf16x8 a16[WM], b16[WN];
#pragma unroll
                        for (int i = 0; i < LV; ++i)
                            a16[i] = h ? e4m3x8_to_bf16(fa[i][c].z, fa[i][c].w) : e4m3x8_to_bf16(fa[i][c].x, fa[i][c].y);
#pragma unroll
                        for (int j = 0; j < WN; ++j)
                            b16[j] = h ? e4m3x8_to_bf16(fb[j][c].z, fb[j][c].w) : e4m3x8_to_bf16(fb[j][c].x, fb[j][c].y);
#pragma unroll
                        for (int i = 0; i < LV; ++i)
#pragma unroll
                            for (int j = 0; j < WN; ++j)
                                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a16[i], b16[j], acc[i][j], 0, 0, 0);
                    }
            } else {
#pragma unroll
                for (int i = 0; i < LV; ++i)
#pragma unroll
                    for (int j = 0; j < WN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                            join(fa[i][0], fa[i][1]), join(fb[j][0], fb[j][1]), acc[i][j], 0, 0, 0, 0, 0, 0);
            }
            phase_end(false);
        }
        if (!second) {
            asm volatile("s_barrier" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
        }
    } else if constexpr (EXACT) {
        // Each lane's 64-k fragment is two 16-byte chunks (lo: chunk kgrp,
        // hi: kgrp+1), each feeding two 32x32x16 bf16 MFMA groups (8 bytes
        // per group, widened exactly).  The chunk of the next half is read
        // while the MFMAs of the current half run: lo(kt) is read during the
        // hi half of step kt-1, hi(kt) during the lo half of step kt.
        u4 lo_a[WM], lo_b[WN], hi_a[WM], hi_b[WN];
        auto mma_half = [&](const u4 (&fa)[WM], const u4 (&fb)[WN]) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                bf16x8 a16[WM], b16[WN];
#pragma unroll
                for (int i = 0; i < LV; ++i) a16[i] = h ? e4m3x8_to_bf16(fa[i].z, fa[i].w) : e4m3x8_to_bf16(fa[i].x, fa[i].y);
#pragma unroll
                for (int j = 0; j < WN; ++j) b16[j] = h ? e4m3x8_to_bf16(fb[j].z, fb[j].w) : e4m3x8_to_bf16(fb[j].x, fb[j].y);
#pragma unroll
                for (int i = 0; i < LV; ++i)
#pragma unroll
                    for (int j = 0; j < WN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a16[i], b16[j], acc[i][j], 0, 0, 0);
            }
        };
        read_chunk(lo_a, lo_b, 0, kgrp, NA{});
        for (int kt = 0; kt < g.nk; ++kt) {
            read_chunk(hi_a, hi_b, kt, kgrp + 1, NA{});
            __builtin_amdgcn_sched_barrier(0);
            mma_half(lo_a, lo_b);
            step_sync(Steady{});  // tile kt+1
            issue_tile(kt + NSTAGE - 1, (kt + NSTAGE - 1) % NSTAGE);
            read_chunk(lo_a, lo_b, kt + 1, kgrp, NA{});  // past the end: an unused stage
            __builtin_amdgcn_sched_barrier(0);
            mma_half(hi_a, hi_b);
        }
    } else {
        // 32x32x64 FP8 MFMAs take the whole 32-byte fragment; the fragments
        // of step kt+1 are read (second register set) while step kt's run.
        // nk is even (K is padded to 128), so steps come in pairs.
        u4 a0[WM][2], b0[WN][2], a1[WM][2], b1[WN][2];
        auto read_frag = [&](u4 (&fa)[WM][2], u4 (&fb)[WN][2], int kt) {
            u4 ta[WM], tb[WN];
            read_chunk(ta, tb, kt, kgrp, NA{});
#pragma unroll
            for (int i = 0; i < LV; ++i) fa[i][0] = ta[i];
#pragma unroll
            for (int j = 0; j < WN; ++j) fb[j][0] = tb[j];
            read_chunk(ta, tb, kt, kgrp + 1, NA{});
#pragma unroll
            for (int i = 0; i < LV; ++i) fa[i][1] = ta[i];
#pragma unroll
            for (int j = 0; j < WN; ++j) fb[j][1] = tb[j];
        };
        auto mma = [&](const u4 (&fa)[WM][2], const u4 (&fb)[WN][2]) {
#pragma unroll
            for (int i = 0; i < LV; ++i)
#pragma unroll
                for (int j = 0; j < WN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(join(fa[i][0], fa[i][1]),
                                                                                join(fb[j][0], fb[j][1]), acc[i][j], 0,
                                                                                0, 0, 0, 0, 0);
        };
        // the step's MFMAs and the next step's fragment reads are issued
        // interleaved (sched_interleave), not as a burst of reads first
        auto interleave = [&]() { sched_interleave<LV * WN, 2 * (LV + WN), T::LOADS>(); };
        read_frag(a0, b0, 0);
        for (int kt = 0; kt < g.nk; kt += 2) {
            step_sync(Steady{});  // tile kt+1
            issue_tile(kt + NSTAGE - 1, (kt + NSTAGE - 1) % NSTAGE);
            read_frag(a1, b1, kt + 1);
            mma(a0, b0);
            interleave();
            step_sync(Steady{});  // tile kt+2
            issue_tile(kt + NSTAGE, (kt + NSTAGE) % NSTAGE);
            read_frag(a0, b0, kt + 2);  // past the end: an unused stage
            mma(a1, b1);
            interleave();
        }
    }
    };
    if constexpr (SLICE) {
        switch (wlive) {
        case 1: tile_loop(std::integral_constant<int, 1>{}); break;
        case 2: tile_loop(std::integral_constant<int, 2>{}); break;
        case 3: tile_loop(std::integral_constant<int, 3>{}); break;
        default: tile_loop(std::integral_constant<int, WM>{}); break;
        }
    } else {
        tile_loop(std::integral_constant<int, WM>{});
    }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the tail's loads land before the LDS is reused
    if constexpr (DIRECT) return;  // every tile's epilogue ran in the persistent loop
    __syncthreads();

    // ---- epilogue --------------------------------------------------------
    // The accumulators go through LDS (free after the last barrier), so the
    // epilogue runs as one rolled loop with fixed columns per lane instead
    // of unrolled copies of the activation code.
    Epilogue e = g.e;
    if (CONV && grp) {  // this group's output channels
        if (e.b_scale && e.b_per_channel) e.b_scale += (int64_t)grp * e.N;
        if (e.c) e.c += (int64_t)grp * e.N;
    }
    const float a_s = e.a_scale ? e.a_scale[0] : 1.0f;
    if constexpr (CONV) {
    float *st = reinterpret_cast<float *>(smem) + wave * (WM * 32 * EP_PITCH);
#pragma unroll
    for (int j = 0; j < WN; ++j) {
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                st[(i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3)) * EP_PITCH + (lane & 31)] = acc[i][j][r];
        __syncthreads();
        if constexpr (CONV) {
            // NCHW output: lanes run along output pixels (rows), so each
            // column's stores are contiguous.  The column's scale and a
            // row-invariant bias are read once per block (lane c holds column
            // c) and taken per column with v_readlane, so the column loop has
            // no memory reads besides the staged sums; a bias that varies over
            // rows is read per element.
            const uint32_t ohw = (uint32_t)(g.cv.OH * g.cv.OW);
            const int64_t colb = n0 + wn * WN * 32 + j * 32;  // first column of this block
            const int ncol = colb < e.N ? (int)(e.N - colb < 32 ? e.N - colb : 32) : 0;
            const bool inv = !e.c || epi_c_row_invariant(e);
            const int64_t lc = colb + (lane & 31) < e.N ? colb + (lane & 31) : e.N - 1;  // in range
            // lane c: column c's scale and (row-invariant C) beta * C
            int sc_l = __builtin_bit_cast(int, epi_scale(e, a_s, lc));
            const float cv = e.c && inv ? epi_c(e, 0, lc) : 0.0f;
            int cb_l = __builtin_bit_cast(int, e.beta == 1.0f ? cv : e.beta * cv);
            // pinned here, where every lane is active: v_readlane below reads
            // lanes that the row test may have switched off
            asm volatile("" : "+v"(sc_l), "+v"(cb_l));

#pragma unroll 1
            for (int h = 0; h < WM / 2; ++h) {
                const int rl = h * 64 + lane;
                const int64_t m = m0 + wrow0 + rl;
                // the wavefront's live rows only (a slice's other rows are
                // the next slice's)
                if (rl < wlive * 32 && m < e.M) {
                    const uint32_t n = (uint32_t)m / ohw, pix = (uint32_t)m - n * ohw;
                    const int64_t ybase = ((int64_t)n * g.cv.CoutTot + (int64_t)grp * e.N) * ohw + pix;
                    if (inv) {
                        // the loop specialised for the epilogue's choices (epi_cols)
                        const float *srow = st + rl * EP_PITCH;
                        void *p = (uint8_t *)e.y + (ybase + colb * ohw) * (e.y_bf16 ? 2 : 4);
                        auto go = [&](auto act, auto has_c, auto bf) {
                            epi_cols<decltype(act)::value, decltype(has_c)::value, decltype(bf)::value>(
                                e, srow, p, ohw, ncol, sc_l, cb_l);
                        };
                        auto by_out = [&](auto act, auto has_c) {
                            if (e.y_bf16)
                                go(act, has_c, std::true_type{});
                            else
                                go(act, has_c, std::false_type{});
                        };
                        auto by_c = [&](auto act) {
                            if (e.c)
                                by_out(act, std::true_type{});
                            else
                                by_out(act, std::false_type{});
                        };
                        // the conv's usual activations specialised; the GELU
                        // forms share one instance that reads e.act (fewer
                        // copies of the loop: the kernel's code size costs
                        // time in every phase)
                        if (e.act == ACT_RELU)
                            by_c(std::integral_constant<int, ACT_RELU>{});
                        else if (e.act == ACT_NONE)
                            by_c(std::integral_constant<int, ACT_NONE>{});
                        else
                            by_c(std::integral_constant<int, -1>{});
                    } else {
#pragma unroll 1
                        for (int c = 0; c < ncol; ++c) {
                            const int64_t col = colb + c;
                            const float v = epi_value(e, __builtin_bit_cast(float, __builtin_amdgcn_readlane(sc_l, c)),
                                                      m, col, st[rl * EP_PITCH + c]);
                            if (e.y_bf16)
                                reinterpret_cast<uint16_t *>(e.y)[ybase + col * ohw] = bf16_rne(v);
                            else
                                reinterpret_cast<float *>(e.y)[ybase + col * ohw] = v;
                        }
                    }
                }
            }
        }
        __syncthreads();
    }
    } else {
        // Row-major output: 64 rows x 64 of the wavefront's columns per pass
        // (two 32-row accumulator blocks of two 32-column blocks), and each
        // lane stores two adjacent columns, so a row's 64 outputs leave as one
        // contiguous 128-byte (bf16) or 256-byte (fp32) run: whole cache
        // lines, where one column per lane wrote half lines of bf16.  Row
        // pitch 72 floats: the two rows of a staging write instruction
        // (lanes 0-31 and 32-63, 4 rows apart) fall in opposite bank halves.
        static_assert(WN % 2 == 0 && WM % 2 == 0, "32-column and 32-row block pairs");
        constexpr int ER = T::EP_ROWS;
        float amax_m = 0.0f;  // AMAX: this lane's max |y|
        // the end of this wavefront's rows: M, or in a row slice the end of
        // its live blocks (the slice's later rows are another slice's)
        const int64_t wend = m0 + wrow0 + (int64_t)wlive * 32;
        const int64_t m_end = wend < e.M ? wend : e.M;
        float *st = reinterpret_cast<float *>(smem) + wave * (ER * EP2_PITCH);
#pragma unroll
        for (int jp = 0; jp < WN / 2; ++jp) {
        // this lane's two columns: col, col + 1
        const int64_t col = n0 + wn * WN * 32 + jp * 64 + 2 * (lane & 31);
        const bool c0ok = col < e.N, c1ok = col + 1 < e.N;
        const float sc0 = c0ok ? epi_scale(e, a_s, col) : 0.0f, sc1 = c1ok ? epi_scale(e, a_s, col + 1) : 0.0f;
        const bool inv = !e.c || epi_c_row_invariant(e);
        const float cv0 = e.c && inv && c0ok ? epi_c(e, 0, col) : 0.0f;
        const float cv1 = e.c && inv && c1ok ? epi_c(e, 0, col + 1) : 0.0f;
        // both columns in one store when both are in range and the pair is
        // aligned: col is even, so an even row pitch and a 4-byte (bf16) or
        // 8-byte (fp32) aligned y suffice
        const bool pair = c1ok && (e.ldy % 2) == 0 &&
                          (reinterpret_cast<uintptr_t>(e.y) & (e.y_bf16 ? 3u : 7u)) == 0;
        // the specialised passes (epi_rows) where C is row-invariant, every
        // lane's columns come in aligned pairs (N and ldy even) and the
        // output's offsets fit 31 bits
        const bool fast = inv && (e.N % 2) == 0 && (e.ldy % 2) == 0 &&
                          (reinterpret_cast<uintptr_t>(e.y) & (e.y_bf16 ? 3u : 7u)) == 0 &&
                          (e.M + 64) * e.ldy * (e.y_bf16 ? 2 : 4) < ((int64_t)1 << 31);
        const float cb0 = e.c ? (e.beta == 1.0f ? cv0 : e.beta * cv0) : 0.0f;
        const float cb1 = e.c ? (e.beta == 1.0f ? cv1 : e.beta * cv1) : 0.0f;
        auto fast_pass = [&](const float *src, int64_t row0) {
            auto go = [&](auto act, auto has_c, auto bf) {
                epi_rows<decltype(act)::value, decltype(has_c)::value, decltype(bf)::value, AMAX>(
                    e, src, row0, col, c0ok, sc0, sc1, cb0, cb1, amax_m, c1ok, m_end);
            };
            auto by_out = [&](auto act, auto has_c) {
                if (e.y_bf16)
                    go(act, has_c, std::true_type{});
                else
                    go(act, has_c, std::false_type{});
            };
            auto by_c = [&](auto act) {
                if (e.c)
                    by_out(act, std::true_type{});
                else
                    by_out(act, std::false_type{});
            };
            switch (e.act) {
            case ACT_RELU: by_c(std::integral_constant<int, ACT_RELU>{}); break;
            case ACT_GELU_ERF: by_c(std::integral_constant<int, ACT_GELU_ERF>{}); break;
            case ACT_GELU_TANH: by_c(std::integral_constant<int, ACT_GELU_TANH>{}); break;
            default: by_c(std::integral_constant<int, ACT_NONE>{}); break;
            }
        };
#pragma unroll
        for (int h = 0; h < WM * 32 / ER; ++h) {
#pragma unroll
            for (int ii = 0; ii < ER / 32; ++ii)
#pragma unroll
                for (int jj = 0; jj < 2; ++jj)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        st[(ii * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3)) * EP2_PITCH + jj * 32 + (lane & 31)] =
                            acc[h * (ER / 32) + ii][2 * jp + jj][r];
            __syncthreads();
#pragma unroll
            for (int sub = 0; sub < ER / 64; ++sub) {
                const int64_t row0 = m0 + wrow0 + h * ER + sub * 64 + (lane >> 5);
                const float *src = st + (sub * 64 + (lane >> 5)) * EP2_PITCH + 2 * (lane & 31);
                if (fast) {
                    fast_pass(src, row0);
                } else if (c0ok) {
                    if (inv) {
#pragma unroll 4
                        for (int q = 0; q < 32; ++q) {
                            const int64_t row = row0 + 2 * q;
                            const float2 a = *reinterpret_cast<const float2 *>(src + 2 * q * EP2_PITCH);
                            const float v0 = epi_value_cv(e, sc0, cv0, a.x), v1 = epi_value_cv(e, sc1, cv1, a.y);
                            if (row < m_end) {
                                if constexpr (AMAX) {
                                    amax_m = fabsf(v0) > amax_m ? fabsf(v0) : amax_m;
                                    amax_m = c1ok && fabsf(v1) > amax_m ? fabsf(v1) : amax_m;
                                }
                                if (pair) {
                                    epi_store2(e, row, col, v0, v1);
                                } else {
                                    epi_store(e, row, col, v0);
                                    if (c1ok) epi_store(e, row, col + 1, v1);
                                }
                            }
                        }
                    } else {
#pragma unroll 1
                        for (int q = 0; q < 32; ++q) {
                            const int64_t row = row0 + 2 * q;
                            if (row >= m_end) break;
                            const float2 a = *reinterpret_cast<const float2 *>(src + 2 * q * EP2_PITCH);
                            const float v0 = epi_value(e, sc0, row, col, a.x);
                            if constexpr (AMAX) amax_m = fabsf(v0) > amax_m ? fabsf(v0) : amax_m;
                            if (c1ok) {
                                const float v1 = epi_value(e, sc1, row, col + 1, a.y);
                                if constexpr (AMAX) amax_m = fabsf(v1) > amax_m ? fabsf(v1) : amax_m;
                                if (pair) {
                                    epi_store2(e, row, col, v0, v1);
                                } else {
                                    epi_store(e, row, col, v0);
                                    epi_store(e, row, col + 1, v1);
                                }
                            } else {
                                epi_store(e, row, col, v0);
                            }
                        }
                    }
                }
            }
            __syncthreads();
        }
        }
        if constexpr (AMAX) {
            // the workgroup's partial: a wavefront max, then the wavefronts'
            // through LDS (free after the last pass's barrier)
            const float wm_max = wave_max(amax_m);
            float *red = reinterpret_cast<float *>(smem);
            if (lane == 0) red[wave] = wm_max;
            __syncthreads();
            if (tid == 0) {
                float m = red[0];
#pragma unroll
                for (int w = 1; w < T::NW; ++w) m = red[w] > m ? red[w] : m;
                e.amax_part[blockIdx.x] = __builtin_bit_cast(uint32_t, m);
            }
        }
    }
}

constexpr int WAVES_M = LCML_GEMM_WAVES_M, WAVES_N = LCML_GEMM_WAVES_N;
#ifndef LCML_GEMM_WM
#define LCML_GEMM_WM 4
#endif
#ifndef LCML_GEMM_WN
#define LCML_GEMM_WN 2
#endif
constexpr int WM = LCML_GEMM_WM, WN = LCML_GEMM_WN;  // 32x32 blocks per wavefront
static_assert(WM % 2 == 0, "the NCHW epilogue walks 64-row halves");
using Shipped = Tile<WAVES_M, WAVES_N, WM, WN>;

// 128x128 tiles (2x2 wavefronts of 64x64): a quarter of the work per tile,
// about half a 256x256 tile's time, and two workgroups per CU (64 KB of
// LDS each).  It serves mid-size GEMMs whose 256x256 grid would leave most
// CUs idle.
using Small = Tile<2, 2, 2, 2>;

// 256x256 tiles of 2x2 wavefronts of 128x128: one wavefront per SIMD and
// a five-stage ring (the k_gemm_mfma loop for Tile::ONE_PER_SIMD).
using Wide = Tile<2, 2, 4, 4>;

// compute units of the current device (the persistent grid's size), cached per device
int device_cus() {
    static std::atomic<int> cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cus[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

#ifndef LCML_CONV_SLICES
#define LCML_CONV_SLICES 1
#endif
#ifndef LCML_GEMM_SLICES
#define LCML_GEMM_SLICES 1
#endif

// Row slices of the 2x4 layout's last round of tiles (one workgroup per
// CU): h = the rows left over the CUs, rounded up to 32 (at least 64, and
// up again while the slices outnumber the CUs); none where h reaches BM.
// One tile column (cols = 0): the last round's rows below the whole tiles,
// e.g. 100352 rows (32 images of 56x56) as 256 whole tiles, then 218 slices
// of 160 rows, instead of 392 whole tiles in two full rounds.  More
// columns: the whole tiles of the first `cols` tile columns, then each
// other column cut into slices, e.g. 4096x11008 as 512 whole tiles (32
// columns), then 11 x 22 slices of 192 rows, instead of 688 whole tiles in
// 2.69 rounds.
struct SlicePlan {
    int first = 0, rows = 0, cols = 0;
    int64_t grid = 0;
};
SlicePlan plan_slices(int64_t M, int tiles_m, int tiles_n, int BM, int64_t cus) {
    SlicePlan p;
    p.grid = (int64_t)tiles_m * tiles_n;
    const int64_t round0 = (p.grid - 1) / cus * cus;  // whole tiles before the last round
    int64_t first, rem, cols = 0;
    if (tiles_n == 1) {
        first = round0;
        rem = M - first * BM;
    } else {
        cols = round0 / tiles_m;  // whole tile columns
        if (cols < 1) return p;
        first = cols * tiles_m;
        rem = (tiles_n - cols) * M;
    }
    int64_t h = ((rem + cus - 1) / cus + 31) / 32 * 32;
    h = h < 64 ? 64 : h;
    auto slices = [&](int64_t hh) { return tiles_n == 1 ? (rem + hh - 1) / hh : (tiles_n - cols) * ((M + hh - 1) / hh); };
    while (h < BM && slices(h) > cus) h += 32;
    if (h >= BM) return p;
    p.first = (int)first;
    p.rows = (int)h;
    p.cols = (int)cols;
    p.grid = first + slices(h);
    return p;
}

template <class Cfg, int WMv, int WNv, int WMb, int WNb, bool EXACT, bool CONV, bool PP = false, bool DIRECT = false,
          bool AMAX = false>
hipError_t launch_cfg(GemmArgs &g, hipStream_t s) {
    auto *fn = k_gemm_mfma<WMv, WNv, WMb, WNb, EXACT, CONV, PP, DIRECT, AMAX>;
    static std::atomic<uint64_t> lds_set{0};
    if (hipError_t err = ensure_dynamic_lds(reinterpret_cast<const void *>(fn), Cfg::LDS_BYTES, lds_set);
        err != hipSuccess)
        return err;
    int64_t Kp = pad_to(g.K, kPackK), Np = pad_to(g.N, kPanelCols);
    g.KC = Kp / 16;
    g.npanels = Np / 64;
    g.tiles_m = (int)((g.M + Cfg::BM - 1) / Cfg::BM);
    g.tiles_n = (int)((g.N + Cfg::BN - 1) / Cfg::BN);
    g.nk = (int)(Kp / BK);
    g.b_bytes = (uint32_t)(g.npanels * g.KC * 1024);
    // launched by name, as every other kernel here: a launch through the
    // pointer variable returned success without running the kernel when the
    // host pass was built with -fsanitize=address,undefined
    // the persistent kernel: one workgroup per CU (its LDS use allows no
    // more), each walking tiles blockIdx.x + k * gridDim.x
    int grid = g.tiles_m * g.tiles_n;
    if constexpr (DIRECT) grid = grid < device_cus() ? grid : device_cus();
    // the 2x4 layout's last round as row slices (plan_slices): the conv on
    // one tile column without groups, and the GEMM
    g.slice_first = g.slice_rows = g.slice_cols = 0;
    if constexpr (WMv == 2 && WMb == 4 && !Cfg::ONE_PER_SIMD)
        if (CONV ? LCML_CONV_SLICES && g.tiles_n == 1 && g.cv.CoutTot == (int)g.N : LCML_GEMM_SLICES) {
            const SlicePlan p = plan_slices(g.M, g.tiles_m, g.tiles_n, Cfg::BM, device_cus());
            g.slice_first = p.first;
            g.slice_rows = p.rows;
            g.slice_cols = p.cols;
            grid = (int)p.grid;
        }
    hipLaunchKernelGGL((k_gemm_mfma<WMv, WNv, WMb, WNb, EXACT, CONV, PP, DIRECT, AMAX>),
                       dim3(grid, CONV ? g.cv.CoutTot / (int)g.N : 1), dim3(Cfg::NT), Cfg::LDS_BYTES, s, g);
    return hipGetLastError();
}

#ifndef LCML_GEMM_PINGPONG
#define LCML_GEMM_PINGPONG 1
#endif
// the ping-pong schedule needs the two wavefronts of each SIMD in different
// groups: WAVES_M == 2 row halves over 4 SIMDs
static_assert(!LCML_GEMM_PINGPONG || (WAVES_M == 2 && WAVES_M * WAVES_N == 8), "ping-pong layout");

// The exact instantiation takes the ping-pong schedule: measured on MI355X
// at 8192^3 and the M = 4096 transformer and conv shapes it is 1-4% faster
// (bitwise-identical results); the native-FP8 one keeps the interleaved
// schedule (mixed: -8% on the conv, within +-1% elsewhere).
// The GEMM takes the one-wavefront-per-SIMD layout where it measured
// faster: a bf16 output (with fp32 the epilogue of its 128x128 wavefront
// tiles costs more than the main loop gains) on a grid of more than one
// tile column.
#ifndef LCML_GEMM_DIRECT
#define LCML_GEMM_DIRECT 1
#endif
// The persistent direct-store variant of the one-wavefront-per-SIMD layout
// takes the outputs its epilogue covers: N and the row pitch multiples of 8,
// a 16-byte aligned y whose M rows of pitch stay below 2^31 bytes, C absent
// or row-invariant, no activation (the others keep the staged epilogue);
// and K > 128, so that a tile has at least four 64-k steps.
bool direct_epilogue_ok(const Epilogue &e) {
    const bool c_ok = !e.c || e.c_ndim == 0 || (e.c_ndim == 1 && (e.c0 == 1 || e.c0 == e.N)) ||
                      (e.c_ndim == 2 && e.c0 == 1);
    return LCML_GEMM_DIRECT && e.y_bf16 && c_ok && e.act == ACT_NONE && e.N % 8 == 0 &&
           e.ldy % 8 == 0 && (reinterpret_cast<uintptr_t>(e.y) & 15) == 0 &&
           e.M * e.ldy * 2 < ((int64_t)1 << 31);
}

template <bool EXACT, bool CONV>
hipError_t launch(GemmArgs &g, hipStream_t s) {
    if constexpr (!CONV)
        if (g.e.amax_part)  // fp32 outputs only (the caller's condition): the 2x4 layout
            return launch_cfg<Shipped, WAVES_M, WAVES_N, WM, WN, EXACT, false, EXACT && (bool)LCML_GEMM_PINGPONG,
                              false, true>(g, s);
    if constexpr (!CONV)
        if (g.e.y_bf16 && g.N > Wide::BN) {
            if (direct_epilogue_ok(g.e) && g.K > kPackK) return launch_cfg<Wide, 2, 2, 4, 4, EXACT, false, false, true>(g, s);
            return launch_cfg<Wide, 2, 2, 4, 4, EXACT, false>(g, s);
        }
    return launch_cfg<Shipped, WAVES_M, WAVES_N, WM, WN, EXACT, CONV, EXACT && (bool)LCML_GEMM_PINGPONG>(g, s);
}

}  // namespace

hipError_t launch_gemm_mfma(int64_t M, int64_t N, int64_t K, const uint8_t *a, int64_t lda,
                            const uint8_t *bp, const Epilogue &e, bool exact, hipStream_t s, bool small_tiles) {
    GemmArgs g = {};
    g.M = M; g.N = N; g.K = K; g.a = a; g.lda = lda; g.bp = bp;
    g.a_bytes = (uint32_t)((M - 1) * lda + K);
    g.e = e;
    if (small_tiles) {
        if (e.amax_part)
            return exact ? launch_cfg<Small, 2, 2, 2, 2, true, false, false, false, true>(g, s)
                         : launch_cfg<Small, 2, 2, 2, 2, false, false, false, false, true>(g, s);
        return exact ? launch_cfg<Small, 2, 2, 2, 2, true, false>(g, s) : launch_cfg<Small, 2, 2, 2, 2, false, false>(g, s);
    }
    return exact ? launch<true, false>(g, s) : launch<false, false>(g, s);
}

int64_t gemm_mfma_workgroups(int64_t M, int64_t N, bool small_tiles) {
    const int64_t t = small_tiles ? 128 : 256;
    const int tm = (int)((M + t - 1) / t), tn = (int)((N + t - 1) / t);
    // the amax-partials launch (an fp32 output) on 256x256 tiles takes the
    // 2x4 layout, whose last round may run as row slices
    if (!small_tiles && LCML_GEMM_SLICES) return plan_slices(M, tm, tn, Shipped::BM, device_cus()).grid;
    return (int64_t)tm * tn;
}

hipError_t launch_conv_mfma(const uint8_t *x_nhwc, int64_t Nb, int C, int H, int W, const uint8_t *bp, int Cout,
                            int KH, int KW, int sh, int sw, int ph, int pw, int dh, int dw, int group, int OH, int OW,
                            const Epilogue &e, bool exact, hipStream_t s, bool small_tiles) {
    GemmArgs g = {};
    const int Cg = C / group;
    g.cv = ConvGeom{H, W, Cg, C, Cout, OH, OW, KH, KW, sh, sw, ph, pw, dh, dw};
    g.M = Nb * OH * OW; g.N = Cout / group; g.K = (int64_t)KH * KW * Cg;
    g.a = x_nhwc; g.lda = 0; g.bp = bp;
    g.a_bytes = (uint32_t)(Nb * H * W * C);
    g.e = e;
    if (small_tiles)
        return exact ? launch_cfg<Small, 2, 2, 2, 2, true, true>(g, s) : launch_cfg<Small, 2, 2, 2, 2, false, true>(g, s);
    return exact ? launch<true, true>(g, s) : launch<false, true>(g, s);
}

}  // namespace lcml
