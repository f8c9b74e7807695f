// gemm_skinny.hip -- small-M (decode-shaped, M <= 16) FP8 GEMM on gfx950.
//
// The weight matrix is read exactly once, straight from HBM into registers
// as 128-bit loads in packed-panel order (no LDS staging: every weight byte
// is used by exactly one wavefront).  A workgroup of WAVES wavefronts owns
// 16*NB output columns (NB = 4: one whole 64-column panel, so every k-chunk
// row of 1 KB is read contiguously by one workgroup); the wavefronts split K,
// each issues the weight loads of UNROLL K blocks before their MFMAs, and the
// partial 16x16 tiles are summed through LDS before the epilogue.  The
// activations (M <= 16 rows, padded to 16 with zeros) are re-read from L2 by
// every workgroup, 16*K bytes each, so NB also sets that re-read traffic.
// The activation rows are the A operand: lane l holds row l%16,
// k = (l/16)*32+0..31 of each 128-k block; the weight operand: lane l holds
// column l%16 of a 16-column block and the same k range, i.e. two
// consecutive 16-byte chunks of the packed panel.
// EXACT (default): the 32 bytes are widened to bf16 (exact) and fed to four
// v_mfma_f32_16x16x32_bf16 (fp32-accurate accumulation).  FAST: one
// v_mfma_f32_16x16x128_f8f6f4 on the raw bytes (gfx950 FP8 MFMAs truncate
// products far below the block maximum; opt-in).
#include "lcml_internal.hpp"

namespace lcml {
namespace {

#ifndef LCML_SKINNY_NB
#define LCML_SKINNY_NB 4
#endif
#ifndef LCML_SKINNY_WAVES
#define LCML_SKINNY_WAVES 8
#endif
#ifndef LCML_SKINNY_UNROLL
#define LCML_SKINNY_UNROLL 1
#endif

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

struct SkinnyArgs {
    int64_t M, N, K;
    const uint8_t *a;
    int64_t lda;
    const uint8_t *bp;
    int64_t KC;      // k-chunks per panel
    int64_t nblk16;  // 16-column blocks in the packed matrix (Np / 16)
    int nkb;         // K blocks of 128
    Epilogue e;
};

__device__ inline v8i join(u4 lo, u4 hi) {
    v8i r;
    r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
    r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
    return r;
}

template <int NB, int WAVES, int UNROLL, bool EXACT>
__global__ __launch_bounds__(WAVES * 64) void k_gemm_skinny(SkinnyArgs g) {
    constexpr int NT = WAVES * 64;
    __shared__ v4f red[WAVES][NB][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t blk0 = (int64_t)blockIdx.x * NB;  // first 16-column block

    // K range of this wavefront
    const int kb_begin = (int)(((int64_t)g.nkb * wave) / WAVES);
    const int kb_end = (int)(((int64_t)g.nkb * (wave + 1)) / WAVES);

    // activation operand: row lane%16, k offset (lane/16)*32 within a K block
    const int arow = lane & 15;
    const bool a_ok = arow < g.M;
    const uint8_t *a_ptr = g.a + (a_ok ? arow : 0) * g.lda + (lane >> 4) * 32;

    // weight operand addresses for each 16-column block
    const uint8_t *b_ptr[NB];
    bool b_ok[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        int64_t blk = blk0 + j;
        b_ok[j] = blk < g.nblk16;
        int64_t panel = (b_ok[j] ? blk : 0) >> 2, sub = blk & 3;
        b_ptr[j] = g.bp + panel * g.KC * 1024 + (sub * 16 + (lane & 15)) * 16 +
                   (int64_t)((lane >> 4) * 2) * 1024;
    }

    v4f acc[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};

    // Register double buffer: the loads of the next UNROLL K blocks are in
    // flight while the current ones are converted and multiplied.
    struct Frag {
        u4 alo[UNROLL], ahi[UNROLL], blo[UNROLL][NB], bhi[UNROLL][NB];
    };
    auto load = [&](Frag &f, int kb0) {
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const int kb = kb0 + u;
            const bool in = kb < kb_end;
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const uint8_t *p = b_ptr[j] + (int64_t)kb * 8 * 1024;
                bool ok = in && b_ok[j];
                f.blo[u][j] = ok ? __builtin_nontemporal_load(reinterpret_cast<const u4 *>(p)) : u4{0, 0, 0, 0};
                f.bhi[u][j] = ok ? __builtin_nontemporal_load(reinterpret_cast<const u4 *>(p + 1024)) : u4{0, 0, 0, 0};
            }
            const int64_t k = (int64_t)kb * 128 + (lane >> 4) * 32;
            const bool ok_lo = in && a_ok && k < g.K;
            const bool ok_hi = in && a_ok && k + 16 < g.K;
            f.alo[u] = ok_lo ? *reinterpret_cast<const u4 *>(a_ptr + (int64_t)kb * 128) : u4{0, 0, 0, 0};
            f.ahi[u] = ok_hi ? *reinterpret_cast<const u4 *>(a_ptr + (int64_t)kb * 128 + 16) : u4{0, 0, 0, 0};
        }
    };
    auto compute = [&](const Frag &f) {
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            if constexpr (EXACT) {
                const uint32_t aw[8] = {f.alo[u].x, f.alo[u].y, f.alo[u].z, f.alo[u].w,
                                        f.ahi[u].x, f.ahi[u].y, f.ahi[u].z, f.ahi[u].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const bf16x8 a16 = e4m3x8_to_bf16(aw[2 * q], aw[2 * q + 1]);
#pragma unroll
                    for (int j = 0; j < NB; ++j) {
                        const uint32_t bw[8] = {f.blo[u][j].x, f.blo[u][j].y, f.blo[u][j].z, f.blo[u][j].w,
                                                f.bhi[u][j].x, f.bhi[u][j].y, f.bhi[u][j].z, f.bhi[u][j].w};
                        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            a16, e4m3x8_to_bf16(bw[2 * q], bw[2 * q + 1]), acc[j], 0, 0, 0);
                    }
                }
            } else {
                v8i af = join(f.alo[u], f.ahi[u]);
#pragma unroll
                for (int j = 0; j < NB; ++j)
                    acc[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        af, join(f.blo[u][j], f.bhi[u][j]), acc[j], 0, 0, 0, 0, 0, 0);
            }
        }
    };
    Frag f0, f1;
    if (kb_begin < kb_end) load(f0, kb_begin);
    for (int kb0 = kb_begin; kb0 < kb_end; kb0 += 2 * UNROLL) {
        if (kb0 + UNROLL < kb_end) load(f1, kb0 + UNROLL);
        compute(f0);
        if (kb0 + 2 * UNROLL < kb_end) load(f0, kb0 + 2 * UNROLL);
        if (kb0 + UNROLL < kb_end) compute(f1);
    }

#pragma unroll
    for (int j = 0; j < NB; ++j) red[wave][j][lane] = acc[j];
    __syncthreads();

    // 16 x 16*NB outputs: (block j, lane l, register r); MFMA output layout:
    // lane l holds column l%16 and rows (l/16)*4 + r.
    const Epilogue &e = g.e;
    const float a_s = e.a_scale ? e.a_scale[0] : 1.0f;
    for (int o = tid; o < NB * 256; o += NT) {
        const int j = o >> 8, l = o & 63, r = (o >> 6) & 3;
        const int64_t row = (l >> 4) * 4 + r;
        const int64_t col = (blk0 + j) * 16 + (l & 15);
        if (row >= e.M || col >= e.N) continue;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) v += red[w][j][l][r];
        epi_store(e, row, col, epi_value(e, epi_scale(e, a_s, col), row, col, v));
    }
}

}  // namespace

hipError_t launch_gemm_skinny(int64_t M, int64_t N, int64_t K, const uint8_t *a, int64_t lda,
                              const uint8_t *bp, const Epilogue &e, bool exact, hipStream_t s) {
    SkinnyArgs g;
    g.M = M; g.N = N; g.K = K; g.a = a; g.lda = lda; g.bp = bp;
    int64_t Kp = pad_to(K, kPackK), Np = pad_to(N, kPanelCols);
    g.KC = Kp / 16;
    g.nblk16 = Np / 16;
    g.nkb = (int)(Kp / 128);
    g.e = e;
    constexpr int NB = LCML_SKINNY_NB, W = LCML_SKINNY_WAVES, U = LCML_SKINNY_UNROLL;
    unsigned grid = (unsigned)((g.nblk16 + NB - 1) / NB);
    if (exact)
        hipLaunchKernelGGL((k_gemm_skinny<NB, W, U, true>), dim3(grid), dim3(W * 64), 0, s, g);
    else
        hipLaunchKernelGGL((k_gemm_skinny<NB, W, U, false>), dim3(grid), dim3(W * 64), 0, s, g);
    return hipGetLastError();
}

}  // namespace lcml
