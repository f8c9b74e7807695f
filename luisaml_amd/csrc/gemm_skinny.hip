// gemm_skinny.hip -- small- and medium-M FP8 GEMM on gfx950 (decode-shaped
// M <= 16, and any M whose 256x256-tile grid would leave CUs idle).
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
// Larger M: a workgroup takes MB = 2 or 4 row blocks of 16 (each weight
// fragment, converted once, feeds MB MFMAs), and M > 16*MB adds row groups
// of 16*MB rows, i.e. more workgroups per weight panel; those are numbered
// so that the row groups of one panel run on one XCD and share its L2.
// The activation rows are the A operand: lane l holds row l%16,
// k = (l/16)*32+0..31 of each 128-k block; the weight operand: lane l holds
// column l%16 of a 16-column block and the same k range, i.e. two
// consecutive 16-byte chunks of the packed panel.
// EXACT (default): the 32 bytes are widened to bf16 (exact) and fed to four
// v_mfma_f32_16x16x32_bf16 (fp32-accurate accumulation).  FAST: one
// v_mfma_f32_16x16x128_f8f6f4 on the raw bytes (gfx950 FP8 MFMAs truncate
// products far below the block maximum; opt-in).
//
// DYN (fused DynamicQuantizeLinear): the activations arrive as fp32 and are
// quantised inside the kernel.  Every workgroup first starts the loads of
// the first two weight K blocks of each wavefront, then reduces amax =
// max|x| over the whole activation matrix (L2-resident: all workgroups read
// the same M*K floats) and derives the per-tensor scale amax/448 exactly as
// the standalone dynamic quantiser does.  Each wavefront then encodes the
// activations of its own K blocks into LDS (row pitch Kp+16 bytes, so the 16
// rows of a fragment read fall in distinct banks; k >= K is zero), one block
// at a time, right after issuing that block's weight loads: the ~40 VALU
// operations per float4 of the exact encode run while the weights are in
// flight, and only the first block's encode delays the stream.  When a
// wavefront's blocks fit its 4 or 8 activation slots (ONE), the amax pass
// already loads x in the per-block layout and the encode reuses those
// registers, so x is read once.  (Encoding all of x before the main loop cost 1.55 us at
// M=1 and 2.6 us at M=4 over the E4M3-in kernel on the 4096x11008 linear;
// per block with one read of x, 0.6 and 1.0 us.)  The redundant
// per-workgroup amax and encode still cost M*K loads and VALU work in every
// workgroup, so the fused kernel only pays off for small M*K.
#include <algorithm>

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
#ifndef LCML_SKINNY_PF
#define LCML_SKINNY_PF 1
#endif

constexpr uint32_t kOOB = 0x80000000u;  // buffer offset past every extent: loads return zeros
constexpr int kRsrcFlags = 0x00020000;  // raw buffer resource word 3 (as the tiled GEMM uses)
constexpr int kNT = 2;                  // buffer load cache policy: non-temporal (streamed weights)

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

struct SkinnyArgs {
    int64_t M, N, K;
    const uint8_t *a;
    int64_t lda;
    const float *x;     // DYN: fp32 activations [M, K], row stride ldx elements
    int64_t ldx;
    float *scale_out;   // DYN: optional, receives the dynamic scale
    const uint8_t *bp;
    int64_t KC;      // k-chunks per panel
    int64_t nblk16;  // 16-column blocks in the packed matrix (Np / 16)
    int nkb;         // K blocks of 128
    int rg;          // row groups of 16*MB rows (workgroups per column range)
    Epilogue e;
};

__device__ inline v8i join(u4 lo, u4 hi) {
    v8i r;
    r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
    r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
    return r;
}

// the kernel's leading scalar arguments, from the launch description g with
// activations act of row stride ld (elements)
#define LCML_SKINNY_LEAD(g, act, ld)                                                                               \
    (g).bp, static_cast<const void *>(act), (int)(ld), (int)(g).M, (int)(g).K, (int)(g).KC, (g).nkb, (g).rg

typedef float f4 __attribute__((ext_vector_type(4)));

// SB (DYN only): activation slots of 4 floats per lane per K block, at least
// ceil(M/2).  ONE (DYN only; 0, 4 or 8): nonzero when every wavefront's K
// blocks fit ONE slots, so that one round of ONE activation loads serves
// both the amax and the encode (4 where they fit: at M <= 2 and K <= 4096
// the four empty slots of an 8-slot round cost 0.1 us per launch).
// The values that the code before the first weight load reads come as
// leading scalar arguments (bp, the activations a or x with their row
// stride, M, K, the panel's k-chunks, the K blocks, the row groups), and
// this file is compiled with -amdgpu-kernarg-preload-count=8: they arrive
// in SGPRs when the wavefront starts, so the first loads wait for no
// kernel-argument fetch.  The struct's copies of them are not read.  On the
// 4096x11008 linear the preload alone saved 0.05-0.15 us per launch, and
// with the 32-bit prologue below (one weight offset per lane, the blocks'
// pieces as immediate offsets) 0.26-0.39 us.
template <int NB, int MB, int WAVES, int UNROLL, bool EXACT, bool DYN, int SB = 0, int ONE = 0>
__global__ __launch_bounds__(WAVES * 64) void k_gemm_skinny(const uint8_t *bp, const void *src, int ld, int M, int K,
                                                            int kc, int nkb, int rg, SkinnyArgs g) {
    static_assert(!DYN || MB == 1, "the fused quantiser serves M <= 16");
    static_assert(NB == 4, "a workgroup reads one whole 64-column panel");
    static_assert(!DYN || (SB >= 1 && SB <= 8 && LCML_SKINNY_PF == 1 && UNROLL == 1),
                  "the fused quantiser: M <= 2*SB <= 16, one K block per load");
    constexpr int NT = WAVES * 64;
    // the wavefronts' partial tiles, register r of lane l of block j at
    // [w][j][r][l]: the epilogue's lanes read consecutive words (no bank
    // conflicts; a [w][j][l] array of 16-byte partials had 4-way ones)
    __shared__ float red[WAVES][NB][4][64];
    extern __shared__ __attribute__((aligned(16))) uint8_t a_lds[];  // DYN: [M][pitch] E4M3
    // the wavefront index is uniform: readfirstlane lets the compiler keep
    // everything derived from it (the K range, the in-range tests) scalar
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Workgroup -> (column range, row group).  With several row groups the
    // workgroups that read one weight panel should share an L2: workgroup
    // ids go round-robin over the 8 XCDs (id % 8), so ids are regrouped into
    // one contiguous range per XCD, in which the row groups of a panel are
    // consecutive.
    // Every instruction before the first weight load delays the whole
    // stream: with MB = 1 (M <= 16) there is one row group, so the mapping
    // needs no division (a 64-bit one costs ~200 instructions, 0.1-0.25 us
    // per launch on the 4096x11008 linear).
    int blk0, row0;  // first 16-column block, first row
    if constexpr (MB == 1) {
        blk0 = (int)blockIdx.x * NB;
        row0 = 0;
    } else {
        int t = blockIdx.x;
        if (rg > 1) {
            const int nwg = (int)gridDim.x, q = nwg >> 3, r = nwg & 7, x = t & 7;
            t = x * q + (x < r ? x : r) + (t >> 3);
        }
        blk0 = (t / rg) * NB;
        row0 = (t - (t / rg) * rg) * 16 * MB;
    }

    // K range of this wavefront (nkb < 2^24; unsigned, so the division is a shift)
    const int kb_begin = (int)((uint32_t)(nkb * wave) / WAVES);
    const int kb_end = (int)((uint32_t)(nkb * (wave + 1)) / WAVES);

    // Every global load below is a buffer load whose out-of-range lanes and
    // blocks carry an offset past the buffer's extent: the hardware returns
    // zeros for them without touching memory.  So no load sits under a
    // branch, the code from a load to its first use is straight-line, and the
    // compiler's vmcnt waits count exactly the loads issued after it (a load
    // under a branch makes it wait for every outstanding load instead, which
    // would drain the weight prefetch at each use).
    const int arow = lane & 15;  // row within a 16-row block
    bool a_ok[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) a_ok[mb] = row0 + mb * 16 + arow < M;

    // weights: this workgroup's 64-column panel (the grid covers the panels
    // exactly, so its four 16-column blocks all exist).  Lane l reads column
    // l%16 of each block and half l/16 of each k-chunk: block j's two
    // 16-byte pieces of a K block lie at b_lane + j*256 and + 1024 from the
    // K block's first byte.
    const __amdgpu_buffer_rsrc_t b_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(bp + (size_t)(blk0 >> 2) * (size_t)kc * 1024), 0, kc * 1024, kRsrcFlags);
    const uint32_t b_lane = (uint32_t)(lane & 15) * 16u + (uint32_t)(lane >> 4) * 2048u;
    // activations (E4M3, without DYN): row lane%16, k offset (lane/16)*32 of a K block
    const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        DYN ? nullptr : const_cast<void *>(src), 0, DYN ? 0 : (int)((int64_t)(M - 1) * ld + K), kRsrcFlags);
    uint32_t a_row_off[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
        a_row_off[mb] = (uint32_t)(row0 + mb * 16 + arow) * (uint32_t)ld + (uint32_t)(lane >> 4) * 32;

    v4f acc[MB][NB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[mb][j] = v4f{0.f, 0.f, 0.f, 0.f};

    struct Frag {
        u4 alo[UNROLL][MB], ahi[UNROLL][MB], blo[UNROLL][NB], bhi[UNROLL][NB];
    };
    auto load = [&](Frag &f, int kb0) {
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const int kb = kb0 + u;
            const bool in = kb < kb_end;
            // past the range: kOOB plus at most 1792, still past every extent
            const uint32_t o = in ? b_lane + (uint32_t)kb * 8192u : kOOB;
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                f.blo[u][j] = __builtin_amdgcn_raw_buffer_load_b128(b_rsrc, (int)(o + j * 256), 0, kNT);
                f.bhi[u][j] = __builtin_amdgcn_raw_buffer_load_b128(b_rsrc, (int)(o + j * 256 + 1024), 0, kNT);
            }
            if constexpr (!DYN) {
                // the weight loads first: the activations' addresses need
                // more arithmetic, and they come from L2
                __builtin_amdgcn_sched_barrier(0);
                const uint32_t k = (uint32_t)kb * 128 + (uint32_t)(lane >> 4) * 32;  // K < 2^31
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    const uint32_t o = a_row_off[mb] + (uint32_t)kb * 128;
                    const bool ok = in & a_ok[mb];
                    const uint32_t o_lo = (ok & (k < (uint32_t)K)) ? o : kOOB;
                    const uint32_t o_hi = (ok & (k + 16 < (uint32_t)K)) ? o + 16 : kOOB;
                    f.alo[u][mb] = __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, (int)o_lo, 0, 0);
                    f.ahi[u][mb] = __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, (int)o_hi, 0, 0);
                }
            }
        }
    };
    // DYN: activation fragments from the LDS copy (zero-padded to Kp)
    const int64_t pitch = pad_to((int64_t)K, kPackK) + 16;
    auto read_a = [&](Frag &f, int kb0) {
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const int kb = kb0 + u;
            const uint8_t *p = a_lds + (a_ok[0] ? arow : 0) * pitch + (int64_t)kb * 128 + (lane >> 4) * 32;
            const bool ok = a_ok[0] && kb < kb_end;
            f.alo[u][0] = ok ? *reinterpret_cast<const u4 *>(p) : u4{0, 0, 0, 0};
            f.ahi[u][0] = ok ? *reinterpret_cast<const u4 *>(p + 16) : u4{0, 0, 0, 0};
        }
    };
    // blocks past the wavefront's range hold zeros and are skipped (a
    // uniform branch around the MFMAs only)
    auto compute = [&](const Frag &f, int kb0) {
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            if (kb0 + u >= kb_end) continue;
            if constexpr (EXACT) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    bf16x8 a16[MB];
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb) {
                        const u4 lo = f.alo[u][mb], hi = f.ahi[u][mb];
                        a16[mb] = q == 0 ? e4m3x8_to_bf16(lo.x, lo.y)
                                : q == 1 ? e4m3x8_to_bf16(lo.z, lo.w)
                                : q == 2 ? e4m3x8_to_bf16(hi.x, hi.y)
                                         : e4m3x8_to_bf16(hi.z, hi.w);
                    }
#pragma unroll
                    for (int j = 0; j < NB; ++j) {
                        const u4 lo = f.blo[u][j], hi = f.bhi[u][j];
                        const bf16x8 b16 = q == 0 ? e4m3x8_to_bf16(lo.x, lo.y)
                                         : q == 1 ? e4m3x8_to_bf16(lo.z, lo.w)
                                         : q == 2 ? e4m3x8_to_bf16(hi.x, hi.y)
                                                  : e4m3x8_to_bf16(hi.z, hi.w);
#pragma unroll
                        for (int mb = 0; mb < MB; ++mb)
                            acc[mb][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a16[mb], b16, acc[mb][j], 0, 0, 0);
                    }
                }
            } else {
                v8i af[MB];
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) af[mb] = join(f.alo[u][mb], f.ahi[u][mb]);
#pragma unroll
                for (int j = 0; j < NB; ++j) {
                    const v8i bf = join(f.blo[u][j], f.bhi[u][j]);
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb)
                        acc[mb][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af[mb], bf, acc[mb][j], 0, 0,
                                                                                     0, 0, 0, 0);
                }
            }
        }
    };
    // Ring of PF register buffers of UNROLL K blocks: the loads of PF-1
    // buffers are in flight while one is converted and multiplied.  PF = 1
    // measures fastest on the 4096x11008 linear (9.9 us at M = 1 against
    // 10.1 us with PF = 2, 11.3-11.9 us with PF = 3-4; medium M gains too):
    // with 8 wavefronts on every CU streaming, more loads in flight per
    // wavefront only queue longer in the memory system.
    constexpr int PF = LCML_SKINNY_PF;
    Frag fr[PF];
    // DYN: the activations as float4 groups i = r * kq + c (K % 16 == 0); UQ
    // loads per thread are issued together, so one pass costs about one
    // memory round trip per UQ * 512 groups.  The first round is issued ahead
    // of the weight prefetch so that it returns from L2 without queueing
    // behind the HBM loads.
    constexpr int UQ = ONE ? ONE : 8;
    const uint32_t kq = (uint32_t)(K / 4);
    const uint32_t nq = (uint32_t)M * kq;
    const __amdgpu_buffer_rsrc_t x_rsrc =
        __builtin_amdgcn_make_buffer_rsrc(DYN ? const_cast<void *>(src) : nullptr, 0,
                                          DYN ? (int)(((int64_t)(M - 1) * ld + K) * 4) : 0, kRsrcFlags);
    // group i -> (row r, float4 c): i < 2^24, so the float quotient is off
    // by at most one and two compares fix it (no integer division)
    const float inv_kq = 1.0f / (float)kq;
    auto split = [&](uint32_t i, uint32_t &r, uint32_t &c) {
        uint32_t rr = (uint32_t)((float)i * inv_kq);
        int cc = (int)i - (int)(rr * kq);
        if (cc < 0) { --rr; cc += (int)kq; }
        if (cc >= (int)kq) { ++rr; cc -= (int)kq; }
        r = rr; c = (uint32_t)cc;
    };
    auto xq = [&](uint32_t i) {
        uint32_t r, c;
        split(i, r, c);
        const uint32_t o = i < nq ? (r * (uint32_t)ld + c * 4) * 4 : kOOB;
        return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, (int)o, 0, 0));
    };
    // DYN: the activations of one K block for the per-block encode: lane l,
    // slot s holds row 2s + l/32, float4 column l%32 of the block (rows past
    // M and columns past K load zeros)
    f4 xb0[DYN ? SB : 1], xb1[DYN ? SB : 1];
    auto xload_block = [&](f4 *xb, int kb) {
        const bool in = kb < kb_end;
#pragma unroll
        for (int sl = 0; sl < SB; ++sl) {
            const uint32_t r = 2 * sl + (lane >> 5), c = (uint32_t)kb * 32 + (lane & 31);
            const bool ok = in & (r < (uint32_t)M) & (c < kq);
            const uint32_t o = ok ? (r * (uint32_t)ld + c * 4) * 4 : kOOB;
            xb[sl] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, (int)o, 0, 0));
        }
    };
    f4 v[UQ];
    static_assert(!ONE || (DYN && (ONE == 4 || ONE == 8) && UQ % SB == 0), "one round: whole blocks of slots");
    if constexpr (ONE) {
        // slot u holds slot u%SB of block kb_begin + u/SB (the per-block
        // layout above): the amax reads these registers, and the encode
        // takes them block by block, with no second load of x (-0.5 us at
        // M=1, -0.75 us at M=4 on the 4096x11008 linear)
#pragma unroll
        for (int u = 0; u < UQ; ++u) {
            const int kb = kb_begin + u / SB, sl = u % SB;
            const uint32_t r = 2 * sl + (lane >> 5), c = (uint32_t)kb * 32 + (lane & 31);
            const bool ok = (kb < kb_end) & (r < (uint32_t)M) & (c < kq);
            const uint32_t o = ok ? (r * (uint32_t)ld + c * 4) * 4 : kOOB;
            v[u] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, (int)o, 0, 0));
        }
        __builtin_amdgcn_sched_barrier(0);
    } else if constexpr (DYN) {
#pragma unroll
        for (int u = 0; u < UQ; ++u) v[u] = xq(u * NT + tid);
        xload_block(xb0, kb_begin);
        xload_block(xb1, kb_begin + 1);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int p = 0; p < PF; ++p) {
        load(fr[p], kb_begin + p * UNROLL);
        __builtin_amdgcn_sched_barrier(0);
    }
    // MB = 1: the epilogue's weight scales (thread t writes outputs t + i*NT),
    // read while the weight stream runs, as buffer loads outside any branch
    // (a load under a branch would make the first K block's wait drain them
    // too); a missing scale reads 0 and is replaced by 1
    constexpr int EPO = (NB * 256 + NT - 1) / NT;
    float bsc[EPO];
    if constexpr (MB == 1) {
        const __amdgpu_buffer_rsrc_t s_rsrc = __builtin_amdgcn_make_buffer_rsrc(
            (void *)g.e.b_scale, 0, g.e.b_scale ? (int)((g.e.b_per_channel ? g.e.N : 1) * 4) : 0, kRsrcFlags);
#pragma unroll
        for (int i = 0; i < EPO; ++i) {
            const int o = tid + i * NT, j = o >> 8, l = o & 63;
            const int64_t col = (blk0 + (j < NB ? j : 0)) * 16 + (l & 15);
            const uint32_t so = g.e.b_per_channel ? (col < g.e.N ? (uint32_t)col * 4 : kOOB) : 0u;
            bsc[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(s_rsrc, (int)so, 0, 0));
        }
        if (!g.e.b_scale) {
#pragma unroll
            for (int i = 0; i < EPO; ++i) bsc[i] = 1.0f;
        }
    }
    // DYN: a second K block in flight while the scale is computed (issued
    // after the scale prefetch: before it, 0.1 us slower at M = 1 and 4)
    Frag fx;
    if constexpr (DYN) {
        load(fx, kb_begin + 1);
        __builtin_amdgcn_sched_barrier(0);
    }
    float a_dyn = 1.0f;
    Recip d{1.0f, 1.0f, true};
    int enc_mode = 2;
    if constexpr (DYN) {
        __shared__ float wmax[WAVES];
        __shared__ uint32_t wbad[WAVES];
        float m = 0.0f;
        float nf = 0.0f;  // x * 0 summed: NaN once any x is NaN or +-inf
        for (uint32_t base = 0; base < (ONE ? 1u : nq); base += NT * UQ) {
            if (base) {
#pragma unroll
                for (int u = 0; u < UQ; ++u) v[u] = xq(base + u * NT + tid);
            }
            // ONE: the slots past this wavefront's blocks hold zeros
            const int nslot = ONE ? (kb_end - kb_begin) * SB : UQ;
#pragma unroll
            for (int u = 0; u < UQ; ++u) {
                if (u >= nslot) break;
                // zeros past the end; NaN compares false and is skipped, as
                // in the standalone amax
                const float ax = fabsf(v[u].x), ay = fabsf(v[u].y), az = fabsf(v[u].z), aw = fabsf(v[u].w);
                m = ax > m ? ax : m; m = ay > m ? ay : m; m = az > m ? az : m; m = aw > m ? aw : m;
                nf = fmaf(v[u].x, 0.0f, nf); nf = fmaf(v[u].y, 0.0f, nf);
                nf = fmaf(v[u].z, 0.0f, nf); nf = fmaf(v[u].w, 0.0f, nf);
            }
        }
        // by DPP within rows and readlane across them (on the critical path:
        // a __shfl_xor ladder here cost 0.1-0.25 us per launch)
        m = wave_max(m);
        const bool wave_bad = __builtin_amdgcn_ballot_w64(nf != nf) != 0;
        if (lane == 0) {
            wmax[wave] = m;
            wbad[wave] = wave_bad ? 1u : 0u;
        }
        __syncthreads();
        m = wmax[0];
        uint32_t bad = wbad[0];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) {
            m = wmax[w] > m ? wmax[w] : m;
            bad |= wbad[w];
        }
        a_dyn = scale_from_amax_bits(f32_bits(m));
        if (g.scale_out && blockIdx.x == 0 && tid == 0) *g.scale_out = a_dyn;
        d = make_recip(a_dyn);
        // the scale's range test and the NaN/inf test are uniform (mode 2:
        // fast scale and clean input, 1: fast scale, 0: IEEE division)
        enc_mode = d.fast ? (bad ? 1 : 2) : 0;
    }
    // DYN: block kb's codes into this wavefront's own columns of the LDS
    // copy (rows below M; columns past K get the zeros x holds there).  Only
    // this wavefront reads them, and a wavefront's LDS accesses take effect
    // in order, so no barrier is needed.
    auto encode_block = [&](const f4 *xb, int kb) {
        if (kb >= kb_end) return;
        auto run = [&](auto mode) {
#pragma unroll
            for (int sl = 0; sl < SB; ++sl) {
                const uint32_t r = 2 * sl + (lane >> 5), c = (uint32_t)kb * 32 + (lane & 31);
                if (r < (uint32_t)M) {
                    const f4 x4 = xb[sl];
                    uint32_t code;
                    if constexpr (decltype(mode)::value == 2)
                        code = quantize4_clean(x4.x, x4.y, x4.z, x4.w, d);
                    else
                        code = quantize4_t<decltype(mode)::value == 1>(x4.x, x4.y, x4.z, x4.w, d);
                    reinterpret_cast<uint32_t *>(a_lds + r * pitch)[c] = code;
                }
            }
        };
        if (enc_mode == 2)
            run(std::integral_constant<int, 2>{});
        else if (enc_mode == 1)
            run(std::integral_constant<int, 1>{});
        else
            run(std::integral_constant<int, 0>{});
    };
    if constexpr (ONE) {
        // the next block's activations are always v[0..SB-1]: after its
        // encode the slots move down by SB
        auto encode_v = [&](int kb) {
            if (kb >= kb_end) return;
            encode_block(v, kb);
#pragma unroll
            for (int u = 0; u + SB < UQ; ++u) v[u] = v[u + SB];
        };
        encode_v(kb_begin);
        read_a(fr[0], kb_begin);
        compute(fr[0], kb_begin);
        __builtin_amdgcn_sched_barrier(0);
        load(fr[0], kb_begin + 2);
        __builtin_amdgcn_sched_barrier(0);
        encode_v(kb_begin + 1);
        read_a(fx, kb_begin + 1);
        compute(fx, kb_begin + 1);
        __builtin_amdgcn_sched_barrier(0);
        encode_v(kb_begin + 2);
        for (int kb = kb_begin + 2; kb < kb_end; ++kb) {
            read_a(fr[0], kb);
            compute(fr[0], kb);
            __builtin_amdgcn_sched_barrier(0);
            load(fr[0], kb + 1);
            __builtin_amdgcn_sched_barrier(0);
            encode_v(kb + 1);
        }
    } else if constexpr (DYN) {
        // blocks 0 and 1 are in flight; each later block's activations are
        // loaded with its weights and encoded while those are in flight
        encode_block(xb0, kb_begin);
        read_a(fr[0], kb_begin);
        compute(fr[0], kb_begin);
        __builtin_amdgcn_sched_barrier(0);
        xload_block(xb0, kb_begin + 2);
        load(fr[0], kb_begin + 2);
        __builtin_amdgcn_sched_barrier(0);
        encode_block(xb1, kb_begin + 1);
        read_a(fx, kb_begin + 1);
        compute(fx, kb_begin + 1);
        __builtin_amdgcn_sched_barrier(0);
        encode_block(xb0, kb_begin + 2);
        for (int kb = kb_begin + 2; kb < kb_end; ++kb) {
            read_a(fr[0], kb);
            compute(fr[0], kb);
            __builtin_amdgcn_sched_barrier(0);
            xload_block(xb0, kb + 1);
            load(fr[0], kb + 1);
            __builtin_amdgcn_sched_barrier(0);
            encode_block(xb0, kb + 1);
        }
    } else {
        // consume buffer p (blocks kb), refill it with the blocks PF*UNROLL
        // ahead (past the end: zeros, no memory traffic).  The scheduling
        // barriers keep each buffer's loads together and in ring order, so
        // the wait before a buffer's first use leaves the other PF-1
        // buffers' loads in flight.
        for (int kb0 = kb_begin; kb0 < kb_end; kb0 += PF * UNROLL) {
#pragma unroll
            for (int p = 0; p < PF; ++p) {
                const int kb = kb0 + p * UNROLL;
                compute(fr[p], kb);
                __builtin_amdgcn_sched_barrier(0);
                load(fr[p], kb + PF * UNROLL);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }

    // 16 x 16*NB outputs per row block: (block j, lane l, register r); MFMA
    // output layout: lane l holds column l%16 and rows (l/16)*4 + r.  Row
    // blocks go through the one LDS reduction buffer in turn.
    const Epilogue &e = g.e;
    const float a_s = DYN ? a_dyn : (e.a_scale ? e.a_scale[0] : 1.0f);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        if (mb) __syncthreads();  // the previous block's sums are read
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[wave][j][r][lane] = acc[mb][j][r];
        __syncthreads();
        if constexpr (MB == 1) {
            // Without C, alpha or an activation (a uniform test) the value is
            // epi_value's first product, and a short path of its own leads to
            // the stores: the generic one's broadcast and activation code
            // between the reduction and the stores cost 0.05-0.2 us per
            // launch on the 4096x11008 linear.
            const bool plain = !e.c && e.alpha == 1.0f && e.act == ACT_NONE;
            auto out = [&](auto pl) {
#pragma unroll
                for (int i = 0; i < EPO; ++i) {
                    const int o = tid + i * NT;
                    const int j = o >> 8, l = o & 63, r = (o >> 6) & 3;
                    const int64_t row = row0 + (l >> 4) * 4 + r;
                    const int64_t col = (blk0 + j) * 16 + (l & 15);
                    if (o >= NB * 256 || row >= e.M || col >= e.N) continue;
                    float v = 0.0f;
#pragma unroll
                    for (int w = 0; w < WAVES; ++w) v += red[w][j][r][l];
                    if constexpr (decltype(pl)::value)
                        epi_store(e, row, col, v * (a_s * bsc[i]));
                    else
                        epi_store(e, row, col, epi_value(e, a_s * bsc[i], row, col, v));
                }
            };
            if (__builtin_expect(plain, 1))  // the short path right after the reduction's barrier
                out(std::true_type{});
            else
                out(std::false_type{});
        } else {
            for (int o = tid; o < NB * 256; o += NT) {
                const int j = o >> 8, l = o & 63, r = (o >> 6) & 3;
                const int64_t row = row0 + mb * 16 + (l >> 4) * 4 + r;
                const int64_t col = (blk0 + j) * 16 + (l & 15);
                if (row >= e.M || col >= e.N) continue;
                float v = 0.0f;
#pragma unroll
                for (int w = 0; w < WAVES; ++w) v += red[w][j][r][l];
                epi_store(e, row, col, epi_value(e, epi_scale(e, a_s, col), row, col, v));
            }
        }
    }
}

}  // namespace

// Row blocks per workgroup.  A workgroup with MB = 4 holds 152-164 VGPRs,
// so one runs per CU; with MB = 2 (99-119 VGPRs) two share a CU.  Measured
// on the 4096x11008 and 11008x4096 linears, in units of one MB = 4
// workgroup's time T (19 us at K = 4096, 38 us at K = 11008): r rounds of
// up to 256 MB = 4 workgroups take 0.2 + 0.8 r; MB = 2 workgroups, n per CU
// at most, take 0.33 + 0.38 n.  So MB = 2 wins where it fills CUs that
// MB = 4 leaves idle (11008x4096 at M = 128: 26 us against 37 us), MB = 4
// where both fill the chip (4096x11008 at M = 64: 19 us against 22 us).
// With two MB = 2 workgroups per CU, the weight panels resident on one XCD
// at a time must also fit its 4 MB L2, or the row groups of a panel re-read
// it from memory (28672x8192 at M = 128: 16 panels of 512 KB per XCD, 133 us
// against 114 us with MB = 4): then MB = 4.
int skinny_row_blocks(int64_t M, int64_t N, int64_t K, double *cost) {
    const int64_t panels = (N + 63) / 64;
    auto rounds = [&](int64_t rows) { return (double)((panels * ((M + rows - 1) / rows) + 255) / 256); };
    int mb;
    double c;
    if (M <= 16) {
        mb = 1;
        c = 0.55 * rounds(16);
    } else {
        const double n = rounds(32), c2 = 0.33 + 0.38 * n, c4 = 0.2 + 0.8 * rounds(64);
        const double rg2 = (double)((M + 31) / 32);
        const double per_xcd = std::min((double)panels * rg2, 512.0) / 8;  // resident MB = 2 workgroups
        const bool l2_fits = per_xcd / rg2 * (double)pad_to(K, kPackK) * 64 <= 4.0 * 1024 * 1024;
        mb = M <= 32 || (c2 <= c4 && (n < 2 || l2_fits)) ? 2 : 4;
        c = mb == 2 ? c2 : c4;
    }
    if (cost) *cost = c;
    return mb;
}

hipError_t launch_gemm_skinny(int64_t M, int64_t N, int64_t K, const uint8_t *a, int64_t lda,
                              const uint8_t *bp, const Epilogue &e, bool exact, hipStream_t s) {
    // 32-bit buffer extents and kernel arguments (the C ABI checks the same)
    if ((M - 1) * lda + K >= ((int64_t)1 << 31) || pad_to(K, kPackK) * 64 >= ((int64_t)1 << 31))
        return hipErrorInvalidValue;
    SkinnyArgs g;
    g.M = M; g.N = N; g.K = K; g.a = a; g.lda = lda; g.bp = bp;
    int64_t Kp = pad_to(K, kPackK), Np = pad_to(N, kPanelCols);
    g.KC = Kp / 16;
    g.nblk16 = Np / 16;
    g.nkb = (int)(Kp / 128);
    g.e = e;
    g.x = nullptr; g.ldx = 0; g.scale_out = nullptr;
    constexpr int NB = LCML_SKINNY_NB, W = LCML_SKINNY_WAVES, U = LCML_SKINNY_UNROLL;
    // row blocks of 16 per workgroup (every weight fragment feeds MB MFMAs),
    // and row groups of 16*MB rows beyond that
    const int mb = skinny_row_blocks(M, N, K, nullptr);
    g.rg = (int)((M + 16 * mb - 1) / (16 * mb));
    const unsigned grid = (unsigned)((g.nblk16 + NB - 1) / NB * g.rg);
#define LCML_SKINNY_LAUNCH(MBV)                                                                                  \
    if (exact)                                                                                                 \
        hipLaunchKernelGGL((k_gemm_skinny<NB, MBV, W, U, true, false>), dim3(grid), dim3(W * 64), 0, s,          \
                           LCML_SKINNY_LEAD(g, g.a, g.lda), g);                                                 \
    else                                                                                                       \
        hipLaunchKernelGGL((k_gemm_skinny<NB, MBV, W, U, false, false>), dim3(grid), dim3(W * 64), 0, s,         \
                           LCML_SKINNY_LEAD(g, g.a, g.lda), g)
    if (mb == 1) {
        LCML_SKINNY_LAUNCH(1);
    } else if (mb == 2) {
        LCML_SKINNY_LAUNCH(2);
    } else {
        LCML_SKINNY_LAUNCH(4);
    }
#undef LCML_SKINNY_LAUNCH
    return hipGetLastError();
}

int64_t skinny_dynamic_lds_bytes(int64_t M, int64_t K) { return M * (pad_to(K, kPackK) + 16); }

hipError_t launch_gemm_skinny_dynamic(int64_t M, int64_t N, int64_t K, const float *x, int64_t ldx,
                                      const uint8_t *bp, const Epilogue &e, float *scale_out, bool exact,
                                      hipStream_t s) {
    // 32-bit buffer extents and kernel arguments (the C ABI checks the same)
    if (((M - 1) * ldx + K) * 4 >= ((int64_t)1 << 31) || pad_to(K, kPackK) * 64 >= ((int64_t)1 << 31))
        return hipErrorInvalidValue;
    SkinnyArgs g;
    g.M = M; g.N = N; g.K = K; g.a = nullptr; g.lda = 0; g.bp = bp;
    g.x = x; g.ldx = ldx; g.scale_out = scale_out;
    int64_t Kp = pad_to(K, kPackK), Np = pad_to(N, kPanelCols);
    g.KC = Kp / 16;
    g.nblk16 = Np / 16;
    g.nkb = (int)(Kp / 128);
    g.rg = 1;
    g.e = e;
    constexpr int NB = LCML_SKINNY_NB, W = LCML_SKINNY_WAVES, U = LCML_SKINNY_UNROLL;
    const unsigned grid = (unsigned)((g.nblk16 + NB - 1) / NB);
    const unsigned lds = (unsigned)skinny_dynamic_lds_bytes(M, K);
    // activation slots per lane per K block: ceil(M/2), rounded up to 1, 2,
    // 4, 8; one round of 4 or 8 activation loads when a wavefront's K blocks
    // (at most ceil(nkb / W)) take at most that many slots
    auto run_one = [&](auto sb, auto one) -> hipError_t {
        constexpr int SB = decltype(sb)::value;
        constexpr int ONE = decltype(one)::value;
        const void *fn = exact ? reinterpret_cast<const void *>(k_gemm_skinny<NB, 1, W, U, true, true, SB, ONE>)
                               : reinterpret_cast<const void *>(k_gemm_skinny<NB, 1, W, U, false, true, SB, ONE>);
        static std::atomic<uint64_t> lds_set[2];
        if (hipError_t err = ensure_dynamic_lds(fn, (int)kSkinnyDynLdsMax, lds_set[exact]); err != hipSuccess)
            return err;
        if (exact)
            hipLaunchKernelGGL((k_gemm_skinny<NB, 1, W, U, true, true, SB, ONE>), dim3(grid), dim3(W * 64), lds, s,
                               LCML_SKINNY_LEAD(g, g.x, g.ldx), g);
        else
            hipLaunchKernelGGL((k_gemm_skinny<NB, 1, W, U, false, true, SB, ONE>), dim3(grid), dim3(W * 64), lds, s,
                               LCML_SKINNY_LEAD(g, g.x, g.ldx), g);
        return hipGetLastError();
    };
    auto run = [&](auto sb) -> hipError_t {
        constexpr int SB = decltype(sb)::value;
        const int slots = ((g.nkb + W - 1) / W) * SB;
        if constexpr (SB <= 4)
            if (slots <= 4) return run_one(sb, std::integral_constant<int, 4>{});
        if (slots <= 8) return run_one(sb, std::integral_constant<int, 8>{});
        return run_one(sb, std::integral_constant<int, 0>{});
    };
    if (M <= 2) return run(std::integral_constant<int, 1>{});
    if (M <= 4) return run(std::integral_constant<int, 2>{});
    if (M <= 8) return run(std::integral_constant<int, 4>{});
    return run(std::integral_constant<int, 8>{});
}

}  // namespace lcml
