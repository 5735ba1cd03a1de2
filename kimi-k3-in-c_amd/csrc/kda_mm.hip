// SPDX-License-Identifier: Apache-2.0
// kda_mm.hip - the layer's projections as hand-written gfx950 MFMA GEMMs.
//
// Replaces the reference's per-token k3_mmw calls (include/k3/k3.h:290-296 ->
// k3_matmul_bf16, src/core/k3_ops.c:1122-1227; call sites :879-886, :946, :948) for a
// T-token prefill: every projection of a token is a row of one GEMM over all T tokens,
//   C[M][N] = A[M][K] . B[N][K]^T      A = activations, B = the weight as stored (row n of
//                                      the reference's [out][in] matrix), both K-contiguous
// with bf16 or fp16 operands and fp32 accumulation.
//
// Two kernels share the workgroup tile (256 x 256, four waves in a 2 x 2 grid, a 128 x 128
// block per wave, one wave per SIMD), the tile order and the persistent grid:
//  * mm16_kernel (whole tiles, one K-range, fp32 or fp16 output: every layer projection but
//    the split-K f_a / b): v_mfma_f32_16x16x32 with the accumulators tied to their AGPRs;
//    K in stages of 32 brought into LDS by direct-to-LDS buffer loads, four stages rotating,
//    each loaded three stages before it is read (its own description below);
//  * mm_kernel (the general form: partial tiles, split-K partial planes, bf16 outputs): each
//    wave's block is 4 x 4 v_mfma_f32_32x32x16 tiles (256 accumulator registers). Per K-step
//    of 64 the workgroup stages A[256][64] and B[256][64] (64 KiB) in LDS, double buffered
//    (128 KiB): each thread loads its 16-byte pieces of step ks+2 into registers while step
//    ks computes and writes them to the other LDS buffer during step ks+1. One barrier per
//    step, placed before the step's last 16-wide substep so the first fragments of the next
//    step load under that substep's MFMAs. Fragment reads are 16 bytes per lane; rows are 128
//    bytes and the 16-byte chunk index is XORed with (row & 7) ^ ((row >> 3) & 1), which keeps
//    every 16-lane group of a fragment read on distinct banks (no LDS bank conflicts,
//    counter-verified). Global loads are buffer loads: a thread's 16 pieces differ only by
//    wave-uniform offsets, so one per-lane offset register per operand addresses all of them,
//    and every LDS offset is one per-lane base plus an immediate; the loop body stays at ~150
//    VGPRs. Each substep is 16 MFMA slots in a fixed order (sched_barrier between slots), each
//    slot also carrying one fragment read or one LDS write + global load, and the same
//    branch-free body runs every K-step (the last steps reload clamped copies that nothing
//    reads).
//
// Tile order is XCD-aware: workgroup b runs on XCD b % 8, and consecutive tile ids (groups
// of 8 M-tiles walked along N) are given to the same XCD, so the tiles running together on
// one XCD share A rows and B rows through that XCD's L2. Shapes with more tiles than compute
// units run on a persistent grid of one workgroup per CU that walks the tiles in rounds; the
// next tile's first K-step is requested before the current tile's fp32 output stores
// (8192 x 4096 x 256: 38.5 against 40.3 us; the 4096-deep shapes gain under 1%).
//
// Split-K: for shapes with fewer tiles than compute units (the narrow f_a / b projection),
// S workgroups per tile each take K/S and write fp32 partial planes P[s][M][N]; the consumer
// adds them in increasing s, so results are bit-reproducible.
#include "kda_internal.h"

#include <algorithm>
#include <type_traits>

namespace k3kda {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 256, BN = 256, BK = 64, NT = 256;
constexpr int WM = 128, WN = 128, TI = WM / 32, TJ = WN / 32;
constexpr int A_BYTES = BM * BK * 2, STAGE = (BM + BN) * BK * 2;
constexpr int NL = (BM + BN) * (BK / 8) / NT;   // 16-byte pieces per thread per K-step
constexpr int S = BK / 16;                       // 16-wide substeps per K-step
constexpr int LDS_BYTES = 2 * STAGE;

enum { OUT_F32 = 0, OUT_F16 = 1, OUT_BF16 = 2, OUT_PART = 3 };

__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

template <int AB>
__device__ __forceinline__ f32x16 mfma(const u32x4 &a, const u32x4 &b, f32x16 c)
{
    if constexpr (AB == K3_DT_F16)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                      0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                       0, 0, 0);
}

// Tile (tm, tn) and K-split s of workgroup b, XCD-aware grouped order.
__device__ __forceinline__ void tile_of(int b, int nb, int tiles_m, int tiles_n, int splits, int &tm, int &tn, int &s)
{
    const int per = nb / 8, rem = nb % 8, x = b % 8, i = b / 8;
    const int L = x * per + (x < rem ? x : rem) + i;
    s = L % splits;
    const int t = L / splits;
    constexpr int GM = 8;
    const int per_group = GM * tiles_n;
    const int g = t / per_group, first_m = g * GM;
    const int gsz = tiles_m - first_m < GM ? tiles_m - first_m : GM;
    tm = first_m + (t % per_group) % gsz;
    tn = (t % per_group) / gsz;
}

// Persistent form: workgroup b of a grid of nb (a multiple of 8) takes, in round r, logical
// tile chunk_start(x) + b / 8 + r * nb / 8 of XCD x = b % 8's contiguous chunk of the tile
// sequence, so the nb / 8 workgroups of one XCD work on consecutive tiles (grouped 8 M-tiles
// along N) at any time. Returns false when the workgroup has no tile in that round.
__device__ __forceinline__ bool ptile_of(int b, int nb, int r, int total, int tiles_m, int tiles_n, int &tm, int &tn)
{
    const int per = total / 8, rem = total % 8, x = b % 8;
    const int size = per + (x < rem ? 1 : 0), i = b / 8 + r * (nb / 8);
    if (i >= size) return false;
    const int t = x * per + (x < rem ? x : rem) + i;
    constexpr int GM = 8;
    const int per_group = GM * tiles_n;
    const int g = t / per_group, first_m = g * GM;
    const int gsz = tiles_m - first_m < GM ? tiles_m - first_m : GM;
    tm = first_m + (t % per_group) % gsz;
    tn = (t % per_group) / gsz;
    return true;
}

// EDGE: M or N below one tile (or leading dimensions beyond 32-bit buffer offsets), rows
// past M / N clamped to the last one in every load (the general form). Otherwise a last
// partial tile is moved back to end at M (or N): the rows it shares with the tile before
// are computed again, with the same bits, and every load of a thread is a wave-uniform
// base plus one fixed per-lane offset.
// PERS: a persistent grid (one workgroup per CU) walks the tiles in rounds (ptile_of). The
// next tile's first K-step is requested before the current tile's output stores, so its load
// latency hides behind them, and the pipeline restarts without a launch per tile.
template <int AB, int OUT, bool EDGE, bool PERS>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(1, 1))) void mm_kernel(
    int M, int N, int K, const uint16_t *__restrict__ A, long lda, const uint16_t *__restrict__ B, long ldb,
    void *__restrict__ Cv, long ldc, int gcols, long gstride, int tiles_m, int tiles_n, int splits)
{
    static_assert(!(PERS && EDGE), "the persistent form needs whole tiles");
    extern __shared__ __attribute__((aligned(1024))) char smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    int tm, tn, sp = 0;
    if constexpr (PERS) {
        if (!ptile_of(blockIdx.x, gridDim.x, 0, tiles_m * tiles_n, tiles_m, tiles_n, tm, tn)) return;
    } else {
        tile_of(blockIdx.x, gridDim.x, tiles_m, tiles_n, splits, tm, tn, sp);
    }
    int m0 = tm * BM, n0 = tn * BN;
    if constexpr (!EDGE) {
        m0 = min(m0, M - BM);
        n0 = min(n0, N - BN);
    }
    const int nks = K / BK / splits, k_first = sp * nks * BK;

    // this thread's 16-byte pieces of a K-step: piece i is row 32 i + prow of the stage's
    // A rows (0-255) then B rows (256-511), 16-byte chunk pc; in LDS at wo + 4096 i (the
    // swizzle of row 32 i + prow equals that of prow)
    const int prow = tid >> 3, pc = tid & 7;
    const int va = (prow * (int)lda + pc * 8) * 2, vb = (prow * (int)ldb + pc * 8) * 2;
    auto rsrc = [&](const uint16_t *base) {
        return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, 0x7fffffff, 0x00020000);
    };
    __amdgpu_buffer_rsrc_t rA = rsrc(A + (long)m0 * lda + k_first), rB = rsrc(B + (long)n0 * ldb + k_first);
    auto gload = [&](int i, int ks) -> u32x4 {
        if constexpr (EDGE) {
            const int row = i * 32 + prow;
            const uint16_t *p = row < BM ? A + (long)min(m0 + row, M - 1) * lda
                                         : B + (long)min(n0 + row - BM, N - 1) * ldb;
            return *reinterpret_cast<const u32x4 *>(p + k_first + ks * BK + pc * 8);
        } else if (i < NL / 2) {
            return __builtin_amdgcn_raw_buffer_load_b128(rA, va, i * 64 * (int)lda + ks * BK * 2, 0);
        } else {
            return __builtin_amdgcn_raw_buffer_load_b128(rB, vb, (i - NL / 2) * 64 * (int)ldb + ks * BK * 2, 0);
        }
    };
    const uint32_t wo = prow * 128 + ((pc ^ swz(prow)) << 4);

    // fragment reads: lane row r32 of a 32-row tile, 16-byte chunk 2 s + kh in substep s;
    // ra / rb hold the per-lane offset of each substep in stage 0, the tile adds 4096 i
    const int r32 = lane & 31, kh = lane >> 5, sw = swz(r32);
    uint32_t ra[S], rb[S];
#pragma unroll
    for (int s = 0; s < S; s++) {
        const uint32_t x = r32 * 128 + (((2 * s + kh) ^ sw) << 4);
        ra[s] = x + wm * WM * 128;
        rb[s] = x + A_BYTES + wn * WN * 128;
    }
    auto lds16 = [&](uint32_t off) { return *reinterpret_cast<const u32x4 *>(smem + off); };

    u32x4 stg[NL];
    // prologue: step 0 into LDS stage 0, step 1 (or step 0 again) into registers
#pragma unroll
    for (int i = 0; i < NL; i++) stg[i] = gload(i, 0);
#pragma unroll
    for (int i = 0; i < NL; i++) *reinterpret_cast<u32x4 *>(smem + wo + 4096 * i) = stg[i];
#pragma unroll
    for (int i = 0; i < NL; i++) stg[i] = gload(i, min(1, nks - 1));
    __syncthreads();

    for (int round = 1;; round++) {
        f32x16 acc[TI][TJ];
#pragma unroll
        for (int i = 0; i < TI; i++)
#pragma unroll
            for (int j = 0; j < TJ; j++) acc[i][j] = f32x16{};
        u32x4 a[2][TI], b[2][TJ];
#pragma unroll
        for (int i = 0; i < TI; i++) a[0][i] = lds16(ra[0] + 4096 * i);
#pragma unroll
        for (int j = 0; j < TJ; j++) b[0][j] = lds16(rb[0] + 4096 * j);

        // K-step ks from LDS stage ks & 1. Each substep is 16 MFMA slots in a fixed order:
        // slots 0-7 also read one fragment of the next substep (in the order the next
        // substep's MFMAs use them), slots 8-13 write one piece of step ks+1 (held in
        // registers) to the other stage and load step ks+2 in its place. The barrier that
        // publishes step ks+1 opens the last substep, whose slots read step ks+1's first
        // fragments. The last steps load and store clamped copies that nothing reads, so
        // every step runs the same branch-free code.
        for (int ks = 0; ks < nks; ks++) {
            const uint32_t so = (ks & 1) * STAGE, wbase = (so ^ STAGE) + wo;
            const int kl = min(ks + 2, nks - 1);
#pragma unroll
            for (int s = 0; s < S; s++) {
                const int cur = s & 1, nx = cur ^ 1;
                constexpr int W0[4] = {0, 6, 11, 16};
                const int wb = s < 3 ? W0[s] : NL, we = s < 3 ? W0[s + 1] : NL;
                const uint32_t rso = s + 1 < S ? so : so ^ STAGE;
                const uint32_t xa = ra[(s + 1) % S] + rso, xb = rb[(s + 1) % S] + rso;
                if (s + 1 == S) __syncthreads();
#pragma unroll
                for (int q = 0; q < TI * TJ; q++) {
                    const int i = q / TJ, j = q % TJ;
                    acc[i][j] = mfma<AB>(a[cur][i], b[cur][j], acc[i][j]);
                    if (q < TI + TJ) {
                        // read order a0 b0 b1 b2 b3 a1 a2 a3
                        if (q == 0) a[nx][0] = lds16(xa);
                        else if (q <= TJ) b[nx][q - 1] = lds16(xb + 4096 * (q - 1));
                        else a[nx][q - TJ] = lds16(xa + 4096 * (q - TJ));
                    }
                    if (q >= TI + TJ && wb + q - (TI + TJ) < we) {
                        const int w = wb + q - (TI + TJ);
                        *reinterpret_cast<u32x4 *>(smem + wbase + 4096 * w) = stg[w];
                        // the reload may not move above the write: stg[w] keeps its registers
                        __builtin_amdgcn_sched_barrier(0);
                        stg[w] = gload(w, kl);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }

        // persistent: the next tile's first K-step goes out before this tile's fp32 stores (a
        // narrower output converts in registers that the prefetch would take: it loads after)
        constexpr bool EARLY = OUT == OUT_F32 || OUT == OUT_PART;
        bool more = false;
        int m1 = m0, n1 = n0;
        if constexpr (PERS) {
            int tm1, tn1;
            more = ptile_of(blockIdx.x, gridDim.x, round, tiles_m * tiles_n, tiles_m, tiles_n, tm1, tn1);
            if (more) {
                m1 = min(tm1 * BM, M - BM);
                n1 = min(tn1 * BN, N - BN);
                rA = rsrc(A + (long)m1 * lda);
                rB = rsrc(B + (long)n1 * ldb);
                if constexpr (EARLY) {
#pragma unroll
                    for (int i = 0; i < NL; i++) stg[i] = gload(i, 0);
                }
            }
        }

        // epilogue: lane holds column r32 of each 32 x 32 tile, rows (r & 3) + 8 (r >> 2) + 4 kh
#pragma unroll
        for (int i = 0; i < TI; i++)
#pragma unroll
            for (int j = 0; j < TJ; j++) {
                const int col = n0 + wn * WN + j * 32 + r32;
                if (col >= N) continue;
                // column groups: columns [g*gcols, (g+1)*gcols) go to the matrix at C + g*gstride
                const int g = col / gcols;
                const long cbase = g * gstride + (col - g * gcols);
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = m0 + wm * WM + i * 32 + (r & 3) + 8 * (r >> 2) + 4 * kh;
                    if (row >= M) continue;
                    const float v = acc[i][j][r];
                    if constexpr (OUT == OUT_F32) {
                        reinterpret_cast<float *>(Cv)[(long)row * ldc + cbase] = v;
                    } else if constexpr (OUT == OUT_F16) {
                        reinterpret_cast<_Float16 *>(Cv)[(long)row * ldc + cbase] = (_Float16)v;
                    } else if constexpr (OUT == OUT_BF16) {
                        reinterpret_cast<uint16_t *>(Cv)[(long)row * ldc + cbase] = f2bf(v);
                    } else {
                        reinterpret_cast<float *>(Cv)[((long)sp * M + row) * N + col] = v;
                    }
                }
                // one 32 x 32 tile's conversions and stores at a time (keeps the epilogue's
                // registers to one tile's worth)
                __builtin_amdgcn_sched_barrier(0);
            }
        if (!more) break;
        if constexpr (!EARLY) {
#pragma unroll
            for (int i = 0; i < NL; i++) stg[i] = gload(i, 0);
        }
        // every wave is past its last fragment read of this tile: stage 0 takes the next
        // tile's first step, the registers its second
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NL; i++) *reinterpret_cast<u32x4 *>(smem + wo + 4096 * i) = stg[i];
        m0 = m1;
        n0 = n1;
#pragma unroll
        for (int i = 0; i < NL; i++) stg[i] = gload(i, min(1, nks - 1));
        __syncthreads();
    }
}

// ---- whole tiles on v_mfma_f32_16x16x32 with direct-to-LDS loads ----------------------
//
// The same 256 x 256 workgroup tile and 2 x 2 waves, each wave's 128 x 128 block as 8 x 8
// tiles of 16 x 16 on the 16x16x32 MFMA (64 accumulators of 4 registers, kept in AGPRs by
// tying them to the instruction). K advances in stages of 32: each stage's A and B rows
// (32 KiB) are brought into LDS by buffer loads that write LDS directly (no VGPR staging and
// no LDS write instructions); four stages rotate, so a stage's loads are issued three stages
// before it is read. The load stream runs on across the tiles a workgroup of the persistent
// grid walks, so the next tile's first stages arrive while the current one finishes.
// Rows are 64 bytes (4 chunks of 16); chunk c of row r sits at c ^ ((r >> 2) & 3), which
// keeps every 16-lane fragment read on 64 distinct banks.
constexpr int QBK = 32, QNST = 4;
constexpr int QROW = QBK * 2;                     // bytes per staged row
constexpr int QSTAGE = (BM + BN) * QROW;          // 32 KiB
constexpr int QLDS = QNST * QSTAGE;               // 128 KiB
constexpr int QDMA = QSTAGE / 1024 / 4;           // 1 KiB loads per wave per stage (8)
constexpr int QT = WM / 16;                       // 16-row tiles per wave side (8)

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

// acc += a . b on the 16x16x32 MFMA with the accumulator tied to its AGPRs (the builtin lets
// the compiler move 64 accumulators between register files inside the loop)
template <int AB>
__device__ __forceinline__ void mfma16(const u32x4 &a, const u32x4 &b, f32x4 &c)
{
    if constexpr (AB == K3_DT_F16)
        asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
    else
        asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}

// Wait states between the accumulators' MFMA writes and their reads (or between their
// writes and the next MFMAs), pinned in order: each statement takes eight accumulators as
// operands, so no read moves above the first and no MFMA above the last.
#define K3_TIE8(nops, r)                                                                                       \
    asm volatile(nops : "+a"(r[0]), "+a"(r[1]), "+a"(r[2]), "+a"(r[3]), "+a"(r[4]), "+a"(r[5]), "+a"(r[6]), \
                 "+a"(r[7]))
#define K3_TIE_ACC(nops, acc)                                                                                  \
    do {                                                                                                       \
        K3_TIE8(nops, acc[0]); K3_TIE8("", acc[1]); K3_TIE8("", acc[2]); K3_TIE8("", acc[3]);                  \
        K3_TIE8("", acc[4]); K3_TIE8("", acc[5]); K3_TIE8("", acc[6]); K3_TIE8("", acc[7]);                    \
    } while (0)

// s_waitcnt vmcnt(n) lgkmcnt(0)
template <int n>
__device__ __forceinline__ void q_wait()
{
    static_assert(n >= 0 && n < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4));
}

template <int AB, int OUT, bool PERS>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(1, 1))) void mm16_kernel(
    int M, int N, int K, const uint16_t *__restrict__ A, long lda, const uint16_t *__restrict__ B, long ldb,
    void *__restrict__ Cv, long ldc, int gcols, long gstride, int tiles_m, int tiles_n)
{
    extern __shared__ __attribute__((aligned(1024))) char smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int nks = K / QBK;   // >= QNST (checked by the launcher)

    auto tile_at = [&](int r, int &m0, int &n0) -> bool {
        int tm, tn, sp;
        if constexpr (PERS) {
            if (!ptile_of(blockIdx.x, gridDim.x, r, tiles_m * tiles_n, tiles_m, tiles_n, tm, tn)) return false;
        } else {
            if (r > 0) return false;
            tile_of(blockIdx.x, gridDim.x, tiles_m, tiles_n, 1, tm, tn, sp);
        }
        m0 = min(tm * BM, M - BM);
        n0 = min(tn * BN, N - BN);
        return true;
    };
    auto rsrc = [&](const uint16_t *base) {
        return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, 0x7fffffff, 0x00020000);
    };

    // loads: instruction j (0 .. QDMA - 1) of wave w fills staged rows 16 (w + 4 j) .. + 15 (1 KiB
    // at stage + 1024 (w + 4 j); A rows for j < QDMA / 2, B rows after); lane l lands at row
    // + l / 4, physical chunk l & 3, so it loads logical chunk (l & 3) ^ ((l >> 4) & 3), the
    // chunk whose swizzled place that is (the row's (r >> 2) & 3 is (l >> 4) & 3 for every j)
    const int lch = (lane & 3) ^ ((lane >> 4) & 3);
    const int voA = ((lane >> 2) * (int)lda + lch * 8) * 2, voB = ((lane >> 2) * (int)ldb + lch * 8) * 2;
    int ir = 0, iks = 0, im0 = 0, in0 = 0;
    if (!tile_at(0, im0, in0)) return;
    __amdgpu_buffer_rsrc_t iA = rsrc(A + (long)im0 * lda), iB = rsrc(B + (long)in0 * ldb);
    // load j of a stage at stream position (rA, rB, ks)
    auto load = [&](int j, uint32_t stage_off, __amdgpu_buffer_rsrc_t rA, __amdgpu_buffer_rsrc_t rB, int ks) {
        const int R = 16 * (wave + 4 * j);
        char *dst = smem + stage_off + 1024 * (wave + 4 * j);
        if (j < QDMA / 2)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lds_void *)dst, 16, voA, R * (int)lda * 2 + ks * QROW, 0, 0);
        else
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, (lds_void *)dst, 16, voB, (R - BM) * (int)ldb * 2 + ks * QROW,
                                                     0, 0);
    };
    // the stream position moves on one stage (past the last stage it stays: the last stage is
    // loaded again into a buffer nothing reads)
    auto advance = [&]() {
        if (iks + 1 < nks) {
            iks++;
            return;
        }
        int m, n;
        if (!tile_at(ir + 1, m, n)) return;
        ir++;
        iks = 0;
        iA = rsrc(A + (long)m * lda);
        iB = rsrc(B + (long)n * ldb);
    };

    // fragments: lane (row r16 of a 16-row tile, K chunk kq) at its swizzled chunk
    const int r16 = lane & 15, kq = lane >> 4;
    const uint32_t fo = r16 * QROW + ((kq ^ ((r16 >> 2) & 3)) << 4);
    const uint32_t ra = fo + wm * WM * QROW, rb = fo + BM * QROW + wn * WN * QROW;
    auto lds16 = [&](uint32_t off) { return *reinterpret_cast<const u32x4 *>(smem + off); };

    // prologue: stages 0 .. 3 requested, stage 0 landed and published, its fragments read
#pragma unroll
    for (int p = 0; p < QNST; p++) {
#pragma unroll
        for (int j = 0; j < QDMA; j++) load(j, p * QSTAGE, iA, iB, iks);
        advance();
    }
    q_wait<(QNST - 1) * QDMA>();
    __builtin_amdgcn_s_barrier();
    u32x4 a[2][QT], b[QT];
#pragma unroll
    for (int i = 0; i < QT; i++) a[0][i] = lds16(ra + 1024 * i);
#pragma unroll
    for (int j = 0; j < QT; j++) b[j] = lds16(rb + 1024 * j);

    f32x4 acc[QT][QT];
#pragma unroll
    for (int i = 0; i < QT; i++)
#pragma unroll
        for (int j = 0; j < QT; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    K3_TIE_ACC("s_nop 4", acc);   // the zeroed AGPRs before the first MFMA reads them

    // stage G from buffer G % 4, its fragments in a[CUR] and b. 64 MFMA slots in column-group
    // order; slot 16 opens with the wait for stage G + 1 (this wave's loads, with G + 2 and
    // G + 3 still in flight) and the barrier after which every wave has read stage G's buffer
    // (it takes stage G + 4, one load every 4 slots from slot 26) and may read stage G + 1's:
    // b[0], b[1] (dead since slots 7, 15) at slots 16, 17, a[1 - CUR] at 18-25, b[j] right
    // after its last use from slot 23 on
    auto stage = [&](auto curc, uint32_t G) {
        constexpr int cur = decltype(curc)::value, nx = cur ^ 1;
        const uint32_t s1 = ((G + 1) % QNST) * QSTAGE, s0 = (G % QNST) * QSTAGE;
        const __amdgpu_buffer_rsrc_t dA = iA, dB = iB;
        const int dks = iks;
        advance();
#pragma unroll
        for (int q = 0; q < QT * QT; q++) {
            const int j = q / QT, i = q % QT;
            if (q == 16) {
                q_wait<(QNST - 2) * QDMA>();
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
            }
            mfma16<AB>(a[cur][i], b[j], acc[i][j]);
            if (q == 16) b[0] = lds16(rb + s1);
            if (q == 17) b[1] = lds16(rb + s1 + 1024);
            if (q >= 18 && q < 18 + QT) a[nx][q - 18] = lds16(ra + s1 + 1024 * (q - 18));
            if (i == QT - 1 && j >= 2) b[j] = lds16(rb + s1 + 1024 * j);
            if (q >= 26 && (q - 26) % 4 == 0 && (q - 26) / 4 < QDMA) load((q - 26) / 4, s0, dA, dB, dks);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    uint32_t G = 0;   // stage being computed, counted over this workgroup's tiles
    int m0, n0;
    for (int r = 0; tile_at(r, m0, n0); r++) {
        // nks is even: stages in pairs, so that the fragment register set is known statically
        for (int ks = 0; ks < nks; ks += 2, G += 2) {
            stage(std::integral_constant<int, 0>{}, G);
            stage(std::integral_constant<int, 1>{}, G + 1);
        }

        // the last MFMAs' results, then the tile out of the accumulators: lane holds rows
        // 4 kq .. 4 kq + 3, column r16 of each 16 x 16 tile
        K3_TIE_ACC("s_nop 15\n s_nop 15\n s_nop 15", acc);
#pragma unroll
        for (int i = 0; i < QT; i++)
#pragma unroll
            for (int j = 0; j < QT; j++) {
                const int col = n0 + wn * WN + j * 16 + r16;
                const int g = col / gcols;
                const long cbase = g * gstride + (col - g * gcols);
                const f32x4 v = acc[i][j];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int row = m0 + wm * WM + i * 16 + 4 * kq + e;
                    if constexpr (OUT == OUT_F32) {
                        reinterpret_cast<float *>(Cv)[(long)row * ldc + cbase] = v[e];
                    } else if constexpr (OUT == OUT_F16) {
                        reinterpret_cast<_Float16 *>(Cv)[(long)row * ldc + cbase] = (_Float16)v[e];
                    } else {
                        reinterpret_cast<uint16_t *>(Cv)[(long)row * ldc + cbase] = f2bf(v[e]);
                    }
                }
                acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                __builtin_amdgcn_sched_barrier(0);
            }
        // the stores count with the loads: let them drain so that the stage waits stay exact
        q_wait<0>();
        K3_TIE_ACC("s_nop 4", acc);
    }
    // no load may still be writing this workgroup's LDS when it ends
    q_wait<0>();
}

template <int AB, int OUT, bool PERS>
int launch_mm16(int M, int N, int K, const void *A, long lda, const void *B, long ldb, void *C, long ldc, int gcols,
                long gstride, long grid, hipStream_t st)
{
    static bool lds_ok[64];
    int dev = 0;
    K3_HIP(hipGetDevice(&dev));
    if (dev >= 0 && dev < 64 && !lds_ok[dev]) {
        K3_HIP(hipFuncSetAttribute((const void *)mm16_kernel<AB, OUT, PERS>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, QLDS));
        lds_ok[dev] = true;
    }
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    if (grid > 0x7fffffffL) K3_FAIL(K3HIP_EUNSUPPORTED, "mm: %dx%d output needs too many workgroups", M, N);
    hipLaunchKernelGGL((mm16_kernel<AB, OUT, PERS>), dim3((unsigned)grid), dim3(NT), QLDS, st, M, N, K,
                       (const uint16_t *)A, lda, (const uint16_t *)B, ldb, C, ldc, gcols, gstride, tiles_m, tiles_n);
    K3_LAUNCHED();
    return K3HIP_OK;
}

template <int AB, int OUT, bool EDGE, bool PERS>
int launch_mm_e(int M, int N, int K, const void *A, long lda, const void *B, long ldb, void *C, long ldc, int gcols,
                long gstride, int splits, long grid, hipStream_t st)
{
    static bool lds_ok[64];
    int dev = 0;
    K3_HIP(hipGetDevice(&dev));
    if (dev >= 0 && dev < 64 && !lds_ok[dev]) {
        K3_HIP(hipFuncSetAttribute((const void *)mm_kernel<AB, OUT, EDGE, PERS>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BYTES));
        lds_ok[dev] = true;
    }
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    if (grid > 0x7fffffffL) K3_FAIL(K3HIP_EUNSUPPORTED, "mm: %dx%d output needs too many workgroups", M, N);
    hipLaunchKernelGGL((mm_kernel<AB, OUT, EDGE, PERS>), dim3((unsigned)grid), dim3(NT), LDS_BYTES, st, M, N, K,
                       (const uint16_t *)A, lda, (const uint16_t *)B, ldb, C, ldc, gcols, gstride, tiles_m, tiles_n,
                       splits);
    K3_LAUNCHED();
    return K3HIP_OK;
}

template <int AB, int OUT>
int launch_mm(int M, int N, int K, const void *A, long lda, const void *B, long ldb, void *C, long ldc, int gcols,
              long gstride, int splits, hipStream_t st)
{
    // the uniform-offset form needs whole tiles and 32-bit buffer offsets
    const long tiles = (long)((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    if (M < BM || N < BN || (long)BM * 2 * std::max(lda, ldb) + 2L * K >= (1L << 31))
        return launch_mm_e<AB, OUT, true, false>(M, N, K, A, lda, B, ldb, C, ldc, gcols, gstride, splits,
                                                 tiles * splits, st);
    // more tiles than compute units: a persistent grid of one workgroup per CU (a multiple of 8,
    // one per XCD in turn); otherwise one workgroup per tile
    int ncu = 0, rc;
    if ((rc = cu_count(ncu))) return rc;
    const int pgrid = ncu / 8 * 8;
    if constexpr (OUT != OUT_PART) {
        // whole tiles in one K-range: the 16x16x32 form with direct-to-LDS stages
        if (splits == 1 && K % (2 * QBK) == 0 && K / QBK >= QNST) {
            if (pgrid >= 8 && tiles > pgrid)
                return launch_mm16<AB, OUT, true>(M, N, K, A, lda, B, ldb, C, ldc, gcols, gstride, pgrid, st);
            return launch_mm16<AB, OUT, false>(M, N, K, A, lda, B, ldb, C, ldc, gcols, gstride, tiles, st);
        }
    }
    if (splits == 1 && pgrid >= 8 && tiles > pgrid)
        return launch_mm_e<AB, OUT, false, true>(M, N, K, A, lda, B, ldb, C, ldc, gcols, gstride, 1, pgrid, st);
    return launch_mm_e<AB, OUT, false, false>(M, N, K, A, lda, B, ldb, C, ldc, gcols, gstride, splits,
                                              tiles * splits, st);
}

int check_shape(const char *who, int M, int N, int K, int ab, const void *A, long lda, const void *B, long ldb)
{
    if (ab != K3HIP_BF16 && ab != K3_DT_F16) K3_FAIL(K3HIP_EINVAL, "%s: operand dtype %d", who, ab);
    if (K % BK || (lda & 7) || (ldb & 7) || ((uintptr_t)A & 15) || ((uintptr_t)B & 15) || lda < K || ldb < K)
        K3_FAIL(K3HIP_EUNSUPPORTED, "%s: K=%d (a multiple of %d), lda=%ld ldb=%ld (multiples of 8), 16-byte "
                "aligned operands needed", who, K, BK, lda, ldb);
    return K3HIP_OK;
}

}  // namespace

bool mm_supported(int K, long lda, long ldb) { return K > 0 && K % BK == 0 && !(lda & 7) && !(ldb & 7); }

int mm(int M, int N, int K, int ab, const void *A, long lda, const void *B, long ldb, void *C, int out, long ldc,
       hipStream_t st, int gcols, long gstride)
{
    if (M <= 0 || N <= 0) return K3HIP_OK;
    int rc;
    if ((rc = check_shape("mm", M, N, K, ab, A, lda, B, ldb))) return rc;
    if (gcols <= 0) {
        gcols = N;
        gstride = 0;
    }
#define K3_MM(AB_, OUT_) launch_mm<AB_, OUT_>(M, N, K, A, lda, B, ldb, C, ldc, gcols, gstride, 1, st)
    if (ab == K3HIP_BF16) {
        if (out == K3HIP_F32) return K3_MM(K3HIP_BF16, OUT_F32);
        if (out == K3_DT_F16) return K3_MM(K3HIP_BF16, OUT_F16);
        if (out == K3HIP_BF16) return K3_MM(K3HIP_BF16, OUT_BF16);
    } else {
        if (out == K3HIP_F32) return K3_MM(K3_DT_F16, OUT_F32);
        if (out == K3_DT_F16) return K3_MM(K3_DT_F16, OUT_F16);
        if (out == K3HIP_BF16) return K3_MM(K3_DT_F16, OUT_BF16);
    }
#undef K3_MM
    K3_FAIL(K3HIP_EINVAL, "mm: output dtype %d", out);
}

int mm_splits(int M, int N, int K, int ncu)
{
    const long tiles = (long)((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    const int steps = K / BK;
    int s = 1;
    // split while the grid is short of the CUs and each split keeps at least 8 K-steps
    while (tiles * s * 2 <= ncu && steps % (s * 2) == 0 && steps / (s * 2) >= 8) s *= 2;
    return s;
}

int mm_splitk(int M, int N, int K, int splits, int ab, const void *A, long lda, const void *B, long ldb, float *P,
              hipStream_t st)
{
    if (M <= 0 || N <= 0) return K3HIP_OK;
    int rc;
    if ((rc = check_shape("mm_splitk", M, N, K, ab, A, lda, B, ldb))) return rc;
    if (splits < 1 || (K / BK) % splits) K3_FAIL(K3HIP_EINVAL, "mm_splitk: %d splits of K=%d", splits, K);
    if (ab == K3HIP_BF16) return launch_mm<K3HIP_BF16, OUT_PART>(M, N, K, A, lda, B, ldb, P, N, N, 0, splits, st);
    return launch_mm<K3_DT_F16, OUT_PART>(M, N, K, A, lda, B, ldb, P, N, N, 0, splits, st);
}

}  // namespace k3kda

using namespace k3kda;

extern "C" int k3hip_proj_gemm(int M, int N, int K, int ab_dtype, const void *A, long lda, const void *B, long ldb,
                               void *C, int c_dtype, long ldc, void *stream)
{
    clear_error();
    if (M < 0 || N < 0 || K <= 0 || (M && N && (!A || !B || !C)) || ldc < N)
        K3_FAIL(K3HIP_EINVAL, "k3hip_proj_gemm: M=%d N=%d K=%d ldc=%ld or NULL operand", M, N, K, ldc);
    if (ab_dtype != K3HIP_BF16 && ab_dtype != K3HIP_F16)
        K3_FAIL(K3HIP_EINVAL, "k3hip_proj_gemm: ab_dtype=%d (bf16 or fp16)", ab_dtype);
    if (c_dtype != K3HIP_F32 && c_dtype != K3HIP_BF16 && c_dtype != K3HIP_F16)
        K3_FAIL(K3HIP_EINVAL, "k3hip_proj_gemm: c_dtype=%d", c_dtype);
    return mm(M, N, K, ab_dtype, A, lda, B, ldb, C, c_dtype, ldc, as_stream(stream));
}
