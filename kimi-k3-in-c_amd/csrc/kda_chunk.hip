// SPDX-License-Identifier: Apache-2.0
// kda_chunk.hip - K2: chunked gated delta-rule prefill on bf16 MFMA (gfx950).
//
// Computes exactly what T sequential calls of the reference k3_kda_step produce per
// head (src/core/k3_ops.c:186-243, driven at :927-938), in chunks of C = 64 tokens.
// Within a chunk, with G_t = sum_{s<=t} g_s (per key channel, from the chunk start) and
// q already scaled by q_scale, the recurrence unrolls to
//   A_kk[t][s] = beta_t sum_i k_ti k_si e^(G_ti - G_si)     s <  t  (STRICTLY lower)
//   A_qk[t][s] =        sum_i q_ti k_si e^(G_ti - G_si)     s <= t  (diagonal INCLUDED)
//   Tm = (I + A_kk)^-1                                      unit lower triangular
//   W  = Tm diag(beta) (K . e^G)          U = Tm diag(beta) V
//   Vn = U - W S0                         (the per-token delta-rule writes w_t)
//   O  = (Q . e^G) S0 + A_qk Vn
//   S1 = diag(e^G_last) S0 + (K . e^(G_last - G))^T Vn
// The strict lower triangle of A_kk and the diagonal of A_qk are what make this equal to
// the sequential order "decay, delta write, read the UPDATED state".
//
// Exponent range. e^(G_t - G_s) for s < t is <= 1, but factoring it into a product of two
// MFMA operands needs a pivot. Row block a (16 rows) uses the pivot p = 16a + 8, its middle
// row: the row factor e^(G_t - G_p) and, inside the diagonal block, the column factor
// e^(G_p - G_s) both lie in [e^(-8 |gate_lb|), e^(8 |gate_lb|)]; for s before the block the
// column factor is <= 1 and only underflows where the true e^(G_t - G_s) does. Keeping both
// factors near 1 keeps a factored operand (k or q times its factor) a normal bf16 number
// for inputs as small as ~1e-20 -- with the pivot at the block's first row the row factor
// reaches e^(-15 |gate_lb|), and tiny (eps-dominated, unnormalised) q and k then fell into
// the denormal range, which the MFMA flushes. The host takes this path when
// 15 |gate_lb| <= 80. Exponentials are v_exp_f32 (2^x) on G pre-multiplied by log2(e).
//
// Precision. Every product whose operands are not exact bf16 is a split-bf16 product:
// x = hi + lo (both bf16), a.b ~ ah.bh + ah.bl + al.bh with fp32 accumulation, i.e. about
// 2^-17 relative per product. The 16x16 block products of the inverse use the fp32 MFMA.
//
// Phase 1 (kda_chunk_intra) is parallel over (chunk, head) and does everything that does
// not depend on the state. It leaves its results in a workspace already split into hi/lo
// bf16 and laid out in MFMA fragment order, so the sequential phase loads each operand
// with one 16-byte access per lane and no conversion work.
// Phase 2 (kda_chunk_state) walks the chunks in order, one workgroup per (head, 16-column
// tile of S): value columns of S are independent of each other, so the tiles never
// exchange data. It prefetches chunk c+1's operands into registers while it computes
// chunk c. Its blocks are mapped so that all tiles of one head sit on one XCD and share
// that XCD's L2 copy of the phase-1 operands.
#include "kda_internal.h"
#include "kda_prep_math.h"

#include <algorithm>
#include <type_traits>

namespace k3kda {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int CH = 64;          // chunk length
constexpr int SB = 16;          // sub-block (MFMA tile) edge
constexpr int P1_THREADS = 512; // phase-1 workgroup
constexpr float LOG2E = 1.4426950408889634f;

// Per-(chunk, head) workspace block, in BYTES. A fragment block (16 rows x 32 K) is 64
// lanes x 8 bf16 hi followed by 64 lanes x 8 bf16 lo (2 KiB). A C block (16 x 16 fp32) is
// 64 lanes x 4 floats (1 KiB).
template <int D> struct Ws {
    static constexpr int KSI = D / 32;                          // K-steps over channels
    static constexpr int NCT = D / 16;                          // 16-column tiles
    static constexpr size_t WF = 0;                             // W    A-frags [4][KSI]
    static constexpr size_t QF = WF + (size_t)4 * KSI * 2048;   // Q e^G A-frags [4][KSI]
    static constexpr size_t AF = QF + (size_t)4 * KSI * 2048;   // A_qk A-frags [4][2]
    static constexpr size_t KF = AF + (size_t)4 * 2 * 2048;     // (K e^(GL-G))^T A-frags [D/16][2]
    static constexpr size_t UC = KF + (size_t)NCT * 2 * 2048;   // U C blocks [4][NCT]
    static constexpr size_t GL = UC + (size_t)4 * NCT * 1024;   // e^G_last [D] fp32
    static constexpr size_t SIZE = GL + (size_t)D * 4;
};

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// x = hi + lo with hi = bf16_rne(x) and lo = bf16_rne(x - hi), two elements per packed
// conversion: the pair's hi bits come back to fp32 with a shift and a mask.
__device__ __forceinline__ void split2(float a, float b, bf16x2 &hi, bf16x2 &lo)
{
    hi = __builtin_convertvector(f2{a, b}, bf16x2);
    const uint32_t u = __builtin_bit_cast(uint32_t, hi);
    const float ha = __uint_as_float(u << 16), hb = __uint_as_float(u & 0xffff0000u);
    lo = __builtin_convertvector(f2{a - ha, b - hb}, bf16x2);
}

__device__ __forceinline__ void split8(const float (&x)[8], bf16x8 &hi, bf16x8 &lo)
{
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        bf16x2 h, l;
        split2(x[e], x[e + 1], h, l);
        hi[e] = h[0]; hi[e + 1] = h[1];
        lo[e] = l[0]; lo[e + 1] = l[1];
    }
}

// acc += a.b with both operands split: the two small cross terms first.
__device__ __forceinline__ f32x4 mma3(f32x4 acc, const bf16x8 &ah, const bf16x8 &al,
                                      const bf16x8 &bh, const bf16x8 &bl)
{
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, acc, 0, 0, 0);
    return acc;
}

__device__ __forceinline__ void load8(float (&x)[8], const float *p)
{
    const f4 a = *reinterpret_cast<const f4 *>(p);
    const f4 b = *reinterpret_cast<const f4 *>(p + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// 8 consecutive floats of a 16-byte aligned LDS row as two 128-bit reads.
__device__ __forceinline__ void lds8(float (&x)[8], const float *p)
{
    const f4 a = *reinterpret_cast<const f4 *>(p);
    const f4 b = *reinterpret_cast<const f4 *>(p + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}

// CPL (2 or 4) consecutive floats to an LDS address aligned to 4 CPL bytes, as one store.
template <int CPL>
__device__ __forceinline__ void store_cpl(float *p, const float (&v)[CPL])
{
    if constexpr (CPL == 4) *reinterpret_cast<f4 *>(p) = f4{v[0], v[1], v[2], v[3]};
    else *reinterpret_cast<f2 *>(p) = f2{v[0], v[1]};
}

// Workspace stores: 16-byte buffer stores with the system-scope non-temporal policy
// (aux 19 = sc0 | nt | sc1: through to memory, kept in no cache), addressed from the item's
// block. The workspace is read back by the next kernel from HBM (its L2 warm-up touches) and
// is larger than the memory-side cache, so keeping any of it only displaces the inputs: phase
// 1 at T=8192, H=32, D=128 -5 us with the compiler's nontemporal stores, and the core step
// 0.5355 -> 0.5333 ms with this policy. They are compiler-visible stores, so the wait states
// a store needs (an MFMA result as data, a VALU overwrite of its data registers) are inserted
// as for any other.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t ws_rsrc(char *blk, size_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(blk, (short)0, (int)bytes, 0x00020000);
}

template <typename V>
__device__ __forceinline__ void store_ws(__amdgpu_buffer_rsrc_t r, int off, const V &v)
{
    static_assert(sizeof(V) == 16, "16-byte stores");
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, 19);
}

// Split x and store it as lane `lane` of the fragment block `off` bytes into the item's block.
__device__ __forceinline__ void store_frag(__amdgpu_buffer_rsrc_t r, int off, int lane, const float (&x)[8])
{
    bf16x8 hi, lo;
    split8(x, hi, lo);
    store_ws(r, off + lane * 16, hi);
    store_ws(r, off + 1024 + lane * 16, lo);
}

struct Frag {
    bf16x8 hi, lo;
};

__device__ __forceinline__ Frag load_frag(const char *blk, int lane)
{
    Frag f;
    f.hi = *reinterpret_cast<const bf16x8 *>(blk + lane * 16);
    f.lo = *reinterpret_cast<const bf16x8 *>(blk + 1024 + lane * 16);
    return f;
}

// --------------------------------------------------------------- phase 1 ----
// LDS (floats): G*log2e, K, X (staging) [64][D+4]; A, Tm [64][68]; beta [64]; Y [4][16][17];
// per-wave scratch for the diagonal-block inverses [4][3][16][17].
template <int D> struct P1Lds {
    static constexpr int PD = D + 4;
    static constexpr int PA = CH + 4;
    static constexpr size_t G = 0;
    static constexpr size_t K = G + (size_t)CH * PD;
    static constexpr size_t X = K + (size_t)CH * PD;
    static constexpr size_t A = X + (size_t)CH * PD;
    static constexpr size_t TM = A + (size_t)CH * PA;
    static constexpr size_t B = TM + (size_t)CH * PA;
    static constexpr size_t Y = B + CH;
    static constexpr size_t NS = Y + 4 * 16 * 17;       // [4 waves][3][16][17] scratch
    static constexpr size_t FLOATS = NS + 4 * 3 * 16 * 17;
};

// Workspace block of (chunk c, head h); blocks are chunk-major.
template <int D>
__device__ __forceinline__ char *blk_addr(char *ws, int c, int H, int h)
{
    return ws + ((size_t)c * H + h) * Ws<D>::SIZE;
}

// Zero the six 16x16 blocks of Tm's staging area sT ([64][PA]) above the diagonal: the A_qk
// fragments and the W/U products read them, and no stage writes them.
template <int D>
__device__ __forceinline__ void zero_upper(float *sT, int tid)
{
    constexpr int PA = P1Lds<D>::PA;
#pragma unroll
    for (int j = 0; j < 6 * 256 / P1_THREADS; j++) {
        const int i = tid + P1_THREADS * j, q = i >> 8;
        const int a = q < 3 ? 0 : q < 5 ? 1 : 2, b = q < 3 ? q + 1 : q < 5 ? q - 1 : 3;
        sT[(SB * a + ((i >> 4) & 15)) * PA + SB * b + (i & 15)] = 0.0f;
    }
}

// Everything of one (chunk, head) item after its inputs are staged: g in sG, k in sK,
// q * q_scale in sX (rows past the end of the sequence zero), beta in sB, the blocks of sT
// above its diagonal zero (zero_upper; nothing else of sA or sT is read before written), and this
// wave's column tile of v in vreg. Writes the item's workspace block. Every LDS read of the
// item is complete when it returns.
// hook(0) .. hook(6) are called between the stages; the fused kernel issues its prefetch of
// the next item's inputs in parts there, so that the loads of all workgroups spread over the
// item instead of reaching HBM as one burst.
template <int D, typename Hook>
__device__ __forceinline__ void p1_item(float *lds, const float (&vreg)[2][8], char *blk, Hook &&hook)
{
    using L = P1Lds<D>;
    using WL = Ws<D>;
    constexpr int PD = L::PD, PA = L::PA, KSI = WL::KSI, NCT = WL::NCT;
    constexpr int NW = P1_THREADS / 64;
    float *sG = lds + L::G, *sK = lds + L::K, *sX = lds + L::X;
    float *sA = lds + L::A, *sT = lds + L::TM, *sB = lds + L::B, *sY = lds + L::Y;
    float *sNS = lds + L::NS;
    // the lane index is re-derived opaquely per item so that a caller's item loop keeps
    // the per-lane LDS addressing inside the loop instead of in registers across items
    int tid_o = threadIdx.x;
    asm volatile("" : "+v"(tid_o));
    const int tid = tid_o, lane = tid & 63, w = threadIdx.x >> 6;
    const int m = lane & 15, kg = lane >> 4;
    const __amdgpu_buffer_rsrc_t wr = ws_rsrc(blk, WL::SIZE);
    static_assert(WL::SIZE < (1u << 31), "workspace offsets are 32-bit");


    // (2) G = cumulative sum of g down the chunk (padded rows add 0), kept as G*log2(e):
    //     each channel's 64 rows are four 16-row segments scanned in registers, then each
    //     segment adds the totals of the segments before it.
    constexpr int SEGS = P1_THREADS / D;   // 4 for D = 128, 8 for D = 64
    constexpr int SEGR = CH / SEGS;
    float *sTot = sY;                      // [SEGS][D] segment totals (sY is free here)
    {
        const int i = tid % D, sg = tid / D;
        float x[SEGR];
#pragma unroll
        for (int r = 0; r < SEGR; r++) x[r] = sG[(sg * SEGR + r) * PD + i];
#pragma unroll
        for (int r = 1; r < SEGR; r++) x[r] += x[r - 1];
        sTot[sg * D + i] = x[SEGR - 1];
        __syncthreads();
        float off = 0.0f;
        for (int p2 = 0; p2 < sg; p2++) off += sTot[p2 * D + i];
#pragma unroll
        for (int r = 0; r < SEGR; r++) sG[(sg * SEGR + r) * PD + i] = (x[r] + off) * LOG2E;
    }
    __syncthreads();

    hook(0);
    // (3) A_kk (times beta_t, strictly lower) into sA; A_qk (lower with the diagonal) staged
    //     in sT (both zeroed beforehand), in 16x16 blocks (a, b), b <= a. A wave takes one
    //     row block a and up to two column blocks, so the row operands (k and q times
    //     e^(G_t - G_p)) are built once for both: waves 0-3 take (3; 0,1), (3; 2,3), (2; 0,1),
    //     (1; 0,1), waves 6 and 7 (2; 2) and (0; 0). Waves 4 and 5 meanwhile build
    //     (k e^(G_last - G))^T as A-fragments [D/16][2], half each. Waves w and w + 4 share a
    //     SIMD, so each SIMD has one two-block wave and one lighter wave.
    if (w == 4 || w == 5) {
        constexpr int NKF = NCT * 2 / 2;   // fragments per wave
#pragma unroll
        for (int q = 0; q < NKF; q++) {
            const int fb = NKF * (w - 4) + q, rt = fb >> 1, ks = fb & 1;
            const int i = SB * rt + m;
            const float gl = sG[(CH - 1) * PD + i];
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int s = 32 * ks + 8 * kg + e;
                x[e] = sK[s * PD + i] * exp2_fast(gl - sG[s * PD + i]);
            }
            store_frag(wr, (int)WL::KF + fb * 2048, lane, x);
        }
    } else {
        // wave -> (row block a, first column block b0, column blocks nb)
        const int a = w == 0 || w == 1 ? 3 : w == 2 || w == 6 ? 2 : w == 3 ? 1 : 0;
        const int b0 = w == 1 ? 2 : w == 6 ? 2 : 0;
        const int nb = w >= 6 ? 1 : 2;
        const int p = SB * a + 8;    // pivot row: the middle of row block a
        const int t = SB * a + m;    // A-operand row (token t)
        f32x4 akk[2] = {0.0f, 0.0f}, aqk[2] = {0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < KSI; ks++) {
            const int i0 = 32 * ks + 8 * kg;
            float lk[8], lq[8], gp[8], gt[8];
            lds8(gp, &sG[p * PD + i0]);
            lds8(gt, &sG[t * PD + i0]);
            lds8(lk, &sK[t * PD + i0]);
            lds8(lq, &sX[t * PD + i0]);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float ft = exp2_fast(gt[e] - gp[e]);
                lk[e] = lk[e] * ft;
                lq[e] = lq[e] * ft;
            }
            bf16x8 kh, kl, qh, ql;
            split8(lk, kh, kl);
            split8(lq, qh, ql);
#pragma unroll
            for (int jb = 0; jb < 2; jb++) {
                if (jb >= nb) break;
                const int s = SB * (b0 + jb) + m;   // B-operand row (token s)
                float r[8], gs[8];
                lds8(gs, &sG[s * PD + i0]);
                lds8(r, &sK[s * PD + i0]);
#pragma unroll
                for (int e = 0; e < 8; e++) r[e] = r[e] * exp2_fast(gp[e] - gs[e]);
                bf16x8 rh, rl;
                split8(r, rh, rl);
                akk[jb] = mma3(akk[jb], kh, kl, rh, rl);
                aqk[jb] = mma3(aqk[jb], qh, ql, rh, rl);
            }
        }
#pragma unroll
        for (int jb = 0; jb < 2; jb++) {
            if (jb >= nb) break;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int tt = SB * a + 4 * kg + e, ss = SB * (b0 + jb) + m;
                sA[tt * PA + ss] = ss < tt ? akk[jb][e] * sB[tt] : 0.0f;
                sT[tt * PA + ss] = ss <= tt ? aqk[jb][e] : 0.0f;
            }
        }
    }
    __syncthreads();

    hook(1);
    // (3b) A_qk as A-fragments [rt 4][ks 2], one fragment lane per thread (q e^G follows
    //      in the shadow of the diagonal inverses, (k e^(G_last - G))^T came with the A blocks).
    {
        const int fb = tid >> 6, rt = fb >> 1, ks = fb & 1;
        float x[8];
        lds8(x, &sT[(SB * rt + m) * PA + 32 * ks + 8 * kg]);
        store_frag(wr, (int)WL::AF + fb * 2048, lane, x);
    }
    __syncthreads();   // the inverse below overwrites every block of sT at or below the diagonal

    hook(2);
    // (4a) diagonal blocks of Tm = (I + A)^-1. A 16x16 strictly lower block N is nilpotent
    //      (N^16 = 0), so (I + N)^-1 = (I - N)(I + N^2)(I + N^4)(I + N^8) exactly: three
    //      squarings and three products, each a 16x16x16 fp32 MFMA product (4 x 16x16x4).
    //      Wave w < 4 inverts block w with all 64 lanes; the factors commute, so X is built
    //      as X = I + N^8, X += N^4 X, X += N^2 X, X -= N X.
    //      The inverting waves raise their issue priority over the filler work of their SIMD.
    if (w < 4) {
        __builtin_amdgcn_s_setprio(3);
        const int o = SB * w;
        float *N2 = sNS + (size_t)w * 3 * 272, *N4 = N2 + 272, *X = N4 + 272;
        const float *Nb = sA + o * PA + o;   // N, pitch PA
        // C = L (pitch pl) * R (pitch pr), both 16x16 in LDS
        auto mm = [&](const float *Lm, int pl, const float *Rm, int pr) {
            f32x4 acc = 0.0f;
#pragma unroll
            for (int kk = 0; kk < 4; kk++)
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(Lm[m * pl + 4 * kk + kg], Rm[(4 * kk + kg) * pr + m], acc, 0, 0, 0);
            return acc;
        };
        auto put = [&](float *Dm, const f32x4 &v) {
#pragma unroll
            for (int e = 0; e < 4; e++) Dm[(4 * kg + e) * 17 + m] = v[e];
        };
        put(N2, mm(Nb, PA, Nb, PA));
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        put(N4, mm(N2, 17, N2, 17));
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        {
            f32x4 x = mm(N4, 17, N4, 17);   // N^8
#pragma unroll
            for (int e = 0; e < 4; e++) x[e] += (4 * kg + e == m) ? 1.0f : 0.0f;
            put(X, x);
        }
        const float *Ps[3] = {N4, N2, Nb};
        const int pp[3] = {17, 17, PA};
#pragma unroll
        for (int st = 0; st < 3; st++) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const f32x4 px = mm(Ps[st], pp[st], X, 17);
            f32x4 x;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float old = X[(4 * kg + e) * 17 + m];
                x[e] = st < 2 ? old + px[e] : old - px[e];
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            if (st < 2) put(X, x);
            else {
#pragma unroll
                for (int e = 0; e < 4; e++) sT[(o + 4 * kg + e) * PA + o + m] = x[e];
            }
        }
        __builtin_amdgcn_s_setprio(0);
    } else {
        // meanwhile waves 4..7: q e^G (q scaled) as A-fragments [rt 4][KSI]
        for (int fb = w - 4; fb < 4 * KSI; fb += 4) {
            const int rt = fb / KSI, ks = fb % KSI;
            const int t = SB * rt + m, i0 = 32 * ks + 8 * kg;
            float x[8], gx[8];
            lds8(x, &sX[t * PD + i0]);
            lds8(gx, &sG[t * PD + i0]);
#pragma unroll
            for (int e = 0; e < 8; e++) x[e] = x[e] * exp2_fast(gx[e]);
            store_frag(wr, (int)WL::QF + fb * 2048, lane, x);
        }
    }
    __syncthreads();

    hook(3);
    // (4b) off-diagonal blocks, by distance d = a - b:
    //      Tm_ab = -Tm_aa * sum_{c=b}^{a-1} A_ac Tm_cb   (fp32 MFMA)
    for (int d = 1; d < 4; d++) {
        const bool act = w < 4 - d;
        const int a = w + d, b = w;
        float *Yw = sY + (w & 3) * 16 * 17;
        if (act) {
            f32x4 y = 0.0f;
            for (int cc = b; cc < a; cc++)
#pragma unroll
                for (int kk = 0; kk < 4; kk++) {
                    const float av = sA[(SB * a + m) * PA + SB * cc + 4 * kk + kg];
                    const float bv = sT[(SB * cc + 4 * kk + kg) * PA + SB * b + m];
                    y = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, y, 0, 0, 0);
                }
#pragma unroll
            for (int e = 0; e < 4; e++) Yw[(4 * kg + e) * 17 + m] = y[e];
        }
        __syncthreads();
        if (act) {
            f32x4 z = 0.0f;
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const float av = sT[(SB * a + m) * PA + SB * a + 4 * kk + kg];
                const float bv = Yw[(4 * kk + kg) * 17 + m];
                z = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, z, 0, 0, 0);
            }
#pragma unroll
            for (int e = 0; e < 4; e++) sT[(SB * a + 4 * kg + e) * PA + SB * b + m] = -z[e];
        }
        __syncthreads();
    }

    hook(4);
    // (5) W = Tm (beta K e^G) staged in sX, U = Tm (beta V) written as C blocks;
    //     wave w takes column tiles w, w+NW, ...
    static_assert(NCT <= NW, "one column tile per wave (v is prefetched for tile w)");
    for (int nt = w; nt < NCT; nt += NW) {
        const int n0 = SB * nt;
        f32x4 aw[4], au[4];
#pragma unroll
        for (int a = 0; a < 4; a++) aw[a] = au[a] = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            float xk[8], xv[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int s = 32 * ks + 8 * kg + e;
                const float bs = sB[s];
                xk[e] = (bs * sK[s * PD + n0 + m]) * exp2_fast(sG[s * PD + n0 + m]);
                xv[e] = bs * vreg[ks][e];
            }
            bf16x8 kh, kl, vh, vl;
            split8(xk, kh, kl);
            split8(xv, vh, vl);
#pragma unroll
            for (int a = 0; a < 4; a++) {
                if (a < 2 * ks) continue;   // Tm rows of block a vanish past column 16a+15
                float tv[8];
                lds8(tv, &sT[(SB * a + m) * PA + 32 * ks + 8 * kg]);
                bf16x8 th, tl;
                split8(tv, th, tl);
                aw[a] = mma3(aw[a], th, tl, kh, kl);
                au[a] = mma3(au[a], th, tl, vh, vl);
            }
        }
#pragma unroll
        for (int a = 0; a < 4; a++) {
            store_ws(wr, (int)WL::UC + ((a * NCT + nt) * 64 + lane) * 16, au[a]);
#pragma unroll
            for (int e = 0; e < 4; e++) sX[(SB * a + 4 * kg + e) * PD + n0 + m] = aw[a][e];
        }
    }
    __syncthreads();

    hook(5);
    // (5b) W as A-fragments [rt 4][KSI]
    for (int f = tid; f < 4 * KSI * 64; f += P1_THREADS) {
        const int fb = f >> 6, rt = fb / KSI, ks = fb % KSI;
        float x[8];
        lds8(x, &sX[(SB * rt + m) * PD + 32 * ks + 8 * kg]);
        store_frag(wr, (int)WL::WF + fb * 2048, lane, x);
    }

    hook(6);
    // (6) e^G_last.
    if (tid < D) reinterpret_cast<float *>(blk + WL::GL)[tid] = exp2_fast(sG[(CH - 1) * PD + tid]);
    __syncthreads();   // every LDS read of this item is done before the next one is staged
}

// Phase 1 from prepared inputs (fp32 q, k, v, g, beta). Persistent: workgroup b handles
// items b, b + gridDim.x, ... (item = chunk * H + head). The next item's inputs are loaded
// into registers while the current item computes; their row indices are clamped into the
// sequence and padding rows are zeroed only when the values are consumed, so no
// instruction waits on these loads before the next item.
template <int D>
__global__ __launch_bounds__(P1_THREADS) void kda_chunk_intra(int T, int H, float qs,
                                                              const float *__restrict__ q,
                                                              const float *__restrict__ k,
                                                              const float *__restrict__ v,
                                                              const float *__restrict__ g,
                                                              const float *__restrict__ beta,
                                                              char *__restrict__ ws)
{
    using L = P1Lds<D>;
    using WL = Ws<D>;
    constexpr int PD = L::PD, NCT = WL::NCT;
    extern __shared__ __attribute__((aligned(16))) float lds[];
    float *sG = lds + L::G, *sK = lds + L::K, *sX = lds + L::X, *sA = lds + L::A, *sB = lds + L::B;

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int m = lane & 15, kg = lane >> 4;
    const size_t P = (size_t)H * D;
    const int nch = (T + CH - 1) / CH, nitems = nch * H;
    constexpr int NPF = CH * D / 4 / P1_THREADS;   // float4s of each tensor per thread

    f4 pg[NPF], pk[NPF], pq[NPF];
    float pv[2][8], pb;
    auto fetch = [&](int item) {
        const int fc = item / H, fh = item % H, ft0 = fc * CH, fTc = min(CH, T - ft0);
#pragma unroll
        for (int j = 0; j < NPF; j++) {
            const int e = tid + j * P1_THREADS, t = e / (D / 4), i4 = (e % (D / 4)) * 4;
            const size_t at = (size_t)(ft0 + min(t, fTc - 1)) * P + (size_t)fh * D + i4;
            pg[j] = *reinterpret_cast<const f4 *>(g + at);
            pk[j] = *reinterpret_cast<const f4 *>(k + at);
            pq[j] = *reinterpret_cast<const f4 *>(q + at);
        }
        const int n0 = SB * (w < NCT ? w : 0);
#pragma unroll
        for (int ks = 0; ks < 2; ks++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int s = 32 * ks + 8 * kg + e;
                pv[ks][e] = v[(size_t)(ft0 + min(s, fTc - 1)) * P + (size_t)fh * D + n0 + m];
            }
        pb = beta[(size_t)(ft0 + min(tid & (CH - 1), fTc - 1)) * H + fh];
    };
    fetch(min((int)blockIdx.x, nitems - 1));

    for (int item = blockIdx.x; item < nitems; item += gridDim.x) {
        const int c = item / H, h = item % H;
        const int Tc = min(CH, T - c * CH);
        // (1) the prefetched inputs go to LDS (q pre-scaled), v stays in registers; A is
        //     cleared; then the next item's loads are issued.
        float vreg[2][8];
#pragma unroll
        for (int ks = 0; ks < 2; ks++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int s = 32 * ks + 8 * kg + e;
                vreg[ks][e] = (w < NCT && s < Tc) ? pv[ks][e] : 0.0f;
            }
#pragma unroll
        for (int j = 0; j < NPF; j++) {
            const int e = tid + j * P1_THREADS, t = e / (D / 4), i4 = (e % (D / 4)) * 4;
            const bool live = t < Tc;
            *reinterpret_cast<f4 *>(&sG[t * PD + i4]) = live ? pg[j] : f4(0.0f);
            *reinterpret_cast<f4 *>(&sK[t * PD + i4]) = live ? pk[j] : f4(0.0f);
            *reinterpret_cast<f4 *>(&sX[t * PD + i4]) = live ? pq[j] * qs : f4(0.0f);
        }
        zero_upper<D>(sA + CH * L::PA, tid);
        if (tid < CH) sB[tid] = tid < Tc ? pb : 0.0f;
        __syncthreads();
        fetch(min(item + (int)gridDim.x, nitems - 1));
        p1_item<D>(lds, vreg, blk_addr<D>(ws, c, H, h), [](int) {});
    }
}

// Phase 1 fused with the input preparation, from the raw conv inputs q_in, k_in, v_in
// [T][H*D] (bf16 or fp32, DT), the fp32 gate pre-activation z [T][H*D] and the beta logits [T][H]:
// per token, short conv + SiLU (taps in order), L2 norm of q and k, the bounded decay gate
// and beta, with the arithmetic of the stand-alone prep kernel (kda_prep_math.h), so the
// staged values -- and hence the workspace -- are bit-identical to prep followed by
// kda_chunk_intra. The prepared q, k, v, g never leave the chip.
//
// Half-wave hw (0..15) prepares tokens 4hw..4hw+3 of the chunk; its 32 lanes own CPL = D/32
// adjacent channels each. The K-1 inputs before the first of its tokens come from the rows
// before it (the previous chunk's last rows at hw = 0), or from the incoming conv history
// before the first token of the sequence (staged in LDS at the head's first chunk). v is
// staged through the A/Tm area (free at that point) to reach the column layout of U.
//
// Persistent over a contiguous range of items in head-major order (item = head * nch +
// chunk), so a workgroup keeps one head -- its conv taps and dt_bias sit in LDS -- for many
// consecutive chunks. The next item's raw rows are prefetched into registers.
template <int D, int K, int DT>
__global__ __launch_bounds__(P1_THREADS) void kda_chunk_intra_act(
    int T, int H, float qs, float lb, const void *__restrict__ q_in,
    const void *__restrict__ k_in, const void *__restrict__ v_in,
    const float *__restrict__ z, const float *__restrict__ b_logit,
    const float *__restrict__ q_conv, const float *__restrict__ k_conv,
    const float *__restrict__ v_conv, const float *__restrict__ A_log,
    const float *__restrict__ dt_bias, const float *__restrict__ conv_state,
    char *__restrict__ ws)
{
    using L = P1Lds<D>;
    using WL = Ws<D>;
    constexpr int PD = L::PD, NCT = WL::NCT;
    constexpr int CPL = D / 32, NH = K - 1, RL = CH / 16, NR = RL + NH;
    static_assert(RL >= NH, "only the first run of a chunk reaches before the chunk");
    static_assert(3 * D * NH <= 4 * 3 * 16 * 17, "conv history fits the inverse scratch area");
    // raw conv inputs of CPL adjacent channels: bf16 (8 or 4 bytes) or fp32 (16 or 8 bytes)
    typedef typename std::conditional<DT == K3HIP_BF16, typename std::conditional<CPL == 4, uint2, uint32_t>::type,
                                      typename std::conditional<CPL == 4, uint4, uint2>::type>::type Raw;
    constexpr int ESZ = DT == K3HIP_BF16 ? 2 : 4;
    extern __shared__ __attribute__((aligned(16))) float lds[];
    float *sG = lds + L::G, *sK = lds + L::K, *sX = lds + L::X, *sA = lds + L::A, *sB = lds + L::B;
    float *sV = lds + L::A;                    // v staging [CH][PD], aliases A and Tm
    float *sW = lds + L::FLOATS;               // conv taps [3][4][D], tap-major: a lane's CPL
                                               // channels of one tap are one conflict-free read
    float *sDT = sW + 3 * D * 4;               // dt_bias [D]
    float *sHist = lds + L::NS;                // incoming conv history [3][D][K-1] at chunk 0

    const int tid = threadIdx.x, w = tid >> 6;
    const int hw = tid >> 5, c0 = (tid & 31) * CPL, r0 = hw * RL;
    const size_t P = (size_t)H * D;
    const int nch = (T + CH - 1) / CH;
    const long nitems = (long)nch * H;
    const int lo = (int)((long)blockIdx.x * nitems / gridDim.x);
    const int hi = (int)((long)(blockIdx.x + 1) * nitems / gridDim.x);
    const char *xin[3] = {(const char *)q_in, (const char *)k_in, (const char *)v_in};
    const float *convw[3] = {q_conv, k_conv, v_conv};

    Raw raw[3][NR];
    float zr[RL][CPL], pbl;
    // the inputs of one item in five parts: raw q, k, v rows (with the K-1 rows before the
    // run), z, the beta logit; issued at the first five stage boundaries of the item before
    auto fetch = [&](int item, int part) {
        const int fh = item / nch, ft0 = (item % nch) * CH;
        if (part < 3) {
#pragma unroll
            for (int j = 0; j < NR; j++) {
                const int p = min(max(ft0 + r0 - NH + j, 0), T - 1);
                raw[part][j] = *reinterpret_cast<const Raw *>(xin[part] + ((size_t)p * P + (size_t)fh * D + c0) * ESZ);
            }
        } else if (part == 3) {
#pragma unroll
            for (int r = 0; r < RL; r++) {
                float x[CPL];
                RowIO<CPL, K3HIP_F32>::load(x, z, (size_t)min(ft0 + r0 + r, T - 1) * P + (size_t)fh * D + c0);
#pragma unroll
                for (int e = 0; e < CPL; e++) zr[r][e] = x[e];
            }
        } else if (part == 4) {
            pbl = b_logit[(size_t)min(ft0 + (tid & (CH - 1)), T - 1) * H + fh];
        }
    };
    if (lo < hi)
#pragma unroll
        for (int part = 0; part < 5; part++) fetch(lo, part);

    int head = -1;
    float a2 = 0.0f;
    for (int item = lo; item < hi; item++) {
        const int h = item / nch, c = item % nch;
        const int t0 = c * CH, Tc = min(CH, T - t0);
        // per-lane indices re-derived opaquely per item, so their LDS addresses are not
        // held in registers across the item loop
        int tid_o = threadIdx.x;
        asm volatile("" : "+v"(tid_o));
        const int tid = tid_o, lane = tid & 63;
        const int m = lane & 15, kg = lane >> 4;
        const int c0 = (tid & 31) * CPL, r0 = (tid >> 5) * RL;
        if (h != head) {   // uniform: a new head's conv taps and dt_bias into LDS
            for (int i = tid; i < 3 * 4 * D; i += P1_THREADS) {
                const int b = i / (4 * D), j = (i / D) % 4, ch = i % D;
                sW[i] = j < K ? convw[b][((size_t)h * D + ch) * K + j] : 0.0f;
            }
            for (int i = tid; i < D; i += P1_THREADS) sDT[i] = dt_bias[(size_t)h * D + i];
            a2 = gate_a2(expf(A_log[h]));
            head = h;
            __syncthreads();
        }
        if (NH > 0 && c == 0) {   // uniform: the head's incoming conv history into LDS, so
                                  // the preparation below never waits on a global load
            for (int i = tid; i < 3 * D * NH; i += P1_THREADS) {
                const int b = i / (D * NH), r = i % (D * NH);
                sHist[i] = conv_state ? conv_state[((size_t)b * P + (size_t)h * D) * NH + r] : 0.0f;
            }
            __syncthreads();
        }
        // (1) prepare this half-wave's RL tokens from the prefetched raw rows
        float y[3][RL][CPL];
#pragma unroll
        for (int b = 0; b < 3; b++) {
            float wq[K][CPL];   // this lane's CPL channels of each tap
#pragma unroll
            for (int j = 0; j < K; j++) {
                if constexpr (CPL == 4) {
                    const f4 t4 = *reinterpret_cast<const f4 *>(&sW[(b * 4 + j) * D + c0]);
                    wq[j][0] = t4.x; wq[j][1] = t4.y; wq[j][2] = t4.z; wq[j][3] = t4.w;
                } else {
                    const f2 t2 = *reinterpret_cast<const f2 *>(&sW[(b * 4 + j) * D + c0]);
                    wq[j][0] = t2.x; wq[j][1] = t2.y;
                }
            }
#pragma unroll
            for (int e = 0; e < CPL; e++) {
                float wt[K], xs[NR];
#pragma unroll
                for (int j = 0; j < K; j++) wt[j] = wq[j][e];
#pragma unroll
                for (int j = 0; j < NR; j++) {
                    if constexpr (DT == K3HIP_BF16) {
                        uint32_t u;
                        if constexpr (CPL == 4) u = (e < 2) ? raw[b][j].x : raw[b][j].y;
                        else u = raw[b][j];
                        xs[j] = __uint_as_float((e & 1) ? (u & 0xffff0000u) : (u << 16));
                    } else {
                        xs[j] = __uint_as_float(e == 0 ? raw[b][j].x : e == 1 ? raw[b][j].y
                                                : e == 2 ? ((const uint32_t *)&raw[b][j])[2]
                                                         : ((const uint32_t *)&raw[b][j])[3]);
                    }
                }
                if (t0 + r0 < NH) {   // first tokens of the sequence: incoming history
#pragma unroll
                    for (int j = 0; j < NH; j++) {
                        const int p = t0 + r0 - NH + j;
                        if (p < 0) xs[j] = sHist[(b * D + c0 + e) * NH + (p + NH)];
                    }
                }
#pragma unroll
                for (int r = 0; r < RL; r++) y[b][r][e] = conv_silu<K>(wt, &xs[r], xs[NH + r]);
            }
        }
#pragma unroll
        for (int r = 0; r < RL; r++) {
            l2norm_half<CPL>(y[0][r]);
            l2norm_half<CPL>(y[1][r]);
            const int t = r0 + r;
            const bool live = t < Tc;
            float vg[CPL], vk[CPL], vx[CPL], vv[CPL];
#pragma unroll
            for (int e = 0; e < CPL; e++) {
                vg[e] = live ? gate_bounded(lb, a2, zr[r][e], sDT[c0 + e]) : 0.0f;
                vk[e] = live ? y[1][r][e] : 0.0f;
                vx[e] = live ? y[0][r][e] * qs : 0.0f;
                vv[e] = live ? y[2][r][e] : 0.0f;
            }
            // one 8- or 16-byte store per row and tensor (c0 and the pitch are multiples of CPL)
            const int i = t * PD + c0;
            store_cpl<CPL>(sG + i, vg);
            store_cpl<CPL>(sK + i, vk);
            store_cpl<CPL>(sX + i, vx);
            store_cpl<CPL>(sV + i, vv);
        }
        if (tid < CH) sB[tid] = tid < Tc ? fast_sigmoid(pbl) : 0.0f;
        __syncthreads();
        float vreg[2][8];
        {
            const int n0 = SB * (w < NCT ? w : 0);
#pragma unroll
            for (int ks = 0; ks < 2; ks++)
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float x = sV[(32 * ks + 8 * kg + e) * PD + n0 + m];
                    vreg[ks][e] = w < NCT ? x : 0.0f;
                }
        }
        __syncthreads();   // v staging read before the A/Tm area is written
        zero_upper<D>(sA + CH * L::PA, tid);
        const int next = min(item + 1, hi - 1);
        p1_item<D>(lds, vreg, blk_addr<D>(ws, c, H, h), [&](int part) { fetch(next, part); });
    }
}

// --------------------------------------------------------------- phase 2 ----
// Eight waves per workgroup, in two roles, for one head and 16 columns j0..j0+15 of S:
//   row waves   (w = 0..3)  own token rows 16w..16w+15 of the chunk:
//                           Vn = U - W S and Q S, then O = Q S + A_qk Vn
//   state waves (w = 4..7)  own state rows 32(w-4)..32(w-4)+31 (two 16-row tiles):
//                           S = diag(e^G_last) S + (K e^(G_last - G))^T Vn
// Per chunk: state waves publish S to LDS -> barrier -> row waves publish Vn -> barrier
// -> row waves finish O while state waves update S. Each role prefetches the next chunk's
// operands into a second register set (used alternately, no copies), issuing the loads in
// windows where it does not hold up the other role: state waves between the two barriers
// (they wait for Vn there), row waves spread over their products (P2_MID). A step's O rows
// are stored at the start of the next step, before its loads, so the stores do not queue
// behind a full vector-memory path (T=8192, H=32 prefill kernels 598 -> 565 us).
template <int D, int NW> struct RowOps {
    static constexpr int KSI = D / 32;
    Frag wf[KSI], qf[KSI], af[2];
    f32x4 u[NW];
};
template <int D> struct StateOps {
    static constexpr int RTW = D / 64;   // 16-row tiles per state wave
    Frag kf[RTW][2];
    f32x4 gl[RTW];
};

// Of the next chunk's row operands (load_row_part parts 0 .. KSI), a row wave issues parts
// 0 .. P2_MID-1 between the K-steps of this step's W S / Q S products and the rest after
// barrier (2), so its loads share the CU's vector-memory path with the state waves' loads
// (issued between the two barriers) instead of all queueing at the start of the step. At
// D = 128 all W and Q e^G K-steps go between the products and A_qk and U after barrier (2)
// (T=8192, H=32: 6 us faster than 3 K-steps before it, 10 us faster than everything before it).
constexpr int P2_MID = 4;

// Row wave w's operands of one chunk: W, Q e^G and A_qk fragments of its 16 token rows
// (shared by all of the workgroup's column tiles) and U for each tile ct0 .. ct0+NW-1.
template <int D, int NW>
__device__ __forceinline__ void load_row_ops(RowOps<D, NW> &op, const char *blk, int w, int lane, int ct0)
{
    using WL = Ws<D>;
    constexpr int KSI = WL::KSI;
#pragma unroll
    for (int ks = 0; ks < KSI; ks++) {
        op.wf[ks] = load_frag(blk + WL::WF + (size_t)(w * KSI + ks) * 2048, lane);
        op.qf[ks] = load_frag(blk + WL::QF + (size_t)(w * KSI + ks) * 2048, lane);
    }
#pragma unroll
    for (int ks = 0; ks < 2; ks++)   // af[1] of waves 0-1 is all zero and unused
        op.af[ks] = load_frag(blk + WL::AF + (size_t)(w * 2 + ks) * 2048, lane);
#pragma unroll
    for (int j = 0; j < NW; j++)
        op.u[j] = *reinterpret_cast<const f32x4 *>(blk + WL::UC + ((size_t)(w * WL::NCT + ct0 + j) * 64 + lane) * 16);
}

// One part of load_row_ops: part < KSI loads K-step `part` of W and Q e^G; part == KSI the
// A_qk fragments and U.
template <int D, int NW>
__device__ __forceinline__ void load_row_part(RowOps<D, NW> &op, const char *blk, int w, int lane, int ct0, int part)
{
    using WL = Ws<D>;
    constexpr int KSI = WL::KSI;
    if (part < KSI) {
        op.wf[part] = load_frag(blk + WL::WF + (size_t)(w * KSI + part) * 2048, lane);
        op.qf[part] = load_frag(blk + WL::QF + (size_t)(w * KSI + part) * 2048, lane);
    } else {
#pragma unroll
        for (int ks = 0; ks < 2; ks++)
            if (ks == 0 || w >= 2) op.af[ks] = load_frag(blk + WL::AF + (size_t)(w * 2 + ks) * 2048, lane);
#pragma unroll
        for (int j = 0; j < NW; j++)
            op.u[j] = *reinterpret_cast<const f32x4 *>(blk + WL::UC + ((size_t)(w * WL::NCT + ct0 + j) * 64 + lane) * 16);
    }
}

// sw = state-wave index 0..3; its tiles are rows 16*(RTW*sw + r) .. +15
template <int D>
__device__ __forceinline__ void load_state_ops(StateOps<D> &op, const char *blk, int sw, int lane)
{
    using WL = Ws<D>;
    constexpr int RTW = D / 64;
    const int kg = lane >> 4;
#pragma unroll
    for (int r = 0; r < RTW; r++) {
        const int rt = RTW * sw + r;
#pragma unroll
        for (int ks = 0; ks < 2; ks++) op.kf[r][ks] = load_frag(blk + WL::KF + (size_t)(rt * 2 + ks) * 2048, lane);
        op.gl[r] = *reinterpret_cast<const f32x4 *>(blk + WL::GL + (size_t)(16 * rt + 4 * kg) * 4);
    }
}

// S and Vn cross between the two roles through LDS as B-operand fragments that the
// producer has already split: block (ks, part) holds, for each lane n + 16 kg, the 8 bf16
// of rows 32 ks + 8 kg .. +7 of column n (part 0 = hi, part 1 = lo). Each value is split
// once by its owner and read back with two 128-bit loads per K-step.
// A producer lane holds 4 consecutive rows (C layout: rows 16 tile + 4 kg' + e', column m);
// they land in lane m + 16 (2 (tile & 1) + kg' / 2) at elements 4 (kg' & 1) .. +3 of K-step
// tile / 2.
__device__ __forceinline__ void publish_frag4(char *buf, int tile, int lane, const f32x4 &x)
{
    const int m = lane & 15, kgp = lane >> 4;
    const int ks = tile >> 1, kg = 2 * (tile & 1) + (kgp >> 1), e0 = 4 * (kgp & 1);
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
    bf16x4 hi, lo;
#pragma unroll
    for (int e = 0; e < 4; e += 2) {
        bf16x2 h, l;
        split2(x[e], x[e + 1], h, l);
        hi[e] = h[0]; hi[e + 1] = h[1];
        lo[e] = l[0]; lo[e + 1] = l[1];
    }
    char *d = buf + ((size_t)(ks * 2) * 64 + m + 16 * kg) * 16 + e0 * 2;
    *reinterpret_cast<bf16x4 *>(d) = hi;
    *reinterpret_cast<bf16x4 *>(d + 1024) = lo;
}

__device__ __forceinline__ Frag read_frag(const char *buf, int ks, int lane)
{
    Frag f;
    f.hi = *reinterpret_cast<const bf16x8 *>(buf + ((size_t)(ks * 2) * 64 + lane) * 16);
    f.lo = *reinterpret_cast<const bf16x8 *>(buf + ((size_t)(ks * 2 + 1) * 64 + lane) * 16);
    return f;
}

// LDS of one column tile: S fragments (D/32 K-steps) then Vn fragments (2 K-steps).
template <int D> struct P2Lds {
    static constexpr size_t SF = (size_t)(D / 32) * 2 * 1024;
    static constexpr size_t VF = (size_t)2 * 2 * 1024;
};

template <int D, int NW, typename Mid, typename After2>
__device__ __forceinline__ void row_step(const RowOps<D, NW> &op, const char *sSF, char *sVF, int w,
                                         int lane, f32x4 (&oval)[NW], Mid &&mid, After2 &&after2)
{
    constexpr int KSI = D / 32;
    f32x4 ao[NW];
    __builtin_amdgcn_s_setprio(3);   // W S -> Vn is the step's critical path: issue it first
#pragma unroll
    for (int j = 0; j < NW; j++) {
        // Vn = U - W S and O = Q S; two accumulators per product shorten the MFMA chains
        const char *sf_j = sSF + (size_t)j * P2Lds<D>::SF;
        f32x4 aw0 = 0.0f, aw1 = 0.0f, ao0 = 0.0f, ao1 = 0.0f;
#pragma unroll
        for (int ks = 0; ks < KSI; ks++) {
            const Frag sf = read_frag(sf_j, ks, lane);
            if (ks & 1) {
                aw1 = mma3(aw1, op.wf[ks].hi, op.wf[ks].lo, sf.hi, sf.lo);
                ao1 = mma3(ao1, op.qf[ks].hi, op.qf[ks].lo, sf.hi, sf.lo);
            } else {
                aw0 = mma3(aw0, op.wf[ks].hi, op.wf[ks].lo, sf.hi, sf.lo);
                ao0 = mma3(ao0, op.qf[ks].hi, op.qf[ks].lo, sf.hi, sf.lo);
            }
            if (j == 0) mid(ks);
        }
        publish_frag4(sVF + (size_t)j * P2Lds<D>::VF, w, lane, op.u[j] - (aw0 + aw1));
        ao[j] = ao0 + ao1;
    }
    __builtin_amdgcn_s_setprio(0);
    __syncthreads();   // (2) Vn published
    after2();
#pragma unroll
    for (int j = 0; j < NW; j++) {
        const char *vf_j = sVF + (size_t)j * P2Lds<D>::VF;
        const Frag v0 = read_frag(vf_j, 0, lane);
        f32x4 a = mma3(ao[j], op.af[0].hi, op.af[0].lo, v0.hi, v0.lo);
        if (w >= 2) {
            const Frag v1 = read_frag(vf_j, 1, lane);
            a = mma3(a, op.af[1].hi, op.af[1].lo, v1.hi, v1.lo);
        }
        oval[j] = a;
    }
}

// O rows of one chunk step from row wave w (stored one step later, ahead of that step's loads)
template <int NW>
__device__ __forceinline__ void store_o(const f32x4 (&oval)[NW], int w, int lane, int nrows, float *ob, size_t P)
{
    const int m = lane & 15, kg = lane >> 4;
#pragma unroll
    for (int j = 0; j < NW; j++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int t = 16 * w + 4 * kg + e;
            if (t < nrows) ob[(size_t)t * P + 16 * j + m] = oval[j][e];
        }
}

template <int D, int NW>
__device__ __forceinline__ void state_publish(const f32x4 (&accS)[D / 64][NW], char *sSF, int sw, int lane)
{
    constexpr int RTW = D / 64;
#pragma unroll
    for (int j = 0; j < NW; j++)
#pragma unroll
        for (int r = 0; r < RTW; r++) publish_frag4(sSF + (size_t)j * P2Lds<D>::SF, RTW * sw + r, lane, accS[r][j]);
}

template <int D, int NW>
__device__ __forceinline__ void state_update(const StateOps<D> &op, f32x4 (&accS)[D / 64][NW],
                                             const char *sVF, int lane)
{
    constexpr int RTW = D / 64;
#pragma unroll
    for (int j = 0; j < NW; j++) {
        const char *vf_j = sVF + (size_t)j * P2Lds<D>::VF;
        const Frag v0 = read_frag(vf_j, 0, lane), v1 = read_frag(vf_j, 1, lane);
#pragma unroll
        for (int r = 0; r < RTW; r++) {
            accS[r][j] = accS[r][j] * op.gl[r];
            accS[r][j] = mma3(accS[r][j], op.kf[r][0].hi, op.kf[r][0].lo, v0.hi, v0.lo);
            accS[r][j] = mma3(accS[r][j], op.kf[r][1].hi, op.kf[r][1].lo, v1.hi, v1.lo);
        }
    }
}

// The outgoing short-conv history of the fused prefill (conv_state_update's result), formed
// by phase 2's state waves: each of the first 3 P of them loads one channel's K-1 newest
// inputs (or, for T < K-1, the older history slots that shift down) before its loop and
// stores them after it, off the critical path. Phase 1 has read the incoming history by then.
struct ConvOut {
    const void *qi, *ki, *vi;   // raw conv inputs [T][P] (bf16 or fp32, dt)
    float *cs;                  // [3][P][K-1], nullptr: nothing to do
    int K, dt;
};

// --- phase 2 kernel: one workgroup per (head, NW consecutive 16-column tiles of S) ---
template <int D, int NW>
__global__ __launch_bounds__(512) void kda_chunk_state(int T, int H, const char *__restrict__ ws,
                                                       float *__restrict__ S,
                                                       float *__restrict__ o, ConvOut co)
{
    using WL = Ws<D>;
    constexpr int NG = D / 16 / NW;      // workgroups per head
    constexpr int RTW = D / 64;
    extern __shared__ __attribute__((aligned(16))) char p2lds[];
    char *sSF = p2lds;                               // [NW] S fragments
    char *sVF = p2lds + (size_t)NW * P2Lds<D>::SF;   // [NW] Vn fragments

    // XCD-aware: block b runs on XCD b % 8; give each XCD whole heads.
    const int nb = gridDim.x, b = blockIdx.x;
    int idx = b;
    if (nb % 8 == 0) idx = (b % 8) * (nb / 8) + b / 8;
    const int h = idx / NG, ct0 = (idx % NG) * NW, j0 = ct0 * 16;

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int kg = lane >> 4, m = lane & 15;
    const size_t P = (size_t)H * D;
    float *Sh = S + (size_t)h * D * D;
    const int nch = (T + CH - 1) / CH;
    // The prefetch is unconditional (the last chunk re-reads itself) so that the compiler's
    // count of outstanding loads is exact on every path and no wait drains the prefetch.
    auto blk_of = [&](int c) { return ws + ((size_t)min(c, nch - 1) * H + h) * WL::SIZE; };

    if (w < 4) {
        RowOps<D, NW> opA, opB;
        float *ob = o + (size_t)h * D + j0;
        load_row_ops<D, NW>(opA, blk_of(0), w, lane, ct0);
        f32x4 pend[NW];
        int pend_c = -1;
        auto mid_of = [&](RowOps<D, NW> &op, int cc) {
            return [&op, cc, &blk_of, w, lane, ct0](int ks) {
                if (ks < P2_MID) load_row_part<D, NW>(op, blk_of(cc), w, lane, ct0, ks);
                if (ks == D / 32 - 1 && P2_MID > D / 32) load_row_part<D, NW>(op, blk_of(cc), w, lane, ct0, D / 32);
            };
        };
        auto after_of = [&](RowOps<D, NW> &op, int cc) {
            return [&op, cc, &blk_of, w, lane, ct0]() {
#pragma unroll
                for (int p = P2_MID; p <= D / 32; p++) load_row_part<D, NW>(op, blk_of(cc), w, lane, ct0, p);
                __builtin_amdgcn_sched_barrier(0);
            };
        };
        auto flush = [&]() {
            if (pend_c >= 0) store_o<NW>(pend, w, lane, T - pend_c * CH, ob + (size_t)pend_c * CH * P, P);
        };
        for (int c = 0; c < nch; c += 2) {
            __syncthreads();   // (1) S published
            flush();
            row_step<D, NW>(opA, sSF, sVF, w, lane, pend, mid_of(opB, c + 1), after_of(opB, c + 1));
            pend_c = c;
            if (c + 1 >= nch) break;
            __syncthreads();
            flush();
            row_step<D, NW>(opB, sSF, sVF, w, lane, pend, mid_of(opA, c + 2), after_of(opA, c + 2));
            pend_c = c + 1;
        }
        flush();
    } else {
        const int sw = w - 4;
        // L2 warm-up. The workgroups of one head together touch every 128-byte L2 line of the
        // item PF chunks ahead (one dword each); when the operand loads of that chunk come,
        // they hit L2 instead of waiting on HBM once per step. A touch is consumed (waited
        // for) two steps after it is issued, just before its register is reused. PF = 2 (the
        // touch one step before the operand loads) measured best: phase 2 at T=8192, H=32 is 7 us faster
        // than at PF = 4 and 50 us faster than without touches; farther touches are evicted
        // from the XCD's L2 before use more often (one touch per 64 bytes cost 6 us more).
        constexpr int PF = 2;
        constexpr int LINES = (int)((WL::SIZE + 127) / 128);
        constexpr int PER_WG = (LINES + NG - 1) / NG;
        constexpr int TPL = (PER_WG + 255) / 256;
        const int line0 = (idx % NG) * PER_WG + sw * 64 + lane;
        auto touch = [&](int (&t)[TPL], int c) {
            const char *bk = blk_of(c);
#pragma unroll
            for (int i = 0; i < TPL; i++)
                t[i] = *reinterpret_cast<const int *>(bk + (size_t)min(line0 + 256 * i, LINES - 1) * 128);
        };
        auto consume = [](const int (&t)[TPL]) {
#pragma unroll
            for (int i = 0; i < TPL; i++) asm volatile("" ::"v"(t[i]));
        };
        int tA[TPL], tB[TPL];
        // this thread's channel of the outgoing conv history: the grid's H NG workgroups have
        // 256 state-wave threads each, one per channel of the 3 H D
        static_assert(256 * NG >= 3 * D, "the state waves must cover the 3 H D conv channels");
        const int NHc = co.K - 1;
        const long chbc = (long)blockIdx.x * 256 + (threadIdx.x - 256);
        const bool chdo = co.cs && NHc > 0 && chbc < 3L * (long)P;
        float chv[3] = {0.0f, 0.0f, 0.0f};
        if (chdo) {
            const int cb = (int)(chbc / (long)P);
            const size_t cc = (size_t)(chbc % (long)P);
            const void *src = cb == 0 ? co.qi : (cb == 1 ? co.ki : co.vi);
            for (int j = 0; j < NHc; j++) {
                const int p = T - NHc + j;
                chv[j] = p >= 0 ? (co.dt == K3HIP_BF16 ? load_act<K3HIP_BF16>(src, (size_t)p * P + cc)
                                                       : load_act<K3HIP_F32>(src, (size_t)p * P + cc))
                                : co.cs[chbc * NHc + j + T];   // T < K-1: an older slot shifts down
            }
        }
        f32x4 accS[RTW][NW];
#pragma unroll
        for (int j = 0; j < NW; j++)
#pragma unroll
            for (int r = 0; r < RTW; r++)
#pragma unroll
                for (int e = 0; e < 4; e++)
                    accS[r][j][e] = Sh[(size_t)(16 * (RTW * sw + r) + 4 * kg + e) * D + j0 + 16 * j + m];
        StateOps<D> opA, opB;
        load_state_ops<D>(opA, blk_of(0), sw, lane);
        touch(tA, PF - 2);
        touch(tB, PF - 1);
        state_publish<D, NW>(accS, sSF, sw, lane);
        for (int c = 0; c < nch; c += 2) {
            __syncthreads();   // (1)
            load_state_ops<D>(opB, blk_of(c + 1), sw, lane);
            consume(tA);
            touch(tA, c + PF);
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();   // (2) Vn published
            __builtin_amdgcn_s_setprio(3);   // the S update is the other half of the critical path
            state_update<D, NW>(opA, accS, sVF, lane);
            state_publish<D, NW>(accS, sSF, sw, lane);
            __builtin_amdgcn_s_setprio(0);   // row waves read sSF before (2)
            if (c + 1 >= nch) break;
            __syncthreads();
            load_state_ops<D>(opA, blk_of(c + 2), sw, lane);
            consume(tB);
            touch(tB, c + 1 + PF);
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();
            __builtin_amdgcn_s_setprio(3);
            state_update<D, NW>(opB, accS, sVF, lane);
            state_publish<D, NW>(accS, sSF, sw, lane);
            __builtin_amdgcn_s_setprio(0);
        }
#pragma unroll
        for (int j = 0; j < NW; j++)
#pragma unroll
            for (int r = 0; r < RTW; r++)
#pragma unroll
                for (int e = 0; e < 4; e++)
                    Sh[(size_t)(16 * (RTW * sw + r) + 4 * kg + e) * D + j0 + 16 * j + m] = accS[r][j][e];
        if (chdo)
            for (int j = 0; j < NHc; j++) co.cs[chbc * NHc + j] = chv[j];
    }
}

bool chunk_ready() { return true; }

// Compute units of the current device (cached per device).
int cu_count(int &ncu)
{
    static int cache[64];
    int dev = 0;
    K3_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) {
        ncu = 256;
        return K3HIP_OK;
    }
    if (!cache[dev]) {
        int n = 0;
        K3_HIP(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
        cache[dev] = n > 0 ? n : 256;
    }
    ncu = cache[dev];
    return K3HIP_OK;
}

// Opt a kernel into more than the default dynamic LDS, once.
static int allow_lds(const void *fn, size_t bytes, bool &done)
{
    if (!done) {
        K3_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
        done = true;
    }
    return K3HIP_OK;
}

template <int D, int NW>
static int launch_state_nw(int T, int H, const char *ws, float *S, float *o, const ConvOut &co, hipStream_t st)
{
    const size_t lds = (size_t)NW * (P2Lds<D>::SF + P2Lds<D>::VF);
    static bool lds_ok = false;
    int rc;
    if ((rc = allow_lds((const void *)kda_chunk_state<D, NW>, lds, lds_ok))) return rc;
    hipLaunchKernelGGL((kda_chunk_state<D, NW>), dim3(H * (D / 16 / NW)), dim3(512), lds, st, T, H, ws, S, o, co);
    K3_LAUNCHED();
    return K3HIP_OK;
}

// One 16-column tile per workgroup. Wider workgroups (NW = 2, 4) give the same bits but run
// slower at H = 32, D = 128: a step's time is set by each CU's own operand loads (the row
// operands of the whole head are needed by every tile), not by the redundant copies that
// the head's other workgroups load from the same L2.
template <int D>
static int launch_state(int T, int H, const char *ws, float *S, float *o, hipStream_t st,
                        const ConvOut &co = ConvOut{nullptr, nullptr, nullptr, nullptr, 0, 0})
{
    return launch_state_nw<D, 1>(T, H, ws, S, o, co, st);
}

template <int D>
static int launch_chunk(int T, int H, const float *q, const float *k, const float *v,
                        const float *g, const float *beta, float qs, float *S, float *o,
                        char *ws, hipStream_t st)
{
    const long nitems = (long)((T + CH - 1) / CH) * H;
    const size_t lds = P1Lds<D>::FLOATS * sizeof(float);
    static bool lds_ok = false;
    int ncu = 0, rc;
    if ((rc = allow_lds((const void *)kda_chunk_intra<D>, lds, lds_ok))) return rc;
    if ((rc = cu_count(ncu))) return rc;
    const int grid = (int)(nitems < ncu ? nitems : ncu);   // one 150 KiB-LDS workgroup per CU
    hipLaunchKernelGGL((kda_chunk_intra<D>), dim3(grid), dim3(P1_THREADS), lds, st, T, H, qs, q, k,
                       v, g, beta, ws);
    K3_LAUNCHED();
    return launch_state<D>(T, H, ws, S, o, st);
}

struct PrefillArgs {
    int T, H;
    float lb, qs;
    int dt_in;
    const void *qi, *ki, *vi;
    const float *z, *bl, *qc, *kc, *vc, *A, *dt;
    float *cs, *S, *o;
    char *ws;
};

template <int D, int K, int DT>
static int launch_prefill(const PrefillArgs &a, hipStream_t st)
{
    const long nitems = (long)((a.T + CH - 1) / CH) * a.H;
    const size_t lds = (P1Lds<D>::FLOATS + 3 * D * 4 + D) * sizeof(float);
    static bool lds_ok = false;
    int ncu = 0, rc;
    if ((rc = allow_lds((const void *)kda_chunk_intra_act<D, K, DT>, lds, lds_ok))) return rc;
    if ((rc = cu_count(ncu))) return rc;
    const int grid = (int)(nitems < ncu ? nitems : ncu);
    hipLaunchKernelGGL((kda_chunk_intra_act<D, K, DT>), dim3(grid), dim3(P1_THREADS), lds, st, a.T,
                       a.H, a.qs, a.lb, a.qi, a.ki, a.vi, a.z, a.bl, a.qc, a.kc, a.vc, a.A, a.dt,
                       a.cs, a.ws);
    K3_LAUNCHED();
    // phase 2 also writes the outgoing conv history (the kernel above has read the incoming one)
    return launch_state<D>(a.T, a.H, a.ws, a.S, a.o, st, ConvOut{a.qi, a.ki, a.vi, a.cs, K, DT});
}

template <int D, int DT>
static int prefill_k(int K, const PrefillArgs &a, hipStream_t st)
{
    switch (K) {
    case 1: return launch_prefill<D, 1, DT>(a, st);
    case 2: return launch_prefill<D, 2, DT>(a, st);
    case 3: return launch_prefill<D, 3, DT>(a, st);
    case 4: return launch_prefill<D, 4, DT>(a, st);
    default: K3_FAIL(K3HIP_EUNSUPPORTED, "k3hip_kda_prefill: conv_k=%d not in 1..4", K);
    }
}

// Tokens per pass: all of T when the workspace holds every chunk of the sequence, otherwise
// the largest multiple of CH whose blocks fit in `avail` bytes (0: not even one chunk). The
// passes then run one after the other on the stream, S carried between them; chunk
// boundaries do not move, so the results are the same bits as one pass.
static long pass_tokens(long T, int H, int D, size_t avail)
{
    const size_t per_chunk = (size_t)H * (D == 128 ? Ws<128>::SIZE : Ws<64>::SIZE);
    const size_t chunks = avail / per_chunk;
    if ((long)chunks * CH >= T) return T;
    return (long)chunks * CH;
}

}  // namespace k3kda

using namespace k3kda;

extern "C" size_t k3hip_kda_chunk_workspace(int T, int H, int D, int chunk)
{
    if (T <= 0 || H <= 0 || chunk != CH) return 0;
    const size_t nch = ((size_t)T + CH - 1) / CH;
    if (D == 128) return nch * H * Ws<128>::SIZE;
    if (D == 64) return nch * H * Ws<64>::SIZE;
    return 0;
}

extern "C" int k3hip_kda_chunk(int T, int H, int D, int chunk, const float *q, const float *k,
                               const float *v, const float *g, const float *beta, float q_scale,
                               float *S, float *o, void *workspace, size_t workspace_bytes,
                               void *stream)
{
    clear_error();
    if (T < 0 || H < 0) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_chunk: T=%d H=%d", T, H);
    if (chunk != CH) K3_FAIL(K3HIP_EUNSUPPORTED, "k3hip_kda_chunk: chunk=%d (only 64)", chunk);
    if (D != 64 && D != 128) K3_FAIL(K3HIP_EUNSUPPORTED, "k3hip_kda_chunk: D=%d (64 or 128)", D);
    if (T == 0 || H == 0) return K3HIP_OK;
    if (!q || !k || !v || !g || !beta || !S || !o) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_chunk: NULL tensor");
    if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)g) & 15)
        K3_FAIL(K3HIP_EINVAL, "k3hip_kda_chunk: q, k, v, g must be 16-byte aligned");
    const long nch = ((long)T + CH - 1) / CH;
    if ((long)nch * H > 0x7fffffffL || H > 65535)
        K3_FAIL(K3HIP_EINVAL, "k3hip_kda_chunk: T=%d H=%d too large", T, H);
    const size_t need = k3hip_kda_chunk_workspace(T, H, D, chunk);
    hipStream_t st = as_stream(stream);
    StreamBuf own;
    char *ws = (char *)workspace;
    long pass = T;
    if (ws) {
        if ((uintptr_t)ws & 15) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_chunk: workspace must be 16-byte aligned");
        pass = pass_tokens(T, H, D, workspace_bytes);
        if (pass == 0)
            K3_FAIL(K3HIP_EINVAL, "k3hip_kda_chunk: workspace %zu bytes < %zu for one chunk", workspace_bytes,
                    k3hip_kda_chunk_workspace(CH, H, D, chunk));
    } else {
        int rc = stream_alloc(own, need, st);
        if (rc) return rc;
        ws = (char *)own.p;
    }
    const size_t P = (size_t)H * D;
    for (long t0 = 0; t0 < T; t0 += pass) {
        const int Ts = (int)std::min(pass, (long)T - t0);
        const size_t r = (size_t)t0 * P;
        const int rc = D == 128 ? launch_chunk<128>(Ts, H, q + r, k + r, v + r, g + r, beta + (size_t)t0 * H, q_scale,
                                                    S, o + r, ws, st)
                                : launch_chunk<64>(Ts, H, q + r, k + r, v + r, g + r, beta + (size_t)t0 * H, q_scale,
                                                   S, o + r, ws, st);
        if (rc) return rc;
    }
    return K3HIP_OK;
}

extern "C" int k3hip_kda_prefill(int T, int H, int D, int K, float gate_lb, int in_dtype,
                                 const void *q_in, const void *k_in, const void *v_in,
                                 const float *z, const float *b_logit, const float *q_conv,
                                 const float *k_conv, const float *v_conv, const float *A_log,
                                 const float *dt_bias, float *conv_state, float q_scale, float *S,
                                 float *o, void *workspace, size_t workspace_bytes, void *stream)
{
    clear_error();
    if (T < 0 || H < 0) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_prefill: T=%d H=%d", T, H);
    if (in_dtype != K3HIP_BF16 && in_dtype != K3HIP_F32)
        K3_FAIL(K3HIP_EINVAL, "k3hip_kda_prefill: in_dtype=%d", in_dtype);
    if (D != 64 && D != 128) K3_FAIL(K3HIP_EUNSUPPORTED, "k3hip_kda_prefill: D=%d (64 or 128)", D);
    if (K < 1 || K > 4) K3_FAIL(K3HIP_EUNSUPPORTED, "k3hip_kda_prefill: conv_k=%d not in 1..4", K);
    if (!(gate_lb < 0.0f && 15.0f * -gate_lb <= 80.0f))
        K3_FAIL(K3HIP_EUNSUPPORTED, "k3hip_kda_prefill: gate_lb=%g (needs -80/15 <= lb < 0)", gate_lb);
    if (T == 0 || H == 0) return K3HIP_OK;
    if (!q_in || !k_in || !v_in || !z || !b_logit || !q_conv || !k_conv || !v_conv || !A_log ||
        !dt_bias || !S || !o)
        K3_FAIL(K3HIP_EINVAL, "k3hip_kda_prefill: NULL tensor");
    if (((uintptr_t)q_in | (uintptr_t)k_in | (uintptr_t)v_in | (uintptr_t)z) & 15)
        K3_FAIL(K3HIP_EINVAL, "k3hip_kda_prefill: q_in, k_in, v_in, z must be 16-byte aligned");
    const long nch = ((long)T + CH - 1) / CH;
    if (nch * H > 0x7fffffffL || H > 65535 || (long)T * H * D > 0x7fffffffL * 4L)
        K3_FAIL(K3HIP_EINVAL, "k3hip_kda_prefill: T=%d H=%d too large", T, H);
    const size_t need = k3hip_kda_chunk_workspace(T, H, D, CH);
    const size_t P = (size_t)H * D;
    hipStream_t st = as_stream(stream);
    StreamBuf own;
    char *ws = (char *)workspace;
    long pass = T;
    float *cs = conv_state;
    if (ws) {
        if ((uintptr_t)ws & 15) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_prefill: workspace must be 16-byte aligned");
        pass = pass_tokens(T, H, D, workspace_bytes);
        if (pass < T && !cs && K > 1) {
            // several passes without a caller's history: the history between passes lives
            // at the start of the workspace, zeroed (a fresh sequence)
            const size_t hist = (3 * P * (K - 1) * sizeof(float) + 255) & ~(size_t)255;
            pass = workspace_bytes > hist ? pass_tokens(T, H, D, workspace_bytes - hist) : 0;
            if (pass) {
                cs = (float *)ws;
                ws += hist;
                int rc = zero_fill(cs, 3 * P * (K - 1), st);
                if (rc) return rc;
            }
        }
        if (pass == 0)
            K3_FAIL(K3HIP_EINVAL, "k3hip_kda_prefill: workspace %zu bytes < %zu for one chunk%s", workspace_bytes,
                    k3hip_kda_chunk_workspace(CH, H, D, CH), cs || K == 1 ? "" : " and the conv history");
    } else {
        int rc = stream_alloc(own, need, st);
        if (rc) return rc;
        ws = (char *)own.p;
    }
    const size_t esz = in_dtype == K3HIP_BF16 ? 2 : 4;
    for (long t0 = 0; t0 < T; t0 += pass) {
        // a pass reads the conv history the pass before it wrote (phase 2 writes the history
        // after the pass's last token into cs)
        const int Ts = (int)std::min(pass, (long)T - t0);
        const size_t r = (size_t)t0 * P;
        const PrefillArgs a{Ts, H, gate_lb, q_scale, in_dtype, (const char *)q_in + r * esz,
                            (const char *)k_in + r * esz, (const char *)v_in + r * esz, z + r,
                            b_logit + (size_t)t0 * H, q_conv, k_conv, v_conv, A_log, dt_bias, cs, S, o + r, ws};
        int rc;
        if (in_dtype == K3HIP_BF16) rc = D == 128 ? prefill_k<128, K3HIP_BF16>(K, a, st) : prefill_k<64, K3HIP_BF16>(K, a, st);
        else rc = D == 128 ? prefill_k<128, K3HIP_F32>(K, a, st) : prefill_k<64, K3HIP_F32>(K, a, st);
        if (rc) return rc;
    }
    return K3HIP_OK;
}
