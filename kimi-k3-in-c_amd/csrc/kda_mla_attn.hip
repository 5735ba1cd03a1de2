// SPDX-License-Identifier: Apache-2.0
// kda_mla_attn.hip - the attention of the absorbed MLA decode step in one pass over the
// compressed-latent cache, for gfx950.
//
// For sequence b and head h, with qcat_h = [W_UK_h^T q_nope_h, q_rope_h] and the cache rows
// cache_t = [latent_t, rope_t] (t < Tn):
//   p_t = softmax_t(scale * qcat_h . cache_t),   chat_h = sum_t p_t latent_t
// which is the reference's k3_mla_cached attention (src/core/k3_ops.c:321-424: fp32 scores
// times (nope+rope)^-0.5, max, exponentials, normalised weights, weighted sum of values) with
// kv_b absorbed. The cache (302 MB at 16 sequences x 8192 positions x 576 floats) dominates
// the bytes, so the kernel reads it exactly once, and everything else stays on the chip:
//
//  * A workgroup (8 waves, two per SIMD) owns one sequence and a contiguous range of
//    positions (~CUs/B ranges per sequence) and walks it in tiles of 16 positions (16
//    contiguous cache rows). Every thread loads its 16-byte units of a tile one iteration
//    ahead into registers, splits them into bf16 hi/lo and stages them row-major in LDS
//    (four tile buffers: the tile being scored, the two being summed, the next one).
//  * The two waves of a SIMD take different roles, so score products and weighted sums
//    share the SIMD's MFMA pipe instead of both waves running the same phase:
//      S waves (0-3), tile it, heads 16 w + (l & 15): scores^T (positions x heads) = cache
//        tile (16 x CW) . qcat^T on split-bf16 MFMA (16x16x32, cache rows read from LDS, the
//        q fragments of all 18 K-steps held in registers for the whole range; K-steps in
//        groups of three on three accumulators, so dependent MFMAs do not wait on each
//        other), then the online softmax in base 2: a reference max M per head (exchanged
//        between the 4 lanes of a head) that moves only when a score passes it by AT_LAZY,
//        per-lane partial sums; P (bf16 hi/lo) and the rescale factor 2^(M_old - M_new)
//        go to LDS;
//      U waves (4-7), latent channel tiles 8 (w - 4) .. + 7 for all heads, tiles it - 2 and
//        it - 1 at even iterations: chat^T (latent channels x heads) += latent^T . P on
//        split-bf16 MFMA with K = the pair's 32 positions (16x16x32, twice the rate of the
//        16-deep form), rescaled only when a max moved; the transposed latent fragments come
//        straight from the row-major tiles through ds_read_b64_tr_b16 (each fragment read by
//        one wave), and P in the score product's output layout.
//    One barrier per iteration: P of tile it and the staging of tile it + 1 are published.
//  * Each workgroup writes its unnormalised sums with (M, l); a second kernel merges the
//    ranges of a sequence (weights 2^(M_s - M*), the sums in a fixed order), divides by the
//    merged sum and writes chat directly as the bf16 hi/lo rows of the W_UV GEMM.
#include <math.h>

#include <algorithm>

#include "kda_internal.h"

namespace k3kda {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef s16x4 __attribute__((address_space(3))) *lds_s16x4_ptr;

constexpr int AT_T = 16;             // positions per tile
constexpr int AT_NT = 512;           // threads per workgroup: 8 waves, two per SIMD
constexpr int AT_MAXKS = 18;         // 32-channel K-steps of the scores (kv_lora + rope <= 576)
constexpr int AT_MAXCT = 32;         // 16-channel tiles of the latent (kv_lora <= 512)
constexpr int AT_MAXU = 5;           // 16-byte cache loads per thread per tile (kv_lora + rope <= 576)
constexpr int AT_NB = 4;             // staged tile buffers
constexpr int AT_UCT = AT_MAXCT / 4; // latent channel tiles per U wave
constexpr int AT_UPF = 2;            // channel tiles of transposed reads in flight (U waves)
constexpr int AT_MAXSPLIT = 64;      // position ranges per sequence
constexpr float AT_LOG2E = 1.4426950408889634f;
constexpr float AT_LAZY = 8.0f;      // log2 of the largest softmax weight before a rescale

// LDS: AT_NB buffers x {hi, lo} x [AT_T][AT_PR] bf16 (152 KB), then P and the rescale
// factors of two tiles (10 KB). Rows hold the 576 channels of the largest shape (smaller
// shapes are zero past their kv_lora + rope, so every shape runs the same products). The
// row pitch is 74 16-byte units and rows 8-15 hold their units in pairs swapped (column c
// at c ^ 8, at_col): the score product's 16-byte reads (16 rows, one unit) and the
// transposed 8-byte reads (per 32-lane pass 8 rows, two adjacent units) then both fall on
// 64 distinct banks. (With an unswizzled 73-unit pitch the transposed reads met 2-way and
// lost ~15% of CU cycles to bank conflicts; no plain pitch serves both patterns.)
constexpr int AT_PR = 32 * AT_MAXKS + 16;

__device__ __forceinline__ int at_col(int row, int col) { return col ^ ((row >> 3) << 3); }
constexpr size_t AT_PLANE = (size_t)AT_T * AT_PR;   // bf16
constexpr size_t AT_P = (size_t)AT_NB * 2 * AT_PLANE * 2;  // bytes: tiles; then P [2][4][64] x 16 B
constexpr size_t AT_A = AT_P + 2 * 4 * 64 * 16;              // rescale factors [2][4][64] fp32
constexpr size_t AT_LDS = AT_A + 2 * 4 * 64 * 4;

struct AtGeom {
    int H, CW, KL;
};

// Where the query rows come from: qcat[b][h] = [A2[b][h] + A2[B+b][h] (the hi and lo halves
// of the batched absorb GEMM, KL floats) | q_rope(b, h) (q [B][H][QH] at column QN)], formed
// while the q fragments are loaded (the same fp32 sums a separate qcat pass would store).
struct AtQ {
    const float *A2, *q;
    int B, QN, QH;
};

// The new position's cache row, written by the workgroup that owns the last range before it
// reads any cache row: the rmsnorm'd latent (weight w, double mean of squares,
// src/core/k3_ops.c:94-102) and the rope slot copied, from row b of src (stride ld). src ==
// nullptr: the row is already in the cache.
struct AtRow {
    const float *src;
    long ld;
    const float *w;
    float eps;
    int pos;
};

__device__ __forceinline__ void split2(float a, float b, bf16x2 &hi, bf16x2 &lo)
{
    hi = __builtin_convertvector(f2{a, b}, bf16x2);
    const uint32_t u = __builtin_bit_cast(uint32_t, hi);
    lo = __builtin_convertvector(f2{a - __uint_as_float(u << 16), b - __uint_as_float(u & 0xffff0000u)}, bf16x2);
}

// Workgroup (sp, b): positions [Tn sp / nsplit, Tn (sp + 1) / nsplit) of sequence b.
// Wave w: S role for w < 4 (head tile ht = w: heads 16 ht .. 16 ht + 15; lane l works for
// head h = 16 ht + (l & 15), kg = l >> 4 picks its K slice in the score product and its 4
// positions of each tile, 4 kg .. 4 kg + 3), U role otherwise (latent channel quarter
// w - 4, all head tiles). FULL: kv_lora + rope = 576, every staging unit of a row exists.
template <bool FULL>
__global__ __launch_bounds__(AT_NT) __attribute__((amdgpu_waves_per_eu(2, 2))) void mla_attn_kernel(
    AtGeom g, int Tn, int cap, int nsplit, float scale2, AtQ qs, AtRow nr,
    float *__restrict__ cache, float *__restrict__ pctx, float *__restrict__ pm, float *__restrict__ pl)
{
    extern __shared__ __attribute__((aligned(16))) uint16_t at_smem[];
    char *sbase = reinterpret_cast<char *>(at_smem);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int m = lane & 15, kg = lane >> 4, ht = w & 3;
    const bool isS = w < 4;
    const int sp = blockIdx.x, b = blockIdx.y;
    const int p0 = (int)((long)Tn * sp / nsplit), p1 = (int)((long)Tn * (sp + 1) / nsplit);
    const int ntile = (p1 - p0 + AT_T - 1) / AT_T;
    const int H = g.H, CW = FULL ? 32 * AT_MAXKS : g.CW, KL = g.KL;
    const int h = 16 * ht + m;
    const bool act = 16 * ht < H;   // wave-uniform: this wave has heads

    if (!FULL) {
        const int padw = 32 * AT_MAXKS - CW;
        for (int i = tid; i < 2 * AT_NB * AT_T * padw; i += AT_NT) {
            const int pl4 = i / (AT_T * padw), r = (i / padw) % AT_T, c = CW + i % padw;
            at_smem[pl4 * AT_PLANE + (size_t)r * AT_PR + at_col(r, c)] = 0;
        }
    }

    const int sr = tid >> 5, sq = 4 * (tid & 31);
    f4 R[AT_MAXU];
#pragma unroll
    for (int k = 0; k < AT_MAXU; k++) R[k] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    auto load_tile = [&](int tile) {
        const int tl = min(tile, ntile - 1);
        const int pos = min(p0 + AT_T * tl + sr, p1 - 1);
        const float *row = cache + ((size_t)b * cap + pos) * CW + sq;
#pragma unroll
        for (int k = 0; k < AT_MAXU; k++)
            if ((FULL && k < AT_MAXU - 1) || sq + 128 * k < CW) R[k] = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(row + 128 * k));
    };
    auto stage = [&](int buf) {
        uint16_t *hi = at_smem + (size_t)(2 * buf) * AT_PLANE + sr * AT_PR + at_col(sr, sq), *lo = hi + AT_PLANE;
#pragma unroll
        for (int k = 0; k < AT_MAXU; k++)
            if ((FULL && k < AT_MAXU - 1) || sq + 128 * k < CW) {
                bf16x2 h0, l0, h1, l1;
                split2(R[k].x, R[k].y, h0, l0);
                split2(R[k].z, R[k].w, h1, l1);
                *reinterpret_cast<uint2 *>(hi + 128 * k) = uint2{__builtin_bit_cast(uint32_t, h0), __builtin_bit_cast(uint32_t, h1)};
                *reinterpret_cast<uint2 *>(lo + 128 * k) = uint2{__builtin_bit_cast(uint32_t, l0), __builtin_bit_cast(uint32_t, l1)};
            }
    };

    // the workgroup of the last range writes the new position's row (Tn - 1 = pos) first;
    // tile 0 goes out before that unless it is the tile that holds the row
    const bool own_row = nr.src && sp == nsplit - 1;
    if (!own_row || ntile > 1) load_tile(0);
    if (own_row) {
        const float *src = nr.src + (size_t)b * nr.ld;
        double ss = 0.0;
        for (int n = tid; n < KL; n += AT_NT) {
            const double v = (double)src[n];
            ss += v * v;
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
        double *red = reinterpret_cast<double *>(at_smem);
        if (lane == 0) red[w] = ss;
        __syncthreads();
        ss = 0.0;
#pragma unroll
        for (int i = 0; i < AT_NT / 64; i++) ss += red[i];
        const float inv = (float)(1.0 / sqrt(ss / (double)KL + (double)nr.eps));
        float *dst = cache + ((size_t)b * cap + nr.pos) * CW;
        for (int n = tid; n < CW; n += AT_NT) {
            const float v = src[n];
            dst[n] = n < KL ? (nr.w[n] * v) * inv : v;
        }
        // the row is read back only by this workgroup's own cache loads (which go to L2: no
        // line of it was loaded here before): its stores complete, then every wave goes on
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
        __syncthreads();
    }
    if (own_row && ntile <= 1) load_tile(0);
    stage(0);
    load_tile(1);
    __syncthreads();
    // the U waves take the tiles in pairs (one K = 32 product per channel tile): an even
    // iteration closes the pair before it, so the loop runs to the even count at or past ntile
    const int itend = ntile + (ntile & 1);
    // iteration it: S scores tile it; at even it the U waves sum tiles it - 2 and it - 1;
    // every thread stages tile it + 1 (loaded one iteration earlier) and loads tile it + 2;
    // both roles pass one barrier per iteration
    if (isS) {
        // S: q B-fragments of all K-steps (channels 32 ks + 8 kg .. +7, column = head h), hi/lo
        bf16x8 qh[AT_MAXKS], ql[AT_MAXKS];
        {
#pragma unroll
            for (int i = 0; i < AT_MAXKS; i++) {
                float x[8];
                const int c = 32 * i + 8 * kg;
                const bool ok = h < H;
                const size_t bh = (size_t)b * H + (ok ? h : 0);
                const float *a2 = qs.A2 + bh * CW, *a2lo = a2 + (size_t)qs.B * H * CW;
                const float *qr = qs.q + bh * qs.QH + qs.QN - KL;
#pragma unroll
                for (int e = 0; e < 8; e += 4) {
                    const int cc = c + e;
                    f4 v = f4{0.0f, 0.0f, 0.0f, 0.0f};
                    if (ok && cc < CW) {
                        if (cc < KL) v = *reinterpret_cast<const f4 *>(a2 + cc) + *reinterpret_cast<const f4 *>(a2lo + cc);
                        else v = *reinterpret_cast<const f4 *>(qr + cc);
                    }
                    x[e] = v.x; x[e + 1] = v.y; x[e + 2] = v.z; x[e + 3] = v.w;
                }
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    bf16x2 hh, ll;
                    split2(x[e], x[e + 1], hh, ll);
                    qh[i][e] = hh[0]; qh[i][e + 1] = hh[1];
                    ql[i][e] = ll[0]; ql[i][e + 1] = ll[1];
                }
            }
        }
        float M = -INFINITY, lsum = 0.0f;   // head h over this lane's positions
        auto s_tile = [&](int it) {
            const int buf = it % AT_NB;
            const uint16_t *hi = at_smem + (size_t)(2 * buf) * AT_PLANE + m * AT_PR + at_col(m, 8 * kg);
            const uint16_t *lo = hi + AT_PLANE;
            // K-steps in groups of three, one accumulator each: each of the three split products
            // runs over the group's accumulators in turn (three independent chains hide the
            // ~40-cycle latency of a dependent MFMA); the next group's lo fragments are read once
            // this group's second product is issued, its hi fragments after the third
            constexpr int SG = 3;
            static_assert(AT_MAXKS % SG == 0, "K-step groups");
            bf16x8 rah[SG], ral[SG];
#pragma unroll
            for (int t = 0; t < SG; t++) {
                ral[t] = *reinterpret_cast<const bf16x8 *>(lo + 32 * t);
                rah[t] = *reinterpret_cast<const bf16x8 *>(hi + 32 * t);
            }
            __builtin_amdgcn_sched_barrier(0);
            f32x4 sa[SG];
#pragma unroll
            for (int t = 0; t < SG; t++) sa[t] = 0.0f;
#pragma unroll
            for (int k0 = 0; k0 < AT_MAXKS; k0 += SG) {
                const bool nxt = k0 + SG < AT_MAXKS;
#pragma unroll
                for (int t = 0; t < SG; t++)
                    sa[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ral[t], qh[k0 + t], sa[t], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int t = 0; t < SG; t++)
                    sa[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(rah[t], ql[k0 + t], sa[t], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                if (nxt) {
#pragma unroll
                    for (int t = 0; t < SG; t++) ral[t] = *reinterpret_cast<const bf16x8 *>(lo + 32 * (k0 + SG + t));
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int t = 0; t < SG; t++)
                    sa[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(rah[t], qh[k0 + t], sa[t], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                if (nxt) {
#pragma unroll
                    for (int t = 0; t < SG; t++) rah[t] = *reinterpret_cast<const bf16x8 *>(hi + 32 * (k0 + SG + t));
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            const f32x4 s = (sa[0] + sa[1]) + sa[2];
            const int t0 = p0 + AT_T * it + 4 * kg;
            float x[4], mt = -INFINITY;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                x[e] = t0 + e < p1 ? s[e] * scale2 : -INFINITY;
                mt = fmaxf(mt, x[e]);
            }
            mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
            mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
            // the reference max moves only when a score passes it by AT_LAZY (base 2): the
            // weights stay below 2^AT_LAZY and the sums are rescaled rarely; the ranges' merge
            // takes each range's reference max with its sums, so the result is the same
            const float mn = mt > M + AT_LAZY ? mt : M;
            const float alpha = __builtin_amdgcn_exp2f(M - mn);
            float p[4];
#pragma unroll
            for (int e = 0; e < 4; e++) p[e] = __builtin_amdgcn_exp2f(x[e] - mn);
            lsum = lsum * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
            M = mn;
            bf16x2 h01, l01, h23, l23;
            split2(p[0], p[1], h01, l01);
            split2(p[2], p[3], h23, l23);
            char *pb = sbase + AT_P + ((size_t)((it & 1) * 4 + ht) * 64 + lane) * 16;
            *reinterpret_cast<uint4 *>(pb) = uint4{__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23),
                                                   __builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23)};
            reinterpret_cast<float *>(sbase + AT_A)[((it & 1) * 4 + ht) * 64 + lane] = alpha;
        };
        for (int it = 0; it <= itend; it++) {
            if (act && it < ntile) s_tile(it);
            stage((it + 1) % AT_NB);   // past the last tile: a copy nothing reads
            load_tile(it + 2);
            __syncthreads();
        }
        lsum += __shfl_xor(lsum, 16, 64);
        lsum += __shfl_xor(lsum, 32, 64);
        if (act && h < H && kg == 0) {
            pm[((size_t)b * nsplit + sp) * H + h] = M;
            pl[((size_t)b * nsplit + sp) * H + h] = lsum;
        }
    } else {
        // U wave u = w - 4 owns latent channel tiles 8 u .. 8 u + 7 for all four head tiles:
        // acc[jj][g] = chat^T[channel 16 (8 u + jj) + 4 kg + e][head 16 g + m], so each latent
        // fragment is read from LDS by one wave only (a wave per head tile would read every
        // fragment four times and make the LDS the bound)
        const int u = w - 4;
        f32x4 acc[AT_UCT][4];
#pragma unroll
        for (int jj = 0; jj < AT_UCT; jj++)
#pragma unroll
            for (int g2 = 0; g2 < 4; g2++) acc[jj][g2] = 0.0f;
        // P operands per head tile g2. Lane (head 16 g2 + m, K slice kg) supplies positions
        // 4 (kg & 1) .. + 3 and 8 + 4 (kg & 1) .. + 3 of the pair's tile kg >> 1 (so that each
        // 32-lane half of a transposed read covers 8 rows of one half of the tile, on distinct
        // banks): the entries (hi01, hi23, lo01, lo23) of the head's S lanes kg & 1 and
        // 2 + (kg & 1). The lanes of the pair's first tile (kg < 2) read theirs one iteration
        // early: the S waves overwrite that P buffer in the pair's iteration.
        uint4 pa[4], pb[4];
        float al0[4];
        const int src0 = m + 16 * (kg & 1), src1 = src0 + 32;
        auto p_entry = [&](int t, int g2, int src) {
            return *reinterpret_cast<const uint4 *>(sbase + AT_P + ((size_t)((t & 1) * 4 + g2) * 64 + src) * 16);
        };
        auto alpha_of = [&](int t, int g2) {
            return reinterpret_cast<const float *>(sbase + AT_A)[((t & 1) * 4 + g2) * 64 + lane];
        };
        auto u_grab = [&](int t0) {
            // every read first, one wait
            float a[4];
            uint4 xa[4], xb[4];
#pragma unroll
            for (int g2 = 0; g2 < 4; g2++) {
                a[g2] = alpha_of(t0, g2);
                xa[g2] = p_entry(t0, g2, src0);
                xb[g2] = p_entry(t0, g2, src1);
            }
#pragma unroll
            for (int g2 = 0; g2 < 4; g2++) {
                const bool hg = 16 * g2 < H;   // head tiles without heads: weight zero
                al0[g2] = hg ? a[g2] : 1.0f;
                if (!(kg >> 1)) {
                    pa[g2] = hg ? xa[g2] : uint4{0, 0, 0, 0};
                    pb[g2] = hg ? xb[g2] : uint4{0, 0, 0, 0};
                }
            }
        };
        // tiles t0, t0 + 1 (the second may lie past the last tile: weight zero)
        auto u_pair = [&](int t0) {
            const int t1 = t0 + 1;
            const bool has1 = t1 < ntile;
            float a[4];
            uint4 xa[4], xb[4];
#pragma unroll
            for (int g2 = 0; g2 < 4; g2++) {
                a[g2] = alpha_of(t1, g2);
                xa[g2] = p_entry(t1, g2, src0);
                xb[g2] = p_entry(t1, g2, src1);
            }
            bf16x8 ph[4], pq[4];
#pragma unroll
            for (int g2 = 0; g2 < 4; g2++) {
                const bool hg = 16 * g2 < H, use1 = has1 && hg;
                const float al1 = use1 ? a[g2] : 1.0f;
                if (kg >> 1) {
                    pa[g2] = use1 ? xa[g2] : uint4{0, 0, 0, 0};
                    pb[g2] = use1 ? xb[g2] : uint4{0, 0, 0, 0};
                } else if (__ballot(al1 != 1.0f)) {
                    // acc a0 a1 + X0 (P0 a1) + X1 P1 = ((acc a0 + X0 P0) a1 + X1 P1)
                    float pv[8];
                    const uint32_t wh[4] = {pa[g2].x, pa[g2].y, pb[g2].x, pb[g2].y};
                    const uint32_t wl[4] = {pa[g2].z, pa[g2].w, pb[g2].z, pb[g2].w};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        pv[2 * e] = (__uint_as_float(wh[e] << 16) + __uint_as_float(wl[e] << 16)) * al1;
                        pv[2 * e + 1] = (__uint_as_float(wh[e] & 0xffff0000u) + __uint_as_float(wl[e] & 0xffff0000u)) * al1;
                    }
                    bf16x2 hh[4], ll[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) split2(pv[2 * e], pv[2 * e + 1], hh[e], ll[e]);
                    pa[g2] = uint4{__builtin_bit_cast(uint32_t, hh[0]), __builtin_bit_cast(uint32_t, hh[1]),
                                   __builtin_bit_cast(uint32_t, ll[0]), __builtin_bit_cast(uint32_t, ll[1])};
                    pb[g2] = uint4{__builtin_bit_cast(uint32_t, hh[2]), __builtin_bit_cast(uint32_t, hh[3]),
                                   __builtin_bit_cast(uint32_t, ll[2]), __builtin_bit_cast(uint32_t, ll[3])};
                }
                const float sc = al0[g2] * al1;
                if (__ballot(sc != 1.0f)) {
#pragma unroll
                    for (int jj = 0; jj < AT_UCT; jj++) acc[jj][g2] *= sc;
                }
                ph[g2] = __builtin_bit_cast(bf16x8, uint4{pa[g2].x, pa[g2].y, pb[g2].x, pb[g2].y});
                pq[g2] = __builtin_bit_cast(bf16x8, uint4{pa[g2].z, pa[g2].w, pb[g2].z, pb[g2].w});
            }
            const int buf = (t0 + (kg >> 1)) % AT_NB;
            const uint16_t *hi = at_smem + (size_t)(2 * buf) * AT_PLANE + 16 * AT_UCT * u, *lo = hi + AT_PLANE;
            const int tr0 = 4 * (kg & 1) + ((lane >> 2) & 3), tr1 = tr0 + 8;
            const int to0 = tr0 * AT_PR + at_col(tr0, 4 * (lane & 3)), to1 = tr1 * AT_PR + at_col(tr1, 4 * (lane & 3));
            auto rd = [&](const uint16_t *pl, int jj) {
                const s16x4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(pl + to0 + 16 * jj));
                const s16x4 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(pl + to1 + 16 * jj));
                return __builtin_bit_cast(bf16x8, uint4{__builtin_bit_cast(uint2, x0).x, __builtin_bit_cast(uint2, x0).y,
                                                        __builtin_bit_cast(uint2, x1).x, __builtin_bit_cast(uint2, x1).y});
            };
            // per channel tile: each of the three split products over the four head tiles (four
            // independent chains hide the ~40-cycle latency of a dependent MFMA); the latent
            // fragments are read AT_UPF channel tiles ahead
            bf16x8 rh[AT_UPF], rl[AT_UPF];
#pragma unroll
            for (int jj = 0; jj < AT_UPF; jj++) {
                rl[jj] = rd(lo, jj);
                rh[jj] = rd(hi, jj);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int jj = 0; jj < AT_UCT; jj++) {
                const bf16x8 ah = rh[jj % AT_UPF], al = rl[jj % AT_UPF];
#pragma unroll
                for (int g2 = 0; g2 < 4; g2++)
                    acc[jj][g2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, ph[g2], acc[jj][g2], 0, 0, 0);
#pragma unroll
                for (int g2 = 0; g2 < 4; g2++)
                    acc[jj][g2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, pq[g2], acc[jj][g2], 0, 0, 0);
#pragma unroll
                for (int g2 = 0; g2 < 4; g2++)
                    acc[jj][g2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, ph[g2], acc[jj][g2], 0, 0, 0);
                if (jj + AT_UPF < AT_UCT) {
                    rl[jj % AT_UPF] = rd(lo, jj + AT_UPF);
                    rh[jj % AT_UPF] = rd(hi, jj + AT_UPF);
                }
                __builtin_amdgcn_sched_barrier(0);   // keep the reads ahead (the scheduler sinks them)
            }
        };
        const bool uact = 16 * AT_UCT * u < KL;   // wave-uniform: this wave has latent channels
        for (int it = 0; it <= itend; it++) {
            if (uact && (it & 1)) u_grab(it - 1);
            if (uact && it >= 2 && !(it & 1)) u_pair(it - 2);
            stage((it + 1) % AT_NB);
            load_tile(it + 2);
            __syncthreads();
        }
        if (uact) {
#pragma unroll
            for (int g2 = 0; g2 < 4; g2++) {
                const int hh = 16 * g2 + m;
                if (hh >= H) continue;
                float *outp = pctx + (((size_t)b * nsplit + sp) * H + hh) * KL + 4 * kg;
#pragma unroll
                for (int jj = 0; jj < AT_UCT; jj++) {
                    const int j = AT_UCT * u + jj;
                    if (16 * j < KL)
                        *reinterpret_cast<f4 *>(outp + 16 * j) = f4{acc[jj][g2][0], acc[jj][g2][1], acc[jj][g2][2], acc[jj][g2][3]};
                }
            }
        }
    }
}

// Block (h, b): merge the nsplit ranges of sequence b, head h, in range order; write
// chat = sum / l as bf16 hi (row b) and lo (row B + b) of ch2 [2B][H KL]. Thread i covers
// channels 4i .. 4i + 3 (and every 4 * blockDim further).
__global__ __launch_bounds__(128) void mla_attn_merge_kernel(int B, int H, int KL, int nsplit,
                                                             const float *__restrict__ pctx,
                                                             const float *__restrict__ pm,
                                                             const float *__restrict__ pl,
                                                             uint16_t *__restrict__ ch2)
{
    __shared__ float sw[AT_MAXSPLIT];
    __shared__ float sl;
    const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
    const float *mrow = pm + (size_t)b * nsplit * H + h, *lrow = pl + (size_t)b * nsplit * H + h;
    if (tid < 64) {
        const float mv = tid < nsplit ? mrow[(size_t)tid * H] : -INFINITY;
        float mx = mv;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        const float wv = tid < nsplit ? __builtin_amdgcn_exp2f(mv - mx) : 0.0f;
        if (tid < nsplit) sw[tid] = wv;
        float lv = tid < nsplit ? wv * lrow[(size_t)tid * H] : 0.0f;
        // the weighted sums of the ranges, added in a fixed tree into lane 0
        for (int o = 1; o < 64; o <<= 1) {
            const float t = __shfl_down(lv, o, 64);
            if ((tid & (2 * o - 1)) == 0) lv += t;
        }
        if (tid == 0) sl = lv;
    }
    __syncthreads();
    const float rl = 1.0f / sl;
    const size_t BN = (size_t)B * H * KL;
    for (int c = 4 * tid; c < KL; c += 4 * blockDim.x) {
        f4 a = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 8
        for (int s = 0; s < nsplit; s++)
            a += sw[s] * *reinterpret_cast<const f4 *>(pctx + (((size_t)b * nsplit + s) * H + h) * KL + c);
        const size_t i = ((size_t)b * H + h) * KL + c;
        const float v[4] = {a.x * rl, a.y * rl, a.z * rl, a.w * rl};
        uint16_t hv[4], lv[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            hv[e] = f2bf(v[e]);
            lv[e] = f2bf(v[e] - bf2f(hv[e]));
        }
        *reinterpret_cast<uint2 *>(ch2 + i) = uint2{hv[0] | ((uint32_t)hv[1] << 16), hv[2] | ((uint32_t)hv[3] << 16)};
        *reinterpret_cast<uint2 *>(ch2 + BN + i) = uint2{lv[0] | ((uint32_t)lv[1] << 16), lv[2] | ((uint32_t)lv[3] << 16)};
    }
}

// o = (chat . W_UV_h^T) * sigmoid(g) per (head h, block of up to 16 sequences) from the merged
// chat's bf16 hi / lo rows (ch2 [2B][H KL]): both halves against the bf16 weight into one fp32
// accumulator on 16x16x32 MFMA (the products exact, the sums fp32), then the output gate
// sigmoid(g) (the reference's 1 / (1 + expf(-g)), src/core/k3_ops.c:105), written as fp32
// rows of o [B][H VH] for o_proj. Replaces a head-batched W_UV GEMM and a gate kernel (two
// launches and the GEMM's two fp32 output planes). W_UV_h = rows h (QN + VH) + QN .. + VH of
// kvb [H (QN + VH)][KL]. zout[0 .. zn) = 0 on the way (may be nullptr) for an o_proj that
// adds its two K-range partials there.
constexpr int AO_NT = 512;                 // 8 waves, one 16-column tile of o each (VH <= 128)
constexpr int AO_KP = 32 * 16 + 8;         // LDS row pitch (bf16): 16 bytes of skew per row
__global__ __launch_bounds__(AO_NT) void mla_attn_out_kernel(int B, int H, int KL, int QN, int VH,
                                                            const uint16_t *__restrict__ ch2,
                                                            const uint16_t *__restrict__ kvb,
                                                            const float *__restrict__ g, long ldg,
                                                            float *__restrict__ o, float *__restrict__ zout, size_t zn)
{
    __shared__ __attribute__((aligned(16))) uint16_t chh[16 * AO_KP], chl[16 * AO_KP];
    const int h = blockIdx.x, b0 = blockIdx.y * 16, nb = min(16, B - b0), tid = threadIdx.x;
    const int lane = tid & 63, wv = tid >> 6;
    const int r16 = lane & 15, kq = lane >> 4;
    const int KLr = (KL + 31) & ~31;
    // this wave's weight fragments (column tile wv of o, every K-step) and gate logits are
    // requested first, with the chat rows, so the step waits for memory once
    const uint16_t *Wuv = kvb + ((size_t)h * (QN + VH) + QN) * KL;   // [VH][KL]
    const int n = wv * 16 + r16;
    const bool nok = n < VH;
    const uint16_t *wrow = Wuv + (size_t)(nok ? n : 0) * KL;
    bf16x8 wf[AT_MAXCT / 2];
#pragma unroll
    for (int ks = 0; ks < AT_MAXCT / 2; ks++) {
        const int k = 32 * ks + 8 * kq;
        wf[ks] = bf16x8{};
        if (nok && k < KL) wf[ks] = *reinterpret_cast<const bf16x8 *>(wrow + k);
    }
    float gv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (g && nok)
#pragma unroll
        for (int e = 0; e < 4; e++)
            if (4 * kq + e < nb) gv[e] = g[(size_t)(b0 + 4 * kq + e) * ldg + (size_t)h * VH + n];
    // the block's chat rows (hi and lo) into LDS, 8 bf16 per thread and pass; rows past nb and
    // channels past KL are zero
    const size_t BN = (size_t)B * H * KL;
    for (int it = tid; it < 16 * (KLr / 8); it += AO_NT) {
        const int r = it / (KLr / 8), c = 8 * (it % (KLr / 8));
        uint4 vh = {0, 0, 0, 0}, vl = {0, 0, 0, 0};
        if (r < nb && c < KL) {
            const size_t i = ((size_t)(b0 + r) * H + h) * KL + c;
            vh = *reinterpret_cast<const uint4 *>(ch2 + i);
            vl = *reinterpret_cast<const uint4 *>(ch2 + BN + i);
        }
        *reinterpret_cast<uint4 *>(chh + r * AO_KP + c) = vh;
        *reinterpret_cast<uint4 *>(chl + r * AO_KP + c) = vl;
    }
    if (zout) {
        const size_t nwg = (size_t)gridDim.x * gridDim.y, id = (size_t)blockIdx.y * gridDim.x + h;
        const size_t per = (zn + nwg - 1) / nwg, z0 = id * per, z1 = min(zn, z0 + per);
        for (size_t i = z0 + tid; i < z1; i += AO_NT) zout[i] = 0.0f;
    }
    __syncthreads();
    if (wv * 16 >= VH) return;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < AT_MAXCT / 2; ks++) {
        if (32 * ks >= KLr) break;
        const int k = 32 * ks + 8 * kq;
        const bf16x8 ah = *reinterpret_cast<const bf16x8 *>(chh + r16 * AO_KP + k);
        const bf16x8 al = *reinterpret_cast<const bf16x8 *>(chl + r16 * AO_KP + k);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, wf[ks], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, wf[ks], acc, 0, 0, 0);
    }
    // C layout: lane holds rows 4 kq + e (sequences), column r16 (value channel n)
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int r = 4 * kq + e;
        if (r >= nb || !nok) continue;
        float v = acc[e];
        if (g) v *= 1.0f / (1.0f + expf(-gv[e]));
        o[(size_t)(b0 + r) * H * VH + (size_t)h * VH + n] = v;
    }
}

int at_cus()
{
    static int n = 0;
    if (!n) {
        int dev = 0, c = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && c > 0)
            n = c;
        else
            n = 256;
    }
    return n;
}

bool at_geom(int H, int KL, int CW, AtGeom &g)
{
    if (H <= 0 || H > 64 || KL <= 0 || (KL % 16) || KL > 16 * AT_MAXCT || CW < KL || (CW % 4) ||
        CW > 32 * AT_MAXKS)
        return false;
    g.H = H;
    g.CW = CW;
    g.KL = KL;
    return true;
}

int at_nsplit(int B, int Tn)
{
    return std::min({AT_MAXSPLIT, std::max(1, (at_cus() + B - 1) / B), std::max(1, Tn / AT_T)});
}

}  // namespace

size_t mla_attention_ws_bytes(int B, int H, int KL, int Tn)
{
    const int nsplit = at_nsplit(B, Tn);
    const size_t r = (size_t)B * nsplit * H;
    return ((r * KL * 4 + 255) & ~(size_t)255) + 2 * ((r * 4 + 255) & ~(size_t)255);
}

bool mla_attention_supported(int H, int KL, int CW)
{
    AtGeom g;
    return at_geom(H, KL, CW, g);
}

int mla_attention(int B, int H, int KL, int CW, int Tn, int cap, float scale, const float *A2, const float *q,
                  int QN, float *cache, const float *lat, long ldlat, const float *lat_w, float lat_eps,
                  const uint16_t *kvb, int VH, const float *gate, long ldg, float *o, float *zout, size_t zn,
                  uint16_t *ch2, void *ws, size_t ws_bytes, hipStream_t st)
{
    AtGeom g;
    if (!at_geom(H, KL, CW, g))
        K3_FAIL(K3HIP_EUNSUPPORTED, "mla attention: heads=%d kv_lora=%d kv_lora+rope=%d outside the fused kernel", H, KL, CW);
    if (B <= 0 || Tn <= 0 || Tn > cap) K3_FAIL(K3HIP_EINVAL, "mla attention: B=%d Tn=%d cap=%d", B, Tn, cap);
    const int nsplit = at_nsplit(B, Tn);
    const size_t need = mla_attention_ws_bytes(B, H, KL, Tn);
    const int QH = QN + (CW - KL);
    if (!ws || ws_bytes < need || ((uintptr_t)ws & 255) || ((uintptr_t)cache & 15) || ((uintptr_t)A2 & 15) ||
        ((uintptr_t)q & 15) || (QN & 3) || (KL & 7) || ((uintptr_t)kvb & 15) || ((uintptr_t)ch2 & 15) ||
        VH < 1 || VH > 16 * (AO_NT / 64))
        K3_FAIL(K3HIP_EINVAL, "mla attention: workspace %zu < %zu bytes, or a misaligned buffer", ws_bytes, need);
    const AtQ qs{A2, q, B, QN, QH};
    const AtRow nr{lat, ldlat, lat_w, lat_eps, Tn - 1};
    const size_t r = (size_t)B * nsplit * H;
    float *pctx = (float *)ws;
    float *pm = (float *)((char *)ws + ((r * KL * 4 + 255) & ~(size_t)255));
    float *pl = (float *)((char *)pm + ((r * 4 + 255) & ~(size_t)255));
    static bool attr = false;
    if (!attr) {
        K3_HIP(hipFuncSetAttribute((const void *)mla_attn_kernel<true>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                   (int)AT_LDS));
        K3_HIP(hipFuncSetAttribute((const void *)mla_attn_kernel<false>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                   (int)AT_LDS));
        attr = true;
    }
    if (CW == 32 * AT_MAXKS)
        hipLaunchKernelGGL(mla_attn_kernel<true>, dim3(nsplit, B), dim3(AT_NT), AT_LDS, st, g, Tn, cap, nsplit,
                           scale * AT_LOG2E, qs, nr, cache, pctx, pm, pl);
    else
        hipLaunchKernelGGL(mla_attn_kernel<false>, dim3(nsplit, B), dim3(AT_NT), AT_LDS, st, g, Tn, cap, nsplit,
                           scale * AT_LOG2E, qs, nr, cache, pctx, pm, pl);
    K3_LAUNCHED();
    hipLaunchKernelGGL(mla_attn_merge_kernel, dim3(H, B), dim3(128), 0, st, B, H, KL, nsplit, pctx, pm, pl, ch2);
    K3_LAUNCHED();
    hipLaunchKernelGGL(mla_attn_out_kernel, dim3(H, (B + 15) / 16), dim3(AO_NT), 0, st, B, H, KL, QN, VH, ch2, kvb,
                       gate, ldg, o, zout, zn);
    K3_LAUNCHED();
    return K3HIP_OK;
}

}  // namespace k3kda
