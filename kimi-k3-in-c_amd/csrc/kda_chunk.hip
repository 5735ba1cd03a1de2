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
// MFMA operands needs a pivot. Row block a (16 rows) uses the pivot p = 16a: the row
// factor e^(G_t - G_p) <= 1, the column factor e^(G_p - G_s) is <= 1 for s < p and at
// most e^(15 |gate_lb|) inside the block. The host only takes this path when
// 15 |gate_lb| <= 80, so every factor is a normal fp32 / bf16 number.
//
// Precision. Every product whose operands are not exact bf16 is a split-bf16 product:
// x = hi + lo (both bf16), a.b ~ ah.bh + ah.bl + al.bh with fp32 accumulation, i.e. about
// 2^-17 relative per product. The 16x16 block products of the inverse use the fp32 MFMA.
//
// Phase 1 (kda_chunk_intra) is parallel over (chunk, head): everything that does not
// depend on the state. Phase 2 (kda_chunk_state) walks the chunks in order, one workgroup
// per (head, 16-column tile of S): value columns of S are independent of each other, so
// the tiles never exchange data. Its blocks are mapped so that all tiles of one head sit
// on one XCD and share that XCD's L2 copy of the phase-1 operands.
#include "kda_internal.h"

namespace k3kda {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int CH = 64;     // chunk length
constexpr int SB = 16;     // sub-block (MFMA tile) edge
constexpr int NT2 = 16;    // columns of S per phase-2 workgroup

// Per-(chunk, head) workspace block, in floats.
template <int D> struct WsLayout {
    static constexpr size_t W = 0;                   // [64][D]   Tm beta K e^G
    static constexpr size_t U = W + (size_t)CH * D;  // [64][D]   Tm beta V
    static constexpr size_t Q = U + (size_t)CH * D;  // [64][D]   q e^G (q scaled)
    static constexpr size_t KT = Q + (size_t)CH * D; // [D][64]   (k e^(G_last - G))^T
    static constexpr size_t A = KT + (size_t)CH * D; // [64][64]  A_qk, zero above the diagonal
    static constexpr size_t GL = A + (size_t)CH * CH;// [D]       e^G_last
    static constexpr size_t SIZE = GL + D;
};

__device__ __forceinline__ void split8(const float (&x)[8], bf16x8 &hi, bf16x8 &lo)
{
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const __bf16 h = (__bf16)x[e];
        hi[e] = h;
        lo[e] = (__bf16)(x[e] - (float)h);
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

// --------------------------------------------------------------- phase 1 ----
// LDS: G, K, V [64][D+4]; A, Tm [64][68]; beta [64]; Y [4][16][17].
template <int D> struct P1Lds {
    static constexpr int PD = D + 4;
    static constexpr int PA = CH + 4;
    static constexpr size_t G = 0;
    static constexpr size_t K = G + (size_t)CH * PD;
    static constexpr size_t V = K + (size_t)CH * PD;
    static constexpr size_t A = V + (size_t)CH * PD;
    static constexpr size_t TM = A + (size_t)CH * PA;
    static constexpr size_t B = TM + (size_t)CH * PA;
    static constexpr size_t Y = B + CH;
    static constexpr size_t FLOATS = Y + 4 * 16 * 17;
};

template <int D>
__global__ __launch_bounds__(256) void kda_chunk_intra(int T, int H, float qs,
                                                       const float *__restrict__ q,
                                                       const float *__restrict__ k,
                                                       const float *__restrict__ v,
                                                       const float *__restrict__ g,
                                                       const float *__restrict__ beta,
                                                       float *__restrict__ ws)
{
    using L = P1Lds<D>;
    using WL = WsLayout<D>;
    constexpr int PD = L::PD, PA = L::PA;
    constexpr int KSI = D / 32;   // K-steps over channels
    extern __shared__ float lds[];
    float *sG = lds + L::G, *sK = lds + L::K, *sV = lds + L::V;
    float *sA = lds + L::A, *sT = lds + L::TM, *sB = lds + L::B, *sY = lds + L::Y;

    const int c = blockIdx.x, h = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int t0 = c * CH;
    const int Tc = min(CH, T - t0);
    const size_t P = (size_t)H * D;
    float *blk = ws + ((size_t)c * H + h) * WL::SIZE;

    // (1) stage g, k, v (zero past the end of the sequence), beta; clear A and Tm
    for (int e = tid; e < CH * D / 4; e += 256) {
        const int t = e / (D / 4), i4 = (e % (D / 4)) * 4;
        f4 gv = 0.0f, kv = 0.0f, vv = 0.0f;
        if (t < Tc) {
            const size_t at = (size_t)(t0 + t) * P + (size_t)h * D + i4;
            gv = *reinterpret_cast<const f4 *>(g + at);
            kv = *reinterpret_cast<const f4 *>(k + at);
            vv = *reinterpret_cast<const f4 *>(v + at);
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            sG[t * PD + i4 + u] = gv[u];
            sK[t * PD + i4 + u] = kv[u];
            sV[t * PD + i4 + u] = vv[u];
        }
    }
    for (int e = tid; e < CH * PA; e += 256) {
        sA[e] = 0.0f;
        sT[e] = 0.0f;
    }
    if (tid < CH) sB[tid] = tid < Tc ? beta[(size_t)(t0 + tid) * H + h] : 0.0f;
    __syncthreads();

    // (2) G = cumulative sum of g down the chunk, per channel (padded rows add 0)
    if (tid < D) {
        float run = 0.0f;
#pragma unroll 16
        for (int t = 0; t < CH; t++) {
            run += sG[t * PD + tid];
            sG[t * PD + tid] = run;
        }
    }
    __syncthreads();

    const int m = lane & 15, kg = lane >> 4;

    // (3) A_kk (to LDS, times beta_t, strictly lower) and A_qk (to the workspace, lower with
    //     the diagonal) for every 16x16 block (a, b), b <= a; blocks above are zero.
    for (int job = w; job < 16; job += 4) {
        const int a = job >> 2, b = job & 3;
        float *gA = blk + WL::A;
        if (b > a) {   // zero block of A_qk
#pragma unroll
            for (int e = 0; e < 4; e++)
                gA[(size_t)(SB * a + 4 * kg + e) * CH + SB * b + m] = 0.0f;
            continue;
        }
        const int p = SB * a;        // pivot row
        const int t = SB * a + m;    // A-operand row (token t)
        const int s = SB * b + m;    // B-operand row (token s)
        f32x4 akk = 0.0f, aqk = 0.0f;
        const size_t qrow = (size_t)(t0 + t) * P + (size_t)h * D;
#pragma unroll
        for (int ks = 0; ks < KSI; ks++) {
            const int i0 = 32 * ks + 8 * kg;
            float lk[8], lq[8], r[8], qv[8];
            if (t < Tc) load8(qv, q + qrow + i0);
            else {
#pragma unroll
                for (int e = 0; e < 8; e++) qv[e] = 0.0f;
            }
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float gp = sG[p * PD + i0 + e];
                const float ft = expf(sG[t * PD + i0 + e] - gp);
                lk[e] = sK[t * PD + i0 + e] * ft;
                lq[e] = (qv[e] * qs) * ft;
                r[e] = sK[s * PD + i0 + e] * expf(gp - sG[s * PD + i0 + e]);
            }
            bf16x8 kh, kl, qh, ql, rh, rl;
            split8(lk, kh, kl);
            split8(lq, qh, ql);
            split8(r, rh, rl);
            akk = mma3(akk, kh, kl, rh, rl);
            aqk = mma3(aqk, qh, ql, rh, rl);
        }
        float *gAq = blk + WL::A;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int tt = SB * a + 4 * kg + e, ss = SB * b + m;
            sA[tt * PA + ss] = ss < tt ? akk[e] * sB[tt] : 0.0f;
            gAq[(size_t)tt * CH + ss] = ss <= tt ? aqk[e] : 0.0f;
        }
    }
    __syncthreads();

    // (4a) diagonal blocks of Tm = (I + A)^-1: wave w inverts block w by forward
    //      substitution; lane s < 16 owns column s and keeps it in registers.
    if (lane < SB) {
        const int s = lane, o = SB * w;
        float col[SB];
#pragma unroll
        for (int t = 0; t < SB; t++) {
            float val = (t == s) ? 1.0f : 0.0f;
            if (t > s) {
                float acc = sA[(o + t) * PA + o + s];
#pragma unroll
                for (int r = 0; r < t; r++)
                    if (r > s) acc += sA[(o + t) * PA + o + r] * col[r];
                val = -acc;
            }
            col[t] = val;
            sT[(o + t) * PA + o + s] = val;
        }
    }
    __syncthreads();

    // (4b) off-diagonal blocks, by distance d = a - b:
    //      Tm_ab = -Tm_aa * sum_{c=b}^{a-1} A_ac Tm_cb   (fp32 MFMA, exact-width products)
    for (int d = 1; d < 4; d++) {
        const bool act = w < 4 - d;
        const int a = w + d, b = w;
        float *Yw = sY + w * 16 * 17;
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

    // (5) W = Tm (beta K e^G), U = Tm (beta V); wave w takes column tiles w, w+4, ...
    for (int nt = w; nt < D / SB; nt += 4) {
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
                xk[e] = (bs * sK[s * PD + n0 + m]) * expf(sG[s * PD + n0 + m]);
                xv[e] = bs * sV[s * PD + n0 + m];
            }
            bf16x8 kh, kl, vh, vl;
            split8(xk, kh, kl);
            split8(xv, vh, vl);
#pragma unroll
            for (int a = 0; a < 4; a++) {
                if (a < 2 * ks) continue;   // Tm rows of block a vanish past column 16a+15
                float tv[8];
#pragma unroll
                for (int e = 0; e < 8; e++) tv[e] = sT[(SB * a + m) * PA + 32 * ks + 8 * kg + e];
                bf16x8 th, tl;
                split8(tv, th, tl);
                aw[a] = mma3(aw[a], th, tl, kh, kl);
                au[a] = mma3(au[a], th, tl, vh, vl);
            }
        }
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int t = SB * a + 4 * kg + e;
                blk[WL::W + (size_t)t * D + n0 + m] = aw[a][e];
                blk[WL::U + (size_t)t * D + n0 + m] = au[a][e];
            }
    }

    // (6) elementwise operands: q e^G (scaled), (k e^(G_last - G))^T, e^G_last
    for (int e = tid; e < CH * D; e += 256) {
        const int t = e / D, i = e % D;
        float val = 0.0f;
        if (t < Tc) val = (q[(size_t)(t0 + t) * P + (size_t)h * D + i] * qs) * expf(sG[t * PD + i]);
        blk[WL::Q + e] = val;
    }
    for (int e = tid; e < CH * D; e += 256) {
        const int i = e / CH, s = e % CH;
        blk[WL::KT + e] = sK[s * PD + i] * expf(sG[(CH - 1) * PD + i] - sG[s * PD + i]);
    }
    if (tid < D) blk[WL::GL + tid] = expf(sG[(CH - 1) * PD + tid]);
}

// --------------------------------------------------------------- phase 2 ----
template <int D>
__global__ __launch_bounds__(256) void kda_chunk_state(int T, int H, const float *__restrict__ ws,
                                                       float *__restrict__ S,
                                                       float *__restrict__ o)
{
    using WL = WsLayout<D>;
    constexpr int NTILE = D / NT2;       // column tiles per head
    constexpr int RT = D / 64;           // 16-row tiles of S per wave
    constexpr int KSI = D / 32;
    constexpr int PS = 18;               // LDS pitch (conflict-free B-operand reads)
    __shared__ float sS[D * PS];
    __shared__ float sW[CH * PS];

    // XCD-aware: block b runs on XCD b % 8; give each XCD whole heads.
    const int nb = gridDim.x, b = blockIdx.x;
    int idx = b;
    if (nb % 8 == 0) idx = (b % 8) * (nb / 8) + b / 8;
    const int h = idx / NTILE, j0 = (idx % NTILE) * NT2;
    if (h >= H) return;

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int m = lane & 15, kg = lane >> 4;
    const size_t P = (size_t)H * D;
    float *Sh = S + (size_t)h * D * D;
    const int nch = (T + CH - 1) / CH;

    f32x4 accS[RT];
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int e = 0; e < 4; e++) accS[r][e] = Sh[(size_t)(64 * r + 16 * w + 4 * kg + e) * D + j0 + m];

    for (int c = 0; c < nch; c++) {
        const float *blk = ws + ((size_t)c * H + h) * WL::SIZE;
        const int t0 = c * CH;
        // (a) S tile -> LDS (B-operand source)
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int e = 0; e < 4; e++) sS[(64 * r + 16 * w + 4 * kg + e) * PS + m] = accS[r][e];
        __syncthreads();

        // (b) rows 16w..16w+15: Vn = U - W S, O = Q S
        f32x4 aw = 0.0f, ao = 0.0f;
#pragma unroll
        for (int ks = 0; ks < KSI; ks++) {
            float wv[8], qv[8], sv[8];
            load8(wv, blk + WL::W + (size_t)(16 * w + m) * D + 32 * ks + 8 * kg);
            load8(qv, blk + WL::Q + (size_t)(16 * w + m) * D + 32 * ks + 8 * kg);
#pragma unroll
            for (int e = 0; e < 8; e++) sv[e] = sS[(32 * ks + 8 * kg + e) * PS + m];
            bf16x8 wh, wl, qh, ql, sh, sl;
            split8(wv, wh, wl);
            split8(qv, qh, ql);
            split8(sv, sh, sl);
            aw = mma3(aw, wh, wl, sh, sl);
            ao = mma3(ao, qh, ql, sh, sl);
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int t = 16 * w + 4 * kg + e;
            sW[t * PS + m] = blk[WL::U + (size_t)t * D + j0 + m] - aw[e];
        }
        __syncthreads();

        // (c) O += A_qk Vn over the columns s <= t (K-steps of 32)
        bf16x8 vh[2], vl[2];
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            float vv[8];
#pragma unroll
            for (int e = 0; e < 8; e++) vv[e] = sW[(32 * ks + 8 * kg + e) * PS + m];
            split8(vv, vh[ks], vl[ks]);
        }
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            if (ks == 1 && w < 2) continue;
            float av[8];
            load8(av, blk + WL::A + (size_t)(16 * w + m) * CH + 32 * ks + 8 * kg);
            bf16x8 ah, al;
            split8(av, ah, al);
            ao = mma3(ao, ah, al, vh[ks], vl[ks]);
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int t = 16 * w + 4 * kg + e;
            if (t0 + t < T) o[(size_t)(t0 + t) * P + (size_t)h * D + j0 + m] = ao[e];
        }

        // (d) S = diag(e^G_last) S + (K e^(G_last - G))^T Vn
#pragma unroll
        for (int r = 0; r < RT; r++) {
            const int i0 = 64 * r + 16 * w;
#pragma unroll
            for (int e = 0; e < 4; e++) accS[r][e] *= blk[WL::GL + i0 + 4 * kg + e];
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                float kv[8];
                load8(kv, blk + WL::KT + (size_t)(i0 + m) * CH + 32 * ks + 8 * kg);
                bf16x8 kh, kl;
                split8(kv, kh, kl);
                accS[r] = mma3(accS[r], kh, kl, vh[ks], vl[ks]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int e = 0; e < 4; e++) Sh[(size_t)(64 * r + 16 * w + 4 * kg + e) * D + j0 + m] = accS[r][e];
}

bool chunk_ready() { return true; }

template <int D>
static int launch_chunk(int T, int H, const float *q, const float *k, const float *v,
                        const float *g, const float *beta, float qs, float *S, float *o,
                        float *ws, hipStream_t st)
{
    const int nch = (T + CH - 1) / CH;
    const size_t lds = P1Lds<D>::FLOATS * sizeof(float);
    static bool attr_set = false;
    if (!attr_set) {
        K3_HIP(hipFuncSetAttribute((const void *)kda_chunk_intra<D>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        attr_set = true;
    }
    hipLaunchKernelGGL((kda_chunk_intra<D>), dim3(nch, H), dim3(256), lds, st, T, H, qs, q, k, v, g,
                       beta, ws);
    K3_LAUNCHED();
    hipLaunchKernelGGL((kda_chunk_state<D>), dim3(H * (D / NT2)), dim3(256), 0, st, T, H, ws, S, o);
    K3_LAUNCHED();
    return K3HIP_OK;
}

}  // namespace k3kda

using namespace k3kda;

extern "C" size_t k3hip_kda_chunk_workspace(int T, int H, int D, int chunk)
{
    if (T <= 0 || H <= 0 || chunk != CH) return 0;
    const size_t nch = ((size_t)T + CH - 1) / CH;
    if (D == 128) return nch * H * WsLayout<128>::SIZE * sizeof(float);
    if (D == 64) return nch * H * WsLayout<64>::SIZE * sizeof(float);
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
    if (nch > 0x7fffffffL || H > 65535 || (long)H * (D / NT2) > 0x7fffffffL)
        K3_FAIL(K3HIP_EINVAL, "k3hip_kda_chunk: T=%d H=%d too large", T, H);
    const size_t need = k3hip_kda_chunk_workspace(T, H, D, chunk);
    hipStream_t st = as_stream(stream);
    StreamBuf own;
    float *ws = (float *)workspace;
    if (ws) {
        if (workspace_bytes < need)
            K3_FAIL(K3HIP_EINVAL, "k3hip_kda_chunk: workspace %zu bytes < %zu needed", workspace_bytes, need);
        if ((uintptr_t)ws & 15) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_chunk: workspace must be 16-byte aligned");
    } else {
        int rc = stream_alloc(own, need, st);
        if (rc) return rc;
        ws = (float *)own.p;
    }
    if (D == 128) return launch_chunk<128>(T, H, q, k, v, g, beta, q_scale, S, o, ws, st);
    return launch_chunk<64>(T, H, q, k, v, g, beta, q_scale, S, o, ws, st);
}
