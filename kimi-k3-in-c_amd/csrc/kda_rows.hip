// SPDX-License-Identifier: Apache-2.0
// kda_rows.hip - C[B][N] = x[B][K] . W[N][K]^T for a few activation rows (decode: one token
// per sequence) on bf16 weights, for gfx950.
//
// Replaces the reference's per-token k3_mmw / k3_matmul_bf16 (include/k3/k3.h:290-296,
// src/core/k3_ops.c:1122-1227) when B sequences decode together: each weight is read once
// for all B rows. The work is bound by reading W (B << the bytes per weight row), so the
// design goal is HBM bandwidth on W, not MFMA rate.
//
// Weight layout: the decode copy of W is stored in MFMA fragment order (rows_frag_pack):
// for each 16-column group g and 32-wide K-step t, the 64 lanes' B-fragments
// W[16 g + (lane & 15)][32 t + 8 (lane >> 4) .. + 7] lie in one contiguous 1 KB, so every
// wave load of the weight is one fully used 1 KB span. Reading the row-major matrix in
// fragment shape touches 16 rows x 64 B per wave load instead and streams about 25% slower.
// The weight is read with nontemporal loads (streamed through, not kept in the caches): the
// batch-16 KDA decode layer at hidden 7168 measured 97.5 -> 83.2 us with them.
//
// Precision: x stays fp32. Each 8-element slice of an x row is split in registers into
// bf16 hi + lo (x = hi + lo to ~2^-17 relative), and both halves go through the same bf16
// MFMA against the bf16 weight (an exact product) into one fp32 accumulator, so every
// product keeps fp32 accuracy with no extra weight traffic.
//
// Work split: a workgroup of 8 waves owns 64 output columns (4 column groups) and one
// K-range; its waves take the K-steps of the range round robin. The number of K-ranges per
// column block (split-K) is chosen so that a launch has about one workgroup per CU: wide N
// runs unsplit, narrow N splits K. The eight wave partials meet in LDS and are summed in a
// fixed order; K-range partials go to a workspace and a second kernel sums them in range
// order. Results are therefore reproducible bit for bit. A caller that has zeroed C may let
// two K-range partials be added into C with atomics instead (no workspace, no second
// launch): a + b = b + a exactly, so the bits do not depend on which range lands first.
#include <algorithm>

#include "kda_internal.h"
#include "kda_split.h"

namespace k3kda {

namespace {

using bsplit::bf16x8;
using bsplit::split_row8;
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int RT_WAVES = 8;   // waves per workgroup
constexpr int RT_NT = 4;      // 16-column groups per workgroup
constexpr int RT_SMAX = 16;   // most K-ranges per column block

// out[u] (16 B) for u = (g KT + t) 64 + lane: W[16 g + (lane & 15)][32 t + 8 (lane >> 4) .. + 7],
// zero past N and K (K % 8 == 0, so a slice is wholly inside or outside)
__global__ void rows_frag_pack_kernel(const uint16_t *__restrict__ W, int N, int K, uint4 *__restrict__ out,
                                      size_t units)
{
    const int KT = (K + 31) / 32;
    for (size_t u = (size_t)blockIdx.x * blockDim.x + threadIdx.x; u < units; u += (size_t)gridDim.x * blockDim.x) {
        const int lane = (int)(u & 63);
        const size_t gt = u >> 6;
        const int t = (int)(gt % KT), g = (int)(gt / KT);
        const int n = 16 * g + (lane & 15), k = 32 * t + 8 * (lane >> 4);
        uint4 v = {0, 0, 0, 0};
        if (n < N && k < K) v = *reinterpret_cast<const uint4 *>(W + (size_t)n * K + k);
        out[u] = v;
    }
}

// One weight's product in a launch: nb column blocks x S K-ranges of tchunk K-steps; the
// outputs go to P + s * split_stride (row stride ldp).
struct RowsJob {
    int N, nb, S, tchunk;
    const uint16_t *Wf;
    float *P;
    long ldp, split_stride;
    // unsplit products only: C also as bf16 hi (row m) and lo (plane hlplane on) rows of
    // stride ldhl, x = hi + lo, for a following GEMM on split rows (nullptr: none)
    uint16_t *hl = nullptr;
    long ldhl = 0, hlplane = 0;
};

// Block (nb, s) of a job: column groups 4 nb .. 4 nb + 3, K-steps [s tchunk, min(KT, (s + 1)
// tchunk)). One launch may carry two jobs over the same x (the first j0.nb * j0.S blocks
// are j0's). MT = 16-row tiles of x (B <= 16 MT). Wave w takes K-steps tbeg + w, tbeg + w +
// 8, ...; each step loads the 4 groups' fragments (4 x 1 KB) and the x slice, then runs the
// hi and lo MFMAs.
// NORM (xw != nullptr): each x row is RMS-normalised on the way in, x'[k] = (xw[k] x[k]) inv with
// inv = 1 / sqrt(mean_k x^2 + xeps) (mean in double; src/core/k3_ops.c:94-102), so a
// normalised input needs no launch of its own.
template <int MT, bool ATOM, bool NORM>
__global__ __launch_bounds__(64 * RT_WAVES) void rows_gemm_kernel(int B, int K, const float *__restrict__ x,
                                                                  long ldx, RowsJob j0, RowsJob j1,
                                                                  const float *__restrict__ xw, float xeps)
{
    __shared__ f32x4 red[RT_WAVES][RT_NT][MT][64];
    __shared__ float xinv[16 * MT];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int r16 = lane & 15, kg = lane >> 4;
    const int n0 = j0.nb * j0.S;
    const bool second = (int)blockIdx.x >= n0;
    const RowsJob &jb = second ? j1 : j0;
    const int lb = second ? (int)blockIdx.x - n0 : (int)blockIdx.x;
    const int nb = lb % jb.nb, s = lb / jb.nb;
    const int N = jb.N, tchunk = jb.tchunk;
    const uint16_t *__restrict__ Wf = jb.Wf;
    float *__restrict__ P = jb.P;
    const long ldp = jb.ldp, split_stride = jb.split_stride;
    const int KT = (K + 31) / 32, NG = (N + 15) / 16;
    const int tbeg = s * tchunk, tend = min(KT, tbeg + tchunk);

    // per-lane fragment streams of the 4 column groups (groups past N clamped to the last
    // one; their results are not stored), x rows of the MT row tiles (clamped to B - 1, zeroed)
    const bf16x8 *wg[RT_NT];
#pragma unroll
    for (int j = 0; j < RT_NT; j++)
        wg[j] = reinterpret_cast<const bf16x8 *>(Wf) + (size_t)min(RT_NT * nb + j, NG - 1) * KT * 64 + lane;
    const float *xrow[MT];
    bool xlive[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        xlive[mt] = 16 * mt + r16 < B;
        xrow[mt] = x + (size_t)min(16 * mt + r16, B - 1) * ldx;
    }

    // with a normalised input, this wave's first weight fragments are requested before the
    // rows' inverse RMS is formed, so that their latency hides behind it
    bf16x8 wv0[RT_NT];
    const int t0 = tbeg + w;
    if (NORM && t0 < tend) {
#pragma unroll
        for (int j = 0; j < RT_NT; j++) wv0[j] = __builtin_nontemporal_load(&wg[j][(size_t)t0 * 64]);
    }
    if constexpr (NORM) {   // the rows' inverse RMS: 32 lanes per row, 16 rows per pass
        for (int rr0 = 0; rr0 < 16 * MT; rr0 += 16) {
            const int rr = rr0 + ((int)threadIdx.x >> 5), ln = threadIdx.x & 31;
            double ss = 0.0;
            if (rr < B) {
                // eight loads in flight per step
                const float *xr = x + (size_t)rr * ldx;
                int k = ln;
                for (; k + 7 * 32 < K; k += 8 * 32) {
                    float v[8];
#pragma unroll
                    for (int u = 0; u < 8; u++) v[u] = xr[k + 32 * u];
#pragma unroll
                    for (int u = 0; u < 8; u++) ss += (double)v[u] * (double)v[u];
                }
                for (; k < K; k += 32) ss += (double)xr[k] * (double)xr[k];
            }
#pragma unroll
            for (int o = 16; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 32);
            if (ln == 0) xinv[rr] = rr < B ? (float)(1.0 / sqrt(ss / (double)K + (double)xeps)) : 0.0f;
        }
        __syncthreads();
    }
    float xiv[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) xiv[mt] = NORM ? xinv[16 * mt + r16] : 1.0f;

    f32x4 acc[RT_NT][MT];
#pragma unroll
    for (int j = 0; j < RT_NT; j++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[j][mt] = 0.0f;

    for (int t = t0; t < tend; t += RT_WAVES) {
        bf16x8 wv[RT_NT];
        if (NORM && t == t0) {
#pragma unroll
            for (int j = 0; j < RT_NT; j++) wv[j] = wv0[j];
        } else {
#pragma unroll
            for (int j = 0; j < RT_NT; j++) wv[j] = __builtin_nontemporal_load(&wg[j][(size_t)t * 64]);
        }
        const int k = 32 * t + 8 * kg;   // K % 8 == 0: the 8-slice is wholly inside or outside
        const bool kin = k < K;
        f4 xa[MT], xb[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            xa[mt] = *reinterpret_cast<const f4 *>(xrow[mt] + (kin ? k : 0));
            xb[mt] = *reinterpret_cast<const f4 *>(xrow[mt] + (kin ? k : 0) + 4);
        }
        if constexpr (NORM) {
            const f4 wa = *reinterpret_cast<const f4 *>(xw + (kin ? k : 0));
            const f4 wb = *reinterpret_cast<const f4 *>(xw + (kin ? k : 0) + 4);
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                xa[mt] = (wa * xa[mt]) * xiv[mt];
                xb[mt] = (wb * xb[mt]) * xiv[mt];
            }
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            bf16x8 xh, xl;
            const bool ok = kin && xlive[mt];
            split_row8(ok ? xa[mt] : f4(0.0f), ok ? xb[mt] : f4(0.0f), xh, xl);
#pragma unroll
            for (int j = 0; j < RT_NT; j++) {
                acc[j][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xh, wv[j], acc[j][mt], 0, 0, 0);
                acc[j][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl, wv[j], acc[j][mt], 0, 0, 0);
            }
        }
    }

    // wave partials -> LDS; wave j < 4 sums column group j over the 8 waves in order
#pragma unroll
    for (int j = 0; j < RT_NT; j++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) red[w][j][mt][lane] = acc[j][mt];
    __syncthreads();
    if (w >= RT_NT) return;
    float *out = ATOM ? P : P + (size_t)s * split_stride;
    const int n = 16 * (RT_NT * nb + w) + r16;
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        f32x4 t = red[0][w][mt][lane];
#pragma unroll
        for (int ww = 1; ww < RT_WAVES; ww++) t = t + red[ww][w][mt][lane];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int m = 16 * mt + 4 * kg + e;   // MFMA C layout: lane n + 16 j holds rows 4j..4j+3
            if (m < B && n < N) {
                if constexpr (ATOM) {
                    unsafeAtomicAdd(&out[(size_t)m * ldp + n], t[e]);
                } else {
                    out[(size_t)m * ldp + n] = t[e];
                    if (jb.hl) {
                        const uint16_t hi = f2bf(t[e]);
                        jb.hl[(size_t)m * jb.ldhl + n] = hi;
                        jb.hl[(size_t)jb.hlplane + (size_t)m * jb.ldhl + n] = f2bf(t[e] - __uint_as_float((uint32_t)hi << 16));
                    }
                }
            }
        }
    }
}

// C[m][n] = sum over s = 0 .. S-1 of P[s][m][n], added in that order; four adjacent
// columns per thread (N % 4 == 0, ldc % 4 == 0, C 16-byte aligned)
__global__ void rows_reduce_kernel(int B, int N, int S, const float *__restrict__ P, float *__restrict__ C,
                                   long ldc)
{
    const size_t total = (size_t)B * N, q = total / 4;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < q; i += (size_t)gridDim.x * blockDim.x) {
        f4 v[RT_SMAX];
#pragma unroll
        for (int s = 0; s < RT_SMAX; s++)
            v[s] = s < S ? reinterpret_cast<const f4 *>(P + (size_t)s * total)[i] : f4(0.0f);
        f4 t = v[0];
#pragma unroll
        for (int s = 1; s < RT_SMAX; s++)
            if (s < S) t = t + v[s];
        const size_t e = 4 * i;
        *reinterpret_cast<f4 *>(C + (e / N) * ldc + e % N) = t;
    }
}
// the same for any N, one element per thread
__global__ void rows_reduce1_kernel(int B, int N, int S, const float *__restrict__ P, float *__restrict__ C,
                                    long ldc)
{
    const size_t total = (size_t)B * N;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        float v[RT_SMAX];
#pragma unroll
        for (int s = 0; s < RT_SMAX; s++) v[s] = s < S ? P[(size_t)s * total + i] : 0.0f;
        float t = v[0];
#pragma unroll
        for (int s = 1; s < RT_SMAX; s++)
            if (s < S) t = t + v[s];
        C[(i / N) * ldc + i % N] = t;
    }
}

RowsJob rows_job(int N, int tchunk, int S, const uint16_t *Wf, float *P, long ldp, long split_stride)
{
    return RowsJob{N, (N + 16 * RT_NT - 1) / (16 * RT_NT), S, tchunk, Wf, P, ldp, split_stride};
}

template <int MT, bool ATOM = false>
int launch_jobs(int B, int K, const float *x, long ldx, const RowsJob &j0, const RowsJob &j1, hipStream_t st,
                const float *xw = nullptr, float xeps = 0.0f)
{
    const long nblk = (long)j0.nb * j0.S + (long)j1.nb * j1.S;
    if (xw)
        hipLaunchKernelGGL((rows_gemm_kernel<MT, ATOM, true>), dim3((unsigned)nblk), dim3(64 * RT_WAVES), 0, st, B, K,
                           x, ldx, j0, j1, xw, xeps);
    else
        hipLaunchKernelGGL((rows_gemm_kernel<MT, ATOM, false>), dim3((unsigned)nblk), dim3(64 * RT_WAVES), 0, st, B,
                           K, x, ldx, j0, j1, xw, xeps);
    K3_LAUNCHED();
    return K3HIP_OK;
}

template <int MT, bool ATOM = false>
int launch_rows(int B, int N, int K, int tchunk, int S, const float *x, long ldx, const uint16_t *Wf,
                float *P, long ldp, long split_stride, hipStream_t st)
{
    const RowsJob none{1, 1, 0, 1, Wf, P, 0, 0};   // no blocks
    return launch_jobs<MT, ATOM>(B, K, x, ldx, rows_job(N, tchunk, S, Wf, P, ldp, split_stride), none, st);
}

// rows for one launch of up to 64 rows (MT = 1, 2 or 4 16-row tiles)
int launch_jobs_b(int bb, int K, const float *x, long ldx, const RowsJob &j0, const RowsJob &j1, hipStream_t st,
                  const float *xw = nullptr, float xeps = 0.0f)
{
    if (bb <= 16) return launch_jobs<1>(bb, K, x, ldx, j0, j1, st, xw, xeps);
    if (bb <= 32) return launch_jobs<2>(bb, K, x, ldx, j0, j1, st, xw, xeps);
    return launch_jobs<4>(bb, K, x, ldx, j0, j1, st, xw, xeps);
}

int cu_total()
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

}  // namespace

namespace {

struct RowsPlan {
    int S, tchunk;
};

// About one workgroup per CU: S = CUs / column blocks K-ranges, rounded up from a fraction of
// 3/4, at most RT_SMAX and at most one per K-step. N wider than ~4/7 of a column block per
// CU runs unsplit (measured: 161 blocks on 256 CUs unsplit beat 322 split workgroups), and
// so does a weight of at most 2 MB, whose launch costs more than its reads.
RowsPlan rows_plan(int N, int K)
{
    const int nblk = (N + 16 * RT_NT - 1) / (16 * RT_NT), KT = (K + 31) / 32;
    int S = (cu_total() + nblk / 4) / nblk;
    if ((size_t)N * K <= ((size_t)1 << 20)) S = 1;
    S = std::max(1, std::min({S, RT_SMAX, KT}));
    RowsPlan p;
    p.tchunk = (KT + S - 1) / S;
    p.S = (KT + p.tchunk - 1) / p.tchunk;
    return p;
}

}  // namespace

size_t rows_frag_elems(int N, int K)
{
    if (N <= 0 || K <= 0) return 0;
    return (size_t)((N + 15) / 16) * 16 * ((K + 31) / 32) * 32;
}

int rows_frag_pack(const uint16_t *W, int N, int K, uint16_t *Wf, hipStream_t st)
{
    if (N <= 0 || K <= 0) return K3HIP_OK;
    if ((K & 7) || (((uintptr_t)W | (uintptr_t)Wf) & 15))
        K3_FAIL(K3HIP_EINVAL, "rows_frag_pack: K=%d needs a multiple of 8 and 16-byte aligned W", K);
    const size_t units = rows_frag_elems(N, K) / 8;
    const int grid = (int)std::min<size_t>((units + 255) / 256, 65536);
    hipLaunchKernelGGL(rows_frag_pack_kernel, dim3(grid), dim3(256), 0, st, W, N, K, (uint4 *)Wf, units);
    K3_LAUNCHED();
    return K3HIP_OK;
}

size_t gemm_rows_ws_floats(int B, int N, int K)
{
    if (B <= 0 || N <= 0 || K <= 0) return 0;
    const RowsPlan p = rows_plan(N, K);
    return p.S > 1 ? (size_t)p.S * std::min(64, B) * N : 0;
}

int gemm_rows_splits(int N, int K)
{
    if (N <= 0 || K <= 0) return 1;
    return rows_plan(N, K).S;
}

int gemm_rows_part(int B, int N, int K, const float *x, long ldx, const uint16_t *Wf, float *P, hipStream_t st)
{
    if (B <= 0 || N <= 0 || K <= 0) return K3HIP_OK;
    if ((K & 7) || (ldx & 3) || (((uintptr_t)x | (uintptr_t)Wf) & 15))
        K3_FAIL(K3HIP_EINVAL, "gemm_rows_part: K=%d ldx=%ld need multiples of 8 / 4 and 16-byte aligned x, W", K, ldx);
    const RowsPlan pl = rows_plan(N, K);
    const long plane = (long)B * N;
    for (int b0 = 0; b0 < B; b0 += 64) {
        const int bb = std::min(64, B - b0);
        const float *xb = x + (size_t)b0 * ldx;
        float *Pb = P + (size_t)b0 * N;
        int rc;
        if (bb <= 16) rc = launch_rows<1>(bb, N, K, pl.tchunk, pl.S, xb, ldx, Wf, Pb, N, plane, st);
        else if (bb <= 32) rc = launch_rows<2>(bb, N, K, pl.tchunk, pl.S, xb, ldx, Wf, Pb, N, plane, st);
        else rc = launch_rows<4>(bb, N, K, pl.tchunk, pl.S, xb, ldx, Wf, Pb, N, plane, st);
        if (rc) return rc;
    }
    return K3HIP_OK;
}

int gemm_rows_with_part(int B, int K, const float *x, long ldx, int N1, const uint16_t *Wf1, float *C1, long ldc1,
                        int N2, const uint16_t *Wf2, float *P2, hipStream_t st, float *ws, size_t ws_floats)
{
    if (B <= 0 || K <= 0) return K3HIP_OK;
    const RowsPlan p1 = rows_plan(N1, K), p2 = rows_plan(N2, K);
    if (N1 <= 0 || N2 <= 0 || p1.S != 1) {   // the first product needs its reduction: two launches
        int rc = gemm_rows(B, N1, K, x, ldx, Wf1, C1, ldc1, st, ws, ws_floats);
        return rc ? rc : gemm_rows_part(B, N2, K, x, ldx, Wf2, P2, st);
    }
    if ((K & 7) || (ldx & 3) || (((uintptr_t)x | (uintptr_t)Wf1 | (uintptr_t)Wf2) & 15))
        K3_FAIL(K3HIP_EINVAL, "gemm_rows_with_part: K=%d ldx=%ld need multiples of 8 / 4 and 16-byte aligned x, W", K, ldx);
    const long plane = (long)B * N2;
    for (int b0 = 0; b0 < B; b0 += 64) {
        const int bb = std::min(64, B - b0);
        const RowsJob j0 = rows_job(N1, p1.tchunk, 1, Wf1, C1 + (size_t)b0 * ldc1, ldc1, 0);
        const RowsJob j1 = rows_job(N2, p2.tchunk, p2.S, Wf2, P2 + (size_t)b0 * N2, N2, plane);
        int rc = launch_jobs_b(bb, K, x + (size_t)b0 * ldx, ldx, j0, j1, st);
        if (rc) return rc;
    }
    return K3HIP_OK;
}

int gemm_rows_hl(int B, int N, int K, const float *x, long ldx, const uint16_t *Wf, float *C, long ldc,
                 uint16_t *hl, long ldhl, hipStream_t st, float *ws, size_t ws_floats, const float *xw, float xeps)
{
    if (B <= 0 || N <= 0 || K <= 0) return K3HIP_OK;
    const RowsPlan pl = rows_plan(N, K);
    if (xw && (pl.S != 1 || (((uintptr_t)xw) & 15)))
        K3_FAIL(K3HIP_EUNSUPPORTED, "gemm_rows_hl: the normalised input needs an unsplit product and 16-byte aligned weights");
    if (pl.S != 1) {   // the split rows from the reduced product
        int rc = gemm_rows(B, N, K, x, ldx, Wf, C, ldc, st, ws, ws_floats);
        if (rc) return rc;
        if (ldhl != N || ldc != N) K3_FAIL(K3HIP_EINVAL, "gemm_rows_hl: a split-K product needs ldc = ldhl = N");
        return split_rows2(C, hl, B, N, st);
    }
    if ((K & 7) || (ldx & 3) || (((uintptr_t)x | (uintptr_t)Wf) & 15))
        K3_FAIL(K3HIP_EINVAL, "gemm_rows_hl: K=%d ldx=%ld need multiples of 8 / 4 and 16-byte aligned x, W", K, ldx);
    const RowsJob none{1, 1, 0, 1, Wf, C, 0, 0};   // no blocks
    for (int b0 = 0; b0 < B; b0 += 64) {
        const int bb = std::min(64, B - b0);
        RowsJob j = rows_job(N, pl.tchunk, 1, Wf, C + (size_t)b0 * ldc, ldc, 0);
        j.hl = hl + (size_t)b0 * ldhl;
        j.ldhl = ldhl;
        j.hlplane = (long)B * ldhl;
        int rc = launch_jobs_b(bb, K, x + (size_t)b0 * ldx, ldx, j, none, st, xw, xeps);
        if (rc) return rc;
    }
    return K3HIP_OK;
}

namespace {

// K-ranges that spread the workgroups most evenly: the most workgroups one CU gets over the
// share of K each reads, least wins, the fewer ranges on a tie (161 column blocks on 256 CUs:
// 3 ranges, at most 2 workgroups per CU, against 1 range on 161 CUs)
RowsPlan rows_plan_even(int N, int K)
{
    const long nblk = (N + 16 * RT_NT - 1) / (16 * RT_NT), ncu = cu_total();
    const int KT = (K + 31) / 32;
    RowsPlan p{1, KT};
    double cost = (double)((nblk + ncu - 1) / ncu);
    for (int s = 2; s <= std::min(8, KT); s++) {
        const int tchunk = (KT + s - 1) / s;
        if ((KT + tchunk - 1) / tchunk != s) continue;   // s ranges of whole K-steps, none empty
        const double c = (double)((nblk * s + ncu - 1) / ncu) / s;
        if (c < cost - 1e-9) {
            cost = c;
            p = RowsPlan{s, tchunk};
        }
    }
    return p;
}

int rows_run(int B, int N, int K, const float *x, long ldx, const uint16_t *Wf, float *C, long ldc,
             hipStream_t st, float *ws, size_t ws_floats, bool c_zeroed, const RowsPlan &pl)
{
    if (B <= 0 || N <= 0 || K <= 0) return K3HIP_OK;
    if ((K & 7) || (ldx & 3) || (((uintptr_t)x | (uintptr_t)Wf) & 15))
        K3_FAIL(K3HIP_EINVAL, "gemm_rows: K=%d ldx=%ld need multiples of 8 / 4 and 16-byte aligned x, W", K, ldx);
    const int S = pl.S, tchunk = pl.tchunk;
    if (c_zeroed && S == 2) {   // the two K-range partials are added into C in place
        for (int b0 = 0; b0 < B; b0 += 64) {
            const int bb = std::min(64, B - b0);
            const float *xb = x + (size_t)b0 * ldx;
            float *Cb = C + (size_t)b0 * ldc;
            int rc;
            if (bb <= 16) rc = launch_rows<1, true>(bb, N, K, tchunk, S, xb, ldx, Wf, Cb, ldc, 0, st);
            else if (bb <= 32) rc = launch_rows<2, true>(bb, N, K, tchunk, S, xb, ldx, Wf, Cb, ldc, 0, st);
            else rc = launch_rows<4, true>(bb, N, K, tchunk, S, xb, ldx, Wf, Cb, ldc, 0, st);
            if (rc) return rc;
        }
        return K3HIP_OK;
    }
    const size_t need = S > 1 ? (size_t)S * std::min(64, B) * N : 0;
    StreamBuf own;
    if (need && (!ws || ws_floats < need || ((uintptr_t)ws & 15))) {
        int rc = stream_alloc(own, need * sizeof(float), st);
        if (rc) return rc;
        ws = (float *)own.p;
    }
    for (int b0 = 0; b0 < B; b0 += 64) {
        const int bb = std::min(64, B - b0);
        float *P = C + (size_t)b0 * ldc;
        long ldp = ldc, sstride = 0;
        if (S > 1) {
            P = ws;
            ldp = N;
            sstride = (long)bb * N;
        }
        const float *xb = x + (size_t)b0 * ldx;
        int rc;
        if (bb <= 16) rc = launch_rows<1>(bb, N, K, tchunk, S, xb, ldx, Wf, P, ldp, sstride, st);
        else if (bb <= 32) rc = launch_rows<2>(bb, N, K, tchunk, S, xb, ldx, Wf, P, ldp, sstride, st);
        else rc = launch_rows<4>(bb, N, K, tchunk, S, xb, ldx, Wf, P, ldp, sstride, st);
        if (rc) return rc;
        if (S > 1) {
            const size_t total = (size_t)bb * N;
            float *Cb = C + (size_t)b0 * ldc;
            if (N % 4 == 0 && ldc % 4 == 0 && ((uintptr_t)Cb & 15) == 0) {
                const int grid = (int)std::min<size_t>((total / 4 + 63) / 64, 16384);
                hipLaunchKernelGGL(rows_reduce_kernel, dim3(grid), dim3(64), 0, st, bb, N, S, P, Cb, ldc);
            } else {
                const int grid = (int)std::min<size_t>((total + 63) / 64, 16384);
                hipLaunchKernelGGL(rows_reduce1_kernel, dim3(grid), dim3(64), 0, st, bb, N, S, P, Cb, ldc);
            }
            K3_LAUNCHED();
        }
    }
    return K3HIP_OK;
}

}  // namespace

int gemm_rows(int B, int N, int K, const float *x, long ldx, const uint16_t *Wf, float *C, long ldc,
              hipStream_t st, float *ws, size_t ws_floats, bool c_zeroed)
{
    if (B <= 0 || N <= 0 || K <= 0) return K3HIP_OK;
    return rows_run(B, N, K, x, ldx, Wf, C, ldc, st, ws, ws_floats, c_zeroed, rows_plan(N, K));
}

int gemm_rows_plane_count(int N, int K)
{
    if (N <= 0 || K <= 0) return 1;
    return rows_plan_even(N, K).S;
}

int gemm_rows_even(int B, int N, int K, const float *x, long ldx, const uint16_t *Wf, float *C, long ldc,
                   hipStream_t st, float *ws, size_t ws_floats)
{
    if (B <= 0 || N <= 0 || K <= 0) return K3HIP_OK;
    return rows_run(B, N, K, x, ldx, Wf, C, ldc, st, ws, ws_floats, false, rows_plan_even(N, K));
}

}  // namespace k3kda
