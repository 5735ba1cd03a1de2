// SPDX-License-Identifier: Apache-2.0
// kda_rows.hip - C[B][N] = x[B][K] . W[N][K]^T for a few activation rows (decode: one token
// per sequence) on bf16 weights, for gfx950.
//
// Replaces the reference's per-token k3_mmw / k3_matmul_bf16 (include/k3/k3.h:290-296,
// src/core/k3_ops.c:1122-1227) when B sequences decode together: each weight is read once
// for all B rows. The work is bound by reading W (B << the bytes per weight row), so the
// design goal is HBM bandwidth on W, not MFMA rate.
//
// Precision: x stays fp32. Each 8-element slice of an x row is split in registers into
// bf16 hi + lo (x = hi + lo to ~2^-17 relative), and both halves go through the same bf16
// MFMA against the bf16 weight (an exact product) into one fp32 accumulator, so every
// product keeps fp32 accuracy with no extra weight traffic.
//
// Work split: a workgroup of 4 waves owns 128 (or 64) output columns (MFMA column tiles of
// 16) and one K-range; the K-ranges of a column block are split over workgroups (split-K)
// so that a launch has about two workgroups per CU. Inside a workgroup the waves take
// interleaved 64-wide K-units, so each wave reads whole 128-byte lines and the four waves
// together stream 512 contiguous bytes of each weight row at a time. The four wave partials meet in LDS and are summed in a fixed
// order; the K-range partials go to a workspace and a second kernel sums them in split
// order. Results are therefore reproducible bit for bit.
#include <algorithm>

#include "kda_internal.h"

namespace k3kda {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int RT_WAVES = 4;   // waves per workgroup
constexpr int RT_U = 2;       // 64-wide K-units per wave whose loads are issued together
constexpr int RT_SMAX = 16;   // most K-ranges per column block

// x = hi + lo, both bf16 (round to nearest even; lo carries the rounding error of hi)
__device__ __forceinline__ void split_row8(const f4 &a, const f4 &b, bf16x8 &hi, bf16x8 &lo)
{
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        const bf16x2 h = __builtin_convertvector(f2{v[e], v[e + 1]}, bf16x2);
        const uint32_t u = __builtin_bit_cast(uint32_t, h);
        const float h0 = __uint_as_float(u << 16), h1 = __uint_as_float(u & 0xffff0000u);
        const bf16x2 l = __builtin_convertvector(f2{v[e] - h0, v[e + 1] - h1}, bf16x2);
        hi[e] = h[0]; hi[e + 1] = h[1];
        lo[e] = l[0]; lo[e + 1] = l[1];
    }
}

// Block (nb, s): columns 16 NT nb .. + 16 NT - 1, K-range [s kchunk, min(K, (s + 1) kchunk)).
// MT = 16-row tiles of x (B <= 16 MT), NT = 16-column tiles. Wave w takes the 64-wide
// K-units kbeg + 64 (4 i + w): two MFMA K-steps, so each wave reads whole 128-byte lines
// of every weight row and x row it touches. Out = P + s * split_stride, row stride ldp.
template <int MT, int NT>
__global__ __launch_bounds__(64 * RT_WAVES) void rows_gemm_kernel(
    int B, int N, int K, int kchunk, const float *__restrict__ x, long ldx,
    const uint16_t *__restrict__ W, float *__restrict__ P, long ldp, long split_stride)
{
    __shared__ f32x4 red[RT_WAVES][NT][MT][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int r16 = lane & 15, kg = lane >> 4;
    const int nb = blockIdx.x, s = blockIdx.y;
    const int kbeg = s * kchunk, kend = min(K, kbeg + kchunk);

    // per-lane row pointers: weight rows of the NT column tiles (clamped to N - 1; their
    // results are not stored), x rows of the MT row tiles (clamped to B - 1, zeroed)
    const uint16_t *wrow[NT];
#pragma unroll
    for (int j = 0; j < NT; j++) wrow[j] = W + (size_t)min(16 * (NT * nb + j) + r16, N - 1) * K;
    const float *xrow[MT];
    bool xlive[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        xlive[mt] = 16 * mt + r16 < B;
        xrow[mt] = x + (size_t)min(16 * mt + r16, B - 1) * ldx;
    }

    f32x4 acc[NT][MT];
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[j][mt] = 0.0f;

    constexpr int NS = 2 * RT_U;   // K-steps of 32 per iteration
    for (int k0 = kbeg + 64 * w; k0 < kend; k0 += 64 * RT_WAVES * RT_U) {
        bf16x8 wv[NS][NT];
        f4 xa[NS][MT], xb[NS][MT];
        bool live[NS];
#pragma unroll
        for (int u = 0; u < NS; u++) {
            const int k = k0 + 64 * RT_WAVES * (u >> 1) + 32 * (u & 1) + 8 * kg;
            live[u] = k < kend;
            const int kc = live[u] ? k : kbeg;   // kbeg + 8 <= K: K and kbeg are multiples of 8
#pragma unroll
            for (int j = 0; j < NT; j++) wv[u][j] = *reinterpret_cast<const bf16x8 *>(wrow[j] + kc);
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                xa[u][mt] = *reinterpret_cast<const f4 *>(xrow[mt] + kc);
                xb[u][mt] = *reinterpret_cast<const f4 *>(xrow[mt] + kc + 4);
            }
        }
        __builtin_amdgcn_sched_barrier(0);   // every load of the iteration in flight first
#pragma unroll
        for (int u = 0; u < NS; u++) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                bf16x8 xh, xl;
                const bool ok = live[u] && xlive[mt];
                split_row8(ok ? xa[u][mt] : f4(0.0f), ok ? xb[u][mt] : f4(0.0f), xh, xl);
#pragma unroll
                for (int j = 0; j < NT; j++) {
                    acc[j][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xh, wv[u][j], acc[j][mt], 0, 0, 0);
                    acc[j][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl, wv[u][j], acc[j][mt], 0, 0, 0);
                }
            }
        }
    }

    // wave partials -> LDS; wave w sums column tiles w, w + 4, .. over the 4 waves in order
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) red[w][j][mt][lane] = acc[j][mt];
    __syncthreads();
    float *out = P + (size_t)s * split_stride;
#pragma unroll
    for (int j = w; j < NT; j += RT_WAVES) {
        const int n = 16 * (NT * nb + j) + r16;
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            f32x4 t = red[0][j][mt][lane];
#pragma unroll
            for (int ww = 1; ww < RT_WAVES; ww++) t = t + red[ww][j][mt][lane];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = 16 * mt + 4 * kg + e;   // MFMA C layout: lane n + 16 j holds rows 4j..4j+3
                if (m < B && n < N) out[(size_t)m * ldp + n] = t[e];
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

template <int MT, int NT>
int launch_rows(int B, int N, int K, int kchunk, int S, const float *x, long ldx, const uint16_t *W,
                float *P, long ldp, long split_stride, hipStream_t st)
{
    hipLaunchKernelGGL((rows_gemm_kernel<MT, NT>), dim3((N + 16 * NT - 1) / (16 * NT), S), dim3(64 * RT_WAVES),
                       0, st, B, N, K, kchunk, x, ldx, W, P, ldp, split_stride);
    K3_LAUNCHED();
    return K3HIP_OK;
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
    int nt, S, kchunk;
};

// 128 output columns per workgroup for very wide N (x is re-read once per column block:
// 25% of the weight bytes at B <= 16), else 64. K is split into ranges of 512 (one
// iteration per wave: all of a wave's loads in flight at once) up to RT_SMAX ranges;
// narrow N (few column blocks) uses no more ranges than about four workgroups per CU.
RowsPlan rows_plan(int N, int K)
{
    RowsPlan p;
    p.nt = N >= 128 * 64 ? 8 : 4;
    const int nblk = (N + 16 * p.nt - 1) / (16 * p.nt);
    const int kunits = (K + 511) / 512;
    int S = std::min(kunits, RT_SMAX);
    S = std::max(1, std::min(S, (4 * cu_total() + nblk - 1) / nblk));
    p.kchunk = ((kunits + S - 1) / S) * 512;
    p.S = (K + p.kchunk - 1) / p.kchunk;
    return p;
}

}  // namespace

size_t gemm_rows_ws_floats(int B, int N, int K)
{
    if (B <= 0 || N <= 0 || K <= 0) return 0;
    const RowsPlan p = rows_plan(N, K);
    return p.S > 1 ? (size_t)p.S * std::min(64, B) * N : 0;
}

int gemm_rows(int B, int N, int K, const float *x, long ldx, const uint16_t *W, float *C, long ldc,
              hipStream_t st, float *ws, size_t ws_floats)
{
    if (B <= 0 || N <= 0 || K <= 0) return K3HIP_OK;
    if ((K & 7) || (ldx & 3) || (((uintptr_t)x | (uintptr_t)W) & 15))
        K3_FAIL(K3HIP_EINVAL, "gemm_rows: K=%d ldx=%ld need multiples of 8 / 4 and 16-byte aligned x, W", K, ldx);
    const RowsPlan pl = rows_plan(N, K);
    const int S = pl.S, kchunk = pl.kchunk;
    const size_t need = gemm_rows_ws_floats(B, N, K);
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
        if (pl.nt == 8) {
            if (bb <= 16) rc = launch_rows<1, 8>(bb, N, K, kchunk, S, xb, ldx, W, P, ldp, sstride, st);
            else if (bb <= 32) rc = launch_rows<2, 8>(bb, N, K, kchunk, S, xb, ldx, W, P, ldp, sstride, st);
            else rc = launch_rows<4, 8>(bb, N, K, kchunk, S, xb, ldx, W, P, ldp, sstride, st);
        } else {
            if (bb <= 16) rc = launch_rows<1, 4>(bb, N, K, kchunk, S, xb, ldx, W, P, ldp, sstride, st);
            else if (bb <= 32) rc = launch_rows<2, 4>(bb, N, K, kchunk, S, xb, ldx, W, P, ldp, sstride, st);
            else rc = launch_rows<4, 4>(bb, N, K, kchunk, S, xb, ldx, W, P, ldp, sstride, st);
        }
        if (rc) return rc;
        if (S > 1) {
            const size_t total = (size_t)bb * N;
            float *Cb = C + (size_t)b0 * ldc;
            if (N % 4 == 0 && ldc % 4 == 0 && ((uintptr_t)Cb & 15) == 0) {
                const int grid = (int)std::min<size_t>((total / 4 + 255) / 256, 8192);
                hipLaunchKernelGGL(rows_reduce_kernel, dim3(grid), dim3(256), 0, st, bb, N, S, P, Cb, ldc);
            } else {
                const int grid = (int)std::min<size_t>((total + 255) / 256, 8192);
                hipLaunchKernelGGL(rows_reduce1_kernel, dim3(grid), dim3(256), 0, st, bb, N, S, P, Cb, ldc);
            }
            K3_LAUNCHED();
        }
    }
    return K3HIP_OK;
}

}  // namespace k3kda
