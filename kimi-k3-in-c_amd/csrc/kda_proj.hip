// SPDX-License-Identifier: Apache-2.0
// kda_proj.hip - projections of the drop-in layer: y[t][o] = W[o][:] . x[t][:] (gfx950).
//
// The reference computes every projection as a per-token GEMV with double accumulators
// (k3_matmul, src/core/k3_ops.c:265-291; bf16 weights widened exactly, :1122-1227). This
// kernel keeps the double accumulation and the exact bf16 widening, so it reproduces the
// reference to within the last bit of the fp32 result; only the summation order differs.
// One wave owns one output row and PROJ_TB tokens: each weight element is read once per
// PROJ_TB tokens and fused into PROJ_TB double accumulators; a wave reduction finishes.
// This is the parity path of k3_kda_layer (small T, fp32 or bf16 weights), not the
// throughput GEMM.
//
// The int8 draft format (K3_WI8, include/k3/k3.h:266-283; k3_matmul_q8,
// src/core/k3_ops.c:1228-1301) stores row o as [f32 scale][int8 * in] (4 + in bytes, so rows
// are byte-aligned only): the int8 weights are dotted with x in double and the row's scale
// applied once at the end, y = (float)dot * scale. The reference sums in float in its SIMD
// order and states no exactness contract for the format; the double sum is within float
// rounding of it.
#include "k3kda_common.h"
#include "kda_internal.h"

namespace k3kda {

constexpr int PROJ_TB = 8;   // tokens per wave
constexpr int PROJ_WAVES = 4;

template <int WDT>
__global__ __launch_bounds__(64 * PROJ_WAVES) void kda_proj_kernel(int T, int in, int out,
                                                                   const float *__restrict__ x,
                                                                   const void *__restrict__ W,
                                                                   float *__restrict__ y)
{
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * PROJ_WAVES + (threadIdx.x >> 6);
    if (row >= out) return;
    const int t0 = blockIdx.y * PROJ_TB;
    const int nt = min(PROJ_TB, T - t0);
    double acc[PROJ_TB];
#pragma unroll
    for (int b = 0; b < PROJ_TB; b++) acc[b] = 0.0;
    const size_t wrow = (size_t)row * in;
    const unsigned char *q8row = reinterpret_cast<const unsigned char *>(W) + (size_t)row * (4 + (size_t)in);
    for (int i = lane; i < in; i += 64) {
        double wv;
        if constexpr (WDT == K3_WBF16) wv = (double)bf2f(reinterpret_cast<const uint16_t *>(W)[wrow + i]);
        else if constexpr (WDT == K3_WI8) wv = (double)(signed char)q8row[4 + i];
        else wv = (double)reinterpret_cast<const float *>(W)[wrow + i];
#pragma unroll
        for (int b = 0; b < PROJ_TB; b++)
            if (b < nt) acc[b] = fma(wv, (double)x[(size_t)(t0 + b) * in + i], acc[b]);
    }
#pragma unroll
    for (int b = 0; b < PROJ_TB; b++) {
        double s = acc[b];
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);
        if constexpr (WDT == K3_WI8) {
            // the row's scale, an unaligned little-endian fp32 at the row's start
            const uint32_t u = (uint32_t)q8row[0] | ((uint32_t)q8row[1] << 8) | ((uint32_t)q8row[2] << 16) |
                               ((uint32_t)q8row[3] << 24);
            if (lane == 0 && b < nt) y[(size_t)(t0 + b) * out + row] = (float)s * __uint_as_float(u);
        } else if (lane == 0 && b < nt) {
            y[(size_t)(t0 + b) * out + row] = (float)s;
        }
    }
}

int proj(int T, int in, int out, const float *x, const void *W, int wdt, float *y, hipStream_t st)
{
    if (T <= 0 || out <= 0) return K3HIP_OK;
    const long ty = ((long)T + PROJ_TB - 1) / PROJ_TB;
    if (ty > 65535) K3_FAIL(K3HIP_EINVAL, "projection: T=%d too large for the GEMV path", T);
    dim3 grid((out + PROJ_WAVES - 1) / PROJ_WAVES, (unsigned)ty);
    if (wdt == K3_WBF16)
        hipLaunchKernelGGL((kda_proj_kernel<K3_WBF16>), grid, dim3(64 * PROJ_WAVES), 0, st, T, in, out, x, W, y);
    else if (wdt == K3_WF32)
        hipLaunchKernelGGL((kda_proj_kernel<K3_WF32>), grid, dim3(64 * PROJ_WAVES), 0, st, T, in, out, x, W, y);
    else if (wdt == K3_WI8)
        hipLaunchKernelGGL((kda_proj_kernel<K3_WI8>), grid, dim3(64 * PROJ_WAVES), 0, st, T, in, out, x, W, y);
    else
        K3_FAIL(K3HIP_EUNSUPPORTED, "projection: weight tag %d (fp32=0, bf16=1, int8 rows=2)", wdt);
    K3_LAUNCHED();
    return K3HIP_OK;
}

}  // namespace k3kda
