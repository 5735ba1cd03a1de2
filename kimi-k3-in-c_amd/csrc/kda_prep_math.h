// SPDX-License-Identifier: Apache-2.0
// kda_prep_math.h - the per-token arithmetic of K1 (short conv + SiLU, L2 norm, decay gate,
// beta) shared by the stand-alone prep kernel and the fused prefill kernel, so that the two
// produce identical bits.
//
// Follows src/core/k3_ops.c: k3_shortconv (:133-165), l2norm_ (:845-851), beta (:903),
// k3_kda_decay (:168-183). Transcendentals use the hardware 2^x and reciprocal (about
// 1 ulp): e^x = 2^(x log2 e), sigmoid(x) = rcp(1 + 2^(-x log2 e)).
#pragma once

#include "k3kda_common.h"

namespace k3kda {

__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
__device__ __forceinline__ float fast_sigmoid(float x) { return __builtin_amdgcn_rcpf(1.0f + fast_exp(-x)); }

// One conv output: taps w[0..K-1] over x_{t-K+1} .. x_t, where win[0..K-2] are the K-1
// older inputs (oldest first) and cur = x_t. acc = w[K-1] x_t, then += w[j] win[j] in
// order of j as fused multiply-adds (the reference rounds product and sum separately: a
// difference of at most an ulp of the partial sum per tap); the result is acc * sigmoid(acc).
template <int K>
__device__ __forceinline__ float conv_silu(const float (&w)[K], const float *win, float cur)
{
    float acc = w[K - 1] * cur;
#pragma unroll
    for (int j = 0; j < K - 1; j++) acc = __builtin_fmaf(w[j], win[j], acc);
    return acc * fast_sigmoid(acc);
}

// Sum over the 32 lanes of a half-wave, the same bits in every lane: swaps of lane pairs
// (xor 1, xor 2 inside quads), the mirror inside each 8-lane half-row and inside each 16-lane
// row (DPP), then the other row of the half-wave (swizzle, xor 16). Every step adds the
// same two values in both lanes of a pair, so all 32 lanes end equal.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float half_wave_sum(float x)
{
#pragma clang fp contract(off)
    x = x + dpp_f<0xB1>(x);    // quad_perm [1,0,3,2]
    x = x + dpp_f<0x4E>(x);    // quad_perm [2,3,0,1]
    x = x + dpp_f<0x141>(x);   // row_half_mirror
    x = x + dpp_f<0x140>(x);   // row_mirror
    return x + __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x401F));   // lane ^ 16
}

// L2 normalisation of one head row held by a 32-lane half-wave, CPL adjacent channels per
// lane: y *= 1/sqrt(sum y^2 + 1e-6), the sum in fp32 (per lane, then across the half-wave)
// and the scale from the hardware reciprocal square root. The reference sums in double
// (k3_ops.c:845-851); for a row of up to 128 squares the fp32 tree differs from it by a
// few 1e-7 relative.
template <int CPL>
__device__ __forceinline__ void l2norm_half(float (&y)[CPL])
{
#pragma clang fp contract(off)
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < CPL; e++) part = part + y[e] * y[e];
    const float r = __builtin_amdgcn_rsqf(half_wave_sum(part) + 1e-6f);
#pragma unroll
    for (int e = 0; e < CPL; e++) y[e] = y[e] * r;
}

// Bounded decay gate g = lb * sigmoid(a (z + dt_bias)), a = expf(A_log[h]), from
// a2 = gate_a2(a) = -a log2(e): lb / (1 + 2^((z + dt_bias) a2)).
__device__ __forceinline__ float gate_a2(float a) { return a * -1.4426950408889634f; }
__device__ __forceinline__ float gate_bounded(float lb, float a2, float z, float dtb)
{
#pragma clang fp contract(off)
    return lb * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f((z + dtb) * a2));
}

// Row access for CPL = 2 / 4 adjacent channels of fp32 or bf16 activations.
template <int CPL, int DT> struct RowIO;
template <> struct RowIO<4, K3HIP_F32> {
    static __device__ __forceinline__ void load(float (&x)[4], const void *p, size_t i)
    {
        const f4 v = *reinterpret_cast<const f4 *>(reinterpret_cast<const float *>(p) + i);
        x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
    }
};
template <> struct RowIO<4, K3HIP_BF16> {
    static __device__ __forceinline__ void load(float (&x)[4], const void *p, size_t i)
    {
        const uint2 v = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(p) + i);
        x[0] = __uint_as_float(v.x << 16); x[1] = __uint_as_float(v.x & 0xffff0000u);
        x[2] = __uint_as_float(v.y << 16); x[3] = __uint_as_float(v.y & 0xffff0000u);
    }
};
template <> struct RowIO<2, K3HIP_F32> {
    static __device__ __forceinline__ void load(float (&x)[2], const void *p, size_t i)
    {
        const f2 v = *reinterpret_cast<const f2 *>(reinterpret_cast<const float *>(p) + i);
        x[0] = v.x; x[1] = v.y;
    }
};
template <> struct RowIO<2, K3HIP_BF16> {
    static __device__ __forceinline__ void load(float (&x)[2], const void *p, size_t i)
    {
        const uint32_t v = *reinterpret_cast<const uint32_t *>(reinterpret_cast<const uint16_t *>(p) + i);
        x[0] = __uint_as_float(v << 16); x[1] = __uint_as_float(v & 0xffff0000u);
    }
};

}  // namespace k3kda
