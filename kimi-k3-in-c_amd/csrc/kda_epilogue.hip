// SPDX-License-Identifier: Apache-2.0
// kda_epilogue.hip - K4: head-wise RMSNorm, then the sigmoid output gate (gfx950).
//
// Replaces src/core/k3_ops.c:940-947 up to the o_proj matmul: per (token, head)
//   y = (o_norm[d] * o[d]) * (float)(1/sqrt(mean(o^2) + eps))     k3_rmsnorm, :94-102
//   y = y * sigmoid(gate[d])                                        norm FIRST, then gate
// o_norm[D] is shared by all heads. The mean of squares is a double, as in the reference.
//
// Bound by HBM. Rows are visited grid-stride. kda_epilogue2_kernel (D = 64, 128) packs
// several rows per wave with 16-byte accesses; kda_epilogue_kernel (every D, the small
// shapes of the reference's fixtures) keeps one row per wave, libm expf and a double sum.
#include "kda_internal.h"

namespace k3kda {

template <int D, int GDT, int YDT>
__global__ __launch_bounds__(256) void kda_epilogue_kernel(long rows, int H, float eps,
                                                           const float *__restrict__ o,
                                                           const void *__restrict__ gate,
                                                           const float *__restrict__ wn,
                                                           void *__restrict__ y)
{
#pragma clang fp contract(off)
    constexpr int CPL = D >= 64 ? D / 64 : 1;
    constexpr int NL = D / CPL;
    const int lane = threadIdx.x & 63;
    const bool active = lane < NL;
    const int d0 = (active ? lane : 0) * CPL;
    float w[CPL];
#pragma unroll
    for (int e = 0; e < CPL; e++) w[e] = wn[d0 + e];
    const long nw = (long)gridDim.x * (blockDim.x >> 6);
    for (long r = (long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); r < rows; r += nw) {
        const size_t base = (size_t)r * D + d0;   // rows are (t, h) in [T][H][D] order
        float x[CPL];
        double ss = 0.0;
#pragma unroll
        for (int e = 0; e < CPL; e++) {
            x[e] = o[base + e];
            if (active) ss += (double)x[e] * (double)x[e];
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
        const float inv = (float)(1.0 / sqrt(ss / (double)D + (double)eps));
        if (active) {
#pragma unroll
            for (int e = 0; e < CPL; e++) {
                const float n = (w[e] * x[e]) * inv;
                const float v = n * sigmoid_ref(load_act<GDT>(gate, base + e));
                if constexpr (YDT == K3HIP_BF16) reinterpret_cast<uint16_t *>(y)[base + e] = f2bf(v);
                else reinterpret_cast<float *>(y)[base + e] = v;
            }
        }
    }
    (void)H;
}

// Wide form for D = 64 / 128: LPR = D/4 lanes own one (token, head) row, 4 adjacent
// channels each (16-byte fp32 / 8-byte bf16 accesses), 64/LPR rows per wave instruction.
// The mean of squares is fp32 per lane and double across lanes; sigmoid uses the hardware
// 2^x and reciprocal (about 1 ulp).
// y as a bf16 hi/lo pair (y = hi + lo to about 2^-17), rows [T][2P]: hi in the first P
// columns, lo in the last P -- the input of a K = 2P bf16 GEMM against [W | W].
constexpr int Y_SPLIT = 2;
// y as fp16 [T][P] (the o_proj GEMM's fp16 operand; |y| <= sqrt(D) max|o_norm|)
constexpr int Y_F16 = K3_DT_F16;

template <int D, int GDT, int YDT>
__global__ __launch_bounds__(256) void kda_epilogue2_kernel(long rows, int H, float eps,
                                                            const float *__restrict__ o,
                                                            const void *__restrict__ gate,
                                                            const float *__restrict__ wn,
                                                            void *__restrict__ y)
{
#pragma clang fp contract(off)
    constexpr int LPR = D / 4, RPW = 64 / LPR;
    const int lane = threadIdx.x & 63, sub = lane / LPR, cl = lane % LPR;
    const f4 w = reinterpret_cast<const f4 *>(wn)[cl];
    const long rpb = (long)(blockDim.x >> 6) * RPW, nw = (long)gridDim.x * rpb;
    // rb, the block's first row, is uniform (the base of the bf16 y stores' buffer resource)
    for (long rb = (long)blockIdx.x * rpb; rb < rows; rb += nw) {
        const long r = rb + (long)(threadIdx.x >> 6) * RPW + sub;
        const bool live = r < rows;
        const size_t base = (size_t)(live ? r : rows - 1) * D + 4 * cl;
        const f4 x = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(o + base));   // read once: streamed
        f4 gt;
        if constexpr (GDT == K3HIP_BF16) {
            typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
            const u32x2 uu = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(reinterpret_cast<const uint16_t *>(gate) + base));
            const uint2 u = {uu.x, uu.y};
            gt = f4{__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                    __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u)};
        } else if constexpr (GDT == K3_DT_F16) {
            typedef _Float16 h4 __attribute__((ext_vector_type(4)));
            const h4 u = *reinterpret_cast<const h4 *>(reinterpret_cast<const _Float16 *>(gate) + base);
            gt = f4{(float)u[0], (float)u[1], (float)u[2], (float)u[3]};
        } else {
            gt = *reinterpret_cast<const f4 *>(reinterpret_cast<const float *>(gate) + base);
        }
        double ss = (double)(((x.x * x.x) + (x.y * x.y)) + ((x.z * x.z) + (x.w * x.w)));
#pragma unroll
        for (int m = LPR / 2; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
        const float inv = (float)(1.0 / sqrt(ss / (double)D + (double)eps));
        f4 v;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-gt[e] * 1.4426950408889634f));
            v[e] = ((w[e] * x[e]) * inv) * sg;
        }
        if (live) {
            if constexpr (YDT == Y_F16) {
                uint16_t hv[4];
#pragma unroll
                for (int e = 0; e < 4; e++) hv[e] = __builtin_bit_cast(uint16_t, (_Float16)v[e]);
                *reinterpret_cast<uint2 *>(reinterpret_cast<uint16_t *>(y) + base) =
                    uint2{(uint32_t)hv[0] | ((uint32_t)hv[1] << 16), (uint32_t)hv[2] | ((uint32_t)hv[3] << 16)};
            } else if constexpr (YDT == Y_SPLIT) {
                // row r = t*H + h of y2 [T][2P]: hi at t*2P + h*D, lo P further
                const size_t at = base + (size_t)(r / H) * (size_t)(H * D);
                uint16_t hb[4], lb[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    hb[e] = f2bf(v[e]);
                    lb[e] = f2bf(v[e] - __uint_as_float((uint32_t)hb[e] << 16));
                }
                uint16_t *yy = reinterpret_cast<uint16_t *>(y);
                *reinterpret_cast<uint2 *>(yy + at) = uint2{(uint32_t)hb[0] | ((uint32_t)hb[1] << 16),
                                                           (uint32_t)hb[2] | ((uint32_t)hb[3] << 16)};
                *reinterpret_cast<uint2 *>(yy + at + (size_t)H * D) =
                    uint2{(uint32_t)lb[0] | ((uint32_t)lb[1] << 16), (uint32_t)lb[2] | ((uint32_t)lb[3] << 16)};
            } else if constexpr (YDT == K3HIP_BF16) {
                const uint2 u = {(uint32_t)f2bf(v.x) | ((uint32_t)f2bf(v.y) << 16),
                                 (uint32_t)f2bf(v.z) | ((uint32_t)f2bf(v.w) << 16)};
                // y is not read again by this step: streamed out past the caches with the
                // system-scope non-temporal policy (aux 19 = sc0 | nt | sc1: through to memory,
                // kept in no cache; T=8192, H=32 prefill core: -1% with the compiler's
                // nontemporal store, then 0.5340 -> 0.5325 ms per core step with this one),
                // as a buffer store from the block's first row
                typedef unsigned int u32x2s __attribute__((ext_vector_type(2)));
                const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(
                    reinterpret_cast<uint16_t *>(y) + (size_t)rb * D, (short)0, (int)(rpb * D * 2), 0x00020000);
                __builtin_amdgcn_raw_buffer_store_b64(u32x2s{u.x, u.y}, yr, (int)((size_t)(r - rb) * D + 4 * cl) * 2, 0, 19);
            } else {
                *reinterpret_cast<f4 *>(reinterpret_cast<float *>(y) + base) = v;
            }
        }
    }
}


// bf16 gate -> bf16 y (the prefill core's form) with 8 channels per lane: o as two float4
// loads, the gate and y as one 16-byte access each (the general kernel above takes 4 channels
// per lane, 8-byte gate and y accesses: T=8192, H=32 core step 0.536-0.538 -> 0.532-0.533 ms).
// The same arithmetic, except that a lane's fp32 sum of squares covers its 8 values.
template <int D>
__global__ __launch_bounds__(256) void kda_epilogue8_kernel(long rows, float eps, const float *__restrict__ o,
                                                            const uint16_t *__restrict__ gate,
                                                            const float *__restrict__ wn, uint16_t *__restrict__ y)
{
#pragma clang fp contract(off)
    constexpr int LPR = D / 8, RPW = 64 / LPR;
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const int lane = threadIdx.x & 63, sub = lane / LPR, cl = lane % LPR;
    const f4 w0 = reinterpret_cast<const f4 *>(wn)[2 * cl], w1 = reinterpret_cast<const f4 *>(wn)[2 * cl + 1];
    const long rpb = (long)(blockDim.x >> 6) * RPW, nw = (long)gridDim.x * rpb;
    for (long rb = (long)blockIdx.x * rpb; rb < rows; rb += nw) {
        const long r = rb + (long)(threadIdx.x >> 6) * RPW + sub;
        const bool live = r < rows;
        const size_t base = (size_t)(live ? r : rows - 1) * D + 8 * cl;
        const f4 x0 = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(o + base));
        const f4 x1 = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(o + base + 4));
        const u32x4 gu = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(gate + base));
        float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
        float g[8];
#pragma unroll
        for (int e = 0; e < 4; e++) { g[2 * e] = __uint_as_float(gu[e] << 16); g[2 * e + 1] = __uint_as_float(gu[e] & 0xffff0000u); }
        double ss = (double)((((x[0] * x[0]) + (x[1] * x[1])) + ((x[2] * x[2]) + (x[3] * x[3]))) +
                             (((x[4] * x[4]) + (x[5] * x[5])) + ((x[6] * x[6]) + (x[7] * x[7]))));
#pragma unroll
        for (int m = LPR / 2; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
        const float inv = (float)(1.0 / sqrt(ss / (double)D + (double)eps));
        uint32_t pk[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float v2[2];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const int i = 2 * e + t;
                const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g[i] * 1.4426950408889634f));
                v2[t] = ((wv[i] * x[i]) * inv) * sg;
            }
            pk[e] = (uint32_t)f2bf(v2[0]) | ((uint32_t)f2bf(v2[1]) << 16);
        }
        if (live) {
            const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(y + (size_t)rb * D, (short)0, (int)(rpb * D * 2), 0x00020000);
            __builtin_amdgcn_raw_buffer_store_b128(u32x4{pk[0], pk[1], pk[2], pk[3]}, yr, (int)((size_t)(r - rb) * D + 8 * cl) * 2, 0, 19);
        }
    }
}

template <int D, int GDT, int YDT>
static int launch_epi(long rows, int H, float eps, const float *o, const void *g,
                      const float *wn, void *y, hipStream_t st)
{
    const bool wide = D >= 64 && ((uintptr_t)o | (uintptr_t)g | (uintptr_t)y | (uintptr_t)wn) % 16 == 0;
    if constexpr (D >= 64 && GDT == K3HIP_BF16 && YDT == K3HIP_BF16) {
        if (wide) {
            long blocks = (rows + 4 * (512 / D) - 1) / (4 * (512 / D));
            if (blocks > 16384) blocks = 16384;
            hipLaunchKernelGGL((kda_epilogue8_kernel<D>), dim3((unsigned)blocks), dim3(256), 0, st, rows, eps, o,
                               (const uint16_t *)g, wn, (uint16_t *)y);
            K3_LAUNCHED();
            return K3HIP_OK;
        }
    }
    if (wide) {
        long blocks = (rows + 4 * (256 / D) - 1) / (4 * (256 / D));
        if (blocks > 16384) blocks = 16384;
        if constexpr (D >= 64)
            hipLaunchKernelGGL((kda_epilogue2_kernel<D, GDT, YDT>), dim3((unsigned)blocks), dim3(256), 0,
                               st, rows, H, eps, o, g, wn, y);
    } else {
        long blocks = (rows + 3) / 4;
        if (blocks > 8192) blocks = 8192;
        hipLaunchKernelGGL((kda_epilogue_kernel<D, GDT, YDT>), dim3((unsigned)blocks), dim3(256), 0,
                           st, rows, H, eps, o, g, wn, y);
    }
    K3_LAUNCHED();
    return K3HIP_OK;
}

template <int D>
static int epi_types(int gdt, int ydt, long rows, int H, float eps, const float *o,
                     const void *g, const float *wn, void *y, hipStream_t st)
{
    if (gdt == K3HIP_F32 && ydt == K3HIP_F32) return launch_epi<D, K3HIP_F32, K3HIP_F32>(rows, H, eps, o, g, wn, y, st);
    if (gdt == K3HIP_F32 && ydt == K3HIP_BF16) return launch_epi<D, K3HIP_F32, K3HIP_BF16>(rows, H, eps, o, g, wn, y, st);
    if (gdt == K3HIP_BF16 && ydt == K3HIP_F32) return launch_epi<D, K3HIP_BF16, K3HIP_F32>(rows, H, eps, o, g, wn, y, st);
    if (gdt == K3HIP_BF16 && ydt == K3HIP_BF16) return launch_epi<D, K3HIP_BF16, K3HIP_BF16>(rows, H, eps, o, g, wn, y, st);
    K3_FAIL(K3HIP_EINVAL, "k3hip_kda_epilogue: gate_dtype=%d y_dtype=%d", gdt, ydt);
}

int epilogue_split(int T, int H, int D, float eps, const float *o, const void *gate, int gate_dtype,
                   const float *o_norm, void *y2, hipStream_t st, bool y_f16)
{
    const long rows = (long)T * H;
    if (rows == 0) return K3HIP_OK;
    if ((D != 64 && D != 128) ||
        ((uintptr_t)o | (uintptr_t)gate | (uintptr_t)o_norm | (uintptr_t)y2) % 16)
        K3_FAIL(K3HIP_EUNSUPPORTED, "epilogue_split: D=%d or unaligned buffers", D);
    long blocks = (rows + 4 * (256 / D) - 1) / (4 * (256 / D));
    if (blocks > 16384) blocks = 16384;
    const bool g16 = gate_dtype == K3HIP_BF16;
    if (y_f16) {
#define K3_EPI16(DD, G) hipLaunchKernelGGL((kda_epilogue2_kernel<DD, G, Y_F16>), dim3((unsigned)blocks), dim3(256), 0, st, rows, H, eps, o, gate, o_norm, y2)
        if (gate_dtype == K3_DT_F16) { if (D == 128) K3_EPI16(128, K3_DT_F16); else K3_EPI16(64, K3_DT_F16); }
        else if (D == 128) { if (g16) K3_EPI16(128, K3HIP_BF16); else K3_EPI16(128, K3HIP_F32); }
        else { if (g16) K3_EPI16(64, K3HIP_BF16); else K3_EPI16(64, K3HIP_F32); }
#undef K3_EPI16
        K3_LAUNCHED();
        return K3HIP_OK;
    }
    if (D == 128) {
        if (g16) hipLaunchKernelGGL((kda_epilogue2_kernel<128, K3HIP_BF16, Y_SPLIT>), dim3((unsigned)blocks), dim3(256), 0, st, rows, H, eps, o, gate, o_norm, y2);
        else hipLaunchKernelGGL((kda_epilogue2_kernel<128, K3HIP_F32, Y_SPLIT>), dim3((unsigned)blocks), dim3(256), 0, st, rows, H, eps, o, gate, o_norm, y2);
    } else {
        if (g16) hipLaunchKernelGGL((kda_epilogue2_kernel<64, K3HIP_BF16, Y_SPLIT>), dim3((unsigned)blocks), dim3(256), 0, st, rows, H, eps, o, gate, o_norm, y2);
        else hipLaunchKernelGGL((kda_epilogue2_kernel<64, K3HIP_F32, Y_SPLIT>), dim3((unsigned)blocks), dim3(256), 0, st, rows, H, eps, o, gate, o_norm, y2);
    }
    K3_LAUNCHED();
    return K3HIP_OK;
}

}  // namespace k3kda

using namespace k3kda;

extern "C" int k3hip_kda_epilogue(int T, int H, int D, float rms_eps, const float *o,
                                  const void *gate, int gate_dtype, const float *o_norm, void *y,
                                  int y_dtype, void *stream)
{
    clear_error();
    if (T < 0 || H < 0) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_epilogue: T=%d H=%d", T, H);
    const long rows = (long)T * H;
    if (rows == 0) return K3HIP_OK;
    if (!o || !gate || !o_norm || !y) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_epilogue: NULL tensor");
    hipStream_t st = as_stream(stream);
    switch (D) {
    case 16: return epi_types<16>(gate_dtype, y_dtype, rows, H, rms_eps, o, gate, o_norm, y, st);
    case 32: return epi_types<32>(gate_dtype, y_dtype, rows, H, rms_eps, o, gate, o_norm, y, st);
    case 64: return epi_types<64>(gate_dtype, y_dtype, rows, H, rms_eps, o, gate, o_norm, y, st);
    case 128: return epi_types<128>(gate_dtype, y_dtype, rows, H, rms_eps, o, gate, o_norm, y, st);
    default: K3_FAIL(K3HIP_EUNSUPPORTED, "k3hip_kda_epilogue: D=%d not in {16,32,64,128}", D);
    }
}
