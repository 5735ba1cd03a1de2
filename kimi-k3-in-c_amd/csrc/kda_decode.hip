// SPDX-License-Identifier: Apache-2.0
// kda_decode.hip - K3: batched single-token KDA recurrence (decode) for gfx950.
//
// Replaces, per (sequence b, head h), k3_kda_step(S, o, q*q_scale, k, v, alpha, beta)
// of the reference (src/core/k3_ops.c:186-243, driven at :927-938 with T = 1):
//   1. S[i][:] *= alpha[i]
//   2. u = S^T k                      (rows with k[i] == 0 contribute nothing)
//   3. S[i][j] += (k[i]*beta)*(v[j]-u[j])
//   4. o = S^T q from the UPDATED S   (q already scaled)
//
// The work is bound by HBM: each (b, h) owns a D x D fp32 state that must be read once
// and written once per token (2*D*D*4 bytes) against ~7*D*D flops. One workgroup holds
// its whole state in registers between the read and the write: NT threads, each owning
// NPASS float4s at rows rs, rs+RPP, ... of column group cg. A pass over the rows is one
// contiguous D*RPP*4-byte span of S per instruction, so every wave issues full 64-byte
// segments. The two reductions over rows (u, then o) go through LDS. The state is read
// with nontemporal loads and written back with system-scope non-temporal stores (the
// `sc0 sc1 nt` cache policy: through to memory, not kept in any cache): it streams through.
// Nontemporal stores measured 54.5 -> 45.5 us per B=64, H=32, D=128 step (5.0 -> 6.0 TB/s)
// on MI355X, the loads a further ~0.6 us; the system-scope form of the stores 49.6 -> 48.0
// us against the compiler's nontemporal store on one box (48.5 for a plain `nt` store,
// 48.5 with the loads in that form too).
// D = 128 uses 512 threads (8 float4s each, 60 VGPRs, 8 waves per SIMD): the 2,048 states
// of a B=64 step then run as two full rounds of 1,024 workgroups; with 256 threads
// (16 float4s, 90 VGPRs, 5 waves per SIMD) they ran as 1,280 + 768, about 1.5% slower.
//
// Element arithmetic is kept in the reference's order with contraction off (decay
// multiply, then products added separately); only the summation order of the two row
// reductions differs (per-thread partial sums, then across row slots).
#include "kda_internal.h"

namespace k3kda {

// One 16-byte state store, `off` bytes into the state, with the system-scope non-temporal
// policy (aux 19 = sc0 | nt | sc1: through to memory): a buffer store the compiler sees as
// one, so the wait states before a VALU overwrite of its data registers are its own.
__device__ __forceinline__ void store_stream(__amdgpu_buffer_rsrc_t r, int off, const f4 &v)
{
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, 19);
}

template <int D, int NT>
__global__ __launch_bounds__(NT) void kda_decode_kernel(
    float *__restrict__ S, float *__restrict__ o, const float *__restrict__ q,
    const float *__restrict__ k, const float *__restrict__ v, const float *__restrict__ alpha,
    const float *__restrict__ beta, float q_scale, int H, long s_stride)
{
#pragma clang fp contract(off)
    constexpr int CPR = D / 4;      // float4 column groups per row
    constexpr int RPP = NT / CPR;   // rows covered by one pass of the workgroup
    constexpr int NPASS = D / RPP;  // passes (float4s held per thread)
    static_assert(CPR * RPP == NT && NPASS * RPP == D, "tile shape");

    __shared__ float s_k[D], s_q[D], s_a[D];
    __shared__ f4 s_red[RPP][CPR];
    __shared__ f4 s_u[CPR];

    const int pair = blockIdx.x;
    const int tid = threadIdx.x;
    const int cg = tid % CPR;
    const int rs = tid / CPR;
    const size_t vo = (size_t)pair * D;

    if (tid < D) {
        s_k[tid] = k[vo + tid];
        s_q[tid] = q[vo + tid] * q_scale;
        s_a[tid] = alpha[vo + tid];
    }
    // sequence pair / H's state starts s_stride floats after the previous one's
    f4 *Sp = reinterpret_cast<f4 *>(S + (size_t)(pair / H) * s_stride + (size_t)(pair % H) * D * D);
    const __amdgpu_buffer_rsrc_t Sr = __builtin_amdgcn_make_buffer_rsrc(Sp, (short)0, D * D * 4, 0x00020000);
    f4 s[NPASS];
#pragma unroll
    for (int m = 0; m < NPASS; m++) s[m] = __builtin_nontemporal_load(&Sp[(rs + m * RPP) * CPR + cg]);
    const f4 vv = reinterpret_cast<const f4 *>(v + vo)[cg];
    const float b = beta[pair];
    __syncthreads();

    // 1-2. decay the rows, partial u over this thread's rows
    f4 u = 0.0f;
#pragma unroll
    for (int m = 0; m < NPASS; m++) {
        const int r = rs + m * RPP;
        const float kr = s_k[r];
        s[m] = s[m] * s_a[r];
        if (kr != 0.0f) u = u + kr * s[m];
    }
    s_red[rs][cg] = u;
    __syncthreads();
    if (tid < CPR) {
        f4 t = s_red[0][tid];
#pragma unroll
        for (int r = 1; r < RPP; r++) t = t + s_red[r][tid];
        s_u[tid] = t;
    }
    __syncthreads();

    // 3-4. delta write, partial o from the updated rows
    const f4 d = vv - s_u[cg];
    f4 acc = 0.0f;
#pragma unroll
    for (int m = 0; m < NPASS; m++) {
        const int r = rs + m * RPP;
        const float kr = s_k[r], qr = s_q[r];
        if (kr != 0.0f) s[m] = s[m] + (kr * b) * d;
        if (qr != 0.0f) acc = acc + qr * s[m];
        store_stream(Sr, ((rs + m * RPP) * CPR + cg) * 16, s[m]);
    }
    s_red[rs][cg] = acc;   // every read of s_red above finished before the last barrier
    __syncthreads();
    if (tid < CPR) {
        f4 t = s_red[0][tid];
#pragma unroll
        for (int r = 1; r < RPP; r++) t = t + s_red[r][tid];
        reinterpret_cast<f4 *>(o + vo)[tid] = t;
    }
}

template <int D, int NT>
static int launch_decode(int pairs, float *S, float *o, const float *q, const float *k,
                         const float *v, const float *alpha, const float *beta, float qs,
                         int H, long s_stride, hipStream_t st)
{
    hipLaunchKernelGGL((kda_decode_kernel<D, NT>), dim3(pairs), dim3(NT), 0, st, S, o, q, k,
                       v, alpha, beta, qs, H, s_stride);
    K3_LAUNCHED();
    return K3HIP_OK;
}

int decode_strided(int B, int H, int D, float *S, long s_stride, float *o, const float *q,
                   const float *k, const float *v, const float *alpha, const float *beta,
                   float qs, hipStream_t st)
{
    const long pairs = (long)B * H;
    if (pairs == 0) return K3HIP_OK;
    if (pairs > 0x7fffffffL) K3_FAIL(K3HIP_EINVAL, "decode: B*H=%ld too large", pairs);
    if (!is_pow2_head(D)) K3_FAIL(K3HIP_EUNSUPPORTED, "decode: D=%d not in {16,32,64,128}", D);
    if (s_stride < (long)H * D * D || (s_stride & 3) || (((uintptr_t)S | (uintptr_t)o | (uintptr_t)v) & 15))
        K3_FAIL(K3HIP_EINVAL, "decode: state stride %ld or alignment", s_stride);
    switch (D) {
    case 16: return launch_decode<16, 64>((int)pairs, S, o, q, k, v, alpha, beta, qs, H, s_stride, st);
    case 32: return launch_decode<32, 128>((int)pairs, S, o, q, k, v, alpha, beta, qs, H, s_stride, st);
    case 64: return launch_decode<64, 256>((int)pairs, S, o, q, k, v, alpha, beta, qs, H, s_stride, st);
    default: return launch_decode<128, 512>((int)pairs, S, o, q, k, v, alpha, beta, qs, H, s_stride, st);
    }
}

}  // namespace k3kda

using namespace k3kda;

extern "C" int k3hip_kda_decode(int B, int H, int D, float *S, float *o, const float *q,
                                const float *k, const float *v, const float *alpha,
                                const float *beta, float q_scale, void *stream)
{
    clear_error();
    if (B < 0 || H < 0) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_decode: B=%d H=%d", B, H);
    if (!is_pow2_head(D)) K3_FAIL(K3HIP_EUNSUPPORTED, "k3hip_kda_decode: D=%d not in {16,32,64,128}", D);
    const long pairs = (long)B * H;
    if (pairs == 0) return K3HIP_OK;
    if (pairs > 0x7fffffffL) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_decode: B*H=%ld too large", pairs);
    if (!S || !o || !q || !k || !v || !alpha || !beta)
        K3_FAIL(K3HIP_EINVAL, "k3hip_kda_decode: NULL tensor");
    if (((uintptr_t)S | (uintptr_t)o | (uintptr_t)v) & 15)
        K3_FAIL(K3HIP_EINVAL, "k3hip_kda_decode: S, o and v must be 16-byte aligned");
    return decode_strided(B, H, D, S, (long)H * D * D, o, q, k, v, alpha, beta, q_scale,
                          as_stream(stream));
}
