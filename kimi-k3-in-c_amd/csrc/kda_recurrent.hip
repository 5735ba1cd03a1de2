// SPDX-License-Identifier: Apache-2.0
// kda_recurrent.hip - sequential-in-T KDA prefill on the GPU (gfx950).
//
// Runs, per head, the reference recurrence token by token (src/core/k3_ops.c:927-938
// calling k3_kda_step, :186-243). Value columns of the state are independent of each
// other (the decay scales rows and the delta write of column j needs only u[j]), so one
// lane owns one column S[:, j] in registers and walks the rows in the reference's order:
//   s_i *= alpha_i;  u += k_i s_i;  s_i += (k_i beta)(v_j - u);  o += q_i s_i
// with the reference's k_i == 0 / q_i == 0 row skips and contraction off. The results
// therefore equal the CPU reference bit for bit, which makes this kernel the second GPU
// opinion the chunked kernel is checked against, and the fallback for gate bounds outside
// the chunked kernel's exponent range.
//
// Only H * D/64 waves run, each serial over T: this is a correctness path, not the
// throughput path.
#include "k3kda_common.h"

namespace k3kda {

constexpr int REC_TT = 16;   // tokens staged in LDS per step

template <int D>
__global__ __launch_bounds__(D < 64 ? D : 64) void kda_recurrent_kernel(
    int T, int H, const float *__restrict__ q, const float *__restrict__ k,
    const float *__restrict__ v, const float *__restrict__ alpha, const float *__restrict__ beta,
    float q_scale, float *__restrict__ S, float *__restrict__ o)
{
#pragma clang fp contract(off)
    constexpr int NJ = D < 64 ? D : 64;   // columns per workgroup = threads
    __shared__ float s_q[REC_TT][D], s_k[REC_TT][D], s_a[REC_TT][D];
    __shared__ float s_v[REC_TT][NJ], s_b[REC_TT];
    const int h = blockIdx.x;
    const int j = blockIdx.y * NJ + threadIdx.x;
    const size_t P = (size_t)H * D;
    float *Sh = S + (size_t)h * D * D;
    float s[D];
#pragma unroll
    for (int i = 0; i < D; i++) s[i] = Sh[(size_t)i * D + j];

    for (int tb = 0; tb < T; tb += REC_TT) {
        const int nt = min(REC_TT, T - tb);
        __syncthreads();
        for (int e = threadIdx.x; e < nt * D; e += NJ) {
            const int tt = e / D, i = e % D;
            const size_t at = (size_t)(tb + tt) * P + (size_t)h * D + i;
            s_q[tt][i] = q[at] * q_scale;
            s_k[tt][i] = k[at];
            s_a[tt][i] = alpha[at];
        }
        for (int tt = 0; tt < nt; tt++) s_v[tt][threadIdx.x] = v[(size_t)(tb + tt) * P + (size_t)h * D + j];
        if (threadIdx.x < nt) s_b[threadIdx.x] = beta[(size_t)(tb + threadIdx.x) * H + h];
        __syncthreads();
        for (int tt = 0; tt < nt; tt++) {
            float u = 0.0f;
#pragma unroll
            for (int i = 0; i < D; i++) {
                s[i] = s[i] * s_a[tt][i];
                const float ki = s_k[tt][i];
                if (ki != 0.0f) u = u + ki * s[i];
            }
            const float d = s_v[tt][threadIdx.x] - u;
            const float b = s_b[tt];
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < D; i++) {
                const float ki = s_k[tt][i];
                if (ki != 0.0f) s[i] = s[i] + (ki * b) * d;
                const float qi = s_q[tt][i];
                if (qi != 0.0f) acc = acc + qi * s[i];
            }
            o[(size_t)(tb + tt) * P + (size_t)h * D + j] = acc;
        }
    }
#pragma unroll
    for (int i = 0; i < D; i++) Sh[(size_t)i * D + j] = s[i];
}

template <int D>
static int launch_rec(int T, int H, const float *q, const float *k, const float *v,
                      const float *a, const float *b, float qs, float *S, float *o, hipStream_t st)
{
    constexpr int NJ = D < 64 ? D : 64;
    hipLaunchKernelGGL((kda_recurrent_kernel<D>), dim3(H, D / NJ), dim3(NJ), 0, st, T, H, q, k, v,
                       a, b, qs, S, o);
    K3_LAUNCHED();
    return K3HIP_OK;
}

}  // namespace k3kda

using namespace k3kda;

extern "C" int k3hip_kda_recurrent(int T, int H, int D, const float *q, const float *k,
                                   const float *v, const float *alpha, const float *beta,
                                   float q_scale, float *S, float *o, void *stream)
{
    clear_error();
    if (T < 0 || H < 0) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_recurrent: T=%d H=%d", T, H);
    if (T == 0 || H == 0) return K3HIP_OK;
    if (H > 65535) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_recurrent: H=%d", H);
    if (!q || !k || !v || !alpha || !beta || !S || !o)
        K3_FAIL(K3HIP_EINVAL, "k3hip_kda_recurrent: NULL tensor");
    hipStream_t st = as_stream(stream);
    switch (D) {
    case 16: return launch_rec<16>(T, H, q, k, v, alpha, beta, q_scale, S, o, st);
    case 32: return launch_rec<32>(T, H, q, k, v, alpha, beta, q_scale, S, o, st);
    case 64: return launch_rec<64>(T, H, q, k, v, alpha, beta, q_scale, S, o, st);
    case 128: return launch_rec<128>(T, H, q, k, v, alpha, beta, q_scale, S, o, st);
    default: K3_FAIL(K3HIP_EUNSUPPORTED, "k3hip_kda_recurrent: D=%d not in {16,32,64,128}", D);
    }
}
