// SPDX-License-Identifier: Apache-2.0
// kda_prep.hip - K1: ShortConv + SiLU, L2-norm, beta and the decay chain (gfx950).
//
// Replaces steps 2-5 of the reference k3_kda_layer (src/core/k3_ops.c:888-906):
//   k3_shortconv (:133-165) on q, k, v     acc = w[K-1]*x_t, then += w[j]*x_{t-K+1+j}
//                                           oldest first; y = acc * sigmoid(acc)
//   l2norm_ (:845-851) on q and k          v *= 1/sqrt(sum v^2 + 1e-6); the reference sums
//                                           in double, kda_prep2_kernel in fp32
//   beta = sigmoid(b_logit) (:903)         one scalar per (token, head)
//   k3_kda_decay (:168-183)                g = lb*sigmoid(expf(A_log[h])*(z+dt_bias)),
//                                           alpha = expf(g)
// gate_lb == 0 selects the gate without a lower bound, g = -expf(A_log[h])*softplus(z+dt_bias)
// (the form the reference records as the one it replaced, tools/k3_ref.py:54-59; it has no
// reference implementation and is checked against its closed form only).
//
// Bound by HBM. A run of consecutive tokens of one head belongs to one (half-)wave; each
// lane owns adjacent channels of the head, so a row of the head is one coalesced access.
// The K-1 previous inputs of each channel live in registers as a sliding window, so every
// input element is loaded once. Contraction is off: the conv taps are added in the
// reference's order with separate rounding. Two forms: kda_prep2_kernel (D = 64, 128)
// with wide accesses and hardware transcendentals, and kda_prep_kernel (D = 16, 32, the
// small shapes of the reference's fixtures) with libm expf and double sums throughout.
//
// The incoming conv history is only read here. kda_conv_state_kernel, launched after on
// the same stream, writes the outgoing history, so no wave can overwrite history that
// another wave has not read yet.
#include "kda_internal.h"
#include "kda_prep_math.h"

namespace k3kda {

constexpr int PREP_WAVES = 4;   // waves per workgroup
constexpr int PREP_TT = 16;     // tokens per wave

template <int D, int K, int DT>
__global__ __launch_bounds__(64 * PREP_WAVES) void kda_prep_kernel(
    int T, int H, float lb, const void *__restrict__ q_in, const void *__restrict__ k_in,
    const void *__restrict__ v_in, const float *__restrict__ z, const float *__restrict__ b_logit,
    const float *__restrict__ q_conv, const float *__restrict__ k_conv,
    const float *__restrict__ v_conv, const float *__restrict__ A_log,
    const float *__restrict__ dt_bias, const float *__restrict__ conv_state,
    float *__restrict__ q_out, float *__restrict__ k_out, float *__restrict__ v_out,
    float *__restrict__ g_out, float *__restrict__ alpha_out, float *__restrict__ beta_out)
{
#pragma clang fp contract(off)
    constexpr int CPL = D >= 64 ? D / 64 : 1;   // channels per lane
    constexpr int NL = D / CPL;                  // active lanes
    constexpr int NH = K - 1;                    // history length
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int h = blockIdx.x;
    const int t0 = (blockIdx.y * PREP_WAVES + wave) * PREP_TT;
    if (t0 >= T) return;
    const int t1 = min(T, t0 + PREP_TT);
    const bool active = lane < NL;
    const size_t P = (size_t)H * D;
    const int c0 = h * D + (active ? lane : 0) * CPL;   // first channel of this lane

    // taps and windows: [tensor][channel-in-lane][tap]
    float w[3][CPL][K];
    float win[3][CPL][NH > 0 ? NH : 1];
    const float *convw[3] = {q_conv, k_conv, v_conv};
    const void *xin[3] = {q_in, k_in, v_in};
#pragma unroll
    for (int b = 0; b < 3; b++)
#pragma unroll
        for (int e = 0; e < CPL; e++) {
#pragma unroll
            for (int j = 0; j < K; j++) w[b][e][j] = convw[b][(size_t)(c0 + e) * K + j];
#pragma unroll
            for (int j = 0; j < NH; j++) {
                const int p = t0 - NH + j;   // input position held in window slot j
                float val = 0.0f;
                if (p >= 0) val = load_act<DT>(xin[b], (size_t)p * P + c0 + e);
                else if (conv_state) val = conv_state[((size_t)b * P + c0 + e) * NH + (p + NH)];
                win[b][e][j] = val;
            }
        }
    float dtb[CPL];
#pragma unroll
    for (int e = 0; e < CPL; e++) dtb[e] = dt_bias[c0 + e];
    const float a = expf(A_log[h]);

    for (int t = t0; t < t1; t++) {
        const size_t row = (size_t)t * P;
        float y[3][CPL];
#pragma unroll
        for (int b = 0; b < 3; b++)
#pragma unroll
            for (int e = 0; e < CPL; e++) {
                const float cur = load_act<DT>(xin[b], row + c0 + e);
                float acc = w[b][e][NH] * cur;
#pragma unroll
                for (int j = 0; j < NH; j++) acc = acc + w[b][e][j] * win[b][e][j];
#pragma unroll
                for (int j = 1; j < NH; j++) win[b][e][j - 1] = win[b][e][j];
                if constexpr (NH > 0) win[b][e][NH - 1] = cur;
                y[b][e] = acc * sigmoid_ref(acc);
            }
        // L2 over the head for q (b=0) and k (b=1); the sums are exact-order-free doubles
#pragma unroll
        for (int b = 0; b < 2; b++) {
            double ss = 0.0;
            if (active)
#pragma unroll
                for (int e = 0; e < CPL; e++) ss += (double)y[b][e] * (double)y[b][e];
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
            const float r = (float)(1.0 / sqrt(ss + 1e-6));
#pragma unroll
            for (int e = 0; e < CPL; e++) y[b][e] = y[b][e] * r;
        }
        if (active) {
#pragma unroll
            for (int e = 0; e < CPL; e++) {
                const size_t i = row + c0 + e;
                q_out[i] = y[0][e];
                k_out[i] = y[1][e];
                v_out[i] = y[2][e];
                float gi;
                if (lb != 0.0f) gi = lb * sigmoid_ref(a * (z[i] + dtb[e]));
                else gi = -a * softplus_ref(z[i] + dtb[e]);   // no lower bound: softplus gate
                if (g_out) g_out[i] = gi;
                if (alpha_out) alpha_out[i] = expf(gi);
            }
        }
        if (lane == 0) beta_out[(size_t)t * H + h] = sigmoid_ref(b_logit[(size_t)t * H + h]);
    }
}

// Wide form for D = 64 / 128 (the throughput path). A wave holds two independent runs of
// PREP2_TT tokens, one per half-wave; each of the 32 lanes of a half owns CPL = D/32
// adjacent channels of the head, so rows are read and written with 8- or 16-byte accesses.
// The arithmetic is that of kda_prep_math.h (hardware 2^x, reciprocal and reciprocal square
// root; fp32 L2 sums), shared with the fused prefill kernel.
constexpr int PREP2_TT = 16;   // tokens per half-wave run

template <int CPL>
__device__ __forceinline__ void store_row(float *p, size_t i, const float (&x)[CPL])
{
    if constexpr (CPL == 4) *reinterpret_cast<f4 *>(p + i) = f4{x[0], x[1], x[2], x[3]};
    else *reinterpret_cast<f2 *>(p + i) = f2{x[0], x[1]};
}

template <int D, int K, int DT>
__global__ __launch_bounds__(256) void kda_prep2_kernel(
    int T, int H, float lb, const void *__restrict__ q_in, const void *__restrict__ k_in,
    const void *__restrict__ v_in, const float *__restrict__ z, const float *__restrict__ b_logit,
    const float *__restrict__ q_conv, const float *__restrict__ k_conv,
    const float *__restrict__ v_conv, const float *__restrict__ A_log,
    const float *__restrict__ dt_bias, const float *__restrict__ conv_state,
    float *__restrict__ q_out, float *__restrict__ k_out, float *__restrict__ v_out,
    float *__restrict__ g_out, float *__restrict__ alpha_out, float *__restrict__ beta_out)
{
#pragma clang fp contract(off)
    constexpr int CPL = D / 32;
    constexpr int NH = K - 1;
    const int lane = threadIdx.x & 63, half = lane >> 5, l32 = lane & 31;
    const int run = (blockIdx.y * 4 + (threadIdx.x >> 6)) * 2 + half;
    const int h = blockIdx.x;
    const int t0 = run * PREP2_TT;
    const int t1 = min(T, t0 + PREP2_TT);
    const size_t P = (size_t)H * D;
    const int c0 = h * D + l32 * CPL;
    const float *convw[3] = {q_conv, k_conv, v_conv};
    const void *xin[3] = {q_in, k_in, v_in};
    float w[3][CPL][K], win[3][CPL][NH > 0 ? NH : 1], dtb[CPL];
#pragma unroll
    for (int b = 0; b < 3; b++)
#pragma unroll
        for (int e = 0; e < CPL; e++) {
#pragma unroll
            for (int j = 0; j < K; j++) w[b][e][j] = convw[b][(size_t)(c0 + e) * K + j];
#pragma unroll
            for (int j = 0; j < NH; j++) {
                const int p = t0 - NH + j;
                float val = 0.0f;
                if (t0 < T) {
                    if (p >= 0) val = load_act<DT>(xin[b], (size_t)p * P + c0 + e);
                    else if (conv_state) val = conv_state[((size_t)b * P + c0 + e) * NH + (p + NH)];
                }
                win[b][e][j] = val;
            }
        }
#pragma unroll
    for (int e = 0; e < CPL; e++) dtb[e] = dt_bias[c0 + e];
    const float a = expf(A_log[h]);

    // Both halves run the same number of iterations (the shorter one masks its stores) so
    // the cross-lane reductions see every lane of the half active.
    for (int t = t0; t < t0 + PREP2_TT; t++) {
        const bool live = t < t1;
        const size_t row = (size_t)min(t, T - 1) * P;
        float y[3][CPL];
#pragma unroll
        for (int b = 0; b < 3; b++) {
            float cur[CPL];
            RowIO<CPL, DT>::load(cur, xin[b], row + c0);
#pragma unroll
            for (int e = 0; e < CPL; e++) {
                y[b][e] = conv_silu<K>(w[b][e], win[b][e], cur[e]);
#pragma unroll
                for (int j = 1; j < NH; j++) win[b][e][j - 1] = win[b][e][j];
                if constexpr (NH > 0) win[b][e][NH - 1] = cur[e];
            }
        }
        l2norm_half<CPL>(y[0]);
        l2norm_half<CPL>(y[1]);
        if (live) {
            float zz[CPL], gv[CPL], av[CPL];
            RowIO<CPL, K3HIP_F32>::load(zz, z, row + c0);
#pragma unroll
            for (int e = 0; e < CPL; e++) {
                if (lb != 0.0f) gv[e] = gate_bounded(lb, gate_a2(a), zz[e], dtb[e]);
                else gv[e] = -a * softplus_ref(zz[e] + dtb[e]);   // no lower bound: softplus gate
                av[e] = fast_exp(gv[e]);
            }
            store_row<CPL>(q_out, row + c0, y[0]);
            store_row<CPL>(k_out, row + c0, y[1]);
            store_row<CPL>(v_out, row + c0, y[2]);
            if (g_out) store_row<CPL>(g_out, row + c0, gv);
            if (alpha_out) store_row<CPL>(alpha_out, row + c0, av);
            if (l32 == 0) beta_out[(size_t)t * H + h] = fast_sigmoid(b_logit[(size_t)t * H + h]);
        }
    }
}

// Outgoing conv history: slot j of channel c holds the input at position T-(K-1)+j,
// taken from the incoming history when that position is before the first token.
template <int DT>
__global__ void kda_conv_state_kernel(int T, int P, int K, const void *__restrict__ q_in,
                                      const void *__restrict__ k_in, const void *__restrict__ v_in,
                                      float *__restrict__ conv_state)
{
    const int NH = K - 1;
    const long n = (long)3 * P * NH;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int j = (int)(i % NH);
    const long bc = i / NH;
    const int c = (int)(bc % P);
    const int b = (int)(bc / P);
    const int p = T - NH + j;
    if (p < 0) return;   // this slot keeps an older history value, which shifts below
    const void *src = b == 0 ? q_in : (b == 1 ? k_in : v_in);
    (void)c;
    conv_state[i] = load_act<DT>(src, (size_t)p * P + c);
}

// For T < K-1 the history shifts by T inside itself: slot j takes old slot j+T. Done by
// one thread per channel, in increasing j, before any new input is placed.
__global__ void kda_conv_shift_kernel(int T, int P, int K, float *__restrict__ conv_state)
{
    const int NH = K - 1;
    const long bc = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (bc >= (long)3 * P) return;
    float *hs = conv_state + bc * NH;
    for (int j = 0; j + T < NH; j++) hs[j] = hs[j + T];
}

int conv_state_update(int T, int P, int K, int dt, const void *qi, const void *ki, const void *vi,
                      float *cs, hipStream_t st)
{
    if (!cs || K <= 1) return K3HIP_OK;
    if (T < K - 1) {
        const long n = 3L * P;
        hipLaunchKernelGGL(kda_conv_shift_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                           T, P, K, cs);
        K3_LAUNCHED();
    }
    const long n = 3L * P * (K - 1);
    if (dt == K3HIP_BF16)
        hipLaunchKernelGGL((kda_conv_state_kernel<K3HIP_BF16>), dim3((unsigned)((n + 255) / 256)),
                           dim3(256), 0, st, T, P, K, qi, ki, vi, cs);
    else
        hipLaunchKernelGGL((kda_conv_state_kernel<K3HIP_F32>), dim3((unsigned)((n + 255) / 256)),
                           dim3(256), 0, st, T, P, K, qi, ki, vi, cs);
    K3_LAUNCHED();
    return K3HIP_OK;
}

template <int D, int K, int DT>
static int launch_prep(int T, int H, float lb, const void *qi, const void *ki, const void *vi,
                       const float *z, const float *bl, const float *qc, const float *kc,
                       const float *vc, const float *A, const float *dt, float *cs, float *qo,
                       float *ko, float *vo, float *go, float *ao, float *bo, hipStream_t st)
{
    // the wide form reads and writes 16-byte aligned channel groups
    const bool wide = D >= 64 && ((uintptr_t)qi | (uintptr_t)ki | (uintptr_t)vi | (uintptr_t)z |
                                  (uintptr_t)qo | (uintptr_t)ko | (uintptr_t)vo | (uintptr_t)go |
                                  (uintptr_t)ao) % 16 == 0;
    if (D >= 64 && wide) {
        const int per_block = 8 * PREP2_TT;   // 4 waves x 2 runs
        dim3 grid(H, (T + per_block - 1) / per_block);
        if constexpr (D >= 64)
            hipLaunchKernelGGL((kda_prep2_kernel<D, K, DT>), grid, dim3(256), 0, st, T, H, lb, qi,
                               ki, vi, z, bl, qc, kc, vc, A, dt, cs, qo, ko, vo, go, ao, bo);
    } else {
        const int per_block = PREP_WAVES * PREP_TT;
        dim3 grid(H, (T + per_block - 1) / per_block);
        hipLaunchKernelGGL((kda_prep_kernel<D, K, DT>), grid, dim3(64 * PREP_WAVES), 0, st, T, H,
                           lb, qi, ki, vi, z, bl, qc, kc, vc, A, dt, cs, qo, ko, vo, go, ao, bo);
    }
    K3_LAUNCHED();
    return conv_state_update(T, H * D, K, DT, qi, ki, vi, cs, st);
}

template <int D, int DT>
static int prep_k(int K, int T, int H, float lb, const void *qi, const void *ki, const void *vi,
                  const float *z, const float *bl, const float *qc, const float *kc,
                  const float *vc, const float *A, const float *dt, float *cs, float *qo,
                  float *ko, float *vo, float *go, float *ao, float *bo, hipStream_t st)
{
    switch (K) {
    case 1: return launch_prep<D, 1, DT>(T, H, lb, qi, ki, vi, z, bl, qc, kc, vc, A, dt, cs, qo, ko, vo, go, ao, bo, st);
    case 2: return launch_prep<D, 2, DT>(T, H, lb, qi, ki, vi, z, bl, qc, kc, vc, A, dt, cs, qo, ko, vo, go, ao, bo, st);
    case 3: return launch_prep<D, 3, DT>(T, H, lb, qi, ki, vi, z, bl, qc, kc, vc, A, dt, cs, qo, ko, vo, go, ao, bo, st);
    case 4: return launch_prep<D, 4, DT>(T, H, lb, qi, ki, vi, z, bl, qc, kc, vc, A, dt, cs, qo, ko, vo, go, ao, bo, st);
    default: K3_FAIL(K3HIP_EUNSUPPORTED, "k3hip_kda_prep: conv_k=%d not in 1..4", K);
    }
}

template <int DT>
static int prep_d(int D, int K, int T, int H, float lb, const void *qi, const void *ki,
                  const void *vi, const float *z, const float *bl, const float *qc,
                  const float *kc, const float *vc, const float *A, const float *dt, float *cs,
                  float *qo, float *ko, float *vo, float *go, float *ao, float *bo, hipStream_t st)
{
    switch (D) {
    case 16: return prep_k<16, DT>(K, T, H, lb, qi, ki, vi, z, bl, qc, kc, vc, A, dt, cs, qo, ko, vo, go, ao, bo, st);
    case 32: return prep_k<32, DT>(K, T, H, lb, qi, ki, vi, z, bl, qc, kc, vc, A, dt, cs, qo, ko, vo, go, ao, bo, st);
    case 64: return prep_k<64, DT>(K, T, H, lb, qi, ki, vi, z, bl, qc, kc, vc, A, dt, cs, qo, ko, vo, go, ao, bo, st);
    case 128: return prep_k<128, DT>(K, T, H, lb, qi, ki, vi, z, bl, qc, kc, vc, A, dt, cs, qo, ko, vo, go, ao, bo, st);
    default: K3_FAIL(K3HIP_EUNSUPPORTED, "k3hip_kda_prep: D=%d not in {16,32,64,128}", D);
    }
}

}  // namespace k3kda

using namespace k3kda;

extern "C" int k3hip_kda_prep(int T, int H, int D, int K, float gate_lb, int in_dtype,
                              const void *q_in, const void *k_in, const void *v_in,
                              const float *z, const float *b_logit, const float *q_conv,
                              const float *k_conv, const float *v_conv, const float *A_log,
                              const float *dt_bias, float *conv_state, float *q_out,
                              float *k_out, float *v_out, float *g_out, float *alpha_out,
                              float *beta_out, void *stream)
{
    clear_error();
    if (T < 0 || H < 0) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_prep: T=%d H=%d", T, H);
    if (T == 0 || H == 0) return K3HIP_OK;
    if ((long)T * H * D > 0x7fffffffL * 4L) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_prep: T*P too large");
    if (H > 65535 || (long)T > 65535L * PREP_WAVES * PREP_TT)
        K3_FAIL(K3HIP_EINVAL, "k3hip_kda_prep: grid too large (T=%d H=%d)", T, H);
    if (!q_in || !k_in || !v_in || !z || !b_logit || !q_conv || !k_conv || !v_conv || !A_log ||
        !dt_bias || !q_out || !k_out || !v_out || !beta_out)
        K3_FAIL(K3HIP_EINVAL, "k3hip_kda_prep: NULL tensor");
    hipStream_t st = as_stream(stream);
    if (in_dtype == K3HIP_F32)
        return prep_d<K3HIP_F32>(D, K, T, H, gate_lb, q_in, k_in, v_in, z, b_logit, q_conv, k_conv,
                                 v_conv, A_log, dt_bias, conv_state, q_out, k_out, v_out, g_out,
                                 alpha_out, beta_out, st);
    if (in_dtype == K3HIP_BF16)
        return prep_d<K3HIP_BF16>(D, K, T, H, gate_lb, q_in, k_in, v_in, z, b_logit, q_conv,
                                  k_conv, v_conv, A_log, dt_bias, conv_state, q_out, k_out, v_out,
                                  g_out, alpha_out, beta_out, st);
    K3_FAIL(K3HIP_EINVAL, "k3hip_kda_prep: in_dtype=%d", in_dtype);
}
