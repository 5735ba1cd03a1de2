// SPDX-License-Identifier: Apache-2.0
// kda_mla.hip - gated MLA (NoPE) decode with absorbed weights, for the hybrid KDA/MLA slice.
//
// The reference's k3_mla_cached (src/core/k3_ops.c:321-424) caches the EXPANDED per-head
// keys and values (kv_b applied, H*(nope+v) floats per position). On the GPU the cache holds
// the compressed latent instead -- rmsnorm'd kv_a output (kv_lora) followed by the shared
// rope slot (rope), kv_lora + rope floats per position -- and kv_b is absorbed:
//   score_h(t) = q_nope_h . (W_UK_h latent_t) + q_rope_h . rope_t
//              = (W_UK_h^T q_nope_h) . latent_t + q_rope_h . rope_t = qcat_h . cache_t
//   o_h        = sum_t p_t (W_UV_h latent_t) = W_UV_h (sum_t p_t latent_t)
// with W_UK_h / W_UV_h the nope / v rows of head h of kv_b. The same maths in another
// order: equal to the reference up to fp32 rounding, and 42x fewer cached bytes.
//
// One decode step for B sequences that each hold `pos` cached positions: the new token's
// latent goes to position pos and attends over 0..pos. Projections are bf16 MFMA GEMMs on
// bf16 weights with the fp32 activation split into a bf16 hi/lo pair stacked as 2B rows
// (each weight is read once; the two halves are summed after), so activations keep fp32
// accuracy. The attention is two strided-batched fp32 GEMMs (scores, then P . cache) around
// the reference's softmax (fp32 scores times (nope+rope)^-0.5, max, expf, double sum).
#include <math.h>
#include <stdlib.h>

#include "kda_internal.h"

struct k3hip_mla_weights {
    int E, H, QL, KL, QN, QR, VH, gate;
    float eps;
    void *q_a, *q_b, *kv_a, *kv_b, *o, *g;   // bf16
    float *q_a_norm, *kv_a_norm;
};

namespace k3kda {

constexpr int MLA_MAXB = 16;   // sequences per absorb / un-absorb pass

__device__ __forceinline__ double block_sum(double v, double *red)
{
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    double t = 0.0;
    for (int i = 0; i < nw; i++) t += red[i];
    return t;
}

// rows b of C2 [2B][N] summed with rows B+b; rmsnorm over the first nn entries (weight w,
// src/core/k3_ops.c:94-102); then either split into hi/lo bf16 rows of y2 [2B][N]
// (cache == nullptr) or written to cache row b at position pos (cache [B][cap][N]).
__global__ void mla_norm_kernel(const float *__restrict__ C2, int B, int N, int nn,
                                const float *__restrict__ w, float eps, uint16_t *__restrict__ y2,
                                float *__restrict__ cache, long cap, int pos)
{
    __shared__ double red[16];
    const int b = blockIdx.x;
    const float *r0 = C2 + (size_t)b * N, *r1 = C2 + (size_t)(B + b) * N;
    double ss = 0.0;
    for (int n = threadIdx.x; n < nn; n += blockDim.x) {
        const double v = (double)(r0[n] + r1[n]);
        ss += v * v;
    }
    ss = block_sum(ss, red);
    const float inv = (float)(1.0 / sqrt(ss / (double)nn + (double)eps));
    for (int n = threadIdx.x; n < N; n += blockDim.x) {
        const float v = r0[n] + r1[n];
        const float y = n < nn ? (w[n] * v) * inv : v;
        if (cache) {
            cache[((size_t)b * cap + pos) * N + n] = y;
        } else {
            const uint16_t hi = f2bf(y);
            y2[(size_t)b * N + n] = hi;
            y2[(size_t)(B + b) * N + n] = f2bf(y - __uint_as_float((uint32_t)hi << 16));
        }
    }
}

// qcat[b][h] = [ W_UK_h^T q_nope(b,h) | q_rope(b,h) ], q = q2[b] + q2[B+b]. Block = head h,
// threads over latent columns c; each W_UK element is read once for all sequences.
__global__ void mla_absorb_kernel(const float *__restrict__ q2, int B, int H, int QN, int QR,
                                  int KL, int VH, const uint16_t *__restrict__ kvb,
                                  float *__restrict__ qcat)
{
    extern __shared__ float sq[];   // [MLA_MAXB][QN + QR]
    const int h = blockIdx.x, QH = QN + QR, W = KL + QR;
    for (int b0 = 0; b0 < B; b0 += MLA_MAXB) {
        const int nb = min(MLA_MAXB, B - b0);
        __syncthreads();
        for (int i = threadIdx.x; i < nb * QH; i += blockDim.x) {
            const int bb = i / QH, e = i % QH;
            const size_t at = (size_t)h * QH + e;
            sq[i] = q2[(size_t)(b0 + bb) * H * QH + at] + q2[(size_t)(B + b0 + bb) * H * QH + at];
        }
        __syncthreads();
        for (int c = threadIdx.x; c < KL; c += blockDim.x) {
            float acc[MLA_MAXB];
#pragma unroll
            for (int bb = 0; bb < MLA_MAXB; bb++) acc[bb] = 0.0f;
            const uint16_t *col = kvb + (size_t)h * (QN + VH) * KL + c;
            for (int i = 0; i < QN; i++) {
                const float wv = bf2f(col[(size_t)i * KL]);
#pragma unroll
                for (int bb = 0; bb < MLA_MAXB; bb++)
                    if (bb < nb) acc[bb] = __builtin_fmaf(sq[bb * QH + i], wv, acc[bb]);
            }
            for (int bb = 0; bb < nb; bb++) qcat[((size_t)(b0 + bb) * H + h) * W + c] = acc[bb];
        }
        for (int i = threadIdx.x; i < nb * QR; i += blockDim.x) {
            const int bb = i / QR, r = i % QR;
            qcat[((size_t)(b0 + bb) * H + h) * W + KL + r] = sq[bb * QH + QN + r];
        }
    }
}

// Row (b, h) of S [B*H][ld]: the first n scores become softmax weights (reference order:
// fp32 score * scale, max, expf(s - m), double sum z, (float)(e / z)); columns n..ld-1 -> 0.
__global__ void mla_softmax_kernel(float *__restrict__ S, int n, int ld, float scale)
{
    __shared__ double red[16];
    __shared__ float smax[16];
    float *row = S + (size_t)blockIdx.x * ld;
    float m = -INFINITY;
    for (int t = threadIdx.x; t < n; t += blockDim.x) m = fmaxf(m, row[t] * scale);
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if (lane == 0) smax[w] = m;
    __syncthreads();
    m = -INFINITY;
    for (int i = 0; i < nw; i++) m = fmaxf(m, smax[i]);
    double z = 0.0;
    for (int t = threadIdx.x; t < n; t += blockDim.x) {
        const float e = expf(row[t] * scale - m);
        row[t] = e;
        z += (double)e;
    }
    z = block_sum(z, red);
    for (int t = threadIdx.x; t < ld; t += blockDim.x) row[t] = t < n ? (float)((double)row[t] / z) : 0.0f;
}

// o(b,h)[j] = W_UV_h[j] . chat(b,h), times sigmoid(g) when gated (g = g2[b] + g2[B+b]);
// written as hi/lo bf16 rows of o2 [2B][H*VH]. Block = head h, threads over j.
__global__ void mla_unabsorb_kernel(const float *__restrict__ chat, int B, int H, int QN, int KL,
                                    int VH, const uint16_t *__restrict__ kvb,
                                    const float *__restrict__ g2, uint16_t *__restrict__ o2)
{
    extern __shared__ float sc[];   // [MLA_MAXB][KL]
    const int h = blockIdx.x;
    const size_t HV = (size_t)H * VH;
    for (int b0 = 0; b0 < B; b0 += MLA_MAXB) {
        const int nb = min(MLA_MAXB, B - b0);
        __syncthreads();
        for (int i = threadIdx.x; i < nb * KL; i += blockDim.x)
            sc[i] = chat[((size_t)(b0 + i / KL) * H + h) * KL + i % KL];
        __syncthreads();
        for (int j = threadIdx.x; j < VH; j += blockDim.x) {
            float acc[MLA_MAXB];
#pragma unroll
            for (int bb = 0; bb < MLA_MAXB; bb++) acc[bb] = 0.0f;
            const uint16_t *row = kvb + ((size_t)h * (QN + VH) + QN + j) * KL;
            for (int c = 0; c < KL; c++) {
                const float wv = bf2f(row[c]);
#pragma unroll
                for (int bb = 0; bb < MLA_MAXB; bb++)
                    if (bb < nb) acc[bb] = __builtin_fmaf(sc[bb * KL + c], wv, acc[bb]);
            }
            for (int bb = 0; bb < nb; bb++) {
                const size_t b = b0 + bb, at = (size_t)h * VH + j;
                float v = acc[bb];
                if (g2) v *= 1.0f / (1.0f + expf(-(g2[b * HV + at] + g2[(B + b) * HV + at])));
                const uint16_t hi = f2bf(v);
                o2[b * HV + at] = hi;
                o2[(B + b) * HV + at] = f2bf(v - __uint_as_float((uint32_t)hi << 16));
            }
        }
    }
}

}  // namespace k3kda

using namespace k3kda;

extern "C" int k3hip_mla_release(k3hip_mla_weights *w)
{
    clear_error();
    if (!w) return K3HIP_OK;
    void *ptrs[] = {w->q_a, w->q_b, w->kv_a, w->kv_b, w->o, w->g, w->q_a_norm, w->kv_a_norm};
    for (void *p : ptrs)
        if (p) (void)hipFree(p);
    free(w);
    return K3HIP_OK;
}

extern "C" int k3hip_mla_upload(const K3MlaW *w, const K3Cfg *c, k3hip_mla_weights **out)
{
    clear_error();
    if (!w || !c || !out) K3_FAIL(K3HIP_EINVAL, "k3hip_mla_upload: NULL argument");
    *out = nullptr;
    if (w->wdt != K3_WBF16) K3_FAIL(K3HIP_EUNSUPPORTED, "k3hip_mla_upload: bf16 weights only");
    if (c->hidden <= 0 || c->n_heads <= 0 || c->q_lora <= 0 || c->kv_lora <= 0 || c->qk_nope <= 0 ||
        c->qk_rope < 0 || c->v_head <= 0)
        K3_FAIL(K3HIP_EINVAL, "k3hip_mla_upload: bad MLA configuration");
    if (!w->q_a || !w->q_b || !w->kv_a || !w->kv_b || !w->o || !w->q_a_norm || !w->kv_a_norm ||
        (c->mla_out_gate && !w->g))
        K3_FAIL(K3HIP_EINVAL, "k3hip_mla_upload: NULL weight");
    k3hip_mla_weights *d = (k3hip_mla_weights *)calloc(1, sizeof *d);
    if (!d) K3_FAIL(K3HIP_ENOMEM, "k3hip_mla_upload: host allocation");
    d->E = c->hidden; d->H = c->n_heads; d->QL = c->q_lora; d->KL = c->kv_lora;
    d->QN = c->qk_nope; d->QR = c->qk_rope; d->VH = c->v_head; d->gate = c->mla_out_gate && w->g;
    d->eps = c->rms_eps;
    const size_t E = d->E, H = d->H, QH = d->QN + d->QR;
    struct { void **dst; const void *src; size_t bytes; } up[] = {
        {&d->q_a, w->q_a, (size_t)d->QL * E * 2},
        {&d->q_b, w->q_b, H * QH * d->QL * 2},
        {&d->kv_a, w->kv_a, (size_t)(d->KL + d->QR) * E * 2},
        {&d->kv_b, w->kv_b, H * (d->QN + d->VH) * d->KL * 2},
        {&d->o, w->o, E * H * d->VH * 2},
        {&d->g, d->gate ? w->g : nullptr, H * d->VH * E * 2},
        {(void **)&d->q_a_norm, w->q_a_norm, (size_t)d->QL * 4},
        {(void **)&d->kv_a_norm, w->kv_a_norm, (size_t)d->KL * 4},
    };
    for (auto &u : up) {
        if (!u.src) continue;
        if (hipMalloc(u.dst, u.bytes) != hipSuccess || hipMemcpy(*u.dst, u.src, u.bytes, hipMemcpyHostToDevice) != hipSuccess) {
            (void)hipGetLastError();
            k3hip_mla_release(d);
            K3_FAIL(K3HIP_ENOMEM, "k3hip_mla_upload: device copy of %zu bytes", u.bytes);
        }
    }
    *out = d;
    return K3HIP_OK;
}

extern "C" size_t k3hip_mla_cache_floats(const K3Cfg *c, int cap)
{
    if (!c || cap <= 0 || c->kv_lora <= 0 || c->qk_rope < 0) return 0;
    return (size_t)cap * (size_t)(c->kv_lora + c->qk_rope);
}

extern "C" int k3hip_mla_decode(const k3hip_mla_weights *w, int B, int pos, int cap, float *cache,
                                const float *x, float *out, void *stream)
{
    clear_error();
    if (!w || !cache || !x || !out) K3_FAIL(K3HIP_EINVAL, "k3hip_mla_decode: NULL argument");
    if (B <= 0 || pos < 0 || pos >= cap)
        K3_FAIL(K3HIP_EINVAL, "k3hip_mla_decode: B=%d pos=%d cap=%d (need 0 <= pos < cap)", B, pos, cap);
    hipStream_t st = as_stream(stream);
    const int E = w->E, H = w->H, QL = w->QL, KL = w->KL, QN = w->QN, QR = w->QR, VH = w->VH;
    const int QH = QN + QR, CW = KL + QR, Tn = pos + 1;
    const int HV = H * VH;
    size_t sizes[] = {(size_t)2 * B * E * 2, (size_t)2 * B * QL * 4, (size_t)2 * B * QL * 2,
                      (size_t)2 * B * H * QH * 4, (size_t)2 * B * CW * 4, (size_t)2 * B * HV * 4,
                      (size_t)B * H * CW * 4, (size_t)B * H * Tn * 4, (size_t)B * H * KL * 4,
                      (size_t)2 * B * HV * 2, (size_t)2 * B * E * 4};
    constexpr int NB = sizeof sizes / sizeof sizes[0];
    size_t off[NB], total = 0;
    for (int i = 0; i < NB; i++) {
        off[i] = total;
        total += (sizes[i] + 255) & ~(size_t)255;
    }
    StreamBuf buf;
    int rc = stream_alloc(buf, total, st);
    if (rc) return rc;
    char *base = (char *)buf.p;
    uint16_t *xs = (uint16_t *)(base + off[0]);
    float *ql2 = (float *)(base + off[1]);
    uint16_t *qls = (uint16_t *)(base + off[2]);
    float *q2 = (float *)(base + off[3]), *c2 = (float *)(base + off[4]), *g2 = (float *)(base + off[5]);
    float *qcat = (float *)(base + off[6]), *S = (float *)(base + off[7]), *chat = (float *)(base + off[8]);
    uint16_t *o2 = (uint16_t *)(base + off[9]);
    float *out2 = (float *)(base + off[10]);

    if ((rc = split_rows2(x, xs, B, E, st))) return rc;
    // q = q_b(rmsnorm(q_a x)), latent + rope = kv_a x (latent rmsnorm'd into the cache), g x
    if ((rc = gemm_bf16(2 * B, QL, E, xs, w->q_a, ql2, K3HIP_F32, st))) return rc;
    hipLaunchKernelGGL(mla_norm_kernel, dim3(B), dim3(256), 0, st, ql2, B, QL, QL, w->q_a_norm, w->eps,
                       qls, (float *)nullptr, 0L, 0);
    K3_LAUNCHED();
    if ((rc = gemm_bf16(2 * B, H * QH, QL, qls, w->q_b, q2, K3HIP_F32, st))) return rc;
    if ((rc = gemm_bf16(2 * B, CW, E, xs, w->kv_a, c2, K3HIP_F32, st))) return rc;
    hipLaunchKernelGGL(mla_norm_kernel, dim3(B), dim3(256), 0, st, c2, B, CW, KL, w->kv_a_norm, w->eps,
                       (uint16_t *)nullptr, cache, (long)cap, pos);
    K3_LAUNCHED();
    if (w->gate && (rc = gemm_bf16(2 * B, HV, E, xs, w->g, g2, K3HIP_F32, st))) return rc;
    // absorb W_UK into q
    hipLaunchKernelGGL(mla_absorb_kernel, dim3(H), dim3(256), (size_t)MLA_MAXB * QH * 4, st, q2, B, H,
                       QN, QR, KL, VH, (const uint16_t *)w->kv_b, qcat);
    K3_LAUNCHED();
    // scores S_b [H][Tn] = qcat_b [H][CW] . cache_b[0..Tn)^T, per sequence
    GemmDesc gs;
    gs.M = H; gs.N = Tn; gs.K = CW; gs.ab_dtype = K3HIP_F32; gs.c_dtype = K3HIP_F32; gs.b_trans = true;
    gs.lda = CW; gs.ldb = CW; gs.ldc = Tn; gs.batch = B;
    gs.sa = (long)H * CW; gs.sb = (long)cap * CW; gs.sc = (long)H * Tn;
    gs.tune = false;   // a new length every step: take the heuristic's first choice
    if ((rc = gemm(gs, qcat, cache, S, st))) return rc;
    hipLaunchKernelGGL(mla_softmax_kernel, dim3(B * H), dim3(256), 0, st, S, Tn, Tn,
                       1.0f / sqrtf((float)QH));
    K3_LAUNCHED();
    // chat_b [H][KL] = P_b [H][Tn] . cache_b[0..Tn)[0..KL)
    GemmDesc gp;
    gp.M = H; gp.N = KL; gp.K = Tn; gp.ab_dtype = K3HIP_F32; gp.c_dtype = K3HIP_F32; gp.b_trans = false;
    gp.lda = Tn; gp.ldb = CW; gp.ldc = KL; gp.batch = B;
    gp.sa = (long)H * Tn; gp.sb = (long)cap * CW; gp.sc = (long)H * KL;
    gp.tune = false;
    if ((rc = gemm(gp, S, cache, chat, st))) return rc;
    // W_UV, the gate, o_proj
    hipLaunchKernelGGL(mla_unabsorb_kernel, dim3(H), dim3(128), (size_t)MLA_MAXB * KL * 4, st, chat, B,
                       H, QN, KL, VH, (const uint16_t *)w->kv_b, w->gate ? g2 : nullptr, o2);
    K3_LAUNCHED();
    if ((rc = gemm_bf16(2 * B, E, HV, o2, w->o, out2, K3HIP_F32, st))) return rc;
    return pair_add(out2, out, B, E, st);
}
