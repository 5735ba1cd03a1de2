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
// latent goes to position pos and attends over 0..pos. The dense projections run on the
// few-rows bf16 GEMM of kda_rows.hip (fp32 activations split into bf16 hi + lo in registers,
// each weight read once for all B; q_a, kv_a and g in one pass over their concatenated
// weights), so activations keep fp32 accuracy. The absorption (W_UK_h^T q) is a bf16 MFMA
// product per head on q's hi/lo row pairs (2B rows) against a transposed copy of W_UK made at
// upload (mla_absorb_kernel, 5.5 us at 64 heads, B = 16, against 6.2 us for the library's
// batched GEMM: 8.4 MB of W_UK read cold each step); the final W_UV_h is applied after the
// attention the same way. The attention reads
// the cache once where the shape fits the fused kernel (kda_mla_attn.hip: split-bf16 MFMA
// scores, online softmax with the reference's scale (nope+rope)^-0.5, split-bf16 weighted
// sum of the latents; heads <= 64, kv_lora <= 512, kv_lora + rope <= 576); other shapes take
// two strided-batched fp32 GEMMs (scores, then P . cache) around the reference's softmax
// (fp32 scores times (nope+rope)^-0.5, max, expf, double sum).
#include <math.h>
#include <stdlib.h>

#include <algorithm>

#include "kda_internal.h"

struct k3hip_mla_weights {
    int E, H, QL, KL, QN, QR, VH, gate;
    float eps;
    // q_a, kv_a and g (when gated) are row blocks of one matrix xin ([QL + KL + QR + H*VH]
    // [hidden], in that order): one pass over them projects a decode step's input. xin, q_b
    // and o are stored in MFMA fragment order for the few-rows GEMM (kda_rows.hip); kv_b
    // stays row-major (bf16) for the head-batched absorb GEMMs.
    void *xin, *q_b, *kv_b, *o;
    float *q_a_norm, *kv_a_norm;
    // W_UK_h^T per head, [H][KL][QNP] bf16 with QNP = QN rounded up to 32 (zeros past QN): the
    // B operand of the absorb product, each lane's 8 consecutive K values one 16-byte load
    void *ukt;   // nullptr when qk_nope > 256
    int QNP;
};

namespace k3kda {

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

// Row b of C (row stride ldc): rmsnorm over the first nn of its N entries (weight w,
// src/core/k3_ops.c:94-102; double mean of squares, eps inside), the rest copied; written
// as fp32 row b of y [B][N] (y != nullptr) or to cache row b at position pos
// (cache [B][cap][N]). Two independent norms share one launch: blockIdx.y picks the job.
struct NormJob {
    const float *C;
    int N, nn;
    const float *w;
    float *y, *cache;
};
// ukt[h][n][k] = W_UK_h[k][n] for k < QN, 0 for QN <= k < QNP; W_UK_h is rows 0..QN-1 of
// head h's (QN + VH) x KL block of kv_b.
__global__ void mla_ukt_kernel(const uint16_t *__restrict__ kvb, uint16_t *__restrict__ ukt, int H, int QN,
                               int VH, int KL, int QNP)
{
    const size_t n = (size_t)H * KL * QNP;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const int k = (int)(i % QNP);
        const size_t hn = i / QNP;
        const int c = (int)(hn % KL), h = (int)(hn / KL);
        ukt[i] = k < QN ? kvb[((size_t)h * (QN + VH) + k) * KL + c] : (uint16_t)0;
    }
}

// The absorb product A2[r][h][c] = sum_k x[r][h QH + k] W_UK_h[k][c] for the M = 2B rows of
// x (q's bf16 hi rows, then its lo rows; row stride ldx) and every head h: one 16 x 16 x 32
// bf16 MFMA tile chain per wave (16 latent columns of one head, the M rows in tiles of 16,
// K-steps of 32 in order), fp32 results at A2 + r ldc + h CW + c. Workgroup (x, h) takes
// columns 64 x .. 64 x + 63 of head h. VEC: x's rows and head offsets are 16-byte aligned
// and QN is a multiple of 8 (QH, QN and ldx multiples of 8), so each lane's 8 K values are
// one load or none. KS = QNP / 32 K-steps, a template constant so that a tile's loads are
// issued together and waited for once (with a run-time count each load waited alone: 5.9 us).
typedef __bf16 mla_bf16x8 __attribute__((ext_vector_type(8)));
typedef float mla_f32x4 __attribute__((ext_vector_type(4)));
template <bool VEC, int KS>
__global__ __launch_bounds__(256) void mla_absorb_kernel(int M, int QH, int QN, int KL, int CW,
                                                         const uint16_t *__restrict__ x, long ldx,
                                                         const uint16_t *__restrict__ ukt, float *__restrict__ A2,
                                                         long ldc)
{
    constexpr int QNP = 32 * KS;
    const int h = blockIdx.y, lane = threadIdx.x & 63;
    const int n0 = 64 * blockIdx.x + 16 * (threadIdx.x >> 6);
    if (n0 >= KL) return;   // wave-uniform; no barrier in this kernel
    const int col = n0 + (lane & 15), kq = 8 * (lane >> 4);
    const bool cok = col < KL;
    const uint16_t *brow = ukt + ((size_t)h * KL + (cok ? col : 0)) * QNP + kq;
    mla_bf16x8 bf[KS];
#pragma unroll
    for (int t = 0; t < KS; t++) bf[t] = *reinterpret_cast<const mla_bf16x8 *>(brow + 32 * t);
    for (int m0 = 0; m0 < M; m0 += 16) {
        const int r = m0 + (lane & 15);
        const uint16_t *xr = x + (size_t)(r < M ? r : 0) * ldx + (size_t)h * QH + kq;
        mla_bf16x8 af[KS];
#pragma unroll
        for (int t = 0; t < KS; t++) {
            mla_bf16x8 a;
            if constexpr (VEC) {
                // QN % 8 == 0: an 8-value group is wholly inside or past QN; a group past it (or
                // a row past M) loads the head's first group instead and is zeroed, so every
                // load is issued unconditionally from an address inside the row
                const bool ok = r < M && 32 * t + kq < QN;
                const mla_bf16x8 v = *reinterpret_cast<const mla_bf16x8 *>(xr + (ok ? 32 * t : -kq));
                a = ok ? v : mla_bf16x8{};
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const int k = 32 * t + kq + e;
                    a[e] = __builtin_bit_cast(__bf16, r < M && k < QN ? xr[32 * t + e] : (uint16_t)0);
                }
            }
            af[t] = a;
        }
        mla_f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < KS; t++) c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[t], bf[t], c, 0, 0, 0);
        // C layout: lane l holds rows 4 (l / 16) + i of the tile, column l % 16
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int rr = m0 + 4 * (lane >> 4) + i;
            if (rr < M && cok) A2[(size_t)rr * ldc + (size_t)h * CW + col] = c[i];
        }
    }
}

template <bool VEC>
static int mla_absorb_v(int M, int H, int QH, int QN, int QNP, int KL, int CW, const uint16_t *x, long ldx,
                        const uint16_t *ukt, float *A2, long ldc, hipStream_t st)
{
    const dim3 grid((unsigned)((KL + 63) / 64), (unsigned)H);
#define K3_ABS(KS) hipLaunchKernelGGL((mla_absorb_kernel<VEC, KS>), grid, dim3(256), 0, st, M, QH, QN, KL, CW, x, ldx, ukt, A2, ldc)
    switch (QNP / 32) {
    case 1: K3_ABS(1); break;
    case 2: K3_ABS(2); break;
    case 3: K3_ABS(3); break;
    case 4: K3_ABS(4); break;
    case 5: K3_ABS(5); break;
    case 6: K3_ABS(6); break;
    case 7: K3_ABS(7); break;
    case 8: K3_ABS(8); break;
    default: K3_FAIL(K3HIP_EUNSUPPORTED, "mla absorb: qk_nope padded to %d above 256", QNP);
    }
#undef K3_ABS
    K3_LAUNCHED();
    return K3HIP_OK;
}

// A2 = per head h, x (M rows, columns h QH .. h QH + QN - 1) . W_UK_h, via mla_absorb_kernel.
static int mla_absorb(int M, int H, int QH, int QN, int QNP, int KL, int CW, const uint16_t *x, long ldx,
                      const uint16_t *ukt, float *A2, long ldc, hipStream_t st)
{
    if (QH % 8 == 0 && QN % 8 == 0 && ldx % 8 == 0 && ((uintptr_t)x & 15) == 0)
        return mla_absorb_v<true>(M, H, QH, QN, QNP, KL, CW, x, ldx, ukt, A2, ldc, st);
    return mla_absorb_v<false>(M, H, QH, QN, QNP, KL, CW, x, ldx, ukt, A2, ldc, st);
}

__global__ void mla_norm_kernel(long ldc, float eps, NormJob j0, NormJob j1, long cap, int pos)
{
    __shared__ double red[16];
    const NormJob &jb = blockIdx.y == 0 ? j0 : j1;
    const float *__restrict__ w = jb.w;
    float *__restrict__ y = jb.y;
    float *__restrict__ cache = jb.cache;
    const int N = jb.N, nn = jb.nn;
    const int b = blockIdx.x;
    const float *r0 = jb.C + (size_t)b * ldc;
    double ss = 0.0;
    for (int n = threadIdx.x; n < nn; n += blockDim.x) {
        const double v = (double)r0[n];
        ss += v * v;
    }
    ss = block_sum(ss, red);
    const float inv = (float)(1.0 / sqrt(ss / (double)nn + (double)eps));
    float *dst = y ? y + (size_t)b * N : cache + ((size_t)b * cap + pos) * N;
    for (int n = threadIdx.x; n < N; n += blockDim.x) {
        const float v = r0[n];
        dst[n] = n < nn ? (w[n] * v) * inv : v;
    }
}

// qcat[b][h] = [ A2[b][h] + A2[B+b][h] (the absorbed W_UK_h^T q_nope, kv_lora floats) |
// q_rope(b,h) ], from the hi/lo halves of the batched absorb GEMM and the fp32 q.
__global__ void mla_qcat_kernel(const float *__restrict__ A2, const float *__restrict__ q, int B,
                                int H, int QN, int QR, int KL, float *__restrict__ qcat)
{
    const int W = KL + QR, QH = QN + QR;
    const size_t n = (size_t)B * H * W;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        const size_t bh = i / W;
        const int c = (int)(i % W);
        qcat[i] = c < KL ? A2[i] + A2[n + i] : q[bh * QH + QN + (c - KL)];
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

// o = O2[b] + O2[B+b] (the halves of the batched W_UV GEMM), times sigmoid(g) when gated
// (g row b at stride ldg), as fp32 rows of o [B][H*VH] for o_proj; zout[0 .. zn) = 0 on the
// way (may be nullptr) for an o_proj that adds its two K-range partials there.
__global__ void mla_gate_kernel(const float *__restrict__ O2, const float *__restrict__ g, long ldg,
                                int B, size_t HV, float *__restrict__ o, float *__restrict__ zout, size_t zn)
{
    const size_t n = (size_t)B * HV, step = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step) {
        float v = O2[i] + O2[n + i];
        if (g) v *= 1.0f / (1.0f + expf(-g[(i / HV) * ldg + i % HV]));
        o[i] = v;
    }
    if (zout)
        for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < zn; i += step) zout[i] = 0.0f;
}

// mla_softmax_kernel for rows of n <= 256 * RPT scores held in registers: one read and one
// write of the row instead of three passes; the same arithmetic (fp32 score * scale, max,
// expf(s - m), double sum over the block, (float)(e / z)).
template <int RPT>
__global__ __launch_bounds__(256) void mla_softmax_reg_kernel(float *__restrict__ S, int n, int ld, float scale)
{
    __shared__ double red[16];
    __shared__ float smax[16];
    float *row = S + (size_t)blockIdx.x * ld;
    float v[RPT];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < RPT; i++) {
        const int t = threadIdx.x + 256 * i;
        v[i] = t < n ? row[t] * scale : -INFINITY;
        m = fmaxf(m, v[i]);
    }
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) smax[w] = m;
    __syncthreads();
    m = fmaxf(fmaxf(smax[0], smax[1]), fmaxf(smax[2], smax[3]));
    double z = 0.0;
#pragma unroll
    for (int i = 0; i < RPT; i++) {
        const int t = threadIdx.x + 256 * i;
        v[i] = t < n ? expf(v[i] - m) : 0.0f;
        z += (double)v[i];
    }
    z = block_sum(z, red);
#pragma unroll
    for (int i = 0; i < RPT; i++) {
        const int t = threadIdx.x + 256 * i;
        if (t < n) row[t] = (float)((double)v[i] / z);
    }
    for (int t = n + threadIdx.x; t < ld; t += 256) row[t] = 0.0f;
}

static unsigned mla_grid(size_t n)
{
    size_t b = (n + 255) / 256;
    return (unsigned)(b > 4096 ? 4096 : (b ? b : 1));
}

}  // namespace k3kda

using namespace k3kda;

extern "C" int k3hip_mla_release(k3hip_mla_weights *w)
{
    clear_error();
    if (!w) return K3HIP_OK;
    void *ptrs[] = {w->xin, w->q_b, w->kv_b, w->o, w->q_a_norm, w->kv_a_norm, w->ukt};
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
    if ((c->hidden & 7) || (c->q_lora & 7) || ((c->n_heads * c->v_head) & 7))
        K3_FAIL(K3HIP_EUNSUPPORTED, "k3hip_mla_upload: hidden=%d, q_lora=%d, heads*v_head=%d not multiples of 8",
                c->hidden, c->q_lora, c->n_heads * c->v_head);
    k3hip_mla_weights *d = (k3hip_mla_weights *)calloc(1, sizeof *d);
    if (!d) K3_FAIL(K3HIP_ENOMEM, "k3hip_mla_upload: host allocation");
    d->E = c->hidden; d->H = c->n_heads; d->QL = c->q_lora; d->KL = c->kv_lora;
    d->QN = c->qk_nope; d->QR = c->qk_rope; d->VH = c->v_head; d->gate = c->mla_out_gate && w->g;
    d->eps = c->rms_eps;
    const size_t E = d->E, H = d->H, QH = d->QN + d->QR;
    const size_t N1 = (size_t)d->QL + d->KL + d->QR + (d->gate ? H * d->VH : 0);
    {
        const size_t rows[3] = {(size_t)d->QL, (size_t)(d->KL + d->QR), d->gate ? H * d->VH : 0};
        const void *src[3] = {w->q_a, w->kv_a, d->gate ? w->g : nullptr};
        if (hipMalloc(&d->xin, N1 * E * 2) != hipSuccess) {
            (void)hipGetLastError();
            d->xin = nullptr;
            k3hip_mla_release(d);
            K3_FAIL(K3HIP_ENOMEM, "k3hip_mla_upload: device allocation");
        }
        size_t at = 0;
        for (int i = 0; i < 3; i++) {
            if (!rows[i]) continue;
            if (hipMemcpy((char *)d->xin + at * E * 2, src[i], rows[i] * E * 2, hipMemcpyHostToDevice) != hipSuccess) {
                (void)hipGetLastError();
                k3hip_mla_release(d);
                K3_FAIL(K3HIP_EHIP, "k3hip_mla_upload: weight copy");
            }
            at += rows[i];
        }
    }
    struct { void **dst; const void *src; size_t bytes; } up[] = {
        {&d->q_b, w->q_b, H * QH * d->QL * 2},
        {&d->kv_b, w->kv_b, H * (d->QN + d->VH) * d->KL * 2},
        {&d->o, w->o, E * H * d->VH * 2},
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
    // W_UK^T per head for the absorb kernel (qk_nope <= 256; wider heads keep the batched
    // library GEMM on kv_b itself)
    d->QNP = (d->QN + 31) / 32 * 32;
    if (d->QNP <= 256) {
        const size_t n = H * d->KL * d->QNP;
        if (hipMalloc(&d->ukt, n * 2) != hipSuccess) {
            (void)hipGetLastError();
            d->ukt = nullptr;
            k3hip_mla_release(d);
            K3_FAIL(K3HIP_ENOMEM, "k3hip_mla_upload: device allocation");
        }
        hipLaunchKernelGGL(mla_ukt_kernel, dim3((unsigned)std::min<size_t>((n + 255) / 256, 65536)), dim3(256), 0,
                           nullptr, (const uint16_t *)d->kv_b, (uint16_t *)d->ukt, (int)H, d->QN, d->VH, d->KL, d->QNP);
        if (hipGetLastError() != hipSuccess || hipStreamSynchronize(nullptr) != hipSuccess) {
            (void)hipGetLastError();
            k3hip_mla_release(d);
            K3_FAIL(K3HIP_EHIP, "k3hip_mla_upload: W_UK transpose failed");
        }
    }
    // xin, q_b and o into MFMA fragment order (the row-major uploads are only the source)
    struct { void **w; int N, K; } fr[] = {
        {&d->xin, (int)N1, (int)E}, {&d->q_b, (int)(H * QH), d->QL}, {&d->o, (int)E, (int)(H * d->VH)}};
    for (auto &f : fr) {
        void *packed = nullptr;
        if (hipMalloc(&packed, rows_frag_elems(f.N, f.K) * 2) != hipSuccess ||
            rows_frag_pack((const uint16_t *)*f.w, f.N, f.K, (uint16_t *)packed, nullptr) != K3HIP_OK ||
            hipStreamSynchronize(nullptr) != hipSuccess) {
            (void)hipGetLastError();
            if (packed) (void)hipFree(packed);
            k3hip_mla_release(d);
            K3_FAIL(K3HIP_EHIP, "k3hip_mla_upload: packing the decode weights failed");
        }
        (void)hipFree(*f.w);
        *f.w = packed;
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
    if ((QL & 7) || (HV & 7))
        K3_FAIL(K3HIP_EUNSUPPORTED, "k3hip_mla_decode: q_lora=%d, heads*v_head=%d not multiples of 8", QL, HV);
    // attention in one pass over the cache (kda_mla_attn.hip) where the shape fits it, else
    // as two strided-batched fp32 GEMMs around the softmax
    const bool fused = mla_attention_supported(H, KL, CW) && !((uintptr_t)cache & 15) && !(QN & 3) && VH <= 128;
    // scratch: q_a kv_a g projections [B][ld1] | q_a normed | q | q hi/lo | absorb halves | qcat |
    //          scores or the fused attention's workspace | chat | chat hi/lo | W_UV halves (chat
    //          and the W_UV halves only without the fused attention) | o | split-K partials
    const int N1 = QL + CW + (w->gate ? HV : 0);
    const long ld1 = (N1 + 3) & ~3;
    // the q_a / kv_a / g product on K-ranges that spread it over every CU, summed by a second
    // launch (161 column blocks at hidden 7168: 3 ranges, 483 workgroups)
    const int np1 = gemm_rows_plane_count(N1, E);
    const size_t wsf = std::max({gemm_rows_ws_floats(B, N1, E), np1 > 1 ? (size_t)np1 * std::min(64, B) * N1 : 0,
                                 gemm_rows_ws_floats(B, H * QH, QL), gemm_rows_ws_floats(B, E, HV)});
    size_t sizes[] = {(size_t)B * ld1 * 4, (size_t)B * QL * 4, (size_t)B * H * QH * 4,
                      (size_t)2 * B * H * QH * 2, (size_t)2 * B * H * CW * 4, (size_t)B * H * CW * 4,
                      fused ? mla_attention_ws_bytes(B, H, KL, Tn) : (size_t)B * H * Tn * 4,
                      fused ? 0 : (size_t)B * H * KL * 4, (size_t)2 * B * H * KL * 2,
                      fused ? 0 : (size_t)2 * B * HV * 4, (size_t)B * HV * 4, wsf * 4};
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
    float *C1 = (float *)(base + off[0]), *qn = (float *)(base + off[1]), *q = (float *)(base + off[2]);
    uint16_t *qs2 = (uint16_t *)(base + off[3]);
    float *A2 = (float *)(base + off[4]), *qcat = (float *)(base + off[5]), *S = (float *)(base + off[6]);
    float *chat = (float *)(base + off[7]);
    uint16_t *ch2 = (uint16_t *)(base + off[8]);
    float *O2 = (float *)(base + off[9]), *o = (float *)(base + off[10]), *ws = (float *)(base + off[11]);
    const uint16_t *kvb = (const uint16_t *)w->kv_b;

    // q_a, kv_a and g in one pass over their weights (fp32 x split hi/lo in registers);
    // q = q_b(rmsnorm(q_a x)); latent + rope = kv_a x, the latent rmsnorm'd into the cache
    if ((rc = gemm_rows_even(B, N1, E, x, E, (const uint16_t *)w->xin, C1, ld1, st, ws, wsf))) return rc;
    // the two rmsnorms: with the fused attention and an unsplit q_b product, the q_b GEMV
    // normalises q_a as it reads it and the attention writes the new latent row itself;
    // otherwise one launch writes qn and the cache row
    const bool fold_norms = fused && gemm_rows_splits(H * QH, QL) == 1 && !((uintptr_t)w->q_a_norm & 15);
    if (!fold_norms) {
        hipLaunchKernelGGL(mla_norm_kernel, dim3(B, 2), dim3(256), 0, st, ld1, w->eps,
                           NormJob{C1, QL, QL, w->q_a_norm, qn, nullptr},
                           NormJob{C1 + QL, CW, KL, w->kv_a_norm, nullptr, cache}, (long)cap, pos);
        K3_LAUNCHED();
    }
    // q, and q as bf16 hi / lo rows for the absorb GEMM, from one launch
    if (fold_norms)
        rc = gemm_rows_hl(B, H * QH, QL, C1, ld1, (const uint16_t *)w->q_b, q, (long)H * QH, qs2, (long)H * QH, st, ws,
                          wsf, w->q_a_norm, w->eps);
    else
        rc = gemm_rows_hl(B, H * QH, QL, qn, QL, (const uint16_t *)w->q_b, q, (long)H * QH, qs2, (long)H * QH, st, ws,
                          wsf);
    if (rc) return rc;
    // absorb: per head h, [q hi; lo] (2B x QN) . W_UK_h (QN x KL)
    if (w->ukt) {
        if ((rc = mla_absorb(2 * B, H, QH, QN, w->QNP, KL, CW, qs2, (long)H * QH, (const uint16_t *)w->ukt, A2,
                             (long)H * CW, st)))
            return rc;
    } else {
        GemmDesc ga;
        ga.M = 2 * B; ga.N = KL; ga.K = QN; ga.ab_dtype = K3HIP_BF16; ga.c_dtype = K3HIP_F32; ga.b_trans = false;
        ga.lda = (long)H * QH; ga.ldb = KL; ga.ldc = (long)H * CW; ga.batch = H;
        ga.sa = QH; ga.sb = (long)(QN + VH) * KL; ga.sc = CW;
        if ((rc = gemm(ga, qs2, kvb, A2, st))) return rc;
    }
    // o_proj as two K-ranges adds into `out`, zeroed by the kernel before it (no reduction
    // launch); atomics on ordinary device memory only
    const bool oz = gemm_rows_splits(E, HV) == 2 && coarse_device_mem(out);
    const float *gl = w->gate ? C1 + QL + CW : nullptr;
    if (fused) {
        // the query rows formed inside the attention from A2 and q; the ranges merged, W_UV and
        // the output gate applied in the launch after it (kda_mla_attn.hip)
        if ((rc = mla_attention(B, H, KL, CW, Tn, cap, 1.0f / sqrtf((float)QH), A2, q, QN, cache,
                                fold_norms ? C1 + QL : nullptr, ld1, w->kv_a_norm, w->eps, kvb, VH, gl, ld1,
                                o, oz ? out : nullptr, oz ? (size_t)B * E : (size_t)0, ch2, S,
                                mla_attention_ws_bytes(B, H, KL, Tn), st)))
            return rc;
        return gemm_rows(B, E, HV, o, HV, (const uint16_t *)w->o, out, E, st, ws, wsf, oz);
    }
    {
        hipLaunchKernelGGL(mla_qcat_kernel, dim3(mla_grid((size_t)B * H * CW)), dim3(256), 0, st, A2, q, B, H,
                           QN, QR, KL, qcat);
        K3_LAUNCHED();
        // scores S_b [H][Tn] = qcat_b [H][CW] . cache_b[0..Tn)^T, per sequence
        GemmDesc gs;
        gs.M = H; gs.N = Tn; gs.K = CW; gs.ab_dtype = K3HIP_F32; gs.c_dtype = K3HIP_F32; gs.b_trans = true;
        gs.lda = CW; gs.ldb = CW; gs.ldc = Tn; gs.batch = B;
        gs.sa = (long)H * CW; gs.sb = (long)cap * CW; gs.sc = (long)H * Tn;
        gs.cache = false;   // a new length every step: no plan kept
        if ((rc = gemm(gs, qcat, cache, S, st))) return rc;
        {
            const float scale = 1.0f / sqrtf((float)QH);
            if (Tn <= 256 * 8)
                hipLaunchKernelGGL((mla_softmax_reg_kernel<8>), dim3(B * H), dim3(256), 0, st, S, Tn, Tn, scale);
            else if (Tn <= 256 * 32)
                hipLaunchKernelGGL((mla_softmax_reg_kernel<32>), dim3(B * H), dim3(256), 0, st, S, Tn, Tn, scale);
            else
                hipLaunchKernelGGL(mla_softmax_kernel, dim3(B * H), dim3(256), 0, st, S, Tn, Tn, scale);
            K3_LAUNCHED();
        }
        // chat_b [H][KL] = P_b [H][Tn] . cache_b[0..Tn)[0..KL)
        GemmDesc gp;
        gp.M = H; gp.N = KL; gp.K = Tn; gp.ab_dtype = K3HIP_F32; gp.c_dtype = K3HIP_F32; gp.b_trans = false;
        gp.lda = Tn; gp.ldb = CW; gp.ldc = KL; gp.batch = B;
        gp.sa = (long)H * Tn; gp.sb = (long)cap * CW; gp.sc = (long)H * KL;
        gp.cache = false;
        if ((rc = gemm(gp, S, cache, chat, st))) return rc;
        if ((rc = split_rows2(chat, ch2, B, H * KL, st))) return rc;
    }
    // W_UV: per head h, [chat hi; lo] (2B x KL) . W_UV_h^T (KL x VH), batched over heads; gate
    GemmDesc gu;
    gu.M = 2 * B; gu.N = VH; gu.K = KL; gu.ab_dtype = K3HIP_BF16; gu.c_dtype = K3HIP_F32; gu.b_trans = true;
    gu.lda = (long)H * KL; gu.ldb = KL; gu.ldc = HV; gu.batch = H;
    gu.sa = KL; gu.sb = (long)(QN + VH) * KL; gu.sc = VH;
    if ((rc = gemm(gu, ch2, kvb + (size_t)QN * KL, O2, st))) return rc;
    hipLaunchKernelGGL(mla_gate_kernel, dim3(mla_grid((size_t)B * HV)), dim3(256), 0, st, O2, gl, ld1, B,
                       (size_t)HV, o, oz ? out : nullptr, oz ? (size_t)B * E : (size_t)0);
    K3_LAUNCHED();
    return gemm_rows(B, E, HV, o, HV, (const uint16_t *)w->o, out, E, st, ws, wsf, oz);
}
