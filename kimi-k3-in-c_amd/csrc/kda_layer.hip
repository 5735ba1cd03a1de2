// SPDX-License-Identifier: Apache-2.0
// kda_layer.hip - the C-ABI shim: error state, device-resident weights, the full layer on
// device pointers, and the drop-in k3_kda_layer / k3_kda_scratch on host pointers.
//
// The layer follows the reference k3_kda_layer (src/core/k3_ops.c:864-951) step for step:
//   1 projections q, k, v, b, f_a -> f_b, g            (:877-886, :946)
//   2-5 K1: conv+SiLU, L2(q,k), beta, decay             (:888-906)
//   6 recurrence with q * (1/sqrtf(D)): K3 decode for T == 1, K2 chunked for T > 1
//     (the sequential GPU recurrence when the gate bound is outside K2's range)
//   7-8 K4: head RMSNorm then sigmoid gate              (:940-947)
//   9 o_proj                                            (:948)
#include <algorithm>
#include <atomic>
#include <math.h>
#include <mutex>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "kda_internal.h"
#include "kda_prep_math.h"

namespace k3kda {

static thread_local char g_err[1024];

void set_error(const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}

void clear_error() { g_err[0] = 0; }

// A kernel rather than hipMemsetAsync, so the call stays correct under graph capture.
__global__ void zero_fill_kernel(float *p, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0.0f;
}

int zero_fill(float *p, size_t n, hipStream_t st)
{
    if (n == 0) return K3HIP_OK;
    size_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(zero_fill_kernel, dim3((unsigned)blocks), dim3(256), 0, st, p, n);
    K3_LAUNCHED();
    return K3HIP_OK;
}

// Set while a no-allocation entry point runs on this thread: any stream allocation its
// call path would make is refused instead (the call then returns an error, allocating nothing).
static thread_local bool g_no_alloc;

int stream_alloc(StreamBuf &b, size_t bytes, hipStream_t st)
{
    b.st = st;
    if (g_no_alloc)
        K3_FAIL(K3HIP_EINVAL, "no-allocation entry point: a step needs %zu bytes of scratch beyond the fixed "
                "array", bytes);
    if (bytes == 0) bytes = 256;
    hipError_t e = hipMallocAsync(&b.p, bytes, st);
    if (e != hipSuccess) {
        b.p = nullptr;
        (void)hipGetLastError();
        K3_FAIL(K3HIP_ENOMEM, "hipMallocAsync(%zu bytes): %s", bytes, hipGetErrorString(e));
    }
    return K3HIP_OK;
}

}  // namespace k3kda

using namespace k3kda;

struct k3hip_kda_weights {
    int hidden, H, D, K, wdt, parts;   // parts: the K3HIP_UPLOAD_* copies that were made
    size_t bytes;                      // device bytes held
    float gate_lb, rms_eps;
    // The DEV part (every matrix in its own storage and the fp32 vectors) is one device block,
    // dev_block, freed on release when owned (the drop-in binds a stream-ordered block of its
    // own). q, k, v, f_a, b are row blocks of xin ([3P + D + H][hidden], in that order) inside
    // it, so a decode step projects into all five with one pass over the weights.
    void *dev_block;
    bool own_dev_block;
    void *xin;
    void *q, *k, *v, *f_a, *f_b, *b, *g, *o;        // matrices, wdt storage
    float *q_conv, *k_conv, *v_conv, *A_log, *dt_bias, *o_norm;
    void *f_b2;   // bf16 only: [W | W] along K, for the f_b GEMM on a hi/lo-split f_a
    void *o16;    // bf16 only: W_o as fp16 (exact), for the prefill o_proj on fp16 y
    // bf16 only: decode copies of xin, g, f_b and o in MFMA fragment order (kda_rows.hip)
    void *xin_f, *g_f, *f_b_f, *o_f;
};

extern "C" const char *k3hip_last_error(void) { return g_err; }

extern "C" const char *k3hip_version(void)
{
    return "k3kda-hip 0.1 gfx950 (K1 prep, K2 chunked prefill, K3 decode, K4 epilogue)";
}

extern "C" int k3hip_device_count(void)
{
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

// bf16 -> fp16: exact for values inside fp16's normal range; *bad = 1 when a value is beyond
// fp16's largest finite value (or not finite)
__global__ void bf16_to_f16_kernel(const uint16_t *__restrict__ w, uint16_t *__restrict__ h, size_t n,
                                   int *__restrict__ bad)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const float f = bf2f(w[i]);
        if (!(fabsf(f) <= 65504.0f)) *bad = 1;
        h[i] = __builtin_bit_cast(uint16_t, (_Float16)f);
    }
}

// Bytes the calling thread's last k3_kda_layer call copied host to device (weights,
// activations, state) and back; the drop-in's cost beyond its arithmetic.
static thread_local size_t g_dropin_h2d, g_dropin_d2h;
static thread_local bool g_in_dropin;   // counting: inside k3_kda_layer

// The DEV part's layout in one block: xin (q, k, v, f_a, b rows), f_b, g, o, then the fp32
// vectors, each region 256-byte aligned. Row bytes of a matrix with `cols` inputs: int8 rows
// carry their fp32 scale in front (include/k3/k3.h:266-283), the other tags are per element.
struct DevPart {
    size_t rowbytes_E, off[10], total;
};
static DevPart dev_part_layout(const K3KdaW *w, const K3Cfg *c)
{
    const size_t E = (size_t)c->hidden, H = (size_t)c->kda_heads, D = (size_t)c->kda_head_dim, K = (size_t)c->conv_k;
    const size_t P = H * D, es = w->wdt == K3_WBF16 ? 2 : 4;
    auto rb = [&](size_t cols) { return w->wdt == K3_WI8 ? 4 + cols : cols * es; };
    const size_t sizes[10] = {(3 * P + D + H) * rb(E), P * rb(D), P * rb(E), E * rb(P), P * K * 4, P * K * 4,
                              P * K * 4, H * 4, P * 4, D * 4};
    DevPart L{};
    L.rowbytes_E = rb(E);
    for (int i = 0; i < 10; i++) {
        L.off[i] = L.total;
        L.total += (sizes[i] + 255) & ~(size_t)255;
    }
    return L;
}
static size_t dev_part_bytes(const K3KdaW *w, const K3Cfg *c) { return dev_part_layout(w, c).total; }

// Copy the DEV part of w into `base` (dev_part_bytes of device memory) on stream st and point
// d's fields at it; d's sizes and tag are set by the caller.
static int bind_dev_part(k3hip_kda_weights *d, const K3KdaW *w, const K3Cfg *c, char *base, hipStream_t st)
{
    const size_t E = (size_t)c->hidden, H = (size_t)c->kda_heads, D = (size_t)c->kda_head_dim, K = (size_t)c->conv_k;
    const size_t P = H * D, es = w->wdt == K3_WBF16 ? 2 : 4;
    auto rb = [&](size_t cols) { return w->wdt == K3_WI8 ? 4 + cols : cols * es; };
    const DevPart L = dev_part_layout(w, c);
    const void *src[14] = {w->q, w->k, w->v, w->f_a, w->b, w->f_b, w->g, w->o,
                           w->q_conv, w->k_conv, w->v_conv, w->A_log, w->dt_bias, w->o_norm};
    for (const void *p : src)
        if (!p) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_upload: NULL weight");
    void **dst[14] = {&d->q, &d->k, &d->v, &d->f_a, &d->b, &d->f_b, &d->g, &d->o,
                      (void **)&d->q_conv, (void **)&d->k_conv, (void **)&d->v_conv, (void **)&d->A_log,
                      (void **)&d->dt_bias, (void **)&d->o_norm};
    size_t off[14], bytes[14];
    const size_t xrows[5] = {P, P, P, D, H};
    size_t at = 0;
    for (int i = 0; i < 5; i++) {   // q k v f_a b: consecutive row blocks of xin
        off[i] = L.off[0] + at * L.rowbytes_E;
        bytes[i] = xrows[i] * L.rowbytes_E;
        at += xrows[i];
    }
    const size_t rest[9] = {P * rb(D), P * rb(E), E * rb(P), P * K * 4, P * K * 4, P * K * 4, H * 4, P * 4, D * 4};
    for (int i = 5; i < 14; i++) {
        off[i] = L.off[i - 4];
        bytes[i] = rest[i - 5];
    }
    for (int i = 0; i < 14; i++) {
        *dst[i] = base + off[i];
        K3_HIP(hipMemcpyAsync(*dst[i], src[i], bytes[i], hipMemcpyHostToDevice, st));
        d->bytes += bytes[i];
        if (g_in_dropin) g_dropin_h2d += bytes[i];
    }
    d->xin = d->q;
    return K3HIP_OK;
}

extern "C" int k3hip_kda_release(k3hip_kda_weights *w)
{
    clear_error();
    if (!w) return K3HIP_OK;
    void *ptrs[] = {w->own_dev_block ? w->dev_block : nullptr, w->f_b2, w->o16, w->xin_f, w->g_f, w->f_b_f,
                    w->o_f};   // the DEV part's matrices and vectors live inside dev_block
    for (void *p : ptrs)
        if (p) (void)hipFree(p);
    free(w);
    return K3HIP_OK;
}

extern "C" int k3hip_kda_upload(const K3KdaW *w, const K3Cfg *c, k3hip_kda_weights **out)
{
    return k3hip_kda_upload_ex(w, c, K3HIP_UPLOAD_ALL, out);
}

extern "C" size_t k3hip_kda_weights_bytes(const k3hip_kda_weights *w) { return w ? w->bytes : 0; }

extern "C" size_t k3hip_kda_dropin_bytes(void) { return g_dropin_h2d + g_dropin_d2h; }

extern "C" int k3hip_kda_upload_ex(const K3KdaW *w, const K3Cfg *c, int parts, k3hip_kda_weights **out)
{
    clear_error();
    if (!w || !c || !out) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_upload: NULL argument");
    if (parts & ~K3HIP_UPLOAD_ALL) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_upload_ex: parts=%#x", parts);
    *out = nullptr;
    const int E = c->hidden, H = c->kda_heads, D = c->kda_head_dim, K = c->conv_k;
    if (E <= 0 || H <= 0 || D <= 0 || K <= 0)
        K3_FAIL(K3HIP_EINVAL, "k3hip_kda_upload: hidden=%d H=%d D=%d conv_k=%d", E, H, D, K);
    if (w->wdt != K3_WF32 && w->wdt != K3_WBF16 && w->wdt != K3_WI8)
        K3_FAIL(K3HIP_EUNSUPPORTED, "k3hip_kda_upload: weight tag %d (fp32=0, bf16=1, int8 rows=2)", w->wdt);
    k3hip_kda_weights *d = (k3hip_kda_weights *)calloc(1, sizeof *d);
    if (!d) K3_FAIL(K3HIP_ENOMEM, "k3hip_kda_upload: host allocation");
    d->hidden = E; d->H = H; d->D = D; d->K = K; d->wdt = w->wdt; d->parts = parts | K3HIP_UPLOAD_DEV;
    d->gate_lb = c->gate_lb; d->rms_eps = c->rms_eps;
    const size_t P = (size_t)H * D;
    int rc = K3HIP_OK;
    {
        void *blk = nullptr;
        const size_t need = dev_part_bytes(w, c);
        if (hipMalloc(&blk, need) != hipSuccess) {
            (void)hipGetLastError();
            set_error("k3hip_kda_upload: hipMalloc(%zu bytes)", need);
            rc = K3HIP_ENOMEM;
        } else {
            d->dev_block = blk;
            d->own_dev_block = true;
            rc = bind_dev_part(d, w, c, (char *)blk, nullptr);
            if (rc == K3HIP_OK && hipStreamSynchronize(nullptr) != hipSuccess) {
                set_error("k3hip_kda_upload: weight copy failed");
                rc = K3HIP_EHIP;
            }
        }
    }
    // [W | W] copies of f_b (P x 2D) and o (E x 2P) for the bf16 prefill path
    auto twice = [&](void **dst, const void *src, size_t rows, size_t cols) -> int {
        const size_t rb = cols * 2;
        K3_HIP(hipMalloc(dst, rows * rb * 2));
        d->bytes += rows * rb * 2;
        K3_HIP(hipMemcpy2D(*dst, 2 * rb, src, rb, rb, rows, hipMemcpyDeviceToDevice));
        K3_HIP(hipMemcpy2D((char *)*dst + rb, 2 * rb, src, rb, rb, rows, hipMemcpyDeviceToDevice));
        return K3HIP_OK;
    };
    // W_o as fp16 for the prefill o_proj (y is RMS-normalised, so fp16 holds it)
    auto to_f16 = [&](void **dst, const void *src, size_t n) -> int {
        int *bad = nullptr, hbad = 0;
        K3_HIP(hipMalloc(dst, n * 2));
        d->bytes += n * 2;
        K3_HIP(hipMalloc(&bad, sizeof(int)));
        int r = K3HIP_OK;
        if (hipMemcpy(bad, &hbad, sizeof(int), hipMemcpyHostToDevice) != hipSuccess) r = K3HIP_EHIP;
        if (r == K3HIP_OK) {
            const size_t blocks = std::min<size_t>((n + 255) / 256, 8192);
            hipLaunchKernelGGL(bf16_to_f16_kernel, dim3((unsigned)blocks), dim3(256), 0, nullptr,
                               (const uint16_t *)src, (uint16_t *)*dst, n, bad);
            if (hipGetLastError() != hipSuccess || hipMemcpy(&hbad, bad, sizeof(int), hipMemcpyDeviceToHost) != hipSuccess)
                r = K3HIP_EHIP;
        }
        (void)hipFree(bad);
        if (r) {
            set_error("k3hip_kda_upload: fp16 copy of W_o failed");
            return r;
        }
        if (hbad) {
            d->bytes -= n * 2;
            (void)hipFree(*dst);
            *dst = nullptr;   // the prefill refuses these weights; decode does not need the copy
        }
        return K3HIP_OK;
    };
    if (rc == K3HIP_OK && w->wdt == K3_WBF16 && (parts & K3HIP_UPLOAD_PREFILL)) {
        rc = twice(&d->f_b2, d->f_b, P, (size_t)D);
        if (rc == K3HIP_OK) rc = to_f16(&d->o16, d->o, (size_t)E * P);
    }
    // fragment-ordered copies for the decode projections (row-major stays for prefill)
    auto frag = [&](void **dst, const void *src, int N, int Kd) -> int {
        K3_HIP(hipMalloc(dst, rows_frag_elems(N, Kd) * 2));
        d->bytes += rows_frag_elems(N, Kd) * 2;
        return rows_frag_pack((const uint16_t *)src, N, Kd, (uint16_t *)*dst, nullptr);
    };
    if (rc == K3HIP_OK && w->wdt == K3_WBF16 && E % 8 == 0 && D % 8 == 0 && (parts & K3HIP_UPLOAD_DECODE)) {
        rc = frag(&d->xin_f, d->xin, (int)(3 * P) + D + H, E);
        if (rc == K3HIP_OK) rc = frag(&d->g_f, d->g, (int)P, E);
        if (rc == K3HIP_OK) rc = frag(&d->f_b_f, d->f_b, (int)P, D);
        if (rc == K3HIP_OK) rc = frag(&d->o_f, d->o, E, (int)P);
        if (rc == K3HIP_OK && hipStreamSynchronize(nullptr) != hipSuccess) {
            set_error("k3hip_kda_upload: packing the decode weights failed");
            rc = K3HIP_EHIP;
        }
    }
    if (rc != K3HIP_OK) {
        char keep[1024];
        snprintf(keep, sizeof keep, "%s", g_err);
        k3hip_kda_release(d);
        set_error("%s", keep);
        return rc;
    }
    *out = d;
    return K3HIP_OK;
}

// The chunked kernel factors e^(G_t - G_s) over 16-token blocks, which needs every log-decay
// in [gate_lb, 0] with 15 |gate_lb| <= 80 (e^80 < FLT_MAX, e^-80 still a normal float).
// The unbounded softplus gate (gate_lb == 0) and steeper bounds take the sequential GPU
// recurrence.
static bool chunk_gate_ok(float lb) { return lb < 0.0f && fabsf(lb) * 15.0f <= 80.0f; }

extern "C" int k3hip_kda_layer_dev(const k3hip_kda_weights *w, int T, float *out, const float *x,
                                   float *state, void *stream)
{
    clear_error();
    if (!w || !out || !x) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_layer_dev: NULL argument");
    if (T < 0) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_layer_dev: T=%d", T);
    if (T == 0) return K3HIP_OK;
    hipStream_t st = as_stream(stream);
    const int E = w->hidden, H = w->H, D = w->D, K = w->K;
    const size_t P = (size_t)H * D, TP = (size_t)T * P;

    // device intermediates, stream-ordered: qp kp vp z gl | q k v g alpha o y | bl beta | fa
    const size_t nf = 12 * TP + 2 * (size_t)T * H + (size_t)T * D + (state ? 0 : (size_t)H * D * D);
    StreamBuf ws;
    int rc = stream_alloc(ws, nf * sizeof(float), st);
    if (rc) return rc;
    float *f = (float *)ws.p;
    float *qp = f, *kp = qp + TP, *vp = kp + TP, *z = vp + TP, *gl = z + TP;
    float *q = gl + TP, *k = q + TP, *v = k + TP, *g = v + TP, *al = g + TP, *o = al + TP;
    float *y = o + TP, *bl = y + TP, *bt = bl + (size_t)T * H, *fa = bt + (size_t)T * H;
    float *S = state;
    if (!S) {
        S = fa + (size_t)T * D;
        if ((rc = zero_fill(S, (size_t)H * D * D, st))) return rc;
    }
    float *cs = state ? state + (size_t)H * D * D : nullptr;

    // Projections. bf16 weights on a T >= 16 prefill: MFMA GEMMs (kda_mm.hip) of the input
    // split into bf16 hi + lo rows, the two halves' fp32 products added, so the products keep
    // fp32 accuracy (x = hi + lo to 2^-17, bf16 x bf16 exact in fp32, fp32 sums over K) and
    // the layer stays within the reference's 1e-4 bar. Otherwise (fp32 or int8 weights,
    // short T, widths that are not multiples of 64) the double-accumulating GEMV.
    const bool mfma = w->wdt == K3_WBF16 && T >= 16 && E % 64 == 0 && D % 64 == 0 && P % 64 == 0 &&
                      ((uintptr_t)x & 15) == 0;
    StreamBuf sbuf;
    uint16_t *xs = nullptr;
    float *C2 = nullptr;
    if (mfma) {
        const size_t maxin = std::max<size_t>(E, P), maxout = std::max<size_t>(E, P);
        const size_t xsb = ((2 * (size_t)T * maxin * 2) + 255) & ~(size_t)255;
        if ((rc = stream_alloc(sbuf, xsb + 2 * (size_t)T * maxout * 4, st))) return rc;
        xs = (uint16_t *)sbuf.p;
        C2 = (float *)((char *)sbuf.p + xsb);
    }
    // y[T][out] = in[T][nin] . W[out][nin]^T, from the split input xs when mfma
    auto project = [&](int nin, int nout, const float *in, const void *W, float *y) -> int {
        if (!mfma) return proj(T, nin, nout, in, W, w->wdt, y, st);
        int r = mm(2 * T, nout, nin, K3HIP_BF16, xs, nin, W, nin, C2, K3HIP_F32, nout, st);
        return r ? r : pair_add(C2, y, T, nout, st);
    };
    if (mfma && (rc = split_rows2(x, xs, T, E, st))) return rc;
    if ((rc = project(E, (int)P, x, w->q, qp))) return rc;
    if ((rc = project(E, (int)P, x, w->k, kp))) return rc;
    if ((rc = project(E, (int)P, x, w->v, vp))) return rc;
    if ((rc = project(E, H, x, w->b, bl))) return rc;
    if ((rc = project(E, D, x, w->f_a, fa))) return rc;
    if ((rc = project(E, (int)P, x, w->g, gl))) return rc;
    if (mfma && (rc = split_rows2(fa, xs, T, D, st))) return rc;
    if ((rc = project(D, (int)P, fa, w->f_b, z))) return rc;

    if ((rc = k3hip_kda_prep(T, H, D, K, w->gate_lb, K3HIP_F32, qp, kp, vp, z, bl, w->q_conv,
                             w->k_conv, w->v_conv, w->A_log, w->dt_bias, cs, q, k, v, g, al, bt,
                             stream)))
        return rc;
    const float qscale = 1.0f / sqrtf((float)D);
    if (T == 1)
        rc = k3hip_kda_decode(1, H, D, S, o, q, k, v, al, bt, qscale, stream);
    else if (chunk_ready() && chunk_gate_ok(w->gate_lb) && (D == 64 || D == 128))
        rc = k3hip_kda_chunk(T, H, D, 64, q, k, v, g, bt, qscale, S, o, nullptr, 0, stream);
    else
        rc = k3hip_kda_recurrent(T, H, D, q, k, v, al, bt, qscale, S, o, stream);
    if (rc) return rc;
    if ((rc = k3hip_kda_epilogue(T, H, D, w->rms_eps, o, gl, K3HIP_F32, w->o_norm, y, K3HIP_F32,
                                 stream)))
        return rc;
    if (mfma && (rc = split_rows2(y, xs, T, (int)P, st))) return rc;
    return project((int)P, E, y, w->o, out);
}

// fp32 -> bf16 (round to nearest even), for fp32 layer inputs of the bf16 prefill path.
__global__ void to_bf16_kernel(const float *__restrict__ x, uint16_t *__restrict__ y, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        y[i] = f2bf(x[i]);
}

// x [rows][D + H] fp32 (the f_a and b projections of one GEMM) -> y [rows][2D] bf16 with
// f_a = hi + lo: hi in columns 0..D-1, lo = bf16(f_a - hi) in D..2D-1 (the input of a K = 2D
// GEMM against [W | W]); the b logits are copied out to bl [rows][H].
__global__ void split_fa_b_kernel(const float *__restrict__ x, uint16_t *__restrict__ y,
                                  float *__restrict__ bl, int D, int H, size_t n)
{
    const int cols = D + H;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / (size_t)cols;
        const int c = (int)(i - r * (size_t)cols);
        const float v = x[i];
        if (c < D) {
            const uint16_t hi = f2bf(v);
            y[r * 2 * D + c] = hi;
            y[r * 2 * D + D + c] = f2bf(v - __uint_as_float((uint32_t)hi << 16));
        } else {
            bl[r * H + (c - D)] = v;
        }
    }
}

// The f_a / b projection left as `splits` K-range partial planes P[s][rows][D + H]: their sum
// in increasing s, f_a (columns 0..D-1) written as the bf16 pair y [rows][2D] (hi | lo, the
// input of the K = 2D GEMM against [W_fb | W_fb]) and the b logits to bl [rows][H].
__global__ void fab_reduce_kernel(const float *__restrict__ P, int splits, uint16_t *__restrict__ y,
                                  float *__restrict__ bl, int D, int H, size_t n)
{
    const int cols = D + H;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        float v = P[i];
        for (int s = 1; s < splits; s++) v += P[(size_t)s * n + i];
        const size_t r = i / (size_t)cols;
        const int c = (int)(i - r * (size_t)cols);
        if (c < D) {
            const uint16_t hi = f2bf(v);
            y[r * 2 * D + c] = hi;
            y[r * 2 * D + D + c] = f2bf(v - __uint_as_float((uint32_t)hi << 16));
        } else {
            bl[r * H + (c - D)] = v;
        }
    }
}

static unsigned grid_for(size_t n)
{
    size_t b = (n + 255) / 256;
    return (unsigned)(b > 8192 ? 8192 : (b ? b : 1));
}

__global__ void split_rows2_kernel(const float *__restrict__ x, uint16_t *__restrict__ y, size_t BN)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < BN;
         i += (size_t)gridDim.x * blockDim.x) {
        const uint16_t hi = f2bf(x[i]);
        y[i] = hi;
        y[BN + i] = f2bf(x[i] - __uint_as_float((uint32_t)hi << 16));
    }
}

__global__ void pair_add_kernel(const float *__restrict__ C2, float *__restrict__ y, size_t BN)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < BN;
         i += (size_t)gridDim.x * blockDim.x)
        y[i] = C2[i] + C2[BN + i];
}

namespace k3kda {
int split_rows2(const float *x, uint16_t *y, int B, int N, hipStream_t st)
{
    const size_t n = (size_t)B * N;
    if (!n) return K3HIP_OK;
    hipLaunchKernelGGL(split_rows2_kernel, dim3(grid_for(n)), dim3(256), 0, st, x, y, n);
    K3_LAUNCHED();
    return K3HIP_OK;
}

int pair_add(const float *C2, float *y, int B, int N, hipStream_t st)
{
    const size_t n = (size_t)B * N;
    if (!n) return K3HIP_OK;
    hipLaunchKernelGGL(pair_add_kernel, dim3(grid_for(n)), dim3(256), 0, st, C2, y, n);
    K3_LAUNCHED();
    return K3HIP_OK;
}
}  // namespace k3kda

// Which projection GEMMs the bf16 layer prefill runs (process-wide).
static std::atomic<int> g_proj_gemm{K3HIP_GEMM_HIPBLASLT};

extern "C" int k3hip_set_projection_gemm(int impl)
{
    clear_error();
    if (impl != K3HIP_GEMM_HIPBLASLT && impl != K3HIP_GEMM_HANDWRITTEN)
        K3_FAIL(K3HIP_EINVAL, "k3hip_set_projection_gemm: impl=%d (0 hipBLASLt, 1 hand-written)", impl);
    g_proj_gemm.store(impl, std::memory_order_relaxed);
    return K3HIP_OK;
}

extern "C" int k3hip_kda_layer_prefill(const k3hip_kda_weights *w, int T, void *out, int out_dtype,
                                       const void *x, int x_dtype, float *state, void *stream)
{
    clear_error();
    if (!w || !out || !x) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_layer_prefill: NULL argument");
    if (T < 0) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_layer_prefill: T=%d", T);
    if ((x_dtype != K3HIP_F32 && x_dtype != K3HIP_BF16) || (out_dtype != K3HIP_F32 && out_dtype != K3HIP_BF16))
        K3_FAIL(K3HIP_EINVAL, "k3hip_kda_layer_prefill: x_dtype=%d out_dtype=%d", x_dtype, out_dtype);
    const int E = w->hidden, H = w->H, D = w->D, K = w->K;
    if (w->wdt != K3_WBF16)
        K3_FAIL(K3HIP_EUNSUPPORTED, "k3hip_kda_layer_prefill: bf16 weights only (use k3hip_kda_layer_dev)");
    if (!(w->parts & K3HIP_UPLOAD_PREFILL))
        K3_FAIL(K3HIP_EINVAL, "k3hip_kda_layer_prefill: weights uploaded without K3HIP_UPLOAD_PREFILL");
    if (!w->o16)
        K3_FAIL(K3HIP_EUNSUPPORTED, "k3hip_kda_layer_prefill: W_o has values beyond fp16 range (use k3hip_kda_layer_dev)");
    if (!chunk_gate_ok(w->gate_lb) || (D != 64 && D != 128) || K > 4)
        K3_FAIL(K3HIP_EUNSUPPORTED, "k3hip_kda_layer_prefill: gate_lb=%g D=%d conv_k=%d outside the "
                "chunked prefill (use k3hip_kda_layer_dev)", w->gate_lb, D, K);
    if (T == 0) return K3HIP_OK;
    hipStream_t st = as_stream(stream);
    const size_t P = (size_t)H * D, TP = (size_t)T * P;
    const size_t wsb = k3hip_kda_chunk_workspace(T, H, D, 64);
    // The 4096-deep projections are plain GEMMs and run on hipBLASLt by default: the
    // hand-written MFMA GEMM (kda_mm.hip, k3hip_proj_gemm) matches it within 1-2% on the
    // 4096-wide ones but not on q/k/v, whose fp32 output stores keep it at ~0.93x; the 256-deep
    // z product runs on the hand-written kernel either way (faster there).
    // k3hip_set_projection_gemm(K3HIP_GEMM_HANDWRITTEN) selects the hand-written kernels for
    // every projection (`own`).
    // The hand-written kernel needs hidden % 64 == 0 and a 16-byte aligned bf16 x (an fp32 x is
    // converted into aligned scratch first); other layers take hipBLASLt, which has no such
    // limits, whatever the setting.
    const bool own = g_proj_gemm.load(std::memory_order_relaxed) == K3HIP_GEMM_HANDWRITTEN &&
                     mm_supported(E, E, E) && (x_dtype == K3HIP_F32 || ((uintptr_t)x & 15) == 0);
    int ncu = 256, rc;
    if ((rc = cu_count(ncu))) return rc;
    const int fab_s = own ? mm_splits(T, D + H, E, ncu) : 1;
    // scratch, 256-byte aligned pieces:
    //   0 x bf16 | 1 q k v projections fp32 | 2 f_a and b fp32 (split-K planes) | 3 f_a hi/lo bf16 |
    //   4 z fp32 | 5 b logits | 6 o fp32 | 7 gate fp16 | 8 y fp16 | 9 zero state | 10 chunk workspace |
    //   11 fp32 o_proj result (fallback path with a bf16 out)
    size_t sizes[] = {x_dtype == K3HIP_F32 ? (size_t)T * E * 2 : 0, 3 * TP * 4, (size_t)fab_s * T * (D + H) * 4,
                      (size_t)T * D * 4, TP * 4, (size_t)T * H * 4, TP * 4, TP * 2, TP * 2,
                      state ? 0 : (size_t)H * D * D * 4, wsb,
                      (!own && out_dtype == K3HIP_BF16) ? (size_t)T * E * 4 : 0};
    constexpr int NB = sizeof sizes / sizeof sizes[0];
    size_t off[NB], total = 0;
    for (int i = 0; i < NB; i++) {
        off[i] = total;
        total += (sizes[i] + 255) & ~(size_t)255;
    }
    StreamBuf buf;
    if ((rc = stream_alloc(buf, total, st))) return rc;
    char *base = (char *)buf.p;
    const void *xb = x;
    if (x_dtype == K3HIP_F32) {
        const size_t n = (size_t)T * E;
        hipLaunchKernelGGL(to_bf16_kernel, dim3(grid_for(n)), dim3(256), 0, st, (const float *)x,
                           (uint16_t *)(base + off[0]), n);
        K3_LAUNCHED();
        xb = base + off[0];
    }
    float *qp = (float *)(base + off[1]), *kp = qp + TP, *vp = kp + TP;
    float *fa = (float *)(base + off[2]);
    uint16_t *fa2 = (uint16_t *)(base + off[3]);
    float *z = (float *)(base + off[4]), *bl = (float *)(base + off[5]);
    float *o = (float *)(base + off[6]);
    uint16_t *g16 = (uint16_t *)(base + off[7]), *y16 = (uint16_t *)(base + off[8]);
    float *S = state;
    if (!S) {
        S = (float *)(base + off[9]);
        if ((rc = zero_fill(S, (size_t)H * D * D, st))) return rc;
    }
    float *cs = state ? state + (size_t)H * D * D : nullptr;
    const uint16_t *wq = (const uint16_t *)w->q;
    if (w->k != wq + P * E || w->v != wq + 2 * P * E || (const char *)w->b != (const char *)w->f_a + (size_t)D * E * 2)
        K3_FAIL(K3HIP_EINVAL, "kda layer: q, k, v (and f_a, b) weights are not one allocation");

    // 1 projections, fp32 results (a single bf16 rounding of q, k or v costs several times the
    //   2e-3 bar): q, k, v as one GEMM over their consecutive weight rows, its three column
    //   groups written to three [T][P] arrays; f_a and b as one split-K GEMM whose reduction
    //   writes f_a as a bf16 hi/lo pair for z = [f_a_hi | f_a_lo] [W_fb | W_fb]^T (fp32 accuracy)
    if (own) {
        if ((rc = mm(T, 3 * (int)P, E, K3HIP_BF16, xb, E, wq, E, qp, K3HIP_F32, (long)P, st, (int)P, (long)TP)))
            return rc;
        if ((rc = mm_splitk(T, D + H, E, fab_s, K3HIP_BF16, xb, E, w->f_a, E, fa, st))) return rc;
        const size_t n = (size_t)T * (D + H);
        hipLaunchKernelGGL(fab_reduce_kernel, dim3(grid_for(n)), dim3(256), 0, st, fa, fab_s, fa2, bl, D, H, n);
        K3_LAUNCHED();
        if ((rc = mm(T, (int)P, 2 * D, K3HIP_BF16, fa2, 2 * D, w->f_b2, 2 * D, z, K3HIP_F32, (long)P, st))) return rc;
    } else {
        GemmDesc g;
        g.M = T; g.N = (int)P; g.K = E;
        g.lda = E; g.ldb = E; g.ldc = (long)P;
        g.batch = 3; g.sa = 0; g.sb = (long)P * E; g.sc = (long)TP;
        if ((rc = gemm(g, xb, w->q, qp, st))) return rc;
        if ((rc = gemm_bf16(T, D + H, E, xb, w->f_a, fa, K3HIP_F32, st))) return rc;
        hipLaunchKernelGGL(split_fa_b_kernel, dim3(grid_for((size_t)T * (D + H))), dim3(256), 0, st, fa,
                           fa2, bl, D, H, (size_t)T * (D + H));
        K3_LAUNCHED();
        if (mm_supported(2 * D, 2 * D, 2 * D))
            rc = mm(T, (int)P, 2 * D, K3HIP_BF16, fa2, 2 * D, w->f_b2, 2 * D, z, K3HIP_F32, (long)P, st);
        else
            rc = gemm_bf16(T, (int)P, 2 * D, fa2, w->f_b2, z, K3HIP_F32, st);
        if (rc) return rc;
    }
    // 2-5 K1 fused into 6 K2 (chunked): the prepared q, k, v, g never reach HBM
    if ((rc = k3hip_kda_prefill(T, H, D, K, w->gate_lb, K3HIP_F32, qp, kp, vp, z, bl, w->q_conv,
                                w->k_conv, w->v_conv, w->A_log, w->dt_bias, cs,
                                1.0f / sqrtf((float)D), S, o, base + off[10], wsb, stream)))
        return rc;
    // 7-8 the output gate's logits in fp16 (only sigmoid(gate) is used: fp16's 2^-11 costs ~0.1
    //   of the bar, and an overflow to +-inf still gives the right limit 1 or 0), head RMSNorm,
    //   then the gate; y in fp16 (RMS-normalised: |y| <= sqrt(D) max|o_norm|)
    if (own) {
        if ((rc = mm(T, (int)P, E, K3HIP_BF16, xb, E, w->g, E, g16, K3_DT_F16, (long)P, st))) return rc;
        if ((rc = epilogue_split(T, H, D, w->rms_eps, o, g16, K3_DT_F16, w->o_norm, y16, st, true))) return rc;
        // 9 o_proj on fp16 MFMA against the fp16 copy of W_o
        return mm(T, E, (int)P, K3_DT_F16, y16, (long)P, w->o16, (long)P, out, out_dtype, E, st);
    }
    // hipBLASLt has no bf16-in, fp16-out algorithm: this path keeps fp32 gate logits (z is
    // consumed by now)
    float *gl = z;
    if ((rc = gemm_bf16(T, (int)P, E, xb, w->g, gl, K3HIP_F32, st))) return rc;
    if ((rc = epilogue_split(T, H, D, w->rms_eps, o, gl, K3HIP_F32, w->o_norm, y16, st, true))) return rc;
    if (out_dtype == K3HIP_F32) return gemm_f16(T, E, (int)P, y16, w->o16, out, K3HIP_F32, st);
    float *o32 = (float *)(base + off[11]);
    if ((rc = gemm_f16(T, E, (int)P, y16, w->o16, o32, K3HIP_F32, st))) return rc;
    const size_t n = (size_t)T * E;
    hipLaunchKernelGGL(to_bf16_kernel, dim3(grid_for(n)), dim3(256), 0, st, o32, (uint16_t *)out, n);
    K3_LAUNCHED();
    return K3HIP_OK;
}

// ------------------------------------------------------------- batched decode ----
// One token for each of B sequences: the q/k/v/f_a/beta and output-gate projections in one
// launch on the fragment-ordered decode copies, then the fused f_b + K1 + K3 + K4 step
// kernel, then o_proj. Three launches per layer step (B <= 64).
// The batched decode step with its scratch either allocated per call on the stream (scr ==
// nullptr) or taken from the caller's scr (scr_bytes, 256-byte aligned). Nothing in the
// scratch has to start at zero: every element a kernel reads was written earlier in the
// same call (the projections, the split-K partial planes, y). The layer output is zeroed by
// the step kernel when o_proj adds its two K-ranges into it.
static int layer_decode_impl(const k3hip_kda_weights *w, int B, float *out, const float *x, float *states,
                             long state_stride, void *stream, char *scr, size_t scr_bytes, const char *who)
{
    if (!w || !out || !x || !states) K3_FAIL(K3HIP_EINVAL, "%s: NULL argument", who);
    if (B < 0) K3_FAIL(K3HIP_EINVAL, "%s: B=%d", who, B);
    if (B == 0) return K3HIP_OK;
    if (w->wdt == K3_WBF16 && !(w->parts & K3HIP_UPLOAD_DECODE))
        K3_FAIL(K3HIP_EINVAL, "%s: weights uploaded without K3HIP_UPLOAD_DECODE", who);
    if (w->wdt != K3_WBF16 || !w->xin_f)
        K3_FAIL(K3HIP_EUNSUPPORTED, "%s: bf16 weights with hidden and head dim multiples "
                                    "of 8 only (use k3hip_kda_layer_dev)", who);
    const int E = w->hidden, H = w->H, D = w->D, K = w->K;
    const size_t P = (size_t)H * D;
    const long kper = (long)(P * D + 3 * P * (size_t)(K - 1));
    if (!is_pow2_head(D) || K < 1 || K > 4)
        K3_FAIL(K3HIP_EUNSUPPORTED, "%s: D=%d conv_k=%d", who, D, K);
    if (state_stride < kper || (state_stride & 3) || ((uintptr_t)states & 15))
        K3_FAIL(K3HIP_EINVAL, "%s: state stride %ld < %ld floats or misaligned", who,
                state_stride, kper);
    hipStream_t st = as_stream(stream);
    const size_t BP = (size_t)B * P;
    if ((E & 7) || (D & 7) || (P & 7) || ((uintptr_t)x & 15))
        K3_FAIL(K3HIP_EUNSUPPORTED, "%s: hidden=%d D=%d need multiples of 8, x 16-byte aligned", who, E, D);
    // scratch: q k v f_a b projections [B][NI] | output-gate partial planes | y |
    //          split-K partials (shared by the projections, which run one after another)
    const int NI = 3 * (int)P + D + H;
    const long ldi = (NI + 3) & ~3;   // a multiple of 4: f_a is read in place as an x operand
    const int gs = gemm_rows_splits((int)P, E);
    const size_t wsf = std::max(gemm_rows_ws_floats(B, NI, E), gemm_rows_ws_floats(B, E, (int)P));
    size_t sizes[] = {(size_t)B * ldi * 4, (size_t)gs * BP * 4, BP * 4, wsf * 4};
    constexpr int NB = sizeof sizes / sizeof sizes[0];
    size_t off[NB], total = 0;
    for (int i = 0; i < NB; i++) {
        off[i] = total;
        total += (sizes[i] + 255) & ~(size_t)255;
    }
    StreamBuf buf;
    int rc;
    char *bs = scr;
    if (!scr) {
        if ((rc = stream_alloc(buf, total, st))) return rc;
        bs = (char *)buf.p;
    } else if (total > scr_bytes) {
        K3_FAIL(K3HIP_EINVAL, "%s: B=%d at hidden %d, %d heads x %d needs %zu bytes of scratch; the no-allocation "
                "entry point has %zu (use k3hip_kda_layer_decode, or fewer sequences per call)", who, B, E, H, D,
                total, scr_bytes);
    }
    float *Cin = (float *)(bs + off[0]);
    float *glp = (float *)(bs + off[1]), *y = (float *)(bs + off[2]);
    float *ws = (float *)(bs + off[3]);
    const uint16_t *Win = (const uint16_t *)w->xin_f, *Wg = (const uint16_t *)w->g_f,
                   *Wfb = (const uint16_t *)w->f_b_f, *Wo = (const uint16_t *)w->o_f;

    // 1 projections: the fp32 rows against bf16 weights, each weight read once for all B
    //   (kda_rows.hip: x split into bf16 hi + lo in registers); q, k, v, f_a and the beta
    //   logits in one pass over their concatenated weights; the output gate left as split-K
    //   planes that the step kernel adds
    if ((rc = gemm_rows_with_part(B, E, x, E, NI, Win, Cin, ldi, (int)P, Wg, glp, st, ws, wsf))) return rc;
    // 2-8 the f_b product, K1, K3 and K4 on one token per sequence (kda_step.hip), conv
    //   history and state in each slot, then 9 o_proj: when it runs as two K-ranges into
    //   ordinary device memory, the step kernel zeroes `out` and both ranges add into it by
    //   float atomics (no reduction launch); other memory takes the ordered reduction
    const bool oz = gemm_rows_splits(E, (int)P) == 2 && coarse_device_mem(out);
    if ((rc = layer_step(B, H, D, K, w->gate_lb, w->rms_eps, 1.0f / sqrtf((float)D), Cin, ldi,
                         3 * (int)P + D, 3 * (int)P, Wfb, glp, gs, (long)BP, w->q_conv, w->k_conv, w->v_conv,
                         w->A_log, w->dt_bias, w->o_norm, states, state_stride, y, oz ? out : nullptr,
                         oz ? (long)B * E : 0, st)))
        return rc;
    return gemm_rows(B, E, (int)P, y, (long)P, Wo, out, E, st, ws, wsf, oz);
}

extern "C" int k3hip_kda_layer_decode(const k3hip_kda_weights *w, int B, float *out, const float *x,
                                      float *states, long state_stride, void *stream)
{
    clear_error();
    return layer_decode_impl(w, B, out, x, states, state_stride, stream, nullptr, 0, "k3hip_kda_layer_decode");
}

// ------------------------------------------------------- no-allocation decode ----
// Scratch of k3hip_kda_layer_decode_noalloc: a file-scope device array, one copy per GPU,
// held until the process ends. Host code never passes `noalloc_scratch` itself (on the host
// it only names the symbol); it takes the array's device address on each device from
// hipGetSymbolAddress, once, with that device current, and passes that address on.
constexpr size_t NOALLOC_SCRATCH_BYTES = 16ull << 20;
static __device__ __align__(256) char noalloc_scratch[NOALLOC_SCRATCH_BYTES];

static constexpr int NOALLOC_MAX_DEV = 64;
static std::mutex g_noalloc_mu;
static char *g_noalloc_ptr[NOALLOC_MAX_DEV];

static int noalloc_scratch_ptr(char **out)
{
    int dev = 0;
    K3_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= NOALLOC_MAX_DEV) K3_FAIL(K3HIP_EUNSUPPORTED, "no-allocation scratch: device %d", dev);
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (!g_noalloc_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(noalloc_scratch));
        if (e != hipSuccess || !p) {
            (void)hipGetLastError();
            K3_FAIL(K3HIP_EHIP, "hipGetSymbolAddress(noalloc_scratch) on device %d: %s", dev, hipGetErrorString(e));
        }
        g_noalloc_ptr[dev] = (char *)p;
    }
    *out = g_noalloc_ptr[dev];
    return K3HIP_OK;
}

extern "C" int k3hip_kda_layer_decode_noalloc(const k3hip_kda_weights *w, int B, float *out, const float *x,
                                              float *states, long state_stride, void *stream)
{
    clear_error();
    char *scr = nullptr;
    int rc;
    if ((rc = noalloc_scratch_ptr(&scr))) return rc;
    struct NoAlloc {
        NoAlloc() { g_no_alloc = true; }
        ~NoAlloc() { g_no_alloc = false; }
    } guard;
    return layer_decode_impl(w, B, out, x, states, state_stride, stream, scr, NOALLOC_SCRATCH_BYTES,
                             "k3hip_kda_layer_decode_noalloc");
}

// ------------------------------------------------------------------ drop-in ----
static void fatal(const char *where)
{
    fprintf(stderr,
            "k3kda: FATAL in %s: %s\n"
            "    Aborting rather than returning an unwritten output buffer.\n",
            where, g_err[0] ? g_err : "(no message)");
    abort();
}

extern "C" size_t k3_kda_scratch(const K3Cfg *c, int T)
{
    const size_t P = (size_t)c->kda_heads * c->kda_head_dim;
    return 6 * (size_t)T * P + (size_t)T * c->kda_heads + 2 * P + (size_t)c->kda_head_dim;
}

extern "C" void k3_kda_layer(float *out, const float *x, const K3KdaW *w, const K3Cfg *c, int T,
                             float *state, float *scratch)
{
    (void)scratch;
    if (T <= 0) return;
    if (!w || !c || !out || !x) {
        set_error("NULL argument");
        fatal("k3_kda_layer");
    }
    const int E = c->hidden, H = c->kda_heads, D = c->kda_head_dim, K = c->conv_k;
    if (E <= 0 || H <= 0 || D <= 0 || K <= 0) {
        set_error("hidden=%d H=%d D=%d conv_k=%d", E, H, D, K);
        fatal("k3_kda_layer");
    }
    if (w->wdt != K3_WF32 && w->wdt != K3_WBF16 && w->wdt != K3_WI8) {
        set_error("weight tag %d (fp32=0, bf16=1, int8 rows=2)", w->wdt);
        fatal("k3_kda_layer");
    }
    const size_t P = (size_t)H * D;
    const size_t nstate = P * D + 3 * P * (size_t)(K - 1);
    g_dropin_h2d = g_dropin_d2h = 0;
    g_in_dropin = true;
    // One stream-ordered block per call for what k3hip_kda_layer_dev reads (the matrices in
    // their own storage, the vectors) and for x, out and the state: no hipMalloc / hipFree.
    const hipStream_t st = nullptr;
    const size_t wbytes = dev_part_bytes(w, c), xb = (size_t)T * E * sizeof(float);
    const size_t sb = state ? nstate * sizeof(float) : 0;
    const size_t xoff = (wbytes + 255) & ~(size_t)255, ooff = xoff + ((xb + 255) & ~(size_t)255),
                 soff = ooff + ((xb + 255) & ~(size_t)255);
    StreamBuf blk;
    if (stream_alloc(blk, soff + sb, st)) fatal("k3_kda_layer");
    char *base = (char *)blk.p;
    k3hip_kda_weights dw{};
    dw.hidden = E; dw.H = H; dw.D = D; dw.K = K; dw.wdt = w->wdt; dw.parts = K3HIP_UPLOAD_DEV;
    dw.gate_lb = c->gate_lb; dw.rms_eps = c->rms_eps;
    dw.dev_block = base;
    if (bind_dev_part(&dw, w, c, base, st)) fatal("k3_kda_layer (weight upload)");
    float *dx = (float *)(base + xoff), *dout = (float *)(base + ooff), *dst = state ? (float *)(base + soff) : nullptr;
    if (hipMemcpyAsync(dx, x, xb, hipMemcpyHostToDevice, st) != hipSuccess ||
        (state && hipMemcpyAsync(dst, state, sb, hipMemcpyHostToDevice, st) != hipSuccess)) {
        set_error("host-to-device copy failed");
        fatal("k3_kda_layer");
    }
    g_dropin_h2d += xb + sb;
    if (k3hip_kda_layer_dev(&dw, T, dout, dx, dst, st)) fatal("k3_kda_layer");
    if (hipMemcpyAsync(out, dout, xb, hipMemcpyDeviceToHost, st) != hipSuccess ||
        (state && hipMemcpyAsync(state, dst, sb, hipMemcpyDeviceToHost, st) != hipSuccess) ||
        hipStreamSynchronize(st) != hipSuccess) {
        set_error("device-to-host copy failed: %s", hipGetErrorString(hipGetLastError()));
        fatal("k3_kda_layer");
    }
    g_dropin_d2h += xb + sb;
    g_in_dropin = false;
}
