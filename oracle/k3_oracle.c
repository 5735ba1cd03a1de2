/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_oracle.c - CPU restatement of the reference KDA path. TEST INFRASTRUCTURE ONLY:
 * the oracle the HIP kernels are tested against, and the CPU baseline of bench.py. The
 * shipped library never links it.
 *
 * Build contract (same as the reference, src/core/k3_ops.c:8-10, Makefile:133-140):
 * -ffp-contract=off, no -ffast-math. Double accumulators exactly where the reference
 * has them; fp32 everywhere else.
 *
 * Pinning, per function (tests/test_oracle_golden.py, tests/test_oracle_ref.py,
 * tests/test_oracle_invariants.py):
 *   orc_rmsnorm        rmsnorm.json; bitwise vs the reference C
 *   orc_shortconv      shortconv.json (out, state_after, continuation pair); bitwise
 *                      vs the reference C; closed form = left-padded conv1d + SiLU
 *   orc_kda_decay      kda_decay.json (A_log linspace gates per-head indexing); bitwise
 *   orc_kda_step       kda_recur1/8.json; bitwise; brute-force invariants (alpha=1,
 *                      beta=0 frozen state; exact-write property)
 *   orc_matmul[_bf16]  bitwise vs the reference C; bf16 path == fp32 path on widened
 *                      weights (the reference's own t_matmul_bf16 property)
 *   orc_matmul_q8      bitwise vs the reference C (its AVX2 order); within float rounding
 *                      of the double-precision dot of the dequantised row
 *   orc_l2norm         closed form (unit norm); kda_layer1/8.json
 *   orc_kda_layer      kda_layer1/8.json (out + recurrent state); bitwise vs reference
 *   orc_kda_core       equals orc_kda_layer minus the projections (tested by composing)
 *   orc_mla_cached     mla.json (uncached path, T tokens); the cached path equals the
 *                      uncached one token by token (tests/test_oracle_golden.py)
 *   orc_kda_decay_softplus  PARITY UNPINNED: the reference has no softplus gate; only
 *                      its closed form is checked. Selected by gate_lb == 0 in orc_kda_core
 *                      and orc_kda_layer (the reference itself would give g = 0 there: no
 *                      decay at all), which is the convention of the benchmark's small
 *                      configuration "-exp(A) softplus(.)" and of gates without a bound.
 */
#include "k3_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static void orc_die(const char *what, size_t bytes)
{
    fprintf(stderr, "k3_oracle: cannot allocate %zu bytes for %s\n", bytes, what);
    abort();
}

static void *orc_alloc(size_t bytes, const char *what)
{
    void *p = malloc(bytes ? bytes : 1);
    if (!p) orc_die(what, bytes);
    return p;
}

/* -------------------------------------------------------- bf16 helpers ---- */
uint16_t orc_f2bf(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu))   /* NaN stays NaN */
        return (uint16_t)((u >> 16) | 0x40u);
    const uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;                                           /* ties to even   */
    return (uint16_t)(u >> 16);
}

/* widening is a 16-bit left shift (include/k3/k3.h:273-280) */
float orc_bf2f(uint16_t h)
{
    const uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* ------------------------------------------------------------ sigmoid ---- */
/* src/core/k3_ops.c:105: 1 / (1 + expf(-x)) in fp32 */
float orc_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

/* ------------------------------------------------------------ rmsnorm ---- */
/* src/core/k3_ops.c:94-102: double sum of squares, mean, eps inside the root, the
 * inverse rounded to fp32 once, then y = w * x * inv in fp32 (w*x first). */
void orc_rmsnorm(float *y, const float *x, const float *w, int n, float eps)
{
    double acc = 0.0;
    for (int i = 0; i < n; i++) {
        const double xi = (double)x[i];
        acc += xi * xi;
    }
    const float r = (float)(1.0 / sqrt(acc / (double)n + (double)eps));
    for (int i = 0; i < n; i++) y[i] = (w[i] * x[i]) * r;
}

/* ------------------------------------------------------------- l2norm ---- */
/* src/core/k3_ops.c:845-851: SUM of squares in double, eps inside the root,
 * v *= (float)(1/sqrt(ss + eps)). */
void orc_l2norm(float *v, int n, float eps)
{
    double acc = 0.0;
    for (int i = 0; i < n; i++) acc += (double)v[i] * (double)v[i];
    const float r = (float)(1.0 / sqrt(acc + (double)eps));
    for (int i = 0; i < n; i++) v[i] = v[i] * r;
}

/* ---------------------------------------------------------- shortconv ---- */
/* src/core/k3_ops.c:133-165. Per channel: taps w[c][0..k-2] multiply the history
 * (oldest first), w[c][k-1] the current input; the fp32 accumulator starts from the
 * current-input product and adds the history taps oldest first; the history shifts
 * left and takes the current input; SiLU = acc * sigmoid(acc). y may alias x: each
 * x element is read before the y element at the same index is written. */
void orc_shortconv(float *y, const float *x, const float *w, float *state,
                   int channels, int k, int T)
{
    const int nh = k - 1;
    float hist[64];
    if (nh > 64) orc_die("shortconv history > 64 taps", (size_t)nh * 4);
    for (int c = 0; c < channels; c++) {
        const float *wc = w + (size_t)c * k;
        for (int j = 0; j < nh; j++) hist[j] = state ? state[(size_t)c * nh + j] : 0.0f;
        for (int t = 0; t < T; t++) {
            const size_t at = (size_t)t * channels + c;
            const float cur = x[at];
            float acc = wc[nh] * cur;
            for (int j = 0; j < nh; j++) acc += wc[j] * hist[j];
            for (int j = 1; j < nh; j++) hist[j - 1] = hist[j];
            if (nh) hist[nh - 1] = cur;
            y[at] = acc * orc_sigmoid(acc);
        }
        if (state)
            for (int j = 0; j < nh; j++) state[(size_t)c * nh + j] = hist[j];
    }
}

/* ------------------------------------------------------------- decay ---- */
/* src/core/k3_ops.c:168-183. a = expf(A_log[h]) PER HEAD; u = a * (z + dt_bias);
 * g = lb * sigmoid(u); alpha = expf(g). g may alias z (the layer writes g over z). */
void orc_kda_decay(float *g, float *alpha, const float *z, const float *A_log,
                   const float *dt_bias, int H, int D, float lb)
{
    for (int h = 0; h < H; h++) {
        const float a = expf(A_log[h]);
        for (int d = 0; d < D; d++) {
            const int i = h * D + d;
            const float u = a * (z[i] + dt_bias[i]);
            const float gi = lb * orc_sigmoid(u);
            g[i] = gi;
            alpha[i] = expf(gi);
        }
    }
}

/* The no-lower-bound form named by the benchmark's small configuration:
 * g = -exp(A_log[h]) * softplus(z + dt_bias). The reference has no such path
 * (tools/k3_ref.py:54-59 records it as the form K3 replaced), so this is PARITY
 * UNPINNED: it is checked only against its closed form. softplus(x) = log1p(exp(x)),
 * taken as x itself above 20 where the two agree in fp32. */
void orc_kda_decay_softplus(float *g, float *alpha, const float *z, const float *A_log,
                            const float *dt_bias, int H, int D)
{
    for (int h = 0; h < H; h++) {
        const float a = expf(A_log[h]);
        for (int d = 0; d < D; d++) {
            const int i = h * D + d;
            const float x = z[i] + dt_bias[i];
            const float sp = x > 20.0f ? x : log1pf(expf(x));
            const float gi = -a * sp;
            g[i] = gi;
            alpha[i] = expf(gi);
        }
    }
}

/* --------------------------------------------------------- recurrence ---- */
/* src/core/k3_ops.c:186-243, in its load-bearing order:
 *   1. S[i][:] *= alpha[i]
 *   2. u = S^T k, fp32, rows in order, rows with k[i] == 0 skipped
 *   3. S[i][j] += (k[i]*beta)*(v[j]-u[j]), rows with k[i] == 0 skipped
 *   4. o = S^T q from the updated S, rows with q[i] == 0 skipped
 * q arrives pre-scaled. */
void orc_kda_step(float *S, float *o, const float *q, const float *k, const float *v,
                  const float *alpha, float beta, int dk, int dv)
{
    float ustack[256];
    float *u = dv <= 256 ? ustack : (float *)orc_alloc((size_t)dv * 4, "step temp");

    for (int i = 0; i < dk; i++) {
        float *r = S + (size_t)i * dv;
        for (int j = 0; j < dv; j++) r[j] = r[j] * alpha[i];
    }
    for (int j = 0; j < dv; j++) u[j] = 0.0f;
    for (int i = 0; i < dk; i++) {
        if (k[i] == 0.0f) continue;
        const float *r = S + (size_t)i * dv;
        for (int j = 0; j < dv; j++) u[j] = u[j] + k[i] * r[j];
    }
    for (int i = 0; i < dk; i++) {
        if (k[i] == 0.0f) continue;
        float *r = S + (size_t)i * dv;
        const float kb = k[i] * beta;
        for (int j = 0; j < dv; j++) r[j] = r[j] + kb * (v[j] - u[j]);
    }
    for (int j = 0; j < dv; j++) o[j] = 0.0f;
    for (int i = 0; i < dk; i++) {
        if (q[i] == 0.0f) continue;
        const float *r = S + (size_t)i * dv;
        for (int j = 0; j < dv; j++) o[j] = o[j] + q[i] * r[j];
    }
    if (u != ustack) free(u);
}

/* ------------------------------------------------------------- matmul ---- */
/* src/core/k3_ops.c:265-291 (fp32 weights) and the scalar branch of :1122-1227 (bf16
 * weights, widened exactly). Per output row: sixteen double accumulators, element i of
 * each 16-block fused into accumulator i%16 with a double fma; the lanes are folded as
 * c_l = (a_l + a_{l+4}) + (a_{l+8} + a_{l+12}) for l = 0..3, then (c0+c1)+(c2+c3); the
 * in%16 tail is fused sequentially into that sum. Rows are independent. */
static double orc_dot16(const float *x, const void *row, int in, int is_bf16)
{
    double lane[16];
    for (int l = 0; l < 16; l++) lane[l] = 0.0;
    const float *rf = (const float *)row;
    const uint16_t *rb = (const uint16_t *)row;
    int i = 0;
    for (; i + 16 <= in; i += 16)
        for (int l = 0; l < 16; l++) {
            const double wv = is_bf16 ? (double)orc_bf2f(rb[i + l]) : (double)rf[i + l];
            lane[l] = fma(wv, (double)x[i + l], lane[l]);
        }
    double c[4];
    for (int l = 0; l < 4; l++) c[l] = (lane[l] + lane[l + 4]) + (lane[l + 8] + lane[l + 12]);
    double s = (c[0] + c[1]) + (c[2] + c[3]);
    for (; i < in; i++) {
        const double wv = is_bf16 ? (double)orc_bf2f(rb[i]) : (double)rf[i];
        s = fma(wv, (double)x[i], s);
    }
    return s;
}

void orc_matmul(float *y, const float *x, const float *W, int in, int out)
{
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (out > 64)
#endif
    for (int o = 0; o < out; o++) y[o] = (float)orc_dot16(x, W + (size_t)o * in, in, 0);
}

void orc_matmul_bf16(float *y, const float *x, const uint16_t *W, int in, int out)
{
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (out > 64)
#endif
    for (int o = 0; o < out; o++) y[o] = (float)orc_dot16(x, W + (size_t)o * in, in, 1);
}

/* src/core/k3_ops.c:1228-1301, the per-row int8 draft format (include/k3/k3.h:266-283): row
 * o is [f32 scale][int8 * in], 4 + in bytes. The reference carries no exactness contract for
 * it and sums in float in the order of its AVX2 branch, which is the build here (-mavx2
 * -mfma); that order is restated so the two agree bit for bit on x86: two 8-lane float
 * accumulators over 16-element blocks (elements i..i+7 into the first, i+8..i+15 into the
 * second, each a fused multiply-add), their lane sum, the 8 lanes folded as
 * (l + l4) for l = 0..3, then (m0 + m2, m1 + m3), then their sum; the in%16 tail added
 * sequentially (product then add); the scale applied once at the end. */
void orc_matmul_q8(float *y, const float *x, const void *W, int in, int out)
{
    const unsigned char *base = (const unsigned char *)W;
    const size_t rowb = (size_t)4 + (size_t)in;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (out > 64)
#endif
    for (int o = 0; o < out; o++) {
        const unsigned char *row = base + (size_t)o * rowb;
        float scale;
        memcpy(&scale, row, 4);
        const signed char *w = (const signed char *)(row + 4);
        float v0[8] = {0}, v1[8] = {0};
        int i = 0;
        for (; i + 15 < in; i += 16)
            for (int l = 0; l < 8; l++) {
                v0[l] = fmaf((float)w[i + l], x[i + l], v0[l]);
                v1[l] = fmaf((float)w[i + 8 + l], x[i + 8 + l], v1[l]);
            }
        float vs[8], lo[4];
        for (int l = 0; l < 8; l++) vs[l] = v0[l] + v1[l];
        for (int l = 0; l < 4; l++) lo[l] = vs[l] + vs[l + 4];
        const float m0 = lo[0] + lo[2], m1 = lo[1] + lo[3];
        float acc = m0 + m1;
        for (; i < in; i++) acc += (float)w[i] * x[i];
        y[o] = acc * scale;
    }
}

/* include/k3/k3.h:290-296 dispatch */
void orc_mmw(float *y, const float *x, const void *W, int wdt, int in, int out)
{
    if (wdt == K3_WBF16) orc_matmul_bf16(y, x, (const uint16_t *)W, in, out);
    else if (wdt == K3_WI8) orc_matmul_q8(y, x, W, in, out);
    else if (wdt == K3_WF32) orc_matmul(y, x, (const float *)W, in, out);
    else { fprintf(stderr, "k3_oracle: weight tag %d not supported\n", wdt); abort(); }
}

/* ------------------------------------------------------------- layer ---- */
/* src/core/k3_ops.c:853-862, the same float count */
size_t orc_kda_scratch(const K3Cfg *c, int T)
{
    const size_t H = (size_t)c->kda_heads, D = (size_t)c->kda_head_dim, P = H * D;
    return 6 * (size_t)T * P + (size_t)T * H + 2 * P + D;
}

/* The recurrence driver of src/core/k3_ops.c:918-938: q scaled by (1/sqrtf(D)) into a
 * work row, then k3_kda_step, heads independent, tokens in order within a head. */
void orc_kda_recurrence(int T, int H, int D, float *S, float *o,
                        const float *q, const float *k, const float *v,
                        const float *alpha, const float *beta, float q_scale,
                        int nthreads)
{
    const size_t P = (size_t)H * D;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
#endif
    for (int h = 0; h < H; h++) {
        float qs[256];
        for (int t = 0; t < T; t++) {
            const size_t off = (size_t)t * P + (size_t)h * D;
            for (int i = 0; i < D; i++) qs[i] = q[off + i] * q_scale;
            orc_kda_step(S + (size_t)h * D * D, o + off, qs, k + off, v + off,
                         alpha + off, beta[(size_t)t * H + h], D, D);
        }
    }
    (void)nthreads;
}

/* Steps 2-8 of src/core/k3_ops.c:888-947 on already-projected inputs. */
void orc_kda_core(float *y, float *o_rec, const float *q_in, const float *k_in,
                  const float *v_in, const float *z, const float *b_logit,
                  const float *gate_logit, const K3KdaW *w, const K3Cfg *c, int T,
                  float *state, int nthreads)
{
    const int H = c->kda_heads, D = c->kda_head_dim, K = c->conv_k, nh = K - 1;
    const size_t P = (size_t)H * D, TP = (size_t)T * P;
    if (D > 256) orc_die("head dim > 256", (size_t)D);
    float *q = (float *)orc_alloc(TP * 4, "q"), *k = (float *)orc_alloc(TP * 4, "k");
    float *v = (float *)orc_alloc(TP * 4, "v"), *g = (float *)orc_alloc(TP * 4, "g");
    float *al = (float *)orc_alloc(TP * 4, "alpha");
    float *bt = (float *)orc_alloc((size_t)T * H * 4, "beta");
    float *o = o_rec ? o_rec : (float *)orc_alloc(TP * 4, "o");

    float *cs = state ? state + (size_t)H * D * D : NULL;
    orc_shortconv(q, q_in, w->q_conv, cs, (int)P, K, T);
    orc_shortconv(k, k_in, w->k_conv, cs ? cs + P * nh : NULL, (int)P, K, T);
    orc_shortconv(v, v_in, w->v_conv, cs ? cs + 2 * P * nh : NULL, (int)P, K, T);
    for (int t = 0; t < T; t++)
        for (int h = 0; h < H; h++) {
            orc_l2norm(q + (size_t)t * P + (size_t)h * D, D, 1e-6f);
            orc_l2norm(k + (size_t)t * P + (size_t)h * D, D, 1e-6f);
        }
    for (int t = 0; t < T; t++) {
        for (int h = 0; h < H; h++)
            bt[(size_t)t * H + h] = orc_sigmoid(b_logit[(size_t)t * H + h]);
        if (c->gate_lb != 0.0f)
            orc_kda_decay(g + (size_t)t * P, al + (size_t)t * P, z + (size_t)t * P,
                          w->A_log, w->dt_bias, H, D, c->gate_lb);
        else   /* no lower bound: the softplus gate (parity unpinned, see orc_kda_decay_softplus) */
            orc_kda_decay_softplus(g + (size_t)t * P, al + (size_t)t * P, z + (size_t)t * P,
                                   w->A_log, w->dt_bias, H, D);
    }
    float *S = state;
    float *Sown = NULL;
    if (!S) {
        Sown = (float *)calloc((size_t)H * D * D, sizeof(float));
        if (!Sown) orc_die("state", (size_t)H * D * D * 4);
        S = Sown;
    }
    orc_kda_recurrence(T, H, D, S, o, q, k, v, al, bt, 1.0f / sqrtf((float)D), nthreads);
    for (int t = 0; t < T; t++) {
        float *yt = y + (size_t)t * P;
        const float *ot = o + (size_t)t * P;
        const float *gt = gate_logit + (size_t)t * P;
        for (int h = 0; h < H; h++)
            orc_rmsnorm(yt + (size_t)h * D, ot + (size_t)h * D, w->o_norm, D, c->rms_eps);
        for (size_t i = 0; i < P; i++) yt[i] = yt[i] * orc_sigmoid(gt[i]);
    }
    free(Sown);
    free(q); free(k); free(v); free(g); free(al); free(bt);
    if (!o_rec) free(o);
}

/* src/core/k3_ops.c:864-951, one sequence:
 *   1 projections per token (q,k,v,b, then f_a -> f_b)       :877-886
 *   2 shortconv x3 with the conv state after the S block     :888-892
 *   3 l2norm on q and k per head                             :894-899
 *   4/5 beta = sigmoid(b), decay chain written over z        :901-906
 *   6 recurrence, q * (1/sqrtf(D))                           :908-938
 *   7-9 per token: head RMSNorm in place, g projection, *= sigmoid, o_proj  :940-949 */
void orc_kda_layer(float *out, const float *x, const K3KdaW *w, const K3Cfg *c,
                   int T, float *state, float *scratch)
{
    const int E = c->hidden, H = c->kda_heads, D = c->kda_head_dim;
    const size_t P = (size_t)H * D, TP = (size_t)T * P;
    (void)scratch;   /* the restatement keeps its own buffers */
    float *qp = (float *)orc_alloc(TP * 4, "q proj"), *kp = (float *)orc_alloc(TP * 4, "k proj");
    float *vp = (float *)orc_alloc(TP * 4, "v proj"), *z = (float *)orc_alloc(TP * 4, "z");
    float *bl = (float *)orc_alloc((size_t)T * H * 4, "b logit");
    float *gl = (float *)orc_alloc(TP * 4, "gate logit");
    float *fa = (float *)orc_alloc((size_t)D * 4, "f_a out");
    float *yc = (float *)orc_alloc(TP * 4, "core out");

    for (int t = 0; t < T; t++) {
        const float *xt = x + (size_t)t * E;
        orc_mmw(qp + (size_t)t * P, xt, w->q, w->wdt, E, (int)P);
        orc_mmw(kp + (size_t)t * P, xt, w->k, w->wdt, E, (int)P);
        orc_mmw(vp + (size_t)t * P, xt, w->v, w->wdt, E, (int)P);
        orc_mmw(bl + (size_t)t * H, xt, w->b, w->wdt, E, H);
        orc_mmw(fa, xt, w->f_a, w->wdt, E, D);
        orc_mmw(z + (size_t)t * P, fa, w->f_b, w->wdt, D, (int)P);
        orc_mmw(gl + (size_t)t * P, xt, w->g, w->wdt, E, (int)P);
    }
    int nt = 1;
#ifdef _OPENMP
    nt = omp_get_max_threads();
#endif
    orc_kda_core(yc, NULL, qp, kp, vp, z, bl, gl, w, c, T, state, nt);
    for (int t = 0; t < T; t++)
        orc_mmw(out + (size_t)t * E, yc + (size_t)t * P, w->o, w->wdt, (int)P, E);
    free(qp); free(kp); free(vp); free(z); free(bl); free(gl); free(fa); free(yc);
}

/* ------------------------------------------------------- batched decode ---- */
void orc_kda_decode_batch(int B, int H, int D, float *S, float *o,
                          const float *q, const float *k, const float *v,
                          const float *alpha, const float *beta, float q_scale,
                          int nthreads)
{
    const long pairs = (long)B * H;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
#endif
    for (long p = 0; p < pairs; p++) {
        float qs[256];
        const size_t off = (size_t)p * D;
        for (int i = 0; i < D; i++) qs[i] = q[off + i] * q_scale;
        orc_kda_step(S + (size_t)p * D * D, o + off, qs, k + off, v + off, alpha + off,
                     beta[p], D, D);
    }
    (void)nthreads;
}

/* ---------------------------------------------------------------- MLA ---- */
/* src/core/k3_ops.c:321-424 (k3_mla_cached): gated MLA, NoPE. Per token: q = q_b(rmsnorm(
 * q_a x)) [H][nope+rope]; ONE projection c = kv_a x gives the latent (rmsnorm'd, the rope
 * slot excluded) and the shared rope slot; the expanded per-head keys/values
 * kv = kv_b(latent) [H][nope+v] are cached (kvc [cap][H*(nope+v)], ropec [cap][rope]) or,
 * with kvc == NULL, kept for this call only. Attention per head, causal over positions
 * 0..p: score = (float)(double dot over nope + rope) * (nope+rope)^-0.5 in fp32, max,
 * expf, double sum z, weights (float)(e/z), fp32 weighted sum of values in position order.
 * Then the gate (sigmoid(g x), multiplied BEFORE o_proj, no norm) and o_proj. */
void orc_mla_cached(float *out, const float *x, const K3MlaW *w, const K3Cfg *c, int T,
                    float *kvc, float *ropec, int cached, int cap)
{
    const int E = c->hidden, H = c->n_heads;
    const int qn = c->qk_nope, qr = c->qk_rope, vh = c->v_head;
    const int qh = qn + qr, kvw = c->kv_lora + qr, kvd = qn + vh;
    const float scale = 1.0f / sqrtf((float)qh);
    if (!kvc) cached = 0;
    const int last = cached + T - 1;
    if (kvc && last >= cap) {
        fprintf(stderr, "k3_oracle: MLA cache position %d past capacity %d\n", last, cap);
        abort();
    }
    float *q = (float *)orc_alloc(sizeof(float) * (size_t)T * H * qh, "mla q");
    float *ct = (float *)orc_alloc(sizeof(float) * (size_t)kvw, "mla ct");
    float *ql = (float *)orc_alloc(sizeof(float) * (size_t)c->q_lora, "mla ql");
    float *acc = (float *)orc_alloc(sizeof(float) * (size_t)H * vh, "mla acc");
    float *gb = (float *)orc_alloc(sizeof(float) * (size_t)H * vh, "mla gate");
    float *sc = (float *)orc_alloc(sizeof(float) * (size_t)(last + 1), "mla scores");
    float *kvs = kvc ? NULL : (float *)orc_alloc(sizeof(float) * (size_t)T * H * kvd, "mla kv");
    float *rps = ropec ? NULL : (float *)orc_alloc(sizeof(float) * (size_t)T * qr + 1, "mla rope");
#define KV_AT(p) (kvc ? kvc + (size_t)(p) * H * kvd : kvs + (size_t)(p) * H * kvd)
#define ROPE_AT(p) (ropec ? ropec + (size_t)(p) * qr : rps + (size_t)(p) * qr)
    for (int t = 0; t < T; t++) {
        const int p = cached + t;
        const float *xt = x + (size_t)t * E;
        orc_mmw(ql, xt, w->q_a, w->wdt, E, c->q_lora);
        orc_rmsnorm(ql, ql, w->q_a_norm, c->q_lora, c->rms_eps);
        orc_mmw(q + (size_t)t * H * qh, ql, w->q_b, w->wdt, c->q_lora, H * qh);
        orc_mmw(ct, xt, w->kv_a, w->wdt, E, kvw);
        orc_rmsnorm(ct, ct, w->kv_a_norm, c->kv_lora, c->rms_eps);
        memcpy(ROPE_AT(p), ct + c->kv_lora, (size_t)qr * sizeof(float));
        orc_mmw(KV_AT(p), ct, w->kv_b, w->wdt, c->kv_lora, H * kvd);
    }
    for (int t = 0; t < T; t++) {
        const int p = cached + t;
        for (int h = 0; h < H; h++) {
            const float *qt = q + ((size_t)t * H + h) * qh;
            float m = -INFINITY;
            for (int s = 0; s <= p; s++) {
                const float *ks = KV_AT(s) + (size_t)h * kvd;
                const float *kr = ROPE_AT(s);
                double d = 0.0;
                for (int i = 0; i < qn; i++) d += (double)qt[i] * (double)ks[i];
                for (int i = 0; i < qr; i++) d += (double)qt[qn + i] * (double)kr[i];
                sc[s] = (float)d * scale;
                if (sc[s] > m) m = sc[s];
            }
            double z = 0.0;
            for (int s = 0; s <= p; s++) {
                sc[s] = expf(sc[s] - m);
                z += sc[s];
            }
            float *o = acc + (size_t)h * vh;
            for (int j = 0; j < vh; j++) o[j] = 0.0f;
            for (int s = 0; s <= p; s++) {
                const float pr = (float)(sc[s] / z);
                const float *vs = KV_AT(s) + (size_t)h * kvd + qn;
                for (int j = 0; j < vh; j++) o[j] += pr * vs[j];
            }
        }
        if (w->g) {
            orc_mmw(gb, x + (size_t)t * E, w->g, w->wdt, E, H * vh);
            for (int i = 0; i < H * vh; i++) acc[i] *= 1.0f / (1.0f + expf(-gb[i]));
        }
        orc_mmw(out + (size_t)t * E, acc, w->o, w->wdt, H * vh, E);
    }
#undef KV_AT
#undef ROPE_AT
    free(q); free(ct); free(ql); free(acc); free(gb); free(sc); free(kvs); free(rps);
}
