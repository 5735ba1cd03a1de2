/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_oracle.h - CPU restatement of the reference KDA path. TEST INFRASTRUCTURE ONLY.
 *
 * This library is the oracle the GPU kernels are compared against, and the CPU
 * baseline that bench.py times beside them. Nothing in the shipped library links or
 * calls it. Every function names the reference lines (kimi-k3-in-c, src/core/k3_ops.c
 * unless stated) whose arithmetic it restates, including accumulation width and
 * summation order where the reference fixes them.
 *
 * Pinning (how each function is known to be right) is listed per function in the .c.
 */
#ifndef K3_ORACLE_H
#define K3_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/k3kda.h"

#ifdef __cplusplus
extern "C" {
#endif

float  orc_sigmoid(float x);
void   orc_rmsnorm(float *y, const float *x, const float *w, int n, float eps);
void   orc_l2norm(float *v, int n, float eps);
void   orc_shortconv(float *y, const float *x, const float *w, float *state,
                     int channels, int k, int T);
void   orc_kda_decay(float *g, float *alpha, const float *z, const float *A_log,
                     const float *dt_bias, int H, int D, float lb);
void   orc_kda_decay_softplus(float *g, float *alpha, const float *z, const float *A_log,
                              const float *dt_bias, int H, int D);
void   orc_kda_step(float *S, float *o, const float *q, const float *k, const float *v,
                    const float *alpha, float beta, int dk, int dv);
void   orc_matmul(float *y, const float *x, const float *W, int in, int out);
void   orc_matmul_bf16(float *y, const float *x, const uint16_t *W, int in, int out);
void   orc_matmul_q8(float *y, const float *x, const void *W, int in, int out);
void   orc_mmw(float *y, const float *x, const void *W, int wdt, int in, int out);
size_t orc_kda_scratch(const K3Cfg *c, int T);
void   orc_kda_layer(float *out, const float *x, const K3KdaW *w, const K3Cfg *c,
                     int T, float *state, float *scratch);

/* Batched decode: k3_kda_step over B*H (sequence, head) pairs, q scaled by q_scale
 * (the loop at src/core/k3_ops.c:927-938 with T = 1, repeated per sequence). OpenMP
 * over all pairs when nthreads > 1; per-pair arithmetic is unchanged. */
void   orc_kda_decode_batch(int B, int H, int D, float *S, float *o,
                            const float *q, const float *k, const float *v,
                            const float *alpha, const float *beta, float q_scale,
                            int nthreads);

/* The core of k3_kda_layer without the projections: steps 2-8 of
 * src/core/k3_ops.c:888-947 (conv+SiLU, L2, beta, decay, recurrence, head RMSNorm,
 * gate), one sequence. q_in/k_in/v_in/z [T][P], b_logit [T][H], gate_logit [T][P]
 * (already projected), out y [T][P]. state as in k3_kda_layer (nullable).
 * If o_rec is non-NULL it receives the raw recurrence output [T][P]. */
void   orc_kda_core(float *y, float *o_rec, const float *q_in, const float *k_in,
                    const float *v_in, const float *z, const float *b_logit,
                    const float *gate_logit, const K3KdaW *w, const K3Cfg *c, int T,
                    float *state, int nthreads);

/* The sequential recurrence alone over T tokens for all heads (src/core/k3_ops.c:927-938),
 * inputs already through K1: q,k,v,alpha [T][P], beta [T][H]. S [H][D][D] in/out. */
void   orc_kda_recurrence(int T, int H, int D, float *S, float *o,
                          const float *q, const float *k, const float *v,
                          const float *alpha, const float *beta, float q_scale,
                          int nthreads);

/* Round-to-nearest-even fp32 -> bf16 and the exact widening back. */
/* Gated MLA with an optional expanded KV cache (src/core/k3_ops.c:321-424). */
void   orc_mla_cached(float *out, const float *x, const K3MlaW *w, const K3Cfg *c, int T,
                      float *kvc, float *ropec, int cached, int cap);

uint16_t orc_f2bf(float f);
float    orc_bf2f(uint16_t h);

#ifdef __cplusplus
}
#endif

#endif
