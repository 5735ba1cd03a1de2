/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3kda.h - MI355X (gfx950) Kimi Delta Attention path, C ABI.
 *
 * Two surfaces live here.
 *
 *   1. The drop-in: k3_kda_scratch / k3_kda_layer with the exact signature and meaning of
 *      the reference engine's CPU entry points (include/k3/k3.h:464-469, defined at
 *      src/core/k3_ops.c:853-951). Host pointers in, host pointers out, `state` updated in
 *      place in the reference layout, NULL state = fresh sequence. A fatal condition
 *      aborts with a message, as the reference does (src/core/k3_ops.c:37-78).
 *
 *   2. The device API (k3hip_*): batched, stream-ordered entry points on device pointers
 *      for the four kernels of the path. They return 0 or a K3HIP_E* code and never abort;
 *      k3hip_last_error() gives the message for the calling thread.
 *
 * K3Cfg and K3KdaW below are LAYOUT MIRRORS of the reference's structs
 * (include/k3/k3.h:73-120 and :448-462) so that an engine built against its own k3.h can
 * pass its structs straight through. They are declared only when the reference header has
 * not been included first (its include guard is K3_H).
 *
 * Tensor layouts (P = H*D, head-major, channel-minor, as in the reference):
 *   activations  [T][P]          token-major rows
 *   beta         [T][H]
 *   state S      [H][D][D]       row i = key channel, column j = value channel
 *   conv state   [3][P][K-1]     q block, k block, v block, oldest input first
 *   full state   S then conv     H*D*D + 3*P*(K-1) floats (src/cli/k3_state.c:23-29)
 */
#ifndef K3KDA_H
#define K3KDA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef K3_H
/* Field-for-field mirror of the reference K3Cfg (include/k3/k3.h:73-120). Only the KDA
 * fields (hidden, rms_eps, kda_heads, kda_head_dim, conv_k, gate_lb) are read here. */
typedef struct {
    int hidden;
    int n_layers;
    int vocab;
    float rms_eps;
    int kda_heads;
    int kda_head_dim;
    int conv_k;
    float gate_lb;
    int n_heads;
    int q_lora;
    int kv_lora;
    int qk_nope;
    int qk_rope;
    int v_head;
    int mla_out_gate;
    int n_experts;
    int topk;
    int n_shared;
    int latent;
    int moe_inter;
    float routed_scale;
    int moe_renorm;
    int latent_norm;
    int first_dense;
    int dense_inter;
    int attn_res_block;
    float situ_b1;
    float situ_b2;
    int  n_full_attn;
    int *full_attn;
} K3Cfg;

/* Weight-storage tags of the reference (include/k3/k3.h:270). */
enum { K3_WF32 = 0, K3_WBF16 = 1, K3_WI8 = 2 };

/* Field-for-field mirror of the reference K3KdaW (include/k3/k3.h:448-462). Matrices are
 * tagged by wdt; conv kernels, A_log, dt_bias and o_norm are always fp32. */
typedef struct {
    const void  *q, *k, *v;                 /* [P][hidden]                   */
    const float *q_conv, *k_conv, *v_conv;  /* [P][conv_k]                   */
    const void  *f_a, *f_b;                 /* [D][hidden], [P][D]           */
    const float *A_log;                     /* [H]  per head                 */
    const float *dt_bias;                   /* [P]                           */
    const void  *b;                         /* [H][hidden]                   */
    const void  *g;                         /* [P][hidden]                   */
    const float *o_norm;                    /* [D]                           */
    const void  *o;                         /* [hidden][P]                   */
    int          wdt;
} K3KdaW;

/* Field-for-field mirror of the reference K3MlaW (include/k3/k3.h:203-210): gated MLA,
 * NoPE. Matrices tagged by wdt; the two layernorm weights are fp32; g may be NULL. */
typedef struct {
    const void  *q_a, *q_b;                 /* [q_lora][hidden], [H*(nope+rope)][q_lora] */
    const void  *kv_a, *kv_b;               /* [kv_lora+rope][hidden], [H*(nope+v)][kv_lora] */
    const void  *o, *g;                     /* [hidden][H*v], [H*v][hidden]  */
    const float *q_a_norm, *kv_a_norm;      /* [q_lora], [kv_lora]           */
    int          wdt;
} K3MlaW;

/* Replaces k3_kda_scratch, include/k3/k3.h:464 (src/core/k3_ops.c:853-862). Returns the
 * same float count, so a caller that sizes scratch from it is unchanged. The GPU path
 * keeps its intermediates in device memory and does not touch the host scratch. */
size_t k3_kda_scratch(const K3Cfg *c, int T);

/* Replaces k3_kda_layer, include/k3/k3.h:468-469 (src/core/k3_ops.c:864-951).
 * out[T][hidden] = KDA(x[T][hidden]); state (nullable) is H*D*D recurrent floats then
 * 3*P*(conv_k-1) conv floats, read and written in place. Weights are uploaded on every
 * call: the reference engine re-binds streamed weights through a ring buffer, so a cache
 * keyed on host pointers would read stale bytes. Use k3hip_kda_upload for resident ones. */
void   k3_kda_layer(float *out, const float *x, const K3KdaW *w, const K3Cfg *c,
                    int T, float *state, float *scratch);
#endif /* K3_H */

/* ------------------------------------------------------------ device API ---- */
enum {
    K3HIP_OK          = 0,
    K3HIP_EINVAL      = 1,   /* a size, pointer or dtype the kernels do not accept  */
    K3HIP_EHIP        = 2,   /* the HIP runtime reported an error                   */
    K3HIP_EUNSUPPORTED= 3,   /* a configuration no kernel here is built for         */
    K3HIP_ENOMEM      = 4    /* device allocation failed                            */
};

/* Activation storage for k3hip_* inputs/outputs that accept either. */
enum { K3HIP_F32 = 0, K3HIP_BF16 = 1 };

/* Message for the last non-zero return on the calling thread ("" when none). */
const char *k3hip_last_error(void);

/* Version string of the library (kernel set and target). */
const char *k3hip_version(void);

/* Number of HIP devices visible (0 on a machine without one); never aborts. */
int k3hip_device_count(void);

/* K3: batched single-token recurrence, one (sequence, head) per workgroup.
 * Replaces, per (b, h), the call k3_kda_step(S, o, q*q_scale, k, v, alpha, beta, D, D)
 * of src/core/k3_ops.c:930-937 (k3_kda_step is include/k3/k3.h:164, defined at
 * src/core/k3_ops.c:186-243): decay rows by alpha, u = S^T k, S += k (beta (v-u))^T,
 * o = S^T q read from the UPDATED state. One read and one write of S.
 *   S      [B][H][D][D] fp32, in/out         q,k,v,alpha  [B][H][D] fp32
 *   o      [B][H][D]    fp32, out            beta         [B][H]    fp32
 * D in {16, 32, 64, 128}. */
int k3hip_kda_decode(int B, int H, int D, float *S, float *o,
                     const float *q, const float *k, const float *v,
                     const float *alpha, const float *beta, float q_scale, void *stream);

/* K1: ShortConv + SiLU on q, k, v, L2-norm on q and k, beta and the decay chain, for one
 * sequence of T tokens. Replaces steps 2-5 of src/core/k3_ops.c:888-906: k3_shortconv
 * (:133-165) x3 with the history carried in conv_state, l2norm_ (:845-851, eps 1e-6,
 * sum of squares), beta = sigmoid(b_logit) (:903), and k3_kda_decay (:168-183).
 *   q_in,k_in,v_in [T][P] (in_dtype)  z [T][P] fp32 = f_b(f_a(x)) before dt_bias
 *   b_logit [T][H] fp32               q_conv,k_conv,v_conv [P][K]; A_log [H]; dt_bias [P]
 *   conv_state [3][P][K-1] in/out, NULL = zero history, not written back
 *   q_out,k_out,v_out [T][P] fp32     g_out, alpha_out [T][P] fp32 (either may be NULL)
 *   beta_out [T][H] fp32 */
int k3hip_kda_prep(int T, int H, int D, int K, float gate_lb, int in_dtype,
                   const void *q_in, const void *k_in, const void *v_in,
                   const float *z, const float *b_logit,
                   const float *q_conv, const float *k_conv, const float *v_conv,
                   const float *A_log, const float *dt_bias, float *conv_state,
                   float *q_out, float *k_out, float *v_out,
                   float *g_out, float *alpha_out, float *beta_out, void *stream);

/* K2: chunked gated delta-rule prefill over T tokens of one sequence, all H heads.
 * Equal (to the stated tolerance) to T sequential k3_kda_step calls per head
 * (src/core/k3_ops.c:927-938) from state S, with q scaled by q_scale. Inputs are K1's
 * outputs: q,k L2-normalised (unscaled), v, g = log-decay, beta.
 *   q,k,v,g [T][P] fp32   beta [T][H] fp32   S [H][D][D] in/out   o [T][P] fp32
 * D = 128 or 64, chunk = 64. workspace: NULL = library-managed (the whole sequence at
 * once), else device memory of workspace_bytes. Given fewer than
 * k3hip_kda_chunk_workspace(T,H,D,chunk) bytes, the sequence is processed in passes of
 * the most whole 64-token chunks that fit (S carried; the same bits as one pass); fewer
 * than k3hip_kda_chunk_workspace(64,H,D,chunk) bytes is K3HIP_EINVAL. */
size_t k3hip_kda_chunk_workspace(int T, int H, int D, int chunk);
int k3hip_kda_chunk(int T, int H, int D, int chunk,
                    const float *q, const float *k, const float *v,
                    const float *g, const float *beta, float q_scale,
                    float *S, float *o, void *workspace, size_t workspace_bytes,
                    void *stream);

/* K1 + K2 fused: the same arguments as k3hip_kda_prep followed by k3hip_kda_chunk, and
 * bit-identical results (o, S and the outgoing conv_state), without the prepared fp32
 * q, k, v, g ever being written to memory. Replaces steps 2-6 of
 * src/core/k3_ops.c:888-938 for a T-token prefill.
 *   in_dtype = K3HIP_BF16 or K3HIP_F32; D = 128 or 64; conv_k 1..4; -80/15 <= gate_lb < 0 (the
 *   bounded gate of k3_kda_decay); q_in, k_in, v_in, z 16-byte aligned; workspace as for
 *   k3hip_kda_chunk (chunk 64; in passes, conv_state carries the history between them,
 *   and with conv_state NULL and conv_k > 1 the workspace also holds 3*P*(conv_k-1) floats
 *   of it, rounded up to 256 bytes). Other shapes return K3HIP_EUNSUPPORTED: use prep + chunk. */
int k3hip_kda_prefill(int T, int H, int D, int K, float gate_lb, int in_dtype,
                      const void *q_in, const void *k_in, const void *v_in,
                      const float *z, const float *b_logit,
                      const float *q_conv, const float *k_conv, const float *v_conv,
                      const float *A_log, const float *dt_bias, float *conv_state,
                      float q_scale, float *S, float *o,
                      void *workspace, size_t workspace_bytes, void *stream);

/* Sequential-in-T prefill on the GPU, parallel over heads and value columns only. The
 * exact step order of k3_kda_step per token; used for gate bounds outside the chunked
 * kernel's exponent range (|gate_lb| * 15 > 80) and as a second GPU opinion in tests.
 * Same arguments and layouts as k3hip_kda_chunk. */
int k3hip_kda_recurrent(int T, int H, int D,
                        const float *q, const float *k, const float *v,
                        const float *alpha, const float *beta, float q_scale,
                        float *S, float *o, void *stream);

/* K1 (T = 1) + K3 + K4 in one launch: one decode token for each of B sequences, the work of
 * k3hip_kda_prep on one token, k3hip_kda_decode and k3hip_kda_epilogue (src/core/k3_ops.c:888-947
 * at T = 1) without q, k, v, alpha, beta or o leaving the chip. One workgroup per (head,
 * sequence); the state is read once and written once.
 *   q_in,k_in,v_in [B][P] (in_dtype)  z [B][P] fp32 = f_b(f_a(x)) before dt_bias
 *   b_logit [B][H] fp32               gate [B][P] output-gate logits (gate_dtype)
 *   conv_state [B][3][P][K-1] in/out (may be NULL only for conv_k = 1)
 *   S [B][H][D][D] in/out             y [B][P] = RMSNorm(o) * sigmoid(gate) (y_dtype)
 * D in {16, 32, 64, 128}, conv_k 1..4, gate_lb <= 0 (0 selects the softplus gate); S and
 * o_norm 16-byte aligned, gate and y 16-byte (fp32) or 8-byte (bf16) aligned. */
int k3hip_kda_decode_step(int B, int H, int D, int K, float gate_lb, float rms_eps, int in_dtype,
                          const void *q_in, const void *k_in, const void *v_in, const float *z,
                          const float *b_logit, const void *gate, int gate_dtype,
                          const float *q_conv, const float *k_conv, const float *v_conv,
                          const float *A_log, const float *dt_bias, const float *o_norm,
                          float *conv_state, float q_scale, float *S, void *y, int y_dtype,
                          void *stream);

/* K4: per (token, head) RMSNorm over D with the shared weight o_norm[D] (eps inside the
 * root, double-width mean in the reference, src/core/k3_ops.c:94-102), THEN multiply by
 * sigmoid(gate). Replaces src/core/k3_ops.c:940-947 up to the o_proj matmul.
 *   o [T][P] fp32   gate [T][P] (gate_dtype)   o_norm [D]   y [T][P] (y_dtype) */
int k3hip_kda_epilogue(int T, int H, int D, float rms_eps,
                       const float *o, const void *gate, int gate_dtype,
                       const float *o_norm, void *y, int y_dtype, void *stream);

/* The projection GEMM of the bf16 prefill path (hand-written gfx950 MFMA kernel): every
 * per-token k3_mmw call of src/core/k3_ops.c:879-886, :946, :948 (k3_matmul_bf16,
 * :1122-1227) for T tokens is one row block of
 *   C[M][N] = A[M][K] . B[N][K]^T      A activations, B the weight as stored ([out][in])
 * with fp32 accumulation. ab_dtype K3HIP_BF16 or K3HIP_F16 (A and B alike); c_dtype
 * K3HIP_F32, K3HIP_BF16 or K3HIP_F16; leading dimensions in elements. Needs K % 64 == 0,
 * lda, ldb multiples of 8, ldc >= N, A and B 16-byte aligned (else K3HIP_EUNSUPPORTED).
 * Stream-ordered, allocates nothing, bit-reproducible. */
enum { K3HIP_F16 = 3 };
int k3hip_proj_gemm(int M, int N, int K, int ab_dtype, const void *A, long lda, const void *B, long ldb,
                    void *C, int c_dtype, long ldc, void *stream);

/* Device-resident weights for the full layer. Matrices keep their wdt: fp32, bf16, or the
 * per-row int8 draft format K3_WI8 (include/k3/k3.h:266-283, each row [f32 scale][int8 * in],
 * which the reference engine binds for its --draft-trunk hybrid decode, src/model/k3_bind.c:441);
 * the small fp32 vectors are copied as is. Int8 weights serve k3hip_kda_layer_dev and the
 * drop-in k3_kda_layer (the reference's k3_matmul_q8 arithmetic, src/core/k3_ops.c:1228-1301,
 * summed in double: within float rounding of the reference, which states no exactness
 * contract for the format); the bf16 prefill and batched decode paths refuse them. */
typedef struct k3hip_kda_weights k3hip_kda_weights;
int k3hip_kda_upload(const K3KdaW *w, const K3Cfg *c, k3hip_kda_weights **out);
int k3hip_kda_release(k3hip_kda_weights *w);

/* What an upload copies. DEV is always made: the matrices in their own storage and the fp32
 * vectors, all that k3hip_kda_layer_dev reads. PREFILL adds the derived copies of the bf16
 * prefill path (k3hip_kda_layer_prefill), DECODE the MFMA fragment-ordered copies of the
 * batched decode path (k3hip_kda_layer_decode); those entry points return K3HIP_EINVAL on
 * weights uploaded without their part. k3hip_kda_upload makes every part. The drop-in
 * k3_kda_layer uploads DEV only, per call (the reference binds weights per call too). */
enum { K3HIP_UPLOAD_DEV = 1, K3HIP_UPLOAD_PREFILL = 2, K3HIP_UPLOAD_DECODE = 4, K3HIP_UPLOAD_ALL = 7 };
int k3hip_kda_upload_ex(const K3KdaW *w, const K3Cfg *c, int parts, k3hip_kda_weights **out);
/* Device bytes an uploaded weight set holds. */
size_t k3hip_kda_weights_bytes(const k3hip_kda_weights *w);
/* Bytes the calling thread's last k3_kda_layer call copied between host and device (its
 * weight upload, x, out and state): the drop-in's transfer cost per call. */
size_t k3hip_kda_dropin_bytes(void);

/* The whole k3_kda_layer on device pointers: projections, K1, K2 (T>1) or K3 (T==1),
 * K4, o_proj. x,out [T][hidden] fp32; state as in k3_kda_layer (device, nullable). */
int k3hip_kda_layer_dev(const k3hip_kda_weights *w, int T, float *out, const float *x,
                        float *state, void *stream);

/* The whole k3_kda_layer for a T-token prefill on bf16 weights (K3_WBF16) and bf16
 * activations: the projections (src/core/k3_ops.c:879-886, :946, :948) as bf16 MFMA GEMMs
 * with fp32 accumulation (hipBLASLt) and fp32 results; f_a enters the f_b GEMM as a bf16
 * hi/lo pair against [W_fb | W_fb], and the epilogue output y (RMS-normalised) enters o_proj
 * in fp16 against an fp16 copy of W_o, so q, k, v and z are never rounded to bf16 (a single
 * bf16 rounding of q, k, v or y alone costs several times the 2e-3 prefill bar). Then K1,
 * K2 (chunked), K4 and o_proj.
 *   x [T][hidden] (x_dtype: fp32 inputs are rounded to bf16 first); out [T][hidden]
 *   (out_dtype); state as in k3_kda_layer (device, nullable).
 * Needs D = 64 / 128, conv_k <= 4 and -80/15 <= gate_lb < 0; otherwise
 * K3HIP_EUNSUPPORTED (k3hip_kda_layer_dev covers every shape in fp32). */
int k3hip_kda_layer_prefill(const k3hip_kda_weights *w, int T, void *out, int out_dtype,
                            const void *x, int x_dtype, float *state, void *stream);

/* Which projection GEMMs k3hip_kda_layer_prefill runs, process-wide: K3HIP_GEMM_HIPBLASLT
 * (the default; hipBLASLt's heuristic first choice for each shape) or K3HIP_GEMM_HANDWRITTEN
 * (k3hip_proj_gemm's kernel for every projection, the gate logits in fp16, f_a/b split over
 * K). Both hold the same 2e-3 bar but give different bits; change it only while no layer
 * prefill is in flight. K3HIP_EINVAL for another value. The hand-written kernel needs
 * hidden % 64 == 0 and, for bf16 x, a 16-byte aligned x: a layer outside that runs its
 * projections on hipBLASLt whatever the setting. No counterpart in the reference,
 * whose projections are one CPU routine (k3_matmul_bf16, src/core/k3_ops.c:1122-1227). */
enum { K3HIP_GEMM_HIPBLASLT = 0, K3HIP_GEMM_HANDWRITTEN = 1 };
int k3hip_set_projection_gemm(int impl);

/* One decode token for each of B sequences through the whole layer on bf16 weights: the
 * per-token path of k3_kda_layer (src/core/k3_ops.c:864-951, T = 1) batched over
 * sequences. The projections read each weight once for all B (bf16 MFMA, each fp32 input
 * element split into bf16 hi + lo in registers); needs hidden % 8 == 0 and x 16-byte
 * aligned. Sequence b's state (S then conv history, the reference layout)
 * starts at states + b * state_stride floats (>= H*D*D + 3*P*(conv_k-1), a multiple of 4).
 * x, out [B][hidden] fp32. When o_proj runs as two K-ranges and `out` is ordinary
 * (coarse-grained) device memory, both ranges are added into `out` by float atomics; on
 * pinned-host, managed or fine-grained memory the ranges are summed by a reduction launch
 * instead (the same bits unless a partial is denormal). */
int k3hip_kda_layer_decode(const k3hip_kda_weights *w, int B, float *out, const float *x,
                           float *states, long state_stride, void *stream);

/* k3hip_kda_layer_decode that allocates nothing: for callers that cannot call hipMalloc
 * (code under HIP graph capture, tight serving loops, harnesses that forbid allocation). No
 * counterpart in the reference. Same arguments, results bit-identical to
 * k3hip_kda_layer_decode. Its scratch (projections, split-K partial planes, y) is a
 * fixed 16 MiB device array inside this library, one per GPU, held until the process ends;
 * a call whose B and layer width need more returns K3HIP_EINVAL (at hidden 7168 with 32 x 128
 * heads: more than 99 sequences), as does any step that would need scratch beyond it (the
 * call allocates nothing, ever). Every call on one GPU uses that GPU's array: calls that
 * overlap on one GPU (other streams, other threads) race; serialise them. */
int k3hip_kda_layer_decode_noalloc(const k3hip_kda_weights *w, int B, float *out, const float *x,
                                   float *states, long state_stride, void *stream);

/* Device-resident state for a decode loop: the reference's kstate[L * kper] array
 * (src/cli/k3_run.c:514-567), kper = H*D*D + 3*P*(conv_k-1) floats per layer
 * (k3_state_geom, src/cli/k3_state.c:23-29), in the same layout on the device. */
typedef struct k3hip_kda_states k3hip_kda_states;
size_t k3hip_kda_state_floats(const K3Cfg *c);                       /* kper; 0 on bad cfg */
int k3hip_kda_states_create(const K3Cfg *c, int n_layers, k3hip_kda_states **out);  /* zeroed */
int k3hip_kda_states_release(k3hip_kda_states *s);
/* Device pointer of layer L's slot: the `state` argument of k3hip_kda_layer_dev /
 * k3hip_kda_layer_prefill. NULL when L is out of range. */
float *k3hip_kda_states_layer(const k3hip_kda_states *s, int layer);
int k3hip_kda_states_zero(k3hip_kda_states *s, void *stream);
/* Spec-decode snapshot / restore (the memcpy of kstate at src/cli/k3_run.c:1969-1984) as a
 * device-to-device copy between two pools of the same geometry. */
int k3hip_kda_states_copy(k3hip_kda_states *dst, const k3hip_kda_states *src, void *stream);
/* Whole array to / from host memory in the reference layout (the payload k3_state_save
 * writes and k3_state_load fills); both synchronize `stream`. */
int k3hip_kda_states_download(const k3hip_kda_states *s, float *host, void *stream);
int k3hip_kda_states_upload(k3hip_kda_states *s, const float *host, void *stream);

/* Gated MLA (NoPE) decode with absorbed kv_b, for the hybrid KDA + MLA slice. Replaces the
 * cached path of k3_mla_cached (src/core/k3_ops.c:321-424) for single-token steps of B
 * sequences. The cache holds, per sequence and position, the rmsnorm'd compressed latent
 * (kv_lora floats) followed by the shared rope slot (qk_rope floats) -- not the reference's
 * expanded per-head keys and values (42x smaller); the attention is the same maths in
 * another order (W_UK absorbed into q, W_UV applied after the weighted sum).
 * bf16 weights (K3_WBF16) only. */
typedef struct k3hip_mla_weights k3hip_mla_weights;
int k3hip_mla_upload(const K3MlaW *w, const K3Cfg *c, k3hip_mla_weights **out);
int k3hip_mla_release(k3hip_mla_weights *w);
size_t k3hip_mla_cache_floats(const K3Cfg *c, int cap);   /* per sequence: cap*(kv_lora+rope) */
/* x, out [B][hidden] fp32; cache [B][cap][kv_lora+rope] fp32; every sequence holds `pos`
 * cached positions: the step writes position pos and attends over 0..pos (pos < cap). */
int k3hip_mla_decode(const k3hip_mla_weights *w, int B, int pos, int cap, float *cache,
                     const float *x, float *out, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* K3KDA_H */
