// SPDX-License-Identifier: Apache-2.0
// kda_internal.h - library-internal entry points shared between translation units.
#pragma once

#include "k3kda_common.h"

namespace k3kda {

// y[T][out] = W[out][in] . x[T][in] with double accumulation; wdt = K3_WF32 | K3_WBF16.
int proj(int T, int in, int out, const float *x, const void *W, int wdt, float *y, hipStream_t st);

// Row-major C[M][N] = A[M][K] . op(B) with fp32 accumulation (hipBLASLt): op(B) = B^T for
// B [N][K] (b_trans) or B for B [K][N]; A and B both bf16 or both fp32; C bf16 or fp32;
// leading dimensions in elements; `batch` strided problems (strides in elements).
// fp16 operands/results, internal only (the public dtypes are K3HIP_F32 and K3HIP_BF16)
constexpr int K3_DT_F16 = K3HIP_F16;

struct GemmDesc {
    int M = 0, N = 0, K = 0;
    int ab_dtype = K3HIP_BF16, c_dtype = K3HIP_F32;
    bool b_trans = true;
    long lda = 0, ldb = 0, ldc = 0;
    int batch = 1;
    long sa = 0, sb = 0, sc = 0;
    bool cache = true;  // keep the plan for later calls of the shape (false: a shape seen once)
};
int gemm(const GemmDesc &g, const void *A, const void *B, void *C, hipStream_t st);

// C[M][N] = A[M][K] . W[N][K]^T on bf16 MFMA, A, W bf16 row-major, C bf16 or fp32.
int gemm_bf16(int M, int N, int K, const void *A, const void *W, void *C, int c_dtype, hipStream_t st);
// The same on fp16 MFMA (A, W fp16 row-major), fp32 accumulation.
int gemm_f16(int M, int N, int K, const void *A, const void *W, void *C, int c_dtype, hipStream_t st);

// Hand-written MFMA GEMM (kda_mm.hip): C[M][N] = A[M][K] . B[N][K]^T, A and B both bf16
// (ab = K3HIP_BF16) or both fp16 (K3_DT_F16), K-contiguous rows (lda, ldb in elements), fp32
// accumulation; C fp32, fp16 or bf16 (out), row stride ldc. With gcols > 0, output columns
// [g*gcols, (g+1)*gcols) are written to the matrix at C + g*gstride elements (one launch
// filling several row-major outputs). Needs K % 64 == 0, lda and ldb multiples of 8 and
// 16-byte aligned A and B (mm_supported); returns K3HIP_EUNSUPPORTED otherwise.
bool mm_supported(int K, long lda, long ldb);
int mm(int M, int N, int K, int ab, const void *A, long lda, const void *B, long ldb, void *C, int out, long ldc,
       hipStream_t st, int gcols = 0, long gstride = 0);
// The same product as `splits` fp32 K-range partial planes P[s][M][N] (ld N), s increasing
// with K; their sum in increasing s is the product, bit for bit on every run.
// mm_splits(M, N, K, CUs) picks a split count that fills the GPU for narrow shapes.
int mm_splits(int M, int N, int K, int ncu);
int mm_splitk(int M, int N, int K, int splits, int ab, const void *A, long lda, const void *B, long ldb, float *P,
              hipStream_t st);

// K4 with y written as a bf16 hi/lo pair into y2 [T][2P] (hi columns 0..P-1, lo P..2P-1),
// for an o_proj GEMM with K = 2P against [W_o | W_o]. D = 64 / 128, 16-byte aligned.
// y as fp16 [T][P] (y_f16 true) or as a bf16 hi/lo pair [T][2P] (hi in the first P columns)
int epilogue_split(int T, int H, int D, float eps, const float *o, const void *gate, int gate_dtype,
                   const float *o_norm, void *y2, hipStream_t st, bool y_f16 = false);

// x [B][N] fp32 -> y [2B][N] bf16: rows 0..B-1 = hi, rows B..2B-1 = lo = bf16(x - hi), the
// input of a GEMM that reads each weight once for both halves.
int split_rows2(const float *x, uint16_t *y, int B, int N, hipStream_t st);
// y[b][n] = C2[b][n] + C2[B+b][n] (the two halves of such a GEMM).
int pair_add(const float *C2, float *y, int B, int N, hipStream_t st);

// K3 over B sequences whose [H][D][D] states start s_stride floats apart (decode slots).
int decode_strided(int B, int H, int D, float *S, long s_stride, float *o, const float *q,
                   const float *k, const float *v, const float *alpha, const float *beta,
                   float qs, hipStream_t st);

// Stream-ordered scratch: hipMallocAsync on `st`, freed with hipFreeAsync on the same stream.
struct StreamBuf {
    void *p = nullptr;
    hipStream_t st = nullptr;
    ~StreamBuf()
    {
        if (p) (void)hipFreeAsync(p, st);
    }
};
int stream_alloc(StreamBuf &b, size_t bytes, hipStream_t st);

// Decode copy of a row-major bf16 weight W[N][K] in MFMA fragment order, for gemm_rows:
// rows_frag_elems(N, K) bf16 elements (N rounded up to 16, K to 32, zero padded). The copy
// is written by a kernel on `st` (W and Wf device pointers, 16-byte aligned, K % 8 == 0).
size_t rows_frag_elems(int N, int K);
int rows_frag_pack(const uint16_t *W, int N, int K, uint16_t *Wf, hipStream_t st);

// C[B][N] (row stride ldc) = x[B][K] (fp32, row stride ldx) . W[N][K]^T (bf16, given as its
// fragment-ordered copy Wf from rows_frag_pack), each x element split into bf16 hi + lo in
// registers so products keep fp32 accuracy; built for few rows (decode batches), bound by
// reading W once. K % 8 == 0, ldx % 4 == 0, x and Wf 16-byte aligned. Stream-ordered.
// Split-K partials go to ws (16-byte aligned, at least gemm_rows_ws_floats(B, N, K) floats);
// with ws == nullptr or too small they are allocated on `st` for the call. c_zeroed: C
// already holds zeros; with exactly two K-ranges they are then added into C by atomics
// instead of a workspace and a second launch. Reproducible: a two-term sum does not depend
// on which range lands first (and equals the reduction kernel's a + b unless a partial is
// denormal, which the atomic unit may flush).
size_t gemm_rows_ws_floats(int B, int N, int K);
int gemm_rows(int B, int N, int K, const float *x, long ldx, const uint16_t *Wf, float *C, long ldc,
              hipStream_t st, float *ws = nullptr, size_t ws_floats = 0, bool c_zeroed = false);
// gemm_rows with C also written as bf16 hi (rows 0 .. B-1) and lo (rows B .. 2B-1) rows of
// hl (row stride ldhl; hi = bf16(c), lo = bf16(c - hi), the bits of split_rows2 on C), in the
// same launch when the product runs unsplit (otherwise split_rows2 after it, ldc = ldhl = N).
// xw != nullptr (unsplit products only, gemm_rows_splits(N, K) == 1): the x rows are
// RMS-normalised with weight xw and eps xeps on the way in (the rmsnorm of k3_ops.c:94-102).
int gemm_rows_hl(int B, int N, int K, const float *x, long ldx, const uint16_t *Wf, float *C, long ldc,
                 uint16_t *hl, long ldhl, hipStream_t st, float *ws = nullptr, size_t ws_floats = 0,
                 const float *xw = nullptr, float xeps = 0.0f);
// gemm_rows on S = gemm_rows_plane_count(N, K) K-ranges, the count that spreads the
// workgroups most evenly over the CUs when N has fewer column blocks than there are CUs (1:
// unsplit), summed in range order into C by a second launch; ws holds S B N floats.
int gemm_rows_plane_count(int N, int K);
int gemm_rows_even(int B, int N, int K, const float *x, long ldx, const uint16_t *Wf, float *C, long ldc,
                   hipStream_t st, float *ws, size_t ws_floats);
// The same product left as its S = gemm_rows_splits(N, K) K-range partials: planes
// P[s][B][N], whose sum in increasing s is C bit for bit, for a consumer that adds them
// itself instead of a reduction launch.
int gemm_rows_splits(int N, int K);
int gemm_rows_part(int B, int N, int K, const float *x, long ldx, const uint16_t *Wf, float *P, hipStream_t st);
// gemm_rows of W1 (N1 columns into C1, row stride ldc1) and gemm_rows_part of W2 (N2 columns,
// planes P2) over the same x in one launch when W1 runs unsplit: the two weights' workgroups
// fill the GPU together and x is read by both in the same pass. The same bits as the two
// calls; when W1 would split K, it is those two calls.
int gemm_rows_with_part(int B, int K, const float *x, long ldx, int N1, const uint16_t *Wf1, float *C1, long ldc1,
                        int N2, const uint16_t *Wf2, float *P2, hipStream_t st, float *ws = nullptr,
                        size_t ws_floats = 0);

// Attention of an absorbed MLA decode step (kda_mla_attn.hip) in one pass over the cache:
// the query rows qcat[b][h] = [A2[b][h] + A2[B+b][h] | q_rope(b, h)] are formed in the kernel
// from the absorb GEMM's hi/lo halves A2 [2B][H CW] (first KL of each head's CW columns) and
// q [B][H][QN + CW - KL] (rope at column QN); cache [B][cap][CW] fp32 (latent = channels
// 0..KL-1), positions 0..Tn-1; chat = softmax(scale qcat . cache^T) . latent (its position
// ranges merged into the bf16 hi / lo rows of ch2 [2B][H KL], 16-byte aligned), then
// o [B][H VH] = (chat_h . W_UV_h^T) * sigmoid(g) with W_UV_h the rows
// h (QN + VH) + QN .. + VH of kvb [H (QN + VH)][KL] (bf16) and g (may be nullptr) the gate
// logits at row stride ldg; zout[0 .. zn) = 0 on the way (may be nullptr). Shapes:
// mla_attention_supported (H <= 64, KL a multiple of 16 up to 512, CW a multiple of 4 up to
// 576), QN % 4 == 0, KL % 8 == 0, VH <= 128. ws: mla_attention_ws_bytes bytes, 256-byte aligned; A2, q,
// cache and kvb 16-byte aligned.
bool mla_attention_supported(int H, int KL, int CW);
size_t mla_attention_ws_bytes(int B, int H, int KL, int Tn);
// lat != nullptr: position Tn - 1's cache row is written first from row b of lat (stride
// ldlat): the first KL floats rmsnorm'd with weight lat_w and eps lat_eps, the rope slot
// copied (the norm launch before the attention otherwise writes it).
int mla_attention(int B, int H, int KL, int CW, int Tn, int cap, float scale, const float *A2, const float *q,
                  int QN, float *cache, const float *lat, long ldlat, const float *lat_w, float lat_eps,
                  const uint16_t *kvb, int VH, const float *g, long ldg, float *o, float *zout, size_t zn,
                  uint16_t *ch2, void *ws, size_t ws_bytes, hipStream_t st);

// One decode token of a KDA layer between its projections (kda_step.hip): K1 + K3 + K4 per
// (head, sequence). Cin rows (stride ldc) hold q | k | v at columns 0, P, 2P and the beta
// logits at bcol, f_a (D wide) at facol; Wfb the f_b weight [P][D] in the decode GEMV's
// fragment order (rows_frag_pack), from which the kernel forms the decay logits z = f_a W_fb^T;
// gl the output-gate logits as
// gsplit planes of gplane floats. states: per sequence (stride floats apart) the H D x D
// state, then the [3][P][conv_k-1] conv history; both updated in place. y [B][P] out.
// zout (may be nullptr): zn floats the kernel sets to zero on the way.
int layer_step(int B, int H, int D, int K, float lb, float eps, float q_scale, const float *Cin,
               long ldc, int bcol, int facol, const uint16_t *Wfb, const float *gl, int gsplit, long gplane,
               const float *q_conv, const float *k_conv, const float *v_conv, const float *A_log,
               const float *dt_bias, const float *o_norm, float *states, long stride, float *y,
               float *zout, long zn, hipStream_t st);

// p[0..n) = 0 on `st` with a kernel (never a memset node).
int zero_fill(float *p, size_t n, hipStream_t st);

// Outgoing short-conv history (3 tensors x P channels x K-1 slots) after T new inputs of
// dtype dt, launched after every reader of the incoming history on `st`.
int conv_state_update(int T, int P, int K, int dt, const void *qi, const void *ki, const void *vi,
                      float *cs, hipStream_t st);

// Compute units of the current device (cached per device).
int cu_count(int &ncu);

// True once the chunked prefill kernel is built into this library.
bool chunk_ready();

}  // namespace k3kda
