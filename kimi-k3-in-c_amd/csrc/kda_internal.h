// SPDX-License-Identifier: Apache-2.0
// kda_internal.h - library-internal entry points shared between translation units.
#pragma once

#include "k3kda_common.h"

namespace k3kda {

// y[T][out] = W[out][in] . x[T][in] with double accumulation; wdt = K3_WF32 | K3_WBF16.
int proj(int T, int in, int out, const float *x, const void *W, int wdt, float *y, hipStream_t st);

// C[M][N] = A[M][K] . W[N][K]^T on bf16 MFMA (hipBLASLt), fp32 accumulation; A, W bf16
// row-major; C bf16 or fp32 (c_dtype) row-major.
int gemm_bf16(int M, int N, int K, const void *A, const void *W, void *C, int c_dtype, hipStream_t st);

// K4 with y written as a bf16 hi/lo pair into y2 [T][2P] (hi columns 0..P-1, lo P..2P-1),
// for an o_proj GEMM with K = 2P against [W_o | W_o]. D = 64 / 128, 16-byte aligned.
int epilogue_split(int T, int H, int D, float eps, const float *o, const void *gate, int gate_dtype,
                   const float *o_norm, void *y2, hipStream_t st);

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

// p[0..n) = 0 on `st` with a kernel (never a memset node).
int zero_fill(float *p, size_t n, hipStream_t st);

// Outgoing short-conv history (3 tensors x P channels x K-1 slots) after T new inputs of
// dtype dt, launched after every reader of the incoming history on `st`.
int conv_state_update(int T, int P, int K, int dt, const void *qi, const void *ki, const void *vi,
                      float *cs, hipStream_t st);

// True once the chunked prefill kernel is built into this library.
bool chunk_ready();

}  // namespace k3kda
