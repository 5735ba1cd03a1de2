// SPDX-License-Identifier: Apache-2.0
// kda_chunk.hip - K2: chunked gated delta-rule prefill (gfx950). Placeholder entry points.
#include "kda_internal.h"

namespace k3kda {
bool chunk_ready() { return false; }
}  // namespace k3kda

using namespace k3kda;

extern "C" size_t k3hip_kda_chunk_workspace(int T, int H, int D, int chunk)
{
    (void)T; (void)H; (void)D; (void)chunk;
    return 0;
}

extern "C" int k3hip_kda_chunk(int T, int H, int D, int chunk, const float *q, const float *k,
                               const float *v, const float *g, const float *beta, float q_scale,
                               float *S, float *o, void *workspace, size_t workspace_bytes,
                               void *stream)
{
    clear_error();
    (void)T; (void)H; (void)D; (void)chunk; (void)q; (void)k; (void)v; (void)g; (void)beta;
    (void)q_scale; (void)S; (void)o; (void)workspace; (void)workspace_bytes; (void)stream;
    K3_FAIL(K3HIP_EUNSUPPORTED, "k3hip_kda_chunk: not built");
}
