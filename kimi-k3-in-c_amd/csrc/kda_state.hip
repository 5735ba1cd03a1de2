// SPDX-License-Identifier: Apache-2.0
// kda_state.hip - device-resident KDA state for a decode loop.
//
// The reference keeps one state slot per KDA layer in a host array kstate[L * kper]
// (src/cli/k3_run.c:514-567), kper = H*D*D recurrent floats followed by 3*P*(conv_k-1)
// ShortConv history floats (k3_state_geom, src/cli/k3_state.c:23-29). Incremental decode
// carries it across steps; speculative decode snapshots it with a memcpy before a draft
// sweep and copies it back when a draft is rejected (src/cli/k3_run.c:1969-1984); the
// state file (k3_state_save / k3_state_load) stores that same array.
//
// Here the array lives in device memory with the identical layout, so
//   - k3hip_kda_states_layer(s, L) is the `state` pointer of layer L for
//     k3hip_kda_layer_dev / k3hip_kda_layer_prefill (and the decode path inside them);
//   - snapshot / restore are device-to-device copies between two pools;
//   - download / upload move the whole array in the reference layout, so the host side
//     can hand it to k3_state_save or fill it from k3_state_load unchanged.
// All transfers are stream-ordered; the zero fill is a kernel (no memset node).
#include "kda_internal.h"

struct k3hip_kda_states {
    int layers;
    size_t kper;   // floats per layer
    float *d;      // [layers][kper]
};

using namespace k3kda;

extern "C" size_t k3hip_kda_state_floats(const K3Cfg *c)
{
    if (!c || c->kda_heads <= 0 || c->kda_head_dim <= 0 || c->conv_k <= 0) return 0;
    const size_t P = (size_t)c->kda_heads * c->kda_head_dim;
    return P * (size_t)c->kda_head_dim + 3 * P * (size_t)(c->conv_k - 1);
}

extern "C" int k3hip_kda_states_create(const K3Cfg *c, int n_layers, k3hip_kda_states **out)
{
    clear_error();
    if (!c || !out || n_layers <= 0) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_states_create: bad argument");
    *out = nullptr;
    const size_t kper = k3hip_kda_state_floats(c);
    if (!kper) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_states_create: H=%d D=%d conv_k=%d", c->kda_heads,
                       c->kda_head_dim, c->conv_k);
    k3hip_kda_states *s = (k3hip_kda_states *)calloc(1, sizeof *s);
    if (!s) K3_FAIL(K3HIP_ENOMEM, "k3hip_kda_states_create: host allocation");
    s->layers = n_layers;
    s->kper = kper;
    const size_t bytes = kper * (size_t)n_layers * sizeof(float);
    if (hipMalloc((void **)&s->d, bytes) != hipSuccess) {
        (void)hipGetLastError();
        free(s);
        K3_FAIL(K3HIP_ENOMEM, "k3hip_kda_states_create: hipMalloc(%zu bytes)", bytes);
    }
    int rc = zero_fill(s->d, kper * (size_t)n_layers, nullptr);
    if (rc == K3HIP_OK && hipStreamSynchronize(nullptr) != hipSuccess) rc = K3HIP_EHIP;
    if (rc) {
        (void)hipFree(s->d);
        free(s);
        return rc;
    }
    *out = s;
    return K3HIP_OK;
}

extern "C" int k3hip_kda_states_release(k3hip_kda_states *s)
{
    clear_error();
    if (!s) return K3HIP_OK;
    if (s->d) (void)hipFree(s->d);
    free(s);
    return K3HIP_OK;
}

extern "C" float *k3hip_kda_states_layer(const k3hip_kda_states *s, int layer)
{
    if (!s || layer < 0 || layer >= s->layers) return nullptr;
    return s->d + s->kper * (size_t)layer;
}

extern "C" int k3hip_kda_states_zero(k3hip_kda_states *s, void *stream)
{
    clear_error();
    if (!s) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_states_zero: NULL pool");
    return zero_fill(s->d, s->kper * (size_t)s->layers, as_stream(stream));
}

extern "C" int k3hip_kda_states_copy(k3hip_kda_states *dst, const k3hip_kda_states *src, void *stream)
{
    clear_error();
    if (!dst || !src) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_states_copy: NULL pool");
    if (dst->layers != src->layers || dst->kper != src->kper)
        K3_FAIL(K3HIP_EINVAL, "k3hip_kda_states_copy: geometry %d x %zu vs %d x %zu", dst->layers,
                dst->kper, src->layers, src->kper);
    if (dst == src) return K3HIP_OK;
    K3_HIP(hipMemcpyAsync(dst->d, src->d, src->kper * (size_t)src->layers * sizeof(float),
                          hipMemcpyDeviceToDevice, as_stream(stream)));
    return K3HIP_OK;
}

extern "C" int k3hip_kda_states_download(const k3hip_kda_states *s, float *host, void *stream)
{
    clear_error();
    if (!s || !host) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_states_download: NULL argument");
    hipStream_t st = as_stream(stream);
    K3_HIP(hipMemcpyAsync(host, s->d, s->kper * (size_t)s->layers * sizeof(float),
                          hipMemcpyDeviceToHost, st));
    K3_HIP(hipStreamSynchronize(st));
    return K3HIP_OK;
}

extern "C" int k3hip_kda_states_upload(k3hip_kda_states *s, const float *host, void *stream)
{
    clear_error();
    if (!s || !host) K3_FAIL(K3HIP_EINVAL, "k3hip_kda_states_upload: NULL argument");
    hipStream_t st = as_stream(stream);
    K3_HIP(hipMemcpyAsync(s->d, host, s->kper * (size_t)s->layers * sizeof(float),
                          hipMemcpyHostToDevice, st));
    K3_HIP(hipStreamSynchronize(st));
    return K3HIP_OK;
}
