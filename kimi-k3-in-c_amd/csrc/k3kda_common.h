// SPDX-License-Identifier: Apache-2.0
// k3kda_common.h - shared helpers for the gfx950 KDA kernels and their C-ABI shims.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "k3kda.h"

namespace k3kda {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- errors ----
// Per-thread message behind k3hip_last_error(); set by fail() and by the HIP check.
void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

#define K3_FAIL(code, ...)            \
    do {                              \
        ::k3kda::set_error(__VA_ARGS__); \
        return (code);                \
    } while (0)

#define K3_HIP(call)                                                              \
    do {                                                                          \
        hipError_t e_ = (call);                                                   \
        if (e_ != hipSuccess)                                                     \
            K3_FAIL(K3HIP_EHIP, "%s: %s (%s:%d)", #call, hipGetErrorString(e_),   \
                    __FILE__, __LINE__);                                          \
    } while (0)

// After a launch: a bad configuration is reported by hipGetLastError.
#define K3_LAUNCHED() K3_HIP(hipGetLastError())

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// ------------------------------------------------------------------ bf16 ----
// bf16 is the top half of an fp32: widening is a 16-bit shift (exact).
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// Round to nearest even; NaN stays NaN.
__device__ __forceinline__ uint16_t f2bf(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Load element i of an activation that is fp32 (dtype 0) or bf16 (dtype 1).
template <int DT>
__device__ __forceinline__ float load_act(const void *p, size_t i)
{
    if constexpr (DT == K3HIP_BF16) return bf2f(reinterpret_cast<const uint16_t *>(p)[i]);
    else return reinterpret_cast<const float *>(p)[i];
}

// 1 / (1 + expf(-x)), the reference's sigmoid (src/core/k3_ops.c:105).
__device__ __forceinline__ float sigmoid_ref(float x) { return 1.0f / (1.0f + expf(-x)); }

// log(1 + e^x), taken as x above 20 where the two agree in fp32.
__device__ __forceinline__ float softplus_ref(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

inline bool is_pow2_head(int D) { return D == 16 || D == 32 || D == 64 || D == 128; }

// True when p is ordinary (coarse-grained) device memory, where the hardware float atomics
// are exact: hipMalloc, hipMallocAsync and torch's allocator. Host-pinned, managed and
// fine-grained allocations (hipHostMalloc, hipMallocManaged, hipExtMallocWithFlags with a
// fine-grained or uncached flag), and pointers HIP does not know, give false.
inline bool coarse_device_mem(const void *p)
{
    hipPointerAttribute_t a{};
    if (hipPointerGetAttributes(&a, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return a.type == hipMemoryTypeDevice && !a.isManaged && (a.allocationFlags & hipDeviceMallocFinegrained) == 0;
}

}  // namespace k3kda
