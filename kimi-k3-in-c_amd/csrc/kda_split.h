// SPDX-License-Identifier: Apache-2.0
// kda_split.h - fp32 -> bf16 hi + lo splitting of an 8-element activation slice, shared by
// the decode GEMV (kda_rows.hip) and the decode step's f_b product (kda_step.hip), so both
// give a product the same bits.
#pragma once

#include "k3kda_common.h"

namespace k3kda {
namespace bsplit {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// x = hi + lo, both bf16 (round to nearest even; lo carries the rounding error of hi)
__device__ __forceinline__ void split_row8(const f4 &a, const f4 &b, bf16x8 &hi, bf16x8 &lo)
{
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        const bf16x2 h = __builtin_convertvector(f2{v[e], v[e + 1]}, bf16x2);
        const uint32_t u = __builtin_bit_cast(uint32_t, h);
        const float h0 = __uint_as_float(u << 16), h1 = __uint_as_float(u & 0xffff0000u);
        const bf16x2 l = __builtin_convertvector(f2{v[e] - h0, v[e + 1] - h1}, bf16x2);
        hi[e] = h[0]; hi[e + 1] = h[1];
        lo[e] = l[0]; lo[e + 1] = l[1];
    }
}

}  // namespace bsplit
}  // namespace k3kda
