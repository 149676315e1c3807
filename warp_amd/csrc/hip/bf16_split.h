// SPDX-License-Identifier: Apache-2.0
//
// bf16_split.h — fp32 values on the bf16 matrix cores without rounding.
//
// An fp32 value has a 24-bit significand; three bf16 values of 8 bits each
// hold it exactly: hi = v with its low 16 bits cleared, mid the same of
// v - hi, lo = v - hi - mid (at most 8 significant bits left, so exactly a
// bf16).  Each subtraction is exact (it removes leading bits of the same
// binade), so hi + mid + lo == v.  Products of bf16 pieces are exact in
// fp32, and v_mfma_f32_32x32x16_bf16 accumulates them in fp32: a dot
// product through the pieces rounds only where an fp32 dot product would.
#pragma once
#include "common.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

WH_INLINE bf16x8 as_b8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }

// bf16 pieces of 8 floats, packed two to a word in element order
WH_INLINE void split3(const float *f, uint4 &p0, uint4 &p1, uint4 &p2)
{
    uint32_t w0[4], w1[4], w2[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t a[2], b[2], c[2];
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const float v = f[2 * i + j];
            const uint32_t hi = __float_as_uint(v) & 0xffff0000u;
            const float r1 = __fsub_rn(v, __uint_as_float(hi));
            const uint32_t mid = __float_as_uint(r1) & 0xffff0000u;
            const float r2 = __fsub_rn(r1, __uint_as_float(mid));
            a[j] = hi >> 16;
            b[j] = mid >> 16;
            c[j] = __float_as_uint(r2) >> 16;
        }
        w0[i] = a[0] | (a[1] << 16);
        w1[i] = b[0] | (b[1] << 16);
        w2[i] = c[0] | (c[1] << 16);
    }
    p0 = make_uint4(w0[0], w0[1], w0[2], w0[3]);
    p1 = make_uint4(w1[0], w1[1], w1[2], w1[3]);
    p2 = make_uint4(w2[0], w2[1], w2[2], w2[3]);
}
