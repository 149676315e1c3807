// SPDX-License-Identifier: Apache-2.0
//
// gemv_dev.h — device pieces of the batch-1 trunk products (F32, Q8G, Q4G
// rows against fp32 or bf16 x), shared by the GEMV kernels and the
// one-launch decode.
#pragma once
#include "common.h"

// elements per 16-byte chunk of a row
template <int FMT> struct chunk_of;
template <> struct chunk_of<0> { static constexpr int NE = 4; };
template <> struct chunk_of<2> { static constexpr int NE = 16; };
template <> struct chunk_of<3> { static constexpr int NE = 32; };

// ---- one token --------------------------------------------------------------
// The decode products are latency-bound unless every load a lane needs is in
// flight at once.  A lane issues its weight chunks (and their group scales)
// and the matching slices of x together, then computes: one memory round
// trip per batch of U chunks.  A wavefront owns RPW rows (RPW = 4 when a row
// is at most one chunk per lane, so x is read once for four rows).

// chunks per lane per batch (about 124 VGPRs: four workgroups per CU); fp32
// x slices are twice the registers of bf16
template <int FMT, bool XBF> struct u_of { static constexpr int U = (FMT == 0 ? 8 : 2) / (XBF ? 1 : 2) > 0 ? (FMT == 0 ? 8 : 2) / (XBF ? 1 : 2) : 1; };

// x slice of one chunk as raw 16-byte words: NE elements, bf16 or fp32
template <int FMT, bool XBF> struct xw_of {
    static constexpr int N = (chunk_of<FMT>::NE * (XBF ? 2 : 4) + 15) / 16;
};

// Loads take a clamped, always valid address and no branch: a load behind a
// divergent branch, or a value converted right after its load, makes the
// compiler wait for every load in flight before issuing the next.
template <int FMT, bool XBF>
__device__ __forceinline__ void load_xs(const void *x, int cols, int k, uint4 *xw)
{
    constexpr int NE = chunk_of<FMT>::NE, NW = xw_of<FMT, XBF>::N;
    const int e0 = k * NE;
    if (NE * (XBF ? 2 : 4) < 16) {                        // F32 weights, bf16 x: 8 bytes
        const uint2 v = *(const uint2 *)((const uint16_t *)x + (e0 < cols ? e0 : 0));
        xw[0] = make_uint4(v.x, v.y, 0, 0);
        return;
    }
#pragma unroll
    for (int i = 0; i < NW; i++) {
        const int e = e0 + i * (XBF ? 8 : 4);
        xw[i] = *(const uint4 *)((const uint8_t *)x + (size_t)(e < cols ? e : 0) * (XBF ? 2 : 4));
    }
}

// zero the x words past the last column (a padded row's tail multiplies 0)
template <int FMT, bool XBF>
__device__ __forceinline__ void mask_xs(int cols, int k, uint4 *xw)
{
    constexpr int NE = chunk_of<FMT>::NE, NW = xw_of<FMT, XBF>::N;
    const int e0 = k * NE;
    if (NE * (XBF ? 2 : 4) < 16) {
        if (e0 >= cols) xw[0] = make_uint4(0, 0, 0, 0);
        return;
    }
#pragma unroll
    for (int i = 0; i < NW; i++)
        if (e0 + i * (XBF ? 8 : 4) >= cols) xw[i] = make_uint4(0, 0, 0, 0);
}

template <int FMT, bool XBF>
__device__ __forceinline__ float chunk_dot(uint4 raw, const uint4 *xw)
{
    constexpr int NE = chunk_of<FMT>::NE;
    const uint32_t uw[4] = {raw.x, raw.y, raw.z, raw.w};
    float a = 0.0f;
#pragma unroll
    for (int q = 0; q < NE / 4; q++) {
        float x[4];
        if (XBF) {
            const uint4 v = xw[q >> 1];
            const uint32_t lo = (q & 1) ? v.z : v.x, hi = (q & 1) ? v.w : v.y;
            x[0] = wh_bf16(lo & 0xffff); x[1] = wh_bf16(lo >> 16);
            x[2] = wh_bf16(hi & 0xffff); x[3] = wh_bf16(hi >> 16);
        } else {
            const uint4 v = xw[q];
            x[0] = __uint_as_float(v.x); x[1] = __uint_as_float(v.y);
            x[2] = __uint_as_float(v.z); x[3] = __uint_as_float(v.w);
        }
        float w[4];
        if (FMT == 0) {
#pragma unroll
            for (int i = 0; i < 4; i++) w[i] = __uint_as_float(uw[i]);
        } else if (FMT == 2) {
#pragma unroll
            for (int i = 0; i < 4; i++) w[i] = (float)(int8_t)((uw[q] >> (i * 8)) & 0xff);
        } else {
#pragma unroll
            for (int i = 0; i < 4; i += 2) {
                const uint32_t b = (uw[q >> 1] >> (((q & 1) * 2 + (i >> 1)) * 8)) & 0xff;
                w[i] = (float)((int)(b & 15) - 8);
                w[i + 1] = (float)((int)(b >> 4) - 8);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) a = __fmaf_rn(w[i], x[i], a);
    }
    return a;
}

// Q4G chunk against bf16 x on the dot-product unit.  A byte of two nibbles
// (n_lo, n_hi) becomes the bf16 pair (128 + n_lo, 128 + n_hi): the code is
// the low mantissa bits under the exponent of 128, exact; one v_dot2 per
// pair multiplies it into the raw bf16 x pair with fp32 accumulation, and
// sum((128 + n) x) - 136 sum(x) = sum((n - 8) x).  sx136 = 136 * sum(x) of
// the chunk, shared by the matrices that read it.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float chunk_dot_q4bf(uint4 raw, const uint4 *xw, float sx136)
{
    const uint32_t uw[4] = {raw.x, raw.y, raw.z, raw.w};
    const uint32_t xd[16] = {xw[0].x, xw[0].y, xw[0].z, xw[0].w, xw[1].x, xw[1].y, xw[1].z, xw[1].w,
                             xw[2].x, xw[2].y, xw[2].z, xw[2].w, xw[3].x, xw[3].y, xw[3].z, xw[3].w};
    float a = 0.0f;
#pragma unroll
    for (int m = 0; m < 4; m++) {
        const uint32_t t = uw[m] & 0x0F0F0F0Fu, u = (uw[m] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            // [t.byte j, 0, u.byte j, 0] | 128.0 in both halves
            const uint32_t pr = __builtin_amdgcn_perm(u, t, 0x0C000C00u | ((4u + j) << 16) | (uint32_t)j) | 0x43004300u;
            a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pr),
                                               __builtin_bit_cast(bf16x2_t, xd[4 * m + j]), a, false);
        }
    }
    return a - sx136;
}

__device__ __forceinline__ float chunk_sum136_bf(const uint4 *xw)
{
    const uint32_t one2 = 0x3F803F80u;                 // (1.0, 1.0) in bf16
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t w4[4] = {xw[i].x, xw[i].y, xw[i].z, xw[i].w};
#pragma unroll
        for (int k = 0; k < 4; k++)
            s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w4[k]),
                                               __builtin_bit_cast(bf16x2_t, one2), s, false);
    }
    return 136.0f * s;
}
