// SPDX-License-Identifier: Apache-2.0
//
// gemv_dev.h — device pieces of the batch-1 trunk products (F32, Q8G, Q4G
// rows against fp32 or bf16 x), shared by the GEMV kernels and the
// one-launch decode.
#pragma once
#include "common.h"
#include "launch.h"

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

// The shared expert's down projection, eight rows r0 .. r0+7 per
// wavefront: each lane a 16-byte chunk of every row per step against the
// matching slice of x (fp32), then eight wave sums.  Used by the combine
// (rows of its block) and by the gate/up launches' spare workgroups.
template <int FMT>
__device__ __forceinline__ void sh_rows8_acc(const whip_mat &W, const float *x, int r0, int H, int lane,
                                             float (&acc)[8])
{
    constexpr int NE = chunk_of<FMT>::NE, NW = xw_of<FMT, false>::N;
    const int ng = FMT == 0 ? 1 : (W.cols + W.group - 1) / W.group;
    const int C = (FMT == 0 ? W.cols : ng * W.group) / NE;
    const uint8_t *Wq = (const uint8_t *)W.q;
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = 0.0f;
    for (int k0 = 0; k0 < C; k0 += 64) {            // uniform
        const int k = k0 + lane, kc = k < C ? k : 0;
        uint4 xw[NW], wv[8];
        uint16_t sv[8];
        load_xs<FMT, false>(x, W.cols, kc, xw);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int r = min(r0 + i, H - 1);
            wv[i] = *(const uint4 *)(Wq + (size_t)r * W.rowbytes + (size_t)kc * 16);
            if (FMT != 0) sv[i] = W.qs[(size_t)r * ng + (size_t)kc * NE / W.group];
        }
        if (k < C) {
            mask_xs<FMT, false>(W.cols, k, xw);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float d = chunk_dot<FMT, false>(wv[i], xw);
                acc[i] = FMT == 0 ? acc[i] + d : __fmaf_rn(wh_f16_scale(sv[i]), d, acc[i]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = wave_sum(acc[i]);
}

// A launch's spare workgroups computing y = W . x (the shared expert's down
// projection, fp32 x): rows in groups of eight, one group per wavefront at
// a time; workgroup g of NG, `waves` wavefronts each.
template <int FMT>
__device__ __forceinline__ void shd_rows_role(const whip_mat &W, const float *x, float *y, int g, int NG, int waves)
{
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int H = W.rows, ngr = (H + 7) / 8;
    for (int rg = g * waves + wv; rg < ngr; rg += NG * waves) {   // wave-uniform
        float acc[8];
        sh_rows8_acc<FMT>(W, x, rg * 8, H, lane, acc);
        if (lane == 0)
#pragma unroll
            for (int i = 0; i < 8; i++)
                if (rg * 8 + i < H) y[rg * 8 + i] = acc[i];
    }
}

__device__ __forceinline__ void shd_rows_any(const whip_mat &W, const float *x, float *y, int g, int NG, int waves)
{
    if (W.fmt == 3) shd_rows_role<3>(W, x, y, g, NG, waves);
    else if (W.fmt == 2) shd_rows_role<2>(W, x, y, g, NG, waves);
    else shd_rows_role<0>(W, x, y, g, NG, waves);
}

// whole 16-byte chunks of fp32 x, F32 / Q8G / Q4G rows (what the roles take)
static inline bool shd_rows_ok(const whip_mat *W, const float *x)
{
    return W && x && (uintptr_t)x % 16 == 0 && W->rows >= 1 && W->rowbytes % 16 == 0 &&
           (W->fmt == 0 || W->fmt == 2 || W->fmt == 3) && (W->fmt == 0 || (W->group % 32 == 0 && W->cols % 8 == 0)) &&
           (W->fmt != 0 || W->cols % 4 == 0);
}

