// SPDX-License-Identifier: Apache-2.0
//
// vq2r.hip — VQ2R experts (two residual stages of 256 entries, one index
// byte a stage: docs/FORMAT.md:180, 205) in the device layer, in the
// engine's own arithmetic: each table entry is vq_build_lut's
// (src/model.c:3864-3880 through lutb_range: model.c:3815-3854 portable,
// simd_avx512.c:90-123 with fma) and each row is vq_rows' generic loop
// (model.c:3966-3970: t = L0[c0] + L1[c1], acc += t over the positions in
// order, y = acc * f16(scale)).  One lane per row, the tables read through
// the caches: this path is exact, not fast.
#include "common.h"
#include "launch.h"

#define R2_EN 256
#define R2_LV 16

// table t = (input row t / kinds, kind t % kinds): lut[t][v][s][e] =
// sum_d x[8v + d] * C[cb + st*kind + s][e][d], booksT [book][8][256]
template <bool FMA>
__global__ void __launch_bounds__(256)
k_r2_lutb(const void *__restrict__ x, int x_bf16, int x_ld, int kinds, int st, const float *__restrict__ booksT,
          int cb, int nv, float *__restrict__ lut)
{
    const int t = blockIdx.y, row = t / kinds, kind = t - row * kinds;
    const int e = threadIdx.x;
    const int v0 = blockIdx.x * R2_LV, v1 = min(nv, v0 + R2_LV);
    for (int s = 0; s < st; s++) {
        const float *CT = booksT + (size_t)(cb + st * kind + s) * 8 * R2_EN;
        float c[8];
#pragma unroll
        for (int d = 0; d < 8; d++) c[d] = CT[d * R2_EN + e];
        for (int v = v0; v < v1; v++) {
            float xv[8];
            if (x_bf16) {
                const uint16_t *xr = (const uint16_t *)x + (size_t)row * x_ld + (size_t)v * 8;
#pragma unroll
                for (int d = 0; d < 8; d++) xv[d] = wh_bf16(xr[d]);
            } else {
                const float *xr = (const float *)x + (size_t)row * x_ld + (size_t)v * 8;
#pragma unroll
                for (int d = 0; d < 8; d++) xv[d] = xr[d];
            }
            float a = 0.0f;
#pragma unroll
            for (int d = 0; d < 8; d++) a = FMA ? __fmaf_rn(xv[d], c[d], a) : __fadd_rn(a, __fmul_rn(xv[d], c[d]));
            lut[(((size_t)t * nv + v) * st + s) * R2_EN + e] = a;
        }
    }
}

extern "C" int whip_r2_lutb(const void *x, int x_bf16, int x_ld, int rows, int kinds, int st, const float *booksT,
                            int cb, int nv, int fma, float *lut, hipStream_t s)
{
    if (rows <= 0 || kinds <= 0 || rows * kinds > 65535 || st < 1 || st > 8 || nv <= 0 || x_ld < nv * 8 || cb < 0)
        return (int)hipErrorInvalidValue;
    const dim3 grid((nv + R2_LV - 1) / R2_LV, rows * kinds);
    if (fma) hipLaunchKernelGGL(k_r2_lutb<true>, grid, dim3(R2_EN), 0, s, x, x_bf16, x_ld, kinds, st, booksT, cb, nv, lut);
    else hipLaunchKernelGGL(k_r2_lutb<false>, grid, dim3(R2_EN), 0, s, x, x_bf16, x_ld, kinds, st, booksT, cb, nv, lut);
    return (int)hipGetLastError();
}

// vq_rows of every pair's matrices, two stages: grid (row blocks, pairs,
// kinds), a lane per row.  Pair p's matrix `kind` is at idx_off[kind] of its
// expert's record (indices blocked [row / 64][v][row % 64][2]), its f16 row
// scales at sc_off[kind]; its table is pair_tok[p] * kinds + kind (per_tok)
// or p.  out[p][kind][M].  An unbound expert writes zeros and raises bit 0
// of err.
__global__ void __launch_bounds__(64)
k_r2_rows_pairs(const uint8_t *const *__restrict__ recs, const int32_t *__restrict__ pair_exp,
                const int32_t *__restrict__ pair_tok, int kinds, uint32_t idx_off0, uint32_t idx_off1,
                uint32_t sc_off0, uint32_t sc_off1, int M, int nv, const float *__restrict__ lut, int per_tok,
                float *__restrict__ out, int *__restrict__ err)
{
    const int p = blockIdx.y, kind = blockIdx.z, rb = blockIdx.x, lane = threadIdx.x;
    const int r = rb * 64 + lane;
    const uint8_t *rec = recs[pair_exp[p]];
    float *y = out + ((size_t)p * kinds + kind) * M;
    if (rec == nullptr) {                            // uniform
        if (r < M) y[r] = 0.0f;
        if (lane == 0) atomicOr(err, 1);
        return;
    }
    if (r >= M) return;
    const size_t tab = per_tok ? (size_t)pair_tok[p] * kinds + kind : (size_t)p;
    const float *L = lut + tab * nv * 2 * R2_EN;
    const uint16_t *ix = (const uint16_t *)(rec + (kind ? idx_off1 : idx_off0) + (size_t)rb * nv * 128) + lane;
    // eight positions' codes, then their sixteen entries, are in flight at
    // once; the sum still runs over the positions in order
    float acc = 0.0f;
    int v = 0;
    for (; v + 8 <= nv; v += 8) {
        uint32_t w[8];
#pragma unroll
        for (int j = 0; j < 8; j++) w[j] = ix[(size_t)(v + j) * 64];
        float t[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float *blk = L + (size_t)(v + j) * 2 * R2_EN;
            t[j] = __fadd_rn(blk[w[j] & 255], blk[R2_EN + (w[j] >> 8)]);
        }
#pragma unroll
        for (int j = 0; j < 8; j++) acc = __fadd_rn(acc, t[j]);
    }
    for (; v < nv; v++) {
        const uint32_t w = ix[(size_t)v * 64];
        const float *blk = L + (size_t)v * 2 * R2_EN;
        acc = __fadd_rn(acc, __fadd_rn(blk[w & 255], blk[R2_EN + (w >> 8)]));
    }
    const uint16_t *sc = (const uint16_t *)(rec + (kind ? sc_off1 : sc_off0));
    y[r] = __fmul_rn(acc, wh_f16_scale(sc[r]));
}

extern "C" int whip_r2_rows_pairs(const uint8_t *const *recs, const int32_t *pair_exp, const int32_t *pair_tok,
                                  int P, int kinds, const uint32_t *idx_off, const uint32_t *sc_off, int M, int nv,
                                  const float *lut, int per_tok, float *out, int *err, hipStream_t s)
{
    if (P <= 0 || P > 65535 || kinds < 1 || kinds > 2 || M <= 0 || nv <= 0 || idx_off[0] % 2 ||
        (kinds > 1 && idx_off[1] % 2))
        return (int)hipErrorInvalidValue;
    const dim3 grid((M + 63) / 64, P, kinds);
    hipLaunchKernelGGL(k_r2_rows_pairs, grid, dim3(64), 0, s, recs, pair_exp, pair_tok, kinds, idx_off[0],
                       kinds > 1 ? idx_off[1] : 0, sc_off[0], kinds > 1 ? sc_off[1] : 0, M, nv, lut, per_tok, out,
                       err);
    return (int)hipGetLastError();
}
