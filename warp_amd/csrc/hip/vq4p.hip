// SPDX-License-Identifier: Apache-2.0
//
// vq4p.hip — the VQ4P path (6-bit residual VQ: four stages of 64 entries,
// the four codes of a (row, position) packed in three bytes) through the
// engine's int8 LUT (src/model.c:3979-4114, the vqp_arg slot vq_rows_p6).
//
// The LUT entries are quantised to int8 per block of 32 positions (one fp32
// scale each), the per-block sums of a row are exact integers, and the
// blocks fold into fp32 in block order.  Both steps are discontinuous
// functions of their inputs, so the kernels reproduce the engine's
// arithmetic exactly: a correctly rounded division for the scale and its
// inverse, one rounded product and round-half-to-even for each code, an
// exact integer sum, and the fold either as the portable C kernel does it
// (a product, then a sum) or as the compilers contract it in the AVX-512
// and NEON kernels (one fused multiply-add).
#include <mutex>
#include <tuple>
#include <vector>

#include "common.h"
#include "gemv_dev.h"
#include "launch.h"

#define P6_BLK 32                      // positions per int8 scale block
#define P6_EN 64                       // entries per stage (the 6-bit codes)
#define QL_THREADS 1024
#define P6_THREADS 1024                // sixteen wavefronts on one 64-row block

// ---- the int8 table, one scale block per workgroup ---------------------------
__global__ void __launch_bounds__(QL_THREADS)
k_vq_quant_lut(const float *__restrict__ lut, int nv, int per_v, int8_t *__restrict__ q,
               float *__restrict__ scale)
{
    __shared__ float s_mx[QL_THREADS / 64];
    const int blk = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    {                                                // table blockIdx.y of a batch
        const size_t tab = blockIdx.y;
        lut += tab * nv * per_v;
        q += tab * nv * per_v;
        scale += tab * gridDim.x;
    }
    const int v0 = blk * P6_BLK, v1 = min(nv, v0 + P6_BLK);
    const size_t n = (size_t)(v1 - v0) * per_v, o = (size_t)v0 * per_v;
    float mx = 0.0f;
    for (size_t i = tid; i < n; i += QL_THREADS) mx = fmaxf(mx, fabsf(lut[o + i]));
    // the block's max |entry| (order-free)
    {
        uint32_t u = __float_as_uint(mx);
        auto m2 = [&](uint32_t p) { u = __uint_as_float(p) > __uint_as_float(u) ? p : u; };
        m2(dpp32<0xB1>(u));
        m2(dpp32<0x4E>(u));
        m2(dpp32<0x141>(u));
        m2(dpp32<0x140>(u));
        { const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false); u = r[0]; m2(r[1]); }
        { const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false); u = r[0]; m2(r[1]); }
        if (lane == 0) s_mx[wv] = __uint_as_float(u);
    }
    __syncthreads();
    mx = s_mx[0];
#pragma unroll
    for (int w = 1; w < QL_THREADS / 64; w++) mx = fmaxf(mx, s_mx[w]);
    if (tid == 0) scale[blk] = __fdiv_rn(mx, 127.0f);
    const float inv = mx > 0.0f ? __fdiv_rn(127.0f, mx) : 0.0f;
    for (size_t i = tid; i < n; i += QL_THREADS) {
        const float t = rintf(__fmul_rn(lut[o + i], inv));        // half to even, as lrintf
        q[o + i] = (int8_t)(int)fminf(127.0f, fmaxf(-127.0f, t));
    }
}

extern "C" int whip_vq_quant_lut(const float *lut, int nv, int stages, int entries, int8_t *q,
                                 float *scale, hipStream_t s)
{
    return whip_vq_quant_lut_n(lut, nv, stages, entries, 1, q, scale, s);
}

extern "C" int whip_vq_quant_lut_n(const float *lut, int nv, int stages, int entries, int ntab, int8_t *q,
                                   float *scale, hipStream_t s)
{
    if (nv <= 0 || stages <= 0 || entries <= 0 || ntab <= 0 || ntab > 65535) return (int)hipErrorInvalidValue;
    const int nblk = (nv + P6_BLK - 1) / P6_BLK;
    hipLaunchKernelGGL(k_vq_quant_lut, dim3(nblk, ntab), dim3(QL_THREADS), 0, s, lut, nv, stages * entries, q,
                       scale);
    return (int)hipGetLastError();
}

// ---- rows through the int8 table ---------------------------------------------
// One 1,024-thread workgroup per 64-row block, a lane per row.  The sixteen
// wavefronts split the block's 32-position scale blocks between them: for
// each, a wavefront stages that block's table (32 positions x 4 stages x 64
// entries, 8 KB) in its own LDS area, reads its rows' three code bytes per
// position (a position's 64 rows are 192 contiguous bytes, so the loads
// coalesce) and adds the four stages' entries into the block's exact integer
// sum.  A stage's table is 64 bytes, sixteen dwords in sixteen banks, so two
// lanes that meet in a bank read the same dword: the lookups never conflict.
// The sums wait in LDS until wavefront 0 folds them into fp32 in block order,
// the engine's order.
#define P6_WAVES (P6_THREADS / 64)
#define P6_GROUP 64                    // scale blocks folded per round

// the three code bytes at p (any alignment) from the aligned words that hold
// them: no read reaches past the aligned word holding the last code byte
__device__ __forceinline__ uint32_t p6_codes(const uint8_t *p)
{
    const uintptr_t a = (uintptr_t)p & ~(uintptr_t)3;
    const uint32_t sh = (uint32_t)((uintptr_t)p & 3);
    const uint32_t w0 = *(const uint32_t *)a;
    const uint32_t w1 = *(const uint32_t *)(a + (sh > 1 ? 4 : 0));
    return (uint32_t)((((uint64_t)w1 << 32) | w0) >> (8 * sh));
}

// Row block rb (rows below r_hi) of one matrix; idx, scale and y from row 0.
template <bool FMA>
__device__ __forceinline__ void p6_rows(const uint8_t *__restrict__ idx, const uint16_t *__restrict__ scale,
                                        const int8_t *__restrict__ lut8, const float *__restrict__ lscale,
                                        int rb, int r_hi, int nv, float *__restrict__ y)
{
    __shared__ __align__(16) int8_t s_t[P6_WAVES][P6_BLK * 4 * P6_EN];
    __shared__ int s_sum[P6_GROUP][64];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int r = rb * 64 + lane;
    const bool live = r < r_hi;
    const uint8_t *base = idx + (size_t)rb * nv * 192 + lane * 3;
    const int nb = (nv + P6_BLK - 1) / P6_BLK;
    int8_t *T = s_t[wv];
    float acc = 0.0f;
    for (int g0 = 0; g0 < nb; g0 += P6_GROUP) {
        const int gn = min(P6_GROUP, nb - g0);
        for (int jj = wv; jj < gn; jj += P6_WAVES) {                  // uniform per wavefront
            const int v0 = (g0 + jj) * P6_BLK, n = min(P6_BLK, nv - v0);
            {
                const uint4 *src = (const uint4 *)(lut8 + (size_t)v0 * 4 * P6_EN);
                for (int i = lane; i < n * 16; i += 64) ((uint4 *)T)[i] = src[i];
            }
            // the table's writes before any lane's lookups (one wavefront:
            // its LDS operations complete in order)
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            int sum = 0;
            if (live) {
                const uint8_t *ix = base + (size_t)v0 * 192;
                auto add = [&](int v, uint32_t c) {
                    const unsigned b0 = c & 0xff, b1 = (c >> 8) & 0xff, b2 = (c >> 16) & 0xff;
                    const int8_t *Tv = T + v * 4 * P6_EN;
                    sum += Tv[b0 & 0x3f] + Tv[P6_EN + (((b0 >> 6) | (b1 << 2)) & 0x3f)] +
                           Tv[2 * P6_EN + (((b1 >> 4) | (b2 << 4)) & 0x3f)] + Tv[3 * P6_EN + ((b2 >> 2) & 0x3f)];
                };
                if (n == P6_BLK) {
                    // every position's codes in flight at once, then the lookups
                    uint32_t c[P6_BLK];
#pragma unroll
                    for (int v = 0; v < P6_BLK; v++) c[v] = p6_codes(ix + (size_t)v * 192);
#pragma unroll
                    for (int v = 0; v < P6_BLK; v++) add(v, c[v]);
                } else {
                    for (int v = 0; v < n; v++) add(v, p6_codes(ix + (size_t)v * 192));
                }
            }
            // at most 4 * 32 * 127 in magnitude: the engine's int16 sum, exactly
            s_sum[jj][lane] = sum;
            // the next block's table overwrites this one: every lane's
            // lookups first
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        __syncthreads();
        if (wv == 0)
            for (int jj = 0; jj < gn; jj++) {
                const float ls = lscale[g0 + jj], sm = (float)s_sum[jj][lane];
                acc = FMA ? __fmaf_rn(ls, sm, acc) : __fadd_rn(acc, __fmul_rn(ls, sm));
            }
        __syncthreads();
    }
    if (wv == 0 && live) y[r] = __fmul_rn(acc, wh_f16_scale(scale[r]));
}

template <bool FMA>
__global__ void __launch_bounds__(P6_THREADS)
k_vq_rows_p6(const uint8_t *__restrict__ idx, const uint16_t *__restrict__ scale,
             const int8_t *__restrict__ lut8, const float *__restrict__ lscale, int r_lo, int r_hi, int nv,
             float *__restrict__ y)
{
    p6_rows<FMA>(idx, scale, lut8, lscale, r_lo / 64 + blockIdx.x, r_hi, nv, y);
}

// (defined with the layer's tile kernels below)
static int p6_rows_tiled(const uint8_t *idx, const uint16_t *scale, const int8_t *lut8, const float *lscale,
                         int r_lo, int nblk, int nv, int fma, float *y, hipStream_t s);

// Rows [r_lo, r_hi) (r_lo a multiple of 64); idx, scale and y are indexed
// from row 0 of the matrix.  fma: the fold as one fused multiply-add.
// With fewer than 64 row blocks (one workgroup each would leave most CUs
// idle) whole blocks go through the tile kernel (their block sums in a
// workspace, then the fold: two launches); a partial last block, whose
// codes end at its last row (the engine's record holds no bytes past them),
// and every block of a taller range through the row kernel above, which
// reads no further.
extern "C" int whip_vq_rows_p6(const uint8_t *idx, const uint16_t *scale, const int8_t *lut8,
                               const float *lscale, int r_lo, int r_hi, int nv, int fma, float *y,
                               hipStream_t s)
{
    if (r_lo < 0 || r_lo % 64 || r_hi <= r_lo || nv <= 0 || (uintptr_t)lut8 % 16) return (int)hipErrorInvalidValue;
    const int full = (r_hi - r_lo) / 64 < 64 ? (r_hi - r_lo) / 64 : 0, tail = r_lo + 64 * full;
    if (full > 0) {
        const int rc = p6_rows_tiled(idx, scale, lut8, lscale, r_lo, full, nv, fma, y, s);
        if (rc) return rc;
    }
    if (tail < r_hi) {
        const dim3 grid((r_hi - tail + 63) / 64);
        if (fma) hipLaunchKernelGGL(k_vq_rows_p6<true>, grid, dim3(P6_THREADS), 0, s, idx, scale, lut8, lscale, tail, r_hi, nv, y);
        else hipLaunchKernelGGL(k_vq_rows_p6<false>, grid, dim3(P6_THREADS), 0, s, idx, scale, lut8, lscale, tail, r_hi, nv, y);
    }
    return (int)hipGetLastError();
}

// ---- the device layer's VQ4P experts ------------------------------------------
// Two tile launches and the combine, each pair's rows the engine's bit for
// bit.  The gate/up launch builds each token's int8 gate and up tables
// from x and sums every pair's gate and up rows through them; the down
// launch folds those sums into the pair's gate and up rows, applies SwiGLU,
// builds the pair's int8 down table from the result and sums the down rows
// through it; the combine folds the down sums.  A row's sums are exact
// integers per 32-position scale block (at most 4 * 32 * 127 in magnitude:
// int16), folded into fp32 in block order, so the sums wait in HBM for the
// launch that needs the whole row, and the tiles are free to run in any
// order.
//
// A tile workgroup takes one (pair, kind), a group of up to P6_MAXG
// consecutive scale blocks and a run of `per` 64-row blocks.  It builds the
// group's tables in LDS (the engine's arithmetic: vq_build_lut's entries,
// src/model.c:3864-3880, in the order of the layer's p6_order: one fused
// multiply-add chain over d from zero as lutb_range_avx512,
// src/simd_avx512.c:90-123, else a rounded product added to the running sum
// as waste_lutb_range, src/model.c:3815-3854; then vq_quant_lut's block
// scale max|lut| / 127 and entries rint(lut * (127 / max)) clamped to
// [-127, 127], src/model.c:3979-4074), while its first tiles are in flight.
// A tile is 32 positions of 64 rows, 192 contiguous bytes a position (three
// code bytes a row).  Lane (quad q = lane % 16, slot k = lane / 16) loads
// the 12 bytes of rows 4q .. 4q+3 at positions k, k+4, .., k+28 (a 16-lane
// group per position: eight 12-byte loads a tile), adds four table bytes per
// row and position, and the four slots' sums meet across lanes (exact
// integer sums, in any order).  A position's table is 256 bytes at a
// 320-byte stride in LDS, so the four positions one instruction reads sit in
// four disjoint groups of sixteen banks and two lanes of a group meet in a
// bank only on one dword: the lookups do not conflict.  Two tiles are in
// flight per wavefront.  S[(pk * nb + b) * M + r], pk = pair * kinds + kind;
// the tables' scales qs[tab][b], tab = pair_tok[p] * kinds + kind (the
// gate/up launch: every pair of a token writes the same values) or p.
#define P6_MAXG 6                      // scale blocks a workgroup builds (x)
#define P6_MAXG_ACT 2                  // (SwiGLU: one row's folds per thread)
#define P6_TS 320                      // LDS bytes a position's table takes
#define P6_MAXB 32                     // gate/up blocks folded from registers

// One scale block of a table: lut[v][s][e] = sum_d x[8v + d] * C[s][e][d]
// (vq_build_lut, src/model.c:3864-3880) in the engine's order for FMA (one
// fused multiply-add chain over d from zero: lutb_range_avx512,
// src/simd_avx512.c:90-123; else a rounded product added to the running
// sum: waste_lutb_range, src/model.c:3815-3854), then the block's scale
// max|lut| / 127 and each entry's rint(lut * (127 / max)) clamped to
// [-127, 127] (vq_quant_lut, src/model.c:3979-4074), as k_vq_quant_lut
// does.  256 threads, thread (stage, entry); s_x holds the block's n
// positions (8n values), CT the four stages' books transposed
// ([stage][dim][64] fp32).  q: the block's first position of the table.
template <bool FMA>
__device__ __forceinline__ void p6_lutq_block(const float *s_x, int n, const float *__restrict__ CT,
                                              int8_t *__restrict__ q, float *__restrict__ scale)
{
    __shared__ float s_mx[4];
    const int tid = threadIdx.x, st = tid >> 6, e = tid & 63;
    const float *C = CT + (size_t)st * 8 * P6_EN;
    float c[8];
#pragma unroll
    for (int d = 0; d < 8; d++) c[d] = C[d * P6_EN + e];
    float l[P6_BLK];
    float mx = 0.0f;
#pragma unroll
    for (int v = 0; v < P6_BLK; v++) {
        float a = 0.0f;
#pragma unroll
        for (int d = 0; d < 8; d++) {
            const float xv = s_x[8 * v + d];
            a = FMA ? __fmaf_rn(xv, c[d], a) : __fadd_rn(a, __fmul_rn(xv, c[d]));
        }
        l[v] = a;
        if (v < n) mx = fmaxf(mx, fabsf(a));
    }
    // the block's max |entry| (order-free: no NaN survives the fmaxf above)
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m));
    if (e == 0) s_mx[st] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(s_mx[0], s_mx[1]), fmaxf(s_mx[2], s_mx[3]));
    if (tid == 0) *scale = __fdiv_rn(mx, 127.0f);
    const float inv = mx > 0.0f ? __fdiv_rn(127.0f, mx) : 0.0f;
#pragma unroll
    for (int v = 0; v < P6_BLK; v++)
        if (v < n) {
            const float t = rintf(__fmul_rn(l[v], inv));             // half to even, as lrintf
            q[v * 4 * P6_EN + st * P6_EN + e] = (int8_t)(int)fminf(127.0f, fmaxf(-127.0f, t));
        }
}

// Tables of rows x kinds inputs, one scale block per workgroup: table
// t = (row t / kinds, kind t % kinds) from x row t / kinds (bf16 or fp32)
// and books cb + 4 kind ..; q[t][nv][4][64], scale[t][nb].
template <bool FMA>
__global__ void __launch_bounds__(256)
k_p6_lutq(const void *__restrict__ x, int x_bf16, int x_ld, int kinds, const float *__restrict__ booksT, int cb,
          int nv, int8_t *__restrict__ q, float *__restrict__ qs)
{
    __shared__ float s_x[8 * P6_BLK];
    const int t = blockIdx.y, row = t / kinds, kind = t - row * kinds, b = blockIdx.x, i = threadIdx.x;
    const int v0 = b * P6_BLK, n = min(P6_BLK, nv - v0);
    float xv = 0.0f;                                 // past the block's positions: zeros, never used
    if (i < 8 * n) {
        const size_t o = (size_t)row * x_ld + (size_t)v0 * 8 + i;
        xv = x_bf16 ? wh_bf16(((const uint16_t *)x)[o]) : ((const float *)x)[o];
    }
    s_x[i] = xv;
    __syncthreads();
    p6_lutq_block<FMA>(s_x, n, booksT + (size_t)(cb + 4 * kind) * 8 * P6_EN, q + ((size_t)t * nv + v0) * 4 * P6_EN,
                       qs + (size_t)t * gridDim.x + b);
}

extern "C" int whip_p6_lutq(const void *x, int x_bf16, int x_ld, int rows, int kinds, const float *booksT, int cb,
                            int nv, int fma, int8_t *q, float *qs, hipStream_t s)
{
    if (rows <= 0 || kinds <= 0 || rows * kinds > 65535 || nv <= 0 || x_ld < nv * 8 || cb < 0)
        return (int)hipErrorInvalidValue;
    const dim3 grid((nv + P6_BLK - 1) / P6_BLK, rows * kinds);
    if (fma) WHIP_LAUNCH(k_p6_lutq<true>, grid, dim3(256), 0, s, x, x_bf16, x_ld, kinds, booksT, cb, nv, q, qs);
    else WHIP_LAUNCH(k_p6_lutq<false>, grid, dim3(256), 0, s, x, x_bf16, x_ld, kinds, booksT, cb, nv, q, qs);
    return (int)hipGetLastError();
}

// The gate/up rows of pair p (I of each), folded from their block sums in
// block order with the token's table scales and scaled by the row's f16
// scale (vq_rows_p6's fold, src/model.c:4076-4114), then h = silu(g) * u
// (waste_act_pair_range), then the pair's down table block from h: a
// workgroup per (down block, pair), thread i the row 8 v0 + i of h.
template <bool FMA>
__global__ void __launch_bounds__(256)
k_p6_act_lutq(const uint8_t *const *__restrict__ recs, const int32_t *__restrict__ pair_exp,
              const int32_t *__restrict__ pair_tok, const int16_t *__restrict__ S, const float *__restrict__ qs_gu,
              uint32_t sc_gate, uint32_t sc_up, int I, int nb_gu, const float *__restrict__ booksT, int cb_d,
              int nv_d, int8_t *__restrict__ q_d, float *__restrict__ qs_d)
{
    __shared__ float s_x[8 * P6_BLK];
    const int b = blockIdx.x, p = blockIdx.y, i = threadIdx.x;
    const int v0 = b * P6_BLK, n = min(P6_BLK, nv_d - v0), r = v0 * 8 + (i < 8 * n ? i : 0);
    // the rows' block sums go out first (they need no record), then the
    // record's scales; a thread past the block's rows reads the first row
    const int16_t *Sg = S + (size_t)p * 2 * nb_gu * I + r, *Su = Sg + (size_t)nb_gu * I;
    const float *lg = qs_gu + (size_t)pair_tok[p] * 2 * nb_gu, *lu = lg + nb_gu;
    const uint8_t *rec = recs[pair_exp[p]];
    float ag = 0.0f, au = 0.0f;
    for (int k0 = 0; k0 < nb_gu; k0 += P6_MAXB) {    // one round unless nb_gu > P6_MAXB
        // every block's sums in flight at once, then the folds in order
        const int kn = min(P6_MAXB, nb_gu - k0);
        int16_t sg[P6_MAXB], su[P6_MAXB];
#pragma unroll
        for (int k = 0; k < P6_MAXB; k++) {
            const int kk = k0 + (k < kn ? k : 0);
            sg[k] = Sg[(size_t)kk * I];
            su[k] = Su[(size_t)kk * I];
        }
#pragma unroll
        for (int k = 0; k < P6_MAXB; k++)
            if (k < kn) {
                const float fg = (float)sg[k], fu = (float)su[k];
                ag = FMA ? __fmaf_rn(lg[k0 + k], fg, ag) : __fadd_rn(ag, __fmul_rn(lg[k0 + k], fg));
                au = FMA ? __fmaf_rn(lu[k0 + k], fu, au) : __fadd_rn(au, __fmul_rn(lu[k0 + k], fu));
            }
    }
    float g = 0.0f, u = 0.0f;                        // an unbound expert's rows: zeros
    if (rec != nullptr) {
        g = __fmul_rn(ag, wh_f16_scale(((const uint16_t *)(rec + sc_gate))[r]));
        u = __fmul_rn(au, wh_f16_scale(((const uint16_t *)(rec + sc_up))[r]));
    }
    s_x[i] = i < 8 * n ? wh_silu_mul(g, u) : 0.0f;
    __syncthreads();
    p6_lutq_block<FMA>(s_x, n, booksT + (size_t)cb_d * 8 * P6_EN, q_d + ((size_t)p * nv_d + v0) * 4 * P6_EN,
                       qs_d + (size_t)p * gridDim.x + b);
}

extern "C" int whip_p6_act_lutq(const uint8_t *const *recs, const int32_t *pair_exp, const int32_t *pair_tok, int P,
                                const int16_t *S, const float *qs_gu, uint32_t sc_gate, uint32_t sc_up, int I,
                                int nv_gu, const float *booksT, int cb_d, int nv_d, int fma, int8_t *q_d,
                                float *qs_d, hipStream_t s)
{
    if (P <= 0 || P > 65535 || I <= 0 || I != nv_d * 8 || nv_gu <= 0 || cb_d < 0 || sc_gate % 2 || sc_up % 2)
        return (int)hipErrorInvalidValue;
    const int nb_gu = (nv_gu + P6_BLK - 1) / P6_BLK;
    const dim3 grid((nv_d + P6_BLK - 1) / P6_BLK, P);
#define AL(F) WHIP_LAUNCH(k_p6_act_lutq<F>, grid, dim3(256), 0, s, recs, pair_exp, pair_tok, S, qs_gu, sc_gate, \
                          sc_up, I, nb_gu, booksT, cb_d, nv_d, q_d, qs_d)
    if (fma) AL(true);
    else AL(false);
#undef AL
    return (int)hipGetLastError();
}

struct p6_tile_args {
    const uint8_t *raw;                // set: one matrix at raw (pair 0, table 0; no records)
    const uint8_t *const *recs;
    const int32_t *pair_exp, *pair_tok;
    int kinds;
    uint32_t idx_off0, idx_off1;
    int M, nv, nb;                     // rows, positions, scale blocks
    int ncb, ngrp, shares, per;        // the launch's partition
    int16_t *S;
    float *qs;
    int *err;
    const int8_t *q;                   // P6_Q: the tables, [tab][nv][4][64]
    const float *booksT;               // [book][8][64] fp32
    int cb;                            // the first book of kind 0's four
    const void *x;                     // gate/up: input rows (bf16 or fp32)
    int x_bf16, x_ld;
    whip_mat shd;                      // gate/up at one token, shd_y set: workgroups from
    const float *shd_x;                //   g_tiles on compute shd_y = shd . shd_x (the shared
    float *shd_y;                      //   expert's down projection) on the CUs the tiles leave
    int g_tiles;
    const int16_t *Sg;                 // down: the gate/up sums [p][2][nb_g][I]
    const float *qs_g;                 //       and their tables' scales [tok][2][nb_g]
    uint32_t sc_gate, sc_up;           //       the gate / up row scales in the record
    int nb_g;
};

#define P6_Q 0                         // tables read from q
#define P6_X 1                         // built from x (gate/up)
#define P6_ACT 2                       // built from SwiGLU of the gate/up sums (down)

template <int MODE, bool FMA>
__global__ void __launch_bounds__(P6_THREADS)
k_p6_tiles(p6_tile_args a)
{
    if (MODE == P6_X && a.shd_y && (int)blockIdx.x >= a.g_tiles) {   // uniform
        shd_rows_any(a.shd, a.shd_x, a.shd_y, blockIdx.x - a.g_tiles, gridDim.x - a.g_tiles, P6_WAVES);
        return;
    }
    constexpr bool ACT = MODE == P6_ACT;
    __shared__ __align__(16) int8_t s_tab[P6_MAXG * P6_BLK * P6_TS];
    __shared__ float s_x[MODE == P6_Q ? 1 : P6_MAXG * 8 * P6_BLK];   // each block's 256 inputs
    __shared__ float s_mx[P6_MAXG][P6_WAVES];
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = blockIdx.x % a.shares, rest = blockIdx.x / a.shares;
    const int bg = rest % a.ngrp, pk = rest / a.ngrp, kind = pk % a.kinds, p = pk / a.kinds;
    const int b0 = bg * a.ncb, nbg = min(a.ncb, a.nb - b0);
    const int rb0 = j * a.per, rb1 = min(a.M / 64, rb0 + a.per), ntile = nbg * (rb1 - rb0);
    const int M = a.M, nv = a.nv;
    int16_t *out = a.S + ((size_t)pk * a.nb + b0) * M;   // block b0 + bl at out + bl * M
    const uint8_t *rec = a.raw ? a.raw : a.recs[a.pair_exp[p]];
    if (rec == nullptr) {                            // uniform
        for (int bl = 0; bl < nbg; bl++)
            for (int r = rb0 * 64 + tid; r < rb1 * 64; r += P6_THREADS) out[(size_t)bl * M + r] = 0;
        if (tid == 0) atomicOr(a.err, 1);
        return;
    }
    const int tok = a.raw ? 0 : a.pair_tok[p];
    const size_t tab = a.kinds == 2 ? (size_t)tok * 2 + kind : (size_t)p;
    g_u8 *mat = as_global(rec) + (kind ? a.idx_off1 : a.idx_off0);
    const int qd = lane & 15, slot = lane >> 4;
    // tile t: scale block b0 + t % nbg, row block rb0 + t / nbg; positions
    // past a short block load position 0 (in bounds; their sums not added)
    auto load = [&](uint3 (&cc)[P6_BLK / 4], int t) {
        const int bl = t % nbg, rb = rb0 + t / nbg;
        const int n = min(P6_BLK, nv - (b0 + bl) * P6_BLK);
        g_u8 *ix = mat + ((size_t)rb * nv + (size_t)(b0 + bl) * P6_BLK) * 192 + 12 * qd;
#pragma unroll
        for (int i = 0; i < P6_BLK / 4; i++) {
            const int v = 4 * i + slot;
            cc[i] = *(const uint3 WH_GLOBAL *)(ix + (size_t)(v < n ? v : 0) * 192);
        }
    };
    auto sum_tile = [&](const uint3 (&cc)[P6_BLK / 4], int t) {
        const int bl = t % nbg, rb = rb0 + t / nbg;
        const int n = min(P6_BLK, nv - (b0 + bl) * P6_BLK);
        const int8_t *Tb = s_tab + bl * P6_BLK * P6_TS;
        int s4[4] = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < P6_BLK / 4; i++) {
            const int v = 4 * i + slot;
            const uint32_t w[4] = {cc[i].x, __builtin_amdgcn_alignbyte(cc[i].y, cc[i].x, 3),
                                   __builtin_amdgcn_alignbyte(cc[i].z, cc[i].y, 2), cc[i].z >> 8};
            const int8_t *T = Tb + v * P6_TS;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int en = T[w[k] & 63] + T[P6_EN + ((w[k] >> 6) & 63)] + T[2 * P6_EN + ((w[k] >> 12) & 63)] +
                               T[3 * P6_EN + ((w[k] >> 18) & 63)];
                s4[k] += v < n ? en : 0;
            }
        }
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const auto x1 = __builtin_amdgcn_permlane16_swap(s4[k], s4[k], false, false);
            s4[k] = (int)x1[0] + (int)x1[1];
            const auto x2 = __builtin_amdgcn_permlane32_swap(s4[k], s4[k], false, false);
            s4[k] = (int)x2[0] + (int)x2[1];
        }
        // each of the four lanes of a quad stores one of its rows
        const int mine = slot == 0 ? s4[0] : slot == 1 ? s4[1] : slot == 2 ? s4[2] : s4[3];
        out[(size_t)bl * M + rb * 64 + 4 * qd + slot] = (int16_t)mine;
    };
    // the wavefront's tiles wv + 16 i, i < cnt; every load is unconditional
    // (past the last tile: the last again), and the scheduling barriers keep
    // each buffer's loads together and in order, so a wait for one buffer
    // never covers the other's
    const int cnt = wv < ntile ? (ntile - wv + P6_WAVES - 1) / P6_WAVES : 0;
    auto tile_at = [&](int i) { return cnt > 0 ? wv + min(i, cnt - 1) * P6_WAVES : 0; };
    uint3 cA[P6_BLK / 4], cB[P6_BLK / 4];
    auto issue = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        load(cA, tile_at(0));
        __builtin_amdgcn_sched_barrier(0);
        load(cB, tile_at(1));
        __builtin_amdgcn_sched_barrier(0);
    };
    if (MODE == P6_Q) {
        // the group's tables (16 uint4s a position; past the group: the
        // first ones, unused), to LDS at the 320-byte stride
        const int v_lo = b0 * P6_BLK, nq = (min(nv, v_lo + nbg * P6_BLK) - v_lo) * 16;
        typedef unsigned v4u __attribute__((ext_vector_type(4)));   // kept in registers, unlike uint4 here
        const v4u *tsrc = (const v4u *)(a.q + (tab * nv + v_lo) * 4 * P6_EN);
        constexpr int TV = P6_MAXG * P6_BLK * 16 / P6_THREADS;
        v4u tv[TV];
#pragma unroll
        for (int k = 0; k < TV; k++) tv[k] = tsrc[tid + k * P6_THREADS < nq ? tid + k * P6_THREADS : 0];
        issue();
#pragma unroll
        for (int k = 0; k < TV; k++) {
            const int g = tid + k * P6_THREADS;
            *(v4u *)(s_tab + (g >> 4) * P6_TS + (g & 15) * 16) = tv[k];
        }
        __syncthreads();
    } else {
        // the table builder's books: thread (stage, entry) of tid % 256
        const int u = tid & 255, st = u >> 6, e = u & 63, quarter = tid >> 8;
        float c[8];
        {
            const float *C = a.booksT + ((size_t)(a.cb + (ACT ? 0 : 4 * kind) + st) * 8) * P6_EN + e;
#pragma unroll
            for (int d = 0; d < 8; d++) c[d] = C[d * P6_EN];
        }
        // the group's inputs: 8 n values a block (zeros past the block)
        const int i_hi = min(nv * 8, (b0 + nbg) * 8 * P6_BLK) - b0 * 8 * P6_BLK;
        if (!ACT) {
            for (int i = tid; i < nbg * 8 * P6_BLK; i += P6_THREADS) {
                float xv = 0.0f;
                if (i < i_hi) {
                    const size_t o = (size_t)tok * a.x_ld + (size_t)b0 * 8 * P6_BLK + i;
                    xv = a.x_bf16 ? wh_bf16(((const uint16_t *)a.x)[o]) : ((const float *)a.x)[o];
                }
                s_x[i] = xv;
            }
        } else if (tid < nbg * 8 * P6_BLK) {
            // h = silu(g) * u of row r: the gate and up rows folded from their
            // block sums in block order with the token's table scales, times
            // the row's f16 scale (vq_rows_p6's fold, src/model.c:4076-4114),
            // as waste_act_pair_range applies SwiGLU
            const int I = 8 * nv, r = b0 * 8 * P6_BLK + min(tid, i_hi > 0 ? i_hi - 1 : 0);
            const int16_t *Sgp = a.Sg + (size_t)p * 2 * a.nb_g * I + r, *Sup = Sgp + (size_t)a.nb_g * I;
            const float *lg = a.qs_g + (size_t)tok * 2 * a.nb_g, *lu = lg + a.nb_g;
            float ag = 0.0f, au = 0.0f;
            for (int k0 = 0; k0 < a.nb_g; k0 += P6_MAXB) {   // one round unless nb_g > P6_MAXB
                const int kn = min(P6_MAXB, a.nb_g - k0);
                int16_t sg[P6_MAXB], su[P6_MAXB];
#pragma unroll
                for (int k = 0; k < P6_MAXB; k++) {
                    const int kk = k0 + (k < kn ? k : 0);
                    sg[k] = Sgp[(size_t)kk * I];
                    su[k] = Sup[(size_t)kk * I];
                }
#pragma unroll
                for (int k = 0; k < P6_MAXB; k++)
                    if (k < kn) {
                        const float fg = (float)sg[k], fu = (float)su[k];
                        ag = FMA ? __fmaf_rn(lg[k0 + k], fg, ag) : __fadd_rn(ag, __fmul_rn(lg[k0 + k], fg));
                        au = FMA ? __fmaf_rn(lu[k0 + k], fu, au) : __fadd_rn(au, __fmul_rn(lu[k0 + k], fu));
                    }
            }
            const float g = __fmul_rn(ag, wh_f16_scale(((const uint16_t *)(rec + a.sc_gate))[r]));
            const float uu = __fmul_rn(au, wh_f16_scale(((const uint16_t *)(rec + a.sc_up))[r]));
            s_x[tid] = tid < i_hi ? wh_silu_mul(g, uu) : 0.0f;
        }
        __syncthreads();
        issue();
        // the tables while the first tiles fly: thread (stage, entry) builds
        // the eight positions quarter*8 .. of each block, twice (once for the
        // block's max, once to quantize: the same operations, the same values)
        auto entry = [&](int bl, int v) {
            float acc = 0.0f;
#pragma unroll
            for (int d = 0; d < 8; d++) {
                const float xv = s_x[bl * 8 * P6_BLK + v * 8 + d];
                acc = FMA ? __fmaf_rn(xv, c[d], acc) : __fadd_rn(acc, __fmul_rn(xv, c[d]));
            }
            return acc;
        };
        for (int bl = 0; bl < nbg; bl++) {           // uniform
            const int n = min(P6_BLK, nv - (b0 + bl) * P6_BLK);
            float mx = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int v = quarter * 8 + k;
                const float l = entry(bl, v);
                if (v < n) mx = fmaxf(mx, fabsf(l));   // order-free: no NaN survives fmaxf
            }
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m));
            if (lane == 0) s_mx[bl][wv] = mx;
        }
        __syncthreads();
        for (int bl = 0; bl < nbg; bl++) {           // uniform
            const int n = min(P6_BLK, nv - (b0 + bl) * P6_BLK);
            float mx = s_mx[bl][0];
#pragma unroll
            for (int w = 1; w < P6_WAVES; w++) mx = fmaxf(mx, s_mx[bl][w]);
            if (tid == 0 && j == 0) a.qs[tab * a.nb + b0 + bl] = __fdiv_rn(mx, 127.0f);
            const float inv = mx > 0.0f ? __fdiv_rn(127.0f, mx) : 0.0f;
            int8_t *T = s_tab + bl * P6_BLK * P6_TS + st * P6_EN + e;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int v = quarter * 8 + k;
                const float t = rintf(__fmul_rn(entry(bl, v), inv));   // half to even, as lrintf
                T[v * P6_TS] = v < n ? (int8_t)(int)fminf(127.0f, fmaxf(-127.0f, t)) : (int8_t)0;
            }
        }
        __syncthreads();
    }
    for (int i = 0; i < cnt; i += 2) {               // uniform
        sum_tile(cA, tile_at(i));
        __builtin_amdgcn_sched_barrier(0);
        load(cA, tile_at(i + 2));
        __builtin_amdgcn_sched_barrier(0);
        if (i + 1 < cnt) sum_tile(cB, tile_at(i + 1));
        __builtin_amdgcn_sched_barrier(0);
        load(cB, tile_at(i + 3));
        __builtin_amdgcn_sched_barrier(0);
    }
}

// the launch's partition: runs of at most 32 row blocks; groups of scale
// blocks so that there is about one workgroup per CU
static int p6_launch(p6_tile_args &a, int P, int mode, int fma, hipStream_t s)
{
    const int nrb = a.M / 64;
    a.nb = (a.nv + P6_BLK - 1) / P6_BLK;
    long shares = (nrb + 31) / 32;
    a.per = (int)((nrb + shares - 1) / shares);
    a.shares = (int)((nrb + a.per - 1) / a.per);
    const long tiles = (long)P * a.kinds * a.nb * nrb, want = (tiles + 255) / 256;
    const int maxg = mode == P6_ACT ? P6_MAXG_ACT : P6_MAXG;
    long ncb = (2 * want + a.per) / (2 * a.per);      // rounded
    if (ncb > maxg) ncb = maxg;
    if (ncb > a.nb) ncb = a.nb;
    if (ncb < 1) ncb = 1;
    a.ncb = (int)ncb;
    a.ngrp = (a.nb + a.ncb - 1) / a.ncb;
    // a small problem (one matrix) spreads over more, shorter runs
    const long groups = (long)P * a.kinds * a.ngrp;
    if (groups * a.shares < 128) {
        long sh = (256 + groups - 1) / groups;
        if (sh > nrb) sh = nrb;
        if (sh > a.shares) {
            a.per = (int)((nrb + sh - 1) / sh);
            a.shares = (nrb + a.per - 1) / a.per;
        }
    }
    long grid = groups * a.shares;
    if (grid > 0x7fffffffL) return (int)hipErrorInvalidValue;
    // the shared down projection on the CUs the tiles leave (at least
    // eight workgroups, which then run where tiles finish first)
    a.g_tiles = (int)grid;
    if (a.shd_y) {
        int n_cu = 256, dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu < 1)
            n_cu = 256;
        grid += n_cu - grid > 8 ? n_cu - grid : 8;
    }
#define TL(A, F) WHIP_LAUNCH((k_p6_tiles<A, F>), dim3((unsigned)grid), dim3(P6_THREADS), 0, s, a)
    if (mode == P6_Q) TL(P6_Q, false);
    else if (mode == P6_ACT) { if (fma) TL(P6_ACT, true); else TL(P6_ACT, false); }
    else { if (fma) TL(P6_X, true); else TL(P6_X, false); }
#undef TL
    return (int)hipGetLastError();
}

extern "C" int whip_p6_gate_up(const uint8_t *const *recs, const int32_t *pair_exp, const int32_t *pair_tok, int P,
                               const uint32_t *idx_off, int I, const void *x, int x_bf16, int x_ld, int nv,
                               const float *booksT, int cb, int fma, const int8_t *q, int16_t *S, float *qs, int *err,
                               const whip_mat *shd, const float *shd_x, float *shd_y, hipStream_t s)
{
    if (P <= 0 || I <= 0 || I % 64 || nv <= 0 || idx_off[0] % 4 || idx_off[1] % 4 || (uintptr_t)q % 16 ||
        (!q && (x_ld < nv * 8 || cb < 0)))
        return (int)hipErrorInvalidValue;
    // the shared down projection rides along only where the tables are
    // built here (one token), in whole 16-byte chunks
    if (shd_y && (q || !shd_rows_ok(shd, shd_x))) return (int)hipErrorInvalidValue;
    p6_tile_args a = {};
    if (shd_y) { a.shd = *shd; a.shd_x = shd_x; a.shd_y = shd_y; }
    a.recs = recs; a.pair_exp = pair_exp; a.pair_tok = pair_tok; a.kinds = 2;
    a.idx_off0 = idx_off[0]; a.idx_off1 = idx_off[1]; a.M = I; a.nv = nv;
    a.S = S; a.qs = qs; a.err = err; a.q = q; a.booksT = booksT; a.cb = cb;
    a.x = x; a.x_bf16 = x_bf16; a.x_ld = x_ld;
    return p6_launch(a, P, q ? P6_Q : P6_X, fma, s);
}

extern "C" int whip_p6_down(const uint8_t *const *recs, const int32_t *pair_exp, const int32_t *pair_tok, int P,
                            uint32_t idx_off, int H, int I, const int16_t *Sg, const float *qs_g, uint32_t sc_gate,
                            uint32_t sc_up, int nv_g, const float *booksT, int cb, int fma, const int8_t *q,
                            int16_t *S, float *qs, int *err, hipStream_t s)
{
    if (P <= 0 || H <= 0 || H % 64 || I <= 0 || I % 8 || idx_off % 4 || (uintptr_t)q % 16 ||
        (!q && (nv_g <= 0 || cb < 0 || sc_gate % 2 || sc_up % 2)))
        return (int)hipErrorInvalidValue;
    p6_tile_args a = {};
    a.recs = recs; a.pair_exp = pair_exp; a.pair_tok = pair_tok; a.kinds = 1;
    a.idx_off0 = idx_off; a.idx_off1 = idx_off; a.M = H; a.nv = I / 8;
    a.S = S; a.qs = qs; a.err = err; a.q = q; a.booksT = booksT; a.cb = cb;
    a.Sg = Sg; a.qs_g = qs_g; a.sc_gate = sc_gate; a.sc_up = sc_up; a.nb_g = (nv_g + P6_BLK - 1) / P6_BLK;
    return p6_launch(a, P, q ? P6_Q : P6_ACT, fma, s);
}

// y[r_lo + i] = fold over the blocks in order of ls[b] * S[b*M + i], times
// the row's f16 scale (vq_rows_p6's fold), i < M.
template <bool FMA>
__global__ void __launch_bounds__(256)
k_p6_fold(const int16_t *__restrict__ S, int nb, int M, const float *__restrict__ ls,
          const uint16_t *__restrict__ scale, int r_lo, float *__restrict__ y)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= M) return;
    float acc = 0.0f;
    for (int k0 = 0; k0 < nb; k0 += P6_MAXB) {        // every block's sums in flight, then the fold
        const int kn = min(P6_MAXB, nb - k0);
        int16_t sv[P6_MAXB];
#pragma unroll
        for (int k = 0; k < P6_MAXB; k++) sv[k] = S[(size_t)(k0 + (k < kn ? k : 0)) * M + i];
#pragma unroll
        for (int k = 0; k < P6_MAXB; k++)
            if (k < kn) {
                const float f = (float)sv[k];
                acc = FMA ? __fmaf_rn(ls[k0 + k], f, acc) : __fadd_rn(acc, __fmul_rn(ls[k0 + k], f));
            }
    }
    y[r_lo + i] = __fmul_rn(acc, wh_f16_scale(scale[r_lo + i]));
}

// The block sums' workspace of whip_vq_rows_p6: one per (device, stream),
// grown when a call needs more (hipFree waits for the device, so the old
// one is idle by then) and kept until the process ends.  Calls on one
// stream run in order; calls on different streams never share one.
static std::mutex g_ws_mu;
static std::vector<std::tuple<int, hipStream_t, void *, size_t>> g_ws;

static int p6_workspace(hipStream_t s, size_t bytes, void **out)
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    std::lock_guard<std::mutex> lk(g_ws_mu);
    for (auto &w : g_ws)
        if (std::get<0>(w) == dev && std::get<1>(w) == s) {
            if (std::get<3>(w) < bytes) {
                e = hipFree(std::get<2>(w));
                std::get<2>(w) = nullptr;
                std::get<3>(w) = 0;
                if (e != hipSuccess) return (int)e;
                e = hipMalloc(&std::get<2>(w), bytes);
                if (e != hipSuccess) return (int)e;
                std::get<3>(w) = bytes;
            }
            *out = std::get<2>(w);
            return 0;
        }
    void *p = nullptr;
    e = hipMalloc(&p, bytes);
    if (e != hipSuccess) return (int)e;
    g_ws.emplace_back(dev, s, p, bytes);
    *out = p;
    return 0;
}

static int p6_rows_tiled(const uint8_t *idx, const uint16_t *scale, const int8_t *lut8, const float *lscale,
                         int r_lo, int nblk, int nv, int fma, float *y, hipStream_t s)
{
    const int M = 64 * nblk, nb = (nv + P6_BLK - 1) / P6_BLK;
    int16_t *S = nullptr;
    const int wrc = p6_workspace(s, (size_t)nb * M * sizeof(int16_t), (void **)&S);
    if (wrc) return wrc;
    p6_tile_args a = {};
    a.raw = idx + (size_t)(r_lo / 64) * nv * 192;
    a.kinds = 1; a.M = M; a.nv = nv; a.S = S; a.q = lut8;
    int rc = p6_launch(a, 1, P6_Q, fma, s);
    if (!rc) {
        const dim3 grid((M + 255) / 256);
        if (fma) hipLaunchKernelGGL(k_p6_fold<true>, grid, dim3(256), 0, s, S, nb, M, lscale, scale, r_lo, y);
        else hipLaunchKernelGGL(k_p6_fold<false>, grid, dim3(256), 0, s, S, nb, M, lscale, scale, r_lo, y);
        rc = (int)hipGetLastError();
    }
    return rc;
}

// Each pair's down rows folded from its block sums (whip_p6_down's S, nb
// blocks of M rows a pair, its table scales ls[p][nb]) in block order, times
// the row's f16 scale at sc_off of its record; an unbound expert's rows are
// zeros.  y[p][M]: the rows the combine adds, one chunk each.
template <bool FMA>
__global__ void __launch_bounds__(256)
k_p6_fold_pairs(const uint8_t *const *__restrict__ recs, const int32_t *__restrict__ pair_exp,
                const int16_t *__restrict__ S, const float *__restrict__ ls, int nb, int M, uint32_t sc_off,
                float *__restrict__ y)
{
    const int p = blockIdx.y, r = blockIdx.x * 256 + threadIdx.x;
    if (r >= M) return;
    const uint8_t *rec = recs[pair_exp[p]];
    const int16_t *Sp = S + (size_t)p * nb * M + r;
    const float *lp = ls + (size_t)p * nb;
    float acc = 0.0f;
    for (int k0 = 0; k0 < nb; k0 += P6_MAXB) {        // every block's sums in flight, then the fold
        const int kn = min(P6_MAXB, nb - k0);
        int16_t sv[P6_MAXB];
#pragma unroll
        for (int k = 0; k < P6_MAXB; k++) sv[k] = Sp[(size_t)(k0 + (k < kn ? k : 0)) * M];
#pragma unroll
        for (int k = 0; k < P6_MAXB; k++)
            if (k < kn) {
                const float f = (float)sv[k];
                acc = FMA ? __fmaf_rn(lp[k0 + k], f, acc) : __fadd_rn(acc, __fmul_rn(lp[k0 + k], f));
            }
    }
    y[(size_t)p * M + r] = rec ? __fmul_rn(acc, wh_f16_scale(((const uint16_t *)(rec + sc_off))[r])) : 0.0f;
}

extern "C" int whip_p6_fold_pairs(const uint8_t *const *recs, const int32_t *pair_exp, int P, const int16_t *S,
                                  const float *ls, int nb, int M, uint32_t sc_off, int fma, float *y, hipStream_t s)
{
    if (P <= 0 || P > 65535 || nb <= 0 || M <= 0 || sc_off % 2) return (int)hipErrorInvalidValue;
    const dim3 grid((M + 255) / 256, P);
    if (fma) WHIP_LAUNCH(k_p6_fold_pairs<true>, grid, dim3(256), 0, s, recs, pair_exp, S, ls, nb, M, sc_off, y);
    else WHIP_LAUNCH(k_p6_fold_pairs<false>, grid, dim3(256), 0, s, recs, pair_exp, S, ls, nb, M, sc_off, y);
    return (int)hipGetLastError();
}

