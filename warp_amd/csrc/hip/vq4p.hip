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
#include "common.h"
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

// Rows [r_lo, r_hi) (r_lo a multiple of 64); idx, scale and y are indexed
// from row 0 of the matrix.  fma: the fold as one fused multiply-add.
extern "C" int whip_vq_rows_p6(const uint8_t *idx, const uint16_t *scale, const int8_t *lut8,
                               const float *lscale, int r_lo, int r_hi, int nv, int fma, float *y,
                               hipStream_t s)
{
    if (r_lo < 0 || r_lo % 64 || r_hi <= r_lo || nv <= 0 || (uintptr_t)lut8 % 16) return (int)hipErrorInvalidValue;
    const dim3 grid((r_hi - r_lo + 63) / 64);
    if (fma) hipLaunchKernelGGL(k_vq_rows_p6<true>, grid, dim3(P6_THREADS), 0, s, idx, scale, lut8, lscale, r_lo, r_hi, nv, y);
    else hipLaunchKernelGGL(k_vq_rows_p6<false>, grid, dim3(P6_THREADS), 0, s, idx, scale, lut8, lscale, r_lo, r_hi, nv, y);
    return (int)hipGetLastError();
}

// ---- the device layer's VQ4P experts ------------------------------------------
// vq_build_lut (src/model.c:3864-3880) for a batch of tables: table
// t = (input row t / kinds, kind t % kinds) is
//   lut[t][v][s][e] = sum_d x[8v + d] * C[cb + 4 kind + s][e][d]
// in the engine's order for `fma`: one fused multiply-add chain over d from
// zero (lutb_range_avx512, src/simd_avx512.c:90-123), else a rounded product
// added to the running sum (waste_lutb_range, src/model.c:3815-3854).  A
// thread owns one (stage, entry) and P6_LV positions; booksT is the books
// transposed, [book][dim][64 entries], fp32 as the loader converts them.
#define P6_LV 16

template <bool FMA>
__global__ void __launch_bounds__(256)
k_p6_lutb(const void *__restrict__ x, int x_bf16, int x_ld, int kinds, const float *__restrict__ booksT,
          int cb, int nv, float *__restrict__ lut)
{
    const int t = blockIdx.y, row = t / kinds, kind = t - row * kinds;
    const int st = threadIdx.x >> 6, e = threadIdx.x & 63;
    const float *CT = booksT + (size_t)(cb + 4 * kind + st) * 8 * P6_EN;
    float c[8];
#pragma unroll
    for (int d = 0; d < 8; d++) c[d] = CT[d * P6_EN + e];
    const int v0 = blockIdx.x * P6_LV, v1 = min(nv, v0 + P6_LV);
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
        lut[((size_t)t * nv + v) * (4 * P6_EN) + st * P6_EN + e] = a;
    }
}

extern "C" int whip_p6_lutb(const void *x, int x_bf16, int x_ld, int rows, int kinds, const float *booksT, int cb,
                            int nv, int fma, float *lut, hipStream_t s)
{
    if (rows <= 0 || kinds <= 0 || rows * kinds > 65535 || nv <= 0 || x_ld < nv * 8 || cb < 0)
        return (int)hipErrorInvalidValue;
    const dim3 grid((nv + P6_LV - 1) / P6_LV, rows * kinds);
    if (fma) hipLaunchKernelGGL(k_p6_lutb<true>, grid, dim3(256), 0, s, x, x_bf16, x_ld, kinds, booksT, cb, nv, lut);
    else hipLaunchKernelGGL(k_p6_lutb<false>, grid, dim3(256), 0, s, x, x_bf16, x_ld, kinds, booksT, cb, nv, lut);
    return (int)hipGetLastError();
}

// vq_apply's rows (src/model.c:4152-4171) of every pair: grid (row blocks,
// pairs, kinds).  Pair p's matrix `kind` is at idx_off[kind] of its
// expert's record, its f16 row scales at sc_off[kind]; its table is
// pair_tok[p] * kinds + kind (per_tok: the token's gate/up tables) or p
// (its own, the down projection's).  out[p][kind][M].  An unbound expert
// writes zeros and raises bit 0 of err.
template <bool FMA>
__global__ void __launch_bounds__(P6_THREADS)
k_p6_rows_pairs(const uint8_t *const *__restrict__ recs, const int32_t *__restrict__ pair_exp,
                const int32_t *__restrict__ pair_tok, int kinds, uint32_t idx_off0, uint32_t idx_off1,
                uint32_t sc_off0, uint32_t sc_off1, int M, int nv, const int8_t *__restrict__ q,
                const float *__restrict__ qs, int per_tok, float *__restrict__ out, int *__restrict__ err)
{
    const int p = blockIdx.y, kind = blockIdx.z, rb = blockIdx.x;
    const uint8_t *rec = recs[pair_exp[p]];
    float *y = out + ((size_t)p * kinds + kind) * M;
    if (rec == nullptr) {                            // uniform
        if (threadIdx.x < 64 && rb * 64 + (int)threadIdx.x < M) y[rb * 64 + threadIdx.x] = 0.0f;
        if (threadIdx.x == 0) atomicOr(err, 1);
        return;
    }
    const size_t tab = per_tok ? (size_t)pair_tok[p] * kinds + kind : (size_t)p;
    const int nblk = (nv + P6_BLK - 1) / P6_BLK;
    p6_rows<FMA>(rec + (kind ? idx_off1 : idx_off0), (const uint16_t *)(rec + (kind ? sc_off1 : sc_off0)),
                 q + tab * nv * (4 * P6_EN), qs + tab * nblk, rb, M, nv, y);
}

extern "C" int whip_p6_rows_pairs(const uint8_t *const *recs, const int32_t *pair_exp, const int32_t *pair_tok,
                                  int P, int kinds, const uint32_t *idx_off, const uint32_t *sc_off, int M, int nv,
                                  const int8_t *q, const float *qs, int per_tok, int fma, float *out, int *err,
                                  hipStream_t s)
{
    if (P <= 0 || P > 65535 || kinds < 1 || kinds > 2 || M <= 0 || nv <= 0 || (uintptr_t)q % 16)
        return (int)hipErrorInvalidValue;
    const dim3 grid((M + 63) / 64, P, kinds);
    const uint32_t i1 = kinds > 1 ? idx_off[1] : 0, s1 = kinds > 1 ? sc_off[1] : 0;
    if (fma)
        hipLaunchKernelGGL(k_p6_rows_pairs<true>, grid, dim3(P6_THREADS), 0, s, recs, pair_exp, pair_tok, kinds,
                           idx_off[0], i1, sc_off[0], s1, M, nv, q, qs, per_tok, out, err);
    else
        hipLaunchKernelGGL(k_p6_rows_pairs<false>, grid, dim3(P6_THREADS), 0, s, recs, pair_exp, pair_tok, kinds,
                           idx_off[0], i1, sc_off[0], s1, M, nv, q, qs, per_tok, out, err);
    return (int)hipGetLastError();
}

// waste_act_pair_range (src/model.c): h = silu(g) * u for each pair's rows,
// gu[p][0][I] the gate rows, gu[p][1][I] the up rows, h[p][I].
__global__ void __launch_bounds__(256)
k_p6_act(const float *__restrict__ gu, int I, size_t n, float *__restrict__ h)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const size_t p = i / I, r = i - p * I;
    h[i] = wh_silu_mul(gu[(2 * p) * I + r], gu[(2 * p + 1) * I + r]);
}

extern "C" int whip_p6_act(const float *gu, int P, int I, float *h, hipStream_t s)
{
    if (P <= 0 || I <= 0) return (int)hipErrorInvalidValue;
    const size_t n = (size_t)P * I;
    hipLaunchKernelGGL(k_p6_act, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, gu, I, n, h);
    return (int)hipGetLastError();
}
