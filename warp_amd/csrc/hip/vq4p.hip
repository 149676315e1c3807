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
#define P6_THREADS 256                 // four 64-row blocks a workgroup

// ---- the int8 table, one scale block per workgroup ---------------------------
__global__ void __launch_bounds__(QL_THREADS)
k_vq_quant_lut(const float *__restrict__ lut, int nv, int per_v, int8_t *__restrict__ q,
               float *__restrict__ scale)
{
    __shared__ float s_mx[QL_THREADS / 64];
    const int blk = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
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
    if (nv <= 0 || stages <= 0 || entries <= 0) return (int)hipErrorInvalidValue;
    const int nblk = (nv + P6_BLK - 1) / P6_BLK;
    hipLaunchKernelGGL(k_vq_quant_lut, dim3(nblk), dim3(QL_THREADS), 0, s, lut, nv, stages * entries, q, scale);
    return (int)hipGetLastError();
}

// ---- rows through the int8 table ---------------------------------------------
// Wavefront w of a workgroup owns the 64-row block blockIdx.x * 4 + w, a
// lane one row.  Per scale block the workgroup stages the block's table
// (32 positions x 4 stages x 64 entries, 8 KB) in LDS; each lane then reads
// its row's three code bytes per position (a block's 64 rows are 192
// contiguous bytes, so the wavefront's reads coalesce) and adds the four
// stages' entries into an exact integer sum.
template <bool FMA>
__global__ void __launch_bounds__(P6_THREADS)
k_vq_rows_p6(const uint8_t *__restrict__ idx, const uint16_t *__restrict__ scale,
             const int8_t *__restrict__ lut8, const float *__restrict__ lscale, int r_lo, int r_hi, int nv,
             float *__restrict__ y)
{
    __shared__ __align__(16) int8_t s_t[P6_BLK * 4 * P6_EN];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int rb = r_lo / 64 + blockIdx.x * (P6_THREADS / 64) + wv;   // 64-row block
    const int r = rb * 64 + lane;
    const bool live = r >= r_lo && r < r_hi;
    const uint8_t *base = idx + (size_t)rb * nv * 192 + lane * 3;
    float acc = 0.0f;
    for (int v0 = 0; v0 < nv; v0 += P6_BLK) {
        const int nb = min(P6_BLK, nv - v0);
        __syncthreads();                             // the last block's table is done with
        {
            const uint4 *src = (const uint4 *)(lut8 + (size_t)v0 * 4 * P6_EN);
            uint4 *dst = (uint4 *)s_t;
            for (int i = tid; i < nb * 4 * P6_EN / 16; i += P6_THREADS) dst[i] = src[i];
        }
        __syncthreads();
        int sum = 0;
        if (live) {
            for (int v = 0; v < nb; v++) {
                const uint8_t *ix = base + (size_t)(v0 + v) * 192;
                const unsigned b0 = ix[0], b1 = ix[1], b2 = ix[2];
                const int8_t *T = s_t + v * 4 * P6_EN;
                sum += T[b0 & 0x3f] + T[P6_EN + (((b0 >> 6) | (b1 << 2)) & 0x3f)] +
                       T[2 * P6_EN + (((b1 >> 4) | (b2 << 4)) & 0x3f)] + T[3 * P6_EN + ((b2 >> 2) & 0x3f)];
            }
        }
        // at most 4 * 32 * 127 in magnitude: the engine's int16 sum, exactly
        const float ls = lscale[v0 / P6_BLK];
        acc = FMA ? __fmaf_rn(ls, (float)sum, acc) : __fadd_rn(acc, __fmul_rn(ls, (float)sum));
    }
    if (live) y[r] = __fmul_rn(acc, wh_f16_scale(scale[r]));
}

// Rows [r_lo, r_hi) (r_lo a multiple of 64); idx, scale and y are indexed
// from row 0 of the matrix.  fma: the fold as one fused multiply-add.
extern "C" int whip_vq_rows_p6(const uint8_t *idx, const uint16_t *scale, const int8_t *lut8,
                               const float *lscale, int r_lo, int r_hi, int nv, int fma, float *y,
                               hipStream_t s)
{
    if (r_lo < 0 || r_lo % 64 || r_hi <= r_lo || nv <= 0 || (uintptr_t)lut8 % 16) return (int)hipErrorInvalidValue;
    const int blocks = (r_hi - r_lo + 63) / 64;
    const dim3 grid((blocks + P6_THREADS / 64 - 1) / (P6_THREADS / 64));
    if (fma) hipLaunchKernelGGL(k_vq_rows_p6<true>, grid, dim3(P6_THREADS), 0, s, idx, scale, lut8, lscale, r_lo, r_hi, nv, y);
    else hipLaunchKernelGGL(k_vq_rows_p6<false>, grid, dim3(P6_THREADS), 0, s, idx, scale, lut8, lscale, r_lo, r_hi, nv, y);
    return (int)hipGetLastError();
}
