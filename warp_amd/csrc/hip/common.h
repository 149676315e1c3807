/* SPDX-License-Identifier: Apache-2.0 */
/*
 * common.h — device helpers shared by the gfx950 kernels.
 *
 * Everything here that produces a number the engine compares bit for bit
 * (expf, the two fp16 conversions) is written in IEEE operations with every
 * fused multiply-add explicit; the kernels are built with -ffp-contract=off
 * so the compiler adds none of its own.
 */
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>

// A launch that honours whip_time_next (launch.h): with timing armed, the
// dispatch records the armed events around the kernel.
bool whip_take_timing(hipEvent_t *start, hipEvent_t *stop);
#define WHIP_LAUNCH(K, GRID, BLOCK, LDS, S, ...)                                                 \
    do {                                                                                       \
        hipEvent_t e0_, e1_;                                                                   \
        if (whip_take_timing(&e0_, &e1_))                                                      \
            hipExtLaunchKernelGGL(K, GRID, BLOCK, LDS, S, e0_, e1_, 0, __VA_ARGS__);           \
        else                                                                                   \
            hipLaunchKernelGGL(K, GRID, BLOCK, LDS, S, __VA_ARGS__);                           \
    } while (0)

#define WH_INLINE __device__ __forceinline__

/* expf of the engine's host libm (glibc 2.35, x86-64 FMA build): the
 * published ARM optimized-routines method — x·32/ln2 = k + r by the
 * 1.5·2^52 shift, 2^(k/32) from a table of 2^(i/32) rounded to double
 * with the exponent pre-subtracted, a cubic in r, everything in double and
 * one rounding to float — with the same fused steps.  Equal to glibc's
 * expf on all 2^32 inputs (checked against the CPU restatement). */
__constant__ const uint64_t wh_exp_tab[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL,
};

// tab: the 32 table entries (wh_exp_tab, or a copy of it in LDS)
WH_INLINE float wh_expf_t(float x, const uint64_t *tab)
{
    const uint32_t ux = __float_as_uint(x);
    const uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) {
        if (ux == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8) return x + x;
        if (x > 0x1.62e42ep6f) return __int_as_float(0x7f800000);
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double inv = 0x1.71547652b82fep+0 * 32.0, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    const double z = __dmul_rn(inv, xd);
    double kd = __dadd_rn(z, shift);
    const uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd = __dsub_rn(kd, shift);
    const double r = __fma_rn(inv, xd, -kd);
    uint64_t t = tab[ki % 32];
    t += ki << 47;
    const double s = __longlong_as_double((long long)t);
    const double p = __fma_rn(c0, r, c1);
    const double r2 = __dmul_rn(r, r);
    double y = __fma_rn(c2, r, 1.0);
    y = __fma_rn(p, r2, y);
    y = __dmul_rn(y, s);
    return (float)y;
}

WH_INLINE float wh_expf(float x) { return wh_expf_t(x, wh_exp_tab); }

/* fp16 per-row / per-group scale: subnormals kept, exponent 31 read as a
 * normal exponent (the engine's waste_f16). */
WH_INLINE float wh_f16_scale(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1f, mn = h & 0x3ff;
    if (e == 0) {
        const float f = __fmul_rn((float)mn, 5.9604644775390625e-08f);
        return sign ? -f : f;
    }
    return __uint_as_float(sign | ((e + 112u) << 23) | (mn << 13));
}

/* fp16 codebook entry as the engine's loader converts it: subnormal -> 0. */
WH_INLINE float wh_f16_book(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1f, mn = h & 0x3ff;
    return __uint_as_float(e ? (sign | ((e + 112u) << 23) | (mn << 13)) : sign);
}

WH_INLINE float wh_bf16(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

WH_INLINE float wh_silu_mul(float g, float u)
{
    /* silu(g) * u with silu(v) = v / (1 + expf(-v)) */
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, wh_expf(-g))), u);
}

/* Cross-lane moves of a full-wave butterfly: DPP inside rows of 16 lanes
 * (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror),
 * then the row swaps permlane16 and permlane32.  Each pairs every lane
 * with one partner outside the set it has already combined, so six steps
 * of an order-free op reduce over all 64 lanes.  The caller's wave must be
 * fully active. */
template <int CTRL> WH_INLINE uint32_t dpp32(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

WH_INLINE float wave_sum(float v)
{
    v += __uint_as_float(dpp32<0xB1>(__float_as_uint(v)));
    v += __uint_as_float(dpp32<0x4E>(__float_as_uint(v)));
    v += __uint_as_float(dpp32<0x141>(__float_as_uint(v)));
    v += __uint_as_float(dpp32<0x140>(__float_as_uint(v)));
    {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    return v;
}

/* A pointer read from memory (a record table entry) is generic to the
 * compiler, which then emits flat loads: those count against the LDS wait
 * counter too, so every LDS read would also wait for the loads in flight.
 * Device records live in global memory; say so. */
#if defined(__HIP_DEVICE_COMPILE__)
#define WH_GLOBAL __attribute__((address_space(1)))
#else
#define WH_GLOBAL
#endif
typedef const uint8_t WH_GLOBAL g_u8;
typedef const uint16_t WH_GLOBAL g_u16;
WH_INLINE g_u8 *as_global(const uint8_t *p) { return (g_u8 *)p; }

/* Unaligned 4-byte read (gfx950 global loads accept any byte address). */
WH_INLINE uint32_t ld_u32_unaligned(const uint8_t *p)
{
    uint32_t w;
    __builtin_memcpy(&w, p, 4);
    return w;
}
