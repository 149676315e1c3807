// SPDX-License-Identifier: Apache-2.0
//
// log1pf.h — log1pf of the engine's host libm (glibc 2.35 on x86-64: the
// fdlibm algorithm, s_log1pf.c), so that the sqrt-softplus router score
// (src/model.c:5478-5484 calls libm's log1pf) is the engine's bit for bit
// on the device.  Plain float operations with no contraction (every HIP
// source here builds with -ffp-contract=off) and a correctly rounded
// division.  Host-compilable so that oracle/log1pf_check can compare it
// with the host libm over every float.
//
//   log1p(x) = k*ln2 + log(1+f),  1+x = 2^k (1+f),  sqrt(2)/2 < 1+f < sqrt(2),
//   log(1+f) = f - (f^2/2 - s*(f^2/2 + R(s^2))),  s = f/(2+f),
// with the correction c for the rounding of 1+x, and R the published
// degree-7 minimax polynomial in s^2 (coefficients Lp1..Lp7).
#pragma once
#include <stdint.h>

#ifdef __HIPCC__
#define WH_L1P_FN __host__ __device__ __forceinline__
#define WH_L1P_DIV(a, b) __fdiv_rn((a), (b))
#else
#define WH_L1P_FN static inline
#define WH_L1P_DIV(a, b) ((a) / (b))
#endif

WH_L1P_FN uint32_t wh_l1p_bits(float f)
{
    uint32_t u;
    __builtin_memcpy(&u, &f, 4);
    return u;
}
WH_L1P_FN float wh_l1p_float(uint32_t u)
{
    float f;
    __builtin_memcpy(&f, &u, 4);
    return f;
}

WH_L1P_FN float wh_log1pf(float x)
{
    const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f, two25 = 3.355443200e+07f;
    const float Lp1 = 6.6666668653e-01f, Lp2 = 4.0000000596e-01f, Lp3 = 2.8571429849e-01f,
                Lp4 = 2.2222198546e-01f, Lp5 = 1.8183572590e-01f, Lp6 = 1.5313838422e-01f,
                Lp7 = 1.4798198640e-01f;
    const int32_t hx = (int32_t)wh_l1p_bits(x), ax = hx & 0x7fffffff;
    float f = 0.0f, c = 0.0f, u;
    int32_t k = 1, hu = 0;
    if (hx < 0x3ed413d7) {                           // x < 0.41422
        if (ax >= 0x3f800000) {                      // x <= -1
            if (x == -1.0f) return WH_L1P_DIV(-two25, 0.0f);
            return WH_L1P_DIV(x - x, x - x);
        }
        if (ax < 0x31000000) {                       // |x| < 2^-29
            if (ax < 0x24800000) return x;           // |x| < 2^-54
            return x - x * x * 0.5f;
        }
        if (hx > 0 || hx <= (int32_t)0xbe95f61f) { k = 0; f = x; hu = 1; }   // -0.2929 < x < 0.41422
    } else if (hx >= 0x7f800000) {
        return x + x;
    }
    if (k != 0) {
        if (hx < 0x5a000000) {
            u = 1.0f + x;
            hu = (int32_t)wh_l1p_bits(u);
            k = (hu >> 23) - 127;
            c = (k > 0) ? 1.0f - (u - x) : x - (u - 1.0f);   // the rounding error of 1+x
            c = WH_L1P_DIV(c, u);
        } else {
            u = x;
            hu = (int32_t)wh_l1p_bits(u);
            k = (hu >> 23) - 127;
            c = 0.0f;
        }
        hu &= 0x007fffff;
        if (hu < 0x3504f7) {
            u = wh_l1p_float((uint32_t)hu | 0x3f800000u);        // 1+f
        } else {
            k += 1;
            u = wh_l1p_float((uint32_t)hu | 0x3f000000u);        // (1+f)/2
            hu = (0x00800000 - hu) >> 2;
        }
        f = u - 1.0f;
    }
    const float hfsq = 0.5f * f * f;
    if (hu == 0) {                                   // |f| < 2^-20
        if (f == 0.0f) {
            if (k == 0) return 0.0f;
            c += (float)k * ln2_lo;
            return (float)k * ln2_hi + c;
        }
        const float R = hfsq * (1.0f - 0.66666666666666666f * f);
        if (k == 0) return f - R;
        return (float)k * ln2_hi - ((R - ((float)k * ln2_lo + c)) - f);
    }
    const float s = WH_L1P_DIV(f, 2.0f + f), z = s * s;
    const float R = z * (Lp1 + z * (Lp2 + z * (Lp3 + z * (Lp4 + z * (Lp5 + z * (Lp6 + z * Lp7))))));
    if (k == 0) return f - (hfsq - s * (hfsq + R));
    return (float)k * ln2_hi - ((hfsq - (s * (hfsq + R) + ((float)k * ln2_lo + c))) - f);
}
