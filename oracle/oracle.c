/* SPDX-License-Identifier: Apache-2.0 */
/*
 * oracle.c — CPU restatement of WARP's MoE expert path, in the reference's
 * exact floating-point order.  TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Built with -ffp-contract=off: every fused multiply-add below is an
 * explicit fmaf()/fma(), standing where the reference has one (an FMA
 * intrinsic, or a contraction its compiler flags allow); every other
 * product is rounded before it is added, as the reference's model.c is
 * compiled on x86-64 (-O2 -std=gnu11, no -mfma: Makefile:15).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define WQ_F32 0
#define WQ_Q8G 2
#define WQ_Q4G 3
#define WQ_Q3G 7
#define WQ_VQ3R 4
#define WQ_VQ4P 8
#define WQ_VQ2R 5
#define MAGIC_EXPERT 0x50584557u

/* ---- expf ----------------------------------------------------------------
 * The reference calls glibc's expf (router scores src/model.c:5474-5484,
 * SiLU src/model.c:1231).  glibc 2.35 on x86-64 with FMA runs the published
 * ARM optimized-routines expf (Szabolcs Nagy, 2017): x·32/ln2 = k + r with
 * the 1.5·2^52 shift trick, 2^(k/32) from a 32-entry table of 2^(i/32)
 * correctly rounded to double with the exponent pre-subtracted, and a
 * degree-3 polynomial in r, all in double, rounded once to float.  Its FMA
 * build contracts r = z - kd with the product z = x·32/ln2 and the three
 * polynomial steps.  The table is 2^(i/32) computed to 60 digits and
 * rounded to double; it is not copied from anywhere.  This restatement
 * agrees with glibc 2.35's expf on all 2^32 float inputs (exhaustive run
 * recorded with the golden fixtures). */
static const uint64_t EXP_T[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL,
};

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint64_t d2u(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
static inline double u2d(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }

float orc_expf(float x)
{
    const uint32_t abstop = (f2u(x) >> 20) & 0x7ff;
    if (abstop >= 0x42b) {                      /* |x| >= 88, inf or nan */
        if (f2u(x) == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8) return x + x;
        if (x > 0x1.62e42ep6f) return INFINITY;
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double inv = 0x1.71547652b82fep+0 * 32.0, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    const double z = inv * xd;
    double kd = z + shift;
    const uint64_t ki = d2u(kd);
    kd -= shift;
    const double r = fma(inv, xd, -kd);
    uint64_t t = EXP_T[ki % 32];
    t += ki << 47;
    const double s = u2d(t);
    const double p = fma(c0, r, c1);
    const double r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(p, r2, y);
    y = y * s;
    return (float)y;
}

/* waste_f16, src/simd.h:81-99: fp16 -> fp32 keeping subnormals (mantissa
 * times 2^-24); exponent 31 is taken as a normal exponent (143 - 127). */
float orc_f16_scale(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1f, mn = h & 0x3ff;
    if (e == 0) {
        const float f = (float)mn * 5.9604644775390625e-08f;
        return sign ? -f : f;
    }
    return u2f(sign | ((e + 112u) << 23) | (mn << 13));
}

/* Codebook loader, src/model.c:2915-2923: same conversion, except that an
 * fp16 subnormal becomes a signed zero. */
float orc_f16_book(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1f, mn = h & 0x3ff;
    return u2f(e ? (sign | ((e + 112u) << 23) | (mn << 13)) : sign);
}

/* zlib's crc32 (reflected 0xEDB88320), as src/crc32.c computes it. */
uint32_t orc_crc32(const uint8_t *p, size_t n)
{
    static uint32_t tab[256];
    static int ready = 0;
    if (!ready) {
        for (uint32_t i = 0; i < 256; i++) {
            uint32_t c = i;
            for (int k = 0; k < 8; k++) c = (c & 1) ? 0xEDB88320u ^ (c >> 1) : c >> 1;
            tab[i] = c;
        }
        ready = 1;
    }
    uint32_t c = 0xFFFFFFFFu;
    for (size_t i = 0; i < n; i++) c = tab[(c ^ p[i]) & 0xff] ^ (c >> 8);
    return c ^ 0xFFFFFFFFu;
}

/* src/model.c:2906-2941: fp16 books to fp32, then the [book][dim][entry]
 * transpose the LUT build reads. */
void orc_books_load(const uint16_t *f16, int n_books, int entries, int vec_dim,
                    float *books, float *booksT)
{
    const size_t per = (size_t)entries * vec_dim;
    for (int b = 0; b < n_books; b++)
        for (size_t i = 0; i < per; i++)
            books[(size_t)b * per + i] = orc_f16_book(f16[(size_t)b * per + i]);
    if (!booksT) return;
    for (int b = 0; b < n_books; b++)
        for (int c = 0; c < entries; c++)
            for (int d = 0; d < vec_dim; d++)
                booksT[(size_t)b * per + (size_t)d * entries + c] =
                    books[(size_t)b * per + (size_t)c * vec_dim + d];
}

/* ---- LUT build -----------------------------------------------------------
 * lut[v][s][c] = sum_d x[8v+d] * C_s[c][d].
 * ORC_PORTABLE: waste_lutb_range, src/model.c:3815-3854 (x86 branch):
 *   t = 0; t += x[d]*C  — product rounded, then added.
 * ORC_AVX512:   lutb_range_avx512, src/simd_avx512.c:90-123: per entry an
 *   fma chain over d from 0, for every block of 64 entries; a ragged tail
 *   of entries is the scalar sum, which that file's -mavx512f build also
 *   contracts into fma. */
void orc_lutb(float *lut, const float *booksT, const float *x, int cb_base,
              int stages, int entries, int vec_dim, int v_lo, int v_hi,
              int order)
{
    const int en = entries, vd = vec_dim, st = stages;
    for (int v = v_lo; v < v_hi; v++) {
        const float *xv = x + (size_t)v * vd;
        for (int s = 0; s < st; s++) {
            const float *CT = booksT + (size_t)(cb_base + s) * en * vd;
            float *dst = lut + ((size_t)v * st + s) * en;
            int c = 0;
            if (order == ORC_AVX512) {
                for (; c + 64 <= en; c += 64)
                    for (int cc = c; cc < c + 64; cc++) {
                        float a = 0.0f;
                        for (int d = 0; d < vd; d++) a = fmaf(xv[d], CT[(size_t)d * en + cc], a);
                        dst[cc] = a;
                    }
            }
            for (; c < en; c++) {
                float t = 0;
                if (order == ORC_AVX512)
                    for (int d = 0; d < vd; d++) t = fmaf(xv[d], CT[(size_t)d * en + c], t);
                else
                    for (int d = 0; d < vd; d++) t += xv[d] * CT[(size_t)d * en + c];
                dst[c] = t;
            }
        }
    }
}

/* ---- VQ3R apply ----------------------------------------------------------
 * vq_rows, src/model.c:3909-3977.  Per row: acc = 0; for v ascending,
 * t = L[v][0][i0] + L[v][1][i1] (+ L[v][2][i2] ...) left to right, acc += t;
 * y = acc * f16(scale).  The 64-row tiling and the 8-row word-load unroll
 * change which rows are worked on together, never a row's own sum.
 * Indices are blocked [row/64][v][row%64][stage] (docs/FORMAT.md:216-223). */
void orc_vq_rows(float *y, const uint8_t *idx, const uint16_t *scale,
                 const float *lut, int r_lo, int r_hi, int nv, int stages,
                 int entries)
{
    const int st = stages, en = entries;
    for (int r = r_lo; r < r_hi; r++) {
        float acc = 0.0f;
        const uint8_t *base = idx + (size_t)(r / 64) * nv * 64 * st + (size_t)(r % 64) * st;
        for (int v = 0; v < nv; v++) {
            const uint8_t *ix = base + (size_t)v * 64 * st;
            const float *blk = lut + (size_t)v * st * en;
            float t = blk[ix[0]];
            for (int s = 1; s < st; s++) t += blk[s * en + ix[s]];
            acc += t;
        }
        y[r] = acc * orc_f16_scale(scale[r]);
    }
}

/* VQ4P's int8 table, src/model.c:3979-4074 (vq_quant_range's scalar
 * loop; its NEON loop is documented there as value-for-value equal): per
 * block of ORC_VQ_LUT_BLK positions, scale = max|lut| / 127 and
 * q = lrintf(lut * (127 / max)) clamped to [-127, 127] (0 for an all-zero
 * block); lrintf rounds half to even in the default mode. */
void orc_vq_quant_lut(const float *lut, int nv, int stages, int entries,
                      int8_t *q, float *scale)
{
    const int st = stages, en = entries;
    for (int blk = 0; blk < (nv + ORC_VQ_LUT_BLK - 1) / ORC_VQ_LUT_BLK; blk++) {
        const int v0 = blk * ORC_VQ_LUT_BLK;
        const int v1 = v0 + ORC_VQ_LUT_BLK < nv ? v0 + ORC_VQ_LUT_BLK : nv;
        const size_t n = (size_t)(v1 - v0) * st * en;
        const float *src = lut + (size_t)v0 * st * en;
        int8_t *dst = q + (size_t)v0 * st * en;
        float mx = 0;
        for (size_t i = 0; i < n; i++) {
            const float f = fabsf(src[i]);
            if (f > mx) mx = f;
        }
        scale[blk] = mx / 127.0f;
        const float inv = mx > 0 ? 127.0f / mx : 0.0f;
        for (size_t i = 0; i < n; i++) {
            int t = (int)lrintf(src[i] * inv);
            if (t > 127) t = 127;
            else if (t < -127) t = -127;
            dst[i] = (int8_t)t;
        }
    }
}

/* VQ4P rows, src/model.c:4076-4114 (waste_vq_rows_p6, ORC_PORTABLE) and
 * src/simd_avx512.c:129-236 (vq_rows_p6_avx512, ORC_AVX512): four 6-bit
 * codes per (row, position) packed in three bytes (src/simd.h:73-76), the
 * stages' int8 entries summed exactly per block of ORC_VQ_LUT_BLK
 * positions (at most 4 * 32 * 127, so int16 holds it), then
 * acc += lscale[blk] * sum in block order: a product and a sum in the
 * portable C kernel, one fused multiply-add where the compiler contracts it
 * (the AVX-512 file, built with FMA available); y = acc * f16(scale). */
void orc_vq_rows_p6(float *y, const uint8_t *idx, const uint16_t *scale,
                    const int8_t *lut8, const float *lscale, int r_lo,
                    int r_hi, int nv, int order)
{
    const int en = 64;
    for (int r = r_lo; r < r_hi; r++) {
        float acc = 0.0f;
        const uint8_t *base = idx + (size_t)(r / 64) * nv * 64 * 3 + (size_t)(r % 64) * 3;
        for (int v0 = 0; v0 < nv; v0 += ORC_VQ_LUT_BLK) {
            const int v1 = v0 + ORC_VQ_LUT_BLK < nv ? v0 + ORC_VQ_LUT_BLK : nv;
            int16_t sum = 0;
            for (int v = v0; v < v1; v++) {
                const uint8_t *ix = base + (size_t)v * 64 * 3;
                const unsigned b0 = ix[0], b1 = ix[1], b2 = ix[2];
                const int8_t *T = lut8 + (size_t)v * 4 * en;
                sum = (int16_t)(sum + T[b0 & 0x3f] + T[en + (((b0 >> 6) | (b1 << 2)) & 0x3f)] +
                                T[2 * en + (((b1 >> 4) | (b2 << 4)) & 0x3f)] + T[3 * en + ((b2 >> 2) & 0x3f)]);
            }
            const float ls = lscale[v0 / ORC_VQ_LUT_BLK];
            acc = order == ORC_AVX512 ? fmaf(ls, (float)sum, acc) : acc + ls * (float)sum;
        }
        y[r] = acc * orc_f16_scale(scale[r]);
    }
}

/* The dequantised matrix in closed form (docs/FORMAT.md:204-214; the
 * Python oracle's Container.expert, tools/kimi_ref.py:240-273):
 *   W[r][8v+d] = (((0 + C0[i0][d]) + C1[i1][d]) + C2[i2][d]) * f16(scale[r])
 * with the books as the C loader converts them (subnormals flushed). */
void orc_dequant(float *W, const uint8_t *idx, const uint16_t *scale,
                 const float *books, int cb_base, int M, int N, int stages,
                 int entries, int vec_dim)
{
    const int nv = N / vec_dim;
    for (int r = 0; r < M; r++) {
        const float sc = orc_f16_scale(scale[r]);
        const uint8_t *base = idx + (size_t)(r / 64) * nv * 64 * stages + (size_t)(r % 64) * stages;
        for (int v = 0; v < nv; v++) {
            const uint8_t *ix = base + (size_t)v * 64 * stages;
            for (int d = 0; d < vec_dim; d++) {
                float a = 0.0f;
                for (int s = 0; s < stages; s++)
                    a += books[((size_t)(cb_base + s) * entries + ix[s]) * vec_dim + d];
                W[(size_t)r * N + (size_t)v * vec_dim + d] = a * sc;
            }
        }
    }
}

/* ---- trunk matvec --------------------------------------------------------
 * One row group of Q8G / Q4G / Q3G unpacked to int8, exactly as both
 * reference kernels unpack it (src/model.c:479-496; src/simd_avx512.c:37-68):
 * Q4G two signed nibbles per byte, low first, minus 8; Q3G the 3-bit code
 * at bit 3i (waste_q3_at, src/simd.h:101-106). */
static void unpack_group(const int8_t *row, int k, int g, int bits, int8_t *unp)
{
    if (bits == 3) {
        const uint8_t *p = (const uint8_t *)row;
        for (int i = 0; i < g; i++) {
            const long off = ((long)k * g + i) * 3;
            const int v = (p[off >> 3] >> (off & 7)) | (p[(off >> 3) + 1] << (8 - (off & 7)));
            unp[i] = (int8_t)((v & 7) - 4);
        }
    } else if (bits == 4) {
        const uint8_t *p4 = (const uint8_t *)row + (size_t)k * g / 2;
        for (int i = 0; i < g / 2; i++) {
            unp[2 * i] = (int8_t)((p4[i] & 0x0F) - 8);
            unp[2 * i + 1] = (int8_t)((p4[i] >> 4) - 8);
        }
    } else {
        memcpy(unp, row + (size_t)k * g, (size_t)g);
    }
}

/* _mm512_reduce_add_ps as GCC 11 defines it: 16 -> 8 (hi+lo) -> 4 (hi+lo)
 * -> pairs {0,2},{1,3} -> sum. */
static float reduce16(const float *a)
{
    float t3[8], t6[4];
    for (int i = 0; i < 8; i++) t3[i] = a[8 + i] + a[i];
    for (int i = 0; i < 4; i++) t6[i] = t3[4 + i] + t3[i];
    const float t80 = t6[0] + t6[2], t81 = t6[1] + t6[3];
    return t80 + t81;
}

/* mvq_rows_f32: quantized rows against fp32 activations.
 * ORC_PORTABLE: waste_mvq_rows_f32, src/model.c:423-519 (x86 branch):
 *   part = sum_i w*x sequential; acc += f16(ws)*part.
 * ORC_AVX512: mvq_rows_f32_avx512, src/simd_avx512.c:20-88: two 16-lane
 *   fma accumulators over 32-wide steps, GCC's reduce tree, a sequential
 *   tail, then acc += f16(ws)*part.  That file is built with -mavx512f,
 *   whose EVEX encoding includes scalar FMA, and GCC contracts the tail and
 *   the acc update into fused multiply-adds (four vfmadd..ss in the object
 *   built from it). */
void orc_mvq_rows(float *y, const int8_t *W, const uint16_t *ws,
                  const float *x, int r_lo, int r_hi, int in, int group,
                  int bits, size_t rowbytes, int order)
{
    const int g = group, ng = (in + g - 1) / g;
    int8_t *unp = (int8_t *)malloc((size_t)g);
    for (int o = r_lo; o < r_hi; o++) {
        const int8_t *row = W + (size_t)o * rowbytes;
        const uint16_t *s = ws + (size_t)o * ng;
        float acc = 0;
        for (int k = 0; k < ng; k++) {
            unpack_group(row, k, g, bits, unp);
            const float *xx = x + (size_t)k * g;
            const int lim = (k * g + g <= in) ? g : in - k * g;
            float part;
            int i = 0;
            if (order == ORC_AVX512) {
                float s0[16] = {0}, s1[16] = {0}, t[16];
                for (; i + 32 <= lim; i += 32)
                    for (int l = 0; l < 16; l++) {
                        s0[l] = fmaf((float)unp[i + l], xx[i + l], s0[l]);
                        s1[l] = fmaf((float)unp[i + 16 + l], xx[i + 16 + l], s1[l]);
                    }
                for (int l = 0; l < 16; l++) t[l] = s0[l] + s1[l];
                part = reduce16(t);
                for (; i < lim; i++) part = fmaf((float)unp[i], xx[i], part);
                acc = fmaf(orc_f16_scale(s[k]), part, acc);
            } else {
                part = 0;
                for (; i < lim; i++) part += (float)unp[i] * xx[i];
                acc += orc_f16_scale(s[k]) * part;
            }
        }
        y[o] = acc;
    }
    free(unp);
}

/* matvec / dotf, src/model.c:784-797 and 199-206 (x86): sequential. */
void orc_matvec_f32(float *y, const float *W, const float *x, int out, int in)
{
    for (int o = 0; o < out; o++) {
        const float *r = W + (size_t)o * in;
        float acc = 0;
        for (int i = 0; i < in; i++) acc += r[i] * x[i];
        y[o] = acc;
    }
}

/* mmq_rows, src/model.c:6964-6992: dequantize one row, w = (float)q * s,
 * then a sequential dotf against each token.  Y is [T][out]. */
void orc_mmq_rows(float *Y, const int8_t *W, const uint16_t *ws,
                  const float *X, int out, int in, int group, int bits,
                  size_t rowbytes, int T)
{
    const int g = group, ng = (in + g - 1) / g;
    float *row = (float *)malloc((size_t)ng * g * sizeof(float));
    int8_t *unp = (int8_t *)malloc((size_t)g);
    for (int o = 0; o < out; o++) {
        const int8_t *q = W + (size_t)o * rowbytes;
        const uint16_t *sc = ws + (size_t)o * ng;
        for (int k = 0; k < ng; k++) {
            const float s = orc_f16_scale(sc[k]);
            const int lim = (k * g + g <= in) ? g : in - k * g;
            unpack_group(q, k, g, bits, unp);
            for (int i = 0; i < lim; i++) row[k * g + i] = (float)unp[i] * s;
        }
        for (int t = 0; t < T; t++) {
            const float *xt = X + (size_t)t * in;
            float acc = 0;
            for (int i = 0; i < in; i++) acc += row[i] * xt[i];
            Y[(size_t)t * out + o] = acc;
        }
    }
    free(row);
    free(unp);
}

/* matmul_f32 / mm_rows, src/model.c:6852-6867. */
void orc_matmul_f32(float *Y, const float *W, const float *X, int out,
                    int in, int T)
{
    for (int o = 0; o < out; o++)
        for (int t = 0; t < T; t++) {
            const float *r = W + (size_t)o * in, *xt = X + (size_t)t * in;
            float acc = 0;
            for (int i = 0; i < in; i++) acc += r[i] * xt[i];
            Y[(size_t)t * out + o] = acc;
        }
}

/* ---- routing ------------------------------------------------------------- */

/* router_scores, src/model.c:5466-5486. */
void orc_router_scores(int score_func, const float *logit, float *score, int E)
{
    if (score_func == 2) {
        for (int e = 0; e < E; e++) {
            const float x = logit[e];
            const float sp = x > 30.0f ? x : log1pf(orc_expf(x));
            score[e] = sqrtf(sp);
        }
    } else if (score_func == 1) {
        float mx = -1e30f;
        for (int e = 0; e < E; e++) if (logit[e] > mx) mx = logit[e];
        float sum = 0;
        for (int e = 0; e < E; e++) { score[e] = orc_expf(logit[e] - mx); sum += score[e]; }
        for (int e = 0; e < E; e++) score[e] /= sum;
    } else {
        for (int e = 0; e < E; e++) score[e] = 1.0f / (1.0f + orc_expf(-logit[e]));
    }
}

/* One selection pass of src/model.c:5534-5547: the first e (ascending)
 * whose value is strictly greater than everything before it and than
 * -1e30, skipping taken ids.  -1 if none qualifies. */
static int pick(const float *v, int n, const unsigned char *taken, float floor_v)
{
    int best = -1;
    float bv = floor_v;
    for (int e = 0; e < n; e++) {
        if (taken[e]) continue;
        if (v[e] > bv) { bv = v[e]; best = e; }
    }
    return best;
}

/* Routing of one token, src/model.c:5496-5553 (selection, renorm, scale).
 *
 * Group-limited selection has no counterpart in the reference (no
 * n_group/topk_group anywhere in src/).  It follows DeepSeek-V3's published
 * noaux_tc router: a group's score is the sum of its two largest selection
 * values (score + bias), the topk_group best groups are kept by the same
 * strict-greater, lowest-index-first passes, and every expert outside them
 * is masked to -inf before the expert passes.  -inf, not 0, because a
 * biased score can be negative.  With n_group <= 1 the function is the
 * reference's plain top-k exactly. */
int orc_route(const orc_route_cfg *c, const float *logit, const float *bias,
              float *score_out, int *idx, float *w)
{
    const int E = c->n_experts, K = c->top_k;
    float *score = score_out ? score_out : (float *)malloc((size_t)E * sizeof(float));
    float *sel = (float *)malloc((size_t)E * sizeof(float));
    unsigned char *taken = (unsigned char *)calloc((size_t)E, 1);
    int rc = K;
    orc_router_scores(c->score_func, logit, score, E);
    for (int e = 0; e < E; e++) sel[e] = score[e] + (bias ? bias[e] : 0.0f);

    if (c->n_group > 1) {
        const int G = c->n_group, gs = E / G;
        float gsc[64];
        unsigned char gtaken[64] = {0}, keep[64] = {0};
        for (int g = 0; g < G; g++) {
            const float *p = sel + (size_t)g * gs;
            unsigned char tk[1024] = {0};
            const int a = pick(p, gs, tk, -INFINITY);
            if (a >= 0) tk[a] = 1;
            const int b = gs > 1 ? pick(p, gs, tk, -INFINITY) : -1;
            gsc[g] = (a >= 0 ? p[a] : -INFINITY) + (b >= 0 ? p[b] : (gs > 1 ? -INFINITY : 0.0f));
        }
        for (int j = 0; j < c->topk_group; j++) {
            const int g = pick(gsc, G, gtaken, -INFINITY);
            if (g < 0) break;
            gtaken[g] = 1;
            keep[g] = 1;
        }
        for (int e = 0; e < E; e++) if (!keep[e / gs]) sel[e] = -INFINITY;
    }

    for (int j = 0; j < K; j++) {
        const int best = pick(sel, E, taken, -1e30f);
        if (best < 0) { rc = -1; for (; j < K; j++) { idx[j] = -1; w[j] = 0.0f; } break; }
        taken[best] = 1;
        idx[j] = best;
        w[j] = score[best];
    }
    if (rc > 0) {
        if (c->renorm && K > 1) {
            float s = 0;
            for (int j = 0; j < K; j++) s += w[j];
            for (int j = 0; j < K; j++) w[j] /= (s + 1e-20f);
        }
        for (int j = 0; j < K; j++) w[j] *= c->routed_scale;
    }
    if (!score_out) free(score);
    free(sel);
    free(taken);
    return rc;
}

/* SwiGLU, waste_act_pair_range's plain branch, src/model.c:1231, 1263-1264:
 * g = silu(g) * u, silu(v) = v / (1 + expf(-v)). */
void orc_act_pair(float *g, const float *u, int n)
{
    for (int i = 0; i < n; i++) {
        const float v = g[i];
        g[i] = (v / (1.0f + orc_expf(-v))) * u[i];
    }
}

/* ---- records ------------------------------------------------------------- */

/* record_check, src/model.c:3645-3692, for a VQ3R layer whose experts are
 * inter x hidden (gate, up) and hidden x inter (down). */
int orc_record_check(const uint8_t *rec, size_t rec_bytes, int layer,
                     int expert, int inter, int hidden, int stages,
                     int n_books, int verify_crc)
{
    uint32_t magic, rec4k, go, uo, dof, co, crc;
    uint16_t lay, eid, cbid, lr;
    uint8_t fmt;
    if (rec_bytes < 48) return 1;
    memcpy(&magic, rec, 4); memcpy(&lay, rec + 4, 2); memcpy(&eid, rec + 6, 2);
    fmt = rec[8]; memcpy(&cbid, rec + 10, 2); memcpy(&lr, rec + 12, 2);
    memcpy(&rec4k, rec + 16, 4); memcpy(&go, rec + 20, 4); memcpy(&uo, rec + 24, 4);
    memcpy(&dof, rec + 28, 4); memcpy(&co, rec + 32, 4); memcpy(&crc, rec + 36, 4);
    if (magic != MAGIC_EXPERT) return 1;
    if (lay != (uint16_t)layer || eid != (uint16_t)expert) return 1;
    if ((size_t)rec4k * 4096u != rec_bytes) return 1;
    /* index_bits 6 (four stages of 64 entries) is VQ4P; one byte a stage
     * is VQ3R, or VQ2R in a two-stage container (src/model.c:3660-3666,
     * docs/FORMAT.md:180) */
    if (fmt != (stages == 4 ? WQ_VQ4P : stages == 2 ? WQ_VQ2R : WQ_VQ3R)) return 1;
    if (lr != 0) return 1;
    if ((long)cbid + 3L * stages > n_books) return 1;
    if (!(go == 48 && go < uo && uo < dof && dof < co && co <= rec_bytes)) return 1;
    const size_t scales = 2u * (size_t)(inter + inter + hidden);
    if (scales > rec_bytes - co) return 1;
    if (!verify_crc) return 0;
    const size_t payload = (size_t)co + scales - 48;
    if (orc_crc32(rec + 48, payload) != crc) return 2;
    return 0;
}

/* ---- the layer ------------------------------------------------------------ */

typedef struct { uint16_t cbid; uint32_t go, uo, dof, co; } rec_view;

static rec_view view(const uint8_t *rec)
{
    rec_view v;
    memcpy(&v.cbid, rec + 10, 2);
    memcpy(&v.go, rec + 20, 4); memcpy(&v.uo, rec + 24, 4);
    memcpy(&v.dof, rec + 28, 4); memcpy(&v.co, rec + 32, 4);
    return v;
}

/* One matrix's table (vq_build_lut, src/model.c:3864-3880): the fp32 LUT,
 * and for VQ4P its int8 shadow with one scale per block of ORC_VQ_LUT_BLK
 * positions; the rows through it (vq_apply, src/model.c:4152-4171): VQ4P
 * through the int8 table, VQ3R through the fp32 one.  VQ4P is the engine's
 * index_bits == 6, the one geometry of four stages of 64 entries. */
static int is_p6(const orc_moe *m) { return m->stages == 4 && m->entries == 64; }

typedef struct { float *lut; int8_t *q; float *qs; } orc_tab;

static void tab_alloc(orc_tab *t, size_t lut_sz)
{
    t->lut = (float *)malloc(lut_sz * sizeof(float));
    t->q = (int8_t *)malloc(lut_sz);
    t->qs = (float *)malloc((lut_sz / ORC_VQ_LUT_BLK + 2) * sizeof(float));
}

static void tab_free(orc_tab *t) { free(t->lut); free(t->q); free(t->qs); }

static void tab_build(const orc_moe *m, orc_tab *t, const float *x, int cb, int nv)
{
    orc_lutb(t->lut, m->booksT, x, cb, m->stages, m->entries, m->vec_dim, 0, nv, m->order);
    if (is_p6(m)) orc_vq_quant_lut(t->lut, nv, m->stages, m->entries, t->q, t->qs);
}

static void tab_rows(const orc_moe *m, float *y, const uint8_t *idx, const uint16_t *sc,
                     const orc_tab *t, int M, int nv)
{
    if (is_p6(m)) orc_vq_rows_p6(y, idx, sc, t->q, t->qs, 0, M, nv, m->order);
    else orc_vq_rows(y, idx, sc, t->lut, 0, M, nv, m->stages, m->entries);
}

/* matvec_t for one token (src/model.c:939-999 on the default trunk kernel):
 * F32 -> matvec; quantized -> mvq_rows_f32; absent -> zeros. */
static void tensor_mv(const orc_tensor *t, const float *x, float *y, int order)
{
    if (!t->rows) return;
    if (t->fmt == WQ_F32) { orc_matvec_f32(y, (const float *)t->q, x, t->rows, t->cols); return; }
    orc_mvq_rows(y, (const int8_t *)t->q, t->qs, x, 0, t->rows, t->cols, t->group,
                 t->fmt == WQ_Q8G ? 8 : t->fmt == WQ_Q4G ? 4 : 3, t->rowbytes, order);
}

/* waste_matmul_t (src/model.c:7001-7030) for T tokens. */
static void tensor_mm(const orc_tensor *t, const float *X, float *Y, int T)
{
    if (!t->rows) return;
    if (t->fmt == WQ_F32) { orc_matmul_f32(Y, (const float *)t->q, X, t->rows, t->cols, T); return; }
    orc_mmq_rows(Y, (const int8_t *)t->q, t->qs, X, t->rows, t->cols, t->group,
                 t->fmt == WQ_Q8G ? 8 : t->fmt == WQ_Q4G ? 4 : 3, t->rowbytes, T);
}

static orc_route_cfg route_cfg(const orc_moe *m)
{
    orc_route_cfg c = { m->n_experts, m->top_k, m->score_func, m->renorm,
                        m->routed_scale, m->n_group, m->topk_group };
    return c;
}

/* moe_layer's serial path, src/model.c:5488-5553 and 5876-5939, with no
 * latent projection (none of the configured shapes has one).  The routed
 * sum is built in `out` (ysum aliases out), then the shared expert's
 * output is added: out[i] += tmp[i], tmp = 0 when there is none. */
int orc_moe_layer(const orc_moe *m, const float *x, float *out, int *idx_o,
                  float *w_o, float *logits_o)
{
    const int E = m->n_experts, K = m->top_k, H = m->hidden, I = m->moe_inter;
    const int st = m->stages, en = m->entries, vd = m->vec_dim;
    float *logit = (float *)calloc((size_t)E, sizeof(float));
    int idx[64];
    float w[64];
    tensor_mv(&m->router, x, logit, m->order);
    orc_route_cfg rc = route_cfg(m);
    const int nsel = orc_route(&rc, logit, m->bias, NULL, idx, w);
    if (logits_o) memcpy(logits_o, logit, (size_t)E * sizeof(float));
    if (idx_o) memcpy(idx_o, idx, (size_t)K * sizeof(int));
    if (w_o) memcpy(w_o, w, (size_t)K * sizeof(float));

    memset(out, 0, (size_t)H * sizeof(float));
    const size_t lut_sz = (size_t)((H > I ? H : I) / vd) * st * en;
    orc_tab tg, tu, td;
    tab_alloc(&tg, lut_sz); tab_alloc(&tu, lut_sz); tab_alloc(&td, lut_sz);
    float *ga = (float *)malloc((size_t)I * sizeof(float));
    float *ub = (float *)malloc((size_t)I * sizeof(float));
    float *acc = (float *)malloc((size_t)H * sizeof(float));
    int lut_ready = 0, rcode = 0;
    for (int j = 0; j < K && nsel > 0; j++) {
        const uint8_t *rec = m->recs[idx[j]];
        if (!rec) { rcode = -2; break; }
        const rec_view h = view(rec);
        const uint16_t *sc = (const uint16_t *)(rec + h.co);
        if (!lut_ready) {
            tab_build(m, &tg, x, h.cbid + 0 * st, H / vd);
            tab_build(m, &tu, x, h.cbid + 1 * st, H / vd);
            lut_ready = 1;
        }
        tab_rows(m, ga, rec + h.go, sc, &tg, I, H / vd);
        tab_rows(m, ub, rec + h.uo, sc + I, &tu, I, H / vd);
        orc_act_pair(ga, ub, I);
        tab_build(m, &td, ga, h.cbid + 2 * st, I / vd);
        tab_rows(m, acc, rec + h.dof, sc + 2 * I, &td, H, I / vd);
        const float wj = w[j];
        for (int i = 0; i < H; i++) out[i] += wj * acc[i];
    }
    /* ffn(shared), src/model.c:5391-5402, 5934-5938 */
    const int SI = I * (m->n_shared ? m->n_shared : 1);
    float *a = (float *)calloc((size_t)SI, sizeof(float));
    float *b = (float *)calloc((size_t)SI, sizeof(float));
    float *tmp = (float *)calloc((size_t)H, sizeof(float));
    tensor_mv(&m->sh_gate, x, a, m->order);
    tensor_mv(&m->sh_up, x, b, m->order);
    orc_act_pair(a, b, SI);
    tensor_mv(&m->sh_down, a, tmp, m->order);
    for (int i = 0; i < H; i++) out[i] += tmp[i];
    free(a); free(b); free(tmp);
    tab_free(&tg); tab_free(&tu); tab_free(&td); free(ga); free(ub); free(acc); free(logit);
    return nsel < 0 ? -1 : rcode;
}

/* moe_chunk, src/model.c:7110-7285: routing per token, distinct experts
 * in ascending id order, per-token gate/up tables, per (expert, token)
 * apply skipping a zero weight, dst += w*acc in that order; the shared
 * expert through waste_matmul_t on the whole chunk. */
int orc_moe_chunk(const orc_moe *m, const float *x, int T, float *out,
                  int *idx_o, float *w_o)
{
    const int E = m->n_experts, K = m->top_k, H = m->hidden, I = m->moe_inter;
    const int st = m->stages, en = m->entries, vd = m->vec_dim;
    int *route = (int *)malloc((size_t)T * K * sizeof(int));
    float *rw = (float *)malloc((size_t)T * K * sizeof(float));
    float *logit = (float *)calloc((size_t)E, sizeof(float));
    orc_route_cfg rc = route_cfg(m);
    int bad = 0;
    for (int t = 0; t < T; t++) {
        memset(logit, 0, (size_t)E * sizeof(float));
        tensor_mv(&m->router, x + (size_t)t * H, logit, m->order);
        if (orc_route(&rc, logit, m->bias, NULL, route + (size_t)t * K, rw + (size_t)t * K) < 0) bad = 1;
    }
    if (idx_o) memcpy(idx_o, route, (size_t)T * K * sizeof(int));
    if (w_o) memcpy(w_o, rw, (size_t)T * K * sizeof(float));
    memset(out, 0, (size_t)T * H * sizeof(float));

    const size_t lut_sz = (size_t)((H > I ? H : I) / vd) * st * en;
    orc_tab *tgu = (orc_tab *)malloc((size_t)T * 2 * sizeof(orc_tab)), td;
    for (int q = 0; q < 2 * T; q++) tab_alloc(&tgu[q], lut_sz);
    tab_alloc(&td, lut_sz);
    float *ga = (float *)malloc((size_t)I * sizeof(float));
    float *ub = (float *)malloc((size_t)I * sizeof(float));
    float *acc = (float *)malloc((size_t)H * sizeof(float));
    int lut_ready = 0, rcode = bad ? -1 : 0;
    for (int e = 0; e < E && !bad; e++) {
        int used = 0;
        for (int i = 0; i < T * K; i++) if (route[i] == e) { used = 1; break; }
        if (!used) continue;
        const uint8_t *rec = m->recs[e];
        if (!rec) { rcode = -2; break; }
        const rec_view h = view(rec);
        const uint16_t *s16 = (const uint16_t *)(rec + h.co);
        if (!lut_ready) {
            for (int t = 0; t < T; t++) {
                tab_build(m, &tgu[2 * t], x + (size_t)t * H, h.cbid + 0 * st, H / vd);
                tab_build(m, &tgu[2 * t + 1], x + (size_t)t * H, h.cbid + 1 * st, H / vd);
            }
            lut_ready = 1;
        }
        for (int t = 0; t < T; t++) {
            float wj = 0;
            for (int j = 0; j < K; j++)
                if (route[(size_t)t * K + j] == e) { wj = rw[(size_t)t * K + j]; break; }
            if (wj == 0.0f) continue;
            tab_rows(m, ga, rec + h.go, s16, &tgu[2 * t], I, H / vd);
            tab_rows(m, ub, rec + h.uo, s16 + I, &tgu[2 * t + 1], I, H / vd);
            orc_act_pair(ga, ub, I);
            tab_build(m, &td, ga, h.cbid + 2 * st, I / vd);
            tab_rows(m, acc, rec + h.dof, s16 + 2 * I, &td, H, I / vd);
            float *dst = out + (size_t)t * H;
            for (int i = 0; i < H; i++) dst[i] += wj * acc[i];
        }
    }
    const int SI = I * (m->n_shared ? m->n_shared : 1);
    float *sa = (float *)calloc((size_t)T * SI, sizeof(float));
    float *sb = (float *)calloc((size_t)T * SI, sizeof(float));
    float *sh = (float *)calloc((size_t)T * H, sizeof(float));
    tensor_mm(&m->sh_gate, x, sa, T);
    tensor_mm(&m->sh_up, x, sb, T);
    orc_act_pair(sa, sb, T * SI);
    tensor_mm(&m->sh_down, sa, sh, T);
    for (size_t i = 0; i < (size_t)T * H; i++) out[i] += sh[i];
    free(sa); free(sb); free(sh);
    for (int q = 0; q < 2 * T; q++) tab_free(&tgu[q]);
    free(tgu); tab_free(&td);
    free(ga); free(ub); free(acc); free(logit); free(route); free(rw);
    return rcode;
}

/* The expert part of the layer with the routing given: moe_layer's serial
 * loop (chunk == 0: one token, selection order, decode shared expert
 * through matvec_t) or moe_chunk's (chunk == 1: ascending expert order,
 * zero weights skipped, shared expert through waste_matmul_t).  Lets a
 * device result be compared on the device's own routing, which is checked
 * bit for bit separately. */
int orc_moe_apply(const orc_moe *m, const float *x, int T, const int *idx,
                  const float *w, int chunk, float *out)
{
    const int K = m->top_k, H = m->hidden, I = m->moe_inter;
    const int st = m->stages, en = m->entries, vd = m->vec_dim, E = m->n_experts;
    const size_t lut_sz = (size_t)((H > I ? H : I) / vd) * st * en;
    orc_tab tg, tu, td;
    tab_alloc(&tg, lut_sz); tab_alloc(&tu, lut_sz); tab_alloc(&td, lut_sz);
    float *ga = (float *)malloc((size_t)I * sizeof(float));
    float *ub = (float *)malloc((size_t)I * sizeof(float));
    float *acc = (float *)malloc((size_t)H * sizeof(float));
    int rc = 0;
    memset(out, 0, (size_t)T * H * sizeof(float));
    for (int t = 0; t < T; t++) {
        const float *xt = x + (size_t)t * H;
        int order[64];
        for (int j = 0; j < K; j++) order[j] = j;
        if (chunk)       /* ascending expert id */
            for (int a = 1; a < K; a++)
                for (int b = a; b > 0 && idx[t * K + order[b]] < idx[t * K + order[b - 1]]; b--) {
                    const int tmp = order[b]; order[b] = order[b - 1]; order[b - 1] = tmp;
                }
        int lut_ready = 0;
        for (int jj = 0; jj < K; jj++) {
            const int j = order[jj], e = idx[t * K + j];
            const float wj = w[t * K + j];
            if (chunk && wj == 0.0f) continue;
            if (e < 0 || e >= E || !m->recs[e]) { rc = -2; continue; }
            const uint8_t *rec = m->recs[e];
            const rec_view h = view(rec);
            const uint16_t *sc = (const uint16_t *)(rec + h.co);
            if (!lut_ready) {
                tab_build(m, &tg, xt, h.cbid, H / vd);
                tab_build(m, &tu, xt, h.cbid + st, H / vd);
                lut_ready = 1;
            }
            tab_rows(m, ga, rec + h.go, sc, &tg, I, H / vd);
            tab_rows(m, ub, rec + h.uo, sc + I, &tu, I, H / vd);
            orc_act_pair(ga, ub, I);
            tab_build(m, &td, ga, h.cbid + 2 * st, I / vd);
            tab_rows(m, acc, rec + h.dof, sc + 2 * I, &td, H, I / vd);
            float *dst = out + (size_t)t * H;
            for (int i = 0; i < H; i++) dst[i] += wj * acc[i];
        }
    }
    const int SI = I * (m->n_shared ? m->n_shared : 1);
    float *a = (float *)calloc((size_t)T * SI, sizeof(float));
    float *b = (float *)calloc((size_t)T * SI, sizeof(float));
    float *sh = (float *)calloc((size_t)T * H, sizeof(float));
    if (chunk) {
        tensor_mm(&m->sh_gate, x, a, T);
        tensor_mm(&m->sh_up, x, b, T);
        orc_act_pair(a, b, T * SI);
        tensor_mm(&m->sh_down, a, sh, T);
    } else {
        for (int t = 0; t < T; t++) {
            tensor_mv(&m->sh_gate, x + (size_t)t * H, a + (size_t)t * SI, m->order);
            tensor_mv(&m->sh_up, x + (size_t)t * H, b + (size_t)t * SI, m->order);
            orc_act_pair(a + (size_t)t * SI, b + (size_t)t * SI, SI);
            tensor_mv(&m->sh_down, a + (size_t)t * SI, sh + (size_t)t * H, m->order);
        }
    }
    for (size_t i = 0; i < (size_t)T * H; i++) out[i] += sh[i];
    free(a); free(b); free(sh);
    tab_free(&tg); tab_free(&tu); tab_free(&td); free(ga); free(ub); free(acc);
    return rc;
}

/* Router logits for T tokens (matvec_t per token). */
void orc_router_logits(const orc_moe *m, const float *x, int T, float *logits)
{
    for (int t = 0; t < T; t++) {
        memset(logits + (size_t)t * m->n_experts, 0, (size_t)m->n_experts * sizeof(float));
        tensor_mv(&m->router, x + (size_t)t * m->hidden, logits + (size_t)t * m->n_experts, m->order);
    }
}

/* ---- expert cache policy ----------------------------------------------------
 * src/ecache.c: victim choice (ec_victim, 454-485), claims (ec_claim
 * 510-526, ec_claim_spec 490-508), the hint pipeline (ec_issue_next
 * 538-576, waste_ecache_hint 599-616), speculative reads
 * (waste_ecache_prefetch 578-597) and the demand path
 * (waste_ecache_get 693-766).  Test infrastructure. */
enum { OE_EMPTY = 0, OE_READY, OE_INFLIGHT };
typedef struct { int32_t key; uint8_t state, fresh; uint32_t hits; uint64_t last, pin; } orc_eslot;
struct orc_ecache {
    orc_eslot *slot;
    int32_t *where;                  /* key -> slot, direct: 128 x 1024     */
    int n_slots, depth, io, lru;
    uint64_t clock, hits, misses, evictions, prefetched, spec_issued, reads, pf_gen;
    uint32_t rng;
    int pf_ids[64], pf_layer, pf_n, pf_issued, last_used;
    int held[64], n_held, fill_cursor;
};
#define OE_KEY(l, e) (((l) << 16) | (e))
#define OE_IDX(k) (((k) >> 16) * 1024 + ((k) & 0xffff))

orc_ecache *orc_ecache_new(int n_slots, int depth, int readahead, int lru)
{
    orc_ecache *c = (orc_ecache *)calloc(1, sizeof *c);
    c->n_slots = n_slots;
    c->slot = (orc_eslot *)calloc((size_t)(n_slots > 0 ? n_slots : 1), sizeof *c->slot);
    c->where = (int32_t *)malloc(128 * 1024 * sizeof(int32_t));
    for (int i = 0; i < 128 * 1024; i++) c->where[i] = -1;
    for (int i = 0; i < n_slots; i++) c->slot[i].key = -1;
    if (depth < 1) depth = 1;
    if (depth > n_slots / 4) depth = n_slots / 4;
    c->io = readahead && depth >= 1;
    c->depth = depth;
    c->lru = lru;
    c->rng = 0x9e3779b9u;
    c->pf_gen = 1;
    c->last_used = -1;
    return c;
}

void orc_ecache_free(orc_ecache *c)
{
    if (!c) return;
    free(c->slot);
    free(c->where);
    free(c);
}

static int oe_lookup(const orc_ecache *c, int32_t key) { return c->where[OE_IDX(key)]; }

static int oe_is_held(const orc_ecache *c, int i)
{
    for (int k = 0; k < c->n_held; k++)
        if (c->held[k] == i) return 1;
    return 0;
}

static int oe_pinned(const orc_ecache *c, int i)
{
    return c->slot[i].state == OE_INFLIGHT || c->slot[i].pin == c->pf_gen || i == c->last_used ||
           oe_is_held(c, i);
}

static int oe_victim(orc_ecache *c)
{
    for (int i = 0; i < c->n_slots; i++)
        if (c->slot[i].state == OE_EMPTY) return i;
    int best = -1;
    uint32_t bh = 0;
    uint64_t bl = 0;
    for (int s = 0; s < 16; s++) {
        c->rng = c->rng * 1664525u + 1013904223u;
        const int i = (int)(c->rng % (uint32_t)c->n_slots);
        if (oe_pinned(c, i)) continue;
        const orc_eslot *sl = &c->slot[i];
        const int better = c->lru ? (best < 0 || sl->last < bl)
                                  : (best < 0 || sl->hits < bh || (sl->hits == bh && sl->last < bl));
        if (better) { best = i; bh = sl->hits; bl = sl->last; }
    }
    if (best < 0)
        for (int i = 0; i < c->n_slots; i++)
            if (!oe_pinned(c, i)) { best = i; break; }
    return best;
}

static void oe_take(orc_ecache *c, int vi, int32_t key)
{
    if (c->slot[vi].key >= 0) { c->where[OE_IDX(c->slot[vi].key)] = -1; c->evictions++; }
    c->slot[vi].key = key;
    c->where[OE_IDX(key)] = vi;
    c->slot[vi].state = OE_INFLIGHT;
    c->slot[vi].hits = 1;
    c->slot[vi].last = c->clock;
    c->reads++;
}

static void oe_issue_next(orc_ecache *c)
{
    if (!c->io) return;
    while (c->pf_issued < c->pf_n) {
        const int32_t key = OE_KEY(c->pf_layer, c->pf_ids[c->pf_issued++]);
        const int si = oe_lookup(c, key);
        if (si >= 0) { c->slot[si].pin = c->pf_gen; continue; }
        const int vi = oe_victim(c);
        if (vi < 0) { c->pf_issued--; return; }
        oe_take(c, vi, key);
        c->slot[vi].fresh = 1;
        c->slot[vi].pin = c->pf_gen;
        c->misses++;
        c->prefetched++;
        return;
    }
}

void orc_ecache_hint(orc_ecache *c, int layer, const int *ids, int n)
{
    if (!c->io || c->n_slots <= 0 || n <= 0) return;
    c->pf_gen++;
    c->pf_layer = layer;
    c->pf_n = n > 64 ? 64 : n;
    if (c->pf_n > c->n_slots / 4) c->pf_n = c->n_slots / 4;
    for (int i = 0; i < c->pf_n; i++) c->pf_ids[i] = ids[i];
    c->pf_issued = 0;
    for (int d = 0; d < c->depth; d++) oe_issue_next(c);
}

void orc_ecache_prefetch(orc_ecache *c, int layer, const int *ids, int n)
{
    if (!c->io || c->n_slots <= 0 || n <= 0) return;
    for (int i = 0; i < n; i++) {
        if (ids[i] < 0) continue;
        const int32_t key = OE_KEY(layer, ids[i]);
        if (oe_lookup(c, key) >= 0) continue;
        const int vi = oe_victim(c);
        if (vi < 0) break;
        oe_take(c, vi, key);
        c->slot[vi].fresh = 0;
        c->slot[vi].pin = 0;
        c->spec_issued++;
    }
}

int orc_ecache_get(orc_ecache *c, int layer, int expert)
{
    const int32_t key = OE_KEY(layer, expert);
    c->clock++;
    c->last_used = -1;
    for (int i = 0; i < c->n_slots; i++)                   /* reads issued so far are done */
        if (c->slot[i].state == OE_INFLIGHT) c->slot[i].state = OE_READY;
    if (c->n_slots <= 0) { c->misses++; c->reads++; return -1; }
    const int si = oe_lookup(c, key);
    if (si >= 0) {
        if (c->slot[si].fresh) c->slot[si].fresh = 0;
        else { c->hits++; c->slot[si].hits++; }
        c->slot[si].last = c->clock;
        c->last_used = si;
        oe_issue_next(c);
        return si;
    }
    const int vi = oe_victim(c);
    if (vi < 0) return -1;
    oe_take(c, vi, key);
    c->slot[vi].fresh = 0;
    c->slot[vi].pin = 0;
    c->misses++;
    c->slot[vi].state = OE_READY;
    c->last_used = vi;
    oe_issue_next(c);
    return vi;
}

/* src/ecache.c:768-798 */
int orc_ecache_hold(orc_ecache *c, int layer, int expert)
{
    if (c->n_slots <= 0 || c->n_held >= 64) return -1;
    const int si = orc_ecache_get(c, layer, expert);
    if (si < 0) return -1;
    if (c->last_used >= 0) {
        if (!oe_is_held(c, c->last_used)) c->held[c->n_held++] = c->last_used;
        c->last_used = -1;
    }
    return si;
}

void orc_ecache_release(orc_ecache *c) { c->n_held = 0; }

/* src/ecache.c:635-678: an empty slot by a monotone cursor, nothing
 * evicted, no hit or miss counted; needs read-ahead. */
int orc_ecache_admit(orc_ecache *c, int layer, int expert)
{
    if (c->n_slots <= 0 || !c->io) return 0;
    const int32_t key = OE_KEY(layer, expert);
    if (oe_lookup(c, key) >= 0) return 0;
    int si = -1;
    while (c->fill_cursor < c->n_slots) {
        const int i = c->fill_cursor++;
        if (c->slot[i].key < 0) { si = i; break; }
    }
    if (si < 0) return 0;
    c->slot[si].key = key;
    c->where[OE_IDX(key)] = si;
    c->slot[si].state = OE_READY;
    c->slot[si].fresh = 0;
    c->slot[si].pin = 0;
    c->slot[si].hits = 1;
    c->slot[si].last = c->clock;
    c->reads++;
    return 1;
}

/* src/ecache.c:618-633: READY only */
void orc_ecache_resident_mask(const orc_ecache *c, int layer, int n, uint8_t *out)
{
    for (int e = 0; e < n; e++) {
        const int si = c->n_slots > 0 ? oe_lookup(c, OE_KEY(layer, e)) : -1;
        out[e] = si >= 0 && c->slot[si].state == OE_READY;
    }
}

/* src/model.c:5419-5449 */
int orc_predict_next(int score_func, int E, const float *logit, const float *bias, int n, int *out)
{
    if (n <= 0 || E <= 0) return 0;
    if (n > E) n = E;
    float *p = (float *)malloc((size_t)E * sizeof *p);
    orc_router_scores(score_func, logit, p, E);
    for (int e = 0; e < E; e++) p[e] += bias ? bias[e] : 0.0f;
    for (int j = 0; j < n; j++) {
        int best = -1;
        float bv = -1e30f;
        for (int e = 0; e < E; e++) {
            int taken = 0;
            for (int q = 0; q < j; q++)
                if (out[q] == e) { taken = 1; break; }
            if (!taken && p[e] > bv) { bv = p[e]; best = e; }
        }
        out[j] = best;
    }
    free(p);
    return n;
}

void orc_ecache_stats(const orc_ecache *c, uint64_t out[6])
{
    out[0] = c->hits; out[1] = c->misses; out[2] = c->evictions;
    out[3] = c->prefetched; out[4] = c->spec_issued; out[5] = c->reads;
}
