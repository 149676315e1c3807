/* SPDX-License-Identifier: Apache-2.0 */
/*
 * synth.c — seeded codebooks and the host half of the synthetic record
 * generator (see include/waste_hip_synth.h).
 *
 * Codebooks follow the converter's recipe in kind, not in its sampler:
 * residual k-means, one book per stage fitted on the running residual
 * (tools/convert.py:745-763), here on 16,384 row-normalised Gaussian
 * vectors per kind, seeded, Lloyd iterations with the encoder's own
 * nearest-entry rule (squared L2, first minimum; src/vq.c:50-96).
 */
#include "waste_hip.h"
#include "waste_hip_synth.h"
#include "../hip/launch.h"

#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define NTRAIN 16384
#define ITERS 6

static uint64_t splitmix(uint64_t *s)
{
    uint64_t z = (*s += 0x9E3779B97F4A7C15ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

static double unif(uint64_t *s) { return ((splitmix(s) >> 11) + 0.5) * (1.0 / 9007199254740992.0); }

static float gauss(uint64_t *s)
{
    const double u1 = unif(s), u2 = unif(s);
    return (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
}

static uint16_t f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    int e = (int)((x >> 23) & 0xff) - 127 + 15;
    uint32_t m = x & 0x7fffffu;
    if (((x >> 23) & 0xff) == 0xff) return (uint16_t)(sign | 0x7c00u | (m ? 0x200u : 0));
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        m |= 0x800000u;
        const int shift = 14 - e;
        uint32_t h = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)e << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h++;
    return (uint16_t)(sign | h);
}

static float f16_book(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1f, mn = h & 0x3ff;
    const uint32_t b = e ? (sign | ((e + 112u) << 23) | (mn << 13)) : sign;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

static int nearest(const float *v, const float *C)
{
    int best = 0;
    float bestd = INFINITY;
    for (int c = 0; c < 256; c++) {
        float d = 0;
        for (int j = 0; j < 8; j++) { const float t = v[j] - C[c * 8 + j]; d += t * t; }
        if (d < bestd) { bestd = d; best = c; }
    }
    return best;
}

/* Three residual stages for one kind, rows of width `width`. */
static void train_kind(uint64_t seed, int width, uint16_t *out /* [3][256][8] */)
{
    float *X = (float *)malloc((size_t)NTRAIN * 8 * sizeof(float));
    float *row = (float *)malloc((size_t)width * sizeof(float));
    int *asg = (int *)malloc(NTRAIN * sizeof(int));
    double *sum = (double *)malloc(256 * 8 * sizeof(double));
    int *cnt = (int *)malloc(256 * sizeof(int));
    float C[256 * 8];
    uint64_t s = seed;
    int n = 0;
    while (n < NTRAIN) {
        float amax = 0;
        for (int i = 0; i < width; i++) { row[i] = gauss(&s); if (fabsf(row[i]) > amax) amax = fabsf(row[i]); }
        for (int v = 0; v < width / 8 && n < NTRAIN; v++, n++)
            for (int j = 0; j < 8; j++) X[n * 8 + j] = row[v * 8 + j] / amax;
    }
    for (int st = 0; st < 3; st++) {
        for (int c = 0; c < 256; c++) {                 /* seeded init from the data */
            const int pick = (int)(splitmix(&s) % NTRAIN);
            memcpy(C + c * 8, X + pick * 8, 8 * sizeof(float));
        }
        for (int it = 0; it < ITERS; it++) {
            #pragma omp parallel for schedule(static)
            for (int i = 0; i < NTRAIN; i++) asg[i] = nearest(X + i * 8, C);
            memset(sum, 0, 256 * 8 * sizeof(double));
            memset(cnt, 0, 256 * sizeof(int));
            for (int i = 0; i < NTRAIN; i++) {
                cnt[asg[i]]++;
                for (int j = 0; j < 8; j++) sum[asg[i] * 8 + j] += X[i * 8 + j];
            }
            for (int c = 0; c < 256; c++)
                if (cnt[c]) for (int j = 0; j < 8; j++) C[c * 8 + j] = (float)(sum[c * 8 + j] / cnt[c]);
        }
        for (int i = 0; i < 256 * 8; i++) out[st * 256 * 8 + i] = f32_to_f16(C[i]);
        /* residual against the book as stored (fp16, as decoded) */
        float Cq[256 * 8];
        for (int i = 0; i < 256 * 8; i++) Cq[i] = f16_book(out[st * 256 * 8 + i]);
        for (int i = 0; i < NTRAIN; i++) {
            const int a = nearest(X + i * 8, Cq);
            for (int j = 0; j < 8; j++) X[i * 8 + j] -= Cq[a * 8 + j];
        }
    }
    free(X); free(row); free(asg); free(sum); free(cnt);
}

size_t waste_hip_record_bytes(int hidden, int moe_inter)
{
    const size_t gu = (size_t)moe_inter * (hidden / 8) * 3, d = (size_t)hidden * (moe_inter / 8) * 3;
    const size_t end = 48 + 2 * gu + d + 2 * (size_t)(2 * moe_inter + hidden);
    return (end + 4095) / 4096 * 4096;
}

int waste_hip_synth_codebooks(uint64_t seed, int hidden, int moe_inter, uint16_t *books_f16)
{
    if (!books_f16 || hidden <= 0 || hidden % 8 || moe_inter <= 0 || moe_inter % 8)
        return WASTE_HIP_EINVAL;
    train_kind(seed * 3 + 1, hidden, books_f16);
    train_kind(seed * 3 + 2, hidden, books_f16 + 3 * 256 * 8);
    train_kind(seed * 3 + 3, moe_inter, books_f16 + 6 * 256 * 8);
    return 0;
}

/* device half in synth.hip */
int whip_synth_records(uint64_t seed, int layer, int H, int I, int cb_base, const float *books,
                       int e0, int n, uint8_t *dst, size_t rec_bytes, float std, float *raw,
                       hipStream_t s);

int waste_hip_synth_records(uint64_t seed, int layer, int hidden, int moe_inter, int cb_base,
                            const uint16_t *books_f16, int e0, int n, void *dst, float std,
                            float *raw, void *stream)
{
    if (!books_f16 || !dst || n <= 0 || e0 < 0 || hidden % 64 || moe_inter % 64 || hidden <= 0 ||
        moe_inter <= 0)
        return WASTE_HIP_EINVAL;
    float *b = (float *)malloc(9 * 256 * 8 * sizeof(float));
    if (!b) return WASTE_HIP_ENOMEM;
    for (int i = 0; i < 9 * 256 * 8; i++) b[i] = f16_book(books_f16[i]);
    float *d = NULL;
    int rc = 0;
    if (hipMalloc((void **)&d, 9 * 256 * 8 * sizeof(float)) != hipSuccess) rc = WASTE_HIP_ENOMEM;
    if (!rc && hipMemcpy(d, b, 9 * 256 * 8 * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)
        rc = WASTE_HIP_EDEVICE;
    if (!rc && whip_synth_records(seed, layer, hidden, moe_inter, cb_base, d, e0, n, (uint8_t *)dst,
                                  waste_hip_record_bytes(hidden, moe_inter), std, raw,
                                  (hipStream_t)stream) != 0)
        rc = WASTE_HIP_EDEVICE;
    if (!rc && hipStreamSynchronize((hipStream_t)stream) != hipSuccess) rc = WASTE_HIP_EDEVICE;
    if (d) hipFree(d);
    free(b);
    return rc;
}
