/* SPDX-License-Identifier: Apache-2.0 */
/*
 * orc_cpu.c — the timed CPU baseline: the reference's x86 MoE decode path
 * at full speed.  TEST INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg and
 * the tests that check it agrees with oracle.c).
 *
 * What runs is what the reference runs on an AVX-512 host
 * (waste_backend_init, src/backend.c:188-191):
 *   - LUT build: 16-lane FMA chains over 64-entry blocks
 *     (lutb_range_avx512, src/simd_avx512.c:90-123);
 *   - VQ3R apply: the scalar gather with the 8-row word-load unroll, rows
 *     in 128-row chunks (vq_rows, src/model.c:3909-3977; VQ_TILE*VQ_SUPER);
 *   - trunk matvec: two 16-lane FMA accumulators per group
 *     (mvq_rows_f32_avx512, src/simd_avx512.c:20-88), or sequential dotf
 *     for an F32 router (src/model.c:199-206, 784-797);
 *   - ranges split over a fork-join pool (OpenMP here, the reference's own
 *     pool there: src/threads.h:325-341), so results do not depend on the
 *     thread count.
 * On a host without AVX-512 the same bits come from oracle.c's scalar
 * restatement of that order, and orc_cpu_isa() says so.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>
#if defined(__x86_64__)
#include <immintrin.h>
#define ORC_X86 1
#define AVX512_FN __attribute__((target("avx512f,avx512bw")))
#endif

static int have_avx512(void)
{
#if ORC_X86
    static int v = -1;
    if (v < 0) {
        __builtin_cpu_init();
        v = __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw");
    }
    return v;
#else
    return 0;
#endif
}

int orc_cpu_isa(void) { return have_avx512() ? 2 : 0; }

static inline float f16s(uint16_t h) { return orc_f16_scale(h); }

#if ORC_X86
AVX512_FN static void lutb_avx512(float *lut, const float *booksT, const float *x,
                                  int cb_base, int st, int en, int vd, int v_lo, int v_hi)
{
        for (int v = v_lo; v < v_hi; v++) {
            const float *xv = x + (size_t)v * vd;
            for (int s = 0; s < st; s++) {
                const float *CT = booksT + (size_t)(cb_base + s) * en * vd;
                float *dst = lut + ((size_t)v * st + s) * en;
                for (int c = 0; c < en; c += 64) {
                    __m512 a0 = _mm512_setzero_ps(), a1 = _mm512_setzero_ps(),
                           a2 = _mm512_setzero_ps(), a3 = _mm512_setzero_ps();
                    for (int d = 0; d < vd; d++) {
                        const __m512 xd = _mm512_set1_ps(xv[d]);
                        const float *cr = CT + (size_t)d * en + c;
                        a0 = _mm512_fmadd_ps(xd, _mm512_loadu_ps(cr), a0);
                        a1 = _mm512_fmadd_ps(xd, _mm512_loadu_ps(cr + 16), a1);
                        a2 = _mm512_fmadd_ps(xd, _mm512_loadu_ps(cr + 32), a2);
                        a3 = _mm512_fmadd_ps(xd, _mm512_loadu_ps(cr + 48), a3);
                    }
                    _mm512_storeu_ps(dst + c, a0);
                    _mm512_storeu_ps(dst + c + 16, a1);
                    _mm512_storeu_ps(dst + c + 32, a2);
                    _mm512_storeu_ps(dst + c + 48, a3);
                }
            }
        }
}
#endif

/* LUT build over [v_lo, v_hi). */
static void lutb_fast(float *lut, const float *booksT, const float *x, int cb_base,
                      int st, int en, int vd, int v_lo, int v_hi)
{
#if ORC_X86
    if (have_avx512() && en % 64 == 0) {
        lutb_avx512(lut, booksT, x, cb_base, st, en, vd, v_lo, v_hi);
        return;
    }
#endif
    orc_lutb(lut, booksT, x, cb_base, st, en, vd, v_lo, v_hi, ORC_AVX512);
}

/* The scalar gather, 8 rows per word-load step for 3 stages. */
static void vq_rows_fast(float *y, const uint8_t *idx, const uint16_t *scale,
                         const float *lut, int r_lo, int r_hi, int nv, int st, int en)
{
    if (st != 3 || (r_lo & 63)) { orc_vq_rows(y, idx, scale, lut, r_lo, r_hi, nv, st, en); return; }
    float acc[128];
    for (int r0 = r_lo; r0 < r_hi; r0 += 128) {
        const int rows = r0 + 128 < r_hi ? 128 : r_hi - r0;
        const int nblk = (rows + 63) / 64;
        memset(acc, 0, sizeof acc);
        for (int v = 0; v < nv; v++) {
            const float *b0 = lut + (size_t)v * st * en, *b1 = b0 + en, *b2 = b0 + 2 * en;
            for (int j = 0; j < nblk; j++) {
                const int nr = (j + 1) * 64 <= rows ? 64 : rows - j * 64;
                const uint8_t *ix = idx + ((size_t)(r0 / 64 + j) * nv + v) * 64 * st;
                float *ac = acc + j * 64;
                int r = 0;
                for (; r + 8 <= nr; r += 8, ix += 24) {
                    uint32_t w0, w1, w2, w3, w4, w5;
                    memcpy(&w0, ix, 4); memcpy(&w1, ix + 4, 4); memcpy(&w2, ix + 8, 4);
                    memcpy(&w3, ix + 12, 4); memcpy(&w4, ix + 16, 4); memcpy(&w5, ix + 20, 4);
                    /* all eight gathers before the first store: a store
                     * to acc may alias the tables for the compiler, and
                     * would otherwise hold back the next row's loads */
                    const float t0 = b0[w0 & 0xff] + b1[(w0 >> 8) & 0xff] + b2[(w0 >> 16) & 0xff];
                    const float t1 = b0[w0 >> 24] + b1[w1 & 0xff] + b2[(w1 >> 8) & 0xff];
                    const float t2 = b0[(w1 >> 16) & 0xff] + b1[w1 >> 24] + b2[w2 & 0xff];
                    const float t3 = b0[(w2 >> 8) & 0xff] + b1[(w2 >> 16) & 0xff] + b2[w2 >> 24];
                    const float t4 = b0[w3 & 0xff] + b1[(w3 >> 8) & 0xff] + b2[(w3 >> 16) & 0xff];
                    const float t5 = b0[w3 >> 24] + b1[w4 & 0xff] + b2[(w4 >> 8) & 0xff];
                    const float t6 = b0[(w4 >> 16) & 0xff] + b1[w4 >> 24] + b2[w5 & 0xff];
                    const float t7 = b0[(w5 >> 8) & 0xff] + b1[(w5 >> 16) & 0xff] + b2[w5 >> 24];
                    ac[r] += t0; ac[r + 1] += t1; ac[r + 2] += t2; ac[r + 3] += t3;
                    ac[r + 4] += t4; ac[r + 5] += t5; ac[r + 6] += t6; ac[r + 7] += t7;
                }
                for (; r < nr; r++, ix += 3) ac[r] += b0[ix[0]] + b1[ix[1]] + b2[ix[2]];
            }
        }
        for (int r = 0; r < rows; r++) y[r0 + r] = acc[r] * f16s(scale[r0 + r]);
    }
}

#if ORC_X86
AVX512_FN static void mvq_avx512(float *y, const int8_t *W, const uint16_t *ws,
                                 const float *x, int r_lo, int r_hi, int in, int g,
                                 int bits, size_t rowbytes)
{
        const int ng = (in + g - 1) / g;
        int8_t unp[1024];
        for (int o = r_lo; o < r_hi; o++) {
            const int8_t *row = W + (size_t)o * rowbytes;
            const uint16_t *s = ws + (size_t)o * ng;
            float acc = 0;
            for (int k = 0; k < ng; k++) {
                const int8_t *w;
                if (bits == 4) {
                    /* element 2i is byte i's low nibble, 2i + 1 its high
                     * one: sixteen bytes unpack to 32 elements in order */
                    const uint8_t *p4 = (const uint8_t *)row + (size_t)k * g / 2;
                    const __m128i m4 = _mm_set1_epi8(0x0F), b8 = _mm_set1_epi8(8);
                    for (int i = 0; i < g / 2; i += 16) {
                        const __m128i b = _mm_loadu_si128((const __m128i *)(p4 + i));
                        const __m128i lo = _mm_sub_epi8(_mm_and_si128(b, m4), b8);
                        const __m128i hi = _mm_sub_epi8(_mm_and_si128(_mm_srli_epi16(b, 4), m4), b8);
                        _mm_storeu_si128((__m128i *)(unp + 2 * i), _mm_unpacklo_epi8(lo, hi));
                        _mm_storeu_si128((__m128i *)(unp + 2 * i + 16), _mm_unpackhi_epi8(lo, hi));
                    }
                    w = unp;
                } else {
                    w = row + (size_t)k * g;
                }
                const float *xx = x + (size_t)k * g;
                const int lim = (k * g + g <= in) ? g : in - k * g;
                __m512 s0 = _mm512_setzero_ps(), s1 = _mm512_setzero_ps();
                int i = 0;
                for (; i + 32 <= lim; i += 32) {
                    const __m512i w0 = _mm512_cvtepi8_epi32(_mm_loadu_si128((const __m128i *)(w + i)));
                    const __m512i w1 = _mm512_cvtepi8_epi32(_mm_loadu_si128((const __m128i *)(w + i + 16)));
                    s0 = _mm512_fmadd_ps(_mm512_cvtepi32_ps(w0), _mm512_loadu_ps(xx + i), s0);
                    s1 = _mm512_fmadd_ps(_mm512_cvtepi32_ps(w1), _mm512_loadu_ps(xx + i + 16), s1);
                }
                float part = _mm512_reduce_add_ps(_mm512_add_ps(s0, s1));
                for (; i < lim; i++) part = fmaf((float)w[i], xx[i], part);
                acc = fmaf(f16s(s[k]), part, acc);
            }
            y[o] = acc;
        }
}
#endif

/* Quantized rows [r_lo, r_hi) against fp32 activations. */
static void mvq_fast(float *y, const int8_t *W, const uint16_t *ws, const float *x,
                     int r_lo, int r_hi, int in, int g, int bits, size_t rowbytes)
{
#if ORC_X86
    if (have_avx512() && (bits == 8 || bits == 4) && g % 64 == 0 && g <= 1024) {
        mvq_avx512(y, W, ws, x, r_lo, r_hi, in, g, bits, rowbytes);
        return;
    }
#endif
    orc_mvq_rows(y, W, ws, x, r_lo, r_hi, in, g, bits, rowbytes, ORC_AVX512);
}

static void tensor_mv_mt(const orc_tensor *t, const float *x, float *y)
{
    if (!t->rows) return;
    const int rows = t->rows;
    if (t->fmt == 0) {
        const float *W = (const float *)t->q;
        #pragma omp parallel for schedule(static)
        for (int o = 0; o < rows; o++) {
            const float *r = W + (size_t)o * t->cols;
            float acc = 0;
            for (int i = 0; i < t->cols; i++) acc += r[i] * x[i];
            y[o] = acc;
        }
        return;
    }
    const int bits = t->fmt == 2 ? 8 : t->fmt == 3 ? 4 : 3;
    const int chunks = (rows + 63) / 64;
    #pragma omp parallel for schedule(static)
    for (int c = 0; c < chunks; c++) {
        const int lo = c * 64, hi = lo + 64 < rows ? lo + 64 : rows;
        mvq_fast(y, (const int8_t *)t->q, t->qs, x, lo, hi, t->cols, t->group, bits, t->rowbytes);
    }
}

static void lutb_mt(float *lut, const float *booksT, const float *x, int cb_base,
                    int st, int en, int vd, int nv)
{
    const int chunks = (nv + 15) / 16;
    #pragma omp parallel for schedule(static)
    for (int c = 0; c < chunks; c++) {
        const int lo = c * 16, hi = lo + 16 < nv ? lo + 16 : nv;
        lutb_fast(lut, booksT, x, cb_base, st, en, vd, lo, hi);
    }
}

static void vq_mt(float *y, const uint8_t *idx, const uint16_t *scale, const float *lut,
                  int M, int nv, int st, int en)
{
    const int chunks = (M + 127) / 128;
    #pragma omp parallel for schedule(static)
    for (int c = 0; c < chunks; c++) {
        const int lo = c * 128, hi = lo + 128 < M ? lo + 128 : M;
        vq_rows_fast(y, idx, scale, lut, lo, hi, nv, st, en);
    }
}

/* orc_moe_layer with the work split over `nthreads`; same result bits. */
int orc_moe_layer_mt(const orc_moe *m, const float *x, float *out, int *idx_o,
                     float *w_o, int nthreads)
{
    const int E = m->n_experts, K = m->top_k, H = m->hidden, I = m->moe_inter;
    const int st = m->stages, en = m->entries, vd = m->vec_dim;
    if (nthreads > 0) omp_set_num_threads(nthreads);
    float *logit = (float *)calloc((size_t)E, sizeof(float));
    int idx[64];
    float w[64];
    tensor_mv_mt(&m->router, x, logit);
    orc_route_cfg rc = { E, K, m->score_func, m->renorm, m->routed_scale, m->n_group, m->topk_group };
    const int nsel = orc_route(&rc, logit, m->bias, NULL, idx, w);
    if (idx_o) memcpy(idx_o, idx, (size_t)K * sizeof(int));
    if (w_o) memcpy(w_o, w, (size_t)K * sizeof(float));
    memset(out, 0, (size_t)H * sizeof(float));
    const size_t lut_sz = (size_t)((H > I ? H : I) / vd) * st * en;
    float *lut_g = (float *)malloc(lut_sz * sizeof(float));
    float *lut_u = (float *)malloc(lut_sz * sizeof(float));
    float *lut_d = (float *)malloc(lut_sz * sizeof(float));
    float *ga = (float *)malloc((size_t)I * sizeof(float));
    float *ub = (float *)malloc((size_t)I * sizeof(float));
    float *acc = (float *)malloc((size_t)H * sizeof(float));
    int lut_ready = 0, rcode = 0;
    for (int j = 0; j < K && nsel > 0; j++) {
        const uint8_t *rec = m->recs[idx[j]];
        if (!rec) { rcode = -2; break; }
        uint16_t cbid; uint32_t go, uo, dof, co;
        memcpy(&cbid, rec + 10, 2); memcpy(&go, rec + 20, 4); memcpy(&uo, rec + 24, 4);
        memcpy(&dof, rec + 28, 4); memcpy(&co, rec + 32, 4);
        const uint16_t *sc = (const uint16_t *)(rec + co);
        if (!lut_ready) {
            lutb_mt(lut_g, m->booksT, x, cbid, st, en, vd, H / vd);
            lutb_mt(lut_u, m->booksT, x, cbid + st, st, en, vd, H / vd);
            lut_ready = 1;
        }
        vq_mt(ga, rec + go, sc, lut_g, I, H / vd, st, en);
        vq_mt(ub, rec + uo, sc + I, lut_u, I, H / vd, st, en);
        orc_act_pair(ga, ub, I);
        lutb_mt(lut_d, m->booksT, ga, cbid + 2 * st, st, en, vd, I / vd);
        vq_mt(acc, rec + dof, sc + 2 * I, lut_d, H, I / vd, st, en);
        const float wj = w[j];
        for (int i = 0; i < H; i++) out[i] += wj * acc[i];
    }
    const int SI = I * (m->n_shared ? m->n_shared : 1);
    float *a = (float *)calloc((size_t)SI, sizeof(float));
    float *b = (float *)calloc((size_t)SI, sizeof(float));
    float *tmp = (float *)calloc((size_t)H, sizeof(float));
    tensor_mv_mt(&m->sh_gate, x, a);
    tensor_mv_mt(&m->sh_up, x, b);
    orc_act_pair(a, b, SI);
    tensor_mv_mt(&m->sh_down, a, tmp);
    for (int i = 0; i < H; i++) out[i] += tmp[i];
    free(a); free(b); free(tmp);
    free(lut_g); free(lut_u); free(lut_d); free(ga); free(ub); free(acc); free(logit);
    return nsel < 0 ? -1 : rcode;
}
