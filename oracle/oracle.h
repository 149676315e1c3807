/* SPDX-License-Identifier: Apache-2.0 */
/*
 * oracle.h — CPU restatement of WARP's MoE expert path.  TEST
 * INFRASTRUCTURE ONLY: the checker that the HIP path is compared against.
 * Nothing in the shipped library links, loads or calls this; only tests/,
 * the smoke check and the CPU-baseline leg of bench.py do.
 *
 * Each function restates one piece of the reference's x86 CPU path in its
 * exact floating-point order (file:line of the reference given at each
 * definition in oracle.c).  Two arithmetic orders are kept where the
 * reference has two on x86:
 *
 *   ORC_PORTABLE  the universal C kernels registered first
 *                 (src/kda.c:119-130; model.c compiled -O2, no FMA)
 *   ORC_AVX512    what waste_backend_init installs on an AVX-512F+BW host
 *                 (src/backend.c:188-191; src/simd_avx512.c:20-123)
 *
 * The order is a property of the arithmetic, not of the instructions:
 * ORC_AVX512 is computed here in scalar C with fmaf() lane by lane and
 * the same horizontal-sum tree, so it runs on any host.  The SIMD
 * implementation in orc_cpu.c (built with -mavx512f when the host has it)
 * is the timed CPU baseline; it produces the same bits.
 *
 * Pinning (which check fixes which function) is listed in tests/ and in
 * the golden fixtures' manifest; every function here has one.
 */
#ifndef WARP_ORACLE_H
#define WARP_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_PORTABLE = 0, ORC_AVX512 = 1 };

/* ---- scalars ------------------------------------------------------------ */
float    orc_expf(float x);                 /* glibc 2.35 expf, restated     */
float    orc_f16_scale(uint16_t h);         /* waste_f16: subnormals kept    */
float    orc_f16_book(uint16_t h);          /* codebook load: subnormals → 0 */
uint32_t orc_crc32(const uint8_t *p, size_t n);

/* Codebooks as the loader leaves them: fp32 [book][entry][dim] and the
 * transposed copy [book][dim][entry]. */
void orc_books_load(const uint16_t *f16, int n_books, int entries, int vec_dim,
                    float *books, float *booksT);

/* ---- kernels ------------------------------------------------------------ */
void orc_lutb(float *lut, const float *booksT, const float *x, int cb_base,
              int stages, int entries, int vec_dim, int v_lo, int v_hi,
              int order);
void orc_vq_rows(float *y, const uint8_t *idx, const uint16_t *scale,
                 const float *lut, int r_lo, int r_hi, int nv, int stages,
                 int entries);
void orc_dequant(float *W, const uint8_t *idx, const uint16_t *scale,
                 const float *books, int cb_base, int M, int N, int stages,
                 int entries, int vec_dim);
/* VQ4P (6-bit indices, 4 stages of 64 entries): the int8 shadow of a LUT,
 * one fp32 scale per ORC_VQ_LUT_BLK positions, and the rows through it. */
#define ORC_VQ_LUT_BLK 32
void orc_vq_quant_lut(const float *lut, int nv, int stages, int entries,
                      int8_t *q, float *scale);
void orc_vq_rows_p6(float *y, const uint8_t *idx, const uint16_t *scale,
                    const int8_t *lut8, const float *lscale, int r_lo,
                    int r_hi, int nv, int order);
void orc_mvq_rows(float *y, const int8_t *W, const uint16_t *ws,
                  const float *x, int r_lo, int r_hi, int in, int group,
                  int bits, size_t rowbytes, int order);
void orc_matvec_f32(float *y, const float *W, const float *x, int out, int in);
void orc_mmq_rows(float *Y, const int8_t *W, const uint16_t *ws,
                  const float *X, int out, int in, int group, int bits,
                  size_t rowbytes, int T);
void orc_matmul_f32(float *Y, const float *W, const float *X, int out,
                    int in, int T);
void orc_router_scores(int score_func, const float *logit, float *score,
                       int E);
void orc_act_pair(float *g, const float *u, int n);

/* Routing of one token: scores, optional group limit, top-k with the
 * reference's tie rule, renormalisation and scaling.  Returns the number
 * of ids written (K), or -1 when a selection pass finds no candidate. */
typedef struct {
    int n_experts, top_k, score_func, renorm;
    float routed_scale;
    int n_group, topk_group;     /* n_group <= 1: plain top-k */
} orc_route_cfg;

int orc_route(const orc_route_cfg *c, const float *logit, const float *bias,
              float *score_out, int *idx, float *w);

/* ---- the layer ---------------------------------------------------------- */
typedef struct {
    int fmt;                     /* WQ_F32, WQ_Q8G or WQ_Q4G; 0 rows = absent */
    int rows, cols, group;
    const void *q;               /* F32: float data; else packed rows        */
    const uint16_t *qs;          /* f16 group scales                         */
    size_t rowbytes;
} orc_tensor;

typedef struct {
    int hidden, n_experts, top_k, moe_inter, n_shared;
    int score_func, renorm;
    float routed_scale;
    int n_group, topk_group;
    int stages, entries, vec_dim;
    int order;                   /* ORC_PORTABLE or ORC_AVX512               */
    orc_tensor router;
    const float *bias;           /* e_score_correction_bias or NULL          */
    orc_tensor sh_gate, sh_up, sh_down;
    const float *booksT;         /* whole codebook table, transposed         */
    int n_books;
    const uint8_t *const *recs;  /* [n_experts] record bases                 */
    size_t rec_bytes;
} orc_moe;

/* Record header checks (src/model.c:3645-3692).  0 when usable. */
int orc_record_check(const uint8_t *rec, size_t rec_bytes, int layer,
                     int expert, int inter, int hidden, int stages,
                     int n_books, int verify_crc);

/* One decode token: moe_layer's serial path.  out[H]; idx/w[K]; logits[E]
 * may be NULL. */
int orc_moe_layer(const orc_moe *m, const float *x, float *out, int *idx,
                  float *w, float *logits);
/* A chunk of T tokens: moe_chunk.  out[T][H]; idx/w[T][K] may be NULL. */
int orc_moe_chunk(const orc_moe *m, const float *x, int T, float *out,
                  int *idx, float *w);

/* The experts and shared expert with the routing given (idx/w [T][K]);
 * chunk selects moe_chunk's order and shared-expert path.  0, or -2 when a
 * routed record is missing. */
int orc_moe_apply(const orc_moe *m, const float *x, int T, const int *idx,
                  const float *w, int chunk, float *out);
void orc_router_logits(const orc_moe *m, const float *x, int T, float *logits);

/* Threaded CPU baseline of orc_moe_layer (same bits): nthreads row-split
 * workers, as the reference's pool does.  Returns as orc_moe_layer. */
int orc_moe_layer_mt(const orc_moe *m, const float *x, float *out, int *idx,
                     float *w, int nthreads);
int orc_cpu_isa(void);           /* 2 AVX-512 kernels in use, 1 AVX2, 0 C  */

/* ---- expert cache policy (src/ecache.c) ------------------------------------
 * The decisions of waste_ecache with read-ahead on or off, made
 * deterministic: a read the hint or the lookahead issues is in flight
 * (and so never a victim) until the next demand get(), when it is done.
 * Keys are (layer << 16) | expert, layers < 128, experts < 1024. */
typedef struct orc_ecache orc_ecache;
orc_ecache *orc_ecache_new(int n_slots, int depth, int readahead, int lru);
void orc_ecache_free(orc_ecache *c);
void orc_ecache_hint(orc_ecache *c, int layer, const int *ids, int n);
void orc_ecache_prefetch(orc_ecache *c, int layer, const int *ids, int n);
/* the slot now holding (layer, expert), or -1 (no slots / all pinned) */
int orc_ecache_get(orc_ecache *c, int layer, int expert);
/* get, and keep the slot claimed until release (at most 64 held) */
int orc_ecache_hold(orc_ecache *c, int layer, int expert);
void orc_ecache_release(orc_ecache *c);
/* 1 when a record went into an empty slot, else 0 */
int orc_ecache_admit(orc_ecache *c, int layer, int expert);
void orc_ecache_resident_mask(const orc_ecache *c, int layer, int n, uint8_t *out);
/* hits, misses, evictions, prefetched, spec_issued, reads */
void orc_ecache_stats(const orc_ecache *c, uint64_t out[6]);

/* The lookahead: the next layer's router on this layer's input, scored,
 * bias added, top n without the group limit (src/model.c:5419-5449).
 * Returns n (clamped to E). */
int orc_predict_next(int score_func, int E, const float *logit, const float *bias, int n,
                     int *out);

#ifdef __cplusplus
}
#endif
#endif
