/* SPDX-License-Identifier: Apache-2.0 */
/*
 * launch.h — the thin C-ABI between the C host code and the gfx950 kernels.
 * Each whip_* call enqueues kernels on `s` and returns a hipError_t as int
 * (0 on success).  Pointers are device pointers unless said otherwise.
 */
#ifndef WARP_HIP_LAUNCH_H
#define WARP_HIP_LAUNCH_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Arms kernel timing for the calling thread's next decode launch (the
 * batch-1 GEMV, the VQ3R apply, the combine): its dispatch records start
 * and stop (hipExtLaunchKernel's events, taken by the dispatch itself, so
 * they bracket the kernel and nothing else). */
void whip_time_next(hipEvent_t start, hipEvent_t stop);

/* bf16 activations to fp32 (exact). */
int whip_bf16_to_f32(const uint16_t *x, float *y, size_t n, hipStream_t s);

/* y[t*y_ld + r] = W[r] . x[t*x_ld + 0..cols) for r < rows, t < T, for up to
 * two matrices in one launch (W1 may be NULL).  fmt 0 F32, 2 Q8G, 3 Q4G. */
typedef struct {
    int fmt, rows, cols, group;
    const void *q;
    const uint16_t *qs;
    size_t rowbytes;
} whip_mat;
int whip_gemv(const whip_mat *W0, const whip_mat *W1, const float *x, int x_ld,
              int T, float *y0, float *y1, int y_ld, hipStream_t s);

/* Up to three independent products in one launch.  With B set, the job is
 * a SwiGLU pair: y = silu(A.x) * (B.x).  x is fp32 or bf16 (x_bf16). */
typedef struct {
    whip_mat A;
    const whip_mat *B;
    const void *x;
    int x_ld, x_bf16;
    float *y;
    int y_ld;
} whip_gemv_job;
int whip_gemv_multi(const whip_gemv_job *jobs, int n, int T, hipStream_t s);

/* Routing, one wavefront per token: scores, group limit, top-k with the
 * engine's tie rule, renormalisation, scaling.  When T == 1 it also lays
 * out the pair list (selection order) that the expert kernels walk. */
typedef struct {
    int E, K, score_func, renorm;
    float routed_scale;
    int n_group, topk_group;
} whip_route_cfg;
int whip_route(const whip_route_cfg *c, const float *logits, const float *bias,
               int T, int32_t *ids, float *w, int32_t *pair_tok,
               int32_t *pair_exp, float *pair_w, int32_t *tok_pairs,
               int *err, hipStream_t s);
/* T > 1: pairs ordered by (expert, token) ascending; each token's pairs in
 * ascending expert order (the chunk's combine order). */
int whip_pairs(const int32_t *ids, const float *w, int T, int K, int E,
               int32_t *pair_tok, int32_t *pair_exp, float *pair_w,
               int32_t *tok_pairs, hipStream_t s);

/* One VQ3R apply stage over P (source row, expert) pairs:
 *   part[((p*kinds + k)*nch + c)*M + r] = sum over chunk c's positions of
 *       L_k[v][0][i0] + L_k[v][1][i1] + L_k[v][2][i2]
 * with L_k built in LDS from src[pair_src[p]] and books cb + 3k.
 * span = P (<= 64) declares a one-token launch, every pair reading source
 * row 0: one table then serves all pairs, and rsplit divides the P*M/64 row
 * blocks of all pairs; span <= 1 splits each pair's M/64 row blocks.
 * part holds P*kinds*nch*M floats plus 64 (a sink for dead stores). */
typedef struct {
    const uint8_t *const *recs;      /* [E] record bases, NULL if unbound   */
    const int32_t *pair_exp;         /* [P]                                 */
    const int32_t *pair_src;         /* [P] row of src; NULL = p            */
    const void *src;                 /* fp32, or bf16 when src_bf16         */
    int src_ld, src_bf16;
    const float *booksT;             /* [n_books][8][256] fp32              */
    int cb;                          /* first book of kind 0                */
    uint32_t idx_off[2];             /* byte offset of kind k's indices     */
    int kinds, M, nv, P, rsplit, span;
    float *part;
    int *err;
    const uint8_t *const *pair_rec;  /* [P] the pairs' records, or NULL     */
    /* Down pass from the gate/up partials (positions-across-lanes kernel
     * only, M of them = nv*8 rows): pair p's x is silu(sum of its act_nch
     * gate partials) * (sum of its up partials), partials a gate/up launch
     * with out_sc_off wrote (already scaled); src is then unused. */
    const float *act_part;
    int act_nch;
    /* Positions-across-lanes kernel, nonzero: every partial of row r of
     * kind k is multiplied by the record's f16 scale at byte out_sc_off +
     * 2*(k*M + r) (the gate|up row scales). */
    uint32_t out_sc_off;
    /* Gate/up pass of the positions-across-lanes kernel, shd_y set: extra
     * workgroups of the launch compute shd_y = shd . shd_x (the shared
     * expert's down projection, shd.rows outputs, fp32 x). */
    whip_mat shd;
    const float *shd_x;
    float *shd_y;
} whip_vq_args;
int whip_vq_apply(const whip_vq_args *a, hipStream_t s);
int whip_vq_chunks(int nv, int M);   /* nch for nv positions, M rows        */

/* h[p*I + r] = silu(scale_g[r]*sum_c gpart) * (scale_u[r]*sum_c upart)
 * for the routed pairs. */
int whip_vq_act(const uint8_t *const *recs, const int32_t *pair_exp, int P,
                const float *part, int nch, int I, uint32_t sc_off, float *h,
                hipStream_t s);

/* y[t*H + i] = sum over token t's pairs (combine order) of
 *   w * (scale_d[i] * sum_c part_d) + sh_t[i] (sh may be NULL), where
 * sh_t[i] = sum over q < sh_n, in order, of sh[q*sh_stride + t*H + i]
 * (the slices of a split product; sh_n 1: sh[t*H + i] itself).
 * sc_off_down 0: part_d is already scaled (a down launch with out_sc_off).
 * T == 1: the token's pairs are pairs 0 .. K-1 (tok_pairs is not read). */
int whip_combine(const uint8_t *const *recs, const int32_t *pair_exp,
                 const float *pair_w, const int32_t *tok_pairs, int T, int K,
                 const float *part_d, int nch, int H, uint32_t sc_off_down,
                 int skip_zero, const float *sh, int sh_n, size_t sh_stride,
                 float *y, hipStream_t s);
/* VQ4P down rows for the combine: pair p's row r is the fold, in block
 * order, of S[(p*nb + b)*H + r] (whip_p6_down's sums) with the pair's table
 * scales ls[p*nb + b] (fma: one fused multiply-add, else a product and a
 * sum), times the f16 row scale at sc_off of the pair's record; an unbound
 * expert's rows are zeros. */
typedef struct {
    const int16_t *S;
    const float *ls;
    int nb;
    uint32_t sc_off;
    int fma;
} whip_fold;
/* whip_combine / whip_combine_sh with the pairs' down rows folded from f. */
int whip_combine_fold(const uint8_t *const *recs, const int32_t *pair_exp, const float *pair_w,
                      const int32_t *tok_pairs, int T, int K, const whip_fold *f, int H, int skip_zero,
                      const float *sh, int sh_n, size_t sh_stride, float *y, hipStream_t s);

/* ---- products of a few tokens on the matrix cores (skinny.hip) ---- */

/* part[q][t][r] (q < nsl, t < T, r < A.rows) = the partial sum of A[r] . x[t]
 * over column slice q; the slices' sum is the product.  x is fp32 or bf16
 * (x_bf16), rows x_ld elements apart (x_ld % 8 == 0, x 16-byte aligned); all
 * jobs of one launch read the same kind of x.  nsl must be
 * whip_sk_slices(&A); whip_sk_ok says whether A's shape is taken (columns a
 * multiple of 128, F32 or Q8G/Q4G with groups a multiple of 128). */
typedef struct {
    whip_mat A;
    const void *x;
    int x_ld, x_bf16;
    float *part;
    int nsl;
} whip_sk_job;
int whip_sk_ok(const whip_mat *A);
int whip_sk_slices(const whip_mat *A);
int whip_sk_run(const whip_sk_job *jobs, int n, int T, hipStream_t s);
/* logits[t*E + e] = sum over q < nsl_r of pr[q][t][e], in order; with pg
 * set, also h[t*SI + i] = silu(sum of pg[q][t][i]) * (sum of pu[q][t][i]). */
int whip_sk_finish(const float *pr, int nsl_r, int E, float *logits, const float *pg,
                   const float *pu, int nsl_g, int SI, float *h, int T, hipStream_t s);
/* whip_sk_finish and whip_route (ids, w; no pair lists) in one launch, for
 * E <= 256 with ceil(E/64)*K <= 64; hipErrorInvalidValue otherwise. */
int whip_sk_route(const whip_route_cfg *c, const float *pr, int nsl_r, float *logits, const float *bias,
                  int T, int32_t *ids, float *w, int *err, const float *pg, const float *pu, int nsl_g,
                  int SI, float *h, hipStream_t s);

/* ---- VQ4P through the int8 LUT (vq4p.hip) ---- */

/* The int8 shadow of an fp32 LUT [nv][stages][entries]: per block of 32
 * positions, scale[blk] = max|lut| / 127 and q = rint(lut * (127 / max))
 * clamped to [-127, 127] (src/model.c:3979-4074). */
int whip_vq_quant_lut(const float *lut, int nv, int stages, int entries, int8_t *q,
                      float *scale, hipStream_t s);
/* The same for ntab tables back to back: table t at lut + t*nv*stages*
 * entries, its int8 copy at the same offset of q, its scales at
 * scale + t*ceil(nv/32). */
int whip_vq_quant_lut_n(const float *lut, int nv, int stages, int entries, int ntab, int8_t *q,
                        float *scale, hipStream_t s);
/* VQ4P int8 tables of rows x kinds inputs (vq_build_lut, then
 * vq_quant_lut): table t = (row t / kinds, kind t % kinds) from x row
 * t / kinds (bf16 or fp32, row stride x_ld) and books cb + 4*kind .. + 3 of
 * booksT ([book][8][64] fp32), in the engine's order (fma: the AVX-512
 * kernel's chain, else the portable C one's products and sums);
 * q[t][nv][4][64], qs[t][ceil(nv/32)]. */
int whip_p6_lutq(const void *x, int x_bf16, int x_ld, int rows, int kinds, const float *booksT, int cb,
                 int nv, int fma, int8_t *q, float *qs, hipStream_t s);
/* Each pair's gate and up rows folded from whip_p6_gate_up's sums (block
 * order, the token's table scales qs_gu, the f16 row scales at sc_gate /
 * sc_up of the record), h = silu(g) * u, and the pair's down table from h
 * (books cb_d ..): q_d[p][nv_d][4][64], qs_d[p][ceil(nv_d/32)].  I == 8 nv_d. */
int whip_p6_act_lutq(const uint8_t *const *recs, const int32_t *pair_exp, const int32_t *pair_tok, int P,
                     const int16_t *S, const float *qs_gu, uint32_t sc_gate, uint32_t sc_up, int I, int nv_gu,
                     const float *booksT, int cb_d, int nv_d, int fma, int8_t *q_d, float *qs_d,
                     hipStream_t s);
/* The VQ4P layer's gate/up tile launch: the exact integer sums of every
 * pair's gate and up rows per 32-position scale block,
 * S[((p*2 + kind)*nb + b)*I + r] (int16, nb = ceil(nv/32)), from the record
 * of expert pair_exp[p] (idx at idx_off[kind]) through the token's tables:
 * whip_p6_lutq's q (table pair_tok[p]*2 + kind), or with q NULL built here
 * from x row pair_tok[p] (bf16 or fp32, row stride x_ld) and books
 * cb .. cb+7 of booksT ([book][8][64] fp32) in the engine's order for fma,
 * their scales written to qs[tok][2][nb].  An unbound expert's sums are
 * zeros and raise bit 0 of err.  I % 64 == 0.  With q NULL and shd_y set,
 * spare workgroups also compute shd_y = shd . shd_x (fp32 x; 16-byte
 * chunks: refused otherwise). */
int whip_p6_gate_up(const uint8_t *const *recs, const int32_t *pair_exp, const int32_t *pair_tok, int P,
                    const uint32_t *idx_off, int I, const void *x, int x_bf16, int x_ld, int nv,
                    const float *booksT, int cb, int fma, const int8_t *q, int16_t *S, float *qs, int *err,
                    const whip_mat *shd, const float *shd_x, float *shd_y, hipStream_t s);
/* The down tile launch: the sums of each pair's down rows (idx at idx_off;
 * S[(p*nb + b)*H + r], nb = I/256 rounded up) through its table: q's table
 * p (whip_p6_act_lutq's), or with q NULL built here as whip_p6_act_lutq
 * builds it (from Sg / qs_g, nv_g positions, the row scales at sc_gate /
 * sc_up, books cb .. cb+3), its scales written to qs[p][nb].  H % 64 == 0. */
int whip_p6_down(const uint8_t *const *recs, const int32_t *pair_exp, const int32_t *pair_tok, int P,
                 uint32_t idx_off, int H, int I, const int16_t *Sg, const float *qs_g, uint32_t sc_gate,
                 uint32_t sc_up, int nv_g, const float *booksT, int cb, int fma, const int8_t *q, int16_t *S,
                 float *qs, int *err, hipStream_t s);
/* Each pair's down rows y[p][M] folded from whip_p6_down's sums S (nb
 * blocks a pair) with its table scales ls[p][nb], times the f16 row scale at
 * sc_off of its record; zeros for an unbound expert. */
int whip_p6_fold_pairs(const uint8_t *const *recs, const int32_t *pair_exp, int P, const int16_t *S,
                       const float *ls, int nb, int M, uint32_t sc_off, int fma, float *y, hipStream_t s);
/* VQ2R (vq2r.hip): fp32 tables lut[t][nv][st][256] of rows x kinds inputs in
 * the engine's order (st == 2; shd_y set: spare workgroups also compute
 * shd_y = shd . shd_x, refused for shapes they do not take), and every
 * pair's rows through them in vq_rows' order (two stages, two index bytes a
 * row and position). */
int whip_r2_lutb(const void *x, int x_bf16, int x_ld, int rows, int kinds, int st, const float *booksT, int cb,
                 int nv, int fma, float *lut, const whip_mat *shd, const float *shd_x, float *shd_y,
                 hipStream_t s);
/* The down tables of P pairs from their gate and up rows gu[p][2][I]:
 * h = silu(g) * u, then whip_r2_lutb's tables of h (one kind, books cb ..). */
int whip_r2_act_lutb(const float *gu, int P, int I, const float *booksT, int cb, int fma, float *lut,
                     hipStream_t s);
int whip_r2_rows_pairs(const uint8_t *const *recs, const int32_t *pair_exp, const int32_t *pair_tok, int P,
                       int kinds, const uint32_t *idx_off, const uint32_t *sc_off, int M, int nv, const float *lut,
                       int per_tok, float *out, int *err, hipStream_t s);
/* Rows [r_lo, r_hi) (r_lo % 64 == 0) of a VQ4P matrix through lut8/lscale
 * (src/model.c:4076-4114); fma: fold the blocks with one fused
 * multiply-add (the AVX-512 and NEON kernels) instead of a product and a
 * sum (the portable C kernel).  lut8 16-byte aligned. */
int whip_vq_rows_p6(const uint8_t *idx, const uint16_t *scale, const int8_t *lut8,
                    const float *lscale, int r_lo, int r_hi, int nv, int fma, float *y,
                    hipStream_t s);

/* ---- many tokens (prefill.hip) ---- */

/* Stable sort of the T*K pairs by expert (id -1 after the last expert);
 * each token's pairs in ascending expert order in tok_pairs; seg_off[e] ..
 * seg_off[e+1] is expert e's segment (E+2 entries); order[] the experts by
 * descending pair count. */
int whip_sort_pairs(const int32_t *ids, const float *w, int T, int K, int E,
                    int32_t *pair_tok, int32_t *pair_exp, float *pair_w,
                    int32_t *tok_pairs, int32_t *pair_pos, int32_t *seg_off,
                    int32_t *order, hipStream_t s);

/* One grouped product on the matrix cores (fp16 in, fp32 accumulate).
 * B: VQ3R records (recs set; kind k's indices at idx_off[k], row scales at
 * sc_off[k], books cb + 3k of books16) or trunk matrices W0/W1 (fmt
 * F32/Q8G/Q4G).  A: rows of x (fp32, bf16 or fp16) — segment position p
 * reads row tok[p] (tok NULL: p).  pair = 1: out[p][n] = silu(gate) * up
 * as fp16; pair = 0: out[p][n] fp32 (times the VQ3R row scale).
 * Segments: seg_off/order as whip_sort_pairs writes them (segs of them),
 * or seg_off NULL for one segment of `rows` rows.  mt: 32-row tiles per
 * workgroup (1 or 4); mblocks: (32*mt)-row blocks per segment the grid
 * covers. */
typedef struct {
    const uint8_t *const *recs;
    uint32_t idx_off[2], sc_off[2];
    const uint16_t *books16;     /* fp16 [n_books][256][8], subnormals flushed */
    int cb;
    const uint8_t *W0, *W1;
    const uint16_t *S0, *S1;
    size_t rowbytes;
    int group;
    int N, Kd;                   /* rows per matrix, reduction length        */
    const void *x;
    int x_mode, x_ld;            /* 0 fp32, 1 bf16, 2 fp16                   */
    const int32_t *tok;
    const int32_t *seg_off, *order;
    int rows;
    void *out;
    int out_ld;
    int *err;
} whip_pf_args;
int whip_pf_gemm(const whip_pf_args *a, int dec, int pair, int mt, int segs, int mblocks, hipStream_t s);
/* One dense Q4G/Q8G product of a.rows tokens (the shared expert): fp16 A
 * (x_mode 2) against the rows W0 (and W1 with pair: SwiGLU to fp16 out),
 * groups a multiple of 128 columns summed exactly and scaled in fp32.
 * hipErrorInvalidValue for a shape it does not take (then whip_pf_gemm). */
int whip_pf_dense(const whip_pf_args *a, int dec, int pair, hipStream_t s);

/* n activations (fp32, or bf16 when bf16) to fp16 for the products' A
 * operand; a value outside fp16's range sets err bit 4. */
int whip_pf_to_f16(const void *x, int bf16, size_t n, uint16_t *y, int *err, hipStream_t s);

/* Router logits for T tokens on the matrix cores (fp32 products), through
 * part[whip_pf_router_part_floats(T, E)]. */
size_t whip_pf_router_part_floats(int T, int E);
int whip_pf_router(const whip_mat *W, const void *x, int x_bf16, int T, float *part,
                   float *logits, hipStream_t s);

/* y[t] = sum over t's pairs (tok_pairs order; zero weights and unbound
 * experts skipped) of w * Y[p], + sh[t] (sh may be NULL). */
int whip_pf_combine(const int32_t *tok_pairs, const int32_t *pair_exp, const float *pair_w,
                    const uint8_t *const *recs, int T, int K, int E, const float *Y, int H,
                    const float *sh, float *y, hipStream_t s);

/* Materialised dequantisation of one VQ3R matrix (fp32 [M][N]). */
int whip_dequant(const uint8_t *idx, const uint16_t *scale, const float *books,
                 int cb, int M, int N, float *W, hipStream_t s);

/* The engine's LUT build, fma chain over the 8 dims per entry. */
int whip_lutb(const float *booksT, const float *x, int cb, int stages,
              int entries, int vec_dim, int nv, float *lut, hipStream_t s);

/* One VQ3R apply per job, each row's sum in the engine's exact order. */
typedef struct {
    float *y;
    const uint8_t *idx;
    const uint16_t *scale;
    const float *lut;
    int m, nv;
} whip_vq_job;
int whip_vq3r_jobs(const whip_vq_job *jobs, int n, hipStream_t s);

/* Table entries written in stream order, each header checked on the
 * device (bit 8 of err when one fails; that entry is left NULL). */
#define WHIP_BIND_MAX 64
typedef struct {
    int n;
    int expert[WHIP_BIND_MAX];
    const uint8_t *rec[WHIP_BIND_MAX];
    uint32_t layer, rec_4k_blocks, off_up, off_down, off_sc;
    int cb;                        /* required codebook id, -1 any          */
    int book0, n_books;            /* ids the layer holds: [book0, n_books - nbk] */
    uint32_t fmt, nbk;             /* the records' format and books per record */
} whip_bind_args;
int whip_bind(const uint8_t **recs, const whip_bind_args *a, int *err, hipStream_t s);
/* err &= ~mask, in stream order. */
int whip_err_clear(int *err, int mask, hipStream_t s);

/* One token: the router (job 0; its y = the logits, E rows) and up to two
 * more batch-1 products (the shared expert's gate/up) in one launch, and
 * the token routed as whip_route_gemv's routing does.  E <= 256 with xchg:
 * the router blocks tag their logits in xchg (1 + E 64-bit words of device
 * memory, zero before the first launch; word 0 holds the last launch's tag,
 * which each launch advances, words 1 .. E the tagged logits) and the last
 * router block routes once all carry this launch's tag.  Layers of any E
 * may share one exchange: tags only grow.  Otherwise the last router block to finish
 * routes; cnt: a device int, zero before the first launch; every launch
 * leaves it zero.  Launches that share xchg or cnt must not overlap. */
int whip_gemv_route(const whip_gemv_job *jobs, int n, const whip_route_cfg *c, const float *bias,
                    int32_t *ids, float *w, int32_t *pair_tok, int32_t *pair_exp, float *pair_w,
                    int32_t *tok_pairs, const uint8_t *const *recs, const uint8_t **pair_rec,
                    int *err, int *cnt, uint64_t *xchg, hipStream_t s);

/* whip_combine with the shared expert's down projection (shd . h_sh[t],
 * F32/Q8G/Q4G rows) computed in each block for its rows. */
int whip_combine_sh(const uint8_t *const *recs, const int32_t *pair_exp,
                    const float *pair_w, const int32_t *tok_pairs, int T, int K,
                    const float *part_d, int nch, int H, uint32_t sc_off_down,
                    int skip_zero, const whip_mat *shd, const float *h_sh, float *y,
                    hipStream_t s);
int whip_combine_sh_fold(const uint8_t *const *recs, const int32_t *pair_exp, const float *pair_w,
                         const int32_t *tok_pairs, int T, int K, const whip_fold *f, int H, int skip_zero,
                         const whip_mat *shd, const float *h_sh, float *y, hipStream_t s);

/* One token's routing (as whip_route with T = 1, plus pair_rec[j] = the
 * selected expert's record) and a batch-1 product that does not depend on
 * it (job; no paired matrix), in one launch. */
int whip_route_gemv(const whip_route_cfg *c, const float *logits, const float *bias,
                    int32_t *ids, float *w, int32_t *pair_tok, int32_t *pair_exp,
                    float *pair_w, int32_t *tok_pairs, const uint8_t *const *recs,
                    const uint8_t **pair_rec, int *err, const whip_gemv_job *job,
                    hipStream_t s);

/* ---- the static scratch area (scratch.hip) ---- */

/* Bytes of the area, and of its head: state that must start at zero (the
 * routing exchange, 1 + 1024 tagged words, and a block counter).  The area
 * is zero when the code object loads, and every launch leaves the head as
 * valid for the next (the counter back at zero, the tags only growing). */
#define WHIP_SCRATCH_BYTES (16u << 20)
#define WHIP_SCRATCH_HEAD  8704u
#define WHIP_SCRATCH_XCHG  0u                /* 1 + E 64-bit words, E <= 1024 */
#define WHIP_SCRATCH_RCNT  8448u             /* one int, zero between launches */
/* The current device's address of the area (hipGetSymbolAddress, once per
 * device). */
int whip_scratch(void **ptr);
/* Zeroes `bytes` (a multiple of 4) at p with a fill kernel on s. */
int whip_zero(void *p, size_t bytes, hipStream_t s);

#ifdef __cplusplus
}
#endif
#endif
