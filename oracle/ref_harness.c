/* SPDX-License-Identifier: Apache-2.0 */
/*
 * ref_harness.c — entry points into the reference engine's own MoE code,
 * for writing golden vectors.  TEST INFRASTRUCTURE ONLY.
 *
 * oracle/Makefile compiles this file with the reference's flags and its
 * source directory on the include path, so the #include below is the
 * reference's src/model.c, compiled where it lies; the other engine
 * sources are compiled from there too and linked beside it into
 * oracle/_ref/libwasteref.so.  Nothing from the reference is copied into
 * this repository.  Including model.c is what reaches its static
 * functions (vq_rows, router_scores, moe_layer, moe_chunk).
 *
 * ref_moe() assembles the smallest waste_model those two functions read:
 * the config, a tensor table holding the router, bias and shared expert,
 * the codebook table, one expert bank served from a memfd through the
 * engine's own bank_fetch/record_check, and the scratch buffers
 * waste_model_load would size.  No expert cache, no lookahead, no
 * read-ahead: the serial paths of moe_layer (model.c:5876-5910) and
 * moe_chunk (model.c:7203-7251).  ref_moe_time() times moe_layer on the
 * same model with the engine's pool and an expert cache that holds the
 * bank, to calibrate the CPU baseline's restatement against it.
 */
#define _GNU_SOURCE
#include "model.c"

#include <sys/mman.h>

static waste_kernels ref_avx512, ref_portable;
static int ref_ready;

int ref_init(void)
{
    if (ref_ready) return ref_ready;
    waste_backend_init(WASTE_BE_NO_DEVICE);
    ref_avx512 = waste_k;
    ref_portable = waste_k;
    ref_portable.mvq_rows_f32 = waste_mvq_rows_f32;
    ref_portable.lutb_range = waste_lutb_range;
    ref_portable.vq_rows_p6 = waste_vq_rows_p6;
    ref_ready = (waste_k.lutb_range != waste_lutb_range) ? 2 : 1;
    return ref_ready;   /* 2: this host runs the AVX-512 kernels */
}

/* 0: universal C kernels; 1: whatever waste_backend_init chose (AVX-512
 * on an AVX-512F+BW host). */
void ref_set_order(int order)
{
    ref_init();
    waste_k = order ? ref_avx512 : ref_portable;
}

void ref_vq_rows(float *y, const uint8_t *idx, const uint16_t *scale,
                 const float *lut, int M, int nv, int stages, int entries)
{
    vq_arg a = { y, idx, scale, lut, nv, stages, entries };
    vq_rows(0, M, &a);
}

/* VQ4P: the engine's LUT quantisation (static in model.c) and its
 * vq_rows_p6 slot as installed for the order (the portable C kernel, or the
 * AVX-512 VBMI one on a host that has it). */
void ref_vq_quant_lut(const float *lut, int nv, int st, int en, int8_t *q, float *scale)
{
    vq_quant_lut(lut, nv, st, en, q, scale);
}

void ref_vq_rows_p6(float *y, const uint8_t *idx, const uint16_t *scale, const int8_t *lut8,
                    const float *lscale, int M, int nv)
{
    vqp_arg a = { y, idx, scale, lut8, lscale, nv };
    waste_k.vq_rows_p6(0, M, &a);
}

/* 1 when this host's engine runs the AVX-512 VBMI VQ4P kernel */
int ref_vq_p6_fast(void)
{
    ref_init();
    return ref_avx512.vq_rows_p6 != waste_vq_rows_p6;
}

void ref_lutb(float *lut, const float *booksT, const float *x, int cb_base,
              int stages, int entries, int vec_dim, int nv)
{
    lutb_arg a = { lut, booksT, x, cb_base, stages, entries, vec_dim };
    waste_k.lutb_range(0, nv, &a);
}

void ref_mvq_rows(float *y, const int8_t *W, const uint16_t *ws,
                  const float *x, int rows, int in, int group, int bits,
                  size_t rowbytes)
{
    mvq_arg a = { y, W, ws, NULL, x, in, (in + group - 1) / group, group,
                  bits, rowbytes };
    waste_k.mvq_rows_f32(0, rows, &a);
}

void ref_matvec_f32(float *y, const float *W, const float *x, int out, int in)
{
    matvec(y, W, x, out, in);
}

void ref_router_scores(int score_func, const float *logit, float *score, int E)
{
    waste_config c;
    memset(&c, 0, sizeof c);
    c.score_func = score_func;
    router_scores(&c, logit, score, E);
}

void ref_act_pair(float *g, const float *u, int n)
{
    waste_config c;
    memset(&c, 0, sizeof c);
    waste_act_pair_range(&c, g, u, n);
}

float ref_expf(float x) { return expf(x); }

typedef struct {
    int fmt, rows, cols, group;
    const void *q;
    const uint16_t *qs;
    size_t rowbytes;
} ref_tensor;

static void put_tensor(waste_tensor *t, const char *name, const ref_tensor *s)
{
    memset(t, 0, sizeof *t);
    snprintf(t->name, sizeof t->name, "%s", name);
    t->shape[0] = s->rows; t->shape[1] = s->cols; t->ndim = 2;
    t->n = (size_t)s->rows * s->cols;
    if (s->fmt == 0) { t->data = (float *)s->q; return; }
    t->q = (int8_t *)s->q;
    t->qs = (uint16_t *)s->qs;
    t->group = s->group;
    t->bits = s->fmt == 2 ? 8 : s->fmt == 3 ? 4 : 3;
    t->rowbytes = s->rowbytes;
}

/* The smallest waste_model moe_layer and moe_chunk read: the config, a
 * tensor table holding the router, bias and shared expert, the codebook
 * table, one expert bank served from a memfd through the engine's own
 * bank_fetch/record_check, and the scratch buffers waste_model_load would
 * size.  NULL on failure. */
/* The container geometry ref_model builds: index_bits 8 with three stages
 * of 256 entries (VQ3R) or two (VQ2R), or 6 (VQ4P, four stages of 64, with
 * the int8 table shadows waste_model_load allocates for it,
 * src/model.c:3340-3356). */
static int ref_ib = 8, ref_st = 3;

void ref_set_index_bits(int ib) { ref_ib = ib == 6 ? 6 : 8; ref_st = ib == 6 ? 4 : 3; }
void ref_set_stages(int st) { if (ref_ib == 8 && (st == 2 || st == 3)) ref_st = st; }

static waste_model *ref_model(int hidden, int n_experts, int top_k, int moe_inter, int n_shared,
                              int score_func, int renorm, float routed_scale,
                              const ref_tensor *router, const float *bias,
                              const ref_tensor *sh_gate, const ref_tensor *sh_up,
                              const ref_tensor *sh_down, const float *booksT, int n_books,
                              const uint8_t *bank, size_t rec_bytes)
{
    ref_init();
    waste_model *m = (waste_model *)calloc(1, sizeof *m);
    waste_config *c = &m->cfg;
    c->n_layers = 1; c->hidden = hidden; c->n_experts = n_experts;
    c->top_k = top_k; c->moe_inter = moe_inter; c->n_shared = n_shared;
    c->score_func = score_func; c->renorm = renorm;
    c->routed_scale = routed_scale;
    const int H = hidden, I = moe_inter, E = n_experts;
    const int SI = I * (n_shared ? n_shared : 1);

    m->t = (waste_tensor *)calloc(5, sizeof(waste_tensor));
    int nt = 0;
    if (router && router->rows)
        put_tensor(&m->t[nt++], "model.layers.0.block_sparse_moe.gate.weight", router);
    if (bias) {
        ref_tensor b = { 0, E, 1, 0, bias, NULL, 0 };
        put_tensor(&m->t[nt++], "model.layers.0.block_sparse_moe.gate.e_score_correction_bias", &b);
    }
    if (sh_gate && sh_gate->rows) {
        put_tensor(&m->t[nt++], "model.layers.0.block_sparse_moe.shared_experts.gate_proj.weight", sh_gate);
        put_tensor(&m->t[nt++], "model.layers.0.block_sparse_moe.shared_experts.up_proj.weight", sh_up);
        put_tensor(&m->t[nt++], "model.layers.0.block_sparse_moe.shared_experts.down_proj.weight", sh_down);
    }
    m->n_tensors = nt;

    m->codebooksT = (float *)booksT;
    m->n_books = n_books; m->vec_dim = 8;
    m->index_bits = ref_ib;
    m->stages = ref_st;
    m->cb_entries = ref_ib == 6 ? 64 : 256;
    m->expert_m[0] = m->expert_m[1] = I; m->expert_m[2] = H;
    m->expert_n[0] = m->expert_n[1] = H; m->expert_n[2] = I;

    const int fd = memfd_create("bank", 0);
    const size_t bank_bytes = rec_bytes * (size_t)E;
    size_t done = 0;
    while (fd >= 0 && done < bank_bytes) {
        const ssize_t w = write(fd, bank + done, bank_bytes - done);
        if (w <= 0) break;
        done += (size_t)w;
    }
    if (fd < 0 || done != bank_bytes) {
        if (fd >= 0) close(fd);
        free(m->t);
        free(m);
        return NULL;
    }
    m->bank[0].fd[0] = fd; m->bank[0].n_shards = 1;
    m->bank[0].rec_bytes = (int64_t)rec_bytes; m->bank[0].n_experts = E;
    m->miss_buf = (uint8_t *)aligned_alloc(4096, rec_bytes);
    pthread_mutex_init(&m->fetch_mu, NULL);

    const size_t lut_sz = (size_t)((H > I ? H : I) / 8) * 3 * 256;
    m->att = (float *)calloc(WASTE_ATT_ROUTER_OFF + 2 * (size_t)E + 64, sizeof(float));
    m->ff = (float *)calloc(2 * (size_t)(SI > I ? SI : I) + 64, sizeof(float));
    m->e_gate = (float *)calloc((size_t)H, sizeof(float));
    m->ares = (float *)calloc(3 * (size_t)H, sizeof(float));
    m->h = (float *)calloc((size_t)H, sizeof(float));
    m->lut = (float *)calloc(3 * lut_sz, sizeof(float));
    m->lut_bytes = 3 * lut_sz * sizeof(float);
    if (ref_ib == 6) {
        const size_t nvmax = (size_t)((H > I ? H : I) / 8);
        m->lut8 = (int8_t *)calloc(3 * nvmax * 4 * 64, 1);
        m->lut8_scale = (float *)calloc(3 * (nvmax / WASTE_VQ_LUT_BLK + 2), sizeof(float));
    }
    return m;
}

static void ref_model_free(waste_model *m)
{
    close(m->bank[0].fd[0]);
    free(m->miss_buf); free(m->att); free(m->ff); free(m->e_gate);
    free(m->ares); free(m->h); free(m->lut); free(m->t);
    free(m->lut8); free(m->lut8_scale);
    pthread_mutex_destroy(&m->fetch_mu);
    free(m);
}

/* Runs moe_layer (T == 1) or moe_chunk (T > 1) over `bank`, E records of
 * rec_bytes each, layer 0.  route/rw receive the chunk's routing (T > 1)
 * or the decode ids (T == 1, rw untouched).  Returns the model's read
 * error (0 when every record passed record_check). */
int ref_moe(int hidden, int n_experts, int top_k, int moe_inter, int n_shared,
            int score_func, int renorm, float routed_scale,
            const ref_tensor *router, const float *bias,
            const ref_tensor *sh_gate, const ref_tensor *sh_up,
            const ref_tensor *sh_down,
            const float *booksT, int n_books,
            const uint8_t *bank, size_t rec_bytes,
            const float *x, int T, float *out, int *route, float *rw)
{
    waste_model *m = ref_model(hidden, n_experts, top_k, moe_inter, n_shared, score_func, renorm,
                               routed_scale, router, bias, sh_gate, sh_up, sh_down, booksT, n_books,
                               bank, rec_bytes);
    if (!m) return -100;
    const int H = hidden, I = moe_inter, E = n_experts, K = top_k;
    const int SI = I * (n_shared ? n_shared : 1);
    const size_t lut_sz = (size_t)((H > I ? H : I) / 8) * 3 * 256;
    if (T == 1) {
        moe_layer(m, 0, x, out, route);
    } else {
        m->croute = (int *)calloc((size_t)T * K, sizeof(int));
        m->crw = (float *)calloc((size_t)T * K, sizeof(float));
        m->cused = (int *)calloc((size_t)E, sizeof(int));
        m->clat = (float *)calloc(2 * (size_t)T * H, sizeof(float));
        m->cq = (float *)calloc(((size_t)2 * T + 1) * lut_sz, sizeof(float));
        if (ref_ib == 6) {      /* moe_chunk's int8 shadows, src/model.c:7052-7065 */
            const size_t nvmax = (size_t)((H > I ? H : I) / 8);
            m->cq8 = (int8_t *)calloc(((size_t)2 * T + 1) * nvmax * 4 * 64 + 64, 1);
            m->cq8_scale = (float *)calloc(((size_t)2 * T + 1) * (nvmax / WASTE_VQ_LUT_BLK + 2) + 64,
                                           sizeof(float));
        }
        m->cff = (float *)calloc(2 * (size_t)I + H, sizeof(float));
        m->ckv = (float *)calloc(2 * (size_t)T * SI + (size_t)T * H, sizeof(float));
        m->chunk_cap = T;
        moe_chunk(m, 0, x, out, T);
        if (route) memcpy(route, m->croute, (size_t)T * K * sizeof(int));
        if (rw) memcpy(rw, m->crw, (size_t)T * K * sizeof(float));
        free(m->croute); free(m->crw); free(m->cused); free(m->clat);
        free(m->cq); free(m->cff); free(m->ckv);
        free(m->cq8); free(m->cq8_scale);
        m->cq8 = NULL; m->cq8_scale = NULL;
    }
    const int err = m->read_error;
    ref_model_free(m);
    return err;
}

/* Seconds moe_layer takes over ntok tokens (xs[ntok][hidden]) with the
 * engine's pool at nthreads and an expert cache that holds every record,
 * after one untimed pass over the same tokens has made each routed record
 * resident: the timed pass is the decode path's arithmetic (the per-expert
 * loop, model.c:5876-5910, each matrix's rows split over the pool,
 * src/threads.h:325-341) with no bank reads.  The pool is shut down again
 * afterwards, so the other entry points stay serial.  out: the last
 * token's output.  < 0 on failure. */
double ref_moe_time(int hidden, int n_experts, int top_k, int moe_inter, int n_shared,
                    int score_func, int renorm, float routed_scale,
                    const ref_tensor *router, const float *bias,
                    const ref_tensor *sh_gate, const ref_tensor *sh_up,
                    const ref_tensor *sh_down,
                    const float *booksT, int n_books,
                    const uint8_t *bank, size_t rec_bytes,
                    const float *xs, int ntok, int nthreads, float *out)
{
    if (ntok <= 0 || top_k > 64) return -1.0;
    waste_model *m = ref_model(hidden, n_experts, top_k, moe_inter, n_shared, score_func, renorm,
                               routed_scale, router, bias, sh_gate, sh_up, sh_down, booksT, n_books,
                               bank, rec_bytes);
    if (!m) return -1.0;
    waste_pool_shutdown();
    waste_pool_init(nthreads, NULL);
    double r = -2.0;
    if (waste_ecache_init(&m->cache, (size_t)n_experts * rec_bytes, rec_bytes, 0) == 0) {
        int route[64];
        for (int t = 0; t < ntok; t++) moe_layer(m, 0, xs + (size_t)t * hidden, out, route);
        struct timespec a, b;
        clock_gettime(CLOCK_MONOTONIC, &a);
        for (int t = 0; t < ntok; t++) moe_layer(m, 0, xs + (size_t)t * hidden, out, route);
        clock_gettime(CLOCK_MONOTONIC, &b);
        r = m->read_error ? -3.0 : (double)(b.tv_sec - a.tv_sec) + 1e-9 * (double)(b.tv_nsec - a.tv_nsec);
        waste_ecache_free(&m->cache);
    }
    waste_pool_shutdown();
    ref_model_free(m);
    return r;
}

/* ---- the engine's expert cache, scripted --------------------------------
 *
 * ref_ecache_run() drives src/ecache.c itself through a script of calls and
 * reports the slot each demand call returned.  With readers (depth > 0) the
 * engine's in-flight reads finish whenever the threads get to them; to make
 * a run repeatable, the reader threads' fetch waits on a gate that opens
 * only just before each get/hold, until every in-flight read has landed.
 * Reads therefore finish exactly "by the next demand get", which is the
 * order the deterministic restatement assumes.  Demand and admit reads run
 * on the calling thread and return at once.
 *
 * Script words: 0 L e get | 1 L e hold | 2 release | 3 L n ids.. hint |
 * 4 L n ids.. prefetch | 5 L e admit.  out[] gets one int per get/hold
 * (slot, -1 NULL) and per admit (its return).  stats: hits, misses,
 * evictions, prefetched, spec_issued, bytes_read / rec_bytes.
 * Returns the number of out[] entries, or -1. */
static pthread_t ref_main;
static int ref_gate;

static int ref_fetch(void *user, int layer, int expert, uint8_t *dst)
{
    (void)user;
    if (!pthread_equal(pthread_self(), ref_main))
        while (!__atomic_load_n(&ref_gate, __ATOMIC_ACQUIRE)) usleep(20);
    const int32_t key = (layer << 16) | expert;
    memcpy(dst, &key, sizeof key);
    return 0;
}

static void ref_quiesce(waste_ecache *c)
{
    if (!c->io) return;
    __atomic_store_n(&ref_gate, 1, __ATOMIC_RELEASE);
    for (;;) {
        int busy = 0;
        for (int i = 0; i < c->n_slots && !busy; i++)
            busy = __atomic_load_n(&c->slot[i].state, __ATOMIC_ACQUIRE) == EC_INFLIGHT;
        if (!busy) break;
        usleep(20);
    }
    __atomic_store_n(&ref_gate, 0, __ATOMIC_RELEASE);
}

static int ref_slot_of(const waste_ecache *c, const uint8_t *p)
{
    if (!p) return -1;
    for (int i = 0; i < c->n_slots; i++)
        if (c->slot[i].data == p) return i;
    return -2;
}

/* Usage files for the next ref_ecache_run: warm from `warm` after init,
 * save to `save` (tokens = the cache's clock) after the script; NULL for
 * neither.  ref_ecache_warmed() is the last warm's return. */
static char ref_warm_path[4096], ref_save_path[4096];
static int ref_warm_n;

void ref_ecache_usage(const char *warm, const char *save)
{
    snprintf(ref_warm_path, sizeof ref_warm_path, "%s", warm ? warm : "");
    snprintf(ref_save_path, sizeof ref_save_path, "%s", save ? save : "");
}

int ref_ecache_warmed(void) { return ref_warm_n; }

int ref_ecache_run(int n_slots, int depth, int policy, const int *ops, int n_words, int *out,
                   uint64_t stats[6])
{
    const size_t rec = 4096;
    waste_ecache c;
    memset(&c, 0, sizeof c);
    if (waste_ecache_init(&c, (size_t)n_slots * rec, rec, policy)) return -1;
    ref_main = pthread_self();
    __atomic_store_n(&ref_gate, 0, __ATOMIC_RELEASE);
    if (depth > 0) waste_ecache_io_start(&c, ref_fetch, NULL, 2, depth);
    ref_warm_n = ref_warm_path[0] ? waste_ecache_warm(&c, ref_warm_path, ref_fetch, NULL) : 0;
    int n_out = 0, bad = 0;
    for (int w = 0; w < n_words && !bad;) {
        const int op = ops[w];
        if (op == 0 || op == 1) {
            ref_quiesce(&c);
            const uint8_t *p = op == 0 ? waste_ecache_get(&c, ops[w + 1], ops[w + 2], ref_fetch, NULL)
                                       : waste_ecache_hold(&c, ops[w + 1], ops[w + 2], ref_fetch, NULL);
            const int si = ref_slot_of(&c, p);
            int32_t k;
            if (p) memcpy(&k, p, sizeof k);
            if (si == -2 || (p && k != ((ops[w + 1] << 16) | ops[w + 2]))) bad = 1;
            out[n_out++] = si;
            w += 3;
        } else if (op == 2) {
            waste_ecache_release(&c);
            w += 1;
        } else if (op == 3 || op == 4) {
            const int n = ops[w + 2];
            if (op == 3) waste_ecache_hint(&c, ops[w + 1], ops + w + 3, n);
            else waste_ecache_prefetch(&c, ops[w + 1], ops + w + 3, n);
            w += 3 + n;
        } else if (op == 5) {
            out[n_out++] = waste_ecache_admit(&c, ops[w + 1], ops[w + 2], ref_fetch, NULL);
            w += 3;
        } else {
            bad = 1;
        }
    }
    ref_quiesce(&c);
    if (ref_save_path[0] && waste_ecache_save_usage(&c, ref_save_path, c.clock)) bad = 1;
    stats[0] = c.hits; stats[1] = c.misses; stats[2] = c.evictions;
    stats[3] = c.prefetched; stats[4] = c.spec_issued; stats[5] = c.bytes_read / rec;
    waste_ecache_io_stop(&c);
    waste_ecache_free(&c);
    return bad ? -1 : n_out;
}
