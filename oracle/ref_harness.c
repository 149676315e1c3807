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
 * moe_chunk (model.c:7203-7251).
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
    ref_init();
    waste_model *m = (waste_model *)calloc(1, sizeof *m);
    waste_config *c = &m->cfg;
    c->n_layers = 1; c->hidden = hidden; c->n_experts = n_experts;
    c->top_k = top_k; c->moe_inter = moe_inter; c->n_shared = n_shared;
    c->score_func = score_func; c->renorm = renorm;
    c->routed_scale = routed_scale;
    const int H = hidden, I = moe_inter, E = n_experts, K = top_k;
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
    m->n_books = n_books; m->vec_dim = 8; m->cb_entries = 256; m->stages = 3;
    m->index_bits = 8;
    m->expert_m[0] = m->expert_m[1] = I; m->expert_m[2] = H;
    m->expert_n[0] = m->expert_n[1] = H; m->expert_n[2] = I;

    const int fd = memfd_create("bank", 0);
    const size_t bank_bytes = rec_bytes * (size_t)E;
    if (fd < 0 || write(fd, bank, bank_bytes) != (ssize_t)bank_bytes) return -100;
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

    if (T == 1) {
        moe_layer(m, 0, x, out, route);
    } else {
        m->croute = (int *)calloc((size_t)T * K, sizeof(int));
        m->crw = (float *)calloc((size_t)T * K, sizeof(float));
        m->cused = (int *)calloc((size_t)E, sizeof(int));
        m->clat = (float *)calloc(2 * (size_t)T * H, sizeof(float));
        m->cq = (float *)calloc(((size_t)2 * T + 1) * lut_sz, sizeof(float));
        m->cff = (float *)calloc(2 * (size_t)I + H, sizeof(float));
        m->ckv = (float *)calloc(2 * (size_t)T * SI + (size_t)T * H, sizeof(float));
        m->chunk_cap = T;
        moe_chunk(m, 0, x, out, T);
        if (route) memcpy(route, m->croute, (size_t)T * K * sizeof(int));
        if (rw) memcpy(rw, m->crw, (size_t)T * K * sizeof(float));
        free(m->croute); free(m->crw); free(m->cused); free(m->clat);
        free(m->cq); free(m->cff); free(m->ckv);
    }
    const int err = m->read_error;
    close(fd);
    free(m->miss_buf); free(m->att); free(m->ff); free(m->e_gate);
    free(m->ares); free(m->h); free(m->lut); free(m->t);
    pthread_mutex_destroy(&m->fetch_mu);
    free(m);
    return err;
}
