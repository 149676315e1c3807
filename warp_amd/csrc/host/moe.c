/* SPDX-License-Identifier: Apache-2.0 */
/*
 * moe.c — the device MoE layer: host orchestration of the gfx950 kernels.
 *
 * One forward enqueues, on the caller's stream:
 *   [bf16->fp32] -> router GEMV -> route (+ pair list) -> shared gate/up
 *   GEMV -> VQ3R gate/up apply -> SwiGLU (routed + shared) -> VQ3R down
 *   apply -> shared down GEMV -> combine.
 * Everything it reads is resident in HBM: expert records in a slab owned
 * by the layer (or bound from an expert-cache slot), codebooks as fp32,
 * the router and shared expert in their stored formats.
 *
 * Host-side semantics follow the engine: records are checked as
 * record_check does before the device ever reads them
 * (src/model.c:3645-3692); the layer's gate/up tables use the codebook id
 * of the records (src/model.c:5844-5849), which must agree across the
 * layer's experts; an unbound or unroutable expert is reported through a
 * sticky error, as the engine's read_error is (src/model.c:3698-3712).
 */
#include "waste_hip.h"
#include "../hip/launch.h"

#include <hip/hip_runtime_api.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define CK(call) do { if ((call) != hipSuccess) return WASTE_HIP_EDEVICE; } while (0)
#define P6_PAIR_CHUNK 256        /* VQ4P pairs whose block sums one pass holds */

/* The device buffers one forward writes and reads back: logits, the
 * selection and its pair lists, the expert partials, the shared expert's
 * activations, the routing launch's exchange.  A layer owns one set
 * (allocated at create); waste_hip_moe_forward_static points them into the
 * library's static scratch area for one call instead. */
typedef struct {
    float *logits;               /* [T][E]                                  */
    float *w, *pair_w;           /* [P]                                     */
    int32_t *ids, *pair_tok, *pair_exp, *tok_pairs;   /* [P]                */
    float *part_gu;              /* [P][2][nch_gu][I] + 64 (a sink)         */
    float *h;                    /* [P][I] (widths the fused SwiGLU misses) */
    float *part_d;               /* [P][nch_d][H] + 64                      */
    float *h_sh;                 /* [T][SI] the shared expert's SwiGLU      */
    float *sh_out;               /* [T][H] its down projection              */
    const uint8_t **pair_rec;    /* [64] records of a T = 1 route's pairs   */
    int *rcnt;                   /* the routing launch's block counter (0)  */
    uint64_t *xchg;              /* [E + 1] its tagged logits, last tag     */
    float *sk_part;              /* column-slice partials of the few-token
                                    products (NULL: the GEMV kernels)       */
} fwd_bufs;

struct waste_hip_moe {
    waste_hip_moe_cfg c;
    int E, K, H, I, SI, T;
    int Td;                      /* most tokens the decode kernels take    */
    int nv_gu, nv_d, nch_gu, nch_d, rsplit_gu, rsplit_d;
    size_t idx_gu, idx_d, rec_min, rec_bytes;
    uint32_t off_gate, off_up, off_down, off_sc;
    int cb;                      /* codebook id shared by the layer (-1)   */
    int bound;                   /* records bound                          */
    /* device */
    const uint8_t **d_recs;      /* [E + 1]; entry E stays NULL            */
    const uint8_t **h_recs;
    uint8_t *slab;               /* owned records, E x rec_bytes (lazy)    */
    float *d_books, *d_booksT;
    uint16_t *d_books16;         /* fp16, subnormals flushed (prefill)     */
    int n_books;                 /* books held, ids [book0, book0 + n_books) */
    int book0;
    whip_mat router, sh[3];
    void *router_mem, *sh_mem[3];
    float *d_bias;
    int has_router, has_shared;
    fwd_bufs b;                  /* the forward's buffers (see fwd_bufs)    */
    /* many-token path (T > Td) */
    int32_t *pair_pos, *seg_off, *order;
    uint16_t *h16, *sh_h16;      /* fp16 [P][I], [T][SI]                   */
    uint16_t *x16;               /* the chunk's activations, fp16 [T][H]    */
    float *ypair, *rpart;        /* [P][H]; router partial sums            */
    int *err;                    /* [0] status bits; [4] the lookahead's    */
    float *plogits, *pw;         /* the lookahead's logits and weights      */
    int routed_T;                /* T of the last route(), 0 none          */
    int32_t *h_sel;              /* pinned: selection [0,64), lookahead [64,128) */
    int *h_err;                  /* pinned: the error word, read after a chunk */
    int32_t *r_ids;              /* the last route's ids and weights (device) */
    float *r_w;
    int pair_rec_ok;             /* pair_rec matches the table (no bind since) */
    int sh_done;                 /* the route's launch ran the shared down  */
    int sh_in_combine;           /* the combine runs the shared down        */
    int32_t *d_look;             /* the lookahead's ids                    */
    int look_groups;             /* predict applies the group limit        */
    /* VQ4P experts (index_bits 6): four stages of 64 entries, 12 books a
     * record; every T on the decode path */
    int p6, stages, entries, nbk;
    int r2;                      /* VQ2R experts: two stages of 256 entries */
    int bpp;                     /* index bytes a (row, position)          */
    struct {
        float *lut_gu, *lut_d;   /* VQ2R: fp32 tables [T][2][nv_gu][512], [P][nv_d][512] */
        int8_t *q_gu, *q_d;      /* VQ4P: int8 tables [T][2][nv_gu][256], [P][nv_d][256] */
        float *s_gu, *s_d;       /* and their scales, one per 32 positions */
        int16_t *S_gu, *S_d;     /* VQ4P block sums [P][2][nb_gu][I], [P][nb_d][H] */
        float *gu, *down;        /* VQ2R: rows [P][2][I], down [P][H]; VQ4P
                                    above P6_PAIR_CHUNK pairs: down [P][H] */
    } p6b;
    /* few-token products on the matrix cores (skinny.hip): column slices of
     * the router, the shared gate/up and the shared down (0: not taken),
     * and the partials' buffer, Td tokens' worth */
    int sk_r, sk_g, sk_d;
    float *sk_mem;
    size_t sk_cap;
    int prof_on;
    hipEvent_t ev[WASTE_HIP_STAGES + 1];
    hipEvent_t kev[2 * WASTE_HIP_STAGES];   /* per-stage kernel start/stop   */
    unsigned ktimed;             /* stages timed by their kernel this forward */
    waste_hip_moe_prof prof;
};

static float f16_book(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1f, mn = h & 0x3ff;
    const uint32_t b = e ? (sign | ((e + 112u) << 23) | (mn << 13)) : sign;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

/* The layer's codebook id is known and its nine books are on the device. */
static int books_ok(const waste_hip_moe *m)
{
    return m->cb >= m->book0 && m->cb + m->nbk <= m->book0 + m->n_books;
}

static int dmalloc(void **p, size_t n)
{
    *p = NULL;
    if (n == 0) return 0;
    return hipMalloc(p, n) == hipSuccess ? 0 : WASTE_HIP_ENOMEM;
}

const char *waste_hip_device_name(void)
{
    static char name[300];
    int n = 0, dev = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return NULL;
    if (hipGetDevice(&dev) != hipSuccess) return NULL;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, dev) != hipSuccess) return NULL;
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0) return NULL;
    snprintf(name, sizeof name, "HIP %s", p.gcnArchName);
    return name;
}

void waste_hip_moe_destroy(waste_hip_moe *m)
{
    if (!m) return;
    void *bufs[] = { m->d_recs, m->slab, m->d_books, m->d_booksT, m->router_mem,
                     m->sh_mem[0], m->sh_mem[1], m->sh_mem[2], m->d_bias,
                     m->b.logits, m->b.w, m->b.pair_w, m->b.part_gu, m->b.h, m->b.part_d,
                     m->b.h_sh, m->b.sh_out, m->b.ids, m->b.pair_tok, m->b.pair_exp,
                     m->b.tok_pairs, m->err, m->pair_pos, m->seg_off, m->order, m->h16,
                     m->sh_h16, m->x16, m->ypair, m->rpart, m->d_books16, m->plogits, m->pw, m->d_look, (void *)m->b.pair_rec,
                     m->b.rcnt, m->b.xchg, m->sk_mem, m->p6b.lut_gu, m->p6b.lut_d, m->p6b.q_gu,
                     m->p6b.q_d, m->p6b.s_gu, m->p6b.s_d, m->p6b.S_gu, m->p6b.S_d, m->p6b.gu,
                     m->p6b.down };
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++) if (bufs[i]) hipFree(bufs[i]);
    if (m->ev[0]) {
        for (int i = 0; i <= WASTE_HIP_STAGES; i++) hipEventDestroy(m->ev[i]);
        for (int i = 0; i < 2 * WASTE_HIP_STAGES; i++) hipEventDestroy(m->kev[i]);
    }
    if (m->h_sel) hipHostFree(m->h_sel);
    if (m->h_err) hipHostFree(m->h_err);
    free(m->h_recs);
    free(m);
}

/* splits of a spanning launch: about 1024 workgroups (four 512-thread
 * workgroups on each of 256 CUs), at least one row block per wavefront */
static int pick_span_split(int work_groups, int row_blocks)
{
    int r = (1024 + work_groups - 1) / (work_groups > 0 ? work_groups : 1);
    const int cap = row_blocks / 8 > 0 ? row_blocks / 8 : 1;
    if (r > cap) r = cap;
    return r < 1 ? 1 : r;
}

static int pick_rsplit(int work_groups, int row_blocks)
{
    /* enough workgroups to cover 256 CUs a few times, at least one row
     * block per wavefront of an 8-wave workgroup */
    int r = (768 + work_groups - 1) / (work_groups > 0 ? work_groups : 1);
    const int cap = row_blocks / 8 > 0 ? row_blocks / 8 : 1;
    if (r > cap) r = cap;
    return r < 1 ? 1 : r;
}

int waste_hip_moe_create(const waste_hip_moe_cfg *cfg, waste_hip_moe **out)
{
    *out = NULL;
    if (!cfg || cfg->hidden <= 0 || cfg->hidden % 64 || cfg->moe_inter <= 0 ||
        cfg->moe_inter % 64 || cfg->n_experts <= 0 || cfg->n_experts > 1024 ||
        cfg->top_k <= 0 || cfg->top_k > 64 || cfg->top_k > cfg->n_experts ||
        cfg->max_tokens <= 0 || cfg->score_func < 0 || cfg->score_func > 2)
        return WASTE_HIP_EINVAL;
    if (cfg->n_group > 1 && (cfg->n_experts % cfg->n_group || cfg->n_group > 64 ||
                             cfg->topk_group < 1 || cfg->topk_group > cfg->n_group ||
                             cfg->topk_group * (cfg->n_experts / cfg->n_group) < cfg->top_k))
        return WASTE_HIP_EINVAL;
    if (cfg->index_bits != 0 && cfg->index_bits != 8 && cfg->index_bits != 6) return WASTE_HIP_EINVAL;
    if (cfg->index_bits == 6 ? cfg->stages != 0 && cfg->stages != 4
                             : cfg->stages != 0 && cfg->stages != 3 && cfg->stages != 2)
        return WASTE_HIP_EINVAL;
    if ((cfg->index_bits == 6 || cfg->stages == 2) && cfg->p6_order != WASTE_HIP_ORDER_PORTABLE &&
        cfg->p6_order != WASTE_HIP_ORDER_FMA)
        return WASTE_HIP_EINVAL;
    if (!waste_hip_device_name()) return WASTE_HIP_ENODEV;
    waste_hip_moe *m = (waste_hip_moe *)calloc(1, sizeof *m);
    if (!m) return WASTE_HIP_ENOMEM;
    m->c = *cfg;
    m->E = cfg->n_experts; m->K = cfg->top_k; m->H = cfg->hidden; m->I = cfg->moe_inter;
    m->SI = cfg->moe_inter * (cfg->n_shared > 0 ? cfg->n_shared : 1);
    m->T = cfg->max_tokens;
    m->p6 = cfg->index_bits == 6;
    m->r2 = !m->p6 && cfg->stages == 2;
    m->stages = m->p6 ? 4 : m->r2 ? 2 : 3;
    m->entries = m->p6 ? 64 : 256;
    m->nbk = 3 * m->stages;
    m->bpp = m->p6 ? 3 : m->stages;
    {
        /* VQ4P and VQ2R: the decode path takes every T (no matrix-core path) */
        const int pm = cfg->prefill_min_tokens > 0 ? cfg->prefill_min_tokens : 32;
        m->Td = m->T < pm || m->p6 || m->r2 ? m->T : pm;
    }
    m->nv_gu = m->H / 8; m->nv_d = m->I / 8;
    m->nch_gu = whip_vq_chunks(m->nv_gu, m->I);
    m->nch_d = whip_vq_chunks(m->nv_d, m->H);
    /* canonical record layout (tools/convert.py:942-977): 48 B header,
     * gate, up, down index streams, then f16 scales gate|up|down */
    m->idx_gu = (size_t)m->I * m->nv_gu * m->bpp;
    m->idx_d = (size_t)m->H * m->nv_d * m->bpp;
    m->off_gate = 48;
    m->off_up = (uint32_t)(48 + m->idx_gu);
    m->off_down = (uint32_t)(48 + 2 * m->idx_gu);
    m->off_sc = (uint32_t)(48 + 2 * m->idx_gu + m->idx_d);
    m->rec_min = m->off_sc + 2 * (size_t)(2 * m->I + m->H);
    m->rec_bytes = (m->rec_min + 4095) / 4096 * 4096;
    m->cb = -1;
    const int P = m->T * m->K, Pd = m->Td * m->K;
    m->rsplit_gu = pick_rsplit(m->nch_gu * 2 * m->K, m->I / 64);
    m->rsplit_d = pick_rsplit(m->nch_d * m->K, m->H / 64);
    m->h_recs = (const uint8_t **)calloc((size_t)m->E + 1, sizeof(void *));
    int rc = 0;
    rc |= dmalloc((void **)&m->d_recs, ((size_t)m->E + 1) * sizeof(void *));
    rc |= dmalloc((void **)&m->b.logits, (size_t)m->T * m->E * 4);
    rc |= dmalloc((void **)&m->b.ids, (size_t)P * 4);
    rc |= dmalloc((void **)&m->b.w, (size_t)P * 4);
    rc |= dmalloc((void **)&m->b.pair_tok, (size_t)P * 4);
    rc |= dmalloc((void **)&m->b.pair_exp, (size_t)P * 4);
    rc |= dmalloc((void **)&m->b.pair_w, (size_t)P * 4);
    rc |= dmalloc((void **)&m->b.tok_pairs, (size_t)P * 4);
    if (m->r2) {
        const size_t tg = (size_t)m->nv_gu * 2 * 256, td = (size_t)m->nv_d * 2 * 256;
        rc |= dmalloc((void **)&m->p6b.lut_gu, (size_t)m->T * 2 * tg * 4);
        rc |= dmalloc((void **)&m->p6b.lut_d, (size_t)P * td * 4);
        rc |= dmalloc((void **)&m->p6b.gu, (size_t)P * 2 * m->I * 4);
        rc |= dmalloc((void **)&m->p6b.down, (size_t)P * m->H * 4);
    } else if (m->p6) {
        /* the pair buffers hold one chunk of at most P6_PAIR_CHUNK pairs;
         * more pairs fold their down rows into p6b.down */
        const size_t tg = (size_t)m->nv_gu * 256, td = (size_t)m->nv_d * 256;
        const size_t bg = (size_t)(m->nv_gu + 31) / 32, bd = (size_t)(m->nv_d + 31) / 32;
        const size_t Pc = P < P6_PAIR_CHUNK ? (size_t)P : P6_PAIR_CHUNK;
        if (m->T > 1) {
            rc |= dmalloc((void **)&m->p6b.q_gu, (size_t)m->T * 2 * tg);
            rc |= dmalloc((void **)&m->p6b.q_d, Pc * td);
        }
        rc |= dmalloc((void **)&m->p6b.s_gu, (size_t)m->T * 2 * bg * 4);
        rc |= dmalloc((void **)&m->p6b.s_d, Pc * bd * 4);
        rc |= dmalloc((void **)&m->p6b.S_gu, Pc * 2 * bg * m->I * 2);
        rc |= dmalloc((void **)&m->p6b.S_d, Pc * bd * m->H * 2);
        if ((size_t)P > Pc) rc |= dmalloc((void **)&m->p6b.down, (size_t)P * m->H * 4);
    } else {
        /* + 64 floats: the apply kernels' sink for rows past a split's end */
        rc |= dmalloc((void **)&m->b.part_gu, ((size_t)Pd * 2 * m->nch_gu * m->I + 64) * 4);
        rc |= dmalloc((void **)&m->b.h, (size_t)Pd * m->I * 4);
        rc |= dmalloc((void **)&m->b.part_d, ((size_t)Pd * m->nch_d * m->H + 64) * 4);
    }
    rc |= dmalloc((void **)&m->err, 64);
    rc |= dmalloc((void **)&m->plogits, (size_t)m->E * 4);
    rc |= dmalloc((void **)&m->pw, 64 * 4);
    rc |= dmalloc((void **)&m->d_look, 64 * 4);
    rc |= dmalloc((void **)&m->b.pair_rec, 64 * sizeof(void *));
    rc |= dmalloc((void **)&m->b.rcnt, 256);
    rc |= dmalloc((void **)&m->b.xchg, ((size_t)m->E + 1) * 8);
    if (m->T > m->Td) {
        rc |= dmalloc((void **)&m->pair_pos, (size_t)P * 4);
        rc |= dmalloc((void **)&m->seg_off, ((size_t)m->E + 2) * 4);
        rc |= dmalloc((void **)&m->order, (size_t)m->E * 4);
        rc |= dmalloc((void **)&m->h16, (size_t)P * m->I * 2);
        rc |= dmalloc((void **)&m->x16, (size_t)m->T * m->H * 2);
        rc |= dmalloc((void **)&m->ypair, (size_t)P * m->H * 4);
        rc |= dmalloc((void **)&m->rpart, whip_pf_router_part_floats(m->T, m->E) * 4);
    }
    if (rc || !m->h_recs) { waste_hip_moe_destroy(m); return WASTE_HIP_ENOMEM; }
    if (hipMemset(m->d_recs, 0, ((size_t)m->E + 1) * sizeof(void *)) != hipSuccess ||
        hipMemset(m->err, 0, 64) != hipSuccess ||
        hipMemset(m->b.rcnt, 0, 256) != hipSuccess || hipMemset(m->b.xchg, 0, ((size_t)m->E + 1) * 8) != hipSuccess) {
        waste_hip_moe_destroy(m);
        return WASTE_HIP_EDEVICE;
    }
    *out = m;
    return 0;
}

/* Uploads a trunk tensor: payload (+ scales) in one allocation. */
static int upload_tensor(const waste_hip_tensor *t, int rows, int cols, whip_mat *dst, void **mem)
{
    if (!t || !t->q || t->rows != rows || t->cols != cols) return WASTE_HIP_EINVAL;
    if (t->fmt != WQ_F32 && t->fmt != WQ_Q8G && t->fmt != WQ_Q4G) return WASTE_HIP_EINVAL;
    size_t qbytes = (size_t)rows * t->rowbytes, sbytes = 0;
    if (t->fmt == WQ_F32) {
        if (t->rowbytes < (size_t)cols * 4 || cols % 4 || t->rowbytes % 16) return WASTE_HIP_EINVAL;
    } else {
        if (t->group <= 0 || t->group % 32 || t->rowbytes % 16 || !t->qs) return WASTE_HIP_EINVAL;
        const int ng = (cols + t->group - 1) / t->group;
        const size_t need = t->fmt == WQ_Q8G ? (size_t)ng * t->group : (size_t)ng * t->group / 2;
        if (t->rowbytes < need) return WASTE_HIP_EINVAL;
        sbytes = (size_t)rows * ng * 2;
    }
    if (*mem) { hipFree(*mem); *mem = NULL; }
    const size_t qpad = (qbytes + 255) / 256 * 256;
    if (dmalloc(mem, qpad + sbytes)) return WASTE_HIP_ENOMEM;
    CK(hipMemcpy(*mem, t->q, qbytes, hipMemcpyHostToDevice));
    if (sbytes) CK(hipMemcpy((uint8_t *)*mem + qpad, t->qs, sbytes, hipMemcpyHostToDevice));
    dst->fmt = t->fmt; dst->rows = rows; dst->cols = cols; dst->group = t->group;
    dst->q = *mem;
    dst->qs = sbytes ? (const uint16_t *)((uint8_t *)*mem + qpad) : NULL;
    dst->rowbytes = t->rowbytes;
    return 0;
}

/* The few-token products' column slices for the trunk tensors held now, and
 * a partials buffer for Td tokens of the larger of the two launches (the
 * router with the shared gate/up; the shared down).  Without a router, or
 * with a shape the matrix-core kernel does not take, the GEMV kernels run. */
static int sk_setup(waste_hip_moe *m)
{
    m->sk_r = m->has_router && m->Td > 1 ? whip_sk_slices(&m->router) : 0;
    m->sk_g = m->sk_r && m->has_shared ? whip_sk_slices(&m->sh[0]) : 0;
    m->sk_d = m->sk_r && m->has_shared ? whip_sk_slices(&m->sh[2]) : 0;
    if (m->has_shared && (!m->sk_g || !m->sk_d)) m->sk_r = m->sk_g = m->sk_d = 0;
    m->b.sk_part = NULL;
    if (!m->sk_r) return 0;
    const size_t a = (size_t)m->sk_r * m->E + 2 * (size_t)m->sk_g * m->SI;
    const size_t d = (size_t)m->sk_d * m->H;
    const size_t need = (size_t)m->Td * (a > d ? a : d) * 4;
    if (need > m->sk_cap) {
        if (m->sk_mem) hipFree(m->sk_mem);
        m->sk_cap = 0;
        if (dmalloc((void **)&m->sk_mem, need)) {
            m->sk_r = m->sk_g = m->sk_d = 0;
            return WASTE_HIP_ENOMEM;
        }
        m->sk_cap = need;
    }
    m->b.sk_part = m->sk_mem;
    return 0;
}

int waste_hip_moe_set_router(waste_hip_moe *m, const waste_hip_tensor *gate, const float *bias)
{
    if (!m) return WASTE_HIP_EINVAL;
    int rc = upload_tensor(gate, m->E, m->H, &m->router, &m->router_mem);
    if (rc) return rc;
    if (m->d_bias) { hipFree(m->d_bias); m->d_bias = NULL; }
    if (bias) {
        if (dmalloc((void **)&m->d_bias, (size_t)m->E * 4)) return WASTE_HIP_ENOMEM;
        CK(hipMemcpy(m->d_bias, bias, (size_t)m->E * 4, hipMemcpyHostToDevice));
    }
    m->has_router = 1;
    return sk_setup(m);
}

int waste_hip_moe_set_shared(waste_hip_moe *m, const waste_hip_tensor *gate,
                             const waste_hip_tensor *up, const waste_hip_tensor *down)
{
    if (!m) return WASTE_HIP_EINVAL;
    if (!gate && !up && !down) { m->has_shared = 0; return sk_setup(m); }
    int rc = upload_tensor(gate, m->SI, m->H, &m->sh[0], &m->sh_mem[0]);
    if (!rc) rc = upload_tensor(up, m->SI, m->H, &m->sh[1], &m->sh_mem[1]);
    if (!rc) rc = upload_tensor(down, m->H, m->SI, &m->sh[2], &m->sh_mem[2]);
    if (rc) return rc;
    if (gate->fmt != up->fmt || gate->group != up->group) return WASTE_HIP_EINVAL;
    if (!m->b.h_sh) {
        rc |= dmalloc((void **)&m->b.h_sh, (size_t)m->Td * m->SI * 4);
        rc |= dmalloc((void **)&m->b.sh_out, (size_t)m->T * m->H * 4);
        if (m->T > m->Td) rc |= dmalloc((void **)&m->sh_h16, (size_t)m->T * m->SI * 2);
        if (rc) return WASTE_HIP_ENOMEM;
    }
    m->has_shared = 1;
    return sk_setup(m);
}

int waste_hip_moe_set_codebooks(waste_hip_moe *m, const uint16_t *f16, int n_books)
{
    return waste_hip_moe_set_codebooks_at(m, f16, 0, n_books);
}

int waste_hip_moe_set_codebooks_at(waste_hip_moe *m, const uint16_t *f16, int first, int n_books)
{
    if (!m || !f16 || n_books < m->nbk || first < 0 || first > 65535 || n_books > 65536 + m->nbk)
        return WASTE_HIP_EINVAL;
    if (m->cb >= 0 && (m->cb < first || m->cb + m->nbk > first + n_books)) return WASTE_HIP_ERECORD;
    /* books of the layer's geometry: [n_books][entries][8] */
    const int en = m->entries;
    const size_t per = (size_t)en * 8;
    float *b = (float *)malloc((size_t)n_books * per * 4);
    float *bt = (float *)malloc((size_t)n_books * per * 4);
    if (!b || !bt) { free(b); free(bt); return WASTE_HIP_ENOMEM; }
    for (size_t i = 0; i < (size_t)n_books * per; i++) b[i] = f16_book(f16[i]);
    for (int k = 0; k < n_books; k++)
        for (int c = 0; c < en; c++)
            for (int d = 0; d < 8; d++)
                bt[(size_t)k * per + (size_t)d * en + c] = b[(size_t)k * per + (size_t)c * 8 + d];
    /* the fp16 copy the matrix-core path decodes from: the loader's flush of
     * subnormals to a signed zero, the rest bit for bit */
    uint16_t *h16 = (uint16_t *)malloc((size_t)n_books * per * 2);
    if (!h16) { free(b); free(bt); return WASTE_HIP_ENOMEM; }
    for (size_t i = 0; i < (size_t)n_books * per; i++)
        h16[i] = ((f16[i] >> 10) & 0x1f) ? f16[i] : (uint16_t)(f16[i] & 0x8000);
    int rc = 0;
    if (m->d_books) { hipFree(m->d_books); hipFree(m->d_booksT); m->d_books = m->d_booksT = NULL; }
    if (m->d_books16) { hipFree(m->d_books16); m->d_books16 = NULL; }
    rc |= dmalloc((void **)&m->d_books, (size_t)n_books * per * 4);
    rc |= dmalloc((void **)&m->d_booksT, (size_t)n_books * per * 4);
    rc |= dmalloc((void **)&m->d_books16, (size_t)n_books * per * 2);
    if (!rc && (hipMemcpy(m->d_books, b, (size_t)n_books * per * 4, hipMemcpyHostToDevice) != hipSuccess ||
                hipMemcpy(m->d_booksT, bt, (size_t)n_books * per * 4, hipMemcpyHostToDevice) != hipSuccess ||
                hipMemcpy(m->d_books16, h16, (size_t)n_books * per * 2, hipMemcpyHostToDevice) != hipSuccess))
        rc = WASTE_HIP_EDEVICE;
    free(b); free(bt); free(h16);
    if (rc) return rc;
    m->n_books = n_books;
    m->book0 = first;
    return 0;
}

/* record_check (src/model.c:3645-3692) plus this layer's canonical
 * offsets.  Returns 0, WASTE_HIP_ERECORD or WASTE_HIP_ECRC. */
static int check_record(const waste_hip_moe *m, int expert, const uint8_t *rec, size_t rec_bytes,
                        int verify)
{
    waste_expert_hdr h;
    if (rec_bytes < sizeof h) return WASTE_HIP_ERECORD;
    memcpy(&h, rec, sizeof h);
    if (h.magic != WASTE_MAGIC_EXPERT) return WASTE_HIP_ERECORD;
    if (h.layer != (uint16_t)m->c.layer || h.expert_id != (uint16_t)expert) return WASTE_HIP_ERECORD;
    if ((size_t)h.rec_4k_blocks * WASTE_ALIGN != rec_bytes) return WASTE_HIP_ERECORD;
    if (h.fmt != (m->p6 ? WQ_VQ4P : m->r2 ? WQ_VQ2R : WQ_VQ3R) || h.lowrank_id != 0) return WASTE_HIP_ERECORD;
    if (m->n_books && (h.codebook_id < m->book0 || (long)h.codebook_id + m->nbk > (long)m->book0 + m->n_books))
        return WASTE_HIP_ERECORD;
    if (!(h.gate_off == 48 && h.gate_off < h.up_off && h.up_off < h.down_off &&
          h.down_off < h.chan_corr_off && h.chan_corr_off <= rec_bytes))
        return WASTE_HIP_ERECORD;
    const size_t scales = 2u * (size_t)(2 * m->I + m->H);
    if (scales > rec_bytes - h.chan_corr_off) return WASTE_HIP_ERECORD;
    /* the kernels read the canonical layout */
    if (h.up_off != m->off_up || h.down_off != m->off_down || h.chan_corr_off != m->off_sc)
        return WASTE_HIP_ERECORD;
    if (m->cb >= 0 && h.codebook_id != m->cb) return WASTE_HIP_ERECORD;
    if (verify) {
        const size_t payload = (size_t)h.chan_corr_off + scales - sizeof h;
        if (waste_hip_crc32(0, rec + sizeof h, payload) != h.crc32) return WASTE_HIP_ECRC;
    }
    return 0;
}

static int set_ptr(waste_hip_moe *m, int expert, const uint8_t *dev)
{
    m->pair_rec_ok = 0;
    if (m->h_recs[expert] && !dev) m->bound--;
    if (!m->h_recs[expert] && dev) m->bound++;
    m->h_recs[expert] = dev;
    CK(hipMemcpy(m->d_recs + expert, &m->h_recs[expert], sizeof(void *), hipMemcpyHostToDevice));
    return 0;
}

int waste_hip_moe_set_expert(waste_hip_moe *m, int expert, const void *record, size_t rec_bytes)
{
    if (!m || !record || expert < 0 || expert >= m->E) return WASTE_HIP_EINVAL;
    if (rec_bytes != m->rec_bytes) return WASTE_HIP_ERECORD;
    const int rc = check_record(m, expert, (const uint8_t *)record, rec_bytes, m->c.verify_records);
    if (rc) return rc;
    if (!m->slab && dmalloc((void **)&m->slab, (size_t)m->E * m->rec_bytes)) return WASTE_HIP_ENOMEM;
    uint8_t *dst = m->slab + (size_t)expert * m->rec_bytes;
    CK(hipMemcpy(dst, record, rec_bytes, hipMemcpyHostToDevice));
    uint16_t cbid;
    memcpy(&cbid, (const uint8_t *)record + 10, 2);
    m->cb = cbid;
    return set_ptr(m, expert, dst);
}

int waste_hip_moe_bind_expert(waste_hip_moe *m, int expert, const void *dev_record, size_t rec_bytes)
{
    if (!m || expert < 0 || expert >= m->E) return WASTE_HIP_EINVAL;
    if (!dev_record) return set_ptr(m, expert, NULL);
    if ((uintptr_t)dev_record % 16) return WASTE_HIP_EINVAL;   /* the kernels' 12-byte loads */
    if (rec_bytes != m->rec_bytes) return WASTE_HIP_ERECORD;
    uint8_t hdr[48];
    CK(hipMemcpy(hdr, dev_record, 48, hipMemcpyDeviceToHost));
    /* header only: the payload checksum needs the bytes on the host */
    const int rc = check_record(m, expert, hdr, rec_bytes, 0);
    if (rc) return rc;
    uint16_t cbid;
    memcpy(&cbid, hdr + 10, 2);
    m->cb = cbid;
    return set_ptr(m, expert, (const uint8_t *)dev_record);
}

static int prof_end(waste_hip_moe *m)
{
    if (!m->prof_on) return 0;
    CK(hipEventSynchronize(m->ev[WASTE_HIP_STAGES]));
    for (int i = 0; i < WASTE_HIP_STAGES; i++) {
        /* a stage's kernel, timed by its own dispatch; else the events
         * around the stage (which also hold the launch gaps) */
        float ms = 0;
        if (m->ktimed) {
            if (m->ktimed >> i & 1) CK(hipEventElapsedTime(&ms, m->kev[2 * i], m->kev[2 * i + 1]));
        } else {
            CK(hipEventElapsedTime(&ms, m->ev[i], m->ev[i + 1]));
        }
        m->prof.ms[i] += ms;
    }
    m->ktimed = 0;
    m->prof.forwards++;
    return 0;
}

#define MARK(i) do { if (m->prof_on) CK(hipEventRecord(m->ev[i], s)); } while (0)
/* the next launch of stage i times itself */
#define KT(i) do { if (m->prof_on) { whip_time_next(m->kev[2 * (i)], m->kev[2 * (i) + 1]); m->ktimed |= 1u << (i); } } while (0)

/* T > Td: moe_chunk (src/model.c:7110-7285) as grouped products on the
 * matrix cores.  Stages as forward(): 0 router (+ shared gate/up), 1
 * routing and the pair sort, 2 routed gate/up with SwiGLU, 3 (empty),
 * 4 routed down, 5 shared down, 6 combine. */
static int route_many(waste_hip_moe *m, const void *x, int x_bf16, int T, int32_t *d_ids,
                      float *d_w, float *lg, hipStream_t s)
{
    const int E = m->E, K = m->K, H = m->H;
    if ((uintptr_t)x % 16) return WASTE_HIP_EINVAL;
    MARK(0);
    CK((hipError_t)whip_pf_router(&m->router, x, x_bf16, T, m->rpart, lg, s));
    /* the products' A operand, converted once (experts() reads it too) */
    CK((hipError_t)whip_pf_to_f16(x, x_bf16, (size_t)T * H, m->x16, m->err, s));
    if (m->has_shared) {
        whip_pf_args a;
        memset(&a, 0, sizeof a);
        a.W0 = (const uint8_t *)m->sh[0].q; a.W1 = (const uint8_t *)m->sh[1].q;
        a.S0 = m->sh[0].qs; a.S1 = m->sh[1].qs; a.rowbytes = m->sh[0].rowbytes; a.group = m->sh[0].group;
        a.N = m->SI; a.Kd = H; a.x = m->x16; a.x_mode = 2; a.x_ld = H;
        a.rows = T; a.out = m->sh_h16; a.out_ld = m->SI; a.err = m->err;
        const int rc = whip_pf_dense(&a, m->sh[0].fmt, 1, s);
        if (rc == (int)hipErrorInvalidValue)
            CK((hipError_t)whip_pf_gemm(&a, m->sh[0].fmt, 1, 1, 1, (T + 31) / 32, s));
        else
            CK((hipError_t)rc);
    }
    MARK(1);
    whip_route_cfg rc = { E, K, m->c.score_func, m->c.renorm, m->c.routed_scale,
                          m->c.n_group, m->c.topk_group };
    CK((hipError_t)whip_route(&rc, lg, m->d_bias, T, d_ids, d_w, NULL, NULL, NULL, NULL, m->err, s));
    CK((hipError_t)whip_sort_pairs(d_ids, d_w, T, K, E, m->b.pair_tok, m->b.pair_exp, m->b.pair_w,
                                   m->b.tok_pairs, m->pair_pos, m->seg_off, m->order, s));
    return 0;
}

static int experts_many(waste_hip_moe *m, const void *x, int x_bf16, int T, float *y, hipStream_t s)
{
    (void)x; (void)x_bf16;       /* the products read route()'s fp16 copy of x */
    const int E = m->E, K = m->K, H = m->H, I = m->I;
    const int mb = (T + 127) / 128;
    MARK(2);
    whip_pf_args a;
    memset(&a, 0, sizeof a);
    a.recs = m->d_recs; a.idx_off[0] = m->off_gate; a.idx_off[1] = m->off_up;
    a.sc_off[0] = m->off_sc; a.sc_off[1] = m->off_sc + 2u * (uint32_t)I;
    a.books16 = m->d_books16; a.cb = m->cb - m->book0;
    a.N = I; a.Kd = H; a.x = m->x16; a.x_mode = 2; a.x_ld = H; a.tok = m->b.pair_tok;   /* route()'s fp16 copy */
    a.seg_off = m->seg_off; a.order = m->order; a.out = m->h16; a.out_ld = I; a.err = m->err;
    CK((hipError_t)whip_pf_gemm(&a, WQ_VQ3R, 1, 4, E, mb, s));
    MARK(3);
    MARK(4);
    a.idx_off[0] = m->off_down; a.idx_off[1] = 0;
    a.sc_off[0] = m->off_sc + 4u * (uint32_t)I; a.sc_off[1] = 0; a.cb = m->cb - m->book0 + 6;
    a.N = H; a.Kd = I; a.x = m->h16; a.x_mode = 2; a.x_ld = I; a.tok = NULL;
    a.out = m->ypair; a.out_ld = H;
    CK((hipError_t)whip_pf_gemm(&a, WQ_VQ3R, 0, 4, E, mb, s));
    MARK(5);
    if (m->has_shared) {
        memset(&a, 0, sizeof a);
        a.W0 = (const uint8_t *)m->sh[2].q; a.S0 = m->sh[2].qs; a.rowbytes = m->sh[2].rowbytes;
        a.group = m->sh[2].group; a.N = H; a.Kd = m->SI; a.x = m->sh_h16; a.x_mode = 2;
        a.x_ld = m->SI; a.rows = T; a.out = m->b.sh_out; a.out_ld = H; a.err = m->err;
        const int rc = whip_pf_dense(&a, m->sh[2].fmt, 0, s);
        if (rc == (int)hipErrorInvalidValue)
            CK((hipError_t)whip_pf_gemm(&a, m->sh[2].fmt, 0, 1, 1, (T + 31) / 32, s));
        else
            CK((hipError_t)rc);
    }
    MARK(6);
    CK((hipError_t)whip_pf_combine(m->b.tok_pairs, m->b.pair_exp, m->b.pair_w, m->d_recs, T, K, E, m->ypair, H,
                                   m->has_shared ? m->b.sh_out : NULL, y, s));
    MARK(7);
    return prof_end(m);
}

/* T <= Td: moe_layer (T = 1, src/model.c:5488-5939) and moe_chunk's order
 * for small chunks, on the decode kernels. */
static int route_few(waste_hip_moe *m, const void *x, int x_bf16, int T, int32_t *d_ids, float *d_w,
                     float *lg, hipStream_t s)
{
    const int E = m->E, K = m->K, H = m->H;
    MARK(0);
    /* router logits and the shared expert's silu(gate.x)*(up.x): one launch
     * (the shared expert on a second stream measured slower: its kernels
     * then compete with the routed path for the same CUs and bandwidth) */
    whip_gemv_job r[2];
    int nr = 0;
    r[nr].A = m->router; r[nr].B = NULL; r[nr].x = x; r[nr].x_ld = H; r[nr].x_bf16 = x_bf16;
    r[nr].y = lg; r[nr].y_ld = E; nr++;
    if (m->has_shared) {
        r[nr].A = m->sh[0]; r[nr].B = &m->sh[1]; r[nr].x = x; r[nr].x_ld = H; r[nr].x_bf16 = x_bf16;
        r[nr].y = m->b.h_sh; r[nr].y_ld = m->SI; nr++;
    }
    whip_route_cfg rc = { E, K, m->c.score_func, m->c.renorm, m->c.routed_scale,
                          m->c.n_group, m->c.topk_group };
    m->sh_done = 0;
    m->sh_in_combine = 0;
    m->pair_rec_ok = 0;
    if (T == 1) {
        /* one launch: the last router block routes the token (with the pair
         * list and the pairs' records) while the shared gate/up rows still
         * stream; the shared down projection then runs in the combine */
        KT(0);
        const int rr = whip_gemv_route(r, nr, &rc, m->d_bias, d_ids, d_w, m->b.pair_tok, m->b.pair_exp, m->b.pair_w,
                                       m->b.tok_pairs, m->d_recs, m->b.pair_rec, m->err, m->b.rcnt, m->b.xchg, s);
        if (rr) { whip_time_next(NULL, NULL); m->ktimed = 0; }
        if (rr == 0) {
            MARK(1);
            m->pair_rec_ok = 1;
            m->sh_in_combine = m->has_shared;
            return 0;
        }
        if (rr != (int)hipErrorInvalidValue) return WASTE_HIP_EDEVICE;
    }
    int routed = 0;
    if (T > 1 && m->b.sk_part && (uintptr_t)x % 16 == 0 && H % 8 == 0) {
        /* a few tokens: the router and the shared gate/up on the matrix
         * cores, column-sliced, then the slices' sums (and the SwiGLU) with
         * the routing in the same launch where its shape allows */
        float *pr = m->b.sk_part, *pg = NULL, *pu = NULL;
        whip_sk_job j[3];
        int nj = 0;
        j[nj].A = m->router; j[nj].x = x; j[nj].x_ld = H; j[nj].x_bf16 = x_bf16; j[nj].part = pr;
        j[nj].nsl = m->sk_r; nj++;
        if (m->has_shared) {
            pg = pr + (size_t)m->sk_r * T * E;
            pu = pg + (size_t)m->sk_g * T * m->SI;
            for (int q = 0; q < 2; q++) {
                j[nj].A = m->sh[q]; j[nj].x = x; j[nj].x_ld = H; j[nj].x_bf16 = x_bf16;
                j[nj].part = q ? pu : pg; j[nj].nsl = m->sk_g; nj++;
            }
        }
        CK((hipError_t)whip_sk_run(j, nj, T, s));
        const int rr = whip_sk_route(&rc, pr, m->sk_r, lg, m->d_bias, T, d_ids, d_w, m->err, pg, pu, m->sk_g,
                                     m->SI, m->b.h_sh, s);
        if (rr == 0) routed = 1;
        else if (rr != (int)hipErrorInvalidValue) return WASTE_HIP_EDEVICE;
        else CK((hipError_t)whip_sk_finish(pr, m->sk_r, E, lg, pg, pu, m->sk_g, m->SI, m->b.h_sh, T, s));
    } else {
        CK((hipError_t)whip_gemv_multi(r, nr, T, s));
    }
    MARK(1);
    if (T == 1 && m->has_shared) {
        /* routing and the shared expert's down projection in one launch;
         * the route also writes the pairs' records */
        whip_gemv_job j;
        j.A = m->sh[2]; j.B = NULL; j.x = m->b.h_sh; j.x_ld = m->SI; j.x_bf16 = 0; j.y = m->b.sh_out;
        j.y_ld = H;
        CK((hipError_t)whip_route_gemv(&rc, lg, m->d_bias, d_ids, d_w, m->b.pair_tok, m->b.pair_exp, m->b.pair_w,
                                       m->b.tok_pairs, m->d_recs, m->b.pair_rec, m->err, &j, s));
        m->sh_done = 1;
        m->pair_rec_ok = 1;
        return 0;
    }
    if (!routed)
        CK((hipError_t)whip_route(&rc, lg, m->d_bias, T, d_ids, d_w, m->b.pair_tok, m->b.pair_exp,
                                  m->b.pair_w, m->b.tok_pairs, m->err, s));
    if (T > 1)
        CK((hipError_t)whip_pairs(d_ids, d_w, T, K, E, m->b.pair_tok, m->b.pair_exp, m->b.pair_w,
                                  m->b.tok_pairs, s));
    return 0;
}

static int experts_few(waste_hip_moe *m, const void *x, int x_bf16, int T, float *y, hipStream_t s)
{
    const int K = m->K, H = m->H, I = m->I, P = T * K;
    MARK(2);
    whip_vq_args a;
    memset(&a, 0, sizeof a);
    a.recs = m->d_recs; a.pair_exp = m->b.pair_exp; a.pair_src = m->b.pair_tok;
    a.pair_rec = (T == 1 && m->pair_rec_ok) ? m->b.pair_rec : NULL;
    a.src = x; a.src_ld = H; a.src_bf16 = x_bf16; a.booksT = m->d_booksT; a.cb = m->cb - m->book0;
    a.idx_off[0] = m->off_gate; a.idx_off[1] = m->off_up;
    a.kinds = 2; a.M = I; a.nv = m->nv_gu; a.P = P; a.rsplit = m->rsplit_gu;
    a.part = m->b.part_gu; a.err = m->err;
    /* the down kernel reduces the gate/up partials and applies SwiGLU in its
     * table build when both passes run positions across lanes (the gate/up
     * partials then leave scaled by their rows' scales); else a separate
     * pass */
    const int act_fused = m->nv_d % 32 == 0 && m->nv_gu % 32 == 0;
    a.out_sc_off = act_fused ? m->off_sc : 0;
    if (T == 1 && P <= 64) {
        /* one token: every pair's gate/up table is the same */
        a.span = P;
        a.rsplit = pick_span_split(m->nch_gu * 2, P * (I / 64));
    }
    /* one token whose shared down projection is still to run: the gate/up
     * launch's spare workgroups take it (it needs only h_sh) */
    int sh_in_gu = 0;
    if (m->sh_in_combine && a.span) {
        a.shd = m->sh[2]; a.shd_x = m->b.h_sh; a.shd_y = m->b.sh_out;
        sh_in_gu = 1;
    }
    if (m->sh_in_combine || m->ktimed) KT(2);
    int arc = whip_vq_apply(&a, s);
    if (arc == (int)hipErrorInvalidValue && sh_in_gu) {   /* a shape it does not take: the combine runs it */
        a.shd_x = NULL; a.shd_y = NULL;
        sh_in_gu = 0;
        arc = whip_vq_apply(&a, s);
    }
    CK((hipError_t)arc);
    a.shd_x = NULL; a.shd_y = NULL;
    MARK(3);
    a.out_sc_off = 0;
    if (!act_fused)
        CK((hipError_t)whip_vq_act(m->d_recs, m->b.pair_exp, P, m->b.part_gu, m->nch_gu, I, m->off_sc,
                                   m->b.h, s));
    MARK(4);
    a.pair_src = NULL; a.src = m->b.h; a.src_ld = I; a.src_bf16 = 0; a.cb = m->cb - m->book0 + 6;
    if (act_fused) {
        a.act_part = m->b.part_gu; a.act_nch = m->nch_gu;
        a.out_sc_off = m->off_sc + 4u * (uint32_t)I;  /* the down partials leave scaled too */
    }
    const uint32_t cmb_sc = act_fused ? 0u : m->off_sc + 4u * (uint32_t)I;
    a.idx_off[0] = m->off_down; a.idx_off[1] = 0;
    a.kinds = 1; a.M = H; a.nv = m->nv_d; a.rsplit = m->rsplit_d; a.part = m->b.part_d;
    a.span = 0;
    if (m->ktimed && act_fused) KT(4);
    CK((hipError_t)whip_vq_apply(&a, s));
    MARK(5);
    if (m->sh_in_combine && !sh_in_gu) {
        /* the shared down projection inside the combine's blocks */
        MARK(6);
        KT(6);
        const int rc = whip_combine_sh(m->d_recs, m->b.pair_exp, m->b.pair_w, m->b.tok_pairs, T, K, m->b.part_d,
                                       m->nch_d, H, cmb_sc, T > 1, &m->sh[2], m->b.h_sh, y, s);
        if (rc == 0) {
            MARK(7);
            return prof_end(m);
        }
        if (rc != (int)hipErrorInvalidValue) return WASTE_HIP_EDEVICE;
        whip_time_next(NULL, NULL);
        m->ktimed = 0;
        CK((hipError_t)whip_gemv(&m->sh[2], NULL, m->b.h_sh, m->SI, T, m->b.sh_out, NULL, H, s));
    }
    const float *shp = m->has_shared ? m->b.sh_out : NULL;
    int sh_n = 1;
    if (m->has_shared && !m->sh_done && !sh_in_gu && !m->sh_in_combine) {
        if (T > 1 && m->b.sk_part) {
            /* column slices on the matrix cores; the combine adds them */
            whip_sk_job j;
            j.A = m->sh[2]; j.x = m->b.h_sh; j.x_ld = m->SI; j.x_bf16 = 0; j.part = m->b.sk_part;
            j.nsl = m->sk_d;
            CK((hipError_t)whip_sk_run(&j, 1, T, s));
            shp = m->b.sk_part;
            sh_n = m->sk_d;
        } else {
            CK((hipError_t)whip_gemv(&m->sh[2], NULL, m->b.h_sh, m->SI, T, m->b.sh_out, NULL, H, s));
        }
    }
    MARK(6);
    if (m->ktimed) KT(6);
    CK((hipError_t)whip_combine(m->d_recs, m->b.pair_exp, m->b.pair_w, m->b.tok_pairs, T, K, m->b.part_d,
                                m->nch_d, H, cmb_sc, T > 1, shp, sh_n, (size_t)T * H, y, s));
    MARK(7);
    return prof_end(m);
}

/* VQ4P experts (index_bits 6), moe_layer's order at T = 1 and moe_chunk's
 * above (src/model.c:5876-5910, 7203-7251), on the routing and pair lists
 * route() left: each token's gate and up tables (fp32 by vq_build_lut, then
 * int8 with one scale per 32 positions), every pair's gate and up rows
 * through them (vq_rows_p6: exact integer sums per scale block, folded into
 * fp32 in block order), SwiGLU, the pair's down table from its SwiGLU
 * output and its down rows, then the combine and the shared expert as for
 * VQ3R.  Two launches and the combine: each tile launch builds the tables
 * it reads, the block sums wait in HBM for the launch that folds them (the
 * down launch, the combine).  The tables and folds follow the engine's
 * arithmetic in the layer's p6_order, so each pair's rows are the engine's
 * bit for bit. */
static int alt_combine(waste_hip_moe *m, int T, float *y, const whip_fold *f, int sh_ready, hipStream_t s);

static int experts_p6(waste_hip_moe *m, const void *x, int x_bf16, int T, float *y, hipStream_t s)
{
    const int K = m->K, H = m->H, I = m->I, P = T * K, fma = m->c.p6_order == WASTE_HIP_ORDER_FMA;
    const int cb = m->cb - m->book0, cb_d = cb + 2 * m->stages, nb_d = (m->nv_d + 31) / 32;
    const uint32_t gu_idx[2] = { m->off_gate, m->off_up };
    const uint32_t sc_g = m->off_sc, sc_u = m->off_sc + 2u * (uint32_t)I, sc_d = m->off_sc + 4u * (uint32_t)I;
    /* one token: the tile launches build their tables (two launches fewer);
     * more: the tables once per token and pair, the tiles read them */
    const int8_t *q_gu = T > 1 ? m->p6b.q_gu : NULL, *q_d = T > 1 ? m->p6b.q_d : NULL;
    m->ktimed = 0;               /* these stages are timed by the events around them */
    MARK(2);
    if (q_gu)
        CK((hipError_t)whip_p6_lutq(x, x_bf16, H, T, 2, m->d_booksT, cb, m->nv_gu, fma, m->p6b.q_gu, m->p6b.s_gu,
                                    s));
    if (P > P6_PAIR_CHUNK) {
        /* many pairs: chunks of P6_PAIR_CHUNK pairs, each pair's down rows
         * folded into p6b.down, which the combine reads */
        for (int c0 = 0; c0 < P; c0 += P6_PAIR_CHUNK) {
            const int n = P - c0 < P6_PAIR_CHUNK ? P - c0 : P6_PAIR_CHUNK;
            const int32_t *pe = m->b.pair_exp + c0, *pt = m->b.pair_tok + c0;
            CK((hipError_t)whip_p6_gate_up(m->d_recs, pe, pt, n, gu_idx, I, x, x_bf16, H, m->nv_gu, m->d_booksT, cb,
                                           fma, q_gu, m->p6b.S_gu, m->p6b.s_gu, m->err, NULL, NULL, NULL, s));
            CK((hipError_t)whip_p6_act_lutq(m->d_recs, pe, pt, n, m->p6b.S_gu, m->p6b.s_gu, sc_g, sc_u, I, m->nv_gu,
                                            m->d_booksT, cb_d, m->nv_d, fma, m->p6b.q_d, m->p6b.s_d, s));
            CK((hipError_t)whip_p6_down(m->d_recs, pe, pt, n, m->off_down, H, I, m->p6b.S_gu, m->p6b.s_gu, sc_g,
                                        sc_u, m->nv_gu, m->d_booksT, cb_d, fma, m->p6b.q_d, m->p6b.S_d, m->p6b.s_d,
                                        m->err, s));
            CK((hipError_t)whip_p6_fold_pairs(m->d_recs, pe, n, m->p6b.S_d, m->p6b.s_d, nb_d, H, sc_d, fma,
                                              m->p6b.down + (size_t)c0 * H, s));
        }
        MARK(3);
        MARK(4);
        MARK(5);
        return alt_combine(m, T, y, NULL, 0, s);
    }
    /* one token whose shared down projection is still to run: the gate/up
     * launch's spare workgroups take it (it needs only h_sh) */
    int sh_ready = 0;
    int grc = -1;
    if (!q_gu && m->sh_in_combine) {
        grc = whip_p6_gate_up(m->d_recs, m->b.pair_exp, m->b.pair_tok, P, gu_idx, I, x, x_bf16, H, m->nv_gu,
                              m->d_booksT, cb, fma, q_gu, m->p6b.S_gu, m->p6b.s_gu, m->err, &m->sh[2], m->b.h_sh,
                              m->b.sh_out, s);
        sh_ready = grc == 0;
        if (grc != 0 && grc != (int)hipErrorInvalidValue) return WASTE_HIP_EDEVICE;
    }
    if (!sh_ready)
        CK((hipError_t)whip_p6_gate_up(m->d_recs, m->b.pair_exp, m->b.pair_tok, P, gu_idx, I, x, x_bf16, H,
                                       m->nv_gu, m->d_booksT, cb, fma, q_gu, m->p6b.S_gu, m->p6b.s_gu, m->err, NULL,
                                       NULL, NULL, s));
    MARK(3);
    if (q_d)
        CK((hipError_t)whip_p6_act_lutq(m->d_recs, m->b.pair_exp, m->b.pair_tok, P, m->p6b.S_gu, m->p6b.s_gu, sc_g,
                                        sc_u, I, m->nv_gu, m->d_booksT, cb_d, m->nv_d, fma, m->p6b.q_d, m->p6b.s_d,
                                        s));
    MARK(4);
    CK((hipError_t)whip_p6_down(m->d_recs, m->b.pair_exp, m->b.pair_tok, P, m->off_down, H, I, m->p6b.S_gu,
                                m->p6b.s_gu, sc_g, sc_u, m->nv_gu, m->d_booksT, cb_d, fma, q_d, m->p6b.S_d,
                                m->p6b.s_d, m->err, s));
    MARK(5);
    const whip_fold f = { m->p6b.S_d, m->p6b.s_d, nb_d, sc_d, fma };
    return alt_combine(m, T, y, &f, sh_ready, s);
}

/* VQ2R experts (two stages of 256 entries), the same order as VQ4P's above
 * with fp32 tables: each token's gate and up tables (vq_build_lut), every
 * pair's gate and up rows through them (vq_rows' generic loop), SwiGLU,
 * the pair's down table and rows, the combine.  The tables follow the
 * engine's build in the layer's order, so each pair's rows are the
 * engine's bit for bit. */
static int experts_r2(waste_hip_moe *m, const void *x, int x_bf16, int T, float *y, hipStream_t s)
{
    const int K = m->K, H = m->H, I = m->I, P = T * K, fma = m->c.p6_order == WASTE_HIP_ORDER_FMA;
    const int cb = m->cb - m->book0;
    m->ktimed = 0;               /* these stages are timed by the events around them */
    MARK(2);
    /* one token whose shared down projection is still to run: the table
     * launch's spare workgroups take it (it needs only h_sh) */
    int sh_ready = 0;
    if (T == 1 && m->sh_in_combine) {
        const int rc = whip_r2_lutb(x, x_bf16, H, T, 2, 2, m->d_booksT, cb, m->nv_gu, fma, m->p6b.lut_gu, &m->sh[2],
                                    m->b.h_sh, m->b.sh_out, s);
        sh_ready = rc == 0;
        if (rc != 0 && rc != (int)hipErrorInvalidValue) return WASTE_HIP_EDEVICE;
    }
    if (!sh_ready)
        CK((hipError_t)whip_r2_lutb(x, x_bf16, H, T, 2, 2, m->d_booksT, cb, m->nv_gu, fma, m->p6b.lut_gu, NULL, NULL,
                                    NULL, s));
    const uint32_t gu_idx[2] = { m->off_gate, m->off_up };
    const uint32_t gu_sc[2] = { m->off_sc, m->off_sc + 2u * (uint32_t)I };
    CK((hipError_t)whip_r2_rows_pairs(m->d_recs, m->b.pair_exp, m->b.pair_tok, P, 2, gu_idx, gu_sc, I, m->nv_gu,
                                      m->p6b.lut_gu, 1, m->p6b.gu, m->err, s));
    MARK(3);
    CK((hipError_t)whip_r2_act_lutb(m->p6b.gu, P, I, m->d_booksT, cb + 2 * m->stages, fma, m->p6b.lut_d, s));
    MARK(4);
    const uint32_t d_idx[1] = { m->off_down }, d_sc[1] = { m->off_sc + 4u * (uint32_t)I };
    CK((hipError_t)whip_r2_rows_pairs(m->d_recs, m->b.pair_exp, m->b.pair_tok, P, 1, d_idx, d_sc, H, m->nv_d,
                                      m->p6b.lut_d, 0, m->p6b.down, m->err, s));
    MARK(5);
    return alt_combine(m, T, y, NULL, sh_ready, s);
}

/* The combine of the VQ4P / VQ2R paths: each pair's down rows folded from
 * f (VQ4P) or in p6b.down, already scaled, one chunk each (VQ2R); the
 * shared expert as for VQ3R (sh_ready: its down projection already in
 * sh_out). */
static int alt_combine(waste_hip_moe *m, int T, float *y, const whip_fold *f, int sh_ready, hipStream_t s)
{
    const int K = m->K, H = m->H;
    if (m->sh_in_combine && !sh_ready) {
        MARK(6);
        const int rc = f ? whip_combine_sh_fold(m->d_recs, m->b.pair_exp, m->b.pair_w, m->b.tok_pairs, T, K, f, H,
                                                T > 1, &m->sh[2], m->b.h_sh, y, s)
                         : whip_combine_sh(m->d_recs, m->b.pair_exp, m->b.pair_w, m->b.tok_pairs, T, K,
                                           m->p6b.down, 1, H, 0, T > 1, &m->sh[2], m->b.h_sh, y, s);
        if (rc == 0) {
            MARK(7);
            return prof_end(m);
        }
        if (rc != (int)hipErrorInvalidValue) return WASTE_HIP_EDEVICE;
        CK((hipError_t)whip_gemv(&m->sh[2], NULL, m->b.h_sh, m->SI, T, m->b.sh_out, NULL, H, s));
    }
    const float *shp = m->has_shared ? m->b.sh_out : NULL;
    int sh_n = 1;
    if (m->has_shared && !m->sh_done && !m->sh_in_combine && !sh_ready) {
        if (T > 1 && m->b.sk_part) {
            whip_sk_job j;
            j.A = m->sh[2]; j.x = m->b.h_sh; j.x_ld = m->SI; j.x_bf16 = 0; j.part = m->b.sk_part;
            j.nsl = m->sk_d;
            CK((hipError_t)whip_sk_run(&j, 1, T, s));
            shp = m->b.sk_part;
            sh_n = m->sk_d;
        } else {
            CK((hipError_t)whip_gemv(&m->sh[2], NULL, m->b.h_sh, m->SI, T, m->b.sh_out, NULL, H, s));
        }
    }
    MARK(6);
    if (f)
        CK((hipError_t)whip_combine_fold(m->d_recs, m->b.pair_exp, m->b.pair_w, m->b.tok_pairs, T, K, f, H, T > 1,
                                         shp, sh_n, (size_t)T * H, y, s));
    else
        CK((hipError_t)whip_combine(m->d_recs, m->b.pair_exp, m->b.pair_w, m->b.tok_pairs, T, K, m->p6b.down, 1,
                                    H, 0, T > 1, shp, sh_n, (size_t)T * H, y, s));
    MARK(7);
    return prof_end(m);
}
#undef MARK

static int ready(const waste_hip_moe *m, const void *x, int T)
{
    if (!m || !x || T <= 0 || T > m->T) return WASTE_HIP_EINVAL;
    if (!m->has_router || !m->d_booksT || m->n_books < m->nbk) return WASTE_HIP_EINVAL;
    return 0;
}

int waste_hip_moe_route(waste_hip_moe *m, const void *x, int x_bf16, int T, int32_t *ids, float *w,
                        float *logits, void *stream)
{
    const int rc = ready(m, x, T);
    if (rc) return rc;
    hipStream_t s = (hipStream_t)stream;
    int32_t *d_ids = ids ? ids : m->b.ids;
    float *d_w = w ? w : m->b.w;
    float *lg = logits ? logits : m->b.logits;
    m->routed_T = 0;
    const int r = T > m->Td ? route_many(m, x, x_bf16, T, d_ids, d_w, lg, s)
                            : route_few(m, x, x_bf16, T, d_ids, d_w, lg, s);
    if (r) return r;
    m->routed_T = T;
    m->r_ids = d_ids;
    m->r_w = d_w;
    return 0;
}

/* A chunk whose fp16 operands left fp16's range (an activation or a SwiGLU
 * output beyond 65504: the matrix-core kernels raise bit 4 and their
 * outputs are not to be used) runs again on the fp32 decode kernels, Td
 * tokens at a time, with the routing it already has: the shared expert's
 * gate/up (fp32), the sub-chunk's pair lists, then the experts, their
 * combine and the shared down projection.  The host reads the error word
 * after the chunk for this; a stream being captured into a graph cannot
 * wait, so there the bit stays raised for waste_hip_moe_status. */
static int range_fallback(waste_hip_moe *m, const void *x, int x_bf16, int T, float *y, hipStream_t s)
{
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return 0;
    if (!m->h_err && hipHostMalloc((void **)&m->h_err, sizeof(int), hipHostMallocDefault) != hipSuccess) {
        m->h_err = NULL;
        return WASTE_HIP_ENOMEM;
    }
    CK(hipMemcpyAsync(m->h_err, m->err, sizeof(int), hipMemcpyDeviceToHost, s));
    CK(hipStreamSynchronize(s));
    if (!(*m->h_err & 4)) return 0;
    CK((hipError_t)whip_err_clear(m->err, 4, s));
    const int K = m->K, H = m->H, Td = m->Td, prof = m->prof_on;
    const size_t esz = x_bf16 ? 2 : 4;
    m->prof_on = 0;
    int rc = 0;
    for (int t0 = 0; t0 < T && !rc; t0 += Td) {
        const int n = T - t0 < Td ? T - t0 : Td;
        const void *xs = (const uint8_t *)x + (size_t)t0 * H * esz;
        if (m->has_shared) {
            whip_gemv_job j;
            j.A = m->sh[0]; j.B = &m->sh[1]; j.x = xs; j.x_ld = H; j.x_bf16 = x_bf16;
            j.y = m->b.h_sh; j.y_ld = m->SI;
            if (whip_gemv_multi(&j, 1, n, s)) { rc = WASTE_HIP_EDEVICE; break; }
        }
        if (whip_pairs(m->r_ids + (size_t)t0 * K, m->r_w + (size_t)t0 * K, n, K, m->E, m->b.pair_tok,
                       m->b.pair_exp, m->b.pair_w, m->b.tok_pairs, s)) {
            rc = WASTE_HIP_EDEVICE;
            break;
        }
        m->sh_done = 0;
        m->sh_in_combine = 0;
        m->pair_rec_ok = 0;
        rc = experts_few(m, xs, x_bf16, n, y + (size_t)t0 * H, s);
    }
    m->prof_on = prof;
    return rc;
}

int waste_hip_moe_experts(waste_hip_moe *m, const void *x, int x_bf16, int T, float *y, void *stream)
{
    const int rc = ready(m, x, T);
    if (rc) return rc;
    if (!y || T != m->routed_T) return WASTE_HIP_EINVAL;
    if (!books_ok(m)) return WASTE_HIP_EINVAL;
    hipStream_t s = (hipStream_t)stream;
    if (m->p6) return experts_p6(m, x, x_bf16, T, y, s);
    if (m->r2) return experts_r2(m, x, x_bf16, T, y, s);
    if (T <= m->Td) return experts_few(m, x, x_bf16, T, y, s);
    const int r = experts_many(m, x, x_bf16, T, y, s);
    return r ? r : range_fallback(m, x, x_bf16, T, y, s);
}

int waste_hip_moe_forward(waste_hip_moe *m, const void *x, int x_bf16, int T, float *y,
                          int32_t *ids, float *w, float *logits, void *stream)
{
    int rc = ready(m, x, T);
    if (rc) return rc;
    if (!y || !books_ok(m)) return WASTE_HIP_EINVAL;
    rc = waste_hip_moe_route(m, x, x_bf16, T, ids, w, logits, stream);
    return rc ? rc : waste_hip_moe_experts(m, x, x_bf16, T, y, stream);
}

/* Bytes of the static area one allocation-free forward of T tokens uses
 * beyond its head, with the regions' offsets when b is set. */
static size_t static_layout(const waste_hip_moe *m, int T, uint8_t *base, fwd_bufs *b)
{
    const size_t P = (size_t)T * m->K;
    const int act_fused = m->nv_d % 32 == 0 && m->nv_gu % 32 == 0;
    size_t off = WHIP_SCRATCH_HEAD;
#define TAKE(field, type, bytes)                                               \
    do {                                                                       \
        if (b) b->field = (type)(base + off);                                  \
        off += ((size_t)(bytes) + 255) / 256 * 256;                            \
    } while (0)
    TAKE(logits, float *, (size_t)T * m->E * 4);
    TAKE(ids, int32_t *, P * 4);
    TAKE(w, float *, P * 4);
    TAKE(pair_tok, int32_t *, P * 4);
    TAKE(pair_exp, int32_t *, P * 4);
    TAKE(pair_w, float *, P * 4);
    TAKE(tok_pairs, int32_t *, P * 4);
    TAKE(pair_rec, const uint8_t **, 64 * sizeof(void *));
    TAKE(part_gu, float *, (P * 2 * m->nch_gu * m->I + 64) * 4);
    TAKE(part_d, float *, (P * m->nch_d * m->H + 64) * 4);
    if (!act_fused) TAKE(h, float *, P * m->I * 4);
    else if (b) b->h = NULL;
    if (m->has_shared) {
        TAKE(h_sh, float *, (size_t)T * m->SI * 4);
        TAKE(sh_out, float *, (size_t)T * m->H * 4);
    } else if (b) {
        b->h_sh = b->sh_out = NULL;
    }
    /* the few-token products' slice partials, as forward() has them */
    if (T > 1 && m->sk_r && m->sk_mem) {
        const size_t a = (size_t)m->sk_r * m->E + 2 * (size_t)m->sk_g * m->SI;
        const size_t d = (size_t)m->sk_d * m->H;
        TAKE(sk_part, float *, (size_t)T * (a > d ? a : d) * 4);
    } else if (b) {
        b->sk_part = NULL;
    }
#undef TAKE
    if (b) {
        b->xchg = (uint64_t *)(base + WHIP_SCRATCH_XCHG);
        b->rcnt = (int *)(base + WHIP_SCRATCH_RCNT);
    }
    return off;
}

size_t waste_hip_moe_static_bytes(const waste_hip_moe *m, int T)
{
    if (!m || T <= 0) return 0;
    return static_layout(m, T, NULL, NULL);
}

int waste_hip_moe_forward_static(waste_hip_moe *m, const void *x, int x_bf16, int T, float *y,
                                 int32_t *ids, float *w, float *logits, void *stream)
{
    int rc = ready(m, x, T);
    if (rc) return rc;
    if (!y || !books_ok(m) || m->p6 || m->r2) return WASTE_HIP_EINVAL;   /* VQ4P / VQ2R: forward() only */
    if (T > m->Td || static_layout(m, T, NULL, NULL) > WHIP_SCRATCH_BYTES)
        return WASTE_HIP_ESCRATCH;
    hipStream_t s = (hipStream_t)stream;
    void *base = NULL;
    if (whip_scratch(&base)) return WASTE_HIP_EDEVICE;
    fwd_bufs sb;
    static_layout(m, T, (uint8_t *)base, &sb);
    /* the staged kernels on the static buffers; the layer's own come back
     * afterwards, and nothing of this call's routing is left for experts() */
    const fwd_bufs own = m->b;
    m->b = sb;
    m->routed_T = 0;
    rc = waste_hip_moe_route(m, x, x_bf16, T, ids, w, logits, stream);
    if (!rc) rc = waste_hip_moe_experts(m, x, x_bf16, T, y, stream);
    m->b = own;
    m->routed_T = 0;
    m->pair_rec_ok = 0;
    return rc;
}

int waste_hip_moe_bind_table(waste_hip_moe *m, const int *experts, const void *const *dev_records, int n,
                             int codebook_id, void *stream)
{
    if (!m || n < 0 || n > WHIP_BIND_MAX || (n && (!experts || !dev_records))) return WASTE_HIP_EINVAL;
    if (codebook_id < -1 || codebook_id > 65535) return WASTE_HIP_EINVAL;
    whip_bind_args a;
    memset(&a, 0, sizeof a);
    for (int i = 0; i < n; i++) {
        const int e = experts[i];
        if (e < 0 || e >= m->E || (uintptr_t)dev_records[i] % 16) return WASTE_HIP_EINVAL;
        for (int j = 0; j < i; j++)
            if (experts[j] == e) return WASTE_HIP_EINVAL;
        a.expert[i] = e;
        a.rec[i] = (const uint8_t *)dev_records[i];
    }
    if (codebook_id >= 0) {
        if (m->cb >= 0 && m->cb != codebook_id) return WASTE_HIP_ERECORD;
        if (m->n_books && (codebook_id < m->book0 || codebook_id + m->nbk > m->book0 + m->n_books))
            return WASTE_HIP_ERECORD;
        m->cb = codebook_id;
    }
    a.n = n;
    a.layer = (uint16_t)m->c.layer;
    a.rec_4k_blocks = (uint32_t)(m->rec_bytes / 4096);
    a.off_up = m->off_up; a.off_down = m->off_down; a.off_sc = m->off_sc;
    a.cb = m->cb;
    a.book0 = m->n_books > 0 ? m->book0 : 0;
    a.n_books = m->n_books > 0 ? m->book0 + m->n_books : 65536 + m->nbk;
    a.fmt = m->p6 ? WQ_VQ4P : m->r2 ? WQ_VQ2R : WQ_VQ3R;
    a.nbk = (uint32_t)m->nbk;
    CK((hipError_t)whip_bind(m->d_recs, &a, m->err, (hipStream_t)stream));
    m->pair_rec_ok = 0;
    for (int i = 0; i < n; i++) {
        const int e = a.expert[i];
        if (m->h_recs[e] && !a.rec[i]) m->bound--;
        if (!m->h_recs[e] && a.rec[i]) m->bound++;
        m->h_recs[e] = a.rec[i];
    }
    return 0;
}

/* The lookahead's guesses a predict() of n on m writes: at most E, and
 * with the group limit at most the experts of the groups it keeps. */
static int look_count(const waste_hip_moe *m, int n)
{
    if (n > m->E) n = m->E;
    if (m->look_groups && m->c.n_group > 1) {
        const int kept = m->c.topk_group * (m->E / m->c.n_group);
        if (n > kept) n = kept;
    }
    return n;
}

int waste_hip_moe_set_lookahead_groups(waste_hip_moe *m, int on)
{
    if (!m || (on != 0 && on != 1)) return WASTE_HIP_EINVAL;
    m->look_groups = on;
    return 0;
}

int waste_hip_moe_predict(waste_hip_moe *m, const void *x, int x_bf16, int n, int32_t *ids, void *stream)
{
    if (!m || !x || !ids || n <= 0 || n > 64 || !m->has_router) return WASTE_HIP_EINVAL;
    n = look_count(m, n);
    hipStream_t s = (hipStream_t)stream;
    whip_gemv_job j;
    j.A = m->router; j.B = NULL; j.x = x; j.x_ld = m->H; j.x_bf16 = x_bf16; j.y = m->plogits;
    j.y_ld = m->E;
    CK((hipError_t)whip_gemv_multi(&j, 1, 1, s));
    /* selection order only, weights unused; the group limit when asked */
    const int grouped = m->look_groups && m->c.n_group > 1;
    whip_route_cfg rc = { m->E, n, m->c.score_func, 0, 1.0f, grouped ? m->c.n_group : 0,
                          grouped ? m->c.topk_group : 0 };
    CK((hipError_t)whip_route(&rc, m->plogits, m->d_bias, 1, ids, m->pw, NULL, NULL, NULL, NULL,
                              m->err + 4, s));
    return 0;
}

int waste_hip_moe_profile(waste_hip_moe *m, int on)
{
    if (!m) return WASTE_HIP_EINVAL;
    if (on && !m->ev[0]) {
        for (int i = 0; i <= WASTE_HIP_STAGES; i++) CK(hipEventCreate(&m->ev[i]));
        for (int i = 0; i < 2 * WASTE_HIP_STAGES; i++) CK(hipEventCreate(&m->kev[i]));
    }
    m->ktimed = 0;
    memset(&m->prof, 0, sizeof m->prof);
    m->prof_on = on;
    return 0;
}

int waste_hip_moe_profile_read(waste_hip_moe *m, waste_hip_moe_prof *out)
{
    if (!m || !out) return WASTE_HIP_EINVAL;
    *out = m->prof;
    return 0;
}

/* moe_layer's cache path (src/model.c:5639-5700 and 5926-5930) for one
 * token: route, the lookahead on the next layer's router, the selection
 * to the host, hint and hold, bind, experts, release, lookahead reads. */
int waste_hip_moe_forward_cached(waste_hip_moe *m, waste_hip_ecache *c, int layer, waste_hip_moe *next,
                                 int lookahead, const void *x, int x_bf16, float *y, int32_t *ids,
                                 float *w, void *stream)
{
    if (!m || !c || !x || !y || layer < 0 || layer > 32767 || lookahead < 0 || lookahead > 64)
        return WASTE_HIP_EINVAL;
    if (!books_ok(m)) return WASTE_HIP_EINVAL;
    hipStream_t s = (hipStream_t)stream;
    const int K = m->K;
    if (!m->h_sel && hipHostMalloc((void **)&m->h_sel, 128 * sizeof(int32_t), hipHostMallocDefault) != hipSuccess) {
        m->h_sel = NULL;
        return WASTE_HIP_ENOMEM;
    }
    int32_t *d_ids = ids ? ids : m->b.ids;
    float *d_w = w ? w : m->b.w;
    int rc = waste_hip_moe_route(m, x, x_bf16, 1, d_ids, d_w, NULL, stream);
    if (rc) return rc;
    const int nl = next && lookahead > 0 ? look_count(next, lookahead) : 0;
    if (nl && (rc = waste_hip_moe_predict(next, x, x_bf16, nl, m->d_look, stream))) return rc;
    CK(hipMemcpyAsync(m->h_sel, d_ids, (size_t)K * sizeof(int32_t), hipMemcpyDeviceToHost, s));
    if (nl) CK(hipMemcpyAsync(m->h_sel + 64, m->d_look, (size_t)nl * sizeof(int32_t), hipMemcpyDeviceToHost, s));
    CK(hipStreamSynchronize(s));
    int routed = 1;
    for (int j = 0; j < K; j++) routed &= m->h_sel[j] >= 0 && m->h_sel[j] < m->E;
    if (routed) {
        /* a failed route leaves -1 ids: the experts then report it */
        const void *recs[64];
        if ((rc = waste_hip_ecache_hint(c, layer, m->h_sel, K))) return rc;
        for (int j = 0; j < K; j++) {
            recs[j] = waste_hip_ecache_hold(c, layer, m->h_sel[j], stream);
            if (!recs[j]) {
                waste_hip_ecache_release(c, stream);
                return WASTE_HIP_EDEVICE;
            }
        }
        if ((rc = waste_hip_moe_bind_table(m, m->h_sel, recs, K, -1, stream))) return rc;
    }
    rc = waste_hip_moe_experts(m, x, x_bf16, 1, y, stream);
    const int rr = waste_hip_ecache_release(c, stream);
    if (rc) return rc;
    if (rr) return rr;
    /* the guess goes out after this layer's reads (src/model.c:5921-5930) */
    int guess[64], ng = 0;
    for (int j = 0; j < nl; j++)
        if (m->h_sel[64 + j] >= 0) guess[ng++] = m->h_sel[64 + j];
    return ng ? waste_hip_ecache_prefetch(c, layer + 1, guess, ng) : 0;
}

int waste_hip_moe_status(waste_hip_moe *m, void *stream)
{
    if (!m) return WASTE_HIP_EINVAL;
    int e = 0;
    CK(hipStreamSynchronize((hipStream_t)stream));
    CK(hipMemcpy(&e, m->err, sizeof e, hipMemcpyDeviceToHost));
    CK(hipMemset(m->err, 0, sizeof e));
    /* a failed route leaves ids of -1, which the expert kernels then see
     * as unbound: report the cause */
    if (e & 2) return WASTE_HIP_EROUTE;
    if (e & 8) return WASTE_HIP_ERECORD;
    if (e & 1) return WASTE_HIP_EUNBOUND;
    if (e & 4) return WASTE_HIP_ERANGE;
    if (e & 16) return WASTE_HIP_ETIMEOUT;
    return 0;
}

size_t waste_hip_moe_bytes(const waste_hip_moe *m, int T, int n_distinct)
{
    if (!m) return 0;
    size_t b = (size_t)n_distinct * (2 * m->idx_gu + m->idx_d + 2 * (size_t)(2 * m->I + m->H));
    if (m->has_router) {
        const whip_mat *r = &m->router;
        b += (size_t)r->rows * r->rowbytes;
        if (r->fmt != WQ_F32) b += (size_t)r->rows * ((r->cols + r->group - 1) / r->group) * 2;
        if (m->d_bias) b += (size_t)m->E * 4;
    }
    if (m->has_shared)
        for (int k = 0; k < 3; k++) {
            const whip_mat *t = &m->sh[k];
            b += (size_t)t->rows * t->rowbytes;
            if (t->fmt != WQ_F32) b += (size_t)t->rows * ((t->cols + t->group - 1) / t->group) * 2;
        }
    b += 9 * 256 * 8 * 2;                      /* the layer's nine codebooks */
    b += (size_t)T * m->H * 4 * 2;             /* activations in and out     */
    return b;
}

int waste_hip_moe_dequant(waste_hip_moe *m, int expert, int kind, float *W, void *stream)
{
    if (!m || expert < 0 || expert >= m->E || kind < 0 || kind > 2 || !W || !m->d_books ||
        !books_ok(m) || m->p6 || m->r2)
        return WASTE_HIP_EINVAL;
    const uint8_t *rec = m->h_recs[expert];
    if (!rec) return WASTE_HIP_EUNBOUND;
    const int M = kind == 2 ? m->H : m->I, N = kind == 2 ? m->I : m->H;
    const uint32_t off = kind == 0 ? m->off_gate : kind == 1 ? m->off_up : m->off_down;
    const uint16_t *sc = (const uint16_t *)(rec + m->off_sc) + (kind == 0 ? 0 : kind == 1 ? m->I : 2 * m->I);
    CK((hipError_t)whip_dequant(rec + off, sc, m->d_books, m->cb - m->book0 + 3 * kind, M, N, W,
                                (hipStream_t)stream));
    return 0;
}
