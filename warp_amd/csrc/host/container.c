/* SPDX-License-Identifier: Apache-2.0 */
/*
 * container.c — reads a WARP container directory on the host.
 *
 * Everything here is untrusted input checked before use: the manifest
 * (format_version 0; the MoE keys of `config` bounded as cfg_sane bounds
 * them, src/model.c:1813-1850; `expert_quant`'s ranges and index_bits
 * rule, src/model.c:2709-2741; each bank's size arithmetic and codebook
 * base, src/model.c:2962-2983; trunk offsets and shapes against the size
 * of trunk.bin, src/model.c:1286-1340), and every record as it is read
 * (record_check, src/model.c:3645-3692).  No GPU calls: a container can be
 * opened and its records read where there is no device.
 *
 * Stricter than the engine where the engine would read wrong bytes:
 * index_block must be 64 (the blocking both the engine's VQ_TILE and these
 * kernels assume; src/model.c:3890), a bank's file name may not be
 * absolute or climb out of the directory, a string that does not fit its
 * buffer is refused instead of truncated, and a trunk tensor's payload must
 * lie inside trunk.bin before it is read.
 */
#include "waste_hip.h"
#include "json.h"

#include <errno.h>
#include <fcntl.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#define CT_MAX_LAYERS 128                 /* WASTE_MAX_LAYERS, src/model.h:73  */
#define CT_MAX_MANIFEST ((size_t)256 << 20)
#define CT_MAX_BOOKS ((size_t)1 << 30)     /* codebooks.bin bytes read whole   */
#define CT_PATH 4096
#define CT_NAME 512

typedef struct {
    char name[CT_NAME];
    int fmt, ndim, shape[4], group;
    int64_t off, soff;
    size_t n;
    int state;                            /* 0 unread, 1 read, < 0 the error  */
    void *q;
    uint16_t *qs;
    size_t rows, cols, rowbytes;
} ct_tensor;

typedef struct {
    int present, fd, n_experts, cb_base;
    int64_t rec_bytes;
} ct_bank;

struct waste_hip_container {
    waste_hip_container_cfg cfg;
    int verify;
    int expert_m[3];                      /* output rows of gate, up, down    */
    uint16_t *books;                      /* [n_books][entries * vec_dim]     */
    ct_bank bank[CT_MAX_LAYERS];
    ct_tensor *t;
    int trunk_fd;
    int64_t trunk_bytes;
    pthread_mutex_t mu;
    int err, err_layer, err_expert;
};

static int64_t fd_size(int fd)
{
    struct stat st;
    if (fstat(fd, &st) != 0 || !S_ISREG(st.st_mode)) return -1;
    return (int64_t)st.st_size;
}

/* pread until n bytes or EOF; returns the bytes read, -1 on error */
static int64_t pread_full(int fd, void *dst, size_t n, int64_t off)
{
    size_t got = 0;
    while (got < n) {
        const ssize_t r = pread(fd, (char *)dst + got, n - got, (off_t)(off + (int64_t)got));
        if (r < 0) {
            if (errno == EINTR) continue;
            return -1;
        }
        if (r == 0) break;
        got += (size_t)r;
    }
    return (int64_t)got;
}

/* A whole small file into memory (NUL-terminated); NULL when missing or
 * larger than cap. */
static char *slurp(const char *path, size_t cap, size_t *len)
{
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return NULL;
    const int64_t n = fd_size(fd);
    char *buf = NULL;
    if (n >= 0 && (size_t)n <= cap) {
        buf = (char *)malloc((size_t)n + 1);
        if (buf && pread_full(fd, buf, (size_t)n, 0) != n) {
            free(buf);
            buf = NULL;
        }
        if (buf) {
            buf[n] = 0;
            *len = (size_t)n;
        }
    }
    close(fd);
    return buf;
}

static int join(char *out, const char *dir, const char *name)
{
    const int n = snprintf(out, CT_PATH, "%s/%s", dir, name);
    return n > 0 && n < CT_PATH ? 0 : -1;
}

/* A bank file name stays inside the container directory. */
static int safe_name(const char *s)
{
    if (!*s || *s == '/') return 0;
    for (const char *p = s; *p;) {
        const char *e = strchr(p, '/');
        const size_t n = e ? (size_t)(e - p) : strlen(p);
        if (n == 2 && p[0] == '.' && p[1] == '.') return 0;
        p += n + (e ? 1 : 0);
    }
    return 1;
}

/* int64 in [lo, hi] from node v (absent: dflt); -1 when out of range */
static int get_int(const jdoc *d, int obj, const char *key, int64_t dflt, int64_t lo, int64_t hi, int *out)
{
    const int64_t v = jint(d, jget(d, obj, key), dflt);
    if (v < lo || v > hi) return -1;
    *out = (int)v;
    return 0;
}

/* The MoE keys of `config` (cfg_from_json, src/model.c:2186-2214), bounded
 * as cfg_sane bounds them (src/model.c:1813-1850). */
static int read_config(const jdoc *d, waste_hip_container_cfg *c)
{
    int cfg = jget(d, 0, "config");
    if (jstr(d, jget(d, 0, "tensor_prefix"), c->prefix, sizeof c->prefix) < 0) {
        if (jtype(d, jget(d, 0, "tensor_prefix")) == JN_STR) return -1;   /* too long */
        c->prefix[0] = 0;
    }
    const int tc = jget(d, cfg, "text_config");
    if (tc >= 0) {
        cfg = tc;
        if (!c->prefix[0]) snprintf(c->prefix, sizeof c->prefix, "language_model.");
    }
    if (get_int(d, cfg, "num_hidden_layers", 0, 1, CT_MAX_LAYERS, &c->n_layers)) return -1;
    if (get_int(d, cfg, "hidden_size", 0, 1, 1 << 20, &c->hidden)) return -1;
    if (get_int(d, cfg, "vocab_size", 0, 1, 1 << 24, &c->vocab)) return -1;
    int heads;
    if (get_int(d, cfg, "num_attention_heads", 0, 1, 1 << 16, &heads)) return -1;
    const double eps = jnum(d, jget(d, cfg, "rms_norm_eps"), 1e-5);
    if (!((float)eps > 0.0f) || !((float)eps < 1.0f)) return -1;
    if (get_int(d, cfg, "num_experts", 0, 0, 1 << 20, &c->n_experts)) return -1;
    if (get_int(d, cfg, "num_experts_per_token", 0, 0, 1 << 20, &c->top_k)) return -1;
    if (!c->top_k && get_int(d, cfg, "num_experts_per_tok", 0, 0, 1 << 20, &c->top_k)) return -1;
    if (c->n_experts && (c->top_k < 1 || c->top_k > c->n_experts || c->top_k > 64)) return -1;
    if (get_int(d, cfg, "moe_intermediate_size", 0, 0, 1 << 20, &c->moe_inter)) return -1;
    if (get_int(d, cfg, "num_shared_experts", 0, 0, 64, &c->n_shared)) return -1;
    if (get_int(d, cfg, "first_k_dense_replace", 0, 0, c->n_layers, &c->first_dense)) return -1;
    if (get_int(d, cfg, "routed_expert_hidden_size", 0, 0, 1 << 20, &c->latent_dim)) return -1;
    c->routed_scale = (float)jnum(d, jget(d, cfg, "routed_scaling_factor"), 1.0);
    c->renorm = jget(d, cfg, "moe_renormalize") >= 0;     /* presence, as the engine reads it */
    char sf[32];
    jstr(d, jget(d, cfg, "scoring_func"), sf, sizeof sf);
    c->score_func = strcmp(sf, "softmax") == 0 ? WASTE_SCORE_SOFTMAX
                  : strcmp(sf, "sqrtsoftplus") == 0 ? WASTE_SCORE_SQRTSOFTPLUS : WASTE_SCORE_SIGMOID;
    /* DeepSeek-V3's group limit, kept for callers that ask for it */
    if (get_int(d, cfg, "n_group", 1, 1, 1 << 16, &c->n_group)) return -1;
    if (get_int(d, cfg, "topk_group", 1, 1, 1 << 16, &c->topk_group)) return -1;
    return 0;
}

/* expert_quant (src/model.c:2709-2741) */
static int read_quant(const jdoc *d, waste_hip_container_cfg *c)
{
    const int eq = jget(d, 0, "expert_quant");
    if (get_int(d, eq, "stages", 3, 1, 8, &c->stages)) return -1;
    if (get_int(d, eq, "vec_dim", 8, 1, 64, &c->vec_dim)) return -1;
    if (get_int(d, eq, "entries", 256, 1, 256, &c->entries)) return -1;
    if (get_int(d, eq, "index_bits", 8, 0, 64, &c->index_bits)) return -1;
    if (c->index_bits != 8 && (c->index_bits != 6 || c->stages != 4 || c->entries != 64)) return -1;
    if (get_int(d, eq, "index_block", 64, 64, 64, &c->index_block)) return -1;
    return 0;
}

/* trunk entries, checked as load_trunk checks them (src/model.c:1306-1330) */
static int read_trunk_index(waste_hip_container *c, const jdoc *d)
{
    const int tr = jget(d, 0, "trunk");
    const int n = jsize(d, tr);
    if (tr >= 0 && jtype(d, tr) != JN_ARR) return WASTE_HIP_EFORMAT;
    c->cfg.n_tensors = n;
    c->t = (ct_tensor *)calloc((size_t)(n > 0 ? n : 1), sizeof *c->t);
    if (!c->t) return WASTE_HIP_ENOMEM;
    const int64_t fsize = c->trunk_bytes;
    for (int i = 0; i < n; i++) {
        const int e = jat(d, tr, i);
        ct_tensor *t = &c->t[i];
        if (jstr(d, jget(d, e, "name"), t->name, sizeof t->name) < 0) return WASTE_HIP_EFORMAT;
        const int64_t fmt = jint(d, jget(d, e, "fmt"), 0);
        t->off = jint(d, jget(d, e, "off"), 0);
        const int64_t g = jint(d, jget(d, e, "group"), 128);
        t->soff = jint(d, jget(d, e, "scale_off"), 0);
        const int sh = jget(d, e, "shape");
        t->ndim = jsize(d, sh);
        if (jtype(d, sh) != JN_ARR || t->ndim < 1 || t->ndim > 4 || g < 1 || g > (1 << 26)) return WASTE_HIP_EFORMAT;
        if (fmt < 0 || fmt > 255) return WASTE_HIP_EFORMAT;
        if (t->off < 0 || t->off > fsize || t->soff < 0 || t->soff > fsize) return WASTE_HIP_EFORMAT;
        t->fmt = (int)fmt;
        t->group = (int)g;
        t->n = 1;
        for (int k = 0; k < 4; k++) t->shape[k] = 1;
        for (int k = 0; k < t->ndim; k++) {
            const int64_t v = jint(d, jat(d, sh, k), 1);
            if (v < 1 || v > (1 << 26)) return WASTE_HIP_EFORMAT;
            t->shape[k] = (int)v;
            t->n *= (size_t)v;
            if (t->n > (size_t)fsize) return WASTE_HIP_EFORMAT;
        }
    }
    return 0;
}

static int read_books(waste_hip_container *c, const char *dir)
{
    char path[CT_PATH];
    if (join(path, dir, "codebooks.bin")) return WASTE_HIP_EFORMAT;
    size_t len = 0;
    char *raw = slurp(path, CT_MAX_BOOKS, &len);
    if (!raw) return WASTE_HIP_EIO;
    const size_t per = (size_t)c->cfg.entries * c->cfg.vec_dim;
    const size_t rec = 16 + per * 2;
    const size_t nb = len / rec;                  /* a partial last record is ignored */
    if (nb > (size_t)1 << 20) {
        free(raw);
        return WASTE_HIP_EFORMAT;
    }
    c->cfg.n_books = (int)nb;
    c->books = (uint16_t *)malloc(nb ? nb * per * 2 : 2);
    if (!c->books) {
        free(raw);
        return WASTE_HIP_ENOMEM;
    }
    for (size_t b = 0; b < nb; b++) memcpy(c->books + b * per, raw + b * rec + 16, per * 2);
    free(raw);
    return 0;
}

/* layers (src/model.c:2957-2983) and the probe of each bank's last record
 * (src/model.c:3060-3100) */
static int open_banks(waste_hip_container *c, const jdoc *d, const char *dir)
{
    const waste_hip_container_cfg *g = &c->cfg;
    const int layers = jget(d, 0, "layers");
    for (int L = 0; L < g->n_layers; L++) {
        char key[16];
        snprintf(key, sizeof key, "%d", L);
        const int e = jget(d, layers, key);
        const int expected = g->n_experts && L >= g->first_dense;
        if (e < 0) {
            if (expected) return WASTE_HIP_EFORMAT;
            continue;
        }
        char fn[CT_NAME];
        if (jstr(d, jget(d, e, "file"), fn, sizeof fn) < 0 || !safe_name(fn)) return WASTE_HIP_EFORMAT;
        const int64_t ne = jint(d, jget(d, e, "experts"), 0);
        const int64_t cb = jint(d, jget(d, e, "codebook_base"), 0);
        const int64_t bytes = jint(d, jget(d, e, "bytes"), 0);
        if (!expected || ne != g->n_experts || bytes <= 0 || bytes % ne != 0 || cb < 0 ||
            3 * g->stages > g->n_books || cb > g->n_books - 3 * g->stages)
            return WASTE_HIP_EFORMAT;
        ct_bank *b = &c->bank[L];
        b->n_experts = (int)ne;
        b->cb_base = (int)cb;
        b->rec_bytes = bytes / ne;
        char path[CT_PATH];
        if (join(path, dir, fn)) return WASTE_HIP_EFORMAT;
        b->fd = open(path, O_RDONLY | O_CLOEXEC);
        if (b->fd < 0) return WASTE_HIP_EIO;
        b->present = 1;
        const int64_t have = fd_size(b->fd);
        if (have < 0) return WASTE_HIP_EIO;
        if (b->rec_bytes >= (int64_t)WASTE_ALIGN && b->rec_bytes % (int64_t)WASTE_ALIGN == 0 &&
            have < (ne - 1) * b->rec_bytes + (int64_t)WASTE_ALIGN)
            return WASTE_HIP_EIO;
    }
    return 0;
}

int waste_hip_container_open(const char *dir, int verify, waste_hip_container **out)
{
    if (!out) return WASTE_HIP_EINVAL;
    *out = NULL;
    if (!dir || strlen(dir) >= CT_PATH - CT_NAME - 2) return WASTE_HIP_EINVAL;
    waste_hip_container *c = (waste_hip_container *)calloc(1, sizeof *c);
    if (!c) return WASTE_HIP_ENOMEM;
    pthread_mutex_init(&c->mu, NULL);
    c->verify = verify != 0;
    c->trunk_fd = -1;
    for (int L = 0; L < CT_MAX_LAYERS; L++) c->bank[L].fd = -1;

    char path[CT_PATH];
    size_t len = 0;
    jdoc d;
    memset(&d, 0, sizeof d);
    char *src = NULL;
    int rc = WASTE_HIP_EIO;
    join(path, dir, "manifest.json");
    if (!(src = slurp(path, CT_MAX_MANIFEST, &len))) goto fail;
    rc = WASTE_HIP_EFORMAT;
    if (jdoc_parse(&d, src, len) || jtype(&d, 0) != JN_OBJ) goto fail;
    /* format_version: present and 0 (src/model.c:2640-2660) */
    const int fv = jget(&d, 0, "format_version");
    if (jtype(&d, fv) != JN_NUM || jint(&d, fv, -1) != 0) goto fail;
    if (read_config(&d, &c->cfg) || read_quant(&d, &c->cfg)) goto fail;
    {
        const waste_hip_container_cfg *g = &c->cfg;
        const int lat = g->latent_dim ? g->latent_dim : g->hidden;
        c->expert_m[0] = c->expert_m[1] = g->moe_inter;
        c->expert_m[2] = lat;
    }
    rc = WASTE_HIP_EIO;
    join(path, dir, "trunk.bin");
    c->trunk_fd = open(path, O_RDONLY | O_CLOEXEC);
    if (c->trunk_fd < 0 || (c->trunk_bytes = fd_size(c->trunk_fd)) < 0) goto fail;
    if ((rc = read_trunk_index(c, &d)) != 0) goto fail;
    if ((rc = read_books(c, dir)) != 0) goto fail;
    if ((rc = open_banks(c, &d, dir)) != 0) goto fail;
    jdoc_free(&d);
    free(src);
    *out = c;
    return 0;
fail:
    jdoc_free(&d);
    free(src);
    waste_hip_container_close(c);
    return rc;
}

void waste_hip_container_close(waste_hip_container *c)
{
    if (!c) return;
    for (int L = 0; L < CT_MAX_LAYERS; L++)
        if (c->bank[L].fd >= 0) close(c->bank[L].fd);
    if (c->trunk_fd >= 0) close(c->trunk_fd);
    if (c->t)
        for (int i = 0; i < c->cfg.n_tensors; i++) {
            free(c->t[i].q);
            free(c->t[i].qs);
        }
    free(c->t);
    free(c->books);
    pthread_mutex_destroy(&c->mu);
    free(c);
}

int waste_hip_container_config(const waste_hip_container *c, waste_hip_container_cfg *out)
{
    if (!c || !out) return WASTE_HIP_EINVAL;
    *out = c->cfg;
    return 0;
}

int waste_hip_container_bank(const waste_hip_container *c, int layer, int *n_experts, int *codebook_base,
                             size_t *rec_bytes)
{
    if (!c || layer < 0 || layer >= CT_MAX_LAYERS || !c->bank[layer].present) return WASTE_HIP_EINVAL;
    const ct_bank *b = &c->bank[layer];
    if (n_experts) *n_experts = b->n_experts;
    if (codebook_base) *codebook_base = b->cb_base;
    if (rec_bytes) *rec_bytes = (size_t)b->rec_bytes;
    return 0;
}

const uint16_t *waste_hip_container_codebooks(const waste_hip_container *c, int *n_books)
{
    if (n_books) *n_books = c ? c->cfg.n_books : 0;
    return c ? c->books : NULL;
}

/* record_check (src/model.c:3645-3692) against the container's geometry */
static int record_ok(const waste_hip_container *c, int layer, int expert, const uint8_t *rec, size_t rec_bytes)
{
    waste_expert_hdr h;
    if (rec_bytes < sizeof h) return WASTE_HIP_ERECORD;
    memcpy(&h, rec, sizeof h);
    if (h.magic != WASTE_MAGIC_EXPERT) return WASTE_HIP_ERECORD;
    if (h.layer != (uint16_t)layer || h.expert_id != (uint16_t)expert) return WASTE_HIP_ERECORD;
    if ((size_t)h.rec_4k_blocks * WASTE_ALIGN != rec_bytes) return WASTE_HIP_ERECORD;
    const int bits = c->cfg.index_bits;
    if (h.fmt != (bits == 6 ? WQ_VQ4P : WQ_VQ3R) && !(bits == 8 && h.fmt == WQ_VQ2R)) return WASTE_HIP_ERECORD;
    if (h.lowrank_id != 0) return WASTE_HIP_ERECORD;
    if ((long)h.codebook_id + 3L * c->cfg.stages > (long)c->cfg.n_books) return WASTE_HIP_ERECORD;
    if (!(h.gate_off == sizeof h && h.gate_off < h.up_off && h.up_off < h.down_off &&
          h.down_off < h.chan_corr_off && h.chan_corr_off <= rec_bytes))
        return WASTE_HIP_ERECORD;
    const size_t scales = 2u * (size_t)(c->expert_m[0] + c->expert_m[1] + c->expert_m[2]);
    if (scales > rec_bytes - h.chan_corr_off) return WASTE_HIP_ERECORD;
    if (!c->verify) return 0;
    const size_t payload = (size_t)h.chan_corr_off + scales - sizeof h;
    return waste_hip_crc32(0, rec + sizeof h, payload) == h.crc32 ? 0 : WASTE_HIP_ECRC;
}

/* first failure wins (bank_fail, src/model.c:3700-3710) */
static int note_fail(waste_hip_container *c, int rc, int layer, int expert)
{
    pthread_mutex_lock(&c->mu);
    if (!c->err) {
        c->err = rc;
        c->err_layer = layer;
        c->err_expert = expert;
    }
    pthread_mutex_unlock(&c->mu);
    return rc;
}

int waste_hip_container_read_expert(waste_hip_container *c, int layer, int expert, void *dst, size_t dst_bytes)
{
    if (!c || !dst) return WASTE_HIP_EINVAL;
    if (layer < 0 || layer >= CT_MAX_LAYERS || !c->bank[layer].present || expert < 0 ||
        expert >= c->bank[layer].n_experts)
        return note_fail(c, WASTE_HIP_EINVAL, layer, expert);
    const ct_bank *b = &c->bank[layer];
    if (dst_bytes < (size_t)b->rec_bytes) return WASTE_HIP_EINVAL;
    const int64_t got = pread_full(b->fd, dst, (size_t)b->rec_bytes, (int64_t)expert * b->rec_bytes);
    if (got != b->rec_bytes) return note_fail(c, WASTE_HIP_EIO, layer, expert);
    const int rc = record_ok(c, layer, expert, (const uint8_t *)dst, (size_t)b->rec_bytes);
    return rc ? note_fail(c, rc, layer, expert) : 0;
}

int waste_hip_container_read_bank(waste_hip_container *c, int layer, void *dst, size_t dst_bytes)
{
    if (!c || !dst || layer < 0 || layer >= CT_MAX_LAYERS || !c->bank[layer].present) return WASTE_HIP_EINVAL;
    const ct_bank *b = &c->bank[layer];
    if (dst_bytes / (size_t)b->rec_bytes < (size_t)b->n_experts) return WASTE_HIP_EINVAL;
    for (int e = 0; e < b->n_experts; e++) {
        const int rc = waste_hip_container_read_expert(c, layer, e, (uint8_t *)dst + (size_t)e * b->rec_bytes,
                                                       (size_t)b->rec_bytes);
        if (rc) return rc;
    }
    return 0;
}

int waste_hip_container_error(const waste_hip_container *c, int *layer, int *expert)
{
    if (!c) return WASTE_HIP_EINVAL;
    pthread_mutex_lock((pthread_mutex_t *)&c->mu);
    const int rc = c->err;
    if (layer) *layer = c->err_layer;
    if (expert) *expert = c->err_expert;
    pthread_mutex_unlock((pthread_mutex_t *)&c->mu);
    return rc;
}

/* Reads tensor t (the load half of load_trunk, src/model.c:1366-1395):
 * F32 as n floats; every other fmt as Q rows of `bits` per weight (4 for
 * Q4G, 3 for Q3G, 8 otherwise) in groups of `group`, 3-bit rows a
 * bitstream plus a guard byte, then rows x groups f16 scales. */
static int load_tensor(waste_hip_container *c, ct_tensor *t)
{
    const int64_t fsize = c->trunk_bytes;
    const size_t N = (size_t)t->shape[t->ndim - 1];
    t->cols = N;
    t->rows = t->n / N;
    if (t->fmt == WQ_F32) {
        const size_t bytes = t->n * 4;
        if ((int64_t)bytes > fsize - t->off) return WASTE_HIP_EFORMAT;
        t->rowbytes = N * 4;
        if (!(t->q = malloc(bytes ? bytes : 4))) return WASTE_HIP_ENOMEM;
        if (pread_full(c->trunk_fd, t->q, bytes, t->off) != (int64_t)bytes) return WASTE_HIP_EIO;
        return 0;
    }
    const size_t g = (size_t)t->group;
    const size_t ng = (N + g - 1) / g;
    const int bits = t->fmt == WQ_Q4G ? 4 : t->fmt == WQ_Q3G ? 3 : 8;
    t->rowbytes = bits == 3 ? (ng * g * 3 + 7) / 8 + 1 : ng * g * (size_t)bits / 8;
    if (t->rowbytes && t->rows > (size_t)fsize / t->rowbytes) return WASTE_HIP_EFORMAT;
    const size_t payload = t->rows * t->rowbytes;
    if (t->rows > (size_t)fsize / (ng * 2)) return WASTE_HIP_EFORMAT;
    const size_t sbytes = t->rows * ng * 2;
    if ((int64_t)payload > fsize - t->off || (int64_t)sbytes > fsize - t->soff) return WASTE_HIP_EFORMAT;
    t->q = malloc(payload ? payload : 1);
    t->qs = (uint16_t *)malloc(sbytes ? sbytes : 2);
    if (!t->q || !t->qs) return WASTE_HIP_ENOMEM;
    if (pread_full(c->trunk_fd, t->q, payload, t->off) != (int64_t)payload ||
        pread_full(c->trunk_fd, t->qs, sbytes, t->soff) != (int64_t)sbytes)
        return WASTE_HIP_EIO;
    return 0;
}

int waste_hip_container_tensor(waste_hip_container *c, const char *name, waste_hip_tensor *out, int *ndim,
                               int shape[4])
{
    if (!c || !name || !out) return WASTE_HIP_EINVAL;
    memset(out, 0, sizeof *out);
    ct_tensor *t = NULL;
    for (int i = 0; i < c->cfg.n_tensors && !t; i++)
        if (strcmp(c->t[i].name, name) == 0) t = &c->t[i];
    if (!t) return WASTE_HIP_EFORMAT;
    pthread_mutex_lock(&c->mu);
    if (t->state == 0) {
        const int rc = load_tensor(c, t);
        t->state = rc ? rc : 1;
        if (rc) {
            free(t->q);
            free(t->qs);
            t->q = NULL;
            t->qs = NULL;
        }
    }
    const int st = t->state;
    pthread_mutex_unlock(&c->mu);
    if (st < 0) return st;
    if (t->rows > (size_t)INT32_MAX || t->cols > (size_t)INT32_MAX) return WASTE_HIP_EFORMAT;
    out->fmt = t->fmt;
    out->rows = (int)t->rows;
    out->cols = (int)t->cols;
    out->group = t->fmt == WQ_F32 ? 0 : t->group;
    out->q = t->q;
    out->qs = t->qs;
    out->rowbytes = t->rowbytes;
    if (ndim) *ndim = t->ndim;
    if (shape) memcpy(shape, t->shape, sizeof t->shape);
    return 0;
}
