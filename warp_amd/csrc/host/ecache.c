/* SPDX-License-Identifier: Apache-2.0 */
/*
 * ecache.c — the engine's expert cache (src/ecache.c) as an HBM slab.
 *
 * Slots are rec_bytes each, carved from one device allocation of the
 * budget.  A miss is filled by hipMemcpyAsync from the record's host copy
 * (pinned memory, so the copy is a DMA) on the cache's own stream.  get()
 * and hold() return the slot's device address at once and make the
 * caller's stream wait for the fill, so the host never blocks on a read.
 *
 * A slot is refilled only after the work that last read it.  release(s)
 * records an event on the caller's stream after its kernels; a later fill
 * into any slot handed out before that release waits for the event on the
 * fill stream.  A slot refilled while still handed out (a get() pointer
 * the policy lets go before the release) waits for the work enqueued so
 * far on the stream it was last handed to.  Releases are expected on one stream (or on streams the
 * caller orders), since an event slot of the ring is reused after RING
 * releases and then stands for a later point of the same stream.
 *
 * The policy is the engine's, decision for decision (src/ecache.c): a free
 * slot first, else the least (hits, last) of 16 slots drawn by the LCG
 * (LRU: least last); a claim resets hits to 1; hints pin their records by
 * generation (at most a quarter of the slots) and release `depth` reads at
 * once and one more per get; lookahead reads are speculative (bytes, not
 * misses); hits and misses count the demand stream only; held slots and the
 * last one handed out are never victims.  The engine's reads finish in the
 * background: here a read counts as in flight, and so is never a victim,
 * until the next demand get.  That is the engine's order when every read
 * lands before the layer asks for the next record.
 */
#include "waste_hip.h"

#include <hip/hip_runtime_api.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

enum { S_EMPTY = 0, S_READY, S_INFLIGHT };
#define SAMPLE 16
#define PF_MAX 64
#define RING 64

typedef struct {
    int32_t key;                     /* (layer << 16) | expert, -1 empty   */
    uint8_t state, fresh, out;
    uint8_t spec;                    /* a lookahead read not demanded yet  */
    uint32_t hits;
    uint64_t last, pin;
    uint64_t use;                    /* release that last covered a reader */
    hipEvent_t filled;
    int has_fill;
    int has_waiter;                  /* `waited` is ordered after the fill */
    void *waited;                    /* (the null stream is a value too)   */
    void *out_stream;                /* the stream it was last handed to   */
} slot_t;

struct waste_hip_ecache {
    slot_t *slot;
    int32_t *hash;                   /* linear probing, -1 empty           */
    uint32_t hmask;
    int n_slots, depth, io, lru, dry;
    size_t rec_bytes;
    uint8_t *slab;
    hipStream_t fill;
    hipEvent_t ring[RING];
    hipEvent_t evict;                /* a handed-out slot's readers so far */
    uint64_t n_release;
    int *out_list, n_out;            /* handed out since the last release  */
    int *inflight, n_inflight;
    int n_used;                      /* slots [0, n_used) have held a key  */
    int fill_cursor;
    const void *const *src;          /* host records [n_layers][n_experts] */
    int src_layers, src_experts;
    uint64_t clock, pf_gen;
    uint32_t rng;
    int pf_ids[PF_MAX], pf_layer, pf_n, pf_issued, last_used;
    int held[PF_MAX], n_held;
    waste_hip_ecache_counts st;
    int failed;
};

static int32_t key_of(int layer, int expert) { return (int32_t)(((uint32_t)layer << 16) | (uint32_t)expert); }

static uint32_t hslot(const waste_hip_ecache *c, int32_t key)
{
    return ((uint32_t)key * 2654435761u) & c->hmask;
}

static int lookup(const waste_hip_ecache *c, int32_t key)
{
    for (uint32_t h = hslot(c, key);; h = (h + 1) & c->hmask) {
        const int32_t si = c->hash[h];
        if (si < 0) return -1;
        if (c->slot[si].key == key) return si;
    }
}

static void h_insert(waste_hip_ecache *c, int32_t key, int si)
{
    uint32_t h = hslot(c, key);
    while (c->hash[h] >= 0) h = (h + 1) & c->hmask;
    c->hash[h] = si;
}

/* Delete by shifting later members of the probe run back (no tombstones,
 * so lookups stay short however many evictions there are). */
static void h_erase(waste_hip_ecache *c, int32_t key)
{
    uint32_t h = hslot(c, key);
    while (c->slot[c->hash[h]].key != key) h = (h + 1) & c->hmask;
    uint32_t hole = h;
    for (uint32_t j = (hole + 1) & c->hmask; c->hash[j] >= 0; j = (j + 1) & c->hmask) {
        const uint32_t home = hslot(c, c->slot[c->hash[j]].key);
        /* j may move to the hole when its home is not in (hole, j] */
        const int stays = hole <= j ? (home > hole && home <= j) : (home > hole || home <= j);
        if (!stays) {
            c->hash[hole] = c->hash[j];
            hole = j;
        }
    }
    c->hash[hole] = -1;
}

static int is_held(const waste_hip_ecache *c, int i)
{
    for (int k = 0; k < c->n_held; k++)
        if (c->held[k] == i) return 1;
    return 0;
}

static int pinned(const waste_hip_ecache *c, int i)
{
    const slot_t *q = &c->slot[i];
    return q->state == S_INFLIGHT || q->pin == c->pf_gen || i == c->last_used || is_held(c, i);
}

static int victim(waste_hip_ecache *c)
{
    if (c->n_used < c->n_slots) return c->n_used;        /* first empty slot */
    int best = -1;
    uint32_t bh = 0;
    uint64_t bl = 0;
    for (int s = 0; s < SAMPLE; s++) {
        c->rng = c->rng * 1664525u + 1013904223u;
        const int i = (int)(c->rng % (uint32_t)c->n_slots);
        if (pinned(c, i)) continue;
        const slot_t *q = &c->slot[i];
        const int better = c->lru ? (best < 0 || q->last < bl)
                                  : (best < 0 || q->hits < bh || (q->hits == bh && q->last < bl));
        if (better) {
            best = i;
            bh = q->hits;
            bl = q->last;
        }
    }
    if (best < 0)
        for (int i = 0; i < c->n_slots; i++)
            if (!pinned(c, i)) return i;
    return best;
}

/* The host copy of (layer, expert), or NULL when the source has none. */
static const void *source_of(const waste_hip_ecache *c, int layer, int expert)
{
    if (c->src && layer >= 0 && layer < c->src_layers && expert >= 0 && expert < c->src_experts)
        return c->src[(size_t)layer * c->src_experts + expert];
    return NULL;
}

/* Copy (layer, expert) into slot si after the slot's last reader. */
static int copy_in(waste_hip_ecache *c, int si, int layer, int expert)
{
    if (c->dry) return 0;
    const void *src = source_of(c, layer, expert);
    slot_t *q = &c->slot[si];
    if (!src) goto fail;
    if (q->use && hipStreamWaitEvent(c->fill, c->ring[q->use % RING], 0) != hipSuccess) goto fail;
    /* A slot handed out by get() and not released yet can be the victim
     * of a later demand (the policy pins only the last one handed out and
     * the held ones).  Its readers are whatever the caller enqueued on the
     * stream it went to before this call: the fill waits for them. */
    if (q->out && (hipEventRecord(c->evict, (hipStream_t)q->out_stream) != hipSuccess ||
                   hipStreamWaitEvent(c->fill, c->evict, 0) != hipSuccess))
        goto fail;
    if (hipMemcpyAsync(c->slab + (size_t)si * c->rec_bytes, src, c->rec_bytes, hipMemcpyHostToDevice,
                       c->fill) != hipSuccess)
        goto fail;
    if (hipEventRecord(q->filled, c->fill) != hipSuccess) goto fail;
    q->has_fill = 1;
    q->has_waiter = 0;
    return 0;
fail:
    c->failed = 1;
    return -1;
}

static int start_fill(waste_hip_ecache *c, int si, int layer, int expert)
{
    c->st.reads++;
    c->st.bytes_read += c->rec_bytes;
    return copy_in(c, si, layer, expert);
}

/* Give slot si to key: the engine's claim (hits 1, last = now). */
static void claim(waste_hip_ecache *c, int si, int32_t key, uint8_t state)
{
    slot_t *q = &c->slot[si];
    if (q->key >= 0) {
        h_erase(c, q->key);
        c->st.evictions++;
        if (q->spec) c->st.spec_wasted++;           /* read ahead, never demanded */
    }
    q->spec = 0;
    if (si >= c->n_used) c->n_used = si + 1;
    q->key = key;
    h_insert(c, key, si);
    q->state = state;
    q->hits = 1;
    q->last = c->clock;
    if (state == S_INFLIGHT) c->inflight[c->n_inflight++] = si;
}

static void issue_next(waste_hip_ecache *c)
{
    if (!c->io) return;
    while (c->pf_issued < c->pf_n) {
        const int eid = c->pf_ids[c->pf_issued++];
        const int32_t key = key_of(c->pf_layer, eid);
        const int si = lookup(c, key);
        if (si >= 0) {
            c->slot[si].pin = c->pf_gen;
            continue;
        }
        const int vi = victim(c);
        if (vi < 0) {
            c->pf_issued--;
            return;
        }
        claim(c, vi, key, S_INFLIGHT);
        c->slot[vi].fresh = 1;
        c->slot[vi].pin = c->pf_gen;
        c->st.misses++;
        c->st.prefetched++;
        start_fill(c, vi, c->pf_layer, eid);
        return;
    }
}

int waste_hip_ecache_create(size_t rec_bytes, size_t budget_bytes, int policy, int depth, int dry,
                            waste_hip_ecache **out)
{
    if (!out) return WASTE_HIP_EINVAL;
    *out = NULL;
    if (!rec_bytes || rec_bytes % 256 || (policy != 0 && policy != 1) || depth < 0)
        return WASTE_HIP_EINVAL;
    const size_t n = budget_bytes / rec_bytes;
    if (n > (1u << 24)) return WASTE_HIP_EINVAL;
    waste_hip_ecache *c = (waste_hip_ecache *)calloc(1, sizeof *c);
    if (!c) return WASTE_HIP_ENOMEM;
    c->rec_bytes = rec_bytes;
    c->n_slots = (int)n;
    c->dry = dry;
    c->lru = policy;
    c->rng = 0x9e3779b9u;
    c->pf_gen = 1;
    c->last_used = -1;
    /* read-ahead as the engine starts it: depth >= 1, at most a quarter
     * of the slots in flight, off when that leaves none */
    int d = depth;
    if (d > c->n_slots / 4) d = c->n_slots / 4;
    c->depth = d;
    c->io = depth > 0 && d >= 1;
    uint32_t hs = 2;
    while (hs < 2u * (uint32_t)(c->n_slots + 1)) hs <<= 1;
    c->hmask = hs - 1;
    const size_t ns = (size_t)(c->n_slots > 0 ? c->n_slots : 1);
    c->slot = (slot_t *)calloc(ns, sizeof *c->slot);
    c->hash = (int32_t *)malloc((size_t)hs * sizeof *c->hash);
    c->out_list = (int *)malloc(ns * sizeof *c->out_list);
    c->inflight = (int *)malloc(ns * sizeof *c->inflight);
    if (!c->slot || !c->hash || !c->out_list || !c->inflight) {
        waste_hip_ecache_destroy(c);
        return WASTE_HIP_ENOMEM;
    }
    memset(c->hash, 0xff, (size_t)hs * sizeof *c->hash);
    for (int i = 0; i < c->n_slots; i++) c->slot[i].key = -1;
    if (!dry && c->n_slots > 0) {
        if (!waste_hip_device_name()) {
            waste_hip_ecache_destroy(c);
            return WASTE_HIP_ENODEV;
        }
        if (hipMalloc((void **)&c->slab, (size_t)c->n_slots * rec_bytes) != hipSuccess) {
            c->slab = NULL;
            waste_hip_ecache_destroy(c);
            return WASTE_HIP_ENOMEM;
        }
        int bad = hipStreamCreateWithFlags(&c->fill, hipStreamNonBlocking) != hipSuccess;
        for (int i = 0; !bad && i < RING; i++)
            bad = hipEventCreateWithFlags(&c->ring[i], hipEventDisableTiming) != hipSuccess;
        if (!bad) bad = hipEventCreateWithFlags(&c->evict, hipEventDisableTiming) != hipSuccess;
        for (int i = 0; !bad && i < c->n_slots; i++)
            bad = hipEventCreateWithFlags(&c->slot[i].filled, hipEventDisableTiming) != hipSuccess;
        if (bad) {
            waste_hip_ecache_destroy(c);
            return WASTE_HIP_EDEVICE;
        }
    }
    *out = c;
    return WASTE_HIP_OK;
}

void waste_hip_ecache_destroy(waste_hip_ecache *c)
{
    if (!c) return;
    if (c->fill) hipStreamSynchronize(c->fill);
    if (c->slot)
        for (int i = 0; i < c->n_slots; i++)
            if (c->slot[i].filled) hipEventDestroy(c->slot[i].filled);
    for (int i = 0; i < RING; i++)
        if (c->ring[i]) hipEventDestroy(c->ring[i]);
    if (c->evict) hipEventDestroy(c->evict);
    if (c->fill) hipStreamDestroy(c->fill);
    if (c->slab) hipFree(c->slab);
    free(c->slot);
    free(c->hash);
    free(c->out_list);
    free(c->inflight);
    free(c);
}

int waste_hip_ecache_set_source(waste_hip_ecache *c, const void *const *records, int n_layers,
                                int n_experts)
{
    if (!c || (records && (n_layers <= 0 || n_experts <= 0 || n_layers > 32768 || n_experts > 65536)))
        return WASTE_HIP_EINVAL;
    c->src = records;
    c->src_layers = records ? n_layers : 0;
    c->src_experts = records ? n_experts : 0;
    return WASTE_HIP_OK;
}

int waste_hip_ecache_hint(waste_hip_ecache *c, int layer, const int *ids, int n)
{
    if (!c) return WASTE_HIP_EINVAL;
    if (!c->io || c->n_slots <= 0 || n <= 0) return WASTE_HIP_OK;
    c->pf_gen++;
    c->pf_layer = layer;
    c->pf_n = n > PF_MAX ? PF_MAX : n;
    if (c->pf_n > c->n_slots / 4) c->pf_n = c->n_slots / 4;
    memcpy(c->pf_ids, ids, (size_t)c->pf_n * sizeof *ids);
    c->pf_issued = 0;
    for (int d = 0; d < c->depth; d++) issue_next(c);
    return c->failed ? WASTE_HIP_EDEVICE : WASTE_HIP_OK;
}

int waste_hip_ecache_prefetch(waste_hip_ecache *c, int layer, const int *ids, int n)
{
    if (!c) return WASTE_HIP_EINVAL;
    if (!c->io || c->n_slots <= 0 || n <= 0) return WASTE_HIP_OK;
    for (int i = 0; i < n; i++) {
        if (ids[i] < 0) continue;
        const int32_t key = key_of(layer, ids[i]);
        if (lookup(c, key) >= 0) continue;
        const int vi = victim(c);
        if (vi < 0) break;
        claim(c, vi, key, S_INFLIGHT);
        c->slot[vi].fresh = 0;
        c->slot[vi].pin = 0;
        c->slot[vi].spec = 1;
        c->st.spec_issued++;
        start_fill(c, vi, layer, ids[i]);
    }
    return c->failed ? WASTE_HIP_EDEVICE : WASTE_HIP_OK;
}

static const void *hand_out(waste_hip_ecache *c, int si, void *stream)
{
    slot_t *q = &c->slot[si];
    if (!q->out) {
        q->out = 1;
        c->out_list[c->n_out++] = si;
    }
    q->out_stream = stream;
    if (c->dry) return (const void *)(uintptr_t)(((size_t)si + 1) * c->rec_bytes);
    if (q->has_fill && !(q->has_waiter && q->waited == stream)) {
        if (hipStreamWaitEvent((hipStream_t)stream, q->filled, 0) != hipSuccess) return NULL;
        q->has_waiter = 1;
        q->waited = stream;
    }
    return c->slab + (size_t)si * c->rec_bytes;
}

/* The demand path: the slot for (layer, expert), claimed and filled on a
 * miss; -1 when every slot is pinned. */
static int demand(waste_hip_ecache *c, int layer, int expert)
{
    const int32_t key = key_of(layer, expert);
    c->clock++;
    c->last_used = -1;
    for (int k = 0; k < c->n_inflight; k++) c->slot[c->inflight[k]].state = S_READY;
    c->n_inflight = 0;
    if (c->n_slots <= 0) {
        c->st.misses++;
        c->st.reads++;
        c->st.bytes_read += c->rec_bytes;
        return -1;
    }
    int si = lookup(c, key);
    if (si >= 0) {
        slot_t *q = &c->slot[si];
        if (q->spec) {                               /* a lookahead read that landed */
            q->spec = 0;
            c->st.spec_used++;
        }
        if (q->fresh) q->fresh = 0;
        else {
            c->st.hits++;
            q->hits++;
        }
        q->last = c->clock;
    } else {
        si = victim(c);
        if (si < 0) return -1;
        claim(c, si, key, S_READY);
        c->slot[si].fresh = 0;
        c->slot[si].pin = 0;
        c->st.misses++;
        start_fill(c, si, layer, expert);
    }
    c->last_used = si;
    issue_next(c);
    return si;
}

const void *waste_hip_ecache_get(waste_hip_ecache *c, int layer, int expert, void *stream)
{
    if (!c) return NULL;
    const int si = demand(c, layer, expert);
    if (si < 0 || c->failed) return NULL;
    return hand_out(c, si, stream);
}

const void *waste_hip_ecache_hold(waste_hip_ecache *c, int layer, int expert, void *stream)
{
    if (!c || c->n_slots <= 0 || c->n_held >= PF_MAX) return NULL;
    const int si = demand(c, layer, expert);
    if (si < 0 || c->failed) return NULL;
    if (c->last_used >= 0) {
        if (!is_held(c, c->last_used)) c->held[c->n_held++] = c->last_used;
        c->last_used = -1;
    }
    return hand_out(c, si, stream);
}

int waste_hip_ecache_release(waste_hip_ecache *c, void *stream)
{
    if (!c) return WASTE_HIP_EINVAL;
    c->n_held = 0;
    if (c->n_out == 0) return WASTE_HIP_OK;
    if (!c->dry) {
        c->n_release++;
        if (hipEventRecord(c->ring[c->n_release % RING], (hipStream_t)stream) != hipSuccess)
            return WASTE_HIP_EDEVICE;
    }
    for (int k = 0; k < c->n_out; k++) {
        slot_t *q = &c->slot[c->out_list[k]];
        q->out = 0;
        q->use = c->n_release;
    }
    c->n_out = 0;
    return WASTE_HIP_OK;
}

int waste_hip_ecache_admit(waste_hip_ecache *c, int layer, int expert)
{
    if (!c) return WASTE_HIP_EINVAL;
    if (c->n_slots <= 0 || !c->io) return 0;
    const int32_t key = key_of(layer, expert);
    if (lookup(c, key) >= 0) return 0;
    int si = -1;
    while (c->fill_cursor < c->n_slots) {
        const int i = c->fill_cursor++;
        if (c->slot[i].key < 0) {
            si = i;
            break;
        }
    }
    if (si < 0) return 0;
    claim(c, si, key, S_READY);
    c->slot[si].fresh = 0;
    c->slot[si].pin = 0;
    return start_fill(c, si, layer, expert) ? WASTE_HIP_EDEVICE : 1;
}

int waste_hip_ecache_resident_mask(const waste_hip_ecache *c, int layer, int n, uint8_t *out)
{
    if (!c || !out || n < 0) return WASTE_HIP_EINVAL;
    for (int e = 0; e < n; e++) {
        const int si = c->n_slots > 0 ? lookup(c, key_of(layer, e)) : -1;
        out[e] = si >= 0 && c->slot[si].state == S_READY;
    }
    return WASTE_HIP_OK;
}

int waste_hip_ecache_resident_all(const waste_hip_ecache *c, int layer, const int *ids, int n)
{
    if (!c || c->n_slots <= 0 || n <= 0) return 0;
    for (int i = 0; i < n; i++) {
        const int si = lookup(c, key_of(layer, ids[i]));
        if (si < 0 || c->slot[si].state != S_READY) return 0;
    }
    return 1;
}

int waste_hip_ecache_stats(const waste_hip_ecache *c, waste_hip_ecache_counts *out)
{
    if (!c || !out) return WASTE_HIP_EINVAL;
    *out = c->st;
    return WASTE_HIP_OK;
}

int waste_hip_ecache_slot(const waste_hip_ecache *c, int layer, int expert)
{
    if (!c || c->n_slots <= 0) return -1;
    return lookup(c, key_of(layer, expert));
}

int waste_hip_ecache_n_slots(const waste_hip_ecache *c) { return c ? c->n_slots : 0; }

int waste_hip_ecache_sync(waste_hip_ecache *c)
{
    if (!c) return WASTE_HIP_EINVAL;
    if (c->failed) return WASTE_HIP_EDEVICE;
    if (c->dry || !c->fill) return WASTE_HIP_OK;
    return hipStreamSynchronize(c->fill) == hipSuccess ? WASTE_HIP_OK : WASTE_HIP_EDEVICE;
}

/* ---- the learned hotlist (src/ecache.c:825-913) --------------------------
 *
 * usage.waste: a 16-byte header (magic "WUSG", version 1, tokens) and one
 * 16-byte entry per resident record (layer, expert, hits, last use, a
 * coupling field written as 0; src/waste_format.h:169-187). */

typedef struct {
    uint32_t magic, version;
    uint64_t tokens;
} usage_hdr;

typedef struct {
    uint16_t layer, expert;
    uint32_t hits, last, next_top;
} usage_ent;

#define MAGIC_USAGE 0x47535557u
#define USAGE_MAX_ENTRIES (1u << 26)

int waste_hip_ecache_save_usage(const waste_hip_ecache *c, const char *path, uint64_t tokens)
{
    if (!c || !path) return WASTE_HIP_EINVAL;
    if (c->n_slots <= 0) return WASTE_HIP_OK;
    FILE *f = fopen(path, "wb");
    if (!f) return WASTE_HIP_EIO;
    const usage_hdr h = { MAGIC_USAGE, 1, tokens };
    int bad = fwrite(&h, sizeof h, 1, f) != 1;
    for (int i = 0; i < c->n_slots && !bad; i++) {
        const slot_t *q = &c->slot[i];
        if (q->key < 0 || q->state != S_READY) continue;
        usage_ent e;
        e.layer = (uint16_t)((uint32_t)q->key >> 16);
        e.expert = (uint16_t)(q->key & 0xFFFF);
        e.hits = q->hits;
        e.last = (uint32_t)q->last;
        e.next_top = 0;
        bad = fwrite(&e, sizeof e, 1, f) != 1;
    }
    if (fclose(f) != 0) bad = 1;
    if (bad) {
        remove(path);
        return WASTE_HIP_EIO;
    }
    return WASTE_HIP_OK;
}

/* hits descending, then (layer, expert): a file warms the same way every
 * run (src/ecache.c:852-862) */
static int hotter(const void *a, const void *b)
{
    const usage_ent *x = (const usage_ent *)a, *y = (const usage_ent *)b;
    if (x->hits != y->hits) return x->hits > y->hits ? -1 : 1;
    if (x->layer != y->layer) return x->layer < y->layer ? -1 : 1;
    if (x->expert != y->expert) return x->expert < y->expert ? -1 : 1;
    return 0;
}

int waste_hip_ecache_warm(waste_hip_ecache *c, const char *path)
{
    if (!c || !path) return WASTE_HIP_EINVAL;
    if (c->n_slots <= 0) return 0;
    FILE *f = fopen(path, "rb");
    if (!f) return WASTE_HIP_EIO;
    usage_hdr h;
    if (fread(&h, sizeof h, 1, f) != 1 || h.magic != MAGIC_USAGE) {
        fclose(f);
        return WASTE_HIP_EFORMAT;
    }
    long n = 0;
    if (fseek(f, 0, SEEK_END) == 0) {
        const long end = ftell(f);
        n = end > (long)sizeof h ? (end - (long)sizeof h) / (long)sizeof(usage_ent) : 0;
    }
    if (n <= 0) {
        fclose(f);
        return 0;
    }
    if ((unsigned long)n > USAGE_MAX_ENTRIES) {
        fclose(f);
        return WASTE_HIP_EFORMAT;
    }
    usage_ent *ent = (usage_ent *)malloc((size_t)n * sizeof *ent);
    if (!ent || fseek(f, (long)sizeof h, SEEK_SET) != 0 || fread(ent, sizeof *ent, (size_t)n, f) != (size_t)n) {
        free(ent);
        fclose(f);
        return ent ? WASTE_HIP_EIO : WASTE_HIP_ENOMEM;
    }
    fclose(f);
    qsort(ent, (size_t)n, sizeof *ent, hotter);
    const int want = n < c->n_slots ? (int)n : c->n_slots;
    int loaded = 0;
    for (int i = 0; i < want; i++) {
        const int32_t key = key_of(ent[i].layer, ent[i].expert);
        if (lookup(c, key) >= 0) continue;
        const int vi = victim(c);
        if (vi < 0) break;
        /* a record the source does not have is stale, not an error: skipped
         * before its slot is touched, as a failed fetch is */
        if (c->src && !source_of(c, ent[i].layer, ent[i].expert)) continue;
        if (!c->dry && !c->src) continue;
        slot_t *q = &c->slot[vi];
        if (q->key >= 0) h_erase(c, q->key);
        if (vi >= c->n_used) c->n_used = vi + 1;
        q->key = key;
        h_insert(c, key, vi);
        q->state = S_READY;
        q->fresh = 0;
        q->pin = 0;
        q->hits = ent[i].hits;
        q->last = ++c->clock;
        if (copy_in(c, vi, ent[i].layer, ent[i].expert)) {
            free(ent);
            return WASTE_HIP_EDEVICE;
        }
        loaded++;
    }
    free(ent);
    return loaded;
}
