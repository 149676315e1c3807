/* SPDX-License-Identifier: Apache-2.0 */
/*
 * waste_hip.h — the MI355X (gfx950) backend for WARP's MoE expert path.
 *
 * A C ABI: plain pointers and sizes, no C++ or framework types.  Three
 * levels, matching the three things a WARP engine would bind:
 *
 *   1. waste_register_hip  — a waste_kernels registration, the slot the
 *      engine's backend init already reserves for a device backend
 *      (src/backend.c:44-62, 206-216; semantics of waste_register_metal,
 *      src/metal.m:464-519).
 *   2. waste_hip_vq3r      — the VQ3R batch apply (waste_metal_vq3r,
 *      src/waste_metal.h:31-44): host jobs in, host rows out,
 *      all-or-nothing.
 *   3. waste_hip_moe_*     — a device-resident MoE layer that takes over
 *      moe_layer (src/model.c:5488-5939) and moe_chunk
 *      (src/model.c:7110-7285) from router logits to the combined output,
 *      with expert records resident in HBM.
 *
 * Return codes: 0 success; WASTE_HIP_E* (negative) on failure.
 */
#ifndef WASTE_HIP_H
#define WASTE_HIP_H

#include <stddef.h>
#include <stdint.h>

#include "waste_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

#define WASTE_HIP_OK          0
#define WASTE_HIP_EINVAL    (-1)   /* bad argument or shape              */
#define WASTE_HIP_ENODEV    (-2)   /* no gfx950 device                   */
#define WASTE_HIP_ENOMEM    (-3)   /* device allocation failed           */
#define WASTE_HIP_ERECORD   (-4)   /* record failed its header checks    */
#define WASTE_HIP_ECRC      (-5)   /* record payload checksum mismatch   */
#define WASTE_HIP_EUNBOUND  (-6)   /* a routed expert has no record      */
#define WASTE_HIP_EROUTE    (-7)   /* a selection pass found no expert   */
#define WASTE_HIP_EDEVICE   (-8)   /* a HIP runtime call failed          */
#define WASTE_HIP_ERANGE    (-9)   /* an fp16 operand of the many-token
                                      path was out of range              */
#define WASTE_HIP_ETIMEOUT  (-10)  /* a device-side wait gave up (~50 ms):
                                      the router launch's wait for the
                                      logits, or a stage of the one-launch
                                      decode (mode 1) */
#define WASTE_HIP_ESCRATCH  (-11)  /* the call needs more device memory than
                                      the library's static scratch area
                                      (16 MiB per GPU) holds             */
#define WASTE_HIP_EFORMAT   (-12)  /* a container's manifest or file layout
                                      is out of range or not understood
                                      (the engine's WASTE_E_FORMAT)      */
#define WASTE_HIP_EIO       (-13)  /* a container file is missing or a read
                                      came back short                    */

/* Library name and device check.  NULL when no usable gfx950 device. */
const char *waste_hip_device_name(void);

/* ---- 1. kernel-table registration ------------------------------------- */

/* Fills t->mvq_rows_f32 with a device implementation (whole range in one
 * call: t->on_device = 1) and t->device_min_bytes, and t->vq_rows_p6 (the
 * VQ4P apply through the engine's int8 LUT, vqp_arg) with one whose rows
 * are bit-identical to the CPU kernel it replaces; leaves every other slot
 * as it was.  A range the device declines or fails goes to that CPU
 * kernel.  Returns "HIP (gfx950)" or NULL to decline (no device).
 * Replaces: the accelerator registration of src/backend.c:206-216. */
const char *waste_register_hip(waste_kernels *t);

/* Drops the device copies of host tensors the slots have cached (keyed by
 * host address).  Call before the engine frees the host buffers.
 * Replaces: waste_metal_release_host_buffers, src/metal.m:521-531. */
void waste_hip_release_host_buffers(void);

/* ---- 2. VQ3R batch ----------------------------------------------------- */

/* Runs every job on the device: y[r] for r < m, each row's sum in the
 * engine's exact vq_rows order (bit-identical to the CPU path).  Host
 * pointers in, host rows out.  0 if every job ran; nonzero means nothing
 * was written and the caller must do them itself.
 * Replaces: waste_metal_vq3r, src/waste_metal.h:31-44. */
int waste_hip_vq3r(const waste_vq_job *jobs, int n);

/* ---- 2b. VQ4P on device pointers ---------------------------------------- */

/* The int8 shadow of an fp32 LUT [nv][stages][entries] (device pointers):
 * per block of 32 positions, scale[blk] = max|lut| / 127 and each entry
 * rint(lut * (127 / max)) clamped to [-127, 127].  Bit-identical to the
 * engine's quantisation.  q: nv*stages*entries bytes, scale: ceil(nv/32).
 * Replaces: vq_quant_lut, src/model.c:3979-4074. */
int waste_hip_vq_quant_lut(const float *lut, int nv, int stages, int entries, int8_t *q,
                           float *scale, void *stream);

/* Rows [r_lo, r_hi) of a VQ4P matrix (6-bit codes, three bytes per row and
 * position, 64-row blocks; idx, scale and y indexed from row 0) through
 * the int8 LUT of nv positions (4 stages x 64 entries each; lut8 16-byte
 * aligned), device pointers.  order WASTE_HIP_ORDER_PORTABLE folds the
 * blocks as the portable C kernel does, WASTE_HIP_ORDER_FMA as the AVX-512
 * and NEON kernels do; either is bit-identical to that kernel.  r_lo a
 * multiple of 64.  Ranges of fewer than 64 whole 64-row blocks keep their
 * integer block sums in a device workspace the library allocates on a
 * stream's first such call (and grows when a call needs more): one per
 * stream, kept until the process ends.
 * Replaces: the vq_rows_p6 slot, src/model.c:4076-4114,
 * src/simd_avx512.c:129-236, src/kda_neon.c:100-190. */
#define WASTE_HIP_ORDER_PORTABLE 0
#define WASTE_HIP_ORDER_FMA      1
int waste_hip_vq_rows_p6(const uint8_t *idx, const uint16_t *scale, const int8_t *lut8,
                         const float *lscale, int r_lo, int r_hi, int nv, int order, float *y,
                         void *stream);

/* The fold order the vq_rows_p6 slot uses on this host: the one of the CPU
 * kernel the engine would install (FMA on an AVX-512 VBMI or AArch64 host). */
int waste_hip_vq_p6_order(void);

/* ---- 3. device MoE layer ------------------------------------------------ */

typedef struct waste_hip_moe waste_hip_moe;

typedef struct {
    int hidden;          /* H                                               */
    int n_experts;       /* E                                               */
    int top_k;           /* K                                               */
    int moe_inter;       /* I (routed expert width)                         */
    int n_shared;        /* shared experts fused into one of width I*n (0)  */
    int score_func;      /* WASTE_SCORE_SIGMOID / _SOFTMAX / _SQRTSOFTPLUS  */
    int renorm;          /* moe_renormalize                                 */
    float routed_scale;  /* routed_scaling_factor                           */
    int n_group;         /* group-limited routing: groups (<= 1: off)       */
    int topk_group;      /* groups kept                                     */
    int layer;           /* the layer id records must carry                 */
    int max_tokens;      /* largest T forward() will see                    */
    int verify_records;  /* check each record's crc32 when it is loaded     */
    int prefill_min_tokens; /* T above this runs the grouped matrix-core
                            path (0: 32); T up to it the decode kernels   */
    int index_bits;      /* the container's (0 = 8): 8 VQ3R experts; 6 VQ4P
                            (four stages of 64 entries, twelve books a
                            record), every T on the decode path through
                            the engine's int8 tables (vq_rows_p6)         */
    int p6_order;        /* VQ4P and VQ2R: WASTE_HIP_ORDER_PORTABLE or _FMA,
                            the arithmetic of the engine's table build
                            (and VQ4P's fold) on a host without / with its
                            AVX-512 kernels (waste_hip_vq_p6_order(): this
                            host's)                                       */
    int stages;          /* index_bits 8: 3 (0) VQ3R; 2 VQ2R (two stages of
                            256 entries, six books a record), every T on
                            the decode path in the engine's exact order  */
} waste_hip_moe_cfg;

/* A trunk tensor as the engine holds it (waste_tensor, src/model.h:32-50):
 * fmt WQ_F32 (q = float rows), WQ_Q8G or WQ_Q4G (q = packed rows, qs = f16
 * group scales, one per `group` inputs).  Host pointers; copied. */
typedef struct {
    int fmt, rows, cols, group;
    const void *q;
    const uint16_t *qs;
    size_t rowbytes;
} waste_hip_tensor;

int  waste_hip_moe_create(const waste_hip_moe_cfg *cfg, waste_hip_moe **out);
void waste_hip_moe_destroy(waste_hip_moe *m);

/* Router gate.weight and e_score_correction_bias (bias may be NULL). */
int waste_hip_moe_set_router(waste_hip_moe *m, const waste_hip_tensor *gate,
                             const float *bias);
/* Shared expert gate/up/down; all NULL for none. */
int waste_hip_moe_set_shared(waste_hip_moe *m, const waste_hip_tensor *gate,
                             const waste_hip_tensor *up,
                             const waste_hip_tensor *down);
/* codebooks.bin payloads, fp16 [n_books][entries][8] (256 entries, or 64
 * for a VQ4P layer), converted as the engine's
 * loader does (subnormals flushed; src/model.c:2906-2941). */
int waste_hip_moe_set_codebooks(waste_hip_moe *m, const uint16_t *f16,
                                int n_books);
/* The same for books [first, first + n_books) of a container's table only
 * (a layer's nine, starting at its bank's codebook_base): record codebook
 * ids keep their container-wide meaning and must fall inside the window. */
int waste_hip_moe_set_codebooks_at(waste_hip_moe *m, const uint16_t *f16,
                                   int first, int n_books);
/* One expert record (host memory), checked as record_check does
 * (src/model.c:3645-3692) and copied into the layer's HBM slab. */
int waste_hip_moe_set_expert(waste_hip_moe *m, int expert,
                             const void *record, size_t rec_bytes);
/* The same for a record already in device memory (an expert-cache slot):
 * the header is checked, the bytes are not copied. NULL unbinds. */
int waste_hip_moe_bind_expert(waste_hip_moe *m, int expert,
                              const void *dev_record, size_t rec_bytes);

/* One forward over T tokens of device activations.
 *   x       [T][H], fp32 (x_bf16 = 0) or bf16 (x_bf16 = 1), device
 *   y       [T][H] fp32, device: routed sum + shared expert
 *   ids, w  [T][K] selection (device, may be NULL)
 *   logits  [T][E] router logits (device, may be NULL)
 * T == 1 follows moe_layer (combine in selection order); T > 1 follows
 * moe_chunk (ascending expert order, zero weights skipped).  T above
 * prefill_min_tokens sorts the pairs by expert and runs each expert's
 * tokens as one product on the matrix cores (fp16 operands, fp32
 * accumulation; the router in fp32).  Enqueued on
 * `stream` (a hipStream_t; NULL = the null stream).  Device-side failures
 * (an unbound expert, a routing pass with no candidate) are sticky: read
 * them with waste_hip_moe_status. */
int waste_hip_moe_forward(waste_hip_moe *m, const void *x, int x_bf16, int T,
                          float *y, int32_t *ids, float *w, float *logits,
                          void *stream);

/* forward() for a caller that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference.  The same staged kernels as forward()
 * for T <= prefill_min_tokens, with every per-forward buffer
 * (logits, selection and pair lists, expert partials, the shared expert's
 * activations, the routing exchange) in one static area of 16 MiB per GPU
 * instead of the layer's own; the call itself allocates nothing (the layer
 * and its weights are set up beforehand as usual).  A shape needing more
 * than the area holds (waste_hip_moe_static_bytes: DeepSeek-V3's layer
 * takes about 5.6 MB per token) or more tokens fails with
 * WASTE_HIP_ESCRATCH before anything is enqueued.  Every layer on a GPU
 * shares that GPU's area, which keeps the last call's contents: calls
 * that overlap on one GPU (other streams, other threads) race; calls
 * ordered on one stream do not.  ids/w/logits as in forward(); NULL
 * leaves them in the area, good until the next call on the GPU.  VQ3R
 * layers only (WASTE_HIP_EINVAL for a VQ4P or VQ2R one). */
int waste_hip_moe_forward_static(waste_hip_moe *m, const void *x, int x_bf16, int T,
                                 float *y, int32_t *ids, float *w, float *logits,
                                 void *stream);
/* Bytes of the static area a call of T tokens would use (its head
 * included); more than 16 MiB means WASTE_HIP_ESCRATCH. */
size_t waste_hip_moe_static_bytes(const waste_hip_moe *m, int T);

/* forward() in two halves, for a caller that must see the selection
 * before the experts run (an expert cache: moe_layer's hint and holds sit
 * between its router and its experts, src/model.c:5639-5700).
 *   route:   router logits, the shared expert's gate/up, the selection
 *            (ids/w as in forward; NULL keeps them internal)
 *   experts: the routed experts on the selection of the last route() of
 *            this layer, the shared down projection and the combine.  x and
 *            T must be the route's.  Records are read as bound when the
 *            stream reaches this call. */
int waste_hip_moe_route(waste_hip_moe *m, const void *x, int x_bf16, int T,
                        int32_t *ids, float *w, float *logits, void *stream);
int waste_hip_moe_experts(waste_hip_moe *m, const void *x, int x_bf16, int T,
                          float *y, void *stream);

/* Binds n device records (expert-cache slots) in stream order, with no
 * host wait: the table entries change when the stream reaches the call,
 * after the work enqueued before it.  Each header is checked on the device
 * as record_check does (src/model.c:3645-3692, the checksum aside); a
 * record that fails is left unbound and status() reports
 * WASTE_HIP_ERECORD.  NULL unbinds.  codebook_id: the id the layer's records
 * carry (-1: the one already known from a bound record).  n <= 64, experts
 * distinct, records 16-byte aligned.
 * Replaces: the pointers waste_ecache_hold hands moe_layer,
 * src/model.c:5695-5700. */
int waste_hip_moe_bind_table(waste_hip_moe *m, const int *experts,
                             const void *const *dev_records, int n,
                             int codebook_id, void *stream);

/* The lookahead: this layer's router on the previous layer's input x (one
 * token), scored, bias added, and the n best experts without the group
 * limit, into ids[n] (device).  Bit-exact with predict_next_moe
 * (src/model.c:5419-5449) on the same logits. n <= 64. */
int waste_hip_moe_predict(waste_hip_moe *m, const void *x, int x_bf16, int n,
                          int32_t *ids, void *stream);

/* on = 1: this layer's predict (and so the lookahead forward_cached makes
 * with it as `next`) applies the layer's own group limit, as its routing
 * does: the n best of score + bias within the topk_group groups it keeps
 * (n capped at those groups' experts; ids past the cap untouched).  0 (the
 * default): predict_next_moe's rule above.  No counterpart in the
 * reference: predict_next_moe ignores the group limit, so on a model with
 * n_group > 1 some of its guesses lie in groups the routing then drops,
 * and those reads are wasted.  No effect when n_group <= 1. */
int waste_hip_moe_set_lookahead_groups(waste_hip_moe *m, int on);

/* Forward declaration; the cache is section 4. */
typedef struct waste_hip_ecache waste_hip_ecache;

/* One decode token through an expert cache, moe_layer's order
 * (src/model.c:5639-5700, 5921-5930): route; the lookahead (next's router
 * on this x, `lookahead` ids, 0 = none); the selection to the host (the
 * one host wait); hint and hold each expert (misses fill on the cache's
 * stream, which `stream` then waits for); bind; experts; release; the
 * lookahead's reads for layer + 1.  `layer` is the cache key's layer (the
 * engine's layer index); the layer's codebook id must be known (a bound
 * record, or bind_table with n = 0).  ids, w as in forward. */
int waste_hip_moe_forward_cached(waste_hip_moe *m, waste_hip_ecache *c, int layer,
                                 waste_hip_moe *next, int lookahead, const void *x,
                                 int x_bf16, float *y, int32_t *ids, float *w,
                                 void *stream);

/* Waits for the layer's work and returns the sticky device error (0, or
 * WASTE_HIP_EROUTE / WASTE_HIP_ERECORD / WASTE_HIP_EUNBOUND /
 * WASTE_HIP_ERANGE / WASTE_HIP_ETIMEOUT), clearing it. */
int waste_hip_moe_status(waste_hip_moe *m, void *stream);

/* Bytes the layer reads from HBM for one forward that touches `n_distinct`
 * experts (index + scales, router, shared expert, codebooks, activations)
 * — the algorithmic traffic a roofline divides by. */
size_t waste_hip_moe_bytes(const waste_hip_moe *m, int T, int n_distinct);

/* Per-stage device time of forward(), from HIP events recorded on the
 * forward's stream around each stage while profiling is on (it then waits
 * for each forward to finish).  Stages: 0 router logits + shared expert
 * gate/up, 1 routing, 2 routed gate/up, 3 SwiGLU, 4 routed down, 5 shared
 * down, 6 combine.  Milliseconds summed over `forwards` calls. */
#define WASTE_HIP_STAGES 7
typedef struct {
    int forwards;
    float ms[WASTE_HIP_STAGES];
} waste_hip_moe_prof;
int waste_hip_moe_profile(waste_hip_moe *m, int on);
int waste_hip_moe_profile_read(waste_hip_moe *m, waste_hip_moe_prof *out);

/* Materialises one bound expert matrix (kind 0 gate, 1 up, 2 down) as
 * fp32 [M][N] in device memory W: the format's closed form, bit-exact. */
int waste_hip_moe_dequant(waste_hip_moe *m, int expert, int kind, float *W,
                          void *stream);

/* ---- 4. expert cache in HBM ------------------------------------------- */

/* The engine's expert cache (waste_ecache, src/ecache.h:64-106) with its
 * slots in one device allocation: budget / rec_bytes slots, filled from
 * host records by hipMemcpyAsync on the cache's own stream.  Every decision
 * (which slot, which victim, what counts as a hit) is the engine's: LFRU or
 * LRU over 16 sampled victims, hints that pin their records and keep
 * `depth` reads in flight, speculative lookahead reads counted as bytes
 * only.  Not thread-safe: one host thread drives it, as moe_layer does.
 *
 * Pointers get/hold return are device addresses.  The caller's stream is
 * made to wait for the slot's fill; the caller enqueues its readers and
 * then calls release(stream), after which a refill of the slot waits for
 * them.  A get() pointer is good until the next get/hold (work already
 * enqueued on its stream by then still reads the old record: a refill of
 * the slot waits for it); a hold() pointer until release.  Releases go on
 * one stream.
 *
 * dry = 1: the policy alone, no device (slot pointers are tokens, nothing
 * is copied) — for replaying a routing trace.
 * Replaces: waste_ecache_init/get/hold/release/hint/prefetch/admit/
 * resident_mask/resident_all, src/ecache.h:128-230. */
typedef struct {
    uint64_t hits, misses, evictions;
    uint64_t prefetched;     /* misses the hint's read-ahead issued        */
    uint64_t spec_issued;    /* lookahead reads (not misses)               */
    uint64_t reads, bytes_read;
    /* what became of the lookahead reads (counters only: no decision reads
     * them): demanded while still resident, or evicted first */
    uint64_t spec_used, spec_wasted;
} waste_hip_ecache_counts;

/* policy 0 LFRU, 1 LRU; depth 0 = no read-ahead (the engine's synchronous
 * cache: hint and prefetch do nothing), else reads kept in flight
 * (clamped to a quarter of the slots). */
int  waste_hip_ecache_create(size_t rec_bytes, size_t budget_bytes, int policy,
                             int depth, int dry, waste_hip_ecache **out);
void waste_hip_ecache_destroy(waste_hip_ecache *c);
/* Host copies of every record, records[layer * n_experts + expert]:
 * pinned memory for the copies to be asynchronous. Kept, not copied. */
int  waste_hip_ecache_set_source(waste_hip_ecache *c, const void *const *records,
                                 int n_layers, int n_experts);
int  waste_hip_ecache_hint(waste_hip_ecache *c, int layer, const int *ids, int n);
int  waste_hip_ecache_prefetch(waste_hip_ecache *c, int layer, const int *ids, int n);
const void *waste_hip_ecache_get(waste_hip_ecache *c, int layer, int expert, void *stream);
const void *waste_hip_ecache_hold(waste_hip_ecache *c, int layer, int expert, void *stream);
int  waste_hip_ecache_release(waste_hip_ecache *c, void *stream);
/* 1 when the record went into an empty slot, 0 when nothing was done */
int  waste_hip_ecache_admit(waste_hip_ecache *c, int layer, int expert);
int  waste_hip_ecache_resident_mask(const waste_hip_ecache *c, int layer, int n, uint8_t *out);
int  waste_hip_ecache_resident_all(const waste_hip_ecache *c, int layer, const int *ids, int n);
int  waste_hip_ecache_stats(const waste_hip_ecache *c, waste_hip_ecache_counts *out);
/* the slot holding (layer, expert), or -1 */
int  waste_hip_ecache_slot(const waste_hip_ecache *c, int layer, int expert);
int  waste_hip_ecache_n_slots(const waste_hip_ecache *c);
/* waits for every fill issued so far */
int  waste_hip_ecache_sync(waste_hip_ecache *c);
/* The learned hotlist, usage.waste: save writes a 16-byte header (magic
 * "WUSG", version 1, `tokens`) and one 16-byte entry (layer, expert, hits,
 * last use, 0) per resident record, slot order; 0 or WASTE_HIP_EIO (the
 * file is removed).  warm reads one, sorts it by hits (ties by layer, then
 * expert) and loads the first min(entries, slots) of that order from the
 * source into victims: entries already resident or missing from the
 * source are skipped and still use up their place.
 * Returns how many records it loaded, or WASTE_HIP_EIO / WASTE_HIP_EFORMAT
 * (bad magic).  Counters are untouched, as the engine's are.
 * Replaces: waste_ecache_save_usage, waste_ecache_warm,
 * src/ecache.c:827-913. */
int  waste_hip_ecache_save_usage(const waste_hip_ecache *c, const char *path, uint64_t tokens);
int  waste_hip_ecache_warm(waste_hip_ecache *c, const char *path);

/* ---- 5. container reader ---------------------------------------------- */

/* A WARP container directory (manifest.json, trunk.bin, codebooks.bin,
 * experts-L<n>.bin) opened read-only, with the engine's checks: the
 * manifest's format_version (0), the MoE half of cfg_sane, expert_quant's
 * ranges, every bank's size arithmetic and codebook base, and each record's
 * header (record_check) as it is read, its crc32 too when `verify` is set.
 * Trunk tensors are read on first request, not at open.  Reads of records
 * are positional (pread): several threads may read one container.
 * Replaces: the container half of waste_model_open, src/model.c:2640-2741,
 * 2906-3060; load_trunk, src/model.c:1286-1420; bank_fetch and
 * record_check, src/model.c:3645-3748. */
typedef struct waste_hip_container waste_hip_container;

typedef struct {
    int n_layers, hidden, vocab;
    int n_experts, top_k, moe_inter;
    int n_shared;             /* num_shared_experts as written (0: one of width I) */
    int first_dense;          /* first_k_dense_replace                        */
    int latent_dim;           /* routed_expert_hidden_size (0: none)          */
    int score_func, renorm;
    float routed_scale;
    int n_group, topk_group;  /* the config's group limit (1, 1 when absent)  */
    int stages, vec_dim, entries, index_bits, index_block;
    int n_books, n_tensors;
    char prefix[64];          /* tensor_prefix                                */
} waste_hip_container_cfg;

int  waste_hip_container_open(const char *dir, int verify, waste_hip_container **out);
void waste_hip_container_close(waste_hip_container *c);
int  waste_hip_container_config(const waste_hip_container *c, waste_hip_container_cfg *out);
/* Layer `layer`'s expert bank: 0, or WASTE_HIP_EINVAL when it has none. */
int  waste_hip_container_bank(const waste_hip_container *c, int layer, int *n_experts,
                              int *codebook_base, size_t *rec_bytes);
/* codebooks.bin's payloads, fp16 [n_books][entries][vec_dim], as stored
 * (subnormals are flushed by whoever converts them). */
const uint16_t *waste_hip_container_codebooks(const waste_hip_container *c, int *n_books);
/* One record read into dst (dst_bytes >= the bank's rec_bytes) and
 * checked: 0, WASTE_HIP_EIO (short read), WASTE_HIP_ERECORD (header),
 * WASTE_HIP_ECRC (payload, with verify), WASTE_HIP_EINVAL (no such
 * record).  Replaces: bank_fetch, src/model.c:3712-3748. */
int  waste_hip_container_read_expert(waste_hip_container *c, int layer, int expert,
                                     void *dst, size_t dst_bytes);
/* Every record of the layer, [n_experts][rec_bytes], each checked. */
int  waste_hip_container_read_bank(waste_hip_container *c, int layer, void *dst,
                                   size_t dst_bytes);
/* The first failed read since open: its code (0 when none), layer and
 * expert.  Replaces: waste_error_detail's record report, src/model.c:3700-3710. */
int  waste_hip_container_error(const waste_hip_container *c, int *layer, int *expert);
/* A trunk tensor by name, as waste_hip_tensor (host memory the container
 * owns until close; F32 rows in q, Q8G/Q4G/Q3G rows in q and f16 group
 * scales in qs), with its manifest shape (ndim, shape may be NULL).
 * WASTE_HIP_EFORMAT when the manifest has no such tensor or its extent
 * does not fit trunk.bin. */
int  waste_hip_container_tensor(waste_hip_container *c, const char *name, waste_hip_tensor *out,
                                int *ndim, int shape[4]);

/* A device MoE layer for container layer `layer`: the config's routing
 * (scoring_func, moe_renormalize, routed_scaling_factor), the router
 * <prefix>model.layers.<L>.block_sparse_moe.gate.weight and its
 * e_score_correction_bias (when present), the shared expert
 * (.shared_experts.{gate,up,down}_proj.weight, width moe_inter times
 * num_shared_experts or 1), the layer's codebooks (nine for VQ3R, twelve
 * for VQ4P, six for VQ2R; the last two then follow this host's p6 order).
 * Flags:
 * WASTE_HIP_CT_RECORDS copies every record of the bank into the layer's
 * slab (otherwise records are bound later, e.g. from an expert cache);
 * WASTE_HIP_CT_GROUP_LIMIT routes with the config's n_group/topk_group
 * (the engine's moe_layer has no group limit, so parity with it wants the
 * flag off).  VQ3R, VQ4P and VQ2R containers without a latent
 * projection only (WASTE_HIP_EINVAL otherwise).  Replaces: the tensor lookups of
 * moe_layer, src/model.c:5494-5497, 5932-5936. */
#define WASTE_HIP_CT_RECORDS     1
#define WASTE_HIP_CT_GROUP_LIMIT 2
int  waste_hip_container_moe(waste_hip_container *c, int layer, int max_tokens,
                             int prefill_min_tokens, int flags, waste_hip_moe **out);

/* zlib's crc32 (running value `crc`, 0 to start): the record checksum.
 * Replaces: waste_crc32, src/crc32.h:22. */
uint32_t waste_hip_crc32(uint32_t crc, const void *data, size_t n);

#ifdef __cplusplus
}
#endif
#endif /* WASTE_HIP_H */
