/* SPDX-License-Identifier: Apache-2.0 */
/*
 * waste_abi.h — the byte layouts this library shares with WARP's engine.
 *
 * WARP's kernel-dispatch boundary passes these structs between the engine
 * and a backend, and its container stores the two record headers on disk.
 * A backend built without WARP's headers still has to agree with them to
 * the byte, so they are declared here from the reference's documented
 * layouts and fenced with static asserts on size and field offsets:
 *
 *   waste_kernels       src/waste_backend.h:69-107 (the dispatch table)
 *   mvq_arg             src/simd.h:35-39
 *   lutb_arg            src/simd.h:52-55
 *   vqp_arg             src/simd.h:57-61
 *   waste_vq_job        src/waste_metal.h:31-40
 *   waste_expert_hdr    src/waste_format.h:98-130
 *   waste_codebook_hdr  src/waste_format.h:139-148
 *
 * Only the layouts are shared.  Every function declared against them in
 * this project is its own implementation.
 */
#ifndef WASTE_ABI_H
#define WASTE_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- container constants (src/waste_format.h:31-72) ------------------- */

#define WASTE_ALIGN          4096u
#define WASTE_MAGIC_EXPERT   0x50584557u /* "WEXP" */
#define WASTE_MAGIC_CODEBOOK 0x4b424357u /* "WCBK" */

enum {
    WQ_F32 = 0, WQ_F16 = 1, WQ_Q8G = 2, WQ_Q4G = 3, WQ_VQ3R = 4,
    WQ_VQ2R = 5, WQ_SUB1 = 6, WQ_Q3G = 7, WQ_VQ4P = 8
};

/* Router score functions, src/model.h:179-181. */
enum {
    WASTE_SCORE_SIGMOID = 0,
    WASTE_SCORE_SOFTMAX = 1,
    WASTE_SCORE_SQRTSOFTPLUS = 2
};

/* One expert record's header.  The record is
 *   [48 B header][gate idx][up idx][down idx][f16 scales gate|up|down]
 * padded to a multiple of 4096 bytes. */
typedef struct {
    uint32_t magic;
    uint16_t layer;
    uint16_t expert_id;
    uint8_t  fmt;
    uint8_t  flags;
    uint16_t codebook_id;
    uint16_t lowrank_id;
    uint16_t reserved0;
    uint32_t rec_4k_blocks;
    uint32_t gate_off;
    uint32_t up_off;
    uint32_t down_off;
    uint32_t chan_corr_off;
    uint32_t crc32;
    uint32_t reserved1[2];
} waste_expert_hdr;

typedef struct {
    uint32_t magic;
    uint16_t codebook_id;
    uint8_t  fmt;
    uint8_t  vec_dim;
    uint32_t n_entries;
    uint32_t reserved;
} waste_codebook_hdr;

/* ---- range-kernel argument structs (src/simd.h:35-61) ----------------- */

typedef struct {
    float *y; const int8_t *W; const uint16_t *ws;
    const int8_t *xq; const float *xs; int in, ng, group, bits;
    size_t rowbytes;
} mvq_arg;

typedef struct {
    float *lut; const float *booksT; const float *x;
    int cb_base, stages, entries, vec_dim;
} lutb_arg;

typedef struct {
    float *y; const uint8_t *idx; const uint16_t *scale;
    const int8_t *lut8; const float *lscale;
    int nv;
} vqp_arg;

/* ---- the dispatch table (src/waste_backend.h:69-107) ------------------ */

typedef struct {
    void (*kda_step)(int H, int K, int V,
                     const float *q, const float *k, const float *v,
                     const float *g_log, const float *beta,
                     float *S, float *o, float *scratch);
    void (*short_conv_step)(int C, int KS, const float *w, const float *bias,
                            float *ring, const float *x, float *y);
    void (*rmsnorm_gated)(int C, const float *x, const float *gate,
                          const float *weight, float eps, float *y);
    void (*mvq_rows_f32)(int b, int e, void *arg);
    void (*lutb_range)(int lo, int hi, void *arg);
    void (*vq_rows_p6)(int b, int e, void *arg);
    void (*vq_rows_e)(int b, int e, void *arg);
    int on_device;
    void (*mvq_rows_cpu)(int b, int e, void *arg);
    size_t device_min_bytes;
} waste_kernels;

/* ---- one VQ3R apply, the batch unit (src/waste_metal.h:31-40) --------- */

typedef struct {
    float         *y;
    const uint8_t *rec;
    size_t         rec_bytes;
    uint32_t       idx_off, sc_off;
    const float   *lut;
    size_t         lut_bytes;
    uint32_t       lut_off;
    int            m, nv, stages, entries;
} waste_vq_job;

#ifdef __cplusplus
}
#endif

#if defined(__cplusplus)
#define WASTE_ABI_ASSERT static_assert
#else
#define WASTE_ABI_ASSERT _Static_assert
#endif
WASTE_ABI_ASSERT(sizeof(waste_expert_hdr) == 48, "expert header layout");
WASTE_ABI_ASSERT(offsetof(waste_expert_hdr, gate_off) == 20, "gate_off");
WASTE_ABI_ASSERT(offsetof(waste_expert_hdr, crc32) == 36, "crc32");
WASTE_ABI_ASSERT(sizeof(waste_codebook_hdr) == 16, "codebook header layout");
WASTE_ABI_ASSERT(sizeof(mvq_arg) == 64, "mvq_arg layout");
WASTE_ABI_ASSERT(offsetof(mvq_arg, rowbytes) == 56, "mvq_arg.rowbytes");
WASTE_ABI_ASSERT(sizeof(lutb_arg) == 40, "lutb_arg layout");
WASTE_ABI_ASSERT(sizeof(vqp_arg) == 48, "vqp_arg layout");
WASTE_ABI_ASSERT(offsetof(waste_kernels, mvq_rows_f32) == 24, "slot offset");
WASTE_ABI_ASSERT(offsetof(waste_kernels, on_device) == 56, "on_device");
WASTE_ABI_ASSERT(offsetof(waste_kernels, mvq_rows_cpu) == 64, "mvq_rows_cpu");
WASTE_ABI_ASSERT(sizeof(waste_kernels) == 80, "waste_kernels layout");
WASTE_ABI_ASSERT(sizeof(waste_vq_job) == 72, "waste_vq_job layout");
#undef WASTE_ABI_ASSERT

#endif /* WASTE_ABI_H */
