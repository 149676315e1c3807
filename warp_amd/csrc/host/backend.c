/* SPDX-License-Identifier: Apache-2.0 */
/*
 * backend.c — the engine-facing registration and the VQ3R batch entry.
 *
 * waste_register_hip fills the waste_kernels slots a device backend can
 * take: the trunk matvec mvq_rows_f32, marked on_device so the engine
 * hands it whole row ranges (src/model.c:805-812), with device_min_bytes
 * below which the engine keeps the CPU kernel; and vq_rows_p6, the VQ4P
 * apply through the engine's int8 LUT, bit-identical to the CPU kernel it
 * replaces.  It does not touch lutb_range: a host-in/host-out LUT build
 * would spend more on moving the table than the build costs, so that slot
 * stays on the CPU, as it does under the Metal backend
 * (src/metal.m:503-516).
 *
 * Host weights are immutable trunk tensors, so the slot keeps an HBM copy
 * of each one it has seen, keyed by host address and size; the engine
 * drops them with waste_hip_release_host_buffers before freeing the
 * tensors (the contract of src/waste_backend.h:129-131).  Activations and
 * outputs cross PCIe per call.
 *
 * waste_hip_vq3r copies each job's record and table to HBM, runs every job
 * in the engine's exact row order, and copies the rows back — only when
 * all of it succeeded (all-or-nothing, src/waste_metal.h:42-44).  Records
 * are not cached: an expert-cache slot is reused for other experts under
 * the same address.
 */
#include "waste_hip.h"
#include "../hip/launch.h"

#include <hip/hip_runtime_api.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static pthread_mutex_t g_mu = PTHREAD_MUTEX_INITIALIZER;

#define MIRRORS 256
static struct { const void *key; size_t bytes; void *dev; } g_mirror[MIRRORS];
static int g_ready;              /* 1 registered, -1 declined              */
static hipStream_t g_stream;
static void (*g_cpu_rows)(int b, int e, void *arg);  /* the engine's CPU kernel */
static void *g_io;               /* staging: x in, y out                   */
static size_t g_io_cap;
static void *g_job;              /* staging for the vq3r batch             */
static size_t g_job_cap;
static void (*g_cpu_p6)(int b, int e, void *arg);    /* the engine's VQ4P kernel */
static void *g_p6;               /* staging for the VQ4P slot              */
static size_t g_p6_cap;

/* The device copy of a host tensor keyed by (host, bytes), NULL when there
 * is none.  A key whose copy is too small is dropped. */
static void *mirror_find(const void *key, size_t bytes)
{
    for (int i = 0; i < MIRRORS; i++) {
        if (g_mirror[i].key != key) continue;
        if (g_mirror[i].bytes >= bytes) return g_mirror[i].dev;
        hipFree(g_mirror[i].dev);                     /* grew: replace      */
        g_mirror[i].key = NULL;
        g_mirror[i].dev = NULL;
        g_mirror[i].bytes = 0;
    }
    return NULL;
}

/* A new device copy under `key` of `bytes` bytes read from `src` (a host
 * buffer of at least that size); NULL when the allocation or the copy
 * failed (nothing is then registered). */
static void *mirror_add(const void *key, const void *src, size_t bytes)
{
    int slot = -1;
    for (int i = 0; i < MIRRORS && slot < 0; i++)
        if (!g_mirror[i].key) slot = i;
    if (slot < 0) {                                   /* evict the first    */
        hipFree(g_mirror[0].dev);
        g_mirror[0].key = NULL;
        slot = 0;
    }
    void *d = NULL;
    if (hipMalloc(&d, bytes) != hipSuccess) return NULL;
    if (hipMemcpy(d, src, bytes, hipMemcpyHostToDevice) != hipSuccess) { hipFree(d); return NULL; }
    g_mirror[slot].key = key;
    g_mirror[slot].bytes = bytes;
    g_mirror[slot].dev = d;
    return d;
}

static void *mirror(const void *host, size_t bytes)
{
    void *d = mirror_find(host, bytes);
    return d ? d : mirror_add(host, host, bytes);
}

static void *staging(void **buf, size_t *cap, size_t bytes)
{
    if (*cap >= bytes) return *buf;
    if (*buf) hipFree(*buf);
    *buf = NULL;
    *cap = 0;
    if (hipMalloc(buf, bytes) != hipSuccess) return NULL;
    *cap = bytes;
    return *buf;
}

/* Q3G rows (3-bit codes at bit 3i, minus 4; waste_q3_at, src/simd.h:101-106)
 * are decoded on the host into Q8G-shaped int8 rows once, then mirrored.
 * A Q3G row holds ng*group codes in rowbytes bytes (the packed tensor is
 * rows*rowbytes, src/model.c:1377); only the decoded rows are copied. */
static void *mirror_q3(const mvq_arg *a, int rows, size_t *rowbytes_out)
{
    const size_t rb8 = (size_t)a->ng * a->group;
    const size_t bytes = (size_t)rows * rb8;
    /* keyed one byte past the packed tensor so it cannot alias its mirror */
    const void *key = (const uint8_t *)a->W + 1;
    *rowbytes_out = rb8;
    void *d = mirror_find(key, bytes);
    if (d) return d;
    if ((rb8 * 3 + 7) / 8 > a->rowbytes) return NULL;  /* codes past the row */
    int8_t *tmp = (int8_t *)malloc(bytes);
    if (!tmp) return NULL;
    for (int r = 0; r < rows; r++) {
        const uint8_t *p = (const uint8_t *)a->W + (size_t)r * a->rowbytes;
        for (size_t i = 0; i < rb8; i++) {
            const size_t off = i * 3;
            /* the second byte only when the code straddles it */
            const int hi = (off & 7) > 5 ? p[(off >> 3) + 1] << (8 - (off & 7)) : 0;
            const int v = (p[off >> 3] >> (off & 7)) | hi;
            tmp[(size_t)r * rb8 + i] = (int8_t)((v & 7) - 4);
        }
    }
    d = mirror_add(key, tmp, bytes);
    free(tmp);
    return d;
}

/* The mvq_rows_f32 slot: rows [b, e) of a quantized tensor against fp32
 * activations (mvq_arg, src/simd.h:35-39; xs carries the activations). */
static void mvq_rows_hip(int b, int e, void *p)
{
    mvq_arg *a = (mvq_arg *)p;
    if (e <= b) return;
    pthread_mutex_lock(&g_mu);
    const int rows = e;          /* on_device: the engine passes [0, n)      */
    const size_t sbytes = (size_t)rows * a->ng * 2;
    whip_mat w;
    w.rows = rows; w.cols = a->in; w.group = a->group;
    w.fmt = a->bits == 4 ? WQ_Q4G : WQ_Q8G;
    w.rowbytes = a->rowbytes;
    if (a->bits == 3) w.q = mirror_q3(a, rows, &w.rowbytes);
    else w.q = mirror(a->W, (size_t)rows * a->rowbytes);
    w.qs = (const uint16_t *)mirror(a->ws, sbytes);
    const size_t xb = ((size_t)a->in * 4 + 255) / 256 * 256;
    uint8_t *io = (uint8_t *)staging(&g_io, &g_io_cap, xb + (size_t)rows * 4);
    int ok = w.q && w.qs && io && (w.rowbytes % 16 == 0) && (a->group % 32 == 0);
    if (ok) ok = hipMemcpyAsync(io, a->xs, (size_t)a->in * 4, hipMemcpyHostToDevice, g_stream) == hipSuccess;
    if (ok) ok = whip_gemv(&w, NULL, (const float *)io, 0, 1, (float *)(io + xb), NULL, 0, g_stream) == 0;
    if (ok) ok = hipMemcpyAsync(a->y + b, io + xb + (size_t)b * 4, (size_t)(e - b) * 4,
                                hipMemcpyDeviceToHost, g_stream) == hipSuccess;
    if (ok) ok = hipStreamSynchronize(g_stream) == hipSuccess;
    pthread_mutex_unlock(&g_mu);
    if (!ok) {
        /* The slot has no error channel (src/waste_backend.h:69-107).  A
         * row range the device declined or failed goes to the CPU kernel
         * the table held before this backend registered (mvq_rows_cpu, the
         * one run_rows uses below device_min_bytes, src/model.c:805-812);
         * without one it is NaN, never stale data. */
        if (g_cpu_rows) {
            g_cpu_rows(b, e, p);
            return;
        }
        const float nan = __builtin_nanf("");
        for (int r = b; r < e; r++) a->y[r] = nan;
    }
}

/* The fold order of the CPU VQ4P kernel the engine installs on this host:
 * its AVX-512 VBMI kernel and its NEON kernel are built where the compiler
 * contracts the fold into a fused multiply-add; the portable C kernel is
 * built without FMA.  The engine installs the VBMI kernel only with its
 * AVX-512 backend, which needs AVX512F and AVX512BW with the OS saving the
 * zmm state (src/backend.c:191, the XCR0 test of waste_cpu_features), and
 * then only with VBMI as well (src/simd_avx512.c:239-242); GCC's
 * __builtin_cpu_supports reports the AVX-512 features only when XCR0 shows
 * that state saved. */
int waste_hip_vq_p6_order(void)
{
#if defined(__x86_64__)
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
                   __builtin_cpu_supports("avx512vbmi")
               ? WASTE_HIP_ORDER_FMA
               : WASTE_HIP_ORDER_PORTABLE;
#elif defined(__aarch64__)
    return WASTE_HIP_ORDER_FMA;
#else
    return WASTE_HIP_ORDER_PORTABLE;
#endif
}

/* The vq_rows_p6 slot: rows [b, e) of a VQ4P matrix through the engine's
 * int8 LUT (vqp_arg, src/simd.h:57-61).  The engine calls it from its pool
 * with block-aligned row ranges (src/model.c:4152-4166); each call stages
 * the ranges' 64-row index blocks, their scales and the table, and copies
 * the rows back. */
static void vq_rows_p6_hip(int b, int e, void *p)
{
    vqp_arg *a = (vqp_arg *)p;
    if (e <= b) return;
    const int nv = a->nv;
    const int b0 = b & ~63, nblk64 = (e - b0 + 63) / 64, nsb = (nv + 31) / 32;
    /* the last block may be partial: the engine addresses its rows at the
     * full block stride but holds no bytes past its last row's codes */
    const size_t idx_bytes = ((size_t)nblk64 * nv - 1) * 192 + (size_t)(e - b0 - (nblk64 - 1) * 64) * 3;
    const size_t sc_off = (idx_bytes + 255) / 256 * 256;
    const size_t lut_off = sc_off + ((size_t)(e - b0) * 2 + 255) / 256 * 256;
    const size_t ls_off = lut_off + ((size_t)nv * 256 + 255) / 256 * 256;
    const size_t y_off = ls_off + ((size_t)nsb * 4 + 255) / 256 * 256;
    const size_t total = y_off + (size_t)(e - b0) * 4;
    pthread_mutex_lock(&g_mu);
    uint8_t *d = (uint8_t *)staging(&g_p6, &g_p6_cap, total);
    int ok = d != NULL;
    if (ok) ok = hipMemcpyAsync(d, a->idx + (size_t)(b0 / 64) * nv * 192, idx_bytes, hipMemcpyHostToDevice,
                                g_stream) == hipSuccess;
    if (ok) ok = hipMemcpyAsync(d + sc_off, a->scale + b0, (size_t)(e - b0) * 2, hipMemcpyHostToDevice,
                                g_stream) == hipSuccess;
    if (ok) ok = hipMemcpyAsync(d + lut_off, a->lut8, (size_t)nv * 256, hipMemcpyHostToDevice, g_stream) == hipSuccess;
    if (ok) ok = hipMemcpyAsync(d + ls_off, a->lscale, (size_t)nsb * 4, hipMemcpyHostToDevice, g_stream) == hipSuccess;
    if (ok) ok = whip_vq_rows_p6(d, (const uint16_t *)(d + sc_off), (const int8_t *)(d + lut_off),
                                 (const float *)(d + ls_off), 0, e - b0, nv, waste_hip_vq_p6_order(),
                                 (float *)(d + y_off), g_stream) == 0;
    if (ok) ok = hipMemcpyAsync(a->y + b, d + y_off + (size_t)(b - b0) * 4, (size_t)(e - b) * 4,
                                hipMemcpyDeviceToHost, g_stream) == hipSuccess;
    if (ok) ok = hipStreamSynchronize(g_stream) == hipSuccess;
    pthread_mutex_unlock(&g_mu);
    if (!ok) {
        if (g_cpu_p6) {
            g_cpu_p6(b, e, p);
            return;
        }
        const float nan = __builtin_nanf("");
        for (int r = b; r < e; r++) a->y[r] = nan;
    }
}

int waste_hip_vq_quant_lut(const float *lut, int nv, int stages, int entries, int8_t *q, float *scale,
                           void *stream)
{
    if (!lut || !q || !scale || nv <= 0 || stages <= 0 || entries <= 0) return WASTE_HIP_EINVAL;
    return whip_vq_quant_lut(lut, nv, stages, entries, q, scale, (hipStream_t)stream) ? WASTE_HIP_EDEVICE : 0;
}

int waste_hip_vq_rows_p6(const uint8_t *idx, const uint16_t *scale, const int8_t *lut8, const float *lscale,
                         int r_lo, int r_hi, int nv, int order, float *y, void *stream)
{
    if (!idx || !scale || !lut8 || !lscale || !y || r_lo < 0 || r_lo % 64 || r_hi <= r_lo || nv <= 0 ||
        (uintptr_t)lut8 % 16 || (order != WASTE_HIP_ORDER_PORTABLE && order != WASTE_HIP_ORDER_FMA))
        return WASTE_HIP_EINVAL;
    return whip_vq_rows_p6(idx, scale, lut8, lscale, r_lo, r_hi, nv, order, y, (hipStream_t)stream)
               ? WASTE_HIP_EDEVICE : 0;
}

const char *waste_register_hip(waste_kernels *t)
{
    pthread_mutex_lock(&g_mu);
    if (!g_ready) {
        if (!waste_hip_device_name() || hipStreamCreate(&g_stream) != hipSuccess) g_ready = -1;
        else g_ready = 1;
    }
    const int ok = g_ready > 0;
    pthread_mutex_unlock(&g_mu);
    if (!ok) return NULL;
    /* the engine snapshots its best CPU kernel before accelerators register
     * (src/backend.c:198-202); without the snapshot the slot itself still
     * holds it */
    if (t->mvq_rows_f32 != mvq_rows_hip)
        g_cpu_rows = t->mvq_rows_cpu ? t->mvq_rows_cpu : t->mvq_rows_f32;
    t->mvq_rows_f32 = mvq_rows_hip;
    /* The VQ4P slot only when asked for (WASTE_HIP_P6=1): the engine calls
     * it once per pool range (pf_wide, src/model.c:4157-4159), and each call
     * is a synchronous round trip over PCIe.  Measured on an MI355X host
     * against the engine's own VBMI kernel on one thread: a Kimi-Linear
     * gate/up matrix (1024 x 288 positions) in one call 86-106 us against
     * 44 us, in the pool's 1024-row ranges 196 us (down, 2304 x 128) against
     * 44 us; a DeepSeek-V3 matrix breaks even only when handed whole.  The
     * device-resident layer is where VQ4P belongs on the GPU. */
    const char *p6 = getenv("WASTE_HIP_P6");
    if (p6 && *p6 == '1') {
        if (t->vq_rows_p6 != vq_rows_p6_hip) g_cpu_p6 = t->vq_rows_p6;
        t->vq_rows_p6 = vq_rows_p6_hip;
    } else if (t->vq_rows_p6 == vq_rows_p6_hip) {
        t->vq_rows_p6 = g_cpu_p6;                    /* a registration before this one installed it */
    }
    t->on_device = 1;
    /* A synchronous dispatch with two PCIe copies costs tens of us; below
     * a megabyte of weights the CPU pool finishes first. */
    const char *env = getenv("WASTE_HIP_MIN_KB");
    t->device_min_bytes = (size_t)(env ? atoi(env) : 1024) << 10;
    return "HIP (gfx950)";
}

void waste_hip_release_host_buffers(void)
{
    pthread_mutex_lock(&g_mu);
    for (int i = 0; i < MIRRORS; i++) {
        if (g_mirror[i].key) hipFree(g_mirror[i].dev);
        g_mirror[i].key = NULL;
        g_mirror[i].dev = NULL;
        g_mirror[i].bytes = 0;
    }
    pthread_mutex_unlock(&g_mu);
}

int waste_hip_vq3r(const waste_vq_job *jobs, int n)
{
    if (n <= 0 || !jobs) return -1;
    for (int i = 0; i < n; i++)
        if (jobs[i].stages != 3 || jobs[i].entries != 256 || jobs[i].m <= 0 || jobs[i].nv <= 0 ||
            (size_t)jobs[i].idx_off + (size_t)((jobs[i].m + 63) / 64) * 64 * jobs[i].nv * 3 >= jobs[i].rec_bytes ||
            (size_t)jobs[i].sc_off + (size_t)jobs[i].m * 2 > jobs[i].rec_bytes ||
            ((size_t)jobs[i].lut_off + (size_t)jobs[i].nv * 768) * 4 > jobs[i].lut_bytes)
            return -1;
    pthread_mutex_lock(&g_mu);
    if (g_ready == 0) {
        if (!waste_hip_device_name() || hipStreamCreate(&g_stream) != hipSuccess) g_ready = -1;
        else g_ready = 1;
    }
    if (g_ready < 0) { pthread_mutex_unlock(&g_mu); return -1; }
    /* stage every distinct record and table once */
    size_t total = 0, ytotal = 0;
    size_t *roff = (size_t *)malloc(sizeof(size_t) * 2 * (size_t)n);
    whip_vq_job *dj = (whip_vq_job *)malloc(sizeof(whip_vq_job) * (size_t)n);
    int ok = roff && dj;
    for (int i = 0; ok && i < n; i++) {
        int seen = -1;
        for (int k = 0; k < i; k++) if (jobs[k].rec == jobs[i].rec) { seen = k; break; }
        if (seen >= 0) roff[2 * i] = roff[2 * seen];
        else { roff[2 * i] = total; total += (jobs[i].rec_bytes + 255) / 256 * 256; }
        seen = -1;
        for (int k = 0; k < i; k++) if (jobs[k].lut == jobs[i].lut) { seen = k; break; }
        if (seen >= 0) roff[2 * i + 1] = roff[2 * seen + 1];
        else { roff[2 * i + 1] = total; total += (jobs[i].lut_bytes + 255) / 256 * 256; }
        ytotal += (size_t)jobs[i].m;
    }
    uint8_t *d = ok ? (uint8_t *)staging(&g_job, &g_job_cap, total + ytotal * 4) : NULL;
    ok = d != NULL;
    for (int i = 0; ok && i < n; i++) {
        int first_rec = 1, first_lut = 1;
        for (int k = 0; k < i; k++) {
            if (jobs[k].rec == jobs[i].rec) first_rec = 0;
            if (jobs[k].lut == jobs[i].lut) first_lut = 0;
        }
        if (first_rec)
            ok = hipMemcpyAsync(d + roff[2 * i], jobs[i].rec, jobs[i].rec_bytes,
                                hipMemcpyHostToDevice, g_stream) == hipSuccess;
        if (ok && first_lut)
            ok = hipMemcpyAsync(d + roff[2 * i + 1], jobs[i].lut, jobs[i].lut_bytes,
                                hipMemcpyHostToDevice, g_stream) == hipSuccess;
    }
    size_t yoff = total;
    for (int i = 0; ok && i < n; i++) {
        dj[i].y = (float *)(d + yoff);
        dj[i].idx = d + roff[2 * i] + jobs[i].idx_off;
        dj[i].scale = (const uint16_t *)(d + roff[2 * i] + jobs[i].sc_off);
        dj[i].lut = (const float *)(d + roff[2 * i + 1]) + jobs[i].lut_off;
        dj[i].m = jobs[i].m;
        dj[i].nv = jobs[i].nv;
        yoff += (size_t)jobs[i].m * 4;
    }
    if (ok) ok = whip_vq3r_jobs(dj, n, g_stream) == 0;
    float *ybuf = ok ? (float *)malloc(ytotal * 4) : NULL;
    if (ok) ok = ybuf && hipMemcpyAsync(ybuf, d + total, ytotal * 4, hipMemcpyDeviceToHost, g_stream) == hipSuccess;
    if (ok) ok = hipStreamSynchronize(g_stream) == hipSuccess;
    if (ok) {
        const float *src = ybuf;
        for (int i = 0; i < n; i++) {
            memcpy(jobs[i].y, src, (size_t)jobs[i].m * 4);
            src += jobs[i].m;
        }
    }
    free(ybuf); free(roff); free(dj);
    pthread_mutex_unlock(&g_mu);
    return ok ? 0 : -1;
}
