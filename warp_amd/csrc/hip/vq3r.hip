// SPDX-License-Identifier: Apache-2.0
//
// vq3r.hip — VQ3R (3-stage residual VQ, 256 entries, 8-dim vectors) expert
// kernels for gfx950.
//
// The decode path never materialises a weight.  For a matrix stored as
// three codebook indices per (row, 8-wide position v), row r's product
// with x is sum_v L[v][0][i0] + L[v][1][i1] + L[v][2][i2] where
// L[v][s][c] = C_s[c] . x[8v..8v+8) depends on the position and code only,
// not on the row (the engine's LUT formulation, src/model.c:3796-3806).
//
// Layout in HBM (the container's, unchanged): one record per expert,
// indices blocked [row/64][v][row%64][stage] (docs/FORMAT.md:216-223), so a
// 64-row block at one position is 192 contiguous bytes.  A wavefront owns a
// row block: lane r reads its 3 index bytes for position v with one 4-byte
// load (gfx950 global loads take any byte address), the 64 lanes together
// covering the block's 192 bytes, which the memory system coalesces.
//
// A workgroup owns a chunk of VC positions for one (pair, kind) and all of
// that matrix's rows (or a 1/rsplit share).  It builds the chunk's table
// in LDS — VC*3*256 fp32 — once, then streams the rows through it: the
// table costs 6144 FMAs per position, amortised over every row.  Row sums
// leave as per-chunk partials; the next kernel reduces them.  The split is
// what lets a decode token's eight experts fill 256 CUs.
#include "common.h"
#include "launch.h"

#define VC 16                       // positions per workgroup chunk
#define LUT_PER_V (3 * 256)

extern "C" int whip_vq_chunks(int nv) { return (nv + VC - 1) / VC; }

__device__ __forceinline__ void load_block(const uint8_t *pp, int vcount, uint32_t *wv)
{
#pragma unroll
    for (int v = 0; v < VC; v++) wv[v] = v < vcount ? ld_u32_unaligned(pp + v * 192) : 0u;
}

__device__ __forceinline__ float apply_block(const float *lut, int vcount, const uint32_t *wv)
{
    float acc = 0.0f;
#pragma unroll
    for (int v = 0; v < VC; v++) {
        if (v >= vcount) break;
        const float *L = lut + v * LUT_PER_V;
        const uint32_t w = wv[v];
        const float t = (L[w & 255] + L[256 + ((w >> 8) & 255)]) + L[512 + ((w >> 16) & 255)];
        acc += t;
    }
    return acc;
}

__device__ __forceinline__ void
vq_apply_body(const uint8_t *const *__restrict__ recs, const int32_t *__restrict__ pair_exp,
              const int32_t *__restrict__ pair_src, const void *__restrict__ src, int src_ld,
              int src_bf16, const float *__restrict__ booksT, int cb, uint32_t off0,
              uint32_t off1, int kinds, int M, int nv, int nch, int rsplit,
              float *__restrict__ part, int *__restrict__ err)
{
    __shared__ float lut[VC * LUT_PER_V];
    __shared__ float xs[VC * 8];
    const int c = blockIdx.x, kind = blockIdx.y / rsplit, rs = blockIdx.y % rsplit;
    const int p = blockIdx.z, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
    const int v0 = c * VC, vcount = min(VC, nv - v0);
    const int nb = (M + 63) >> 6;
    const int rb_lo = rs * nb / rsplit, rb_hi = (rs + 1) * nb / rsplit;
    float *out = part + (((size_t)p * kinds + kind) * nch + c) * (size_t)M;

    const uint8_t *rec = recs[pair_exp[p]];
    if (rec == nullptr) {                       // unbound expert: zeros + flag
        if (tid == 0) atomicOr(err, 1);
        for (int r = rb_lo * 64 + tid; r < min(rb_hi * 64, M); r += blockDim.x) out[r] = 0.0f;
        return;
    }
    // The wavefront's row blocks are rb_lo + wave + nw*k.  Up to four of
    // them are in flight at once, the first four issued before the table
    // is built, so the index stream is moving while the LUT is computed.
    const uint8_t *idx = rec + (kind ? off1 : off0) + (size_t)v0 * 192 + lane * 3;
    uint32_t cur[2][VC], nxt[2][VC];
    const int rb0 = rb_lo + wave;
#pragma unroll
    for (int q = 0; q < 2; q++) {
        const int rb = rb0 + q * nw;
        if (rb < rb_hi) load_block(idx + (size_t)rb * nv * 192, vcount, cur[q]);
        const int rn = rb0 + (q + 2) * nw;
        if (rn < rb_hi) load_block(idx + (size_t)rn * nv * 192, vcount, nxt[q]);
    }

    const int srow = pair_src ? pair_src[p] : p;
    if (tid < vcount * 8) {
        const size_t o = (size_t)srow * src_ld + (size_t)v0 * 8 + tid;
        xs[tid] = src_bf16 ? wh_bf16(((const uint16_t *)src)[o]) : ((const float *)src)[o];
    }
    __syncthreads();

    // L[v][s][c] = fma chain over d from 0 (the engine's AVX-512 order).
    // A thread owns one (stage, code): its 8 codebook values stay in
    // registers while it sweeps the chunk's positions.
    const float *bT = booksT + (size_t)(cb + kind * 3) * 8 * 256;
    for (int q = tid; q < LUT_PER_V; q += blockDim.x) {
        const float *cr = bT + (size_t)(q >> 8) * 8 * 256 + (q & 255);
        float cv[8];
#pragma unroll
        for (int d = 0; d < 8; d++) cv[d] = cr[d * 256];
        for (int v = 0; v < vcount; v++) {
            const float *xx = xs + v * 8;
            float a = 0.0f;
#pragma unroll
            for (int d = 0; d < 8; d++) a = __fmaf_rn(xx[d], cv[d], a);
            lut[v * LUT_PER_V + q] = a;
        }
    }
    __syncthreads();

    for (int k = 0; rb0 + k * nw < rb_hi; k += 2) {
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const int rb = rb0 + (k + q) * nw;
            if (rb >= rb_hi) break;
            const float acc = apply_block(lut, vcount, cur[q]);
            const int r = rb * 64 + lane;
            if (r < M) out[r] = acc;
        }
#pragma unroll
        for (int q = 0; q < 2; q++) {
#pragma unroll
            for (int v = 0; v < VC; v++) cur[q][v] = nxt[q][v];
            const int rn = rb0 + (k + 4 + q) * nw;
            if (rn < rb_hi) load_block(idx + (size_t)rn * nv * 192, vcount, nxt[q]);
        }
    }
}

// Two symbols for one body, so that profiles tell the gate/up pass (two
// kinds per pair, the hidden-wide tables) from the down pass.
#define VQ_THREADS 512
#define VQ_KERNEL(NAME)                                                                         \
    __global__ void __launch_bounds__(VQ_THREADS)                                               \
    NAME(const uint8_t *const *__restrict__ recs, const int32_t *__restrict__ pair_exp,         \
         const int32_t *__restrict__ pair_src, const void *__restrict__ src, int src_ld,        \
         int src_bf16, const float *__restrict__ booksT, int cb, uint32_t off0, uint32_t off1,  \
         int kinds, int M, int nv, int nch, int rsplit, float *__restrict__ part,               \
         int *__restrict__ err)                                                                 \
    {                                                                                           \
        vq_apply_body(recs, pair_exp, pair_src, src, src_ld, src_bf16, booksT, cb, off0, off1,  \
                      kinds, M, nv, nch, rsplit, part, err);                                    \
    }
VQ_KERNEL(k_vq_gate_up)
VQ_KERNEL(k_vq_down)

extern "C" int whip_vq_apply(const whip_vq_args *a, hipStream_t s)
{
    const int nch = whip_vq_chunks(a->nv);
    dim3 grid(nch, a->kinds * a->rsplit, a->P);
    hipLaunchKernelGGL(a->kinds == 2 ? k_vq_gate_up : k_vq_down, grid, dim3(VQ_THREADS), 0, s, a->recs,
                       a->pair_exp, a->pair_src, a->src, a->src_ld, a->src_bf16, a->booksT, a->cb,
                       a->idx_off[0], a->idx_off[1], a->kinds, a->M, a->nv, nch, a->rsplit,
                       a->part, a->err);
    return (int)hipGetLastError();
}

// ---- SwiGLU over the reduced gate/up partials ------------------------------
// A workgroup owns 128 rows of one pair: 32 float4 row groups x 8 slices of
// the chunk range, so every thread has its whole slice's loads in flight;
// the slices are then added in chunk order.
#define ACT_ROWS 128
#define ACT_SLICES 8

__global__ void __launch_bounds__(256)
k_vq_act(const uint8_t *const *__restrict__ recs, const int32_t *__restrict__ pair_exp,
         const float *__restrict__ part, int nch, int I, uint32_t sc_off, float *__restrict__ h)
{
    __shared__ float4 red[2][ACT_SLICES][ACT_ROWS / 4];
    const int p = blockIdx.y, tid = threadIdx.x;
    const int g = tid & 31, sl = tid >> 5;
    const int r0 = blockIdx.x * ACT_ROWS + g * 4;
    const int per = (nch + ACT_SLICES - 1) / ACT_SLICES;
    const int c0 = sl * per, c1 = min(nch, c0 + per);
    float4 sg = make_float4(0, 0, 0, 0), su = sg;
    if (r0 < I) {
        const float *gp = part + ((size_t)p * 2 + 0) * nch * (size_t)I + r0;
        const float *up = part + ((size_t)p * 2 + 1) * nch * (size_t)I + r0;
        float4 vg[8], vu[8];
        for (int cb = c0; cb < c1; cb += 8) {
#pragma unroll
            for (int k = 0; k < 8; k++)
                if (cb + k < c1) {
                    vg[k] = *(const float4 *)(gp + (size_t)(cb + k) * I);
                    vu[k] = *(const float4 *)(up + (size_t)(cb + k) * I);
                }
#pragma unroll
            for (int k = 0; k < 8; k++)
                if (cb + k < c1) {
                    sg.x += vg[k].x; sg.y += vg[k].y; sg.z += vg[k].z; sg.w += vg[k].w;
                    su.x += vu[k].x; su.y += vu[k].y; su.z += vu[k].z; su.w += vu[k].w;
                }
        }
    }
    red[0][sl][g] = sg;
    red[1][sl][g] = su;
    __syncthreads();
    if (tid >= 32 || r0 >= I) return;
    float gg[4] = {0, 0, 0, 0}, uu[4] = {0, 0, 0, 0};
    for (int k = 0; k < ACT_SLICES; k++) {
        const float4 a = red[0][k][g], b = red[1][k][g];
        gg[0] += a.x; gg[1] += a.y; gg[2] += a.z; gg[3] += a.w;
        uu[0] += b.x; uu[1] += b.y; uu[2] += b.z; uu[3] += b.w;
    }
    const uint8_t *rec = recs[pair_exp[p]];
    float out[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        float sgc = 0.0f, suc = 0.0f;
        if (rec) {
            const uint16_t *sc = (const uint16_t *)(rec + sc_off);
            sgc = wh_f16_scale(sc[r0 + q]);
            suc = wh_f16_scale(sc[I + r0 + q]);
        }
        out[q] = wh_silu_mul(__fmul_rn(gg[q], sgc), __fmul_rn(uu[q], suc));
    }
    *(float4 *)(h + (size_t)p * I + r0) = make_float4(out[0], out[1], out[2], out[3]);
}

extern "C" int whip_vq_act(const uint8_t *const *recs, const int32_t *pair_exp, int P,
                           const float *part, int nch, int I, uint32_t sc_off, float *h,
                           hipStream_t s)
{
    if (I % 4) return (int)hipErrorInvalidValue;
    dim3 grid((I + ACT_ROWS - 1) / ACT_ROWS, P);
    hipLaunchKernelGGL(k_vq_act, grid, dim3(256), 0, s, recs, pair_exp, part, nch, I, sc_off, h);
    return (int)hipGetLastError();
}

// ---- weighted combine + shared expert --------------------------------------
// A workgroup owns 128 output rows of one token: thread (row group, pair
// slot j) reduces pair j's chunk partials for 4 rows (all loads in flight)
// and scales them; the pairs are then added in the token's combine order.
#define CMB_ROWS 128

__global__ void __launch_bounds__(256)
k_combine(const uint8_t *const *__restrict__ recs, const int32_t *__restrict__ pair_exp,
          const float *__restrict__ pair_w, const int32_t *__restrict__ tok_pairs, int K,
          const float *__restrict__ part_d, int nch, int H, uint32_t sc_off_down,
          int skip_zero, const float *__restrict__ sh, float *__restrict__ y)
{
    extern __shared__ float4 cred[];                 // [K][32]
    const int t = blockIdx.y, tid = threadIdx.x;
    const int g = tid & 31;
    const int r0 = blockIdx.x * CMB_ROWS + g * 4;
    for (int j = tid >> 5; j < K; j += 8) {
        float4 acc = make_float4(0, 0, 0, 0);
        const int p = tok_pairs[t * K + j];
        const float wj = pair_w[p];
        if (r0 < H && !(skip_zero && wj == 0.0f)) {
            const uint8_t *rec = recs[pair_exp[p]];
            const float *pd = part_d + (size_t)p * nch * H + r0;
            float4 s = make_float4(0, 0, 0, 0);
            for (int cb = 0; cb < nch; cb += 8) {
                float4 v[8];
#pragma unroll
                for (int k = 0; k < 8; k++)
                    if (cb + k < nch) v[k] = *(const float4 *)(pd + (size_t)(cb + k) * H);
#pragma unroll
                for (int k = 0; k < 8; k++)
                    if (cb + k < nch) { s.x += v[k].x; s.y += v[k].y; s.z += v[k].z; s.w += v[k].w; }
            }
            if (rec) {
                const uint16_t *sc = (const uint16_t *)(rec + sc_off_down) + r0;
                acc.x = __fmul_rn(wj, __fmul_rn(s.x, wh_f16_scale(sc[0])));
                acc.y = __fmul_rn(wj, __fmul_rn(s.y, wh_f16_scale(sc[1])));
                acc.z = __fmul_rn(wj, __fmul_rn(s.z, wh_f16_scale(sc[2])));
                acc.w = __fmul_rn(wj, __fmul_rn(s.w, wh_f16_scale(sc[3])));
            }
        }
        cred[j * 32 + g] = acc;
    }
    __syncthreads();
    if (tid >= 32 || r0 >= H) return;
    float o[4] = {0, 0, 0, 0};
    for (int j = 0; j < K; j++) {                    // combine order
        const float4 a = cred[j * 32 + g];
        o[0] = __fadd_rn(o[0], a.x); o[1] = __fadd_rn(o[1], a.y);
        o[2] = __fadd_rn(o[2], a.z); o[3] = __fadd_rn(o[3], a.w);
    }
    float4 r;
    const float *shr = sh ? sh + (size_t)t * H + r0 : nullptr;
    r.x = __fadd_rn(o[0], shr ? shr[0] : 0.0f);
    r.y = __fadd_rn(o[1], shr ? shr[1] : 0.0f);
    r.z = __fadd_rn(o[2], shr ? shr[2] : 0.0f);
    r.w = __fadd_rn(o[3], shr ? shr[3] : 0.0f);
    *(float4 *)(y + (size_t)t * H + r0) = r;
}

extern "C" int whip_combine(const uint8_t *const *recs, const int32_t *pair_exp,
                            const float *pair_w, const int32_t *tok_pairs, int T, int K,
                            const float *part_d, int nch, int H, uint32_t sc_off_down,
                            int skip_zero, const float *sh, float *y, hipStream_t s)
{
    if (H % 4) return (int)hipErrorInvalidValue;
    dim3 grid((H + CMB_ROWS - 1) / CMB_ROWS, T);
    hipLaunchKernelGGL(k_combine, grid, dim3(256), (size_t)K * 32 * sizeof(float4), s, recs,
                       pair_exp, pair_w, tok_pairs, K, part_d, nch, H, sc_off_down, skip_zero, sh, y);
    return (int)hipGetLastError();
}

// ---- materialised dequantisation (closed form, bit-exact) ------------------
// W[r][8v+d] = (((0 + C0[i0][d]) + C1[i1][d]) + C2[i2][d]) * f16(scale[r]),
// docs/FORMAT.md:204-214; books are fp32 [book][entry][dim] as loaded.
__global__ void __launch_bounds__(256)
k_dequant(const uint8_t *__restrict__ idx, const uint16_t *__restrict__ scale,
          const float *__restrict__ books, int cb, int M, int N, float *__restrict__ W)
{
    const int nv = N / 8;
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= (size_t)M * nv) return;
    const int r = (int)(q / nv), v = (int)(q % nv);
    const uint8_t *ix = idx + ((size_t)(r >> 6) * nv + v) * 192 + (r & 63) * 3;
    const float sc = wh_f16_scale(scale[r]);
    const float *c0 = books + ((size_t)(cb + 0) * 256 + ix[0]) * 8;
    const float *c1 = books + ((size_t)(cb + 1) * 256 + ix[1]) * 8;
    const float *c2 = books + ((size_t)(cb + 2) * 256 + ix[2]) * 8;
    float *o = W + (size_t)r * N + (size_t)v * 8;
#pragma unroll
    for (int d = 0; d < 8; d++) {
        float a = __fadd_rn(0.0f, c0[d]);
        a = __fadd_rn(a, c1[d]);
        a = __fadd_rn(a, c2[d]);
        o[d] = __fmul_rn(a, sc);
    }
}

extern "C" int whip_dequant(const uint8_t *idx, const uint16_t *scale, const float *books,
                            int cb, int M, int N, float *W, hipStream_t s)
{
    const size_t n = (size_t)M * (N / 8);
    hipLaunchKernelGGL(k_dequant, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, idx, scale,
                       books, cb, M, N, W);
    return (int)hipGetLastError();
}

// ---- LUT build (the lutb_range slot on the device) -------------------------
__global__ void __launch_bounds__(256)
k_lutb(const float *__restrict__ booksT, const float *__restrict__ x, int cb, int st, int en,
       int vd, int nv, float *__restrict__ lut)
{
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= (size_t)nv * st * en) return;
    const int c = (int)(q % en), s = (int)((q / en) % st), v = (int)(q / ((size_t)en * st));
    const float *CT = booksT + (size_t)(cb + s) * en * vd;
    float a = 0.0f;
    for (int d = 0; d < vd; d++) a = __fmaf_rn(x[(size_t)v * vd + d], CT[(size_t)d * en + c], a);
    lut[q] = a;
}

extern "C" int whip_lutb(const float *booksT, const float *x, int cb, int stages, int entries,
                         int vec_dim, int nv, float *lut, hipStream_t s)
{
    const size_t n = (size_t)nv * stages * entries;
    hipLaunchKernelGGL(k_lutb, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, booksT, x, cb,
                       stages, entries, vec_dim, nv, lut);
    return (int)hipGetLastError();
}

// ---- exact-order apply, one job per grid row -------------------------------
// Each row's sum is the engine's vq_rows order: acc = 0; for v ascending
// acc += (L0 + L1) + L2; y = acc * f16(scale) (src/model.c:3909-3977).
// Tables are read from HBM/L2, one lane per row.
#define MAX_JOBS_PER_LAUNCH 32
struct job_pack { whip_vq_job j[MAX_JOBS_PER_LAUNCH]; };

__global__ void __launch_bounds__(64)
k_vq3r_jobs(job_pack pk)
{
    const whip_vq_job jb = pk.j[blockIdx.y];
    const int rb = blockIdx.x, lane = threadIdx.x, r = rb * 64 + lane;
    if (rb * 64 >= jb.m) return;
    const uint8_t *pp = jb.idx + (size_t)rb * jb.nv * 192 + lane * 3;
    float acc = 0.0f;
    for (int v = 0; v < jb.nv; v++) {
        const uint32_t w = ld_u32_unaligned(pp + (size_t)v * 192);
        const float *L = jb.lut + (size_t)v * LUT_PER_V;
        const float t = __fadd_rn(__fadd_rn(L[w & 255], L[256 + ((w >> 8) & 255)]),
                                  L[512 + ((w >> 16) & 255)]);
        acc = __fadd_rn(acc, t);
    }
    if (r < jb.m) jb.y[r] = __fmul_rn(acc, wh_f16_scale(jb.scale[r]));
}

extern "C" int whip_vq3r_jobs(const whip_vq_job *jobs, int n, hipStream_t s)
{
    for (int j0 = 0; j0 < n; j0 += MAX_JOBS_PER_LAUNCH) {
        const int nj = n - j0 < MAX_JOBS_PER_LAUNCH ? n - j0 : MAX_JOBS_PER_LAUNCH;
        job_pack pk;
        int maxm = 0;
        for (int j = 0; j < nj; j++) {
            pk.j[j] = jobs[j0 + j];
            if (pk.j[j].m > maxm) maxm = pk.j[j].m;
        }
        hipLaunchKernelGGL(k_vq3r_jobs, dim3((maxm + 63) / 64, nj), dim3(64), 0, s, pk);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return (int)e;
    }
    return 0;
}
