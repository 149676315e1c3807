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

__device__ __forceinline__ void
vq_apply_body(const uint8_t *const *__restrict__ recs, const int32_t *__restrict__ pair_exp,
              const int32_t *__restrict__ pair_src, const float *__restrict__ src, int src_ld,
              const float *__restrict__ booksT, int cb, uint32_t off0, uint32_t off1,
              int kinds, int M, int nv, int nch, int rsplit, float *__restrict__ part,
              int *__restrict__ err)
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
    const int srow = pair_src ? pair_src[p] : p;
    const float *xv = src + (size_t)srow * src_ld + (size_t)v0 * 8;
    if (tid < vcount * 8) xs[tid] = xv[tid];
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

    const uint8_t *idx = rec + (kind ? off1 : off0);
    for (int rb = rb_lo + wave; rb < rb_hi; rb += nw) {
        const uint8_t *pp = idx + ((size_t)rb * nv + v0) * 192 + lane * 3;
        float acc = 0.0f;
        if (vcount == VC) {
            uint32_t wv[VC];
#pragma unroll
            for (int v = 0; v < VC; v++) wv[v] = ld_u32_unaligned(pp + v * 192);
#pragma unroll
            for (int v = 0; v < VC; v++) {
                const float *L = lut + v * LUT_PER_V;
                const uint32_t w = wv[v];
                const float t = (L[w & 255] + L[256 + ((w >> 8) & 255)]) + L[512 + ((w >> 16) & 255)];
                acc += t;
            }
        } else {
            for (int v = 0; v < vcount; v++) {
                const float *L = lut + v * LUT_PER_V;
                const uint32_t w = ld_u32_unaligned(pp + v * 192);
                const float t = (L[w & 255] + L[256 + ((w >> 8) & 255)]) + L[512 + ((w >> 16) & 255)];
                acc += t;
            }
        }
        const int r = rb * 64 + lane;
        if (r < M) out[r] = acc;
    }
}

// Two symbols for one body, so that profiles tell the gate/up pass (two
// kinds per pair, the hidden-wide tables) from the down pass.
#define VQ_KERNEL(NAME)                                                                         \
    __global__ void __launch_bounds__(256)                                                      \
    NAME(const uint8_t *const *__restrict__ recs, const int32_t *__restrict__ pair_exp,         \
         const int32_t *__restrict__ pair_src, const float *__restrict__ src, int src_ld,       \
         const float *__restrict__ booksT, int cb, uint32_t off0, uint32_t off1, int kinds,     \
         int M, int nv, int nch, int rsplit, float *__restrict__ part, int *__restrict__ err)   \
    {                                                                                           \
        vq_apply_body(recs, pair_exp, pair_src, src, src_ld, booksT, cb, off0, off1, kinds, M,  \
                      nv, nch, rsplit, part, err);                                              \
    }
VQ_KERNEL(k_vq_gate_up)
VQ_KERNEL(k_vq_down)

extern "C" int whip_vq_apply(const whip_vq_args *a, hipStream_t s)
{
    const int nch = whip_vq_chunks(a->nv);
    dim3 grid(nch, a->kinds * a->rsplit, a->P);
    hipLaunchKernelGGL(a->kinds == 2 ? k_vq_gate_up : k_vq_down, grid, dim3(256), 0, s, a->recs,
                       a->pair_exp, a->pair_src, a->src, a->src_ld, a->booksT, a->cb,
                       a->idx_off[0], a->idx_off[1], a->kinds, a->M, a->nv, nch, a->rsplit,
                       a->part, a->err);
    return (int)hipGetLastError();
}

// ---- SwiGLU over the reduced gate/up partials ------------------------------
__global__ void __launch_bounds__(256)
k_vq_act(const uint8_t *const *__restrict__ recs, const int32_t *__restrict__ pair_exp, int P,
         const float *__restrict__ part, int nch, int I, uint32_t sc_off, float *__restrict__ h,
         const float *__restrict__ sh_a, const float *__restrict__ sh_b, int SI,
         float *__restrict__ h_sh)
{
    const int p = blockIdx.y;
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (p < P) {
        if (r >= I) return;
        const uint8_t *rec = recs[pair_exp[p]];
        const float *gp = part + ((size_t)p * 2 + 0) * nch * (size_t)I + r;
        const float *up = part + ((size_t)p * 2 + 1) * nch * (size_t)I + r;
        float g = 0.0f, u = 0.0f;
        for (int c = 0; c < nch; c++) { g += gp[(size_t)c * I]; u += up[(size_t)c * I]; }
        float sg = 0.0f, su = 0.0f;
        if (rec) {
            const uint16_t *sc = (const uint16_t *)(rec + sc_off);
            sg = wh_f16_scale(sc[r]);
            su = wh_f16_scale(sc[I + r]);
        }
        h[(size_t)p * I + r] = wh_silu_mul(__fmul_rn(g, sg), __fmul_rn(u, su));
    } else {
        const int t = p - P;
        if (r >= SI) return;
        const size_t o = (size_t)t * SI + r;
        h_sh[o] = wh_silu_mul(sh_a[o], sh_b[o]);
    }
}

extern "C" int whip_vq_act(const uint8_t *const *recs, const int32_t *pair_exp, int P,
                           const float *part, int nch, int I, uint32_t sc_off, float *h,
                           const float *sh_a, const float *sh_b, int T, int SI,
                           float *h_sh, hipStream_t s)
{
    const int rows = I > SI ? I : SI;
    dim3 grid((rows + 255) / 256, P + (h_sh ? T : 0));
    hipLaunchKernelGGL(k_vq_act, grid, dim3(256), 0, s, recs, pair_exp, P, part, nch, I, sc_off,
                       h, sh_a, sh_b, SI, h_sh);
    return (int)hipGetLastError();
}

// ---- weighted combine + shared expert --------------------------------------
__global__ void __launch_bounds__(256)
k_combine(const uint8_t *const *__restrict__ recs, const int32_t *__restrict__ pair_exp,
          const float *__restrict__ pair_w, const int32_t *__restrict__ tok_pairs, int K,
          const float *__restrict__ part_d, int nch, int H, uint32_t sc_off_down,
          int skip_zero, const float *__restrict__ sh, float *__restrict__ y)
{
    const int t = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= H) return;
    float acc = 0.0f;
    for (int j = 0; j < K; j++) {
        const int p = tok_pairs[t * K + j];
        const float wj = pair_w[p];
        if (skip_zero && wj == 0.0f) continue;
        const uint8_t *rec = recs[pair_exp[p]];
        const float *pd = part_d + (size_t)p * nch * H + i;
        float s = 0.0f;
        for (int c = 0; c < nch; c++) s += pd[(size_t)c * H];
        const float sc = rec ? wh_f16_scale(((const uint16_t *)(rec + sc_off_down))[i]) : 0.0f;
        acc = __fadd_rn(acc, __fmul_rn(wj, __fmul_rn(s, sc)));
    }
    y[(size_t)t * H + i] = __fadd_rn(acc, sh ? sh[(size_t)t * H + i] : 0.0f);
}

extern "C" int whip_combine(const uint8_t *const *recs, const int32_t *pair_exp,
                            const float *pair_w, const int32_t *tok_pairs, int T, int K,
                            const float *part_d, int nch, int H, uint32_t sc_off_down,
                            int skip_zero, const float *sh, float *y, hipStream_t s)
{
    dim3 grid((H + 255) / 256, T);
    hipLaunchKernelGGL(k_combine, grid, dim3(256), 0, s, recs, pair_exp, pair_w, tok_pairs, K,
                       part_d, nch, H, sc_off_down, skip_zero, sh, y);
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
