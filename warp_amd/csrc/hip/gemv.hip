// SPDX-License-Identifier: Apache-2.0
//
// gemv.hip — trunk matrix-vector products for the MoE layer: the router
// logits and the shared expert (F32, Q8G int8 + f16 group scale, Q4G two
// signed nibbles per byte, low first, minus 8; tools/convert.py:893-924).
//
// One launch runs up to three independent products ("jobs"), each over its
// own range of workgroups, so the router and the shared expert's gate/up
// leave in one dispatch.  A job may pair two matrices of one shape (gate
// and up): the wavefronts that own row r of both then write
// silu(gate.x) * (up.x) directly, so the shared expert needs no separate
// activation pass.
//
// A row is split across wpr wavefronts; each lane streams 16-byte chunks
// (coalesced 128-bit loads), UNROLL of them in flight at once, and keeps a
// partial per token; a chunk never straddles a quantisation group, so the
// group scale multiplies the chunk's partial once.  Activations may be
// fp32 or bf16 (converted as they are read).
#include "common.h"
#include "launch.h"
#include "route.h"

static thread_local hipEvent_t t_start = nullptr, t_stop = nullptr;

extern "C" void whip_time_next(hipEvent_t start, hipEvent_t stop)
{
    t_start = start;
    t_stop = stop;
}

bool whip_take_timing(hipEvent_t *start, hipEvent_t *stop)
{
    if (!t_start) return false;
    *start = t_start;
    *stop = t_stop;
    t_start = t_stop = nullptr;
    return true;
}

#define TB 4          // tokens sharing one pass over the weights
#define UNROLL 4      // 16-byte chunks in flight per lane

#include "gemv_dev.h"
#include "trace.h"

// n activations starting at element e of token row xr (fp32 or bf16)
template <int N>
__device__ __forceinline__ void load_x(const void *xr, int bf16, int e, float *x)
{
    if (bf16) {
        const uint16_t *p = (const uint16_t *)xr + e;
#pragma unroll
        for (int i = 0; i < N; i += 4) {
            const uint2 v = *(const uint2 *)(p + i);
            x[i] = wh_bf16(v.x & 0xffff); x[i + 1] = wh_bf16(v.x >> 16);
            x[i + 2] = wh_bf16(v.y & 0xffff); x[i + 3] = wh_bf16(v.y >> 16);
        }
    } else {
        const float *p = (const float *)xr + e;
#pragma unroll
        for (int i = 0; i < N; i += 4) {
            const float4 v = *(const float4 *)(p + i);
            x[i] = v.x; x[i + 1] = v.y; x[i + 2] = v.z; x[i + 3] = v.w;
        }
    }
}

struct gemv_job {
    const uint8_t *W0, *W1;
    const uint16_t *S0, *S1;
    size_t rowbytes;
    int fmt, rows, cols, group;
    const void *x;
    int x_ld, x_bf16;
    float *y;
    int y_ld;
    int wpr, blk0, nblk;
    int rpw;                   // rows per wavefront (one-token kernel)
    int coh;                   // y read by other workgroups of the launch: device-coherent stores
    uint64_t *xchg;            // also (epoch << 32 | bits) of y[r] at xchg[r], device-coherent
    uint32_t epoch;
};
struct gemv_pack {
    gemv_job j[3];
    int n, T;
};

// partial dot products of one wavefront's share of row r, for TBT tokens;
// a chunk is decoded eight weights at a time to keep registers low
template <int FMT, int TBT>
__device__ __forceinline__ void row_partial(const gemv_job &J, const uint8_t *W, const uint16_t *S,
                                            int r, int part, int lane, int t0, int tn, float *acc)
{
    constexpr int NE = chunk_of<FMT>::NE;
    const int ng = FMT == 0 ? 1 : (J.cols + J.group - 1) / J.group;
    const int padded = FMT == 0 ? J.cols : ng * J.group;
    const int nchunk = (padded + NE - 1) / NE;
    const uint8_t *row = W + (size_t)r * J.rowbytes;
    const uint16_t *sr = FMT == 0 ? nullptr : S + (size_t)r * ng;
    const int stride = 64 * J.wpr;
    const size_t xstride = (size_t)J.x_ld * (J.x_bf16 ? 2 : 4);
    for (int k0 = part * 64 + lane; k0 < nchunk; k0 += stride * UNROLL) {
        uint4 raw[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; u++) {
            const int k = k0 + u * stride;
            raw[u] = k < nchunk ? *(const uint4 *)(row + (size_t)k * 16) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < UNROLL; u++) {
            const int k = k0 + u * stride;
            if (k >= nchunk) break;
            const int e0 = k * NE;
            const float sc = FMT == 0 ? 1.0f : wh_f16_scale(sr[e0 / J.group]);
            const uint32_t uw[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
            float part_t[TBT];
#pragma unroll
            for (int t = 0; t < TBT; t++) part_t[t] = 0.0f;
#pragma unroll
            for (int sub = 0; sub < (NE + 7) / 8; sub++) {
                constexpr int SN = NE < 8 ? NE : 8;
                float w[SN];
                if (FMT == 0) {
#pragma unroll
                    for (int i = 0; i < SN; i++) w[i] = __uint_as_float(uw[i]);
                } else if (FMT == 2) {
#pragma unroll
                    for (int i = 0; i < SN; i++) {
                        const int q = sub * 8 + i;
                        w[i] = (float)(int8_t)((uw[q >> 2] >> ((q & 3) * 8)) & 0xff);
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < SN; i += 2) {
                        const int q = (sub * 8 + i) >> 1;
                        const uint32_t b = (uw[q >> 2] >> ((q & 3) * 8)) & 0xff;
                        w[i] = (float)((int)(b & 15) - 8);
                        w[i + 1] = (float)((int)(b >> 4) - 8);
                    }
                }
                const int es = e0 + sub * 8;
#pragma unroll
                for (int t = 0; t < TBT; t++) {
                    if (t >= tn) break;
                    const uint8_t *xr = (const uint8_t *)J.x + (size_t)(t0 + t) * xstride;
                    if (es + SN <= J.cols) {
                        float xv[SN];
                        load_x<SN>(xr, J.x_bf16, es, xv);
#pragma unroll
                        for (int i = 0; i < SN; i++) part_t[t] = __fmaf_rn(w[i], xv[i], part_t[t]);
                    } else {
                        for (int i = 0; i < SN && es + i < J.cols; i++) {
                            const float xi = J.x_bf16 ? wh_bf16(((const uint16_t *)xr)[es + i])
                                                      : ((const float *)xr)[es + i];
                            part_t[t] = __fmaf_rn(w[i], xi, part_t[t]);
                        }
                    }
                }
            }
#pragma unroll
            for (int t = 0; t < TBT; t++) acc[t] = __fmaf_rn(sc, part_t[t], acc[t]);
        }
    }
}

template <int FMT, int TBT>
__device__ __forceinline__ void run_job(const gemv_job &J, int T, int blk, float (*red)[2][TB])
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rows_per_blk = 4 / J.wpr;
    const int r = blk * rows_per_blk + wave / J.wpr, part = wave % J.wpr;
    const bool live = r < J.rows;
    for (int t0 = 0; t0 < T; t0 += TBT) {
        const int tn = min(TBT, T - t0);
        float a0[TBT], a1[TBT];
#pragma unroll
        for (int t = 0; t < TBT; t++) { a0[t] = 0.0f; a1[t] = 0.0f; }
        if (live) {
            row_partial<FMT, TBT>(J, J.W0, J.S0, r, part, lane, t0, tn, a0);
            if (J.W1) row_partial<FMT, TBT>(J, J.W1, J.S1, r, part, lane, t0, tn, a1);
        }
#pragma unroll
        for (int t = 0; t < TBT; t++) {
            a0[t] = wave_sum(a0[t]);
            a1[t] = wave_sum(a1[t]);
        }
        if (J.wpr > 1) {
            __syncthreads();
            if (lane == 0)
#pragma unroll
                for (int t = 0; t < TBT; t++) { red[wave][0][t] = a0[t]; red[wave][1][t] = a1[t]; }
            __syncthreads();
            if (part == 0 && lane == 0)
#pragma unroll
                for (int t = 0; t < TBT; t++) {
                    float s0 = red[wave][0][t], s1 = red[wave][1][t];
                    for (int q = 1; q < J.wpr; q++) { s0 += red[wave + q][0][t]; s1 += red[wave + q][1][t]; }
                    a0[t] = s0; a1[t] = s1;
                }
        }
        if (live && part == 0 && lane == 0)
#pragma unroll
            for (int t = 0; t < TBT; t++)
                if (t < tn)
                    J.y[(size_t)(t0 + t) * J.y_ld + r] = J.W1 ? wh_silu_mul(a0[t], a1[t]) : a0[t];
    }
}

template <int TBT>
__global__ void __launch_bounds__(256) k_gemv_multi(gemv_pack pk)
{
    __shared__ float red[4][2][TB];
    const int b = blockIdx.x;
    // the job is copied field by field from the argument block: a reference
    // into it, or a whole-struct select, would put the block in scratch
    const int ji = (pk.n > 2 && b >= pk.j[2].blk0) ? 2 : (pk.n > 1 && b >= pk.j[1].blk0) ? 1 : 0;
#define SEL(f) (ji == 2 ? pk.j[2].f : ji == 1 ? pk.j[1].f : pk.j[0].f)
    gemv_job J;
    J.W0 = SEL(W0); J.W1 = SEL(W1); J.S0 = SEL(S0); J.S1 = SEL(S1); J.rowbytes = SEL(rowbytes);
    J.fmt = SEL(fmt); J.rows = SEL(rows); J.cols = SEL(cols); J.group = SEL(group);
    J.x = SEL(x); J.x_ld = SEL(x_ld); J.x_bf16 = SEL(x_bf16); J.y = SEL(y); J.y_ld = SEL(y_ld);
    J.wpr = SEL(wpr); J.blk0 = SEL(blk0); J.nblk = SEL(nblk);
#undef SEL
    const int blk = b - J.blk0;
    if (J.fmt == 0) run_job<0, TBT>(J, pk.T, blk, red);
    else if (J.fmt == 2) run_job<2, TBT>(J, pk.T, blk, red);
    else run_job<3, TBT>(J, pk.T, blk, red);
}

template <int FMT, int RPW, bool XBF>
__device__ __forceinline__ void run_job1(const gemv_job &J, int blk, float (*red)[4][2])
{
    constexpr int NE = chunk_of<FMT>::NE, NW = xw_of<FMT, XBF>::N;
    constexpr int U = u_of<FMT, XBF>::U / RPW > 0 ? u_of<FMT, XBF>::U / RPW : 1;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wpr = J.wpr, groups = 4 / wpr;
    const int rg = blk * groups + wave / wpr, part = wave % wpr;
    const int r0 = rg * RPW;
    const int ng = FMT == 0 ? 1 : (J.cols + J.group - 1) / J.group;
    const int nchunk = (FMT == 0 ? J.cols : ng * J.group) / NE;
    const int stride = 64 * wpr;
    const bool pair = J.W1 != nullptr;

    float a0[RPW], a1[RPW];
#pragma unroll
    for (int i = 0; i < RPW; i++) { a0[i] = 0.0f; a1[i] = 0.0f; }
    for (int k0 = part * 64 + lane; k0 - lane < nchunk; k0 += stride * U) {   // wave-uniform test
        uint4 w0[RPW][U], w1[RPW][U], xw[U][NW];
        uint16_t s0[RPW][U], s1[RPW][U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int k = k0 + u * stride, kc = k < nchunk ? k : 0;
            load_xs<FMT, XBF>(J.x, J.cols, kc, xw[u]);
#pragma unroll
            for (int i = 0; i < RPW; i++) {
                const int rc = r0 + i < J.rows ? r0 + i : 0;
                const size_t o = (size_t)rc * J.rowbytes + (size_t)kc * 16;
                w0[i][u] = *(const uint4 *)(J.W0 + o);
                if (FMT != 0) s0[i][u] = J.S0[(size_t)rc * ng + (size_t)kc * NE / J.group];
            }
        }
        if (pair) {                                    // uniform
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int k = k0 + u * stride, kc = k < nchunk ? k : 0;
#pragma unroll
                for (int i = 0; i < RPW; i++) {
                    const int rc = r0 + i < J.rows ? r0 + i : 0;
                    const size_t o = (size_t)rc * J.rowbytes + (size_t)kc * 16;
                    w1[i][u] = *(const uint4 *)(J.W1 + o);
                    if (FMT != 0) s1[i][u] = J.S1[(size_t)rc * ng + (size_t)kc * NE / J.group];
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int k = k0 + u * stride;
            if (k >= nchunk) continue;                 // rows past the end are never written
            mask_xs<FMT, XBF>(J.cols, k, xw[u]);
            if (FMT == 3 && XBF) {
                const float sx = chunk_sum136_bf(xw[u]);
#pragma unroll
                for (int i = 0; i < RPW; i++) {
                    a0[i] = __fmaf_rn(wh_f16_scale(s0[i][u]), chunk_dot_q4bf(w0[i][u], xw[u], sx), a0[i]);
                    if (pair)
                        a1[i] = __fmaf_rn(wh_f16_scale(s1[i][u]), chunk_dot_q4bf(w1[i][u], xw[u], sx), a1[i]);
                }
                continue;
            }
#pragma unroll
            for (int i = 0; i < RPW; i++) {
                const float d0 = chunk_dot<FMT, XBF>(w0[i][u], xw[u]);
                a0[i] = FMT == 0 ? a0[i] + d0 : __fmaf_rn(wh_f16_scale(s0[i][u]), d0, a0[i]);
                if (pair) {
                    const float d1 = chunk_dot<FMT, XBF>(w1[i][u], xw[u]);
                    a1[i] = FMT == 0 ? a1[i] + d1 : __fmaf_rn(wh_f16_scale(s1[i][u]), d1, a1[i]);
                }
            }
        }
    }

#pragma unroll
    for (int i = 0; i < RPW; i++) {
        a0[i] = wave_sum(a0[i]);
        if (pair) a1[i] = wave_sum(a1[i]);
    }
    if (wpr > 1) {
        if (lane == 0)
#pragma unroll
            for (int i = 0; i < RPW; i++) { red[wave][i][0] = a0[i]; red[wave][i][1] = a1[i]; }
        __syncthreads();
        if (part == 0 && lane == 0)
#pragma unroll
            for (int i = 0; i < RPW; i++) {
                float t0 = red[wave][i][0], t1 = red[wave][i][1];
                for (int q = 1; q < wpr; q++) { t0 += red[wave + q][i][0]; t1 += red[wave + q][i][1]; }
                a0[i] = t0; a1[i] = t1;
            }
    }
    if (part == 0 && lane == 0)
#pragma unroll
        for (int i = 0; i < RPW; i++)
            if (r0 + i < J.rows) {
                const float v = pair ? wh_silu_mul(a0[i], a1[i]) : a0[i];
                if (J.coh) __hip_atomic_store(J.y + r0 + i, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                else J.y[r0 + i] = v;
                if (J.xchg)
                    __hip_atomic_store(J.xchg + r0 + i, ((uint64_t)J.epoch << 32) | __float_as_uint(v),
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
}

template <int FMT, bool XBF>
__device__ __forceinline__ void run_fmt1(const gemv_job &J, int blk, float (*red)[4][2])
{
    if (J.rpw == 4) run_job1<FMT, 4, XBF>(J, blk, red);
    else run_job1<FMT, 1, XBF>(J, blk, red);
}

// block b of a batch-1 launch; every job of one launch reads x of one type
template <bool XBF>
__device__ __forceinline__ void gemv1_block(const gemv_pack &pk, int b, float (*red)[4][2], uint32_t epoch = 0)
{
    const int ji = (pk.n > 2 && b >= pk.j[2].blk0) ? 2 : (pk.n > 1 && b >= pk.j[1].blk0) ? 1 : 0;
#define SEL(f) (ji == 2 ? pk.j[2].f : ji == 1 ? pk.j[1].f : pk.j[0].f)
    gemv_job J;
    J.W0 = SEL(W0); J.W1 = SEL(W1); J.S0 = SEL(S0); J.S1 = SEL(S1); J.rowbytes = SEL(rowbytes);
    J.fmt = SEL(fmt); J.rows = SEL(rows); J.cols = SEL(cols); J.group = SEL(group);
    J.x = SEL(x); J.x_ld = SEL(x_ld); J.x_bf16 = SEL(x_bf16); J.y = SEL(y); J.y_ld = SEL(y_ld);
    J.wpr = SEL(wpr); J.blk0 = SEL(blk0); J.nblk = SEL(nblk); J.rpw = SEL(rpw); J.coh = SEL(coh);
    J.xchg = SEL(xchg); J.epoch = epoch;
#undef SEL
    const int blk = b - J.blk0;
    if (J.fmt == 0) run_fmt1<0, XBF>(J, blk, red);
    else if (J.fmt == 2) run_fmt1<2, XBF>(J, blk, red);
    else run_fmt1<3, XBF>(J, blk, red);
}

template <bool XBF>
__global__ void __launch_bounds__(256) k_gemv1(gemv_pack pk)
{
    __shared__ float red[4][4][2];
    gemv1_block<XBF>(pk, blockIdx.x, red);
}

// One token's routing in block 0 (all four wavefronts compute the same
// selection, see route.h) beside a batch-1 product that needs no routing
// (the shared expert's down projection) in the other blocks: the one
// wavefront of routing hides behind the product instead of running alone.
template <int NPL, bool XBF>
__global__ void __launch_bounds__(256)
k_route_gemv1(whip_route_cfg c, const float *__restrict__ logits, const float *__restrict__ bias,
              int32_t *__restrict__ ids, float *__restrict__ wout, int32_t *__restrict__ pair_tok,
              int32_t *__restrict__ pair_exp, float *__restrict__ pair_w, int32_t *__restrict__ tok_pairs,
              const uint8_t *const *__restrict__ recs, const uint8_t **__restrict__ pair_rec,
              int *__restrict__ err, gemv_pack pk)
{
    __shared__ float red[4][4][2];
    __shared__ float rl[ROUTE_LDS_FLOATS(NPL)];
    if (blockIdx.x == 0) {
        route_body<NPL>(c, logits, bias, 1, 0, threadIdx.x & 63, ids, wout, pair_tok, pair_exp, pair_w,
                        tok_pairs, recs, pair_rec, err, rl);
        return;
    }
    gemv1_block<XBF>(pk, blockIdx.x - 1, red);
}

// The batch-1 launch with the router as job 0: when the last of the
// router's blocks has written its logits, that block routes the token
// (route.h, the pair list and the pairs' records for the expert kernels)
// while the other jobs' blocks (the shared expert's gate/up) still run.
// Every router block loads what the routing reads besides the logits (the
// bias, the record table, the exp table) beside its product's loads and
// keeps it in LDS, so the block that turns out last routes with no other
// memory round trip than the logits'.  cnt: a device counter, zero between
// launches (the routing block resets it).
template <bool XBF, int NPL>
__global__ void __launch_bounds__(256)
k_gemv1_route(gemv_pack pk, whip_route_cfg c, const float *__restrict__ bias, int32_t *__restrict__ ids,
              float *__restrict__ wout, int32_t *__restrict__ pair_tok, int32_t *__restrict__ pair_exp,
              float *__restrict__ pair_w, int32_t *__restrict__ tok_pairs,
              const uint8_t *const *__restrict__ recs, const uint8_t **__restrict__ pair_rec,
              int *__restrict__ err, int *__restrict__ cnt)
{
    constexpr int PER = (64 * NPL + 255) / 256;       // table entries per thread
    __shared__ float red[4][4][2];
    __shared__ float rl[ROUTE_LDS_FLOATS(NPL)];
    __shared__ float s_bias[64 * NPL];
    __shared__ const uint8_t *s_recs[64 * NPL];
    __shared__ uint64_t s_etab[32];
    __shared__ int s_last;
    WT_SPAN(0, 0);
    WT_DECL;
    WT_KEEP(0);
    const int nrb = pk.j[0].nblk;                     // the router's blocks come first
    const bool router = (int)blockIdx.x < nrb;        // uniform
    const int tid = threadIdx.x, E = c.E;
    float bv[PER];
    const uint8_t *rv[PER];
    uint64_t ev = 0;
    if (router) {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int e = tid + 256 * i, ec = e < E ? e : 0;
            bv[i] = bias ? bias[ec] : 0.0f;
            rv[i] = recs[ec];
        }
        ev = wh_exp_tab[tid & 31];
    }
    gemv1_block<XBF>(pk, blockIdx.x, red);
    WT_SPAN(0, 1);
    WT_KEEP(1);
    if (!router) return;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int e = tid + 256 * i;
        if (e < E) { s_bias[e] = bv[i]; s_recs[e] = rv[i]; }
    }
    if (tid < 32) s_etab[tid] = ev;
    // the logits went out device-coherent (through the per-XCD caches);
    // once they are acknowledged the block counts itself, and the last one
    // reads them all device-coherent: no cache flush or invalidate
    __builtin_amdgcn_s_waitcnt(0x0F70);               // vmcnt(0): this thread's stores completed
    __syncthreads();
    WT_KEEP(2);
    if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nrb - 1;
    __syncthreads();
    WT_KEEP(3);
    if (!s_last) return;
    route_body<NPL, true>(c, pk.j[0].y, bias ? s_bias : nullptr, 1, 0, threadIdx.x & 63, ids, wout, pair_tok,
                          pair_exp, pair_w, tok_pairs, s_recs, pair_rec, err, rl, s_etab);
    if (threadIdx.x == 0) *cnt = 0;
    WT_KEEP(4);
    if (threadIdx.x == 0)                             // the routing block's stages
        for (int i = 0; i < 5; i++) WT_PUTAT(0, 1, i);
    WT(0, 2);                                         // the routing block's end
}

// ---- one token, x staged in LDS --------------------------------------------
// The batch-1 launch that carries the router.  A block first copies x (the
// one activation row every job of the launch reads) into LDS: those loads
// go out before the block's weight loads, so they come back first.  Each
// lane then has all its weight chunks in flight at once (GX_U per matrix,
// a row split over wpr wavefronts so that they cover it) and reads x from
// LDS beside them.  Keeping x once per block instead of per lane leaves the
// launch about 80 VGPRs, so all of its blocks are resident from the start
// and the whole launch's traffic is requested at once.
//
// LDS layout of x: chunk k's slice (NE elements) at 16-byte word k*(NW+1)
// when a slice is NW >= 2 words (a spare word after each slice spreads
// consecutive lanes' 128-bit reads over all banks), else packed.
template <int FMT, bool PAIR> struct gx_u { static constexpr int U = FMT == 0 && !PAIR ? 8 : 4; };

template <int FMT, bool XBF> struct gx_lay {
    static constexpr int NW = xw_of<FMT, XBF>::N;     // 16-byte words per chunk slice
    static constexpr bool PAD = NW >= 2 && chunk_of<FMT>::NE * (XBF ? 2 : 4) >= 32;
    __device__ static int word(int i) { return PAD ? i + i / NW : i; }   // x word i -> LDS word
};

template <int NXL>
__device__ __forceinline__ void gx_x_issue(const void *x, int xbytes, uint4 (&xr)[NXL])
{
#pragma unroll
    for (int i = 0; i < NXL; i++) {
        const int o = (threadIdx.x + 256 * i) * 16;
        xr[i] = *(const uint4 *)((const uint8_t *)x + (o < xbytes ? o : 0));
    }
}

template <int FMT, bool XBF, int NXL, bool PAIR>
__device__ __forceinline__ void gx_rows(const gemv_job &J, int blk, const uint4 (&xr)[NXL], int xbytes,
                                        int xl_bytes, uint4 *xs, float (*red)[2], uint32_t epoch)
{
    constexpr int NE = chunk_of<FMT>::NE, NW = gx_lay<FMT, XBF>::NW, U = gx_u<FMT, PAIR>::U;
    constexpr bool pair = PAIR;
    constexpr int XS = gx_lay<FMT, XBF>::PAD ? NW + 1 : NW;      // LDS words per slice
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wpr = J.wpr, part = wave % wpr;
    const int r = blk * (4 / wpr) + wave / wpr;
    const int rc = r < J.rows ? r : J.rows - 1;
    const int ng = FMT == 0 ? 1 : (J.cols + J.group - 1) / J.group;
    const int nchunk = (FMT == 0 ? J.cols : ng * J.group) / NE;
    const int stride = 64 * wpr;
    const uint8_t *row0 = J.W0 + (size_t)rc * J.rowbytes;
    const uint8_t *row1 = pair ? J.W1 + (size_t)rc * J.rowbytes : row0;
    const uint16_t *sr0 = FMT == 0 ? nullptr : J.S0 + (size_t)rc * ng;
    const uint16_t *sr1 = FMT == 0 ? nullptr : (pair ? J.S1 : J.S0) + (size_t)rc * ng;
    uint4 w0[U], w1[PAIR ? U : 1];
    uint16_t s0[U], s1[PAIR ? U : 1];
    auto issue = [&](int k0) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int k = k0 + u * stride, kc = k < nchunk ? k : 0;
            w0[u] = *(const uint4 *)(row0 + (size_t)kc * 16);
            if (FMT != 0) s0[u] = sr0[(size_t)kc * NE / J.group];
        }
        if (PAIR)
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int k = k0 + u * stride, kc = k < nchunk ? k : 0;
                w1[PAIR ? u : 0] = *(const uint4 *)(row1 + (size_t)kc * 16);
                if (FMT != 0) s1[PAIR ? u : 0] = sr1[(size_t)kc * NE / J.group];
            }
    };
    int k0 = part * 64 + lane;
    issue(k0);
    // x to LDS (its loads were issued before the weights'), zero past the
    // last column up to the whole groups the rows are padded to
#pragma unroll
    for (int i = 0; i < NXL; i++) {
        const int w = threadIdx.x + 256 * i;
        if (w * 16 < xl_bytes) xs[gx_lay<FMT, XBF>::word(w)] = w * 16 < xbytes ? xr[i] : make_uint4(0, 0, 0, 0);
    }
    __syncthreads();
    WT_L(8);
    float a0 = 0.0f, a1 = 0.0f;
    for (;;) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int k = k0 + u * stride;
            if (k >= nchunk) continue;
            // x slices are read as they are needed, not hoisted for all chunks
            __builtin_amdgcn_sched_barrier(0);
            uint4 xw[NW > 0 ? NW : 1];
            if (NE * (XBF ? 2 : 4) < 16) {             // F32 rows, bf16 x: 8 bytes
                const uint2 v = *((const uint2 *)xs + k);
                xw[0] = make_uint4(v.x, v.y, 0, 0);
            } else {
#pragma unroll
                for (int j = 0; j < NW; j++) xw[j] = xs[k * XS + j];
            }
            if (FMT == 3 && XBF) {
                const float sx = chunk_sum136_bf(xw);
                a0 = __fmaf_rn(wh_f16_scale(s0[u]), chunk_dot_q4bf(w0[u], xw, sx), a0);
                if (PAIR) a1 = __fmaf_rn(wh_f16_scale(s1[PAIR ? u : 0]), chunk_dot_q4bf(w1[PAIR ? u : 0], xw, sx), a1);
                continue;
            }
            const float d0 = chunk_dot<FMT, XBF>(w0[u], xw);
            a0 = FMT == 0 ? a0 + d0 : __fmaf_rn(wh_f16_scale(s0[u]), d0, a0);
            if (PAIR) {
                const float d1 = chunk_dot<FMT, XBF>(w1[PAIR ? u : 0], xw);
                a1 = FMT == 0 ? a1 + d1 : __fmaf_rn(wh_f16_scale(s1[PAIR ? u : 0]), d1, a1);
            }
        }
        k0 += stride * U;
        if (k0 - lane >= nchunk) break;                // uniform
        issue(k0);
    }
    a0 = wave_sum(a0);
    if (pair) a1 = wave_sum(a1);
    if (wpr > 1) {                                     // uniform
        if (lane == 0) { red[wave][0] = a0; red[wave][1] = a1; }
        __syncthreads();
        if (part == 0 && lane == 0)
            for (int q = 1; q < wpr; q++) { a0 += red[wave + q][0]; a1 += red[wave + q][1]; }
    }
    if (part == 0 && lane == 0 && r < J.rows) {
        const float v = pair ? wh_silu_mul(a0, a1) : a0;
        J.y[r] = v;
        if (J.xchg)
            __hip_atomic_store(J.xchg + r, ((uint64_t)epoch << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
}

// block b of the launch (jobs as gemv_pack; all read pk.j[0].x)
template <bool XBF, int NXL>
__device__ __forceinline__ void gx_block(const gemv_pack &pk, int b, int xbytes, int xl_bytes, uint4 *xs,
                                         float (*red)[2], uint32_t epoch)
{
    uint4 xr[NXL];
    gx_x_issue<NXL>(pk.j[0].x, xbytes, xr);
    const int ji = (pk.n > 2 && b >= pk.j[2].blk0) ? 2 : (pk.n > 1 && b >= pk.j[1].blk0) ? 1 : 0;
#define SEL(f) (ji == 2 ? pk.j[2].f : ji == 1 ? pk.j[1].f : pk.j[0].f)
    gemv_job J;
    J.W0 = SEL(W0); J.W1 = SEL(W1); J.S0 = SEL(S0); J.S1 = SEL(S1); J.rowbytes = SEL(rowbytes);
    J.fmt = SEL(fmt); J.rows = SEL(rows); J.cols = SEL(cols); J.group = SEL(group);
    J.y = SEL(y); J.wpr = SEL(wpr); J.blk0 = SEL(blk0); J.xchg = SEL(xchg);
#undef SEL
    const int blk = b - J.blk0;
    const bool pair = J.W1 != nullptr;               // uniform
#define GR(F, P) gx_rows<F, XBF, NXL, P>(J, blk, xr, xbytes, xl_bytes, xs, red, epoch)
    if (J.fmt == 0) { if (pair) GR(0, true); else GR(0, false); }
    else if (J.fmt == 2) { if (pair) GR(2, true); else GR(2, false); }
    else { if (pair) GR(3, true); else GR(3, false); }
#undef GR
}

// E <= 256: the same launch without a counter.  Every router block tags
// its logits with the launch's epoch in xchg (device-coherent); the last
// router block, which the dispatcher starts after all the others, waits
// for the E tagged words (each thread its expert's, a bounded wait) and
// selects with all 256 threads (route_wg's two-level ranks instead of K
// dependent passes).  A logit that never arrives sets the status's time-out bit and
// selects nothing.
#define XWAIT_TICKS 5000000ull         // 50 ms of the 100 MHz constant clock
template <bool XBF, int NXL>
__global__ void __launch_bounds__(256)
k_gemv1_xroute(gemv_pack pk, whip_route_cfg c, const float *__restrict__ bias, int32_t *__restrict__ ids,
               float *__restrict__ wout, int32_t *__restrict__ pair_tok, int32_t *__restrict__ pair_exp,
               float *__restrict__ pair_w, int32_t *__restrict__ tok_pairs,
               const uint8_t *const *__restrict__ recs, const uint8_t **__restrict__ pair_rec,
               int *__restrict__ err, int xbytes, int xl_bytes)
{
    extern __shared__ uint4 xs[];                     // x, as gx_lay lays it out
    __shared__ float red[4][2];
    __shared__ __align__(16) float s_sc[ROUTE_FAST_FLOATS(256) > 256 ? ROUTE_FAST_FLOATS(256) : 256];
    __shared__ float s_sel[256];
    __shared__ uint64_t s_key[256], s_cand[64];
    __shared__ int s_rank[256];
    __shared__ float s_g[64], s_wraw[64], s_w[64];
    __shared__ int s_keep[64];
    __shared__ int32_t s_ids[64];
    __shared__ const uint8_t *s_recs[256];
    __shared__ const uint8_t *s_rec[64];
    __shared__ uint64_t s_etab[32];
    __shared__ int s_late;                            // a logit missed its tag (routing block)
    WT_SPAN(0, 0);
    WT_DECL;
    WT_KEEP(0);
    const int nrb = pk.j[0].nblk, tid = threadIdx.x, E = c.E, K = c.K;
    if (tid == 0) s_late = 0;                         // the product's barriers order it before the ORs
    const bool routing = (int)blockIdx.x == nrb - 1;  // uniform
    // This launch's tag: one past the last launch's, kept in the word before
    // the exchange (the routing block advances it once every router block
    // has tagged its logits, so every router block has read it by then).
    // A launch replayed from a graph, or another layer sharing the buffer,
    // therefore never meets a word carrying its own tag before it is written.
    uint64_t *const ew = pk.j[0].xchg - 1;
    uint32_t epoch = 0;
    if ((int)blockIdx.x < nrb) {                      // uniform
        epoch = (uint32_t)coh_ld(ew) + 1u;
        epoch = epoch ? epoch : 1u;                   // 0 is the buffer's initial tag
    }
    // the routing's other inputs, loaded beside the product's
    float be = 0.0f;
    const uint8_t *rv = nullptr;
    uint64_t ev = 0;
    if (routing) {
        const int ec = tid < E ? tid : 0;
        be = bias ? bias[ec] : 0.0f;
        rv = recs[ec];
        ev = wh_exp_tab[tid & 31];
    }
    gx_block<XBF, NXL>(pk, blockIdx.x, xbytes, xl_bytes, xs, red, epoch);
    WT_SPAN(0, 1);
    WT_KEEP(1);
#ifdef WH_TRACE
    if (threadIdx.x == 0 && blockIdx.x < 1024) {
        wt_buf[blockIdx.x * WT_SLOTS + 16] = wt_keep_[0];
        wt_buf[blockIdx.x * WT_SLOTS + 17] = wt_lds_[8];
        wt_buf[blockIdx.x * WT_SLOTS + 18] = wt_keep_[1];
    }
#endif
    if (!routing) return;
    if (tid < E) s_recs[tid] = rv;
    if (tid < 32) s_etab[tid] = ev;
    float l = 0.0f;
    int late = 0;
    if (tid < E) {
        const uint64_t *q = pk.j[0].xchg + tid;
        uint64_t v = coh_ld(q);
        if ((uint32_t)(v >> 32) != epoch) {
            const uint64_t t0 = wall_clock64();
            do {
                __builtin_amdgcn_s_sleep(2);
                v = coh_ld(q);
            } while ((uint32_t)(v >> 32) != epoch && wall_clock64() - t0 < XWAIT_TICKS);
            late = (uint32_t)(v >> 32) != epoch;
        }
        l = __uint_as_float((uint32_t)v);
    }
    // The OR through LDS and a plain barrier: __syncthreads_or reads the
    // workgroup size from the kernel's implicit arguments, a scalar load
    // that here, after the product's stream, misses every cache and sits
    // on the routing's critical path.
    if (late) s_late = 1;
    __syncthreads();
    const int any_late = s_late;
    if (tid == 0) coh_st(ew, (uint64_t)epoch);       // the next launch's tag follows this one
    if (any_late) {
        if (tid == 0) atomicOr(err, 16);
        if (tid < K) {
            ids[tid] = -1; wout[tid] = 0.0f;
            pair_tok[tid] = 0; pair_exp[tid] = E; pair_w[tid] = 0.0f; tok_pairs[tid] = tid;
            pair_rec[tid] = nullptr;
        }
        return;
    }
    WT_KEEP(2);
#ifdef WH_TRACE
    wt_keep_[5] = clock64();
#endif
    WT_L(0);
    if (((E + 63) >> 6) * K <= 64) {                  // uniform
        route_fast<256>(c, l, be, s_recs, s_etab, s_sc, s_ids, s_w, s_rec, err);
    } else {
        route_lds R;
        R.sc = s_sc; R.sel = s_sel; R.key = s_key; R.rank = s_rank; R.g = s_g; R.keep = s_keep; R.wraw = s_wraw;
        R.cand = s_cand;
        route_wg<256, true>(c, l, be, s_recs, s_etab, R, s_ids, s_w, s_rec, err);
    }
    WT_KEEP(3);
    WT_L(6);
#ifdef WH_TRACE
    wt_keep_[6] = clock64();
#endif
    if (tid < K) {
        const int e = s_ids[tid];
        ids[tid] = e;
        wout[tid] = s_w[tid];
        pair_tok[tid] = 0;
        pair_exp[tid] = e < 0 ? E : e;               // E: the table's NULL sentinel
        pair_w[tid] = s_w[tid];
        tok_pairs[tid] = tid;
        pair_rec[tid] = s_rec[tid];
    }
    WT_KEEP(4);
    if (tid == 0)
        for (int i = 0; i < 7; i++) WT_PUTAT(0, 1, i);
    WT_LPUT(0, 2);
}

WT_READER(whip_trace_gemv)

extern "C" int whip_gemv_route(const whip_gemv_job *jobs, int n, const whip_route_cfg *c, const float *bias,
                               int32_t *ids, float *w, int32_t *pair_tok, int32_t *pair_exp, float *pair_w,
                               int32_t *tok_pairs, const uint8_t *const *recs, const uint8_t **pair_rec,
                               int *err, int *cnt, uint64_t *xchg, hipStream_t s);

// padded columns of a matrix (whole quantisation groups)
static int padded_cols(const whip_mat *A)
{
    if (A->fmt == 0) return A->cols;
    return (A->cols + A->group - 1) / A->group * A->group;
}

// the batch-1 launch's job table; returns its block count
static int pack_gemv1(const whip_gemv_job *jobs, int n, gemv_pack &pk)
{
    int blk = 0;
    for (int i = 0; i < n; i++) {
        const whip_gemv_job *q = &jobs[i];
        const int ne = q->A.fmt == 0 ? 4 : q->A.fmt == 2 ? 16 : 32;
        const int nchunk = padded_cols(&q->A) / ne;
        gemv_job &J = pk.j[i];
        J.W0 = (const uint8_t *)q->A.q; J.S0 = q->A.qs;
        J.W1 = q->B ? (const uint8_t *)q->B->q : nullptr; J.S1 = q->B ? q->B->qs : nullptr;
        J.rowbytes = q->A.rowbytes; J.fmt = q->A.fmt; J.rows = q->A.rows; J.cols = q->A.cols;
        J.group = q->A.group; J.x = q->x; J.x_bf16 = q->x_bf16; J.y = q->y; J.y_ld = q->y_ld;
        const int U = q->A.fmt == 0 ? (q->x_bf16 ? 8 : 4) : (q->x_bf16 ? 2 : 1);
        int rpw = 1, wpr = 1;
        if (nchunk <= 64) rpw = 4;
        else wpr = nchunk > 64 * U * 2 ? 4 : nchunk > 64 * U ? 2 : 1;
        J.x_ld = q->x_ld;
        J.rpw = rpw;
        J.wpr = wpr;
        J.coh = 0;
        J.xchg = nullptr;
        J.epoch = 0;
        const int groups = (J.rows + rpw - 1) / rpw;
        J.nblk = (groups + 4 / wpr - 1) / (4 / wpr);
        J.blk0 = blk;
        blk += J.nblk;
    }
    pk.n = n;
    pk.T = 1;
    return blk;
}

// the x-in-LDS launch's job table: rows split over wpr wavefronts so that a
// lane's chunks fit gx_u; returns the block count, and the bytes of x
// (xbytes), of its padded columns (xl_bytes) and of its LDS layout (lds)
static int pack_gx(const whip_gemv_job *jobs, int n, gemv_pack &pk, int &xbytes, int &xl_bytes, int &lds)
{
    int blk = 0;
    const int esz = jobs[0].x_bf16 ? 2 : 4;
    xbytes = jobs[0].A.cols * esz;
    xl_bytes = 0;
    lds = 0;
    for (int i = 0; i < n; i++) {
        const whip_gemv_job *q = &jobs[i];
        const int fmt = q->A.fmt;
        const int ne = fmt == 0 ? 4 : fmt == 2 ? 16 : 32;
        const int nchunk = padded_cols(&q->A) / ne;
        const int U = fmt == 0 && !q->B ? 8 : 4;
        gemv_job &J = pk.j[i];
        J.W0 = (const uint8_t *)q->A.q; J.S0 = q->A.qs;
        J.W1 = q->B ? (const uint8_t *)q->B->q : nullptr; J.S1 = q->B ? q->B->qs : nullptr;
        J.rowbytes = q->A.rowbytes; J.fmt = fmt; J.rows = q->A.rows; J.cols = q->A.cols;
        J.group = q->A.group; J.x = q->x; J.x_bf16 = q->x_bf16; J.y = q->y; J.y_ld = q->y_ld;
        J.x_ld = q->x_ld;
        J.wpr = nchunk <= 64 * U ? 1 : nchunk <= 128 * U ? 2 : 4;
        J.rpw = 1;
        J.coh = 0;
        J.xchg = nullptr;
        J.epoch = 0;
        const int rpb = 4 / J.wpr;
        J.nblk = (J.rows + rpb - 1) / rpb;
        J.blk0 = blk;
        blk += J.nblk;
        const int xl = padded_cols(&q->A) * esz;
        const int nw = (ne * esz + 15) / 16;
        const bool pad = nw >= 2 && ne * esz >= 32;
        const int l = pad ? xl / 16 / nw * (nw + 1) * 16 : xl;
        if (xl > xl_bytes) xl_bytes = xl;
        if (l > lds) lds = l;
    }
    pk.n = n;
    pk.T = 1;
    return blk;
}

static int launch_gemv1(const whip_gemv_job *jobs, int n, hipStream_t s)
{
    gemv_pack pk;
    const int blk = pack_gemv1(jobs, n, pk);
    if (jobs[0].x_bf16) WHIP_LAUNCH(k_gemv1<true>, dim3(blk), dim3(256), 0, s, pk);
    else WHIP_LAUNCH(k_gemv1<false>, dim3(blk), dim3(256), 0, s, pk);
    return (int)hipGetLastError();
}

static int waves_per_row(const whip_mat *A)
{
    // about UNROLL chunks per lane and at least one full pass of loads
    const int ne = A->fmt == 0 ? 4 : A->fmt == 2 ? 16 : 32;
    const int ng = A->fmt == 0 ? 1 : (A->cols + A->group - 1) / A->group;
    const int padded = A->fmt == 0 ? A->cols : ng * A->group;
    const int nchunk = (padded + ne - 1) / ne;
    if (nchunk >= 64 * UNROLL * 4 && A->rows <= 1024) return 4;
    if (nchunk >= 64 * UNROLL * 2 && A->rows <= 2048) return 2;
    return 1;
}

static int check_mat(const whip_mat *A)
{
    if (A->fmt == 0) return (A->cols % 4 || A->rowbytes % 16) ? -1 : 0;
    if (A->fmt != 2 && A->fmt != 3) return -1;
    return (A->group % 32 || A->rowbytes % 16) ? -1 : 0;
}

extern "C" int whip_gemv_multi(const whip_gemv_job *jobs, int n, int T, hipStream_t s)
{
    if (n < 1 || n > 3 || T < 1) return (int)hipErrorInvalidValue;
    gemv_pack pk;
    int blk = 0;
    for (int i = 0; i < n; i++) {
        const whip_gemv_job *q = &jobs[i];
        if (check_mat(&q->A) || (q->B && (q->B->fmt != q->A.fmt || q->B->rows != q->A.rows ||
                                          q->B->cols != q->A.cols || q->B->group != q->A.group ||
                                          q->B->rowbytes != q->A.rowbytes)))
            return (int)hipErrorInvalidValue;
        if (q->x_ld % 4) return (int)hipErrorInvalidValue;
        gemv_job &J = pk.j[i];
        J.W0 = (const uint8_t *)q->A.q; J.S0 = q->A.qs;
        J.W1 = q->B ? (const uint8_t *)q->B->q : nullptr; J.S1 = q->B ? q->B->qs : nullptr;
        J.rowbytes = q->A.rowbytes; J.fmt = q->A.fmt; J.rows = q->A.rows; J.cols = q->A.cols;
        J.group = q->A.group; J.x = q->x; J.x_ld = q->x_ld; J.x_bf16 = q->x_bf16;
        J.y = q->y; J.y_ld = q->y_ld;
        J.wpr = waves_per_row(&q->A);
        J.rpw = 1;
        J.coh = 0;
        J.xchg = nullptr;
        J.epoch = 0;
        J.blk0 = blk;
        J.nblk = (J.rows + (4 / J.wpr) - 1) / (4 / J.wpr);
        blk += J.nblk;
    }
    pk.n = n;
    pk.T = T;
    if (T == 1) {
        bool fits = true;
        for (int i = 0; i < n; i++)
            // x slices are read 16 bytes at a time and never past the last column
            fits = fits && (uintptr_t)jobs[i].x % 16 == 0 && (jobs[i].A.fmt == 0 || jobs[i].A.cols % 8 == 0) &&
                   jobs[i].x_bf16 == jobs[0].x_bf16;
        if (fits) return launch_gemv1(jobs, n, s);
    }
    if (T == 1) hipLaunchKernelGGL(k_gemv_multi<1>, dim3(blk), dim3(256), 0, s, pk);
    else hipLaunchKernelGGL(k_gemv_multi<TB>, dim3(blk), dim3(256), 0, s, pk);
    return (int)hipGetLastError();
}

extern "C" int whip_gemv(const whip_mat *A, const whip_mat *B, const float *x, int x_ld, int T,
                         float *y0, float *y1, int y_ld, hipStream_t s)
{
    whip_gemv_job j[2];
    int n = 0;
    j[n].A = *A; j[n].B = NULL; j[n].x = x; j[n].x_ld = x_ld; j[n].x_bf16 = 0; j[n].y = y0;
    j[n].y_ld = y_ld; n++;
    if (B) {
        j[n].A = *B; j[n].B = NULL; j[n].x = x; j[n].x_ld = x_ld; j[n].x_bf16 = 0; j[n].y = y1;
        j[n].y_ld = y_ld; n++;
    }
    return whip_gemv_multi(j, n, T, s);
}

// One token: routing plus a batch-1 product independent of it, in one launch.
extern "C" int whip_route_gemv(const whip_route_cfg *c, const float *logits, const float *bias,
                               int32_t *ids, float *w, int32_t *pair_tok, int32_t *pair_exp,
                               float *pair_w, int32_t *tok_pairs, const uint8_t *const *recs,
                               const uint8_t **pair_rec, int *err, const whip_gemv_job *job,
                               hipStream_t s)
{
    if (c->E > MAXE || c->E <= 0 || c->K <= 0 || c->K > 64 || c->K > c->E || !pair_exp)
        return (int)hipErrorInvalidValue;
    if (c->n_group > 1 && (c->n_group > 64 || c->E % c->n_group || c->topk_group < 1))
        return (int)hipErrorInvalidValue;
    if (check_mat(&job->A) || job->B || job->x_ld % 4 || (uintptr_t)job->x % 16 ||
        (job->A.fmt != 0 && job->A.cols % 8))
        return (int)hipErrorInvalidValue;
    gemv_pack pk;
    const int blk = pack_gemv1(job, 1, pk);
    const int E = c->E;
#define RG(N, XB) hipLaunchKernelGGL((k_route_gemv1<N, XB>), dim3(blk + 1), dim3(256), 0, s, *c, logits, bias, \
                                     ids, w, pair_tok, pair_exp, pair_w, tok_pairs, recs, pair_rec, err, pk)
#define RGX(N) do { if (job->x_bf16) RG(N, true); else RG(N, false); } while (0)
    if (E <= 64) RGX(1);
    else if (E <= 128) RGX(2);
    else if (E <= 256) RGX(4);
    else if (E <= 512) RGX(8);
    else RGX(16);
#undef RGX
#undef RG
    return (int)hipGetLastError();
}

// One token: router logits (job 0, writing logits[E]) and up to two more
// batch-1 products in one launch, the token routed by the launch's last
// router block.
extern "C" int whip_gemv_route(const whip_gemv_job *jobs, int n, const whip_route_cfg *c, const float *bias,
                               int32_t *ids, float *w, int32_t *pair_tok, int32_t *pair_exp, float *pair_w,
                               int32_t *tok_pairs, const uint8_t *const *recs, const uint8_t **pair_rec,
                               int *err, int *cnt, uint64_t *xchg, hipStream_t s)
{
    if (n < 1 || n > 3 || c->E > MAXE || c->E <= 0 || c->K <= 0 || c->K > 64 || c->K > c->E || !pair_exp ||
        (!cnt && !xchg) || jobs[0].A.rows != c->E)
        return (int)hipErrorInvalidValue;
    if (c->n_group > 1 && (c->n_group > 64 || c->E % c->n_group || c->topk_group < 1))
        return (int)hipErrorInvalidValue;
    for (int i = 0; i < n; i++) {
        const whip_gemv_job *q = &jobs[i];
        if (check_mat(&q->A) || (q->B && (q->B->fmt != q->A.fmt || q->B->rows != q->A.rows ||
                                          q->B->cols != q->A.cols || q->B->group != q->A.group ||
                                          q->B->rowbytes != q->A.rowbytes)))
            return (int)hipErrorInvalidValue;
        if (q->x_ld % 4 || (uintptr_t)q->x % 16 || (q->A.fmt != 0 && q->A.cols % 8) ||
            q->x_bf16 != jobs[0].x_bf16)
            return (int)hipErrorInvalidValue;
    }
    gemv_pack pk;
    const int blk = pack_gemv1(jobs, n, pk);
    const int E = c->E;
    bool one_x = true;                                // every job reads the router's x
    for (int i = 1; i < n; i++) one_x = one_x && jobs[i].x == jobs[0].x && jobs[i].A.cols == jobs[0].A.cols;
    if (xchg && E <= 256 && pair_rec && one_x) {
        gemv_pack gp;
        int xbytes, xl_bytes, lds;
        const int gblk = pack_gx(jobs, n, gp, xbytes, xl_bytes, lds);
        gp.j[0].xchg = xchg + 1;                      // word 0: the last launch's tag
        const int nxl = (xl_bytes + 4095) / 4096;     // 16-byte x loads per thread
        if (nxl <= 16 && lds <= 48 * 1024) {
#define XR(XB, NX) WHIP_LAUNCH((k_gemv1_xroute<XB, NX>), dim3(gblk), dim3(256), (size_t)lds, s, gp, *c, bias, ids, \
                               w, pair_tok, pair_exp, pair_w, tok_pairs, recs, pair_rec, err, xbytes, xl_bytes)
#define XRB(NX) do { if (jobs[0].x_bf16) XR(true, NX); else XR(false, NX); } while (0)
            if (nxl <= 2) XRB(2);
            else if (nxl <= 4) XRB(4);
            else if (nxl <= 8) XRB(8);
            else XRB(16);
#undef XRB
#undef XR
            return (int)hipGetLastError();
        }
    }
    if (!cnt) return (int)hipErrorInvalidValue;
    pk.j[0].coh = 1;
#define RG(N, XB) WHIP_LAUNCH((k_gemv1_route<XB, N>), dim3(blk), dim3(256), 0, s, pk, *c, bias, ids, w, \
                                     pair_tok, pair_exp, pair_w, tok_pairs, recs, pair_rec, err, cnt)
#define RGX(N) do { if (jobs[0].x_bf16) RG(N, true); else RG(N, false); } while (0)
    if (E <= 64) RGX(1);
    else if (E <= 128) RGX(2);
    else if (E <= 256) RGX(4);
    else if (E <= 512) RGX(8);
    else RGX(16);
#undef RGX
#undef RG
    return (int)hipGetLastError();
}
