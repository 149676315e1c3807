// SPDX-License-Identifier: Apache-2.0
//
// vq2r.hip — VQ2R experts (two residual stages of 256 entries, one index
// byte a stage: docs/FORMAT.md:180, 205) in the device layer, in the
// engine's own arithmetic: each table entry is vq_build_lut's
// (src/model.c:3864-3880 through lutb_range: model.c:3815-3854 portable,
// simd_avx512.c:90-123 with fma) and each row is vq_rows' generic loop
// (model.c:3966-3970: t = L0[c0] + L1[c1], acc += t over the positions in
// order, y = acc * f16(scale)).  One lane per row owns its sum; the tables
// are read through the caches.
#include "common.h"
#include "gemv_dev.h"
#include "launch.h"

#define R2_EN 256
#define R2_LV 16

// table t = (input row t / kinds, kind t % kinds): lut[t][v][s][e] =
// sum_d x[8v + d] * C[cb + 2 kind + s][e][d], booksT [book][8][256], two
// stages.  ACT: the input row of pair t is h = silu(g) * u of its gate and
// up rows gu[t][0][.], gu[t][1][.] (waste_act_pair_range), built here.  A
// workgroup stages its R2_LV positions' inputs in LDS, then thread e builds
// entry e of both stages for each.
template <bool FMA, bool ACT>
__global__ void __launch_bounds__(R2_EN)
k_r2_lutb(const void *__restrict__ x, int x_bf16, int x_ld, int kinds, const float *__restrict__ booksT, int cb,
          int nv, float *__restrict__ lut, whip_mat shd, const float *__restrict__ shd_x, float *__restrict__ shd_y,
          int tabs)
{
    __shared__ float s_x[R2_LV * 8];
    if (!ACT && (int)blockIdx.y >= tabs) {           // uniform: the rows past the tables' run the shared down
        shd_rows_any(shd, shd_x, shd_y, (blockIdx.y - tabs) * gridDim.x + blockIdx.x, (gridDim.y - tabs) * gridDim.x,
                     R2_EN / 64);
        return;
    }
    const int t = blockIdx.y, row = t / kinds, kind = t - row * kinds;
    const int e = threadIdx.x;
    const int v0 = blockIdx.x * R2_LV, n = min(R2_LV, nv - v0);
    float c[2][8];
#pragma unroll
    for (int st = 0; st < 2; st++)
#pragma unroll
        for (int d = 0; d < 8; d++) c[st][d] = booksT[((size_t)(cb + 2 * kind + st) * 8 + d) * R2_EN + e];
    if (e < 8 * n) {
        const size_t i = (size_t)v0 * 8 + e;
        float xv;
        if (ACT) {
            const float *gu = (const float *)x + (size_t)row * 2 * x_ld;
            xv = wh_silu_mul(gu[i], gu[x_ld + i]);
        } else {
            xv = x_bf16 ? wh_bf16(((const uint16_t *)x)[(size_t)row * x_ld + i]) : ((const float *)x)[(size_t)row * x_ld + i];
        }
        s_x[e] = xv;
    }
    __syncthreads();
    for (int v = 0; v < n; v++) {
#pragma unroll
        for (int st = 0; st < 2; st++) {
            float a = 0.0f;
#pragma unroll
            for (int d = 0; d < 8; d++) {
                const float xd = s_x[v * 8 + d];
                a = FMA ? __fmaf_rn(xd, c[st][d], a) : __fadd_rn(a, __fmul_rn(xd, c[st][d]));
            }
            lut[(((size_t)t * nv + v0 + v) * 2 + st) * R2_EN + e] = a;
        }
    }
}

extern "C" int whip_r2_lutb(const void *x, int x_bf16, int x_ld, int rows, int kinds, int st, const float *booksT,
                            int cb, int nv, int fma, float *lut, const whip_mat *shd, const float *shd_x,
                            float *shd_y, hipStream_t s)
{
    if (rows <= 0 || kinds <= 0 || rows * kinds > 65535 || st != 2 || nv <= 0 || x_ld < nv * 8 || cb < 0 ||
        (shd_y && !shd_rows_ok(shd, shd_x)))
        return (int)hipErrorInvalidValue;
    const int gx = (nv + R2_LV - 1) / R2_LV, tabs = rows * kinds;
    // shd_y: rows of spare workgroups (four wavefronts each) for the shared
    // down projection, to about two workgroups per CU beside the tables'
    int ry = 0;
    if (shd_y) {
        const int spare = 512 - gx * tabs;
        ry = (spare > 8 * 1 ? spare : 8) / gx + 1;
    }
    const dim3 grid(gx, tabs + ry);
    const whip_mat W = shd_y ? *shd : whip_mat{};
    if (fma) WHIP_LAUNCH((k_r2_lutb<true, false>), grid, dim3(R2_EN), 0, s, x, x_bf16, x_ld, kinds, booksT, cb, nv, lut,
                         W, shd_x, shd_y, tabs);
    else WHIP_LAUNCH((k_r2_lutb<false, false>), grid, dim3(R2_EN), 0, s, x, x_bf16, x_ld, kinds, booksT, cb, nv, lut,
                     W, shd_x, shd_y, tabs);
    return (int)hipGetLastError();
}

extern "C" int whip_r2_act_lutb(const float *gu, int P, int I, const float *booksT, int cb, int fma, float *lut,
                                hipStream_t s)
{
    if (P <= 0 || P > 65535 || I <= 0 || I % 8 || cb < 0) return (int)hipErrorInvalidValue;
    const int nv = I / 8;
    const dim3 grid((nv + R2_LV - 1) / R2_LV, P);
    if (fma) WHIP_LAUNCH((k_r2_lutb<true, true>), grid, dim3(R2_EN), 0, s, gu, 0, I, 1, booksT, cb, nv, lut,
                         whip_mat{}, nullptr, nullptr, P);
    else WHIP_LAUNCH((k_r2_lutb<false, true>), grid, dim3(R2_EN), 0, s, gu, 0, I, 1, booksT, cb, nv, lut,
                     whip_mat{}, nullptr, nullptr, P);
    return (int)hipGetLastError();
}

// vq_rows of every pair's matrices, two stages: grid (row-block groups,
// pairs, kinds), a lane per row.  Pair p's matrix `kind` is at idx_off[kind]
// of its expert's record (indices blocked [row / 64][v][row % 64][2]), its
// f16 row scales at sc_off[kind]; its table is pair_tok[p] * kinds + kind
// (per_tok) or p.  out[p][kind][M].  An unbound expert writes zeros and
// raises bit 0 of err.
//
// A row's sum runs over the positions in order, so one lane owns it.  The
// table entries a lane needs are random within each position's 2 KB: read
// through the vector memory path that is one cache-line lookup per lane
// group, read from LDS a few bank cycles.  So a workgroup of R2_WAVES
// wavefronts (one 64-row block each, one matrix) streams the table through
// LDS R2_W positions at a time, double-buffered: each round the next
// window's entries and codes are in flight while the wavefronts add the
// current window's.
#define R2_WAVES 4
#define R2_W 8                         // positions a round
#define R2_WIN (R2_W * 2 * R2_EN)      // floats of a window
#define R2_TV (R2_WIN / 4 / (R2_WAVES * 64))   // uint4s a thread stages a round

__global__ void __launch_bounds__(R2_WAVES * 64)
k_r2_rows_pairs(const uint8_t *const *__restrict__ recs, const int32_t *__restrict__ pair_exp,
                const int32_t *__restrict__ pair_tok, int kinds, uint32_t idx_off0, uint32_t idx_off1,
                uint32_t sc_off0, uint32_t sc_off1, int M, int nv, const float *__restrict__ lut, int per_tok,
                float *__restrict__ out, int *__restrict__ err)
{
    __shared__ __align__(16) float s_l[2][R2_WIN];
    const int p = blockIdx.y, kind = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rb = blockIdx.x * R2_WAVES + wv, r = rb * 64 + lane;
    const bool live = r < M;
    const uint8_t *rec = recs[pair_exp[p]];
    float *y = out + ((size_t)p * kinds + kind) * M;
    if (rec == nullptr) {                            // uniform
        if (live) y[r] = 0.0f;
        if (tid == 0) atomicOr(err, 1);
        return;
    }
    const size_t tab = per_tok ? (size_t)pair_tok[p] * kinds + kind : (size_t)p;
    typedef unsigned v4u __attribute__((ext_vector_type(4)));   // promoted to registers, unlike uint4 here
    const v4u WH_GLOBAL *L = (const v4u WH_GLOBAL *)(lut + tab * nv * 2 * R2_EN);
    // rows past M read row 0's codes (in bounds; not stored)
    const uint16_t WH_GLOBAL *ix =
        (const uint16_t WH_GLOBAL *)(as_global(rec) + (kind ? idx_off1 : idx_off0)) +
        (live ? (size_t)rb * nv * 64 + lane : 0);
    const int nr = (nv + R2_W - 1) / R2_W, nq = nv * 2 * R2_EN / 4;
    // round rr: the window's uint4s (past the table: its first ones, unused)
    // and this lane's codes (past nv: the last position's, not added)
    auto fetch = [&](v4u (&tv)[R2_TV], uint32_t (&w)[R2_W], int rr) {
        const int q0 = rr * (R2_WIN / 4);
#pragma unroll
        for (int k = 0; k < R2_TV; k++) {
            const int q = q0 + tid + k * R2_WAVES * 64;
            tv[k] = L[q < nq ? q : 0];
        }
#pragma unroll
        for (int k = 0; k < R2_W; k++) w[k] = ix[(size_t)min(rr * R2_W + k, nv - 1) * 64];
    };
    auto stage = [&](const v4u (&tv)[R2_TV], int b) {
#pragma unroll
        for (int k = 0; k < R2_TV; k++) ((v4u *)s_l[b])[tid + k * R2_WAVES * 64] = tv[k];
    };
    float acc = 0.0f;
    auto add = [&](const uint32_t (&w)[R2_W], int rr, int b) {
        const int n = min(R2_W, nv - rr * R2_W);
#pragma unroll
        for (int k = 0; k < R2_W; k++) {
            const float *blk = s_l[b] + k * 2 * R2_EN;
            const float t = __fadd_rn(blk[w[k] & 255], blk[R2_EN + (w[k] >> 8)]);
            acc = k < n ? __fadd_rn(acc, t) : acc;
        }
    };
    v4u tA[R2_TV], tB[R2_TV];
    uint32_t wA[R2_W], wB[R2_W];
    fetch(tA, wA, 0);
    __builtin_amdgcn_sched_barrier(0);
    stage(tA, 0);
    fetch(tB, wB, 1);                                // past the last round: harmless repeats
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    for (int rr = 0; rr < nr; rr += 2) {             // uniform
        add(wA, rr, 0);
        __builtin_amdgcn_sched_barrier(0);
        stage(tB, 1);                                // window rr + 1: its loads went out a round ago
        __syncthreads();                             // (and every wavefront is done with window rr)
        fetch(tA, wA, rr + 2);
        __builtin_amdgcn_sched_barrier(0);
        add(wB, rr + 1, 1);                          // past the last round: adds nothing
        __builtin_amdgcn_sched_barrier(0);
        stage(tA, 0);
        __syncthreads();
        fetch(tB, wB, rr + 3);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (live) {
        const uint16_t *sc = (const uint16_t *)(rec + (kind ? sc_off1 : sc_off0));
        y[r] = __fmul_rn(acc, wh_f16_scale(sc[r]));
    }
}

// The same rows with the entries fetched through the vector memory path,
// for launches with too few rows a table to spread the LDS kernel's
// workgroups over the CUs: grid (row blocks, pairs, kinds).  Four
// wavefronts share a 64-row block: each round, wavefront w fetches the
// codes of positions 64 round + 16 w .. (the next round's already in
// flight) and their two table entries, and leaves the entries' sums in LDS;
// wavefront 0 then adds the round's 64 positions in order while the others
// fetch the next round.
#define R2F_WAVES 4
#define R2F_PW 16                       // positions a wavefront fetches a round
#define R2F_ROUND (R2F_WAVES * R2F_PW)

__global__ void __launch_bounds__(R2F_WAVES * 64)
k_r2_rows_fetch(const uint8_t *const *__restrict__ recs, const int32_t *__restrict__ pair_exp,
                const int32_t *__restrict__ pair_tok, int kinds, uint32_t idx_off0, uint32_t idx_off1,
                uint32_t sc_off0, uint32_t sc_off1, int M, int nv, const float *__restrict__ lut, int per_tok,
                float *__restrict__ out, int *__restrict__ err)
{
    __shared__ float s_t[2][R2F_ROUND][64];
    const int p = blockIdx.y, kind = blockIdx.z, rb = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = rb * 64 + lane;
    const uint8_t *rec = recs[pair_exp[p]];
    float *y = out + ((size_t)p * kinds + kind) * M;
    if (rec == nullptr) {                            // uniform
        if (tid < 64 && r < M) y[r] = 0.0f;
        if (tid == 0) atomicOr(err, 1);
        return;
    }
    const size_t tab = per_tok ? (size_t)pair_tok[p] * kinds + kind : (size_t)p;
    const float WH_GLOBAL *L = (const float WH_GLOBAL *)(lut + tab * nv * 2 * R2_EN);
    // rows past M read row 0's codes (in bounds); their sums are not stored
    const uint16_t WH_GLOBAL *ix =
        (const uint16_t WH_GLOBAL *)(as_global(rec) + (kind ? idx_off1 : idx_off0) + (size_t)rb * nv * 128) +
        (r < M ? lane : 0);
    const int nr = (nv + R2F_ROUND - 1) / R2F_ROUND;
    // the codes of this wavefront's positions in round rr (past nv: the last
    // position's, not added)
    auto fetch = [&](uint32_t (&w)[R2F_PW], int rr) {
#pragma unroll
        for (int k = 0; k < R2F_PW; k++) {
            const int v = min(rr * R2F_ROUND + wv * R2F_PW + k, nv - 1);
            w[k] = ix[(size_t)v * 64];
        }
    };
    auto gather = [&](const uint32_t (&w)[R2F_PW], int rr, int b) {
        float g[2 * R2F_PW];
#pragma unroll
        for (int k = 0; k < R2F_PW; k++) {
            const int v = min(rr * R2F_ROUND + wv * R2F_PW + k, nv - 1);
            const float WH_GLOBAL *blk = L + (size_t)v * 2 * R2_EN;
            g[2 * k] = blk[w[k] & 255];
            g[2 * k + 1] = blk[R2_EN + (w[k] >> 8)];
        }
#pragma unroll
        for (int k = 0; k < R2F_PW; k++) s_t[b][wv * R2F_PW + k][lane] = __fadd_rn(g[2 * k], g[2 * k + 1]);
    };
    float acc = 0.0f;
    auto consume = [&](int rr, int b) {
        const int n = min(R2F_ROUND, nv - rr * R2F_ROUND);
#pragma unroll 8
        for (int k = 0; k < n; k++) acc = __fadd_rn(acc, s_t[b][k][lane]);
    };
    // a round's entries go out before the next round's codes: loads complete
    // in issue order, so the wait for the entries does not cover the codes
    uint32_t wA[R2F_PW], wB[R2F_PW];
    fetch(wA, 0);
    __builtin_amdgcn_sched_barrier(0);
    fetch(wB, 1);                                    // past the last round: harmless repeats
    __builtin_amdgcn_sched_barrier(0);
    for (int rr = 0; rr < nr; rr += 2) {             // uniform
        gather(wA, rr, 0);
        __builtin_amdgcn_sched_barrier(0);
        fetch(wA, rr + 2);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        if (wv == 0) consume(rr, 0);
        if (rr + 1 >= nr) break;                     // uniform: the whole workgroup
        gather(wB, rr + 1, 1);
        __builtin_amdgcn_sched_barrier(0);
        fetch(wB, rr + 3);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        if (wv == 0) consume(rr + 1, 1);
    }
    if (wv == 0 && r < M) {
        const uint16_t *sc = (const uint16_t *)(rec + (kind ? sc_off1 : sc_off0));
        y[r] = __fmul_rn(acc, wh_f16_scale(sc[r]));
    }
}

extern "C" int whip_r2_rows_pairs(const uint8_t *const *recs, const int32_t *pair_exp, const int32_t *pair_tok,
                                  int P, int kinds, const uint32_t *idx_off, const uint32_t *sc_off, int M, int nv,
                                  const float *lut, int per_tok, float *out, int *err, hipStream_t s)
{
    if (P <= 0 || P > 65535 || kinds < 1 || kinds > 2 || M <= 0 || nv <= 0 || idx_off[0] % 2 ||
        (kinds > 1 && idx_off[1] % 2))
        return (int)hipErrorInvalidValue;
    // the LDS kernel stages a table's every window per workgroup: with
    // fewer than 192 workgroups (one token's gate/up at batch 1) the
    // fetching kernel, which spreads over four times as many, is faster
    const int groups = (M + 64 * R2_WAVES - 1) / (64 * R2_WAVES);
    const uint32_t i1 = kinds > 1 ? idx_off[1] : 0, s1 = kinds > 1 ? sc_off[1] : 0;
    if ((long)groups * P * kinds >= 192)
        WHIP_LAUNCH(k_r2_rows_pairs, dim3(groups, P, kinds), dim3(R2_WAVES * 64), 0, s, recs, pair_exp, pair_tok,
                    kinds, idx_off[0], i1, sc_off[0], s1, M, nv, lut, per_tok, out, err);
    else
        WHIP_LAUNCH(k_r2_rows_fetch, dim3((M + 63) / 64, P, kinds), dim3(R2F_WAVES * 64), 0, s, recs, pair_exp,
                    pair_tok, kinds, idx_off[0], i1, sc_off[0], s1, M, nv, lut, per_tok, out, err);
    return (int)hipGetLastError();
}
