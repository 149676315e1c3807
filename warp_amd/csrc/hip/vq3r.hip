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
// 64-row block at one position is 192 contiguous bytes.  Lane (g, rq) of a
// wavefront reads the 12 bytes of rows 4rq..4rq+3 of row block g of its
// group of four, one dwordx3 per position: the four 16-lane groups take
// four row blocks at the same position.  The table address is then the
// same for the whole wave (its position) and folds into the LDS read's
// offset; each lane keeps its four rows' sums over the chunk's positions,
// so no cross-lane reduction is needed.
//
// A workgroup owns a chunk of VC positions for one kind and a share of the
// row blocks of one pair (or, when every pair reads the same source row,
// of all pairs).  It builds the chunk's table in LDS — VC*3*256 fp32 —
// once, then streams the rows through it: the table costs 6144 FMAs per
// position, amortised over every row.  Row sums leave as per-chunk
// partials; the next kernel reduces them.  The split is what lets a decode
// token's eight experts fill 256 CUs.
#include "common.h"
#include "launch.h"
#include "gemv_dev.h"
#include "route.h"
#include "trace.h"

#ifndef WH_VC
#define WH_VC 8
#endif
#define VC WH_VC                    // positions per workgroup chunk
#ifndef WH_LANES
#define WH_LANES 1                  // the positions-across-lanes kernel when nv % 32 == 0
#endif
#define LUT_PER_V (3 * 256)

// The tile kernels take whole 32-position chunks and pairs of 64-row blocks.
#define LANES_OK(nv, M) (WH_LANES && (nv) % 32 == 0 && (M) % 128 == 0)

extern "C" int whip_vq_chunks(int nv, int M) { return LANES_OK(nv, M) ? nv / 32 : (nv + VC - 1) / VC; }

typedef const uint3 WH_GLOBAL g_uint3;

// Row blocks are numbered over the pairs a workgroup may span: vb = q*nb + rb
// is row block rb of pair p0 + q.  With span 1 a workgroup owns (a share of)
// one pair's rows; with span = P every pair reads source row 0 (a one-token
// decode's gate/up), so one table serves all of their rows and a
// workgroup's share runs across experts.
#define SPAN_MAX 64
#define VQ_THREADS 512
#define LUT_ITERS ((LUT_PER_V + VQ_THREADS - 1) / VQ_THREADS)

__device__ __forceinline__ void
vq_apply_body(const uint8_t *const *__restrict__ recs, const int32_t *__restrict__ pair_exp,
              const int32_t *__restrict__ pair_src, const void *__restrict__ src, int src_ld,
              int src_bf16, const float *__restrict__ booksT, int cb, uint32_t off0,
              uint32_t off1, int kinds, int M, int nv, int nch, int rsplit, int P, int span,
              float *__restrict__ part, int *__restrict__ err)
{
    __shared__ float lut[VC * LUT_PER_V];
    __shared__ float xs[VC * 8];
    __shared__ const uint8_t *s_rec[SPAN_MAX];
    const int c = blockIdx.x, kind = blockIdx.y / rsplit, rs = blockIdx.y % rsplit;
    const int tid = threadIdx.x;
    const int lane = tid & 63, nw = VQ_THREADS >> 6;
    const int v0 = c * VC;                       // nv % VC == 0 (host contract)
    const int nb = M >> 6;                       // M % 64 == 0 (host contract)
    const int p0 = span > 1 ? 0 : blockIdx.z, np = span > 1 ? P : 1;
    const int V = np * nb;
    const int vlo = (int)((long)rs * V / rsplit), vhi = (int)((long)(rs + 1) * V / rsplit);

    // everything the table needs is requested before the first barrier
    if (tid < np) s_rec[tid] = recs[pair_exp[p0 + tid]];
    const float *bT = booksT + (size_t)(cb + kind * 3) * 8 * 256;
    float cv[LUT_ITERS][8];
#pragma unroll
    for (int i = 0; i < LUT_ITERS; i++) {
        const int q = tid + i * VQ_THREADS < LUT_PER_V ? tid + i * VQ_THREADS : 0;
        const float *cr = bT + (size_t)(q >> 8) * 8 * 256 + (q & 255);
#pragma unroll
        for (int d = 0; d < 8; d++) cv[i][d] = cr[d * 256];
    }
    const int srow = pair_src ? pair_src[p0] : p0;
    if (tid < VC * 8) {
        const size_t o = (size_t)srow * src_ld + (size_t)v0 * 8 + tid;
        xs[tid] = src_bf16 ? wh_bf16(((const uint16_t *)src)[o]) : ((const float *)src)[o];
    }
    __syncthreads();

    // A wavefront takes groups of four row blocks: vlo + 4*(wave + nw*it) + g.
    // The buffer rolls: position k of the next group is requested as soon as
    // position k of this one is consumed, so a load has a whole group's
    // compute to arrive, in VC registers' worth of buffer.  Loads are never
    // behind a branch (the compiler, unsure how many are in flight, would
    // wait for all): a row block past the share's end or with no record
    // reads a fixed in-bounds dummy, the codebook buffer (73 KB, beyond the
    // 1.6 KB a lane's offsets reach), stores into the sink after the
    // partials, and counts as dead.
    const int g = lane >> 4, rq = lane & 15;
    const uint32_t off = kind ? off1 : off0;
    const size_t rstride = (size_t)nv * 192;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    g_u8 *dummy = as_global((const uint8_t *)booksT) + rq * 12;
    float *sink = part + (size_t)(span > 1 ? P : gridDim.z) * kinds * nch * M;
    auto src_of = [&](int vb, bool &lv, float *&out) -> g_u8 * {
        const uint8_t *r = nullptr;
        int q = 0, rb = 0;
        if (vb < vhi) { q = vb / nb; rb = vb - q * nb; r = s_rec[q]; }
        lv = r != nullptr;
        out = vb < vhi ? part + (((size_t)(p0 + q) * kinds + kind) * nch + c) * (size_t)M + rb * 64 + rq * 4
                       : sink + rq * 4;
        return r ? as_global(r) + off + (size_t)v0 * 192 + (size_t)rb * rstride + rq * 12 : dummy;
    };
    uint3 buf[VC];
    bool live;
    float *outp;
    {
        g_u8 *pp = src_of(vlo + 4 * wv + g, live, outp);
#pragma unroll
        for (int k = 0; k < VC; k++) buf[k] = *(g_uint3 *)(pp + k * 192);
    }

    // L[v][s][c] = fma chain over d from 0 (the engine's AVX-512 order).
    // A thread owns one (stage, code) per pass: its 8 codebook values stay
    // in registers while it sweeps the chunk's positions.
#pragma unroll
    for (int i = 0; i < LUT_ITERS; i++) {
        const int q = tid + i * VQ_THREADS;
        if (q < LUT_PER_V) {
#pragma unroll 1
            for (int v = 0; v < VC; v++) {
                float a = 0.0f;
#pragma unroll
                for (int d = 0; d < 8; d++) a = __fmaf_rn(xs[v * 8 + d], cv[i][d], a);
                lut[v * LUT_PER_V + q] = a;
            }
        }
    }
    __syncthreads();

    bool unbound = false;
    const int iters = (vhi - vlo + 4 * nw - 1) / (4 * nw);
    for (int it = 0; it < iters; it++) {
        const bool was = live;
        float *o = outp;
        bool ln;
        float *on;
        g_u8 *pn = src_of(vlo + 4 * (wv + (it + 1) * nw) + g, ln, on);
        float acc[4];
#pragma unroll
        for (int k = 0; k < VC; k++) {
            const float *L = lut + k * LUT_PER_V;
            const uint32_t u[3] = {buf[k].x, buf[k].y, buf[k].z};
            buf[k] = *(g_uint3 *)(pn + k * 192);                   // next group, same position
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int b0 = 3 * r, b1 = 3 * r + 1, b2 = 3 * r + 2;
                const uint32_t i0 = (u[b0 >> 2] >> ((b0 & 3) * 8)) & 255;
                const uint32_t i1 = (u[b1 >> 2] >> ((b1 & 3) * 8)) & 255;
                const uint32_t i2 = (u[b2 >> 2] >> ((b2 & 3) * 8)) & 255;
                const float t = (L[i0] + L[256 + i1]) + L[512 + i2];
                acc[r] = k == 0 ? t : acc[r] + t;
            }
        }
        *(float4 *)o = was ? make_float4(acc[0], acc[1], acc[2], acc[3]) : make_float4(0, 0, 0, 0);
        unbound |= !was && o < sink;
        live = ln;
        outp = on;
    }
    if (unbound) atomicOr(err, 1);
}

// Two symbols for one body, so that profiles tell the gate/up pass (two
// kinds per pair, the hidden-wide tables) from the down pass.
#define VQ_KERNEL(NAME)                                                                         \
    __global__ void __launch_bounds__(VQ_THREADS) __attribute__((amdgpu_waves_per_eu(8)))       \
    NAME(const uint8_t *const *__restrict__ recs, const int32_t *__restrict__ pair_exp,         \
         const int32_t *__restrict__ pair_src, const void *__restrict__ src, int src_ld,        \
         int src_bf16, const float *__restrict__ booksT, int cb, uint32_t off0, uint32_t off1,  \
         int kinds, int M, int nv, int nch, int rsplit, int P, int span,                        \
         float *__restrict__ part, int *__restrict__ err)                                       \
    {                                                                                           \
        vq_apply_body(recs, pair_exp, pair_src, src, src_ld, src_bf16, booksT, cb, off0, off1,  \
                      kinds, M, nv, nch, rsplit, P, span, part, err);                           \
    }
VQ_KERNEL(k_vq_rows_gate_up)
VQ_KERNEL(k_vq_rows_down)

#include "vq_tile.h"

// rows row0 + 8w .. of the block's wavefront w into shs (LDS)
template <int FMT>
__device__ __forceinline__ void sh_rows8(const whip_mat &W, const float *x, int row0, int H, float *shs)
{
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    float acc[8];
    sh_rows8_acc<FMT>(W, x, row0 + w * 8, H, lane, acc);
    if (lane == 0)
#pragma unroll
        for (int i = 0; i < 8; i++) shs[w * 8 + i] = acc[i];
}

// Every global load below is unconditional (clamped addresses, selects
// instead of branches): the hardware counts loads in issue order, and a
// load on only one side of a branch leaves the compiler unsure how many are
// in flight, so it would wait for all of them, the prefetched tiles too.
//
// Issue order, so that no wait covers a load it does not need: the pairs'
// records; then the first class's books and x (SPAN: every pair reads
// source row 0) or, for ACT, its gate/up partials (summed as they arrive,
// with the records), staged in LDS; then each wavefront's first tile, which
// flies while the first tables are built; then its second.  Two tiles stay
// in flight per wavefront from there on.  (The small loads the build needs
// are waited for before any tile goes out: sent together, they queue
// behind the launch-wide burst of tile loads, which measured slower.)
#define ACT_PF 8                                     // partials per kind a thread prefetches
template <bool ACT, bool SPAN>
__device__ __forceinline__ void
vq_lanes_body(const whip_vq_args &a, int nch, int tiles, int per_wg, int shares)
{
    __shared__ float smem[2 * 256 * 64];             // table A | table B
    __shared__ float sbook[3 * 8 * 256];             // a kind's books, [stage][dim][code]
    __shared__ const uint8_t *s_rec[SPAN_MAX];       // records of pairs p_lo ..
    __shared__ int s_xr[SPAN_MAX];                   // and their source rows
    __shared__ float s_h[256];                       // x of a class reduced from partials (act_part)
    __shared__ int4 s_cur[2 * LW];                   // tiles t0 + i decoded: (p, kind, chunk, rb)
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int v = lane & 31, h = lane >> 5;
    const int wk = a.kinds == 2 ? 1 : 2;             // trace row of this pass
    WT_DECL;
    WT_KEEP(0);
    tile_map tm;
    tm.span = SPAN; tm.nch = nch; tm.kinds = a.kinds; tm.nb = a.M >> 6;
    tm.tpc = SPAN ? a.P * tm.nb : tm.nb;
    // shares > 0: workgroup = (class, share), a share never leaves its class
    int t0, t1;
    if (shares > 0) {
        // ACT: a class's shares each reduce the class's gate/up partials;
        // with a multiple of eight classes, workgroup w = cls + j * ncls puts
        // them all on XCD cls % 8, where the second to fourth reads are
        // served by that XCD's L2 (workgroup w runs on XCD w % 8)
        const int ncls = gridDim.x / shares;
        const bool xcd = ACT && ncls % 8 == 0;           // uniform
        const int cls = xcd ? blockIdx.x % ncls : blockIdx.x / shares;
        const int j = xcd ? blockIdx.x / ncls : blockIdx.x - cls * shares;
        t0 = cls * tm.tpc + j * per_wg;
        t1 = min(t0 + per_wg, (cls + 1) * tm.tpc);
    } else {
        // runs in tile order.  Without SPAN a run is about one pair's
        // classes, and pairs of one expert are neighbours in the pair order:
        // they read the same index tiles in the same order.  Workgroup w
        // runs on XCD w % 8, so consecutive runs go to one XCD (a bijection
        // of [0, G)); those workgroups start together and the expert's
        // second read is served by that XCD's L2.
        int w = blockIdx.x;
        if (!SPAN) {
            const int G = (tiles + per_wg - 1) / per_wg, x = w & 7;
            w = x * (G >> 3) + min(x, G & 7) + (w >> 3);
        }
        t0 = w * per_wg;
        t1 = min(tiles, t0 + per_wg);
    }
    if (t0 >= t1) return;                            // whole workgroup
    const size_t rstride = (size_t)a.nv * 192;
    const uint32_t bA0 = (h ? 128u : 0u) + 4u * v, bA1 = (h ? 0u : 128u) + 4u * v;
    const uint32_t bB = 65536u + 128u * h + 4u * v;
    const uint32_t s0 = h ? 0x04020001u : 0x03020100u, s1 = h ? 0x06070503u : 0x07060504u;
    const uint32_t s2 = h ? 0x03010200u : 0x03020100u;
    const int rho = 16 * ((v >> 4) & 1) + 8 * ((v >> 3) & 1) + 4 * ((v >> 2) & 1) + 2 * (v & 1) + ((v >> 1) & 1);
    // every address is a wave-uniform base plus one of two per-lane offsets
    const uint32_t loff = v * 192 + h * 96;          // index bytes of a tile
    const uint32_t lrow = 32 * h + rho;              // output row in a block
    g_u8 *dummy = as_global((const uint8_t *)a.booksT);
    float *sink = a.part + (size_t)a.P * a.kinds * nch * a.M;
    int p_lo = 0, p_hi = a.P - 1, u0, u1, u2, p_first, chunk_first;
    if (!SPAN) {                                     // p_hi - p_lo < SPAN_MAX (host)
        tm.at(t0, p_lo, u0, u1, u2);
        tm.at(t1 - 1, p_hi, u0, u1, u2);
    }
    tm.at(t0, p_first, u0, chunk_first, u2);

    auto uni = [](const void *q) -> const uint8_t * {
        const uint64_t u = (uint64_t)q;
        const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
        const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
        return (const uint8_t *)(((uint64_t)hi << 32) | lo);
    };
    // tile t of a class ending at hi -> uniform bases of its index bytes
    // (or the dummy, past the class) and output block
    // (out_sc_off: and the f16 scales of its 64 rows, else the dummy)
    auto where_rec = [&](const tile_cur &c, int hi, const uint8_t *rec, g_u8 *&src, float *&out, bool &live,
                         g_u16 *&scb) {
        scb = (g_u16 *)dummy;
        if (c.t >= hi) { src = dummy; out = sink; live = true; return; }
        const int p = c.p, kind = c.kind, chunk = c.chunk, rb = c.rb;
        live = rec != nullptr;
        src = rec ? as_global(rec) + a.idx_off[kind] + (size_t)rb * rstride + (size_t)chunk * PW * 192 : dummy;
        out = a.part + (((size_t)p * a.kinds + kind) * nch + chunk) * (size_t)a.M + rb * 64;
        if (a.out_sc_off && rec) scb = (g_u16 *)(as_global(rec) + a.out_sc_off) + (size_t)kind * a.M + rb * 64;
    };
    auto where = [&](const tile_cur &c, int hi, g_u8 *&src, float *&out, bool &live, g_u16 *&scb) {
        where_rec(c, hi, c.t < hi ? uni(s_rec[c.p - p_lo]) : nullptr, src, out, live, scb);
    };

    // act_part: x of class (pair p, chunk) is silu(g) * u for the 256
    // rows chunk*256 .. of pair p, g and u the sums of its gate and up
    // partials, which the gate/up launch scaled by their rows' scales (the
    // SwiGLU the separate act kernel does).  Thread (row i, quarter q) sums a quarter of the chunks of both
    // kinds, the first ACT_PF of them with the class's other loads (summed
    // at once, before any tile is in flight); the quarters meet in LDS (the
    // tables' space, rebuilt next).
    // thread = (row a_i, quarter a_q): the quarter and the row's 64-row
    // group are wavefront-uniform, so every partial address is a scalar
    // base plus the lane's offset (few vector registers)
    const int a_q = wv >> 2, a_g = (wv & 3) * 64, a_i = a_g + lane;
    auto act_range = [&](int &c_lo, int &c_hi) {
        const int nc = a.act_nch, ns = (nc + 3) / 4;
        c_lo = min(nc, a_q * ns);
        c_hi = min(nc, c_lo + ns);
    };
    float sg0 = 0.0f, su0 = 0.0f;                    // sums of the prefetched partials
    auto act_loads = [&](int p, int chunk) {
        const int I = a.nv * 8, nc = a.act_nch;
        int c_lo, c_hi;
        act_range(c_lo, c_hi);
        const float *pgp = a.act_part + (size_t)p * 2 * nc * I + chunk * 256 + a_g;
        float pg[ACT_PF], pu[ACT_PF];
#pragma unroll
        for (int k = 0; k < ACT_PF; k++) {
            const int c = c_lo + k < c_hi ? c_lo + k : 0;
            pg[k] = (pgp + (size_t)c * I)[lane];
            pu[k] = (pgp + (size_t)(nc + c) * I)[lane];
        }
        sg0 = su0 = 0.0f;
#pragma unroll
        for (int k = 0; k < ACT_PF; k++)
            if (c_lo + k < c_hi) { sg0 += pg[k]; su0 += pu[k]; }
    };
    auto act_x = [&](int p, int chunk) {
        const int I = a.nv * 8, nc = a.act_nch;
        int c_lo, c_hi;
        act_range(c_lo, c_hi);
        const float *pgp = a.act_part + (size_t)p * 2 * nc * I + chunk * 256 + a_g;
        float sg = sg0, su = su0;
        for (int c = c_lo + ACT_PF; c < c_hi; c++) {  // past the prefetched ones (rare)
            sg += (pgp + (size_t)c * I)[lane];
            su += (pgp + (size_t)(nc + c) * I)[lane];
        }
        const bool live = s_rec[p - p_lo] != nullptr;
        __syncthreads();                             // the old tables' readers are done
        smem[(a_q * 256 + a_i) * 2] = sg;
        smem[(a_q * 256 + a_i) * 2 + 1] = su;
        __syncthreads();
        if (wv < 4) {
            float gg = 0.0f, uu = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; k++) { gg += smem[(k * 256 + a_i) * 2]; uu += smem[(k * 256 + a_i) * 2 + 1]; }
            s_h[a_i] = live ? wh_silu_mul(gg, uu) : 0.0f;
        }
        __syncthreads();
    };

    // the build's loads for the class of tile t: the kind's books and x
    // (or, for ACT, the class's partials)
    float bv[3 * 8 * 256 / LT];
    uint4 xq0, xq1;
    auto build_loads = [&](int t, int xr) {
        int p, kind, chunk, rb;
        tm.at(t, p, kind, chunk, rb);
        const float *bk = a.booksT + (size_t)(a.cb + kind * 3) * 8 * 256;
#pragma unroll
        for (int i = 0; i < 3 * 8 * 256 / LT; i++) bv[i] = bk[tid + i * LT];
        if (ACT) {
            act_loads(p, chunk);
            return;
        }
        if (wv == 0) {                               // uniform: the wavefront that stages x
            const size_t e0 = (size_t)xr * a.src_ld + (size_t)(chunk * PW + v) * 8;
            const uint8_t *xb = (const uint8_t *)a.src + e0 * (a.src_bf16 ? 2 : 4);
            xq0 = *(const uint4 *)xb;
            xq1 = *(const uint4 *)(xb + (a.src_bf16 ? 0 : 16));
        }
    };
    // The build in two steps.  stage: the books to LDS and the class's x
    // (converted, or for ACT reduced from the partials) to s_h, both LDS
    // writes, which the compiler cannot move past the barrier that follows,
    // so the tiles' loads go out after the build's own have arrived.
    // tables: 24 products of 32 codes x 32 positions on the matrix cores
    // (books[code][dim] x x[dim][position]).
    auto stage = [&](int t) {
#pragma unroll
        for (int i = 0; i < 3 * 8 * 256 / LT; i++) sbook[tid + i * LT] = bv[i];
        if (ACT) {
            int p, kind, chunk, rb;
            tm.at(t, p, kind, chunk, rb);
            act_x(p, chunk);                         // ends with a barrier
        } else {
            if (wv == 0) {                           // uniform: only wavefront 0 loaded x
                const uint32_t w8[8] = {xq0.x, xq0.y, xq0.z, xq0.w, xq1.x, xq1.y, xq1.z, xq1.w};
                float xv[8];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float lo16 = wh_bf16(w8[i] & 0xffff), hi16 = wh_bf16(w8[i] >> 16);
                    xv[2 * i] = a.src_bf16 ? lo16 : __uint_as_float(w8[2 * i]);
                    xv[2 * i + 1] = a.src_bf16 ? hi16 : __uint_as_float(w8[2 * i + 1]);
                }
                if (lane < 32) {
#pragma unroll
                    for (int k = 0; k < 8; k++) s_h[v * 8 + k] = xv[k];
                }
            }
            __syncthreads();
        }
    };
    // x of this lane's position as bf16 pieces: bf16 activations are one
    // exact piece; fp32 ones (and the down pass's SwiGLU) three
    const bool x3 = ACT || !a.src_bf16;
    auto tables = [&]() {
        float xv[8];
#pragma unroll
        for (int k = 0; k < 8; k++) xv[k] = s_h[v * 8 + k];
        uint4 xb[3];
        split3(xv, xb[0], xb[1], xb[2]);
        table_mfma(smem, sbook, xb[0], xb[1], xb[2], x3, wv, lane);
        WT_KEEP(4);
        __syncthreads();
    };

    tile_buf A, B;
    g_u8 *src;
    g_u16 *scb;
    float *outA, *outB;
    uint16_t scA, scB;                               // the lane's row scale of each tile
    bool liveA, liveB, unbound = false;
    const bool presc = a.out_sc_off != 0;            // uniform
    tile_cur cA, cB;                                 // the tiles buffers A and B hold
    // A run inside one class (shares > 0) is walked interleaved: wavefront
    // wv takes tiles t0 + wv + LW j.  A run across classes is walked in
    // pairs of adjacent row blocks (t, t + 1), t = t0 + 2 wv + 2 LW k: its
    // classes and its length are even (host), so no pair straddles two
    // classes and A and B stay in step across the classes.
    const bool paired = shares == 0;                 // uniform
    const int d1 = paired ? 2 : 1, d2 = paired ? 1 : LW;
    // prologue: the records (one load each: the router wrote them, else
    // through the pair's expert), then the first build's loads
    {
        const int q = p_lo + min(tid, p_hi - p_lo);
        const int32_t *psrc = a.pair_src ? a.pair_src : a.pair_exp;
        const uint8_t *myrec;
        int xq, xf = 0;
        if (a.pair_rec) {
            myrec = a.pair_rec[q];
            xq = psrc[q];
            if (!(ACT || SPAN)) xf = psrc[p_first];
        } else {
            const int e = a.pair_exp[q];
            xq = psrc[q];
            if (!(ACT || SPAN)) xf = psrc[p_first];
            myrec = a.recs[e];
        }
        const int myxr = a.pair_src ? xq : q;
        build_loads(t0, (ACT || SPAN) ? 0 : (a.pair_src ? xf : p_first));
        if (tid <= p_hi - p_lo) { s_rec[tid] = myrec; s_xr[tid] = myxr; }
        if (tid < 2 * LW) {                          // each wavefront's first two tiles
            int cp, ck, cc, cr;
            tm.at(t0 + tid, cp, ck, cc, cr);
            s_cur[tid] = make_int4(cp, ck, cc, cr);
        }
    }
    WT_KEEP(5);
    __syncthreads();
    stage(t0);
    WT_KEEP(1);
    int t = t0 + d1 * wv;
    {
        const int4 qa = s_cur[d1 * wv], qb = s_cur[d1 * wv + d2];
        cA.t = t; cA.p = __builtin_amdgcn_readfirstlane(qa.x); cA.kind = __builtin_amdgcn_readfirstlane(qa.y);
        cA.chunk = __builtin_amdgcn_readfirstlane(qa.z); cA.rb = __builtin_amdgcn_readfirstlane(qa.w);
        cB.t = t + d2; cB.p = __builtin_amdgcn_readfirstlane(qb.x); cB.kind = __builtin_amdgcn_readfirstlane(qb.y);
        cB.chunk = __builtin_amdgcn_readfirstlane(qb.z); cB.rb = __builtin_amdgcn_readfirstlane(qb.w);
    }
    // A holds the wavefront's next tile, B the one after.  After each tile,
    // the tile two ahead goes out into the buffer it freed (the dummy past
    // the run): across classes, a class's first pair is in flight while its
    // tables are built.  The buffers never trade contents: that would be a
    // register copy, which waits for the loads in flight.
    //
    // Order at the start, measured on the batch-1 launch timelines: the
    // build's inputs go out first and are staged (a tile sent ahead of them
    // delays them by the whole launch's first burst: every wavefront's
    // loads come back in issue order, and the first tiles of 224 workgroups
    // fill the memory system); then the first tile goes out, the first
    // tables are built while it flies, and only then the second tile.  With
    // both tiles sent before the build, wavefronts stall issuing the second
    // tile's loads and the barrier after the build waits for them: tables
    // ready 9.3 us into the gate/up launch instead of 5.5.
    where(cA, t1, src, outA, liveA, scb);
    load_tile(A, src, loff);
    scA = scb[presc ? lrow : 0];
    tables();                                        // the first class's
    WT_KEEP(3);
    where(cB, t1, src, outB, liveB, scb);
    load_tile(B, src, loff);
    scB = scb[presc ? lrow : 0];
    WT_KEEP(2);
    // A run across classes: the next class's build inputs go out at the
    // start of a class, ahead of the reloads that bring the next class's
    // tiles, so at the class boundary they have landed and the build waits
    // for nothing in flight.  (ACT: at the boundary; its inputs are summed
    // as they arrive.)
    for (int lo = t0; lo < t1;) {
        const int hi = min(t1, (lo / tm.tpc + 1) * tm.tpc);
        if (lo > t0) {                               // uniform
            if (ACT) {
                int pn, k_, c_, r_;
                tm.at(lo, pn, k_, c_, r_);
                build_loads(lo, s_xr[pn - p_lo]);
            }
            __syncthreads();                         // the old tables and s_h are done with
            stage(lo);
            tables();
        }
        if (!ACT && hi < t1) {                       // uniform
            int pn, k_, c_, r_;
            tm.at(hi, pn, k_, c_, r_);
            build_loads(hi, s_xr[pn - p_lo]);
        }
        // A counted loop of pairs and an odd tile after it: an exit in the
        // middle of a round leaves the compiler unsure which loads are in
        // flight at the loop's head, and it then waits for all of them.
        // Only a single-class run has an odd count (its last class).
        const int n = t >= hi ? 0 : paired ? 2 * ((hi - t + 2 * LW - 1) / (2 * LW)) : (hi - t + LW - 1) / LW;
        for (int i = 0; i + 1 < n; i += 2) {
            float r = tile_sum(A, smem, bA0, bA1, bB, s0, s1, s2, lane);
#ifdef WH_TRACE
            if (lo == t0 && i == 0) WT_KEEP(6);
#endif
            r = presc ? __fmul_rn(r, wh_f16_scale(scA)) : r;
            __builtin_nontemporal_store(liveA ? r : 0.0f, outA + lrow);
            unbound |= !liveA;
            cA.step(tm, a.P, 2 * LW);
            where(cA, t1, src, outA, liveA, scb);
            load_tile(A, src, loff);
            scA = scb[presc ? lrow : 0];
            __builtin_amdgcn_sched_barrier(0);       // the reload goes out before B's tile is read
            r = tile_sum(B, smem, bA0, bA1, bB, s0, s1, s2, lane);
            r = presc ? __fmul_rn(r, wh_f16_scale(scB)) : r;
            __builtin_nontemporal_store(liveB ? r : 0.0f, outB + lrow);
            unbound |= !liveB;
            cB.step(tm, a.P, 2 * LW);
            where(cB, t1, src, outB, liveB, scb);
            load_tile(B, src, loff);
            scB = scb[presc ? lrow : 0];
            __builtin_amdgcn_sched_barrier(0);
        }
        if (n & 1) {
            float r = tile_sum(A, smem, bA0, bA1, bB, s0, s1, s2, lane);
            r = presc ? __fmul_rn(r, wh_f16_scale(scA)) : r;
            __builtin_nontemporal_store(liveA ? r : 0.0f, outA + lrow);
            unbound |= !liveA;
        }
        t += n * LW;
        lo = hi;
    }
    WT(wk, 6 + wv);
    if (wv == 0) { WT_PUT(wk, 0); WT_PUT(wk, 1); WT_PUT(wk, 2); WT_PUT(wk, 3); WT_PUT(wk, 4); WT_PUT(wk, 5); }
#ifdef WH_TRACE
    if (wv == 0 && lane == 0) wt_buf[(wk * 256 + (blockIdx.x & 255)) * WT_SLOTS + 22] = wt_keep_[6];
#endif
    if (unbound) atomicOr(a.err, 1);
}

// The gate/up launch's workgroups past its tile workgroups (g of NG) run
// the shared expert's down projection, which needs only the launch before
// (h_sh), on CUs the tiles leave idle: rows in groups of eight, one group
// per wavefront at a time.
template <int FMT>
__device__ __forceinline__ void shd_role(const whip_vq_args &a, int g, int NG)
{
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int H = a.shd.rows, ngr = (H + 7) / 8;
    for (int rg = g * LW + wv; rg < ngr; rg += NG * LW) {   // wave-uniform
        float acc[8];
        sh_rows8_acc<FMT>(a.shd, a.shd_x, rg * 8, H, lane, acc);
        if (lane == 0)
#pragma unroll
            for (int i = 0; i < 8; i++)
                if (rg * 8 + i < H) a.shd_y[rg * 8 + i] = acc[i];
    }
}

// Separate symbols, so that profiles tell the gate/up pass from the down
// pass.  SPAN: one token, every pair reads source row 0.  Workgroups from
// g_vq on take the shared down projection (a.shd_y set).
template <bool SPAN>
__global__ void __launch_bounds__(LT)
k_vq_gate_up(whip_vq_args a, int nch, int tiles, int per_wg, int shares, int g_vq)
{
    if ((int)blockIdx.x >= g_vq) {                   // uniform
        const int g = blockIdx.x - g_vq, NG = gridDim.x - g_vq;
        if (a.shd.fmt == 3) shd_role<3>(a, g, NG);
        else if (a.shd.fmt == 2) shd_role<2>(a, g, NG);
        else shd_role<0>(a, g, NG);
        return;
    }
    vq_lanes_body<false, SPAN>(a, nch, tiles, per_wg, shares);
}

__global__ void __launch_bounds__(LT)
k_vq_down(whip_vq_args a, int nch, int tiles, int per_wg, int shares)
{
    vq_lanes_body<false, false>(a, nch, tiles, per_wg, shares);
}

// The down pass with SwiGLU of the gate/up partials in its table build.
__global__ void __launch_bounds__(LT)
k_vq_act_down(whip_vq_args a, int nch, int tiles, int per_wg, int shares)
{
    vq_lanes_body<true, false>(a, nch, tiles, per_wg, shares);
}

extern "C" int whip_vq_apply(const whip_vq_args *a, hipStream_t s)
{
    // whole row blocks and chunks; 4-byte aligned index streams; a spanning
    // launch covers every pair (all read one source row)
    const int span = a->span > 1 ? a->span : 1;
    const int rows = (a->M / 64) * (span > 1 ? a->P : 1);
    if (a->M <= 0 || a->M % 64 || a->nv <= 0 || a->nv % VC || a->idx_off[0] % 4 || a->idx_off[1] % 4 ||
        a->P < 1 || a->rsplit < 1 || a->rsplit > rows || (span > 1 && (span != a->P || span > SPAN_MAX)))
        return (int)hipErrorInvalidValue;
    const int nch = whip_vq_chunks(a->nv, a->M);
    if (a->act_part && (!(LANES_OK(a->nv, a->M)) || a->act_nch < 1 || a->kinds != 1 || span > 1))
        return (int)hipErrorInvalidValue;
    if (a->out_sc_off && (!(LANES_OK(a->nv, a->M)) || a->out_sc_off % 2))
        return (int)hipErrorInvalidValue;
    if (a->shd_y) {
        // the gate/up pass of the tile kernel only; whole 16-byte chunks
        const whip_mat *d = &a->shd;
        if (a->kinds != 2 || !(LANES_OK(a->nv, a->M)) || !a->shd_x || (uintptr_t)a->shd_x % 16 ||
            d->rows < 1 || d->rowbytes % 16 || (d->fmt != 0 && d->fmt != 2 && d->fmt != 3) ||
            (d->fmt != 0 && (d->group % 32 || d->cols % 8)) || (d->fmt == 0 && d->cols % 4))
            return (int)hipErrorInvalidValue;
    }
    if (LANES_OK(a->nv, a->M)) {
        // 16-byte aligned tiles (the kernel's 128-bit loads)
        if (a->idx_off[0] % 16 || a->idx_off[1] % 16) return (int)hipErrorInvalidValue;
        static int n_cu = 0;
        if (!n_cu) {
            int dev = 0;
            if (hipGetDevice(&dev) != hipSuccess ||
                hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu < 1)
                n_cu = 256;
        }
        const int nb = a->M / 64, sp = span > 1;
        const long tpc = sp ? (long)a->P * nb : nb;
        const long classes = (long)a->kinds * nch * (sp ? 1 : a->P);
        const long tiles = classes * tpc;
        if (tiles > (1L << 30)) return (int)hipErrorInvalidValue;
        long G, per_wg, shares = 0;
        if (classes <= n_cu) {
            // whole classes: `shares` workgroups per class, one build each
            const long k = n_cu / classes;
            per_wg = (tpc + k - 1) / k;
            shares = (tpc + per_wg - 1) / per_wg;
            G = classes * shares;
        } else {
            // runs across classes: an even number of tiles (the kernel's
            // tile pairs; every class is even, M % 128 == 0)
            per_wg = (tiles + n_cu - 1) / n_cu;
            per_wg += per_wg & 1;
            G = (tiles + per_wg - 1) / per_wg;
        }
        // a workgroup's records fit its table (at most SPAN_MAX pairs)
        const long tiles_per_pair = sp ? tiles : (long)a->kinds * nch * nb;
        if (!sp && shares == 0 && per_wg > (long)(SPAN_MAX - 1) * tiles_per_pair) {
            per_wg = (long)(SPAN_MAX - 1) * tiles_per_pair;
            G = (tiles + per_wg - 1) / per_wg;
        }
        // the shared down projection on the CUs the tiles leave (at least
        // eight workgroups, which then run where tiles finish first)
        const long roles = a->shd_y ? (n_cu - G > 8 ? n_cu - G : 8) : 0;
        if (a->kinds == 2 && sp)
            WHIP_LAUNCH(k_vq_gate_up<true>, dim3((unsigned)(G + roles)), dim3(LT), 0, s, *a, nch, (int)tiles,
                        (int)per_wg, (int)shares, (int)G);
        else if (a->kinds == 2)
            WHIP_LAUNCH(k_vq_gate_up<false>, dim3((unsigned)(G + roles)), dim3(LT), 0, s, *a, nch, (int)tiles,
                        (int)per_wg, (int)shares, (int)G);
        else if (a->act_part)
            WHIP_LAUNCH(k_vq_act_down, dim3((unsigned)G), dim3(LT), 0, s, *a, nch, (int)tiles,
                        (int)per_wg, (int)shares);
        else
            WHIP_LAUNCH(k_vq_down, dim3((unsigned)G), dim3(LT), 0, s, *a, nch, (int)tiles,
                        (int)per_wg, (int)shares);
        return (int)hipGetLastError();
    }
    dim3 grid(nch, a->kinds * a->rsplit, span > 1 ? 1 : a->P);
    hipLaunchKernelGGL(a->kinds == 2 ? k_vq_rows_gate_up : k_vq_rows_down, grid, dim3(VQ_THREADS), 0, s, a->recs,
                       a->pair_exp, a->pair_src, a->src, a->src_ld, a->src_bf16, a->booksT, a->cb,
                       a->idx_off[0], a->idx_off[1], a->kinds, a->M, a->nv, nch, a->rsplit, a->P, span,
                       a->part, a->err);
    return (int)hipGetLastError();
}

// ---- SwiGLU over the reduced gate/up partials ------------------------------
// A workgroup owns 64 rows of one pair: thread (slice, row group of 4) sums
// its slice of the chunk partials for gate and up with every load in flight
// (clamped addresses, no branches around loads); the slices then meet in
// chunk order through LDS.
#define ACT_ROWS 64
#define ACT_SLICES 16
#define RED_BATCH 8

// sum of partial rows [c0, c1) of a [nch][ld] block at column r0 (float4)
__device__ __forceinline__ float4 sum_chunks(const float *__restrict__ base, size_t ld, int c0, int c1)
{
    float4 acc = make_float4(0, 0, 0, 0);
    for (int cb = c0; cb < c1; cb += RED_BATCH) {
        float4 v[RED_BATCH];
#pragma unroll
        for (int k = 0; k < RED_BATCH; k++) {
            const int c = cb + k < c1 ? cb + k : c0;
            v[k] = *(const float4 *)(base + (size_t)c * ld);
        }
#pragma unroll
        for (int k = 0; k < RED_BATCH; k++)
            if (cb + k < c1) { acc.x += v[k].x; acc.y += v[k].y; acc.z += v[k].z; acc.w += v[k].w; }
    }
    return acc;
}

__global__ void __launch_bounds__(256)
k_vq_act(const uint8_t *const *__restrict__ recs, const int32_t *__restrict__ pair_exp,
         const float *__restrict__ part, int nch, int I, uint32_t sc_off, float *__restrict__ h)
{
    __shared__ float4 red[2][ACT_SLICES][ACT_ROWS / 4];
    const int p = blockIdx.y, tid = threadIdx.x;
    const int g = tid & (ACT_ROWS / 4 - 1), sl = tid / (ACT_ROWS / 4);
    const int r0 = blockIdx.x * ACT_ROWS + g * 4;
    const int per = (nch + ACT_SLICES - 1) / ACT_SLICES;
    const int c0 = min(nch, sl * per), c1 = min(nch, c0 + per);
    // the record (uniform per workgroup) and this row group's scales are
    // fetched before the partials, so they are in hand after the barrier
    const uint8_t *rec = recs[pair_exp[p]];
    uint16_t rsg[4] = {0, 0, 0, 0}, rsu[4] = {0, 0, 0, 0};
    if (rec && r0 < I) {
        g_u16 *sc = (g_u16 *)(as_global(rec) + sc_off);
#pragma unroll
        for (int q = 0; q < 4; q++) { rsg[q] = sc[r0 + q]; rsu[q] = sc[I + r0 + q]; }
    }
    float4 sg = make_float4(0, 0, 0, 0), su = sg;
    if (r0 < I) {
        sg = sum_chunks(part + ((size_t)p * 2 + 0) * nch * (size_t)I + r0, I, c0, c1);
        su = sum_chunks(part + ((size_t)p * 2 + 1) * nch * (size_t)I + r0, I, c0, c1);
    }
    red[0][sl][g] = sg;
    red[1][sl][g] = su;
    __syncthreads();
    if (tid >= ACT_ROWS / 4 || r0 >= I) return;
    float gg[4] = {0, 0, 0, 0}, uu[4] = {0, 0, 0, 0};
    for (int k = 0; k < ACT_SLICES; k++) {
        const float4 a = red[0][k][g], b = red[1][k][g];
        gg[0] += a.x; gg[1] += a.y; gg[2] += a.z; gg[3] += a.w;
        uu[0] += b.x; uu[1] += b.y; uu[2] += b.z; uu[3] += b.w;
    }
    float out[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const float sgc = rec ? wh_f16_scale(rsg[q]) : 0.0f, suc = rec ? wh_f16_scale(rsu[q]) : 0.0f;
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
// A workgroup owns 32 output rows of one token.  Work item (pair slot j,
// chunk slice) of a row group of 4 sums its slice of pair j's down partials;
// items are spread over the workgroup's threads so that every load of a
// thread is in flight at once.  Then the first threads add, per row group,
// the slices of each pair, scale by f16(scale) and the route weight, and add
// the pairs in the token's combine order, then the shared expert.
#define CMB_ROWS 32
#define CMB_SLICES 4

// One (pair j, chunk slice sl) of a combine block: the slice's partial sums
// of four rows, the rows' scales, the pair's weight and whether it counts.
// One token (T == 1): pair j is the token's j-th pair (the routing's order),
// so no load stands before the weight's and the partials'.  sc_off_down 0:
// the down launch scaled its partials already (no record or scale loads;
// an unbound expert's partials are zeros).  The loads do not wait for the
// record: every address is valid.
//
// FOLD (1: a product and a sum, 2: one fused multiply-add): the pairs' down
// rows are VQ4P block sums instead of partials, folded here in block order
// by slice 0 (whip_fold); the other slices hold zeros.
template <bool FMA>
__device__ __forceinline__ float4 p6_fold4(const whip_fold &f, int p, int r, int H, const uint8_t *rec)
{
    const int16_t *S = f.S + (size_t)p * f.nb * H + r;
    const float *ls = f.ls + (size_t)p * f.nb;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 8
    for (int b = 0; b < f.nb; b++) {
        const uint2 w = *(const uint2 *)(S + (size_t)b * H);
        const float l = ls[b];
        const float s4[4] = {(float)(int16_t)(w.x & 0xffff), (float)(int16_t)(w.x >> 16),
                             (float)(int16_t)(w.y & 0xffff), (float)(int16_t)(w.y >> 16)};
#pragma unroll
        for (int k = 0; k < 4; k++) acc[k] = FMA ? __fmaf_rn(l, s4[k], acc[k]) : __fadd_rn(acc[k], __fmul_rn(l, s4[k]));
    }
    if (rec == nullptr) return make_float4(0.0f, 0.0f, 0.0f, 0.0f);   // unbound: zeros
    const uint16_t *sc = (const uint16_t *)(rec + f.sc_off) + r;
    return make_float4(__fmul_rn(acc[0], wh_f16_scale(sc[0])), __fmul_rn(acc[1], wh_f16_scale(sc[1])),
                       __fmul_rn(acc[2], wh_f16_scale(sc[2])), __fmul_rn(acc[3], wh_f16_scale(sc[3])));
}

template <int FOLD>
__device__ __forceinline__ void
cmb_gather(const uint8_t *const *__restrict__ recs, const int32_t *__restrict__ pair_exp,
           const float *__restrict__ pair_w, const int32_t *__restrict__ tok_pairs, int K,
           const float *__restrict__ part_d, const whip_fold &f, int nch, int H, uint32_t sc_off_down,
           int skip_zero, int t, int it, int g, int r0, int per, float4 *cred, float4 *csc, float *cw, int *cl)
{
    constexpr int G = CMB_ROWS / 4;
    const int j = it / CMB_SLICES, sl = it % CMB_SLICES;
    const int p = gridDim.y == 1 ? j : tok_pairs[t * K + j];
    const float wj = pair_w[p];
    const int rr = r0 < H ? r0 : 0;
    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (FOLD) {
        if (sl == 0) v = p6_fold4<FOLD == 2>(f, p, rr, H, recs[pair_exp[p]]);
    } else {
        const int c0 = min(nch, sl * per), c1 = min(nch, c0 + per);
        v = sum_chunks(part_d + (size_t)p * nch * H + rr, H, c0, c1);
    }
    bool live = !(skip_zero && wj == 0.0f);          // else the pair adds nothing
    float4 scv = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
    if (sc_off_down) {                               // uniform
        const uint8_t *rec = recs[pair_exp[p]];
        live = live && rec;
        uint16_t rs[4] = {0, 0, 0, 0};
        if (sl == 0 && rec) {
            g_u16 *sc = (g_u16 *)(as_global(rec) + sc_off_down) + rr;
#pragma unroll
            for (int q = 0; q < 4; q++) rs[q] = sc[q];
        }
        scv = make_float4(wh_f16_scale(rs[0]), wh_f16_scale(rs[1]), wh_f16_scale(rs[2]), wh_f16_scale(rs[3]));
    }
    if (!live || r0 >= H) v = make_float4(0, 0, 0, 0);
    cred[(j * CMB_SLICES + sl) * G + g] = v;
    if (sl == 0) {
        csc[j * G + g] = scv;
        if (g == 0) { cw[j] = wj; cl[j] = live; }
    }
}

template <int FOLD>
__global__ void __launch_bounds__(256)
k_combine(const uint8_t *const *__restrict__ recs, const int32_t *__restrict__ pair_exp,
          const float *__restrict__ pair_w, const int32_t *__restrict__ tok_pairs, int K,
          const float *__restrict__ part_d, whip_fold f, int nch, int H, uint32_t sc_off_down,
          int skip_zero, const float *__restrict__ sh, int sh_n, size_t sh_stride, float *__restrict__ y)
{
    // [K][CMB_SLICES][G] slice sums, [K][G] row scales, [K] weights, [K] live
    extern __shared__ float4 cred[];
    constexpr int G = CMB_ROWS / 4;
    float4 *csc = cred + K * CMB_SLICES * G;
    float *cw = (float *)(csc + K * G);
    int *cl = (int *)(cw + K);
    const int t = blockIdx.y, tid = threadIdx.x;
    const int g = tid % G;
    const int r0 = blockIdx.x * CMB_ROWS + g * 4;
    const int per = (nch + CMB_SLICES - 1) / CMB_SLICES;
    WT_SPAN(3, 0);
    // the shared expert's slices, summed in order while the gathers fly
    float4 shv = make_float4(0, 0, 0, 0);
    const bool has_sh = sh != nullptr;
    if (has_sh && tid < G && r0 < H) {
        const float *shr = sh + (size_t)t * H + r0;
        shv = *(const float4 *)shr;
        for (int q = 1; q < sh_n; q++) {
            const float4 v = *(const float4 *)(shr + (size_t)q * sh_stride);
            shv.x = __fadd_rn(shv.x, v.x); shv.y = __fadd_rn(shv.y, v.y);
            shv.z = __fadd_rn(shv.z, v.z); shv.w = __fadd_rn(shv.w, v.w);
        }
    }
    for (int it = tid / G; it < K * CMB_SLICES; it += 256 / G)
        cmb_gather<FOLD>(recs, pair_exp, pair_w, tok_pairs, K, part_d, f, nch, H, sc_off_down, skip_zero, t, it,
                         g, r0, per, cred, csc, cw, cl);
    __syncthreads();
    WT_SPAN(3, 1);
    if (tid >= G || r0 >= H) return;
    float o[4] = {0, 0, 0, 0};
    for (int j = 0; j < K; j++) {                    // combine order
        if (!cl[j]) continue;                        // unbound, or a skipped zero weight
        const float wj = cw[j];
        float sum[4] = {0, 0, 0, 0};
        for (int sl = 0; sl < CMB_SLICES; sl++) {
            const float4 a = cred[(j * CMB_SLICES + sl) * G + g];
            sum[0] += a.x; sum[1] += a.y; sum[2] += a.z; sum[3] += a.w;
        }
        const float4 sc = csc[j * G + g];
        o[0] = __fadd_rn(o[0], __fmul_rn(wj, __fmul_rn(sum[0], sc.x)));
        o[1] = __fadd_rn(o[1], __fmul_rn(wj, __fmul_rn(sum[1], sc.y)));
        o[2] = __fadd_rn(o[2], __fmul_rn(wj, __fmul_rn(sum[2], sc.z)));
        o[3] = __fadd_rn(o[3], __fmul_rn(wj, __fmul_rn(sum[3], sc.w)));
    }
    float4 r;
    r.x = __fadd_rn(o[0], shv.x);
    r.y = __fadd_rn(o[1], shv.y);
    r.z = __fadd_rn(o[2], shv.z);
    r.w = __fadd_rn(o[3], shv.w);
    *(float4 *)(y + (size_t)t * H + r0) = r;
}


template <int FMT, int FOLD>
__global__ void __launch_bounds__(256)
k_combine_sh(const uint8_t *const *__restrict__ recs, const int32_t *__restrict__ pair_exp,
             const float *__restrict__ pair_w, const int32_t *__restrict__ tok_pairs, int K,
             const float *__restrict__ part_d, whip_fold f, int nch, int H, uint32_t sc_off_down, int skip_zero,
             whip_mat shd, const float *__restrict__ h_sh, float *__restrict__ y)
{
    extern __shared__ float4 cred[];
    __shared__ float shs[CMB_ROWS];
    constexpr int G = CMB_ROWS / 4;
    float4 *csc = cred + K * CMB_SLICES * G;
    float *cw = (float *)(csc + K * G);
    int *cl = (int *)(cw + K);
    const int t = blockIdx.y, tid = threadIdx.x;
    const int g = tid % G;
    const int r0 = blockIdx.x * CMB_ROWS + g * 4;
    const int per = (nch + CMB_SLICES - 1) / CMB_SLICES;
    WT_SPAN(3, 0);
    sh_rows8<FMT>(shd, h_sh + (size_t)t * shd.cols, blockIdx.x * CMB_ROWS, H, shs);
    for (int it = tid / G; it < K * CMB_SLICES; it += 256 / G)
        cmb_gather<FOLD>(recs, pair_exp, pair_w, tok_pairs, K, part_d, f, nch, H, sc_off_down, skip_zero, t, it,
                         g, r0, per, cred, csc, cw, cl);
    __syncthreads();
    if (tid >= G || r0 >= H) return;
    float o[4] = {0, 0, 0, 0};
    for (int j = 0; j < K; j++) {                    // combine order
        if (!cl[j]) continue;
        const float wj = cw[j];
        float sum[4] = {0, 0, 0, 0};
        for (int sl = 0; sl < CMB_SLICES; sl++) {
            const float4 a = cred[(j * CMB_SLICES + sl) * G + g];
            sum[0] += a.x; sum[1] += a.y; sum[2] += a.z; sum[3] += a.w;
        }
        const float4 sc = csc[j * G + g];
        o[0] = __fadd_rn(o[0], __fmul_rn(wj, __fmul_rn(sum[0], sc.x)));
        o[1] = __fadd_rn(o[1], __fmul_rn(wj, __fmul_rn(sum[1], sc.y)));
        o[2] = __fadd_rn(o[2], __fmul_rn(wj, __fmul_rn(sum[2], sc.z)));
        o[3] = __fadd_rn(o[3], __fmul_rn(wj, __fmul_rn(sum[3], sc.w)));
    }
    float4 r;
    r.x = __fadd_rn(o[0], shs[g * 4 + 0]);
    r.y = __fadd_rn(o[1], shs[g * 4 + 1]);
    r.z = __fadd_rn(o[2], shs[g * 4 + 2]);
    r.w = __fadd_rn(o[3], shs[g * 4 + 3]);
    *(float4 *)(y + (size_t)t * H + r0) = r;
    WT_SPAN(3, 1);
}

WT_READER(whip_trace_vq)

// fold: the VQ4P block sums in place of part_d (nch 1, sc_off_down 0)
static int combine_sh(const uint8_t *const *recs, const int32_t *pair_exp, const float *pair_w,
                      const int32_t *tok_pairs, int T, int K, const float *part_d, const whip_fold *fold, int nch,
                      int H, uint32_t sc_off_down, int skip_zero, const whip_mat *shd, const float *h_sh, float *y,
                      hipStream_t s)
{
    if (H % 4 || K < 1 || K > 64 || shd->rows != H || (uintptr_t)h_sh % 16 || shd->rowbytes % 16 ||
        (shd->fmt != 0 && (shd->group % 32 || shd->cols % 8)) || (shd->fmt == 0 && shd->cols % 4) ||
        (shd->fmt != 0 && shd->fmt != 2 && shd->fmt != 3))
        return (int)hipErrorInvalidValue;
    const whip_fold f = fold ? *fold : whip_fold{};
    const int fm = fold ? (fold->fma ? 2 : 1) : 0;
    dim3 grid((H + CMB_ROWS - 1) / CMB_ROWS, T);
    const size_t lds = (size_t)K * (CMB_SLICES + 1) * (CMB_ROWS / 4) * sizeof(float4) + (size_t)K * 8;
#define CS(F, D) WHIP_LAUNCH((k_combine_sh<F, D>), grid, dim3(256), lds, s, recs, pair_exp, pair_w, tok_pairs, K, \
                             part_d, f, nch, H, sc_off_down, skip_zero, *shd, h_sh, y)
#define CSF(F) do { if (fm == 2) CS(F, 2); else if (fm == 1) CS(F, 1); else CS(F, 0); } while (0)
    if (shd->fmt == 3) CSF(3);
    else if (shd->fmt == 2) CSF(2);
    else CSF(0);
#undef CSF
#undef CS
    return (int)hipGetLastError();
}

static int combine(const uint8_t *const *recs, const int32_t *pair_exp, const float *pair_w,
                   const int32_t *tok_pairs, int T, int K, const float *part_d, const whip_fold *fold, int nch, int H,
                   uint32_t sc_off_down, int skip_zero, const float *sh, int sh_n, size_t sh_stride, float *y,
                   hipStream_t s)
{
    if (H % 4 || K < 1 || K > 64 || (sh && (sh_n < 1 || sh_stride % 4 || (uintptr_t)sh % 16)))
        return (int)hipErrorInvalidValue;
    const whip_fold f = fold ? *fold : whip_fold{};
    const int fm = fold ? (fold->fma ? 2 : 1) : 0;
    dim3 grid((H + CMB_ROWS - 1) / CMB_ROWS, T);
    const size_t lds = (size_t)K * (CMB_SLICES + 1) * (CMB_ROWS / 4) * sizeof(float4) + (size_t)K * 8;
#define CB(D) WHIP_LAUNCH(k_combine<D>, grid, dim3(256), lds, s, recs, pair_exp, pair_w, tok_pairs, K, part_d, f, \
                          nch, H, sc_off_down, skip_zero, sh, sh_n, sh_stride, y)
    if (fm == 2) CB(2);
    else if (fm == 1) CB(1);
    else CB(0);
#undef CB
    return (int)hipGetLastError();
}

extern "C" int whip_combine_sh(const uint8_t *const *recs, const int32_t *pair_exp,
                               const float *pair_w, const int32_t *tok_pairs, int T, int K,
                               const float *part_d, int nch, int H, uint32_t sc_off_down,
                               int skip_zero, const whip_mat *shd, const float *h_sh, float *y,
                               hipStream_t s)
{
    return combine_sh(recs, pair_exp, pair_w, tok_pairs, T, K, part_d, nullptr, nch, H, sc_off_down, skip_zero, shd,
                      h_sh, y, s);
}

extern "C" int whip_combine(const uint8_t *const *recs, const int32_t *pair_exp,
                            const float *pair_w, const int32_t *tok_pairs, int T, int K,
                            const float *part_d, int nch, int H, uint32_t sc_off_down,
                            int skip_zero, const float *sh, int sh_n, size_t sh_stride, float *y,
                            hipStream_t s)
{
    return combine(recs, pair_exp, pair_w, tok_pairs, T, K, part_d, nullptr, nch, H, sc_off_down, skip_zero, sh,
                   sh_n, sh_stride, y, s);
}

extern "C" int whip_combine_fold(const uint8_t *const *recs, const int32_t *pair_exp, const float *pair_w,
                                 const int32_t *tok_pairs, int T, int K, const whip_fold *f, int H, int skip_zero,
                                 const float *sh, int sh_n, size_t sh_stride, float *y, hipStream_t s)
{
    if (!f || !f->S || !f->ls || f->nb < 1 || f->sc_off % 2) return (int)hipErrorInvalidValue;
    return combine(recs, pair_exp, pair_w, tok_pairs, T, K, nullptr, f, 1, H, 0, skip_zero, sh, sh_n, sh_stride, y,
                   s);
}

extern "C" int whip_combine_sh_fold(const uint8_t *const *recs, const int32_t *pair_exp, const float *pair_w,
                                    const int32_t *tok_pairs, int T, int K, const whip_fold *f, int H, int skip_zero,
                                    const whip_mat *shd, const float *h_sh, float *y, hipStream_t s)
{
    if (!f || !f->S || !f->ls || f->nb < 1 || f->sc_off % 2) return (int)hipErrorInvalidValue;
    return combine_sh(recs, pair_exp, pair_w, tok_pairs, T, K, nullptr, f, 1, H, 0, skip_zero, shd, h_sh, y, s);
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
