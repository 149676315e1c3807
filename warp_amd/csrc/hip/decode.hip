// SPDX-License-Identifier: Apache-2.0
//
// decode.hip — one token's experts in one persistent launch (moe_layer,
// src/model.c:5488-5939, for T = 1), the opt-in decode mode (the staged
// kernels are the default).
//
// The launch follows the batch-1 GEMV launch that writes the router logits
// and the shared expert's silu(gate.x)*(up.x) (h_sh).  One workgroup per CU
// (1,024 threads, the tables' LDS) then walks the rest of the layer, with
// the dependencies between its stages held in counters in device memory
// instead of kernel boundaries:
//
//   shared down rows (x = h_sh staged in LDS), while each workgroup routes
//     the logits itself (every workgroup computes the same selection)
//   the first gate/up tables; routed gate/up tiles -> partials -- barrier U
//   first down tile requested, wait U, SwiGLU of this workgroup's chunk from
//     the gate/up partials, down tables, down tiles -> partials -- barrier E
//   wait E; combine rows [g*H/G, ...) in selection order, + the shared rows
//   barrier X: its last arriver zeroes every counter for the next launch
//
// Each stage's tiles are shared out by whole (kind, chunk) or (pair, chunk)
// classes, so a workgroup builds its tables once per stage.  Every wait is on
// work that workgroups resident at the same time produce (the grid is one
// workgroup per CU); a wait that exceeds WAIT_TICKS gives up, raises the
// timeout bit, and its workgroup skips the remaining work but still arrives
// everywhere, so the counters stay consistent and the launch ends.
//
// Cross-workgroup data (partials, sh_out) is written with device-coherent
// stores (sc1: through the per-XCD L2s to the device's coherence point) and
// read with device-coherent loads; a producer waits for its stores to
// complete before it arrives.  Barriers count per XCD first (workgroup g
// runs on XCD g % 8) and then across the XCDs, and release one flag line per
// XCD, so no address sees more than 32 atomics.
//
// Measured against the staged kernels on the DeepSeek-V3-shaped layer: the
// tile streams run faster here (gate/up 14 us for 88 MB, down 4.7 us), but
// each barrier costs what a kernel boundary does: a workgroup's last
// partial stores take ~6 us to be acknowledged while ~24 MB of other
// workgroups' tile reads are queued ahead of them, so the exchange is
// bound by the HBM queue, not by the launch.
#include "common.h"
#include "launch.h"
#include "route.h"
#include "gemv_dev.h"
#include "vq_tile.h"

#define DT 1024
#define DW 16
#define NX 8                          // XCDs: workgroup g is dispatched to g % 8
#define LINE 32                       // ints per 128-byte line
#define BAR_INTS ((2 * NX + 1) * LINE)
enum { BAR_U, BAR_E, BAR_X, N_BARS };
#define ERR_TIMEOUT 16
#define WAIT_TICKS 5000000ull         // 50 ms of the 100 MHz constant clock

// WH_DEC_TRACE (off in the library): each workgroup's constant-clock time
// at the stage boundaries, read back with whip_decode1_trace.
#ifdef WH_DEC_TRACE
#define TR_SLOTS 16
__device__ uint64_t dec_trace[1024 * TR_SLOTS];
#define TR(i) do { if (threadIdx.x == 0) dec_trace[blockIdx.x * TR_SLOTS + (i)] = wall_clock64(); } while (0)
extern "C" int whip_decode1_trace(uint64_t *host, int n)
{
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(dec_trace), (size_t)n * TR_SLOTS * 8, 0, hipMemcpyDeviceToHost);
}
#else
#define TR(i) do { } while (0)
#endif

extern "C" size_t whip_decode1_sync_ints(int H) { return (size_t)N_BARS * BAR_INTS; }

// ---- device-coherent access ------------------------------------------------
typedef __amdgpu_buffer_rsrc_t rsrc_t;
#define SC1 16                        // buffer cache policy: device scope

__device__ __forceinline__ rsrc_t mk_rsrc(const void *base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ float cld(rsrc_t r, uint32_t off)
{
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, SC1));
}
__device__ __forceinline__ uint4 cld16(rsrc_t r, uint32_t off)
{
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, SC1);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void cst(float *p, float v) { coh_st(p, v); }
// every store this thread issued has completed
__device__ __forceinline__ void stores_done() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// ---- barriers ----------------------------------------------------------------
// A barrier counts the workgroups of a range [lo, hi): per XCD first, then
// across the XCDs that have members, and releases one flag line per XCD.
struct dsync {
    int *base;
    int g, G;
    int *err;
    __device__ int *bar(int b) const { return base + b * BAR_INTS; }
};

// members of [lo, hi) on virtual XCD x (workgroup g runs on g % NX)
__device__ __forceinline__ int xcd_members(int lo, int hi, int x)
{
    const int first = lo + ((x - lo % NX) % NX + NX) % NX;    // smallest g >= lo with g % NX == x
    return first < hi ? (hi - 1 - first) / NX + 1 : 0;
}

// thread 0 of a member: count it in; true for the range's last arriver
__device__ __forceinline__ bool bar_arrive(const dsync &s, int b, int lo, int hi)
{
    int *w = s.bar(b);
    const int x = s.g % NX;
    int groups = 0;
    for (int q = 0; q < NX; q++) groups += xcd_members(lo, hi, q) > 0;
    const int o = __hip_atomic_fetch_add(w + x * LINE, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (o != xcd_members(lo, hi, x) - 1) return false;
    const int o2 = __hip_atomic_fetch_add(w + NX * LINE, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return o2 == groups - 1;
}

__device__ __forceinline__ void bar_release(const dsync &s, int b)
{
    int *w = s.bar(b);
    for (int x = 0; x < NX; x++) coh_st(w + (NX + 1 + x) * LINE, 1);
}

// whole workgroup: its stores complete, then it arrives; returns (to every
// thread) whether it was the last; the last releases the waiters
__device__ __forceinline__ bool wg_arrive(const dsync &s, int b, int lo, int hi, int *s_flag)
{
    stores_done();
    __syncthreads();
    if (threadIdx.x == 0) {
        const bool last = bar_arrive(s, b, lo, hi);
        if (last) bar_release(s, b);
        *s_flag = last;
    }
    __syncthreads();
    return *s_flag != 0;
}

// whole workgroup: wait for barrier b's release; false on a timeout
__device__ __forceinline__ bool wg_wait(const dsync &s, int b, int *s_flag)
{
    if (threadIdx.x == 0) {
        const int *f = s.bar(b) + (NX + 1 + s.g % NX) * LINE;
        int ok = 1;
        if (coh_ld(f) == 0) {
            const uint64_t t0 = wall_clock64();
            while (coh_ld(f) == 0) {
                if (wall_clock64() - t0 > WAIT_TICKS) { ok = 0; atomicOr(s.err, ERR_TIMEOUT); break; }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        *s_flag = ok;
    }
    __syncthreads();
    return *s_flag != 0;
}

// ---- trunk rows ------------------------------------------------------------
// y[r] = W[r].x, or silu(A[r].x) * (B[r].x) for a pair, for rows [r_lo, r_hi)
// (F32, Q8G, Q4G rows).  The rows are cut into segments of 64 16-byte
// chunks; wavefront w takes the contiguous run [w*n/16, (w+1)*n/16) of the
// workgroup's n segments, lane l chunk l of each, with the next PF
// segments' loads always in flight.  x is read from LDS (fp32 or bf16,
// zero past the last column up to whole groups).  A segment's wave sum lands
// in segv; a row's value is its segments' sum in order, so the result does
// not depend on the timing.  issue_more() runs after the first loads are in
// flight (the caller stages x there); every thread calls this.
template <int FMT, bool XBF, bool PAIR, typename F>
__device__ __forceinline__ void seg_rows(const whip_mat &A, const whip_mat &B, const void *xs, int r_lo, int r_hi,
                                         float *segv, float *y, F issue_more)
{
    constexpr int NE = chunk_of<FMT>::NE, NW = xw_of<FMT, XBF>::N, PF = 4;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int ng = FMT == 0 ? 1 : (A.cols + A.group - 1) / A.group;
    const int C = (FMT == 0 ? A.cols : ng * A.group) / NE;
    const int spr = (C + 63) / 64;
    const int nseg = max(0, r_hi - r_lo) * spr;
    const int s0 = wv * nseg / DW, s1 = (wv + 1) * nseg / DW;
    const uint8_t *W0 = (const uint8_t *)A.q, *W1 = (const uint8_t *)B.q;
    uint4 wa[PF], wb[PF];
    uint16_t sa[PF], sb[PF];
    auto issue = [&](int sg, int j) {
        const int sc = sg < s1 ? sg : s0;             // past the run: a valid repeat, never used
        const int r = r_lo + sc / spr, k = (sc % spr) * 64 + lane, kc = k < C ? k : 0;
        const size_t o = (size_t)r * A.rowbytes + (size_t)kc * 16;
        wa[j] = *(const uint4 *)(W0 + o);
        if (FMT != 0) sa[j] = A.qs[(size_t)r * ng + (size_t)kc * NE / A.group];
        if (PAIR) {
            wb[j] = *(const uint4 *)(W1 + o);
            if (FMT != 0) sb[j] = B.qs[(size_t)r * ng + (size_t)kc * NE / A.group];
        }
    };
    if (s0 < s1) {
#pragma unroll
        for (int j = 0; j < PF; j++) issue(s0 + j, j);
    }
    issue_more();
    __syncthreads();                                   // x staged
    for (int sg = s0; sg < s1; sg += PF) {             // wave-uniform
#pragma unroll
        for (int j = 0; j < PF; j++) {
            const int cur = sg + j;
            if (cur >= s1) break;
            const int k = (cur % spr) * 64 + lane;
            float d0 = 0.0f, d1 = 0.0f;
            if (k < C) {
                uint4 xw[NW];
                const uint8_t *xp = (const uint8_t *)xs + (size_t)k * NE * (XBF ? 2 : 4);
                if (NE * (XBF ? 2 : 4) < 16) {
                    const uint2 q = *(const uint2 *)xp;
                    xw[0] = make_uint4(q.x, q.y, 0, 0);
                } else {
#pragma unroll
                    for (int i = 0; i < NW; i++) xw[i] = *(const uint4 *)(xp + 16 * i);
                }
                if (FMT == 3 && XBF) {
                    const float sx = chunk_sum136_bf(xw);
                    d0 = __fmul_rn(wh_f16_scale(sa[j]), chunk_dot_q4bf(wa[j], xw, sx));
                    if (PAIR) d1 = __fmul_rn(wh_f16_scale(sb[j]), chunk_dot_q4bf(wb[j], xw, sx));
                } else {
                    d0 = chunk_dot<FMT, XBF>(wa[j], xw);
                    if (FMT != 0) d0 = __fmul_rn(wh_f16_scale(sa[j]), d0);
                    if (PAIR) {
                        d1 = chunk_dot<FMT, XBF>(wb[j], xw);
                        if (FMT != 0) d1 = __fmul_rn(wh_f16_scale(sb[j]), d1);
                    }
                }
            }
            issue(cur + PF, j);
            d0 = wave_sum(d0);
            if (PAIR) d1 = wave_sum(d1);
            if (lane == 0) {
                segv[(cur) * (PAIR ? 2 : 1)] = d0;
                if (PAIR) segv[cur * 2 + 1] = d1;
            }
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < r_hi - r_lo; i += DT) {
        float a0 = 0.0f, a1 = 0.0f;
        for (int q = 0; q < spr; q++) {
            a0 += segv[(i * spr + q) * (PAIR ? 2 : 1)];
            if (PAIR) a1 += segv[(i * spr + q) * 2 + 1];
        }
        cst(y + r_lo + i, PAIR ? wh_silu_mul(a0, a1) : a0);
    }
    __syncthreads();
}

template <bool XBF, bool PAIR, typename F>
__device__ __forceinline__ void seg_rows_fmt(const whip_mat &A, const whip_mat &B, const void *xs, int r_lo,
                                             int r_hi, float *segv, float *y, F issue_more)
{
    if (A.fmt == 0) seg_rows<0, XBF, PAIR>(A, B, xs, r_lo, r_hi, segv, y, issue_more);
    else if (A.fmt == 2) seg_rows<2, XBF, PAIR>(A, B, xs, r_lo, r_hi, segv, y, issue_more);
    else seg_rows<3, XBF, PAIR>(A, B, xs, r_lo, r_hi, segv, y, issue_more);
}

// padded columns (whole groups) of a matrix
__device__ __forceinline__ int padded_cols_d(const whip_mat &A)
{
    return A.fmt == 0 ? A.cols : (A.cols + A.group - 1) / A.group * A.group;
}


// ---- the launch ----------------------------------------------------------------
// A stage's tiles split over the workgroups: whole classes of tpc tiles
// each get floor or ceil of G / classes workgroups, so no workgroup
// crosses a class (its tables are built once); with more classes than
// workgroups, contiguous runs.  Returns [t0, t1) for workgroup g.
__device__ __forceinline__ void class_share(int g, int G, int classes, int tpc, int &t0, int &t1)
{
    const int base = G / classes, extra = G % classes;
    if (base == 0) {
        const int tiles = classes * tpc, per = (tiles + G - 1) / G;
        t0 = min(tiles, g * per);
        t1 = min(tiles, t0 + per);
        return;
    }
    int c, j, n;
    if (g < extra * (base + 1)) { c = g / (base + 1); j = g % (base + 1); n = base + 1; }
    else { const int q = g - extra * (base + 1); c = extra + q / base; j = q % base; n = base; }
    t0 = c * tpc + (int)((long)j * tpc / n);
    t1 = c * tpc + (int)((long)(j + 1) * tpc / n);
}

template <bool XBF>
__global__ void __launch_bounds__(DT) k_moe_decode1(whip_dec1_args a)
{
    __shared__ __align__(16) float smem[2 * 256 * 64]; // tables; h_sh or SwiGLU scratch between
    __shared__ __align__(16) float sbook[3 * 8 * 256]; // the current kind's books; scratch outside the tiles
    __shared__ const uint8_t *s_recs[256];            // the layer's record table
    __shared__ uint64_t s_etab[32];                   // expf's table
    __shared__ const uint8_t *s_rec[16];              // the selection's records
    __shared__ float s_w[16];                         // and weights
    __shared__ int32_t s_ids[16];
    __shared__ __align__(16) float s_h[256];          // a down class's h chunk; routing scratch
    __shared__ uint64_t s_rkey[256];                  // routing: keys, ranks, group scores
    __shared__ int s_rrank[256], s_rkeep[64];
    __shared__ float s_rg[64], s_rwraw[64];
    __shared__ int s_flag, s_dead;

    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int v = lane & 31, h = lane >> 5;
    const int g = blockIdx.x, G = gridDim.x;
    dsync S;
    S.base = a.sync; S.g = g; S.G = G; S.err = a.err;
    const int K = a.K, H = a.H, I = a.I;
    const int nch_gu = H / 256, nch_d = I / 256;       // 32-position chunks
    const int nb_gu = I / 64, nb_d = H / 64;           // 64-row blocks
    const int tpc_gu = K * nb_gu, tpc_d = nb_d;
    int gu0, gu1, d0, d1;
    class_share(g, G, 2 * nch_gu, tpc_gu, gu0, gu1);
    class_share(g, G, K * nch_d, tpc_d, d0, d1);
    if (tid == 0) s_dead = 0;
    TR(0);

    // lane constants of the tile loop (vq_tile.h)
    const uint32_t bA0 = (h ? 128u : 0u) + 4u * v, bA1 = (h ? 0u : 128u) + 4u * v;
    const uint32_t bB = 65536u + 128u * h + 4u * v;
    const uint32_t s0 = h ? 0x04020001u : 0x03020100u, s1 = h ? 0x06070503u : 0x07060504u;
    const uint32_t s2 = h ? 0x03010200u : 0x03020100u;
    const int rho = 16 * ((v >> 4) & 1) + 8 * ((v >> 3) & 1) + 4 * ((v >> 2) & 1) + 2 * (v & 1) + ((v >> 1) & 1);
    const uint32_t loff = v * 192 + h * 96, lrow = 32 * h + rho;
    g_u8 *dummy = as_global((const uint8_t *)a.booksT);
    const size_t rs_gu = (size_t)(H / 8) * 192, rs_d = (size_t)(I / 8) * 192;
    float *sink_gu = a.part_gu + (size_t)K * 2 * nch_gu * I, *sink_d = a.part_d + (size_t)K * nch_d * H;

    auto uni = [](const void *q) -> const uint8_t * {
        const uint64_t u = (uint64_t)q;
        const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
        const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
        return (const uint8_t *)(((uint64_t)hi << 32) | lo);
    };
    // gate/up tile t: class (kind, chunk), then (pair, row block)
    auto gu_at = [&](int t, int &p, int &kind, int &chunk, int &rb) {
        const int cls = t / tpc_gu, w = t - cls * tpc_gu;
        kind = cls / nch_gu; chunk = cls - kind * nch_gu; p = w / nb_gu; rb = w - p * nb_gu;
    };
    // down tile t: class (pair, chunk), then row block
    auto d_at = [&](int t, int &p, int &chunk, int &rb) {
        const int cls = t / tpc_d;
        p = cls / nch_d; chunk = cls - p * nch_d; rb = t - cls * tpc_d;
    };
    auto gu_where = [&](int t, g_u8 *&src, float *&out, bool &live) {
        if (t >= gu1) { src = dummy; out = sink_gu; live = true; return; }
        int p, kind, chunk, rb;
        gu_at(t, p, kind, chunk, rb);
        const uint8_t *rec = uni(s_rec[p]);
        live = rec != nullptr;
        src = rec ? as_global(rec) + (kind ? a.off_up : a.off_gate) + (size_t)rb * rs_gu + (size_t)chunk * PW * 192
                  : dummy;
        out = a.part_gu + (((size_t)p * 2 + kind) * nch_gu + chunk) * (size_t)I + rb * 64;
    };
    auto d_where = [&](int t, g_u8 *&src, float *&out, bool &live) {
        if (t >= d1) { src = dummy; out = sink_d; live = true; return; }
        int p, chunk, rb;
        d_at(t, p, chunk, rb);
        const uint8_t *rec = uni(s_rec[p]);
        live = rec != nullptr;
        src = rec ? as_global(rec) + a.off_down + (size_t)rb * rs_d + (size_t)chunk * PW * 192 : dummy;
        out = a.part_d + ((size_t)p * nch_d + chunk) * (size_t)H + rb * 64;
    };

    // books: one kind's three (6 per thread) through registers into sbook,
    // where they stay for every class of that kind
    float bv[3 * 8 * 256 / DT];
    int bkind = -1;
    auto book_loads = [&](int kind) {
        const float *bk = a.booksT + (size_t)(a.cb + kind * 3) * 8 * 256;
#pragma unroll
        for (int i = 0; i < 3 * 8 * 256 / DT; i++) bv[i] = bk[tid + i * DT];
    };
    auto books_to_lds = [&](int kind) {               // the old tables' readers are done
#pragma unroll
        for (int i = 0; i < 3 * 8 * 256 / DT; i++) sbook[tid + i * DT] = bv[i];
        bkind = kind;
    };
    auto tables = [&](const float *xv) {
        __syncthreads();
        table_mfma(smem, sbook, xv, wv, v, h);
        __syncthreads();
    };
    // the token's x at position chunk*32 + v
    auto x_raw = [&](int chunk, uint4 *q) {
        const size_t e0 = (size_t)(chunk * PW + v) * 8;
        if (XBF) { q[0] = *(const uint4 *)((const uint16_t *)a.x + e0); q[1] = q[0]; }
        else { q[0] = *(const uint4 *)((const float *)a.x + e0); q[1] = *(const uint4 *)((const float *)a.x + e0 + 4); }
    };
    auto x_of = [&](const uint4 *q, float *xv) {
        if (XBF) {
            const uint32_t w4[4] = {q[0].x, q[0].y, q[0].z, q[0].w};
#pragma unroll
            for (int i = 0; i < 4; i++) { xv[2 * i] = wh_bf16(w4[i] & 0xffff); xv[2 * i + 1] = wh_bf16(w4[i] >> 16); }
        } else {
            xv[0] = __uint_as_float(q[0].x); xv[1] = __uint_as_float(q[0].y); xv[2] = __uint_as_float(q[0].z);
            xv[3] = __uint_as_float(q[0].w); xv[4] = __uint_as_float(q[1].x); xv[5] = __uint_as_float(q[1].y);
            xv[6] = __uint_as_float(q[1].z); xv[7] = __uint_as_float(q[1].w);
        }
    };

    // this wavefront's tiles t0 + wv, t0 + wv + 16, ...; the next one always
    // in flight; a class change (uniform) rebuilds the tables
    tile_buf A, B;
    bool unbound = false;
    auto run_tiles = [&](int t0, int t1, int tpc, auto where, auto rebuild, bool preloaded, int tA) {
        g_u8 *src;
        float *outA, *outB;
        bool liveA, liveB, inA = true;
        int t = tA;
        where(t, src, outA, liveA);
        if (!preloaded) load_tile(A, src, loff);
        for (int lo = t0; lo < t1;) {
            const int hi = min(t1, (lo / tpc + 1) * tpc);     // this class's end
            while (t < hi) {
                float r;
                g_u8 *cur = src;
                if (inA) {
                    where(t + LW, src, outB, liveB);
                    src = t + LW < t1 ? src : cur;              // past the share: the tile just read
                    load_tile(B, src, loff);
                    r = tile_sum(A, smem, bA0, bA1, bB, s0, s1, s2, lane);
                    cst(outA + lrow, liveA ? r : 0.0f);
                    unbound |= !liveA;
                } else {
                    where(t + LW, src, outA, liveA);
                    src = t + LW < t1 ? src : cur;
                    load_tile(A, src, loff);
                    r = tile_sum(B, smem, bA0, bA1, bB, s0, s1, s2, lane);
                    cst(outB + lrow, liveB ? r : 0.0f);
                    unbound |= !liveB;
                }
                inA = !inA;
                t += LW;
            }
            lo = hi;
            if (lo < t1) rebuild(lo);
        }
    };

    // ---- start: the shared down projection (its input h_sh is the previous
    // launch's) streams while the workgroup routes the logits itself; the
    // first gate/up tables' books and x are requested with them ----
    uint4 nx[2];
    int kind0 = 0;
    auto route_here = [&] {
        float l = 0.0f, be = 0.0f;
        if (tid < a.E) {
            l = a.logits[tid];
            be = a.bias ? a.bias[tid] : 0.0f;
            s_recs[tid] = a.recs[tid];
        }
        if (tid < 32) s_etab[tid] = wh_exp_tab[tid];
        if (gu0 < gu1) {
            int p, chunk, rb;
            gu_at(gu0, p, kind0, chunk, rb);
            book_loads(kind0);
            x_raw(chunk, nx);
        }
        __syncthreads();
        route_lds R;
        R.sc = s_h; R.sel = s_h; R.key = s_rkey; R.rank = s_rrank;
        R.g = s_rg; R.keep = s_rkeep; R.wraw = s_rwraw;
        route_wg<DT>(a.rc, l, be, s_recs, s_etab, R, s_ids, s_w, s_rec, a.err);
        TR(1);
    };
    if (a.has_shared) {
        const int per = (H + G - 1) / G;
        const int r_lo = min(H, g * per), r_hi = min(H, r_lo + per);
        const int pc = padded_cols_d(a.sh[2]);
        auto stage_and_route = [&] {
            for (int i = tid; i < pc / 4; i += DT) {
                const int e = 4 * i;
                *(uint4 *)(smem + e) = e + 4 <= a.SI ? *(const uint4 *)(a.h_sh + e) : make_uint4(0, 0, 0, 0);
            }
            route_here();
        };
        seg_rows_fmt<false, false>(a.sh[2], a.sh[2], smem, r_lo, r_hi, sbook, a.sh_out, stage_and_route);
    } else {
        route_here();
    }
    if (g == 0 && tid < K) {                          // the selection, for the caller
        const int id = s_ids[tid];
        a.ids[tid] = id; a.w[tid] = s_w[tid];
        a.pair_tok[tid] = 0; a.pair_exp[tid] = id < 0 ? a.E : id; a.pair_w[tid] = s_w[tid];
        a.tok_pairs[tid] = tid; a.pair_rec[tid] = s_rec[tid];
    }
    TR(4);
    if (gu0 < gu1) {
        float xv[8];
        x_of(nx, xv);
        __syncthreads();                               // sbook: the segment sums are read
        books_to_lds(kind0);
        tables(xv);
    }
    TR(2);

    // ---- routed gate/up tiles ----
    if (gu0 < gu1) {
        auto gu_rebuild = [&](int t) {                 // a share crosses classes only when G < classes
            int p, kind, chunk, rb;
            gu_at(t, p, kind, chunk, rb);
            x_raw(chunk, nx);
            if (kind != bkind) book_loads(kind);
            float xv[8];
            x_of(nx, xv);
            if (kind != bkind) {                       // uniform
                __syncthreads();
                books_to_lds(kind);
            }
            tables(xv);
        };
        run_tiles(gu0, gu1, tpc_gu, gu_where, gu_rebuild, false, gu0 + wv);
    }
    TR(3);
    wg_arrive(S, BAR_U, 0, G, &s_flag);

    // ---- down: first tile in flight, wait for every gate/up partial ----
    if (d0 < d1) {
        int p, chunk, rb;
        d_at(d0, p, chunk, rb);
        {
            g_u8 *src;
            float *o;
            bool l;
            d_where(d0 + wv, src, o, l);
            load_tile(A, src, loff);
        }
        book_loads(2);
        if (!wg_wait(S, BAR_U, &s_flag)) s_dead = 1;
        TR(5);
        // SwiGLU of rows chunk*256 .. +256 of pair p from the gate/up
        // partials: thread (row i, quarter q) sums a quarter of the chunks of
        // both kinds; scratch in the tables' LDS (rebuilt next)
        auto act = [&](int p, int chunk) {
            const int i = tid & 255, q = tid >> 8, r = chunk * 256 + i;
            const int ns = (nch_gu + 3) / 4, c_lo = min(nch_gu, q * ns), c_hi = min(nch_gu, c_lo + ns);
            const rsrc_t pr = mk_rsrc(a.part_gu + (size_t)p * 2 * nch_gu * I, (uint32_t)(2 * nch_gu * I * 4));
            float sg = 0.0f, su = 0.0f;
            for (int cb = c_lo; cb < c_hi; cb += 8) {
                float gv[8], uv[8];
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const int c = cb + k < c_hi ? cb + k : c_lo;
                    gv[k] = cld(pr, (uint32_t)(c * I + r) * 4);
                    uv[k] = cld(pr, (uint32_t)((nch_gu + c) * I + r) * 4);
                }
#pragma unroll
                for (int k = 0; k < 8; k++)
                    if (cb + k < c_hi) { sg += gv[k]; su += uv[k]; }
            }
            float *red = smem;                         // [4][256][2]
            __syncthreads();                           // the old tables' readers are done
            red[(q * 256 + i) * 2] = sg;
            red[(q * 256 + i) * 2 + 1] = su;
            __syncthreads();
            if (tid < 256) {
                float gg = 0.0f, uu = 0.0f;
#pragma unroll
                for (int k = 0; k < 4; k++) { gg += red[(k * 256 + i) * 2]; uu += red[(k * 256 + i) * 2 + 1]; }
                const uint8_t *rec = s_rec[p];
                float hv = 0.0f;
                if (rec) {
                    g_u16 *sc = (g_u16 *)(as_global(rec) + a.off_sc);
                    hv = wh_silu_mul(__fmul_rn(gg, wh_f16_scale(sc[r])), __fmul_rn(uu, wh_f16_scale(sc[I + r])));
                }
                s_h[i] = hv;
            }
            __syncthreads();
        };
        auto d_build = [&](int p, int chunk) {
            act(p, chunk);
            float xv[8];
#pragma unroll
            for (int k = 0; k < 8; k++) xv[k] = s_h[v * 8 + k];
            if (bkind != 2) books_to_lds(2);           // uniform; sbook's last readers synchronised in act
            tables(xv);
        };
        if (!s_dead) {
            d_build(p, chunk);
            TR(6);
            auto d_rebuild = [&](int t) {
                int p2, c2, r2;
                d_at(t, p2, c2, r2);
                d_build(p2, c2);
            };
            run_tiles(d0, d1, tpc_d, d_where, d_rebuild, true, d0 + wv);
        }
    }
    if (unbound) atomicOr(a.err, 1);
    TR(7);
    wg_arrive(S, BAR_E, 0, G, &s_flag);

    // ---- combine: rows [g*per, ...) of y, pairs in selection order ----
    {
        const int per = (H + G - 1) / G;
        const int r_lo = min(H, g * per), r_hi = min(H, r_lo + per);
        if (r_lo < r_hi) {
            // every workgroup arrived after its shared rows and down tiles
            if (!wg_wait(S, BAR_E, &s_flag)) s_dead = 1;
            TR(8);
            float *red = sbook;                        // [K + 1][per]
            const int it = tid / per, i = tid - it * per, r = r_lo + i;
            if (!s_dead && it < K && r < r_hi) {
                const uint8_t *rec = s_rec[it];
                const rsrc_t pr = mk_rsrc(a.part_d + (size_t)it * nch_d * H, (uint32_t)(nch_d * H * 4));
                float pv[16];
#pragma unroll
                for (int c = 0; c < 16; c++) pv[c] = cld(pr, (uint32_t)((c < nch_d ? c : 0) * H + r) * 4);
                const float sc = rec ? wh_f16_scale(((g_u16 *)(as_global(rec) + a.off_sc))[2 * I + r]) : 0.0f;
                float sum = 0.0f;
#pragma unroll
                for (int c = 0; c < 16; c++)
                    if (c < nch_d) sum += pv[c];
                red[it * per + i] = rec ? __fmul_rn(s_w[it], __fmul_rn(sum, sc)) : 0.0f;
            }
            if (tid >= DT - per) {
                const int j = tid - (DT - per);
                red[K * per + j] = (!s_dead && a.has_shared && j < r_hi - r_lo) ? coh_ld(a.sh_out + r_lo + j) : 0.0f;
            }
            __syncthreads();
            if (!s_dead && tid < r_hi - r_lo) {
                float o = 0.0f;
                for (int j = 0; j < K; j++)            // selection order
                    if (s_rec[j]) o = __fadd_rn(o, red[j * per + tid]);
                a.y[r_lo + tid] = __fadd_rn(o, red[K * per + tid]);
            }
        }
    }
    TR(9);

    // ---- exit: the last arriver zeroes the counters for the next launch ----
    if (wg_arrive(S, BAR_X, 0, G, &s_flag)) {
        const int n = N_BARS * BAR_INTS;
        for (int i = tid; i < n; i += DT) coh_st(a.sync + i, 0);
    }
}

// 0 when the launch takes this shape, else hipErrorInvalidValue
extern "C" int whip_decode1_check(const whip_dec1_args *a)
{
    // shapes the tile loop and the combine take: whole 32-position chunks,
    // at most 16 selected experts, E <= 256 (the routing's key table)
    if (a->H <= 0 || a->H % 256 || a->I <= 0 || a->I % 256 || a->K < 1 || a->K > 16 || a->E < a->K ||
        a->E > 256 || a->off_gate % 16 || a->off_up % 16 || a->off_down % 16 || a->cb < 0 || !a->sync)
        return (int)hipErrorInvalidValue;
    if (a->H / 256 > 64 || a->I / 256 > 16) return (int)hipErrorInvalidValue;
    static int n_cu = 0;
    if (!n_cu) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu < 1)
            return (int)hipErrorInvalidValue;
    }
    const int G = n_cu;
    if (G < NX) return (int)hipErrorInvalidValue;
    if (a->has_shared) {
        // h_sh staged in the tables' LDS, zero-padded to whole groups; the
        // down rows' segment sums in sbook; 16-byte reads of h_sh
        const whip_mat &m = a->sh[2];
        if (m.fmt == 0 || m.cols != a->SI || a->SI % 4 || (uintptr_t)a->h_sh % 16) return (int)hipErrorInvalidValue;
        const int pc = (m.cols + m.group - 1) / m.group * m.group, ne = m.fmt == 2 ? 16 : 32;
        if ((long)pc * 4 > 2 * 256 * 64 * 4) return (int)hipErrorInvalidValue;
        const long spr = (pc / ne + 63) / 64;
        if ((long)((a->H + NX - 1) / NX) * spr > 3 * 8 * 256) return (int)hipErrorInvalidValue;
    }
    // the combine: K pairs x (H / G) rows, one thread each, and the shared row
    if ((long)(a->K + 1) * ((a->H + G - 1) / G) > DT) return (int)hipErrorInvalidValue;
    return 0;
}

extern "C" int whip_decode1(const whip_dec1_args *a, hipStream_t s)
{
    const int r = whip_decode1_check(a);
    if (r) return r;
    int G = 0, dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&G, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return (int)hipErrorInvalidValue;
    if (a->x_bf16) hipLaunchKernelGGL(k_moe_decode1<true>, dim3(G), dim3(DT), 0, s, *a);
    else hipLaunchKernelGGL(k_moe_decode1<false>, dim3(G), dim3(DT), 0, s, *a);
    return (int)hipGetLastError();
}
