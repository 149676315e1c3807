// SPDX-License-Identifier: Apache-2.0
//
// skinny.hip — the trunk products of a small decode batch (2 to a few dozen
// tokens) on the matrix cores: the router's logits (src/model.c:5496, the
// rows kernels of 423-519 through 794/939) and the shared expert's gate/up
// and down projections (model.c:5391-5402, 5932-5938) for T tokens at once.
//
// At these batch sizes the products are HBM-bound: every weight is read once
// and used T times.  A VALU dot product per (weight, token) is not: its
// decode and per-token multiply-adds cost more than the stream.  Here the
// weights go to the matrix cores as the B operand of
// v_mfma_f32_32x32x16_bf16 (output rows on N, tokens on M, fp32
// accumulation), and the arithmetic stays exact where it must:
//
//   Q4G / Q8G  the integer q of a weight enters as bf16(q + 136) (4-bit:
//              0x4300 | nibble, two bit operations per pair) or
//              bf16(q + 128) (8-bit, a byte convert); both are exact.  The
//              offset comes off per 128-column group as 136 (or 128) times
//              the group's sum of x, then the group's f16 scale multiplies:
//              sum_k q_k x_k = sum_k (q_k + c) x_k - c sum_k x_k.
//   F32        each weight is split exactly into three bf16 pieces
//              (truncations: hi + mid + lo == w), one product each.
//   x          bf16 activations are the A operand as they are; fp32
//              activations are split the same way into three pieces.
//
// Products of bf16 pieces are exact in fp32, so the only rounding is the
// fp32 accumulation (and, for F32 weights against fp32 x, the three
// smallest cross terms, below 2^-24 of the product, are left out).
//
// A wavefront owns 32 output rows and one slice of the columns: NC chunks
// of 128 (4 for 4-bit rows, 2 for 8-bit, 1 for fp32: 8-16 KB of weights a
// wavefront).  Every load a lane needs is issued at the start — the
// slice's activations first, then all of its weights — so the whole
// product is in flight at once; the chunks are then multiplied in the
// order their weights arrive.  The slices' partial sums land in
// part[slice][t][row] and a second launch (or the combine, for the shared
// down projection) adds them in slice order, so results do not depend on
// scheduling.  Within a chunk lane half h of the B operand holds the
// chunk's columns 64h .. 64h+63 of its row, eight per product: each lane's
// weights for a chunk are one contiguous run (32 bytes of nibbles, 64 of
// bytes, 256 of floats).  The activations are staged in LDS already in the
// A operand's order, one 16-byte read per lane per product.
#include "common.h"
#include "launch.h"
#include "route.h"
#include "bf16_split.h"

typedef float acc16 __attribute__((ext_vector_type(16)));

#define SK_WAVES 4
#define SK_ROWS (SK_WAVES * 32)     // output rows per workgroup
#define SK_KC 128                   // columns per chunk (one scale group)
#define SK_TOK 32                   // tokens per tile (the M of a product)
#define SK_NCMAX 4

// chunks per slice, and 16-byte words per lane per chunk
template <int FMT> struct sk_nc { static constexpr int NC = FMT == 0 ? 1 : FMT == 2 ? 2 : 4; };
template <int FMT> struct sk_nw { static constexpr int N = FMT == 0 ? 16 : FMT == 2 ? 4 : 2; };
static int sk_chunks(int fmt) { return fmt == 0 ? 1 : fmt == 2 ? 2 : 4; }

struct sk_job {
    const uint8_t *W;
    const uint16_t *S;
    size_t rowbytes;
    int fmt, rows, cols, group;
    const void *x;
    int x_ld;
    float *part;                    // [nsl][T][rows]
    int nsl, nrb, blk0;
};
struct sk_pack {
    sk_job j[3];
    int n, T;
};

// eight nibbles (low first) as bf16(n + 128): 0x4300 | n, exact
WH_INLINE uint4 q4_frag(uint32_t d)
{
    const uint32_t lo = d & 0x0f0f0f0fu, hi = (d >> 4) & 0x0f0f0f0fu;
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; j++)
        w[j] = __builtin_amdgcn_perm(hi, lo, 0x0c000c00u | (uint32_t)j | ((4u + (uint32_t)j) << 16)) | 0x43004300u;
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// eight int8 weights as bf16(q + 128), exact (q + 128 < 256)
WH_INLINE uint4 q8_frag(uint32_t d0, uint32_t d1)
{
    uint32_t w[4];
    const uint32_t d[2] = {d0 ^ 0x80808080u, d1 ^ 0x80808080u};
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t u = d[j >> 1], sh = 16 * (j & 1);
        const float a = (float)((u >> sh) & 255), b = (float)((u >> (sh + 8)) & 255);
        w[j] = (__float_as_uint(a) >> 16) | (__float_as_uint(b) & 0xffff0000u);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
}

WH_INLINE acc16 mfma(const bf16x8 &a, uint4 b, const acc16 &c)
{
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, as_b8(b), c, 0, 0, 0);
}

template <int FMT, int XS>
__device__ __forceinline__ void sk_body(const sk_job &J, int T, int blk, uint4 (*frag)[XS][8][64],
                                        float (*xs)[SK_TOK])
{
    constexpr int NC = sk_nc<FMT>::NC, NW = sk_nw<FMT>::N, XW = XS == 1 ? 2 : 4;
    const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, n = lane & 31;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rb = blk % J.nrb, sl = blk / J.nrb;
    const int t0 = blockIdx.y * SK_TOK;
    const int k_lo = sl * NC * SK_KC;
    const int nc = min(NC, (J.cols - k_lo) / SK_KC);  // >= 1 (host)
    const int ng = FMT == 0 ? 1 : J.cols / J.group;
    const int row = rb * SK_ROWS + wv * 32 + n;
    const int rc = min(row, J.rows - 1);
    const uint8_t *wp = J.W + (size_t)rc * J.rowbytes;
    const uint16_t *sp = FMT == 0 ? nullptr : J.S + (size_t)rc * ng;

    // every load first: chunk c is k_lo + 128c, or the slice's last chunk
    // again past its end (all unconditional, so no load waits behind a
    // branch).  Staging: thread -> token sm of the tile, 16 columns at
    // 64*shh + 16*sq of each chunk (products 2sq and 2sq + 1 of half shh).
    // A tile row past the last token reads token 0 again: its products
    // land only in outputs that are never stored, and a select between
    // the loaded words and zero would let the compiler move the loads
    // behind a branch (and then wait for every load in flight).
    const int sm = tid >> 3, sj = tid & 7, shh = sj >> 2, sq = sj & 3;
    const bool slive = t0 + sm < T;
    const uint8_t *xrow = (const uint8_t *)J.x + (size_t)(slive ? t0 + sm : 0) * J.x_ld * (XS == 1 ? 2 : 4);
    uint4 xr[NC][XW];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const int e = k_lo + min(c, nc - 1) * SK_KC + 64 * shh + 16 * sq;
#pragma unroll
        for (int i = 0; i < XW; i++) xr[c][i] = *(const uint4 *)(xrow + (size_t)e * (XS == 1 ? 2 : 4) + 16 * i);
    }
    uint4 w[NC][NW];
    uint16_t sc[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const int k0 = k_lo + min(c, nc - 1) * SK_KC, kk = k0 + 64 * h;
        const size_t off = FMT == 0 ? (size_t)kk * 4 : FMT == 2 ? (size_t)kk : (size_t)kk / 2;
#pragma unroll
        for (int i = 0; i < NW; i++) w[c][i] = *(const uint4 *)(wp + off + 16 * i);
        sc[c] = FMT == 0 ? 0 : sp[k0 / J.group];
    }

    // stage the slice's activations: A fragments and each chunk's column sum
#pragma unroll
    for (int c = 0; c < NC; c++) {
        float v[16];
        uint4 raw[XW];
#pragma unroll
        for (int i = 0; i < XW; i++) raw[i] = xr[c][i];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            if (XS == 1) {
                const uint4 q = raw[i >> 3];
                const uint32_t wd[4] = {q.x, q.y, q.z, q.w};
                const uint32_t u = wd[(i >> 1) & 3];
                v[i] = wh_bf16((i & 1) ? (uint16_t)(u >> 16) : (uint16_t)(u & 0xffff));
            } else {
                const uint4 q = raw[(i >> 2) & (XW - 1)];
                const uint32_t wd[4] = {q.x, q.y, q.z, q.w};
                v[i] = __uint_as_float(wd[i & 3]);
            }
        }
        if (FMT != 0) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) s = __fadd_rn(s, v[i]);
            // the token's eight threads are consecutive lanes: a butterfly
            // leaves every one of them the same sum (addition commutes)
            s = __fadd_rn(s, __shfl_xor(s, 1));
            s = __fadd_rn(s, __shfl_xor(s, 2));
            s = __fadd_rn(s, __shfl_xor(s, 4));
            if (sj == 0) xs[c][sm] = s;
        }
        const int slot = shh * 32 + sm;
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++) {
            if (XS == 1) {
                frag[c][0][2 * sq + s2][slot] = raw[s2];
            } else {
                uint4 p0, p1, p2;
                split3(v + 8 * s2, p0, p1, p2);
                frag[c][0][2 * sq + s2][slot] = p0;
                frag[c][XS > 1 ? 1 : 0][2 * sq + s2][slot] = p1;
                frag[c][XS > 2 ? 2 : 0][2 * sq + s2][slot] = p2;
            }
        }
    }
    __syncthreads();

    acc16 acc;
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; c++) {
        if (c >= nc) break;                          // uniform
        acc16 ag;
#pragma unroll
        for (int s = 0; s < 8; s++) {
            bf16x8 a[XS];
#pragma unroll
            for (int p = 0; p < XS; p++) a[p] = as_b8(frag[c][p][s][lane]);
            if (FMT == 0) {
                const uint4 f0 = w[c][2 * s], f1 = w[c][2 * s + 1];
                const float f[8] = {__uint_as_float(f0.x), __uint_as_float(f0.y), __uint_as_float(f0.z),
                                    __uint_as_float(f0.w), __uint_as_float(f1.x), __uint_as_float(f1.y),
                                    __uint_as_float(f1.z), __uint_as_float(f1.w)};
                uint4 bh, bm, bl;
                split3(f, bh, bm, bl);
                // smallest terms first
                acc = mfma(a[0], bl, acc);
                if (XS == 3) {
                    acc = mfma(a[XS > 2 ? 2 : 0], bh, acc);
                    acc = mfma(a[XS > 1 ? 1 : 0], bm, acc);
                }
                acc = mfma(a[0], bm, acc);
                if (XS == 3) acc = mfma(a[XS > 1 ? 1 : 0], bh, acc);
                acc = mfma(a[0], bh, acc);
            } else {
                uint4 bq;
                if (FMT == 3) {
                    const uint4 q = w[c][(s >> 2) & (NW - 1)];
                    const uint32_t wd[4] = {q.x, q.y, q.z, q.w};
                    bq = q4_frag(wd[s & 3]);
                } else {
                    const uint4 q = w[c][(s >> 1) & (NW - 1)];
                    bq = (s & 1) ? q8_frag(q.z, q.w) : q8_frag(q.x, q.y);
                }
#pragma unroll
                for (int p = XS - 1; p >= 0; p--) {
                    if (s == 0 && p == XS - 1) {
                        acc16 z;
#pragma unroll
                        for (int r = 0; r < 16; r++) z[r] = 0.0f;
                        ag = mfma(a[p], bq, z);
                    } else {
                        ag = mfma(a[p], bq, ag);
                    }
                }
            }
        }
        if (FMT != 0) {
            // lane (n, h), register r: token 8(r/4) + 4h + r%4 of the tile
            const float off = FMT == 3 ? -136.0f : -128.0f;
            const float g = wh_f16_scale(sc[c]);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float xm = xs[c][8 * (r >> 2) + 4 * h + (r & 3)];
                acc[r] = __fmaf_rn(g, __fmaf_rn(off, xm, ag[r]), acc[r]);
            }
        }
    }
    if (row >= J.rows) return;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int t = t0 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (t < T) J.part[((size_t)sl * T + t) * J.rows + row] = acc[r];
    }
}

template <int XS>
__global__ void __launch_bounds__(SK_WAVES * 64) k_sk(sk_pack pk)
{
    __shared__ uint4 frag[SK_NCMAX][XS][8][64];
    __shared__ float xs[SK_NCMAX][SK_TOK];
    const int b = blockIdx.x;
    const int ji = (pk.n > 2 && b >= pk.j[2].blk0) ? 2 : (pk.n > 1 && b >= pk.j[1].blk0) ? 1 : 0;
    // field by field from the argument block (a reference into it, or a
    // whole-struct select, would put the block in scratch)
#define SEL(f) (ji == 2 ? pk.j[2].f : ji == 1 ? pk.j[1].f : pk.j[0].f)
    sk_job J;
    J.W = SEL(W); J.S = SEL(S); J.rowbytes = SEL(rowbytes); J.fmt = SEL(fmt); J.rows = SEL(rows);
    J.cols = SEL(cols); J.group = SEL(group); J.x = SEL(x); J.x_ld = SEL(x_ld); J.part = SEL(part);
    J.nsl = SEL(nsl); J.nrb = SEL(nrb); J.blk0 = SEL(blk0);
#undef SEL
    const int blk = b - J.blk0;
    if (J.fmt == 0) sk_body<0, XS>(J, pk.T, blk, frag, xs);
    else if (J.fmt == 2) sk_body<2, XS>(J, pk.T, blk, frag, xs);
    else sk_body<3, XS>(J, pk.T, blk, frag, xs);
}

// Sum of n slices q*stride + i, in slice order, with the loads issued eight
// at a time (a loop of dependent round trips would take n of them).
WH_INLINE float sum_slices(const float *p, int n, size_t stride)
{
    float s = p[0];
    for (int q0 = 1; q0 < n; q0 += 8) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = p[(size_t)min(q0 + k, n - 1) * stride];
#pragma unroll
        for (int k = 0; k < 8; k++)
            if (q0 + k < n) s = __fadd_rn(s, v[k]);
    }
    return s;
}

// logits[t][e] = sum over slices of the router's partials, in slice order;
// h[t][i] = silu(sum of the gate's) * (sum of the up's)
__global__ void __launch_bounds__(256)
k_sk_finish(const float *__restrict__ pr, int nsl_r, int E, float *__restrict__ logits,
            const float *__restrict__ pg, const float *__restrict__ pu, int nsl_g, int SI,
            float *__restrict__ h, int T)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int nr = T * E;
    if (i < nr) {
        logits[i] = sum_slices(pr + i, nsl_r, (size_t)nr);
        return;
    }
    const int j = i - nr, nh = T * SI;
    if (!pg || j >= nh) return;
    const float g = sum_slices(pg + j, nsl_g, (size_t)nh);
    const float u = sum_slices(pu + j, nsl_g, (size_t)nh);
    h[j] = wh_silu_mul(g, u);
}

// The same sums and the routing in one launch: block t < T sums token t's
// router slices into its logits (written out) and selects its experts with
// the batch-1 router launch's workgroup selection (route_fast: the engine's
// scores, group limit, tie rule and selection-order weights); blocks from T
// on sum the shared gate/up slices and apply the SwiGLU.
__global__ void __launch_bounds__(256)
k_sk_route(whip_route_cfg c, const float *__restrict__ pr, int nsl_r, float *__restrict__ logits,
           const float *__restrict__ bias, int T, int32_t *__restrict__ ids, float *__restrict__ wout,
           int *__restrict__ err, const float *__restrict__ pg, const float *__restrict__ pu, int nsl_g,
           int SI, float *__restrict__ h)
{
    __shared__ __align__(16) float s_lds[ROUTE_FAST_FLOATS(256)];
    __shared__ int32_t s_ids[64];
    __shared__ float s_w[64];
    __shared__ const uint8_t *s_tab[256];
    __shared__ const uint8_t *s_rec[64];
    __shared__ uint64_t s_etab[32];
    const int tid = threadIdx.x, E = c.E, K = c.K;
    if ((int)blockIdx.x >= T) {                      // uniform
        const int j = ((int)blockIdx.x - T) * 256 + tid, nh = T * SI;
        if (j < nh) h[j] = wh_silu_mul(sum_slices(pg + j, nsl_g, (size_t)nh), sum_slices(pu + j, nsl_g, (size_t)nh));
        return;
    }
    const int t = blockIdx.x;
    float l = 0.0f, be = 0.0f;
    if (tid < E) {
        l = sum_slices(pr + (size_t)t * E + tid, nsl_r, (size_t)T * E);
        logits[(size_t)t * E + tid] = l;
        be = bias ? bias[tid] : 0.0f;
    }
    s_tab[tid] = nullptr;                            // no records wanted: pairs come after
    if (tid < 32) s_etab[tid] = wh_exp_tab[tid];
    __syncthreads();
    route_fast<256>(c, l, be, s_tab, s_etab, s_lds, s_ids, s_w, s_rec, err);
    if (tid < K) {
        ids[(size_t)t * K + tid] = s_ids[tid];
        wout[(size_t)t * K + tid] = s_w[tid];
    }
}

extern "C" int whip_sk_route(const whip_route_cfg *c, const float *pr, int nsl_r, float *logits, const float *bias,
                             int T, int32_t *ids, float *w, int *err, const float *pg, const float *pu, int nsl_g,
                             int SI, float *h, hipStream_t s)
{
    // route_fast's shapes: every expert a thread, the candidates one wavefront
    if (T < 1 || c->E < 1 || c->E > 256 || c->K < 1 || ((c->E + 63) >> 6) * c->K > 64 || nsl_r < 1 ||
        (c->n_group > 1 && (c->n_group > 64 || c->E % c->n_group || c->topk_group < 1)) ||
        (pg && (!pu || !h || nsl_g < 1 || SI < 1)))
        return (int)hipErrorInvalidValue;
    const int nb = T + (pg ? (T * SI + 255) / 256 : 0);
    WHIP_LAUNCH(k_sk_route, dim3(nb), dim3(256), 0, s, *c, pr, nsl_r, logits, bias, T, ids, w, err, pg, pu, nsl_g,
                SI, h);
    return (int)hipGetLastError();
}

extern "C" int whip_sk_ok(const whip_mat *A)
{
    if (A->rows < 1 || A->cols < SK_KC || A->cols % SK_KC || A->rowbytes % 16) return 0;
    if (A->fmt == 0) return 1;
    if (A->fmt != 2 && A->fmt != 3) return 0;
    return A->qs && A->group >= SK_KC && A->group % SK_KC == 0 && A->cols % A->group == 0;
}

// Column slices of NC chunks each (every slice non-empty).
extern "C" int whip_sk_slices(const whip_mat *A)
{
    if (!whip_sk_ok(A)) return 0;
    const int nck = A->cols / SK_KC, NC = sk_chunks(A->fmt);
    return (nck + NC - 1) / NC;
}

extern "C" int whip_sk_run(const whip_sk_job *jobs, int n, int T, hipStream_t s)
{
    if (n < 1 || n > 3 || T < 1) return (int)hipErrorInvalidValue;
    sk_pack pk;
    int blk = 0;
    const int xbf = jobs[0].x_bf16;
    for (int i = 0; i < n; i++) {
        const whip_sk_job *q = &jobs[i];
        const int nsl = whip_sk_slices(&q->A);
        if (!nsl || nsl != q->nsl || q->x_bf16 != xbf || q->x_ld % 8 || q->x_ld < q->A.cols ||
            (uintptr_t)q->x % 16 || !q->part)
            return (int)hipErrorInvalidValue;
        sk_job &J = pk.j[i];
        J.W = (const uint8_t *)q->A.q; J.S = q->A.qs; J.rowbytes = q->A.rowbytes; J.fmt = q->A.fmt;
        J.rows = q->A.rows; J.cols = q->A.cols; J.group = q->A.group; J.x = q->x; J.x_ld = q->x_ld;
        J.part = q->part; J.nsl = nsl;
        J.nrb = (q->A.rows + SK_ROWS - 1) / SK_ROWS;
        J.blk0 = blk;
        blk += J.nrb * nsl;
    }
    pk.n = n;
    pk.T = T;
    const dim3 grid(blk, (T + SK_TOK - 1) / SK_TOK);
    if (xbf) WHIP_LAUNCH(k_sk<1>, grid, dim3(SK_WAVES * 64), 0, s, pk);
    else WHIP_LAUNCH(k_sk<3>, grid, dim3(SK_WAVES * 64), 0, s, pk);
    return (int)hipGetLastError();
}

extern "C" int whip_sk_finish(const float *pr, int nsl_r, int E, float *logits, const float *pg,
                              const float *pu, int nsl_g, int SI, float *h, int T, hipStream_t s)
{
    if (T < 1 || E < 1 || nsl_r < 1 || (pg && (!pu || !h || nsl_g < 1 || SI < 1))) return (int)hipErrorInvalidValue;
    const size_t n = (size_t)T * E + (pg ? (size_t)T * SI : 0);
    WHIP_LAUNCH(k_sk_finish, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, pr, nsl_r, E, logits, pg, pu,
                nsl_g, SI, h, T);
    return (int)hipGetLastError();
}
