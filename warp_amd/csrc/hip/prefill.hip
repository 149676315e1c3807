// SPDX-License-Identifier: Apache-2.0
//
// prefill.hip — the MoE layer over many tokens (moe_chunk,
// src/model.c:7110-7285) as grouped GEMMs on the matrix cores.
//
// Pairs (token, selected expert) are sorted by expert, so each expert's
// tokens form one segment; every expert's weights are then read once per
// block of up to 128 of its tokens, not once per pair.  Per segment:
//
//   h[p]  = silu(X[tok(p)] . Wg^T * sg) * (X[tok(p)] . Wu^T * su)   (fp16)
//   Y[p]  = h[p] . Wd^T * sd                                         (fp32)
//   y[t]  = sum over t's pairs, ascending expert, zero weights skipped,
//           of w * Y[p]; plus the shared expert
//
// The products run on v_mfma_f32_32x32x16_f16: tokens on M (32 per tile,
// four tiles per workgroup), output rows on N, fp32 accumulation.  Lane l
// of the B operand holds W[n0 + l%32][k0 + 8(l/32) .. +8): exactly one
// (row, position) vector of the container, which the lane decodes itself —
// VQ3R: C0[i0] + (C1[i1] + C2[i2]) from the fp16 codebooks in LDS (the
// container stores them in fp16, subnormals flushed as the engine's loader
// does), summed in fp32 and rounded once; Q4G / Q8G: the integer times its
// group scale.  Row scales of VQ3R
// apply in the epilogue, exactly, in fp32.  A (activations) is staged in LDS
// per 64-wide k chunk, converted to fp16; a value outside fp16's range
// raises the sticky range error instead of turning into inf.
//
// The router runs on v_mfma_f32_32x32x2_f32 (fp32 products, so the logits
// stay within the decode path's 1e-5 and routing decisions keep their
// meaning), split over k with the partial sums added in a fixed order.
#include "common.h"
#include "launch.h"
#include "bf16_split.h"

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float acc16 __attribute__((ext_vector_type(16)));

#define ERR_RANGE 4                  // sticky error bit: fp16 range exceeded

// ---- pair sort ---------------------------------------------------------------
// Stable counting sort of the T*K pairs by expert (failed selections, id -1,
// go to the segment after the last expert), in (token, slot) order within
// an expert; each token's pairs listed in ascending expert order (the
// chunk's combine order); experts ranked by size, largest first, so the
// longest segments are dispatched first.
#define SORT_THREADS 1024
#define SORT_LDS_PAIRS 8192

__global__ void __launch_bounds__(SORT_THREADS)
k_sort_pairs(const int32_t *__restrict__ ids, const float *__restrict__ w, int T, int K, int E,
             int32_t *__restrict__ pair_tok, int32_t *__restrict__ pair_exp, float *__restrict__ pair_w,
             int32_t *__restrict__ tok_pairs, int32_t *__restrict__ pair_pos,
             int32_t *__restrict__ seg_off, int32_t *__restrict__ order)
{
    extern __shared__ int sm[];
    const int NE = E + 1, P = T * K, tid = threadIdx.x;
    int *cnt = sm, *off = sm + NE, *run = sm + 2 * NE;
    // the pairs' experts (failed selections mapped to E), staged once: the
    // ordered scatter below reads them from LDS, not with a global round
    // trip per 64 pairs (P <= SORT_LDS_PAIRS; else read from global)
    int *eid = sm + 3 * NE, *pos = eid + (P <= SORT_LDS_PAIRS ? P : 0);
    const bool staged = P <= SORT_LDS_PAIRS;
    for (int i = tid; i < NE; i += SORT_THREADS) { cnt[i] = 0; run[i] = 0; }
    for (int q = tid; staged && q < P; q += SORT_THREADS) eid[q] = ids[q] < 0 ? E : ids[q];
    __syncthreads();
    for (int q = tid; q < P; q += SORT_THREADS) atomicAdd(&cnt[staged ? eid[q] : (ids[q] < 0 ? E : ids[q])], 1);
    __syncthreads();
    if (tid < 64) {                                   // exclusive scan, one wave
        const int per = (NE + 63) / 64;
        int s = 0;
        for (int i = 0; i < per; i++) { const int k = tid * per + i; if (k < NE) s += cnt[k]; }
        int inc = s;
        for (int o = 1; o < 64; o <<= 1) { const int v = __shfl_up(inc, o, 64); if (tid >= o) inc += v; }
        int base = inc - s;
        for (int i = 0; i < per; i++) {
            const int k = tid * per + i;
            if (k < NE) { off[k] = base; base += cnt[k]; }
        }
    }
    __syncthreads();
    if (tid < 64) {                                   // stable scatter, 64 pairs at a time, in order
        const uint64_t lt = (1ull << tid) - 1, gt = ~lt & ~(1ull << tid);
        for (int c0 = 0; c0 < P; c0 += 64) {
            const int q = c0 + tid;
            const bool valid = q < P;
            const int e = valid ? (staged ? eid[q] : (ids[q] < 0 ? E : ids[q])) : 0;
            uint64_t m = __ballot(valid);
            for (int b = 0; b < 11; b++) {            // lanes holding the same expert
                const bool bit = (e >> b) & 1;
                const uint64_t bb = __ballot(bit);
                m &= bit ? bb : ~bb;
            }
            if (valid) {
                const int base = run[e];
                const int p = off[e] + base + __popcll(m & lt);
                if (staged) pos[q] = p; else pair_pos[q] = p;
                if (!(m & gt)) run[e] = base + __popcll(m);
            }
        }
    }
    __syncthreads();
    for (int q = tid; q < P; q += SORT_THREADS) {
        const int p = staged ? pos[q] : pair_pos[q];
        if (staged) pair_pos[q] = p;
        pair_tok[p] = q / K;
        pair_exp[p] = staged ? eid[q] : (ids[q] < 0 ? E : ids[q]);
        pair_w[p] = w[q];
    }
    for (int q = tid; q < P; q += SORT_THREADS) {
        const int t = q / K, j = q - t * K;
        // the token's experts from LDS when staged (a global read per
        // comparison, waited for one at a time, made this loop most of the
        // launch)
        const int e = staged ? eid[q] : (ids[q] < 0 ? E : ids[q]);
        int rk = 0;
        for (int j2 = 0; j2 < K; j2++) {
            const int q2 = t * K + j2;
            const int e2 = staged ? eid[q2] : (ids[q2] < 0 ? E : ids[q2]);
            rk += e2 < e || (e2 == e && j2 < j);
        }
        tok_pairs[t * K + rk] = staged ? pos[q] : pair_pos[q];
    }
    for (int i = tid; i <= NE; i += SORT_THREADS) seg_off[i] = i < NE ? off[i] : P;
    for (int e = tid; e < E; e += SORT_THREADS) {
        const int c = cnt[e];
        int r = 0;
        for (int e2 = 0; e2 < E; e2++) {
            const int c2 = cnt[e2];
            r += c2 > c || (c2 == c && e2 < e);
        }
        order[r] = e;
    }
}

extern "C" int whip_sort_pairs(const int32_t *ids, const float *w, int T, int K, int E,
                               int32_t *pair_tok, int32_t *pair_exp, float *pair_w,
                               int32_t *tok_pairs, int32_t *pair_pos, int32_t *seg_off,
                               int32_t *order, hipStream_t s)
{
    if (T < 1 || K < 1 || E < 1 || E > 1024) return (int)hipErrorInvalidValue;
    const size_t lds = ((size_t)3 * (E + 1) + (T * K <= SORT_LDS_PAIRS ? (size_t)2 * T * K : 0)) * sizeof(int);
    hipLaunchKernelGGL(k_sort_pairs, dim3(1), dim3(SORT_THREADS), lds, s,
                       ids, w, T, K, E, pair_tok, pair_exp, pair_w, tok_pairs, pair_pos, seg_off, order);
    return (int)hipGetLastError();
}

// ---- grouped GEMM ----------------------------------------------------------
#define PF_THREADS 512
#define PF_KC 64                     // k per LDS chunk
#define PF_ALD (PF_KC + 8)           // A row stride in halves (144 B: rows fall on different banks)
#define PF_BIG 64                    // expert segments this long take the 256 x 256 tile kernel
#define PF_SHORT 32                  // and segments up to this long the one-tile kernel

enum { DEC_F32 = 0, DEC_Q8 = 2, DEC_Q4 = 3, DEC_VQ = 4 };

WH_INLINE _Float16 to_h(float v, bool &bad)
{
    bad |= !(fabsf(v) <= 65504.0f);                  // also NaN
    return (_Float16)v;
}

WH_INLINE h8 as_h8(uint4 u) { return __builtin_bit_cast(h8, u); }
WH_INLINE uint4 as_u4(h8 h) { return __builtin_bit_cast(uint4, h); }

// One VQ3R weight vector from its three fp16 codebook rows: C0 + (C1 + C2)
// summed in fp32 (exact for the books' magnitudes) and rounded to fp16 once,
// the nearest fp16 to the container's fp32 weight/scale (docs/FORMAT.md:
// 204-214).  Two fp16 additions would round twice, which doubled the
// products' error.  Each element is two mixed-precision fmas (fp16 sources
// read in place, fp32 arithmetic, the second rounding straight to fp16): the
// 1.0 they multiply by is opaque to the compiler, which would otherwise
// rewrite them as conversions and adds (five instructions an element).
WH_INLINE h8 vq_sum3(h8 c0, h8 c1, h8 c2)
{
    float one;
    asm volatile("v_mov_b32 %0, 1.0" : "=v"(one));
    h8 w;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float t = __builtin_fmaf((float)c1[i], one, (float)c2[i]);
        w[i] = (_Float16)__builtin_fmaf((float)c0[i], one, t);
    }
    return w;
}

template <int DEC, int EPI, int MT>
__global__ void __launch_bounds__(PF_THREADS) k_pf_gemm(whip_pf_args a)
{
    // EPI 0: gate/up pair, N tile 128 (waves 0-3 gate, 4-7 up), SwiGLU -> fp16
    // EPI 1: one matrix, N tile 256, fp32 rows (times the VQ3R row scale)
    // MT: M tiles of 32 rows per workgroup (4 for expert segments; 1 for one
    // long segment, which then spreads over more workgroups)
    constexpr int NBOOK = DEC == DEC_VQ ? (EPI == 0 ? 6 : 3) : 1;
    constexpr int ABUF = MT * 32 * PF_ALD;                          // halves per A buffer
    constexpr int SMEM = 2 * ABUF * 2 > 16384 ? 2 * ABUF * 2 : 16384; // A double buffer / SwiGLU exchange
    __shared__ uint4 cbk[NBOOK * 256];
    __shared__ __attribute__((aligned(16))) uint8_t smem[SMEM];
    _Float16 *As = (_Float16 *)smem;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int seg = a.order ? a.order[blockIdx.y] : (int)blockIdx.y;
    const int s0 = a.seg_off ? a.seg_off[seg] : 0;
    const int n_seg = a.seg_off ? a.seg_off[seg + 1] - s0 : a.rows;
    const int r0 = blockIdx.z * (MT * 32);           // this workgroup's rows of the segment
    if (r0 >= n_seg) return;
    if (DEC == DEC_VQ && MT == 4 && a.seg_off && n_seg >= PF_BIG) return;   // long segments: k_pf_gemm8
    // expert segments of at most 32 tokens take the one-tile instantiation
    // (a quarter of the accumulators, so more workgroups on a CU hide the
    // index loads' latency); the four-tile one takes those up to PF_BIG
    if (DEC == DEC_VQ && a.seg_off && (MT == 4 ? n_seg <= PF_SHORT : n_seg > PF_SHORT)) return;
    const int mrows = min(MT * 32, n_seg - r0);
    const int kind = EPI == 0 ? wave >> 2 : 0;
    const int ncol = blockIdx.x * (EPI == 0 ? 128 : 256) + (EPI == 0 ? (wave & 3) : wave) * 32 + (lane & 31);
    const bool ncol_ok = ncol < a.N;
    const int nc = ncol_ok ? ncol : 0;               // clamped row for loads

    const uint8_t *rec = nullptr;
    if (DEC == DEC_VQ) {
        rec = a.recs[seg];
        if (rec == nullptr) {                        // unbound expert: zeros + flag
            for (int m = wave; m < mrows; m += PF_THREADS / 64) {
                const size_t row = (size_t)(s0 + r0 + m);
                if (ncol_ok) {
                    if (EPI == 0) { if (kind == 0) ((_Float16 *)a.out)[row * a.out_ld + ncol] = (_Float16)0.0f; }
                    else ((float *)a.out)[row * a.out_ld + ncol] = 0.0f;
                }
            }
            if (tid == 0) atomicOr(a.err, 1);
            return;
        }
        for (int i = tid; i < NBOOK * 256; i += PF_THREADS)
            cbk[i] = *(const uint4 *)(a.books16 + ((size_t)(a.cb + i / 256) * 256 + (i & 255)) * 8);
    }
    const int nv = a.Kd / 8;
    const size_t rstride = (size_t)nv * 192;
    g_u8 *ib = DEC == DEC_VQ ? as_global(rec) + (kind ? a.idx_off[1] : a.idx_off[0]) + (size_t)(nc >> 6) * rstride +
                                   (nc & 63) * 3
                             : nullptr;
    const uint8_t *Wrow = DEC != DEC_VQ ? (kind ? a.W1 : a.W0) + (size_t)nc * a.rowbytes : nullptr;
    const uint16_t *Srow = (DEC == DEC_Q4 || DEC == DEC_Q8) ? (kind ? a.S1 : a.S0) + (size_t)nc * ((a.Kd + a.group - 1) / a.group)
                                                             : nullptr;
    bool bad = false;

    acc16 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[t][r] = 0.0f;

    // Software pipeline over 64-wide k chunks: chunk kc+1's A rows (raw, in
    // registers) and B inputs are requested before chunk kc's products, so
    // their latency hides behind the matrix work; the A tile is double
    // buffered, one barrier per chunk.  Loads take clamped addresses and no
    // branch; rows past the segment's end are zeroed when stored.  A thread
    // owns A items tid + 512q (row item/8, 8 k) below MT*32*8.
    const int nchunk = a.Kd / PF_KC;
    constexpr int NITEM = MT * 32 * (PF_KC / 8);
    constexpr int NA = (NITEM + PF_THREADS - 1) / PF_THREADS;
    size_t abase[NA];
    bool alive[NA];
#pragma unroll
    for (int q = 0; q < NA; q++) {
        const int it = tid + q * PF_THREADS, m = it >> 3;
        alive[q] = it < NITEM && m < mrows;
        const int mm = alive[q] ? m : 0;
        const int row = a.tok ? a.tok[s0 + r0 + mm] : s0 + r0 + mm;
        abase[q] = (size_t)row * a.x_ld + (it & 7) * 8;
    }
    uint4 ra[NA][2];
    auto load_a = [&](int kc) {
#pragma unroll
        for (int q = 0; q < NA; q++) {
            const size_t e0 = abase[q] + (size_t)kc * PF_KC;
            if (a.x_mode == 0) {
                ra[q][0] = *(const uint4 *)((const float *)a.x + e0);
                ra[q][1] = *(const uint4 *)((const float *)a.x + e0 + 4);
            } else {
                ra[q][0] = *(const uint4 *)((const uint16_t *)a.x + e0);
            }
        }
    };
    uint32_t bw[4][2], bwn[4][2];
    uint16_t bs[4], bsn[4];
    float4 bf[DEC == DEC_F32 ? 4 : 1][2], bfn[DEC == DEC_F32 ? 4 : 1][2];
    auto load_b = [&](int kc) {
#pragma unroll
        for (int st = 0; st < 4; st++) {
            const int k = kc * PF_KC + st * 16 + 8 * (lane >> 5);
            if (DEC == DEC_VQ) {
                bwn[st][0] = ld_u32_unaligned((const uint8_t *)(ib + (size_t)(k >> 3) * 192));
            } else if (DEC == DEC_Q4) {
                bwn[st][0] = *(const uint32_t *)(Wrow + (k >> 1));
                bsn[st] = Srow[k / a.group];
            } else if (DEC == DEC_Q8) {
                const uint2 v = *(const uint2 *)(Wrow + k);
                bwn[st][0] = v.x; bwn[st][1] = v.y;
                bsn[st] = Srow[k / a.group];
            } else {                                 // F32: 8 floats, converted at use
                bfn[DEC == DEC_F32 ? st : 0][0] = *(const float4 *)(Wrow + (size_t)k * 4);
                bfn[DEC == DEC_F32 ? st : 0][1] = *(const float4 *)(Wrow + (size_t)k * 4 + 16);
            }
        }
    };
    load_a(0);
    load_b(0);
    for (int kc = 0; kc < nchunk; kc++) {
#pragma unroll
        for (int st = 0; st < 4; st++) {
            bw[st][0] = bwn[st][0]; bw[st][1] = bwn[st][1]; bs[st] = bsn[st];
            if (DEC == DEC_F32) { bf[st][0] = bfn[st][0]; bf[st][1] = bfn[st][1]; }
        }
        h8 av8[NA];
#pragma unroll
        for (int q = 0; q < NA; q++) {
            h8 v;
            if (a.x_mode == 2) {
                v = as_h8(ra[q][0]);
            } else if (a.x_mode == 1) {
                const uint32_t uu[4] = {ra[q][0].x, ra[q][0].y, ra[q][0].z, ra[q][0].w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    v[2 * i] = to_h(wh_bf16(uu[i] & 0xffff), bad);
                    v[2 * i + 1] = to_h(wh_bf16(uu[i] >> 16), bad);
                }
            } else {
                const float f[8] = {__uint_as_float(ra[q][0].x), __uint_as_float(ra[q][0].y),
                                    __uint_as_float(ra[q][0].z), __uint_as_float(ra[q][0].w),
                                    __uint_as_float(ra[q][1].x), __uint_as_float(ra[q][1].y),
                                    __uint_as_float(ra[q][1].z), __uint_as_float(ra[q][1].w)};
#pragma unroll
                for (int i = 0; i < 8; i++) v[i] = to_h(f[i], bad);
            }
            if (!alive[q])
#pragma unroll
                for (int i = 0; i < 8; i++) v[i] = (_Float16)0.0f;
            av8[q] = v;
        }
        // buffer kc&1 was last read two chunks ago; the barrier of the chunk
        // between guarantees every wave is done with it
        _Float16 *Ab = As + (kc & 1) * ABUF;
#pragma unroll
        for (int q = 0; q < NA; q++) {
            const int it = tid + q * PF_THREADS;
            if (it < NITEM) *(uint4 *)(Ab + (it >> 3) * PF_ALD + (it & 7) * 8) = as_u4(av8[q]);
        }
        __syncthreads();
        if (kc + 1 < nchunk) {                       // uniform: the next chunk's loads fly now
            load_a(kc + 1);
            load_b(kc + 1);
        }
#pragma unroll
        for (int st = 0; st < 4; st++) {
            h8 b;
            if (DEC == DEC_VQ) {
                const uint32_t u = bw[st][0];
                const uint4 *bk = cbk + kind * 3 * 256;
                const h8 c0 = as_h8(bk[u & 255]);
                const h8 c1 = as_h8(bk[256 + ((u >> 8) & 255)]);
                const h8 c2 = as_h8(bk[512 + ((u >> 16) & 255)]);
                b = vq_sum3(c0, c1, c2);
            } else if (DEC == DEC_Q4) {
                const _Float16 sc = __builtin_bit_cast(_Float16, bs[st]);
                const uint32_t u = bw[st][0];
#pragma unroll
                for (int q = 0; q < 8; q++) b[q] = (_Float16)(float)((int)((u >> (4 * q)) & 15) - 8) * sc;
            } else if (DEC == DEC_Q8) {
                const _Float16 sc = __builtin_bit_cast(_Float16, bs[st]);
#pragma unroll
                for (int q = 0; q < 8; q++)
                    b[q] = (_Float16)(float)(int8_t)((bw[st][q >> 2] >> (8 * (q & 3))) & 0xff) * sc;
            } else {
                const float4 f0 = bf[DEC == DEC_F32 ? st : 0][0], f1 = bf[DEC == DEC_F32 ? st : 0][1];
                b[0] = to_h(f0.x, bad); b[1] = to_h(f0.y, bad); b[2] = to_h(f0.z, bad); b[3] = to_h(f0.w, bad);
                b[4] = to_h(f1.x, bad); b[5] = to_h(f1.y, bad); b[6] = to_h(f1.z, bad); b[7] = to_h(f1.w, bad);
            }
#pragma unroll
            for (int t = 0; t < MT; t++) {
                if (t * 32 >= mrows) continue;        // uniform
                const h8 av = as_h8(*(const uint4 *)(Ab + (t * 32 + (lane & 31)) * PF_ALD + st * 16 + 8 * (lane >> 5)));
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, b, acc[t], 0, 0, 0);
            }
        }
    }

    // epilogue: lane l, register r of tile t holds row t*32 + (r/4)*8 + (l/32)*4 + r%4, column ncol
    float rsc = 1.0f;
    if (DEC == DEC_VQ && ncol_ok) {
        g_u16 *sc = (g_u16 *)(as_global(rec) + a.sc_off[kind]);
        rsc = wh_f16_scale(sc[ncol]);
    }
    if (EPI == 0) {
        float *ex = (float *)smem;                    // [4 waves][16][64]: the gate values
#pragma unroll
        for (int t = 0; t < MT; t++) {
            if (t * 32 >= mrows) continue;            // uniform
            __syncthreads();
            if (kind == 0)
#pragma unroll
                for (int r = 0; r < 16; r++) ex[((wave & 3) * 16 + r) * 64 + lane] = acc[t][r] * rsc;
            __syncthreads();
            if (kind == 1 && ncol_ok)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int m = t * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                    if (m < mrows) {
                        const float h = wh_silu_mul(ex[((wave & 3) * 16 + r) * 64 + lane], acc[t][r] * rsc);
                        ((_Float16 *)a.out)[(size_t)(s0 + r0 + m) * a.out_ld + ncol] = to_h(h, bad);
                    }
                }
        }
    } else if (ncol_ok) {
#pragma unroll
        for (int t = 0; t < MT; t++) {
            if (t * 32 >= mrows) continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = t * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                if (m < mrows) ((float *)a.out)[(size_t)(s0 + r0 + m) * a.out_ld + ncol] = acc[t][r] * rsc;
            }
        }
    }
    if (bad) atomicOr(a.err, ERR_RANGE);
}

// ---- 256 x 256 tiles for long segments ---------------------------------------
// Segments of PF_BIG tokens or more: a workgroup takes 256 tokens and 256 B
// columns (VQ3R rows: 128 gate + 128 up for EPI 0, 256 of one matrix for
// EPI 1), and decodes its B tile once per 64-wide k chunk into LDS, where
// all eight wavefronts read it as they read A.  In k_pf_gemm each wavefront
// decodes the B fragments it multiplies, for up to four 32-token M tiles;
// here a decoded fragment feeds eight (the M tiles of the four wavefronts
// that share its columns), so the codebook gathers per product halve, and a
// wavefront's k step is 8 products from 2 A and 4 B fragment reads.  Rows
// past a segment's end are zeros in the A tile: every product runs, and the
// epilogue drops their rows.
// Both tiles are [256][8] slots of 8 halves (one VQ vector, or 8 k of a
// token) with the slot index XOR-swizzled by (row >> 1) & 7: every 16-lane
// pass of a 128-bit read or write, operand reads included, touches sixteen
// different bank groups.  The tiles are double buffered: chunk kc's products
// read one pair while chunk kc+1 is staged and decoded into the other, one
// barrier per chunk.  Wavefront w owns rows (w & 3) * 64 and columns
// (w >> 2) * 64 (EPI 0: gate and up of the same 64, SwiGLU in registers) or
// (w >> 2) * 128 (EPI 1).
#define PF8_M 256
#define PF8_N 256                    // B columns a workgroup decodes
#define PF8_THREADS 512

WH_INLINE int pf8_slot(int r, int g) { return r * 8 + (g ^ ((r >> 1) & 7)); }

// XM: the activations' format (0 fp32, 1 bf16, 2 fp16), fixed per launch
template <int EPI, int XM>
__global__ void __launch_bounds__(PF8_THREADS) k_pf_gemm8(whip_pf_args a)
{
    constexpr int NBOOK = EPI == 0 ? 6 : 3;
    constexpr int OUTN = EPI == 0 ? PF8_N / 2 : PF8_N;                // output columns per workgroup
    __shared__ uint4 cbk[NBOOK * 256];
    __shared__ uint4 sA[2][PF8_M * 8];
    __shared__ uint4 sB[2][PF8_N * 8];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int mw = wave & 3, nw = wave >> 2;
    const int seg = a.order ? a.order[blockIdx.y] : (int)blockIdx.y;
    const int s0 = a.seg_off[seg];
    const int n_seg = a.seg_off[seg + 1] - s0;
    const int r0 = blockIdx.z * PF8_M;
    if (r0 >= n_seg || n_seg < PF_BIG) return;       // shorter segments: k_pf_gemm
    const int mrows = min(PF8_M, n_seg - r0);
    const uint8_t *rec = a.recs[seg];

    // this thread's B column to decode (4 of its 8 positions per chunk)
    const int dc = tid & (PF8_N - 1), dv0 = tid >> 8;
    const int dkind = EPI == 0 ? dc >> 7 : 0;
    const int dwr = blockIdx.x * OUTN + (EPI == 0 ? (dc & 127) : dc);
    // the wavefront's four B fragments: columns in the tile, W rows, kinds
    int bcol[4], wrow[4], bkind[4];
    bool nok[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        if (EPI == 0) {
            bkind[j] = j >> 1;
            bcol[j] = bkind[j] * 128 + nw * 64 + (j & 1) * 32;
            wrow[j] = blockIdx.x * OUTN + nw * 64 + (j & 1) * 32 + (lane & 31);
        } else {
            bkind[j] = 0;
            bcol[j] = nw * 128 + j * 32;
            wrow[j] = blockIdx.x * OUTN + nw * 128 + j * 32 + (lane & 31);
        }
        nok[j] = wrow[j] < a.N;
    }
    if (rec == nullptr) {                            // unbound expert: zeros + flag
        if (mw == 0)                                 // one wavefront per column half
            for (int m = 0; m < mrows; m++) {
                const size_t row = (size_t)(s0 + r0 + m);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    if (!nok[j] || (EPI == 0 && bkind[j] != 0)) continue;
                    if (EPI == 0) ((_Float16 *)a.out)[row * a.out_ld + wrow[j]] = (_Float16)0.0f;
                    else ((float *)a.out)[row * a.out_ld + wrow[j]] = 0.0f;
                }
            }
        if (tid == 0) atomicOr(a.err, 1);
        return;
    }
    for (int i = tid; i < NBOOK * 256; i += PF8_THREADS)
        cbk[i] = *(const uint4 *)(a.books16 + ((size_t)(a.cb + i / 256) * 256 + (i & 255)) * 8);
    const int nv = a.Kd / 8;
    const size_t rstride = (size_t)nv * 192;
    g_u8 *dib = as_global(rec) + a.idx_off[dkind] + (size_t)((dwr < a.N ? dwr : 0) >> 6) * rstride +
                ((dwr < a.N ? dwr : 0) & 63) * 3;
    bool bad = false;

    // A items: it = tid + 512 q -> token row it >> 3, k group it & 7
    size_t abase[4];
    bool alive[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int it = tid + q * PF8_THREADS, m = it >> 3;
        alive[q] = m < mrows;
        const int mm = alive[q] ? m : 0;
        const int row = a.tok ? a.tok[s0 + r0 + mm] : s0 + r0 + mm;
        abase[q] = (size_t)row * a.x_ld + (it & 7) * 8;
    }
    const int nchunk = a.Kd / PF_KC;
    uint4 ra[4][2];
    uint32_t bw[4];
    auto load = [&](int kc) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const size_t e0 = abase[q] + (size_t)kc * PF_KC;
            if (XM == 0) {
                ra[q][0] = *(const uint4 *)((const float *)a.x + e0);
                ra[q][1] = *(const uint4 *)((const float *)a.x + e0 + 4);
            } else {
                ra[q][0] = *(const uint4 *)((const uint16_t *)a.x + e0);
            }
        }
#pragma unroll
        for (int q = 0; q < 4; q++)
            bw[q] = ld_u32_unaligned((const uint8_t *)(dib + (size_t)(kc * 8 + dv0 + 2 * q) * 192));
    };
    auto stage_a = [&](int buf) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            h8 v;
            if (XM == 2) {
                v = as_h8(ra[q][0]);
            } else if (XM == 1) {
                const uint32_t uu[4] = {ra[q][0].x, ra[q][0].y, ra[q][0].z, ra[q][0].w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    v[2 * i] = to_h(wh_bf16(uu[i] & 0xffff), bad);
                    v[2 * i + 1] = to_h(wh_bf16(uu[i] >> 16), bad);
                }
            } else {
                const float f[8] = {__uint_as_float(ra[q][0].x), __uint_as_float(ra[q][0].y),
                                    __uint_as_float(ra[q][0].z), __uint_as_float(ra[q][0].w),
                                    __uint_as_float(ra[q][1].x), __uint_as_float(ra[q][1].y),
                                    __uint_as_float(ra[q][1].z), __uint_as_float(ra[q][1].w)};
#pragma unroll
                for (int i = 0; i < 8; i++) v[i] = to_h(f[i], bad);
            }
            if (!alive[q])
#pragma unroll
                for (int i = 0; i < 8; i++) v[i] = (_Float16)0.0f;
            const int it = tid + q * PF8_THREADS;
            sA[buf][pf8_slot(it >> 3, it & 7)] = as_u4(v);
        }
    };
    const uint4 *bk = cbk + dkind * 3 * 256;
    auto decode = [&](int buf, int q) {
        const uint32_t u = bw[q];
        const h8 w = vq_sum3(as_h8(bk[u & 255]), as_h8(bk[256 + ((u >> 8) & 255)]), as_h8(bk[512 + ((u >> 16) & 255)]));
        sB[buf][pf8_slot(dc, dv0 + 2 * q)] = as_u4(w);
    };

    acc16 acc[2][4];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[t][j][r] = 0.0f;
    bool tlive[2];
#pragma unroll
    for (int t = 0; t < 2; t++) tlive[t] = mw * 64 + t * 32 < mrows;

    load(0);
    __syncthreads();                                 // the books
    stage_a(0);
#pragma unroll
    for (int q = 0; q < 4; q++) decode(0, q);
    if (nchunk > 1) load(1);
    __syncthreads();
    // operands of k step st: 2 A and 4 B fragments
    auto read_ops = [&](int buf, int st, h8 (&av)[2], h8 (&bv)[4]) {
        const int g = 2 * st + (lane >> 5);
#pragma unroll
        for (int t = 0; t < 2; t++) av[t] = as_h8(sA[buf][pf8_slot(mw * 64 + t * 32 + (lane & 31), g)]);
#pragma unroll
        for (int j = 0; j < 4; j++) bv[j] = as_h8(sB[buf][pf8_slot(bcol[j] + (lane & 31), g)]);
    };
    for (int kc = 0; kc < nchunk; kc++) {
        const int buf = kc & 1;
        const bool more = kc + 1 < nchunk;           // uniform
        if (more) stage_a(buf ^ 1);
        h8 av[2], bv[4];
        read_ops(buf, 0, av, bv);
#pragma unroll
        for (int st = 0; st < 4; st++) {
            // the next step's operands are read before this step's products
            // go out; rows past the segment are zeros, so every tile runs
            h8 avn[2], bvn[4];
            if (st < 3) read_ops(buf, st + 1, avn, bvn);
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    acc[t][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[t], bv[j], acc[t][j], 0, 0, 0);
            if (more) decode(buf ^ 1, st);           // chunk kc+1's B, one vector per k step
            if (st < 3) {
#pragma unroll
                for (int t = 0; t < 2; t++) av[t] = avn[t];
#pragma unroll
                for (int j = 0; j < 4; j++) bv[j] = bvn[j];
            }
        }
        if (kc + 2 < nchunk) load(kc + 2);
        __syncthreads();
    }

    // epilogue: lane l, register r of tile t holds row mw*64 + t*32 + (r/4)*8 + (l/32)*4 + r%4
    float rsc[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        g_u16 *sc = (g_u16 *)(as_global(rec) + a.sc_off[bkind[j]]);
        rsc[j] = wh_f16_scale(sc[nok[j] ? wrow[j] : 0]);
    }
#pragma unroll
    for (int t = 0; t < 2; t++) {
        if (!tlive[t]) continue;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = mw * 64 + t * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
            if (m >= mrows) continue;
            const size_t row = (size_t)(s0 + r0 + m);
            if (EPI == 0) {
#pragma unroll
                for (int f = 0; f < 2; f++)
                    if (nok[f]) {
                        const float h = wh_silu_mul(acc[t][f][r] * rsc[f], acc[t][f + 2][r] * rsc[f + 2]);
                        ((_Float16 *)a.out)[row * a.out_ld + wrow[f]] = to_h(h, bad);
                    }
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (nok[j]) ((float *)a.out)[row * a.out_ld + wrow[j]] = acc[t][j][r] * rsc[j];
            }
        }
    }
    if (bad) atomicOr(a.err, ERR_RANGE);
}

extern "C" int whip_pf_gemm(const whip_pf_args *a, int dec, int pair, int mt, int segs, int mblocks,
                            hipStream_t s)
{
    if (mt != 1 && mt != 4) return (int)hipErrorInvalidValue;
    if (a->Kd <= 0 || a->Kd % PF_KC || a->N <= 0 || segs < 1 || mblocks < 1) return (int)hipErrorInvalidValue;
    if ((dec == DEC_Q4 || dec == DEC_Q8) && (a->group <= 0 || a->group % 8)) return (int)hipErrorInvalidValue;
    if (dec != DEC_VQ && a->rowbytes % 16) return (int)hipErrorInvalidValue;
    if (dec == DEC_VQ && a->N % 64) return (int)hipErrorInvalidValue;
    if (a->x_ld % 8) return (int)hipErrorInvalidValue;
    if (dec == DEC_VQ && mt == 4 && a->seg_off) {
        // expert segments of PF_BIG tokens or more: 256 x 256 tiles; shorter
        // ones below (each workgroup checks its segment)
        const int n8 = pair ? PF8_N / 2 : PF8_N;
        dim3 grid8((a->N + n8 - 1) / n8, segs, (mblocks + 1) / 2);
        if (pair && a->x_mode == 2) hipLaunchKernelGGL((k_pf_gemm8<0, 2>), grid8, dim3(PF8_THREADS), 0, s, *a);
        else if (pair && a->x_mode == 1) hipLaunchKernelGGL((k_pf_gemm8<0, 1>), grid8, dim3(PF8_THREADS), 0, s, *a);
        else if (pair) hipLaunchKernelGGL((k_pf_gemm8<0, 0>), grid8, dim3(PF8_THREADS), 0, s, *a);
        else if (a->x_mode == 2) hipLaunchKernelGGL((k_pf_gemm8<1, 2>), grid8, dim3(PF8_THREADS), 0, s, *a);
        else if (a->x_mode == 1) hipLaunchKernelGGL((k_pf_gemm8<1, 1>), grid8, dim3(PF8_THREADS), 0, s, *a);
        else hipLaunchKernelGGL((k_pf_gemm8<1, 0>), grid8, dim3(PF8_THREADS), 0, s, *a);
        const int e = (int)hipGetLastError();
        if (e) return e;
        // segments of at most PF_SHORT tokens: one 32-token tile each
        dim3 grid1((a->N + (pair ? 128 : 256) - 1) / (pair ? 128 : 256), segs, 1);
        if (pair) hipLaunchKernelGGL((k_pf_gemm<DEC_VQ, 0, 1>), grid1, dim3(PF_THREADS), 0, s, *a);
        else hipLaunchKernelGGL((k_pf_gemm<DEC_VQ, 1, 1>), grid1, dim3(PF_THREADS), 0, s, *a);
        const int e1 = (int)hipGetLastError();
        if (e1) return e1;
    }
    const int ntile = pair ? 128 : 256;
    dim3 grid((a->N + ntile - 1) / ntile, segs, mblocks);
#define PF(D, E)                                                                                 \
    do {                                                                                         \
        if (mt == 4) hipLaunchKernelGGL((k_pf_gemm<D, E, 4>), grid, dim3(PF_THREADS), 0, s, *a); \
        else hipLaunchKernelGGL((k_pf_gemm<D, E, 1>), grid, dim3(PF_THREADS), 0, s, *a);         \
    } while (0)
    if (dec == DEC_VQ) { if (pair) PF(DEC_VQ, 0); else PF(DEC_VQ, 1); }
    else if (dec == DEC_Q4) { if (pair) PF(DEC_Q4, 0); else PF(DEC_Q4, 1); }
    else if (dec == DEC_Q8) { if (pair) PF(DEC_Q8, 0); else PF(DEC_Q8, 1); }
    else if (dec == DEC_F32) { if (pair) PF(DEC_F32, 0); else PF(DEC_F32, 1); }
    else return (int)hipErrorInvalidValue;
#undef PF
    return (int)hipGetLastError();
}

// ---- activations to fp16, once per chunk ---------------------------------------
// The products' A operand: each token row is staged by every column block
// of every expert it is routed to, so its conversion (and range check) is
// done once here.  n8: elements / 8; x 16-byte aligned.
__global__ void __launch_bounds__(256)
k_pf_to_f16(const void *__restrict__ x, int bf16, size_t n8, uint4 *__restrict__ y, int *err)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n8) return;
    bool bad = false;
    h8 v;
    if (bf16) {
        const uint4 u = ((const uint4 *)x)[i];
        const uint32_t uu[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            v[2 * k] = to_h(wh_bf16(uu[k] & 0xffff), bad);
            v[2 * k + 1] = to_h(wh_bf16(uu[k] >> 16), bad);
        }
    } else {
        const float4 f0 = ((const float4 *)x)[2 * i], f1 = ((const float4 *)x)[2 * i + 1];
        v[0] = to_h(f0.x, bad); v[1] = to_h(f0.y, bad); v[2] = to_h(f0.z, bad); v[3] = to_h(f0.w, bad);
        v[4] = to_h(f1.x, bad); v[5] = to_h(f1.y, bad); v[6] = to_h(f1.z, bad); v[7] = to_h(f1.w, bad);
    }
    y[i] = as_u4(v);
    if (bad) atomicOr(err, ERR_RANGE);
}

extern "C" int whip_pf_to_f16(const void *x, int bf16, size_t n, uint16_t *y, int *err, hipStream_t s)
{
    if (n % 8 || (uintptr_t)x % 16 || (uintptr_t)y % 16) return (int)hipErrorInvalidValue;
    const size_t n8 = n / 8;
    if (!n8) return 0;
    hipLaunchKernelGGL(k_pf_to_f16, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, s, x, bf16, n8, (uint4 *)y, err);
    return (int)hipGetLastError();
}

// ---- the shared expert over many tokens --------------------------------------
// Q4G / Q8G rows (model.c:484-492) against the chunk's fp16 activations on
// v_mfma_f32_32x32x16_f16.  Each 128-column group's integer products are
// summed in fp32 and then multiplied by the group's f16 scale, in fp32 (the
// engine's order: the group's dot product, then its scale); no weight is
// rounded.  A weight enters as the fp16 of its integer: 0x6400 | code is
// 1024 + code, and one packed fp16 subtraction of 1032 (4-bit: code = q + 8)
// or 1152 (8-bit: code = q + 128) leaves q exactly, two weights per
// instruction.  The pairs come out interleaved (codes j and j + 4 of a
// word, or bytes j and j + 2), and the A fragments are staged in LDS in the
// same interleaved column order, so every product still pairs each weight
// with its own activation.
//
// A workgroup: 64 tokens x 128 weight rows, a wavefront per 32 rows, the k
// loop in 128-column chunks (one scale group); A double-buffered in LDS in
// the operand's order, B one chunk ahead in registers.
//   EPI 0: 64 gate rows (waves 0-1) and the same 64 up rows (waves 2-3);
//          h = silu(gate) * up leaves as fp16 (range-checked).
//   EPI 1: 128 rows of one matrix, fp32 out.
#define DN_KC 128
typedef _Float16 dn_h2 __attribute__((ext_vector_type(2)));

template <int FMT>
WH_INLINE h8 dn_frag(const uint4 *w, int s)
{
    uint32_t o[4];
    if constexpr (FMT == DEC_Q4) {
        const uint4 q = w[s >> 2];
        const uint32_t wd[4] = {q.x, q.y, q.z, q.w};
        const uint32_t d = wd[s & 3];
#pragma unroll
        for (int j = 0; j < 4; j++) o[j] = ((d >> (4 * j)) & 0x000f000fu) | 0x64006400u;
    } else {
        const uint4 q = w[(s >> 1) & 3];
        const uint32_t d0 = ((s & 1) ? q.z : q.x) ^ 0x80808080u, d1 = ((s & 1) ? q.w : q.y) ^ 0x80808080u;
        o[0] = (d0 & 0x00ff00ffu) | 0x64006400u;
        o[1] = ((d0 >> 8) & 0x00ff00ffu) | 0x64006400u;
        o[2] = (d1 & 0x00ff00ffu) | 0x64006400u;
        o[3] = ((d1 >> 8) & 0x00ff00ffu) | 0x64006400u;
    }
    const _Float16 c = FMT == DEC_Q4 ? (_Float16)-1032.0f : (_Float16)-1152.0f;
    const dn_h2 off = {c, c};
#pragma unroll
    for (int j = 0; j < 4; j++) o[j] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(dn_h2, o[j]) + off);
    return as_h8(make_uint4(o[0], o[1], o[2], o[3]));
}

// eight fp16 activations (words [x0 x1][x2 x3][x4 x5][x6 x7]) in dn_frag's
// column order
template <int FMT>
WH_INLINE uint4 dn_order(uint4 v)
{
    if constexpr (FMT == DEC_Q4)                     // x0 x4 x1 x5 x2 x6 x3 x7
        return make_uint4(__builtin_amdgcn_perm(v.z, v.x, 0x05040100u), __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
                          __builtin_amdgcn_perm(v.w, v.y, 0x05040100u), __builtin_amdgcn_perm(v.w, v.y, 0x07060302u));
    return make_uint4(__builtin_amdgcn_perm(v.y, v.x, 0x05040100u), __builtin_amdgcn_perm(v.y, v.x, 0x07060302u),
                      __builtin_amdgcn_perm(v.w, v.z, 0x05040100u), __builtin_amdgcn_perm(v.w, v.z, 0x07060302u));
}

template <int FMT, int EPI>
__global__ void __launch_bounds__(256) k_pf_dense(whip_pf_args a)
{
    __shared__ uint4 Af[2][2][8][64];                // [buffer][M fragment][product][lane]
    constexpr int NW = FMT == DEC_Q4 ? 2 : 4;        // 16-byte words of a lane's chunk
    const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, n = lane & 31;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t0 = blockIdx.y * 64;
    const int kind = EPI == 0 ? (w >> 1) : 0;
    const int row = EPI == 0 ? blockIdx.x * 64 + (w & 1) * 32 + n : blockIdx.x * 128 + w * 32 + n;
    const bool row_ok = row < a.N;
    const int rc = row_ok ? row : a.N - 1;
    const int ng = a.Kd / a.group;
    const uint8_t *Wr = (kind ? a.W1 : a.W0) + (size_t)rc * a.rowbytes;
    const uint16_t *Sr = (kind ? a.S1 : a.S0) + (size_t)rc * ng;
    // staging: thread -> token sm of the tile, columns 32sj .. 32sj+31 of the
    // chunk: half sj/2, products 4(sj&1) .. +3.  Tokens past the chunk read
    // its last token again (their outputs are never stored).
    const int sm = tid >> 2, sj = tid & 3;
    const int tok = min(t0 + sm, a.rows - 1);
    const uint16_t *xr = (const uint16_t *)a.x + (size_t)tok * a.x_ld + 32 * sj;
    const int mf = sm >> 5, slot = (sj >> 1) * 32 + (sm & 31), s_base = 4 * (sj & 1);
    uint4 ra[4], wn[NW], wc[NW];
    uint16_t scn, scc;
    auto load = [&](int c) {
        const int k0 = c * DN_KC;
#pragma unroll
        for (int i = 0; i < 4; i++) ra[i] = *(const uint4 *)(xr + k0 + 8 * i);
        const int kk = k0 + 64 * h;
        const uint8_t *p = Wr + (FMT == DEC_Q4 ? kk / 2 : kk);
#pragma unroll
        for (int i = 0; i < NW; i++) wn[i] = *(const uint4 *)(p + 16 * i);
        scn = Sr[k0 / a.group];
    };
    auto stage = [&](int b) {
#pragma unroll
        for (int i = 0; i < 4; i++) Af[b][mf][s_base + i][slot] = dn_order<FMT>(ra[i]);
    };
    const int nch = a.Kd / DN_KC;
    acc16 acc[2];
#pragma unroll
    for (int f = 0; f < 2; f++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[f][r] = 0.0f;
    load(0);
    stage(0);
#pragma unroll
    for (int i = 0; i < NW; i++) wc[i] = wn[i];
    scc = scn;
    __syncthreads();
    for (int c = 0; c < nch; c++) {
        load(min(c + 1, nch - 1));                   // unconditional: the last chunk again at the end
        acc16 ag[2];
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const h8 b = dn_frag<FMT>(wc, s);
#pragma unroll
            for (int f = 0; f < 2; f++) {
                const h8 av = as_h8(Af[c & 1][f][s][lane]);
                if (s == 0) {
                    acc16 z;
#pragma unroll
                    for (int r = 0; r < 16; r++) z[r] = 0.0f;
                    ag[f] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, b, z, 0, 0, 0);
                } else {
                    ag[f] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, b, ag[f], 0, 0, 0);
                }
            }
        }
        const float g = wh_f16_scale(scc);
#pragma unroll
        for (int f = 0; f < 2; f++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[f][r] = __fmaf_rn(g, ag[f][r], acc[f][r]);
        stage((c + 1) & 1);
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NW; i++) wc[i] = wn[i];
        scc = scn;
    }
    // lane (n, h), register r of M fragment f: token t0 + 32f + 8(r/4) + 4h + r%4
    if (EPI == 1) {
        if (!row_ok) return;
#pragma unroll
        for (int f = 0; f < 2; f++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int t = t0 + 32 * f + 8 * (r >> 2) + 4 * h + (r & 3);
                if (t < a.rows) ((float *)a.out)[(size_t)t * a.out_ld + row] = acc[f][r];
            }
        return;
    }
    float *ex = (float *)Af;                         // [gate wave][f][16][64]
    if (w < 2)
#pragma unroll
        for (int f = 0; f < 2; f++)
#pragma unroll
            for (int r = 0; r < 16; r++) ex[((w * 2 + f) * 16 + r) * 64 + lane] = acc[f][r];
    __syncthreads();
    if (w < 2 || !row_ok) return;
    bool bad = false;
#pragma unroll
    for (int f = 0; f < 2; f++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int t = t0 + 32 * f + 8 * (r >> 2) + 4 * h + (r & 3);
            if (t < a.rows) {
                const float v = wh_silu_mul(ex[(((w - 2) * 2 + f) * 16 + r) * 64 + lane], acc[f][r]);
                ((_Float16 *)a.out)[(size_t)t * a.out_ld + row] = to_h(v, bad);
            }
        }
    if (bad) atomicOr(a.err, ERR_RANGE);
}

extern "C" int whip_pf_dense(const whip_pf_args *a, int dec, int pair, hipStream_t s)
{
    if ((dec != DEC_Q4 && dec != DEC_Q8) || a->x_mode != 2 || a->rows < 1 || a->N < 1 || a->Kd < DN_KC ||
        a->Kd % DN_KC || a->group < DN_KC || a->group % DN_KC || a->Kd % a->group || a->rowbytes % 16 ||
        a->x_ld % 8 || (uintptr_t)a->x % 16 || !a->S0 || (pair && (!a->W1 || !a->S1)))
        return (int)hipErrorInvalidValue;
    const dim3 grid(pair ? (a->N + 63) / 64 : (a->N + 127) / 128, (a->rows + 63) / 64);
    if (dec == DEC_Q4) {
        if (pair) WHIP_LAUNCH((k_pf_dense<DEC_Q4, 0>), grid, dim3(256), 0, s, *a);
        else WHIP_LAUNCH((k_pf_dense<DEC_Q4, 1>), grid, dim3(256), 0, s, *a);
    } else {
        if (pair) WHIP_LAUNCH((k_pf_dense<DEC_Q8, 0>), grid, dim3(256), 0, s, *a);
        else WHIP_LAUNCH((k_pf_dense<DEC_Q8, 1>), grid, dim3(256), 0, s, *a);
    }
    return (int)hipGetLastError();
}

// ---- router on the matrix cores (fp32) -------------------------------------
// logits[t][e] = W[e] . x[t] with fp32 products (v_mfma_f32_32x32x2_f32),
// split over k into RT_KS ranges whose partial sums are then added in
// range order.  A workgroup: 4 waves x 32 experts, 32 tokens, one k range,
// in 64-wide chunks.  Within a chunk lane half h takes k0 + 32h + j at
// product j, so a lane's weights are 32 consecutive values of its row:
// 8 16-byte loads (F32), requested a chunk ahead.
#define RT_KS 8
#define RT_KC 64

template <int FMT>
__device__ __forceinline__ void rt_load(const uint8_t *wr, int k, uint4 *raw)
{
    if (FMT == 0) {
#pragma unroll
        for (int i = 0; i < 8; i++) raw[i] = *(const uint4 *)(wr + (size_t)(k + 4 * i) * 4);
    } else if (FMT == 2) {
        raw[0] = *(const uint4 *)(wr + k);
        raw[1] = *(const uint4 *)(wr + k + 16);
    } else {
        raw[0] = *(const uint4 *)(wr + k / 2);
    }
}

template <int FMT>
__device__ __forceinline__ float rt_w(const uint4 *raw, int j, float sc)
{
    if (FMT == 0) {
        const uint4 v = raw[j >> 2];
        const uint32_t u[4] = {v.x, v.y, v.z, v.w};
        return __uint_as_float(u[j & 3]);
    } else if (FMT == 2) {
        const uint4 v = raw[j >> 4];
        const uint32_t u[4] = {v.x, v.y, v.z, v.w};
        return (float)(int8_t)((u[(j >> 2) & 3] >> (8 * (j & 3))) & 0xff) * sc;
    } else {
        const uint4 v = raw[0];
        const uint32_t u[4] = {v.x, v.y, v.z, v.w};
        return (float)((int)((u[j >> 3] >> (4 * (j & 7))) & 15) - 8) * sc;
    }
}

template <int FMT>
__global__ void __launch_bounds__(256)
k_pf_router(whip_mat W, const void *__restrict__ x, int x_bf16, int T, float *__restrict__ part)
{
    __shared__ float Xs[32][RT_KC + 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, h = lane >> 5;
    const int e = blockIdx.x * 128 + wave * 32 + (lane & 31);
    const int t0 = blockIdx.y * 32, ks = blockIdx.z;
    const int H = W.cols;                        // H % 64 == 0
    const int klen = ((H / RT_KS) + RT_KC - 1) / RT_KC * RT_KC;
    const int k_lo = ks * klen, k_hi = min(H, k_lo + klen);
    const int ec = e < W.rows ? e : 0;
    const int ng = FMT == 0 ? 1 : (H + W.group - 1) / W.group;
    const uint8_t *wr = (const uint8_t *)W.q + (size_t)ec * W.rowbytes;
    const uint16_t *sr = FMT == 0 ? nullptr : W.qs + (size_t)ec * ng;
    acc16 acc;
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.0f;
    uint4 raw[8], rawn[8];
    float sc = 1.0f, scn = 1.0f;
    if (k_lo < k_hi) {
        rt_load<FMT>(wr, k_lo + 32 * h, rawn);
        if (FMT != 0) scn = wh_f16_scale(sr[(k_lo + 32 * h) / W.group]);
    }
    for (int k0 = k_lo; k0 < k_hi; k0 += RT_KC) {
#pragma unroll
        for (int i = 0; i < 8; i++) raw[i] = rawn[i];
        sc = scn;
        __syncthreads();
        for (int i = tid; i < 32 * RT_KC; i += 256) {
            const int m = i / RT_KC, kk = i % RT_KC, t = t0 + m;
            float v = 0.0f;
            if (t < T) {
                const size_t o = (size_t)t * H + k0 + kk;
                v = x_bf16 ? wh_bf16(((const uint16_t *)x)[o]) : ((const float *)x)[o];
            }
            Xs[m][kk] = v;
        }
        __syncthreads();
        if (k0 + RT_KC < k_hi) {                // uniform: the next chunk's weights fly now
            rt_load<FMT>(wr, k0 + RT_KC + 32 * h, rawn);
            if (FMT != 0) scn = wh_f16_scale(sr[(k0 + RT_KC + 32 * h) / W.group]);
        }
#pragma unroll
        for (int j = 0; j < 32; j++) {
            const float av = Xs[lane & 31][32 * h + j];
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av, rt_w<FMT>(raw, j, sc), acc, 0, 0, 0);
        }
    }
    if (e < W.rows)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int t = t0 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
            if (t < T) part[((size_t)ks * T + t) * W.rows + e] = acc[r];
        }
}

// The same logits for F32 router rows on the bf16 matrix cores: each weight
// split exactly into three bf16 pieces, bf16 activations used as they are
// (fp32 ones split the same way, XS = 3), so every product is exact and
// only the fp32 accumulation rounds (bf16_split.h); three or six bf16
// products cost a fifth of the fp32 ones.  A workgroup: 32 tokens x 128
// rows (a wavefront per 32 rows) x one of RT_KS column ranges, 128-column
// chunks, the A fragments staged in LDS in the operand's order (double
// buffered), a lane's 64 floats of the next chunk in flight during this one.
// Partial sums in the k_pf_router layout, added by k_pf_router_sum.
template <int XS>
__global__ void __launch_bounds__(256) k_pf_router16(whip_mat W, const void *__restrict__ x, int T,
                                                     float *__restrict__ part)
{
    __shared__ uint4 frag[2][XS][8][64];
    const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, n = lane & 31;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t0 = blockIdx.y * 32, ks = blockIdx.z, H = W.cols;
    const int nck = H / DN_KC, per = (nck + RT_KS - 1) / RT_KS;
    const int c_lo = ks * per, nc = max(0, min(nck, c_lo + per) - c_lo);
    const int row = blockIdx.x * 128 + w * 32 + n;
    const uint8_t *wr = (const uint8_t *)W.q + (size_t)min(row, W.rows - 1) * W.rowbytes;
    // staging: thread -> token sm, 16 columns at 64*shh + 16*sq (products
    // 2sq and 2sq + 1 of lane half shh); tokens past T read token 0 again
    const int sm = tid >> 3, sj = tid & 7, shh = sj >> 2, sq = sj & 3;
    const uint8_t *xrow = (const uint8_t *)x + (size_t)(t0 + sm < T ? t0 + sm : 0) * H * (XS == 1 ? 2 : 4);
    constexpr int XW = XS == 1 ? 2 : 4;
    uint4 xr[XW], wc[16], wn[16];
    auto load = [&](int c) {                         // chunk c's activations and weights (into wn)
        const int k0 = (c_lo + c) * DN_KC;
        const int e = k0 + 64 * shh + 16 * sq;
#pragma unroll
        for (int i = 0; i < XW; i++) xr[i] = *(const uint4 *)(xrow + (size_t)e * (XS == 1 ? 2 : 4) + 16 * i);
        const uint8_t *p = wr + (size_t)(k0 + 64 * h) * 4;
#pragma unroll
        for (int i = 0; i < 16; i++) wn[i] = *(const uint4 *)(p + 16 * i);
    };
    auto stage = [&](int b) {
        const int slot = shh * 32 + sm;
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++) {
            if (XS == 1) {
                frag[b][0][2 * sq + s2][slot] = xr[s2];
            } else {
                const float f[8] = {__uint_as_float(xr[2 * s2].x), __uint_as_float(xr[2 * s2].y),
                                    __uint_as_float(xr[2 * s2].z), __uint_as_float(xr[2 * s2].w),
                                    __uint_as_float(xr[2 * s2 + 1].x), __uint_as_float(xr[2 * s2 + 1].y),
                                    __uint_as_float(xr[2 * s2 + 1].z), __uint_as_float(xr[2 * s2 + 1].w)};
                uint4 p0, p1, p2;
                split3(f, p0, p1, p2);
                frag[b][0][2 * sq + s2][slot] = p0;
                frag[b][XS > 1 ? 1 : 0][2 * sq + s2][slot] = p1;
                frag[b][XS > 2 ? 2 : 0][2 * sq + s2][slot] = p2;
            }
        }
    };
    acc16 acc;
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.0f;
    if (nc > 0) {                                    // uniform
        load(0);
        stage(0);
#pragma unroll
        for (int i = 0; i < 16; i++) wc[i] = wn[i];
        __syncthreads();
        for (int c = 0; c < nc; c++) {
            load(min(c + 1, nc - 1));                // unconditional: the last chunk again at the end
#pragma unroll
            for (int s = 0; s < 8; s++) {
                bf16x8 a[XS];
#pragma unroll
                for (int p = 0; p < XS; p++) a[p] = as_b8(frag[c & 1][p][s][lane]);
                const float f[8] = {__uint_as_float(wc[2 * s].x), __uint_as_float(wc[2 * s].y),
                                    __uint_as_float(wc[2 * s].z), __uint_as_float(wc[2 * s].w),
                                    __uint_as_float(wc[2 * s + 1].x), __uint_as_float(wc[2 * s + 1].y),
                                    __uint_as_float(wc[2 * s + 1].z), __uint_as_float(wc[2 * s + 1].w)};
                uint4 bh, bm, bl;
                split3(f, bh, bm, bl);
                // smallest terms first; for fp32 x the three below 2^-24 of
                // the product are left out
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], as_b8(bl), acc, 0, 0, 0);
                if (XS == 3) {
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[XS > 2 ? 2 : 0], as_b8(bh), acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[XS > 1 ? 1 : 0], as_b8(bm), acc, 0, 0, 0);
                }
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], as_b8(bm), acc, 0, 0, 0);
                if (XS == 3) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[XS > 1 ? 1 : 0], as_b8(bh), acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], as_b8(bh), acc, 0, 0, 0);
            }
            stage((c + 1) & 1);
            __syncthreads();
#pragma unroll
            for (int i = 0; i < 16; i++) wc[i] = wn[i];
        }
    }
    if (row >= W.rows) return;
    // lane (n, h), register r: token t0 + 8(r/4) + 4h + r%4
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int t = t0 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (t < T) part[((size_t)ks * T + t) * W.rows + row] = acc[r];
    }
}

__global__ void __launch_bounds__(256)
k_pf_router_sum(const float *__restrict__ part, int n, float *__restrict__ logits)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)n) return;
    float s = part[i];
    for (int ks = 1; ks < RT_KS; ks++) s += part[(size_t)ks * n + i];
    logits[i] = s;
}

extern "C" size_t whip_pf_router_part_floats(int T, int E) { return (size_t)RT_KS * T * E; }

extern "C" int whip_pf_router(const whip_mat *W, const void *x, int x_bf16, int T, float *part,
                              float *logits, hipStream_t s)
{
    // 32-wide k runs: a Q8G/Q4G run stays inside one scale group
    if (W->cols % RT_KC || (W->fmt != 0 && (W->group % 32 || (W->fmt != 2 && W->fmt != 3))))
        return (int)hipErrorInvalidValue;
    dim3 grid((W->rows + 127) / 128, (T + 31) / 32, RT_KS);
    const bool split = W->fmt == 0 && W->cols % DN_KC == 0 && W->rowbytes % 16 == 0 && (uintptr_t)x % 16 == 0 &&
                       W->cols % 8 == 0;
    if (split && x_bf16) hipLaunchKernelGGL(k_pf_router16<1>, grid, dim3(256), 0, s, *W, x, T, part);
    else if (split) hipLaunchKernelGGL(k_pf_router16<3>, grid, dim3(256), 0, s, *W, x, T, part);
    else if (W->fmt == 0) hipLaunchKernelGGL(k_pf_router<0>, grid, dim3(256), 0, s, *W, x, x_bf16, T, part);
    else if (W->fmt == 2) hipLaunchKernelGGL(k_pf_router<2>, grid, dim3(256), 0, s, *W, x, x_bf16, T, part);
    else hipLaunchKernelGGL(k_pf_router<3>, grid, dim3(256), 0, s, *W, x, x_bf16, T, part);
    const int n = T * W->rows;
    hipLaunchKernelGGL(k_pf_router_sum, dim3((n + 255) / 256), dim3(256), 0, s, part, n, logits);
    return (int)hipGetLastError();
}

// ---- combine ---------------------------------------------------------------
// y[t][c] = sum over t's pairs in ascending expert order (zero weights and
// unbound experts skipped) of w * Y[p][c], then + sh[t][c].
__global__ void __launch_bounds__(256)
k_pf_combine(const int32_t *__restrict__ tok_pairs, const int32_t *__restrict__ pair_exp,
             const float *__restrict__ pair_w, const uint8_t *const *__restrict__ recs, int K, int E,
             const float *__restrict__ Y, int H, const float *__restrict__ sh, float *__restrict__ y)
{
    const int t = blockIdx.y, c = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (c >= H) return;
    float4 o = make_float4(0, 0, 0, 0);
    for (int j = 0; j < K; j++) {
        const int p = tok_pairs[t * K + j];
        const float w = pair_w[p];
        const int e = pair_exp[p];
        if (w == 0.0f || e >= E || recs[e] == nullptr) continue;
        const float4 v = *(const float4 *)(Y + (size_t)p * H + c);
        o.x = __fadd_rn(o.x, __fmul_rn(w, v.x)); o.y = __fadd_rn(o.y, __fmul_rn(w, v.y));
        o.z = __fadd_rn(o.z, __fmul_rn(w, v.z)); o.w = __fadd_rn(o.w, __fmul_rn(w, v.w));
    }
    if (sh) {
        const float4 v = *(const float4 *)(sh + (size_t)t * H + c);
        o.x = __fadd_rn(o.x, v.x); o.y = __fadd_rn(o.y, v.y); o.z = __fadd_rn(o.z, v.z); o.w = __fadd_rn(o.w, v.w);
    }
    *(float4 *)(y + (size_t)t * H + c) = o;
}

extern "C" int whip_pf_combine(const int32_t *tok_pairs, const int32_t *pair_exp, const float *pair_w,
                               const uint8_t *const *recs, int T, int K, int E, const float *Y, int H,
                               const float *sh, float *y, hipStream_t s)
{
    if (H % 4) return (int)hipErrorInvalidValue;
    dim3 grid((H / 4 + 255) / 256, T);
    hipLaunchKernelGGL(k_pf_combine, grid, dim3(256), 0, s, tok_pairs, pair_exp, pair_w, recs, K, E, Y, H, sh, y);
    return (int)hipGetLastError();
}
