// SPDX-License-Identifier: Apache-2.0
//
// route.h — the routing body (scores, group limit, top-k) shared by the
// routing kernel and the launch that pairs routing with the shared
// expert's down projection.  See route.hip for the engine semantics.
#pragma once
#include "common.h"
#include "launch.h"
#include "trace.h"
#include "log1pf.h"

#define MAXE 1024

#define NEG_INF (-__int_as_float(0x7f800000))

// (a, ea) precedes (b, eb) in the engine's selection order: larger value
// first, the lower id among equal values (a strict-greater scan keeps the
// first maximum it meets).
__device__ __forceinline__ bool before(float a, int ea, float b, int eb)
{
    return a > b || (a == b && ea < eb);
}

// Selection key: one unsigned 64-bit number whose order is the selection
// order.  High word: the value's bits mapped so unsigned order is float
// order (-0 is first folded into +0, which compares equal to it); low word:
// ~e, so the lower id is the larger key among equal values.  0 marks "not a
// candidate" (value not above the scan's floor -1e30, NaN, or taken).
__device__ __forceinline__ uint64_t sel_key(float v, int e)
{
    if (!(v > -1e30f)) return 0;
    const uint32_t u = __float_as_uint(__fadd_rn(v, 0.0f));
    const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)o << 32) | (uint32_t)~(uint32_t)e;
}

// Wave maxima over the butterfly of common.h's wave_sum.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k)
{
    uint32_t lo = (uint32_t)k, hi = (uint32_t)(k >> 32);
    auto mx = [&](uint32_t l2, uint32_t h2) {
        const uint64_t a = ((uint64_t)hi << 32) | lo, b = ((uint64_t)h2 << 32) | l2;
        if (b > a) { lo = l2; hi = h2; }
    };
    mx(dpp32<0xB1>(lo), dpp32<0xB1>(hi));     // quad_perm [1,0,3,2]
    mx(dpp32<0x4E>(lo), dpp32<0x4E>(hi));     // quad_perm [2,3,0,1]
    mx(dpp32<0x141>(lo), dpp32<0x141>(hi));   // row_half_mirror
    mx(dpp32<0x140>(lo), dpp32<0x140>(hi));   // row_mirror
    {
        auto a = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
        auto b = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
        lo = a[0]; hi = b[0];
        mx(a[1], b[1]);
    }
    {
        auto a = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
        auto b = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
        lo = a[0]; hi = b[0];
        mx(a[1], b[1]);
    }
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ float wave_max_f32(float v)
{
    // values are never NaN here, so the order-free max is exact
    uint32_t u = __float_as_uint(v);
    auto mx = [&](uint32_t o) { const float a = __uint_as_float(o); if (a > __uint_as_float(u)) u = o; };
    mx(dpp32<0xB1>(u));
    mx(dpp32<0x4E>(u));
    mx(dpp32<0x141>(u));
    mx(dpp32<0x140>(u));
    { auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false); u = a[0]; mx(a[1]); }
    { auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false); u = a[0]; mx(a[1]); }
    return __uint_as_float(u);
}

// One wavefront per token; lane L holds experts L*NPL .. L*NPL+NPL-1 in
// registers.  Each of the K selection passes is one wave max over the
// selection keys, which picks exactly the expert the engine's pass picks.
// Every wavefront that runs it for one token computes the same values and
// writes them to the same places, so a workgroup of several wavefronts may
// run it (its barriers then meet).  lds: ROUTE_LDS_FLOATS(NPL) floats of
// workgroup scratch.  COH: the logits were written by other workgroups of
// the same launch, so they are read device-coherent (past the
// non-coherent caches).  etab: expf's table (NULL: the constant one).
#define ROUTE_LDS_FLOATS(NPL) (64 * (NPL) + 128)

template <typename T> __device__ __forceinline__ T coh_ld(const T *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T> __device__ __forceinline__ void coh_st(T *p, T v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One token's selection by one wavefront from its logits in registers:
// lane L holds experts L*NPL .. L*NPL+NPL-1 (sc: their logits; entries past
// E are ignored).  Lane p < K returns the p-th selected expert (myid, -1
// when fewer than K experts are candidates: err bit 2) and its weight.
// Every wavefront that runs it for one token computes the same values, so a
// workgroup of several wavefronts may run it (its barriers then meet).
template <int NPL>
__device__ __forceinline__ void
route_wave(const whip_route_cfg &c, float (&sc)[NPL], const float *__restrict__ bias, int L,
           int *__restrict__ err, float *lds, const uint64_t *et, int &myid, float &myw)
{
    float *s_v = lds, *s_g = lds + 64 * NPL;
    int *s_keep = (int *)(lds + 64 * NPL + 64);
    const int E = c.E, K = c.K;
    float sel[NPL];
#pragma unroll
    for (int j = 0; j < NPL; j++) sc[j] = L * NPL + j < E ? sc[j] : 0.0f;

    if (c.score_func == 1) {
        // max (order-free), then the engine's sum in expert order
        float mx = -1e30f;
#pragma unroll
        for (int j = 0; j < NPL; j++)
            if (L * NPL + j < E && sc[j] > mx) mx = sc[j];
        mx = wave_max_f32(mx);
#pragma unroll
        for (int j = 0; j < NPL; j++) {
            const int e = L * NPL + j;
            sc[j] = e < E ? wh_expf_t(__fsub_rn(sc[j], mx), et) : 0.0f;
            if (e < E) s_v[e] = sc[j];
        }
        __syncthreads();
        float sum = 0.0f;
        for (int k = 0; k < E; k++) sum = __fadd_rn(sum, s_v[k]);
#pragma unroll
        for (int j = 0; j < NPL; j++) sc[j] = __fdiv_rn(sc[j], sum);
    } else if (c.score_func == 2) {
#pragma unroll
        for (int j = 0; j < NPL; j++) {
            const float l = sc[j];
            const float sp = l > 30.0f ? l : wh_log1pf(wh_expf_t(l, et));
            sc[j] = sqrtf(sp);              // correctly rounded (HIP's __fsqrt_rn is the native approximation)
        }
    } else {
#pragma unroll
        for (int j = 0; j < NPL; j++) sc[j] = __fdiv_rn(1.0f, __fadd_rn(1.0f, wh_expf_t(-sc[j], et)));
    }
#pragma unroll
    for (int j = 0; j < NPL; j++) {
        const int e = L * NPL + j;
        sel[j] = e < E ? __fadd_rn(sc[j], bias ? bias[e] : 0.0f) : NEG_INF;
    }

    if (c.n_group > 1) {
        // a group's score: the sum of its two largest values above -inf
        // (-inf when it has fewer); keep the topk_group groups that come
        // first under `before` among those above -inf; mask the rest
        const int G = c.n_group, gs = E / G;
        const int lpg = gs % NPL == 0 ? gs / NPL : 0;           // lanes per group
        int keep;
        if (lpg > 0 && (lpg & (lpg - 1)) == 0) {
            // groups tile the wave in aligned runs of lpg lanes: lane-local
            // top two, then a butterfly inside the run (values only: which
            // expert holds them does not matter)
            float a = NEG_INF, b = NEG_INF;
#pragma unroll
            for (int j = 0; j < NPL; j++) {
                const float v = sel[j];
                if (v > a) { b = a; a = v; }
                else if (v > b) b = v;
            }
            for (int o = 1; o < lpg; o <<= 1) {
                const float pa = __shfl_xor(a, o, 64), pb = __shfl_xor(b, o, 64);
                const float hi = fmaxf(a, pa), lo = fminf(a, pa);
                b = fmaxf(lo, fmaxf(b, pb));
                a = hi;
            }
            const float mine = __fadd_rn(a, gs > 1 ? b : 0.0f);
            const int g = L / lpg;
            int rk = 0;
            for (int k = 0; k < G; k++) {
                const float o = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), k * lpg));
                rk += (o > NEG_INF) && before(o, k, mine, g);
            }
            keep = mine > NEG_INF && rk < c.topk_group;
        } else {
            __syncthreads();                                     // softmax's reads of s_v
#pragma unroll
            for (int j = 0; j < NPL; j++)
                if (L * NPL + j < E) s_v[L * NPL + j] = sel[j];
            __syncthreads();
            if (L < G) {
                float a = NEG_INF, b = NEG_INF;
                for (int k = L * gs; k < (L + 1) * gs; k++) {
                    const float v = s_v[k];
                    if (v > a) { b = a; a = v; }
                    else if (v > b) b = v;
                }
                s_g[L] = __fadd_rn(a, gs > 1 ? b : 0.0f);
            }
            __syncthreads();
            if (L < G) {
                const float mine = s_g[L];
                int rk = 0;
                for (int k = 0; k < G; k++) {
                    const float o = s_g[k];
                    rk += (o > NEG_INF) && before(o, k, mine, L);
                }
                s_keep[L] = mine > NEG_INF && rk < c.topk_group;
            }
            __syncthreads();
            keep = -1;
        }
#pragma unroll
        for (int j = 0; j < NPL; j++) {
            const int e = L * NPL + j;
            if (e < E && !(keep >= 0 ? keep : s_keep[e / gs])) sel[j] = NEG_INF;
        }
    }

    uint64_t key[NPL];
#pragma unroll
    for (int j = 0; j < NPL; j++) key[j] = L * NPL + j < E ? sel_key(sel[j], L * NPL + j) : 0;

    float wsum = 0.0f;
    int ok = 1;
    myw = 0.0f;
    myid = -1;
    for (int p = 0; p < K; p++) {
        uint64_t best = key[0];
#pragma unroll
        for (int j = 1; j < NPL; j++) best = key[j] > best ? key[j] : best;
        best = wave_max_u64(best);
        if (best == 0) { ok = 0; break; }
        const int e = __builtin_amdgcn_readfirstlane((int)~(uint32_t)best);
        const int owner = e / NPL, slot = e - owner * NPL;
        float v = sc[0];
#pragma unroll
        for (int j = 1; j < NPL; j++) v = j == slot ? sc[j] : v;
        const float wf = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), owner));
        if (L == owner) {
#pragma unroll
            for (int j = 0; j < NPL; j++) if (j == slot) key[j] = 0;
        }
        wsum = __fadd_rn(wsum, wf);
        if (L == p) { myid = e; myw = wf; }
    }
    if (ok) {
        if (c.renorm && K > 1) myw = __fdiv_rn(myw, __fadd_rn(wsum, 1e-20f));
        myw = __fmul_rn(myw, c.routed_scale);
    } else {
        myid = -1;
        myw = 0.0f;
        if (L == 0) atomicOr(err, 2);
    }
}

template <int NPL, bool COH = false>
__device__ __forceinline__ void
route_body(const whip_route_cfg &c, const float *__restrict__ logits, const float *__restrict__ bias,
           int T, int t, int L, int32_t *__restrict__ ids, float *__restrict__ wout,
           int32_t *__restrict__ pair_tok, int32_t *__restrict__ pair_exp, float *__restrict__ pair_w,
           int32_t *__restrict__ tok_pairs, const uint8_t *const *__restrict__ recs,
           const uint8_t **__restrict__ pair_rec, int *__restrict__ err, float *lds,
           const uint64_t *etab = nullptr)
{
    const uint64_t *et = etab ? etab : wh_exp_tab;
    const int E = c.E, K = c.K;
    const float *lg = logits + (size_t)t * E;
    float sc[NPL];
#pragma unroll
    for (int j = 0; j < NPL; j++) {
        const int e = L * NPL + j;
        const int ec = e < E ? e : 0;
        const float l = COH ? coh_ld(lg + ec) : lg[ec];
        sc[j] = e < E ? l : 0.0f;
    }
    int myid;
    float myw;
    route_wave<NPL>(c, sc, bias, L, err, lds, et, myid, myw);
    if (L < K) {
        ids[(size_t)t * K + L] = myid;
        wout[(size_t)t * K + L] = myw;
        if (pair_exp && T == 1) {
            pair_tok[L] = 0;
            pair_exp[L] = myid < 0 ? E : myid;       // E: the table's NULL sentinel
            pair_w[L] = myw;
            tok_pairs[L] = L;
            // the pair's record, for kernels that start on it at once
            if (pair_rec) pair_rec[L] = myid < 0 ? nullptr : recs[myid];
        }
    }
}

// ---- routing by the whole workgroup ----------------------------------------------
// One token's selection with the engine's semantics (route.h: the same
// scores, group limit and keys), computed without its K dependent passes:
// the keys are distinct (the expert id is in the low word), so the expert
// the engine's pass p picks is the one with exactly p keys above it.  Each
// expert's rank is counted by NT/E threads over slices of the keys in LDS
// (NT: the workgroup's threads, at least E).
// The weights are summed for the renormalisation in selection order, as
// the passes add them.  Every thread calls it; results in s_ids/s_w/s_rec
// (K entries; ids -1, weights 0, records NULL and err bit 2 when fewer than
// K experts are candidates).
struct route_lds {
    float *sc, *sel;           // [E] scores, biased scores (may share storage unless TWO)
    uint64_t *key;             // [E]
    int *rank;                 // [E]
    float *g;                  // [64] group scores
    int *keep;                 // [64]
    float *wraw;               // [64]
    uint64_t *cand;            // [64] (TWO only)
};

// Keys above `key` among the lanes of this lane's segment of the wavefront
// (seg 1 .. 64 lanes, a power of two, aligned): the segment's keys come to
// every lane by row rotations (DPP) of its own row of 16 and, for
// segments past one row, of the rows the lane-swaps bring; the rotations
// are independent of each other, so they issue back to back.
template <int R> __device__ __forceinline__ void cnt_rot(uint32_t slo, uint32_t shi, uint64_t key, int i, int seg,
                                                        bool self, int &n)
{
    const uint32_t olo = R ? dpp32<0x120 + R>(slo) : slo, ohi = R ? dpp32<0x120 + R>(shi) : shi;
    const uint64_t o = ((uint64_t)ohi << 32) | olo;
    const int j = (i - R) & 15;                      // the source lane's place in its row
    n += (o > key) & !(self && R == 0) & (seg >= 16 || (j ^ i) < seg);
}
__device__ __forceinline__ int seg_rank(uint64_t key, int seg)
{
    const int lane = threadIdx.x & 63, i = lane & 15;
    const bool odd16 = (lane >> 4) & 1, hi32 = lane >= 32;
    int n = 0;
    auto row = [&](uint32_t slo, uint32_t shi, bool self) {
        cnt_rot<0>(slo, shi, key, i, seg, self, n);   cnt_rot<1>(slo, shi, key, i, seg, self, n);
        cnt_rot<2>(slo, shi, key, i, seg, self, n);   cnt_rot<3>(slo, shi, key, i, seg, self, n);
        cnt_rot<4>(slo, shi, key, i, seg, self, n);   cnt_rot<5>(slo, shi, key, i, seg, self, n);
        cnt_rot<6>(slo, shi, key, i, seg, self, n);   cnt_rot<7>(slo, shi, key, i, seg, self, n);
        cnt_rot<8>(slo, shi, key, i, seg, self, n);   cnt_rot<9>(slo, shi, key, i, seg, self, n);
        cnt_rot<10>(slo, shi, key, i, seg, self, n);  cnt_rot<11>(slo, shi, key, i, seg, self, n);
        cnt_rot<12>(slo, shi, key, i, seg, self, n);  cnt_rot<13>(slo, shi, key, i, seg, self, n);
        cnt_rot<14>(slo, shi, key, i, seg, self, n);  cnt_rot<15>(slo, shi, key, i, seg, self, n);
    };
    auto p16 = [&](uint32_t v) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return odd16 ? r[0] : r[1];                  // the same place in the other row of the pair
    };
    auto p32 = [&](uint32_t v) {
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return hi32 ? r[0] : r[1];                   // the same place in the other half
    };
    const uint32_t lo = (uint32_t)key, hi = (uint32_t)(key >> 32);
    row(lo, hi, true);
    if (seg >= 32) row(p16(lo), p16(hi), false);     // uniform
    if (seg >= 64) {
        const uint32_t lo2 = p32(lo), hi2 = p32(hi);
        row(lo2, hi2, false);
        row(p16(lo2), p16(hi2), false);
    }
    return n;
}

// TWO: the ranks in two levels where they fit, for a workgroup too small
// to split every expert's count over several threads.  Level one: each
// lane's rank among the lanes of its segment (its group when groups are a
// power of two of at most 64 experts, else its wavefront), by moving the
// segment's keys across lanes (seg_rank); a segment's experts of rank
// below K are the only ones that can be selected.  Level two: one wavefront ranks
// those candidates (at most 64) the same way.  A key's rank is the number
// of keys above it either way, so the selection is the same.
template <int NT, bool TWO = false>
__device__ __forceinline__ void route_wg(const whip_route_cfg &c, float l, float bias_e,
                                         const uint8_t *const *s_recs, const uint64_t *etab,
                                         const route_lds &R, int32_t *s_ids, float *s_w,
                                         const uint8_t **s_rec, int *err)
{
    const int tid = threadIdx.x, E = c.E, K = c.K;
    float sc = 0.0f;
    if (tid < E) {
        if (c.score_func == 2) {
            const float sp = l > 30.0f ? l : wh_log1pf(wh_expf_t(l, etab));
            sc = sqrtf(sp);
        } else if (c.score_func == 0) {
            sc = __fdiv_rn(1.0f, __fadd_rn(1.0f, wh_expf_t(-l, etab)));
        } else {
            sc = l;
        }
        R.sc[tid] = sc;
    }
    if (c.score_func == 1) {                          // softmax: max, then the sum in expert order
        __syncthreads();
        if (tid < 64) {
            float mx = -1e30f;
            for (int e = tid; e < E; e += 64) mx = R.sc[e] > mx ? R.sc[e] : mx;
            mx = wave_max_f32(mx);
            if (tid == 0) R.g[0] = mx;
        }
        __syncthreads();
        if (tid < E) {
            sc = wh_expf_t(__fsub_rn(sc, R.g[0]), etab);
            R.sc[tid] = sc;
        }
        __syncthreads();
        if (tid == 0) {
            float sum = 0.0f;
            for (int e = 0; e < E; e++) sum = __fadd_rn(sum, R.sc[e]);
            R.g[1] = sum;
        }
        __syncthreads();
        if (tid < E) {
            sc = __fdiv_rn(sc, R.g[1]);
            R.sc[tid] = sc;
        }
    }
    WT(0, 12);
    const float selv = tid < E ? __fadd_rn(sc, bias_e) : NEG_INF;
    if (tid < E) R.sel[tid] = selv;
    const int G = c.n_group > 1 ? c.n_group : 1, gs = E / G;
    if (G > 1 && gs <= 64 && (gs & (gs - 1)) == 0) {
        // a group's score: the sum of its two largest values above -inf,
        // merged across the group's lanes (values only)
        float a = selv, b = NEG_INF;
        for (int o = 1; o < gs; o <<= 1) {
            const float pa = __shfl_xor(a, o, 64), pb = __shfl_xor(b, o, 64);
            const float hi = fmaxf(a, pa), lo = fminf(a, pa);
            b = fmaxf(lo, fmaxf(b, pb));
            a = hi;
        }
        if (tid < E && tid % gs == 0) R.g[tid / gs] = __fadd_rn(a, gs > 1 ? b : 0.0f);
    }
    __syncthreads();
    if (G > 1) {
        if (!(gs <= 64 && (gs & (gs - 1)) == 0)) {
            if (tid < G) {
                float a = NEG_INF, b = NEG_INF;
                for (int k = tid * gs; k < (tid + 1) * gs; k++) {
                    const float v = R.sel[k];
                    if (v > a) { b = a; a = v; }
                    else if (v > b) b = v;
                }
                R.g[tid] = __fadd_rn(a, gs > 1 ? b : 0.0f);
            }
            __syncthreads();
        }
        if (tid < G) {
            const float mine = R.g[tid];
            int rk = 0;
            for (int k = 0; k < G; k++) {
                const float o = R.g[k];
                rk += (o > NEG_INF) && before(o, k, mine, tid);
            }
            R.keep[tid] = mine > NEG_INF && rk < c.topk_group;
        }
        __syncthreads();
    }
    WT(0, 13);
    uint64_t key = 0;
    if (tid < E) {
        const bool kept = G > 1 ? R.keep[tid / gs] != 0 : true;
        key = sel_key(kept ? selv : NEG_INF, tid);
        R.key[tid] = key;
        R.rank[tid] = 0;
    }
    const int seg = (G > 1 && gs <= 64 && (gs & (gs - 1)) == 0) ? gs : 64;
    const int kc = K < seg ? K : seg, ns = (E + seg - 1) / seg * kc;
    const bool two = TWO && ns <= 64;                 // uniform
    if (two && tid < 64) R.cand[tid] = 0;
    const int nvalid = __syncthreads_count(key != 0);
    WT(0, 14);
    if (two) {
        const int r1 = seg_rank(key, seg);
        if (tid < E && key && r1 < kc) R.cand[(tid / seg) * kc + r1] = key;
        __syncthreads();
        if (tid < 64) {
            const uint64_t cv = tid < ns ? R.cand[tid] : 0;
            const uint32_t clo = (uint32_t)cv;
            const int r2 = seg_rank(cv, 64);
            if (cv && r2 < K) {
                const int e = (int)~clo;                 // the key's low word
                s_ids[r2] = e;
                R.wraw[r2] = R.sc[e];
                s_rec[r2] = s_recs[e];
            }
        }
        __syncthreads();
    } else {
        // NT/E threads per expert, each over a slice of the keys, eight
        // loads in flight at a time; the lanes of a wavefront hold
        // consecutive experts and read the same key (one LDS broadcast)
        const int Q = NT / E, part = tid / E, e = tid % E;   // a wavefront reads one key at a time
        const int per = (E + Q - 1) / Q, lo = part * per, hi = min(E, lo + per);
        if (e < E) {
            const uint64_t mine = R.key[e];
            int n = 0;
            int k = lo;
            for (; k + 8 <= hi; k += 8) {
                uint64_t q[8];
#pragma unroll
                for (int j = 0; j < 8; j++) q[j] = R.key[k + j];
#pragma unroll
                for (int j = 0; j < 8; j++) n += q[j] > mine;
            }
            for (; k < hi; k++) n += R.key[k] > mine;
            if (mine && n) atomicAdd(R.rank + e, n);
        }
        __syncthreads();
        if (tid < E && R.key[tid] && R.rank[tid] < K) {
            const int r = R.rank[tid];
            s_ids[r] = tid;
            R.wraw[r] = sc;
            s_rec[r] = s_recs[tid];
        }
        __syncthreads();
    }
    WT(0, 15);
    if (tid < K) {
        const bool ok = nvalid >= K;
        float wsum = 0.0f;
        for (int p = 0; p < K; p++) wsum = __fadd_rn(wsum, R.wraw[p]);
        float myw = R.wraw[tid];
        if (ok) {
            if (c.renorm && K > 1) myw = __fdiv_rn(myw, __fadd_rn(wsum, 1e-20f));
            myw = __fmul_rn(myw, c.routed_scale);
        } else {
            myw = 0.0f;
            s_ids[tid] = -1;
            s_rec[tid] = nullptr;
            if (tid == 0) atomicOr(err, 2);
        }
        s_w[tid] = myw;
    }
    __syncthreads();
}


// ---- routing by the whole workgroup, sorted in registers -----------------------
// The same selection as route_wg (scores, group limit, keys, selection order,
// weights summed in selection order) with far fewer instructions, for a
// workgroup of NT threads (a multiple of 64, >= E) whose thread e holds
// expert e's logit:
//  - group scores: each group's top two merged across its lanes by DPP and
//    lane swaps (groups of a power of two experts, at most 64, so a group
//    lies inside one wavefront), else as route_wg does;
//  - top K: each wavefront holding experts sorts its 64 keys (one per
//    lane) with a bitonic network on lane moves; the wavefronts' first K
//    are then sorted once more by wavefront 0.  Keys are distinct, so the
//    order of the sorted keys is the engine's selection order.
// LDS: ROUTE_FAST_FLOATS(E) floats at lds (16-byte aligned).  E <= 64 * 64 / K
// (the candidates fit one wavefront).  Results in s_ids/s_w/s_rec (K <= 64
// entries; ids -1, weights 0, records NULL and err bit 2 when fewer than K
// experts are candidates).  Every thread calls it.
#define ROUTE_FAST_FLOATS(E) (2 * (E) + 2 * (E) + 128 + 128 + 64 + 8)

__device__ __forceinline__ void top2_merge(float &a, float &b, float pa, float pb)
{
    const float hi = fmaxf(a, pa), lo = fminf(a, pa);
    b = fmaxf(lo, fmaxf(b, pb));
    a = hi;
}

// the key of lane i ^ (2^s - 1) (FLIP) or i ^ d (otherwise), a whole wave
template <bool FLIP, int D> __device__ __forceinline__ uint32_t lane_partner(uint32_t v, int lane)
{
    const bool odd16 = (lane >> 4) & 1, hi32 = lane >= 32;
    auto p16 = [&](uint32_t x) { const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false); return odd16 ? r[0] : r[1]; };
    auto p32 = [&](uint32_t x) { const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false); return hi32 ? r[0] : r[1]; };
    if (FLIP) {                                      // D = 2^s: mirror inside blocks of D lanes
        if (D == 2) return dpp32<0xB1>(v);           // i ^ 1
        if (D == 4) return dpp32<0x1B>(v);           // quad_perm [3,2,1,0]: i ^ 3
        if (D == 8) return dpp32<0x141>(v);          // row_half_mirror: i ^ 7
        if (D == 16) return dpp32<0x140>(v);         // row_mirror: i ^ 15
        if (D == 32) return p16(dpp32<0x140>(v));    // i ^ 31
        return p32(p16(dpp32<0x140>(v)));            // i ^ 63
    }
    if (D == 1) return dpp32<0xB1>(v);
    if (D == 2) return dpp32<0x4E>(v);               // quad_perm [2,3,0,1]
    if (D == 4) return dpp32<0x1B>(dpp32<0x141>(v)); // (i ^ 7) ^ 3
    if (D == 8) return dpp32<0x128>(v);              // row_ror:8 is i ^ 8 in a row of 16
    if (D == 16) return p16(v);
    return p32(v);                                   // D == 32
}

// one comparator layer: the lower lane of each pair keeps the larger key
template <bool FLIP, int D> __device__ __forceinline__ uint64_t cmp_layer(uint64_t v, int lane)
{
    const uint32_t lo = lane_partner<FLIP, D>((uint32_t)v, lane);
    const uint32_t hi = lane_partner<FLIP, D>((uint32_t)(v >> 32), lane);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    const bool upper = FLIP ? (lane & (D >> 1)) != 0 : (lane & D) != 0;
    return (o > v) != upper ? o : v;
}

// the wave's 64 keys sorted, largest at lane 0
__device__ __forceinline__ uint64_t wave_sort_desc(uint64_t v, int lane)
{
    v = cmp_layer<true, 2>(v, lane);
    v = cmp_layer<true, 4>(v, lane);  v = cmp_layer<false, 1>(v, lane);
    v = cmp_layer<true, 8>(v, lane);  v = cmp_layer<false, 2>(v, lane);  v = cmp_layer<false, 1>(v, lane);
    v = cmp_layer<true, 16>(v, lane); v = cmp_layer<false, 4>(v, lane);  v = cmp_layer<false, 2>(v, lane);
    v = cmp_layer<false, 1>(v, lane);
    v = cmp_layer<true, 32>(v, lane); v = cmp_layer<false, 8>(v, lane);  v = cmp_layer<false, 4>(v, lane);
    v = cmp_layer<false, 2>(v, lane); v = cmp_layer<false, 1>(v, lane);
    v = cmp_layer<true, 64>(v, lane); v = cmp_layer<false, 16>(v, lane); v = cmp_layer<false, 8>(v, lane);
    v = cmp_layer<false, 4>(v, lane); v = cmp_layer<false, 2>(v, lane);  v = cmp_layer<false, 1>(v, lane);
    return v;
}

template <int NT>
__device__ __forceinline__ void route_fast(const whip_route_cfg &c, float l, float bias_e,
                                           const uint8_t *const *s_tab, const uint64_t *etab, float *lds,
                                           int32_t *s_ids, float *s_w, const uint8_t **s_rec, int *err)
{
    constexpr int NWV = NT / 64;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, E = c.E, K = c.K;
    const int ewv = (E + 63) >> 6;                           // wavefronts holding experts
    uint64_t *s_cand = (uint64_t *)lds;                      // [64] the wavefronts' first K
    float *s_g = lds + 128;                                  // [64] group scores (16-byte aligned)
    float *s_part = s_g + 64;                                // [NWV + 1] softmax
    float *s_sc = s_part + 64;                               // [E]
    float *s_sel = s_sc + E;                                 // [E] (group scan fallback)
    // scores
    float sc = 0.0f;
    if (tid < E) {
        if (c.score_func == 2) {
            const float sp = l > 30.0f ? l : wh_log1pf(wh_expf_t(l, etab));
            sc = sqrtf(sp);
        } else if (c.score_func == 0) {
            sc = __fdiv_rn(1.0f, __fadd_rn(1.0f, wh_expf_t(-l, etab)));
        }
    }
    if (c.score_func == 1) {                                 // softmax: max, then the sum in expert order
        if (wv < ewv) {
            const float mx_w = wave_max_f32(tid < E ? l : -1e30f);
            if (lane == 0) s_part[wv] = mx_w;
        }
        __syncthreads();
        float mx = -1e30f;
        for (int w = 0; w < ewv; w++) mx = s_part[w] > mx ? s_part[w] : mx;
        if (tid < E) {
            sc = wh_expf_t(__fsub_rn(l, mx), etab);
            s_sc[tid] = sc;
        }
        __syncthreads();
        if (tid == 0) {
            float sum = 0.0f;
            for (int e = 0; e < E; e++) sum = __fadd_rn(sum, s_sc[e]);
            s_part[NWV] = sum;
        }
        __syncthreads();
        if (tid < E) sc = __fdiv_rn(sc, s_part[NWV]);
    }
    if (tid < E) s_sc[tid] = sc;
    WT_L(1);
    const float selv = tid < E ? __fadd_rn(sc, bias_e) : NEG_INF;
    // group limit
    const int G = c.n_group > 1 ? c.n_group : 1;
    const int gsh = G > 1 ? __builtin_ctz((unsigned)(E / G)) : 0, gs = E / G;
    bool kept = true;
    if (G > 1) {
        if (gs <= 64 && (gs & (gs - 1)) == 0) {
            if (wv < ewv) {                                  // uniform
                float a = selv, b = NEG_INF;
                auto step = [&](uint32_t pa, uint32_t pb) {
                    top2_merge(a, b, __uint_as_float(pa), __uint_as_float(pb));
                };
                if (gs > 1) step(dpp32<0xB1>(__float_as_uint(a)), dpp32<0xB1>(__float_as_uint(b)));
                if (gs > 2) step(dpp32<0x4E>(__float_as_uint(a)), dpp32<0x4E>(__float_as_uint(b)));
                if (gs > 4) step(dpp32<0x141>(__float_as_uint(a)), dpp32<0x141>(__float_as_uint(b)));
                if (gs > 8) step(dpp32<0x140>(__float_as_uint(a)), dpp32<0x140>(__float_as_uint(b)));
                if (gs > 16)
                    step(lane_partner<false, 16>(__float_as_uint(a), lane),
                         lane_partner<false, 16>(__float_as_uint(b), lane));
                if (gs > 32)
                    step(lane_partner<false, 32>(__float_as_uint(a), lane),
                         lane_partner<false, 32>(__float_as_uint(b), lane));
                if (tid < E && (tid & (gs - 1)) == 0) s_g[tid >> gsh] = __fadd_rn(a, gs > 1 ? b : 0.0f);
            }
        } else {
            if (tid < E) s_sel[tid] = selv;
            __syncthreads();
            if (tid < G) {
                float a = NEG_INF, b = NEG_INF;
                for (int k = tid * gs; k < (tid + 1) * gs; k++) {
                    const float v = s_sel[k];
                    if (v > a) { b = a; a = v; }
                    else if (v > b) b = v;
                }
                s_g[tid] = __fadd_rn(a, gs > 1 ? b : 0.0f);
            }
        }
        __syncthreads();
        WT_L(2);
        if (tid < E) {
            // every group's score, four to a 16-byte read (s_g has 64
            // entries; those past G are not compared)
            const int g = (gs & (gs - 1)) == 0 ? tid >> gsh : tid / gs;
            const float mine = s_g[g];
            int rk = 0;
            for (int k0 = 0; k0 < G; k0 += 8) {
                const float4 q0 = *(const float4 *)(s_g + k0), q1 = *(const float4 *)(s_g + k0 + 4);
                const float o[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
                for (int i = 0; i < 8; i++)
                    rk += (k0 + i < G) && (o[i] > NEG_INF) && before(o[i], k0 + i, mine, g);
            }
            kept = mine > NEG_INF && rk < c.topk_group;
        }
    }
    WT_L(3);
    // each wavefront's keys sorted; its first K are the candidates.  With
    // one wavefront of experts, wavefront 0 sorts its own keys: no exchange.
    uint64_t key0 = 0;
    if (wv < ewv) {                                          // uniform
        const uint64_t key = tid < E ? sel_key(kept ? selv : NEG_INF, tid) : 0;
        if (ewv > 1) {
            const uint64_t srt = wave_sort_desc(key, lane);
            if (lane < K) s_cand[wv * K + lane] = srt;
        } else {
            key0 = key;
        }
    }
    if (ewv > 1) __syncthreads();                            // uniform
    WT_L(4);
    if (wv == 0) {
        const uint64_t cv = ewv > 1 ? (lane < ewv * K ? s_cand[lane] : 0) : key0;
        const uint64_t srt = wave_sort_desc(cv, lane);
        WT_L(5);
        // lane p < K: the p-th selection; its weight the unbiased score.
        // The renormalising sum runs in selection order, the engine's, as a
        // chain over the lanes' values (no LDS round trip per term).
        const int e = srt ? (int)~(uint32_t)srt : -1;       // the key's low word is ~id
        const float wr = lane < K && e >= 0 ? s_sc[e] : 0.0f;
        const bool ok = __builtin_amdgcn_readlane(e, K - 1) >= 0;   // K candidates
        float wsum = 0.0f;
        for (int p = 0; p < K; p++) wsum = __fadd_rn(wsum, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wr), p)));
        float myw = wr;
        if (ok) {
            if (c.renorm && K > 1) myw = __fdiv_rn(myw, __fadd_rn(wsum, 1e-20f));
            myw = __fmul_rn(myw, c.routed_scale);
        } else {
            myw = 0.0f;
            if (lane == 0) atomicOr(err, 2);
        }
        if (lane < K) {
            s_ids[lane] = ok ? e : -1;
            s_rec[lane] = ok && e >= 0 ? s_tab[e] : nullptr;
            s_w[lane] = myw;
        }
    }
    __syncthreads();
}
