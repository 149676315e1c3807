// SPDX-License-Identifier: Apache-2.0
//
// route.hip — the router's scores and top-k, one wavefront per token.
//
// Bit-exact with the engine's CPU path on identical logits
// (src/model.c:5466-5553):
//   scores    sigmoid 1/(1+expf(-l)); softmax expf(l-max)/sum with the sum
//             taken sequentially in expert order; sqrt-softplus (its log1pf
//             is the device's, not restated);
//   select    K passes, each the first expert (ascending id) whose value
//             score+bias is strictly greater than every earlier one and
//             than -1e30, skipping taken ids.  A pass is one wave
//             reduction under the total order (value desc, id asc) over
//             the candidates value > -1e30, which picks the same expert;
//   weights   the unbiased score, renormalised by (sum + 1e-20) with the
//             sum in selection order, then times routed_scale.
// Group-limited selection (DeepSeek-V3 noaux_tc; no counterpart in the
// engine): a group's score is the sum of its two largest values, the
// topk_group best groups are kept by the same ordered passes, and the
// other groups' experts are masked to -inf.
#include "common.h"
#include "launch.h"

#define MAXE 1024

__device__ __forceinline__ bool better(float ov, int oe, float bv, int be)
{
    return oe >= 0 && (be < 0 || ov > bv || (ov == bv && oe < be));
}

#define NEG_INF (-__int_as_float(0x7f800000))

// top-2 of a multiset of values (NaN never counts, as in a strict-greater scan)
__device__ __forceinline__ void top2_merge(float &a1, float &a2, float b1, float b2)
{
    const float hi = b1 > a1 ? b1 : a1;
    const float lo = b1 > a1 ? a1 : b1;
    const float r2 = b2 > a2 ? b2 : a2;
    a1 = hi;
    a2 = r2 > lo ? r2 : lo;
}

// NPL experts per lane (E <= 64 * NPL), a template so that the unrolled
// per-lane loops hold only what the layer's E needs: the kernel runs once
// per token on a cold instruction cache.
template <int NPL>
__global__ void __launch_bounds__(64)
k_route(whip_route_cfg c, const float *__restrict__ logits, const float *__restrict__ bias,
        int T, int32_t *__restrict__ ids, float *__restrict__ wout, int32_t *__restrict__ pair_tok,
        int32_t *__restrict__ pair_exp, float *__restrict__ pair_w, int32_t *__restrict__ tok_pairs,
        int *__restrict__ err)
{
    __shared__ float lds[MAXE];
    __shared__ float gsc[64];
    const int t = blockIdx.x, lane = threadIdx.x, E = c.E, K = c.K;
    const int npl = (E + 63) >> 6;
    const float *lg = logits + (size_t)t * E;
    float sc[NPL], sel[NPL];

#pragma unroll
    for (int i = 0; i < NPL; i++) {
        const int e = lane + 64 * i;
        sc[i] = (i < npl && e < E) ? lg[e] : 0.0f;
    }
    if (c.score_func == 1) {
        float mx = -1e30f;
#pragma unroll
        for (int i = 0; i < NPL; i++)
            if (i < npl && lane + 64 * i < E && sc[i] > mx) mx = sc[i];
        for (int o = 32; o > 0; o >>= 1) {
            const float m2 = __shfl_xor(mx, o, 64);
            if (m2 > mx) mx = m2;
        }
#pragma unroll
        for (int i = 0; i < NPL; i++)
            if (i < npl && lane + 64 * i < E) {
                sc[i] = wh_expf(__fsub_rn(sc[i], mx));
                lds[lane + 64 * i] = sc[i];
            }
        __syncthreads();
        if (lane == 0) {                 // the engine's sum, in expert order
            float sum = 0.0f;
            for (int e = 0; e < E; e++) sum = __fadd_rn(sum, lds[e]);
            gsc[0] = sum;
        }
        __syncthreads();
        const float sum = gsc[0];
#pragma unroll
        for (int i = 0; i < NPL; i++) sc[i] = __fdiv_rn(sc[i], sum);
    } else if (c.score_func == 2) {
#pragma unroll
        for (int i = 0; i < NPL; i++) {
            const float x = sc[i];
            const float sp = x > 30.0f ? x : log1pf(wh_expf(x));
            sc[i] = __fsqrt_rn(sp);
        }
    } else {
#pragma unroll
        for (int i = 0; i < NPL; i++) sc[i] = __fdiv_rn(1.0f, __fadd_rn(1.0f, wh_expf(-sc[i])));
    }
#pragma unroll
    for (int i = 0; i < NPL; i++) {
        const int e = lane + 64 * i;
        sel[i] = (i < npl && e < E) ? __fadd_rn(sc[i], bias ? bias[e] : 0.0f) : NEG_INF;
    }

    if (c.n_group > 1) {
        const int G = c.n_group, gs = E / G;
        if (gs <= 64 && (64 % gs) == 0) {
            // groups tile the wave: a segmented top-2 merge over gs lanes
#pragma unroll
            for (int i = 0; i < NPL; i++) {
                if (i >= npl) break;
                float a1 = sel[i] == sel[i] ? sel[i] : NEG_INF, a2 = NEG_INF;
                for (int o = 1; o < gs; o <<= 1) {
                    const float b1 = __shfl_xor(a1, o, 64), b2 = __shfl_xor(a2, o, 64);
                    top2_merge(a1, a2, b1, b2);
                }
                const int e = lane + 64 * i;
                if (e % gs == 0 && e < E) gsc[e / gs] = __fadd_rn(a1, gs > 1 ? a2 : 0.0f);
            }
        } else {
            // wide groups: scan each group from LDS
#pragma unroll
            for (int i = 0; i < NPL; i++)
                if (i < npl && lane + 64 * i < E) lds[lane + 64 * i] = sel[i];
            __syncthreads();
            if (lane < G) {
                float a1 = NEG_INF, a2 = NEG_INF;
                for (int k = 0; k < gs; k++) {
                    const float v = lds[lane * gs + k];
                    if (v == v) top2_merge(a1, a2, v, NEG_INF);
                }
                gsc[lane] = __fadd_rn(a1, gs > 1 ? a2 : 0.0f);
            }
        }
        __syncthreads();
        // keep topk_group groups: strict-greater passes, lowest index first
        uint64_t keep = 0;
        for (int j = 0; j < c.topk_group; j++) {
            int best = -1;
            float bv = NEG_INF;
            for (int g = 0; g < G; g++)
                if (!((keep >> g) & 1) && gsc[g] > bv) { bv = gsc[g]; best = g; }
            if (best < 0) break;
            keep |= 1ull << best;
        }
#pragma unroll
        for (int i = 0; i < NPL; i++) {
            const int e = lane + 64 * i;
            if (i < npl && e < E && !((keep >> (e / gs)) & 1)) sel[i] = NEG_INF;
        }
    }

    // K selection passes; lane j keeps pass j's expert and weight
    uint32_t taken = 0;
    int my_id = -1;
    float my_w = 0.0f;
    int bad = 0;
    for (int j = 0; j < K; j++) {
        float bv = -1e30f;
        int be = -1;
        float bs = 0.0f;
#pragma unroll
        for (int i = 0; i < NPL; i++)
            if (i < npl && !((taken >> i) & 1) && sel[i] > bv) { bv = sel[i]; be = lane + 64 * i; bs = sc[i]; }
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int oe = __shfl_xor(be, o, 64);
            const float os = __shfl_xor(bs, o, 64);
            if (better(ov, oe, bv, be)) { bv = ov; be = oe; bs = os; }
        }
        if (be < 0) { bad = 1; continue; }
        if ((be & 63) == lane) taken |= 1u << (be >> 6);
        if (lane == j) { my_id = be; my_w = bs; }
    }
    if (!bad) {
        if (c.renorm && K > 1) {
            float s = 0.0f;                  // selection order
            for (int j = 0; j < K; j++) s = __fadd_rn(s, __shfl(my_w, j, 64));
            my_w = __fdiv_rn(my_w, __fadd_rn(s, 1e-20f));
        }
        my_w = __fmul_rn(my_w, c.routed_scale);
    } else {
        my_id = -1;
        my_w = 0.0f;
        if (lane == 0) atomicOr(err, 2);
    }
    if (lane < K) {
        ids[(size_t)t * K + lane] = my_id;
        wout[(size_t)t * K + lane] = my_w;
        if (pair_exp && T == 1) {
            pair_tok[lane] = 0;
            pair_exp[lane] = my_id < 0 ? E : my_id;    // E: the table's NULL sentinel
            pair_w[lane] = my_w;
            tok_pairs[lane] = lane;
        }
    }
}

extern "C" int whip_route(const whip_route_cfg *c, const float *logits, const float *bias, int T,
                          int32_t *ids, float *w, int32_t *pair_tok, int32_t *pair_exp,
                          float *pair_w, int32_t *tok_pairs, int *err, hipStream_t s)
{
    if (c->E > MAXE || c->E <= 0 || c->K <= 0 || c->K > 64 || c->K > c->E) return (int)hipErrorInvalidValue;
    if (c->n_group > 1 && (c->n_group > 64 || c->E % c->n_group || c->topk_group < 1))
        return (int)hipErrorInvalidValue;
#define ROUTE_LAUNCH(N)                                                                        \
    hipLaunchKernelGGL(k_route<N>, dim3(T), dim3(64), 0, s, *c, logits, bias, T, ids, w, pair_tok, \
                       pair_exp, pair_w, tok_pairs, err)
    const int npl = (c->E + 63) / 64;
    if (npl <= 1) ROUTE_LAUNCH(1);
    else if (npl <= 2) ROUTE_LAUNCH(2);
    else if (npl <= 4) ROUTE_LAUNCH(4);
    else if (npl <= 8) ROUTE_LAUNCH(8);
    else ROUTE_LAUNCH(16);
#undef ROUTE_LAUNCH
    return (int)hipGetLastError();
}

// Pairs of a chunk in (expert, token) order — the order moe_chunk reads
// experts in (src/model.c:7193-7197) — and each token's pairs in ascending
// expert order, its combine order (src/model.c:7230-7250).  Keys carry the
// selection slot as the last tie-break so every position is written once.
__global__ void __launch_bounds__(256)
k_pairs(const int32_t *__restrict__ ids, const float *__restrict__ w, int T, int K, int E,
        int32_t *__restrict__ pair_tok, int32_t *__restrict__ pair_exp, float *__restrict__ pair_w,
        int32_t *__restrict__ tok_pairs)
{
    const int P = T * K;
    for (int q = threadIdx.x; q < P; q += blockDim.x) {
        const int t = q / K, j = q % K;
        const int e = ids[q] < 0 ? E : ids[q];
        int pos = 0;
        for (int q2 = 0; q2 < P; q2++) {
            const int e2 = ids[q2] < 0 ? E : ids[q2], t2 = q2 / K, j2 = q2 % K;
            pos += (e2 < e) || (e2 == e && (t2 < t || (t2 == t && j2 < j)));
        }
        int rk = 0;
        for (int j2 = 0; j2 < K; j2++) {
            const int e2 = ids[t * K + j2] < 0 ? E : ids[t * K + j2];
            rk += (e2 < e) || (e2 == e && j2 < j);
        }
        pair_tok[pos] = t;
        pair_exp[pos] = e;
        pair_w[pos] = w[q];
        tok_pairs[t * K + rk] = pos;
    }
}

extern "C" int whip_pairs(const int32_t *ids, const float *w, int T, int K, int E,
                            int32_t *pair_tok, int32_t *pair_exp, float *pair_w,
                            int32_t *tok_pairs, hipStream_t s)
{
    hipLaunchKernelGGL(k_pairs, dim3(1), dim3(256), 0, s, ids, w, T, K, E, pair_tok, pair_exp,
                       pair_w, tok_pairs);
    return (int)hipGetLastError();
}
