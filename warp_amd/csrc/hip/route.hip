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

#define NEG_INF (-__int_as_float(0x7f800000))

// (a, ea) precedes (b, eb) in the engine's selection order: larger value
// first, the lower id among equal values (a strict-greater scan keeps the
// first maximum it meets).
__device__ __forceinline__ bool before(float a, int ea, float b, int eb)
{
    return a > b || (a == b && ea < eb);
}

// One workgroup per token, one thread per expert.  K strict-greater passes
// select, in order, the experts that come first under `before`; so expert e
// is selected in pass j exactly when j experts precede it, and this kernel
// computes that rank directly, every thread against the table in LDS
// (broadcast reads), instead of running K dependent reductions.
__global__ void __launch_bounds__(1024)
k_route(whip_route_cfg c, const float *__restrict__ logits, const float *__restrict__ bias,
        int T, int32_t *__restrict__ ids, float *__restrict__ wout, int32_t *__restrict__ pair_tok,
        int32_t *__restrict__ pair_exp, float *__restrict__ pair_w, int32_t *__restrict__ tok_pairs,
        int *__restrict__ err)
{
    __shared__ float s_sel[MAXE], s_tmp[MAXE];
    __shared__ float s_g1[64], s_g2[64], s_g[64];
    __shared__ int s_id[64], s_ncand;
    __shared__ float s_w[64], s_red;
    const int t = blockIdx.x, e = threadIdx.x, E = c.E, K = c.K;
    const bool valid = e < E;
    const float *lg = logits + (size_t)t * E;
    const float l = valid ? lg[e] : 0.0f;
    if (e == 0) s_ncand = 0;

    float sc;
    if (c.score_func == 1) {
        // max (order-free), then the engine's sequential sum
        s_tmp[e] = valid ? l : -1e30f;
        __syncthreads();
        if (e < 64) {
            float mx = -1e30f;
            for (int k = e; k < E; k += 64) if (s_tmp[k] > mx) mx = s_tmp[k];
            for (int o = 32; o > 0; o >>= 1) {
                const float m2 = __shfl_xor(mx, o, 64);
                if (m2 > mx) mx = m2;
            }
            if (e == 0) s_red = mx;
        }
        __syncthreads();
        const float ex = valid ? wh_expf(__fsub_rn(l, s_red)) : 0.0f;
        __syncthreads();
        s_tmp[e] = ex;
        __syncthreads();
        if (e == 0) {
            float sum = 0.0f;
            for (int k = 0; k < E; k++) sum = __fadd_rn(sum, s_tmp[k]);
            s_red = sum;
        }
        __syncthreads();
        sc = __fdiv_rn(ex, s_red);
    } else if (c.score_func == 2) {
        const float sp = l > 30.0f ? l : log1pf(wh_expf(l));
        sc = __fsqrt_rn(sp);
    } else {
        sc = __fdiv_rn(1.0f, __fadd_rn(1.0f, wh_expf(-l)));
    }
    float sel = valid ? __fadd_rn(sc, bias ? bias[e] : 0.0f) : NEG_INF;
    s_sel[e] = sel;
    __syncthreads();

    if (c.n_group > 1) {
        // group score: the sum of the group's two largest values (NaN never
        // counts); keep the topk_group groups that come first under
        // `before`, never one scored -inf; mask the rest to -inf
        const int G = c.n_group, gs = E / G, g = e / gs;
        const float gv = sel == sel ? sel : NEG_INF;
        if (valid) {
            int rk = 0;
            for (int k = g * gs; k < (g + 1) * gs; k++) {
                const float o = s_sel[k];
                rk += before(o == o ? o : NEG_INF, k, gv, e);
            }
            if (rk == 0) s_g1[g] = gv;
            if (rk == 1) s_g2[g] = gv;
        }
        __syncthreads();
        if (e < G) s_g[e] = __fadd_rn(s_g1[e], gs > 1 ? s_g2[e] : 0.0f);
        __syncthreads();
        if (valid) {
            const float mine = s_g[g];
            int grk = 0;
            for (int k = 0; k < G; k++) grk += before(s_g[k], k, mine, g);
            if (!(grk < c.topk_group && mine > NEG_INF)) sel = NEG_INF;
        }
        __syncthreads();
        s_sel[e] = sel;
        __syncthreads();
    }

    // candidates: strictly above the scan's floor -1e30 (never NaN)
    const bool cand = valid && sel > -1e30f;
    if (cand) {
        atomicAdd(&s_ncand, 1);
        int rk = 0;
        for (int k = 0; k < E; k++) {
            const float o = s_sel[k];
            rk += (o > -1e30f) && before(o, k, sel, e);
        }
        if (rk < K) { s_id[rk] = e; s_w[rk] = sc; }
    }
    __syncthreads();
    const int bad = s_ncand < K;
    if (e == 0) {
        if (!bad) {
            if (c.renorm && K > 1) {
                float s = 0.0f;              // selection order
                for (int j = 0; j < K; j++) s = __fadd_rn(s, s_w[j]);
                const float d = __fadd_rn(s, 1e-20f);
                for (int j = 0; j < K; j++) s_w[j] = __fdiv_rn(s_w[j], d);
            }
            for (int j = 0; j < K; j++) s_w[j] = __fmul_rn(s_w[j], c.routed_scale);
        } else {
            atomicOr(err, 2);
        }
    }
    __syncthreads();
    if (e < K) {
        const int id = bad ? -1 : s_id[e];
        const float wv = bad ? 0.0f : s_w[e];
        ids[(size_t)t * K + e] = id;
        wout[(size_t)t * K + e] = wv;
        if (pair_exp && T == 1) {
            pair_tok[e] = 0;
            pair_exp[e] = id < 0 ? E : id;       // E: the table's NULL sentinel
            pair_w[e] = wv;
            tok_pairs[e] = e;
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
    const int threads = (c->E + 63) / 64 * 64;
    hipLaunchKernelGGL(k_route, dim3(T), dim3(threads), 0, s, *c, logits, bias, T, ids, w, pair_tok,
                       pair_exp, pair_w, tok_pairs, err);
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
