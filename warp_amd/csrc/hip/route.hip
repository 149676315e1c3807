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

__global__ void __launch_bounds__(64)
k_route(whip_route_cfg c, const float *__restrict__ logits, const float *__restrict__ bias,
        int T, int32_t *__restrict__ ids, float *__restrict__ wout, int32_t *__restrict__ pair_tok,
        int32_t *__restrict__ pair_exp, float *__restrict__ pair_w, int32_t *__restrict__ tok_pairs,
        int *__restrict__ err)
{
    __shared__ float sc[MAXE], sel[MAXE], gsc[64];
    __shared__ float red;
    __shared__ int keep[64];
    __shared__ int sid[64];
    __shared__ float sw[64];
    const int t = blockIdx.x, lane = threadIdx.x, E = c.E, K = c.K;
    const float *lg = logits + (size_t)t * E;

    if (c.score_func == 1) {
        float mx = -1e30f;
        for (int e = lane; e < E; e += 64) if (lg[e] > mx) mx = lg[e];
        for (int o = 32; o > 0; o >>= 1) {
            const float m2 = __shfl_xor(mx, o, 64);
            if (m2 > mx) mx = m2;
        }
        for (int e = lane; e < E; e += 64) sc[e] = wh_expf(__fsub_rn(lg[e], mx));
        __syncthreads();
        if (lane == 0) {
            float sum = 0.0f;
            for (int e = 0; e < E; e++) sum = __fadd_rn(sum, sc[e]);
            red = sum;
        }
        __syncthreads();
        const float sum = red;
        for (int e = lane; e < E; e += 64) sc[e] = __fdiv_rn(sc[e], sum);
    } else if (c.score_func == 2) {
        for (int e = lane; e < E; e += 64) {
            const float x = lg[e];
            const float sp = x > 30.0f ? x : log1pf(wh_expf(x));
            sc[e] = __fsqrt_rn(sp);
        }
    } else {
        for (int e = lane; e < E; e += 64) sc[e] = __fdiv_rn(1.0f, __fadd_rn(1.0f, wh_expf(-lg[e])));
    }
    for (int e = lane; e < E; e += 64) sel[e] = __fadd_rn(sc[e], bias ? bias[e] : 0.0f);
    __syncthreads();

    if (c.n_group > 1) {
        const int G = c.n_group, gs = E / G;
        if (lane < G) {
            const float *p = sel + lane * gs;
            int a = -1, b = -1;
            float av = -__int_as_float(0x7f800000), bv2 = av;
            for (int i = 0; i < gs; i++) if (p[i] > av) { av = p[i]; a = i; }
            for (int i = 0; i < gs; i++) if (i != a && p[i] > bv2) { bv2 = p[i]; b = i; }
            const float ninf = -__int_as_float(0x7f800000);
            gsc[lane] = __fadd_rn(a >= 0 ? p[a] : ninf, b >= 0 ? p[b] : (gs > 1 ? ninf : 0.0f));
            keep[lane] = 0;
        }
        __syncthreads();
        if (lane == 0) {
            unsigned long long taken = 0;
            for (int j = 0; j < c.topk_group; j++) {
                int best = -1;
                float bv = -__int_as_float(0x7f800000);
                for (int g = 0; g < G; g++)
                    if (!((taken >> g) & 1) && gsc[g] > bv) { bv = gsc[g]; best = g; }
                if (best < 0) break;
                taken |= 1ull << best;
                keep[best] = 1;
            }
        }
        __syncthreads();
        for (int e = lane; e < E; e += 64) if (!keep[e / gs]) sel[e] = -__int_as_float(0x7f800000);
        __syncthreads();
    }

    uint32_t taken = 0;                 // bit i: expert lane + 64 i taken
    int bad = 0;
    for (int j = 0; j < K; j++) {
        float bv = -1e30f;
        int be = -1;
        for (int i = 0, e = lane; e < E; i++, e += 64)
            if (!((taken >> i) & 1) && sel[e] > bv) { bv = sel[e]; be = e; }
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int oe = __shfl_xor(be, o, 64);
            if (better(ov, oe, bv, be)) { bv = ov; be = oe; }
        }
        if (be < 0) {
            bad = 1;
            if (lane == 0) { sid[j] = -1; sw[j] = 0.0f; }
            continue;
        }
        if ((be & 63) == lane) taken |= 1u << (be >> 6);
        if (lane == 0) { sid[j] = be; sw[j] = sc[be]; }
    }
    if (lane != 0) return;
    int *myid = sid;
    float *myw = sw;
    if (!bad) {
        if (c.renorm && K > 1) {
            float s = 0.0f;
            for (int j = 0; j < K; j++) s = __fadd_rn(s, myw[j]);
            const float d = __fadd_rn(s, 1e-20f);
            for (int j = 0; j < K; j++) myw[j] = __fdiv_rn(myw[j], d);
        }
        for (int j = 0; j < K; j++) myw[j] = __fmul_rn(myw[j], c.routed_scale);
    } else {
        atomicOr(err, 2);
    }
    for (int j = 0; j < K; j++) {
        ids[(size_t)t * K + j] = myid[j];
        wout[(size_t)t * K + j] = myw[j];
    }
    if (pair_exp && T == 1) {
        for (int j = 0; j < K; j++) {
            pair_tok[j] = 0;
            pair_exp[j] = myid[j] < 0 ? E : myid[j];     // E: the table's NULL sentinel
            pair_w[j] = myw[j];
            tok_pairs[j] = j;
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
    hipLaunchKernelGGL(k_route, dim3(T), dim3(64), 0, s, *c, logits, bias, T, ids, w, pair_tok,
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
