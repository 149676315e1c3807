// SPDX-License-Identifier: Apache-2.0
//
// route.hip — the router's scores and top-k, one wavefront per token.
//
// Bit-exact with the engine's CPU path on identical logits
// (src/model.c:5466-5553):
//   scores    sigmoid 1/(1+expf(-l)); softmax expf(l-max)/sum with the sum
//             taken sequentially in expert order; sqrt-softplus with the
//             host libm's log1pf restated (log1pf.h);
//   select    K passes, each the first expert (ascending id) whose value
//             score+bias is strictly greater than every earlier one and
//             than -1e30, skipping taken ids.  A pass is one wave max of a
//             64-bit key ordered as (value desc, id asc) over the
//             candidates value > -1e30, which picks the same expert;
//   weights   the unbiased score, renormalised by (sum + 1e-20) with the
//             sum in selection order, then times routed_scale.
// Group-limited selection (DeepSeek-V3 noaux_tc; no counterpart in the
// engine): a group's score is the sum of its two largest values, the
// topk_group best groups are kept by the same ordered passes, and the
// other groups' experts are masked to -inf.
#include "route.h"

template <int NPL>
__global__ void __launch_bounds__(64)
k_route(whip_route_cfg c, const float *__restrict__ logits, const float *__restrict__ bias,
        int T, int32_t *__restrict__ ids, float *__restrict__ wout, int32_t *__restrict__ pair_tok,
        int32_t *__restrict__ pair_exp, float *__restrict__ pair_w, int32_t *__restrict__ tok_pairs,
        int *__restrict__ err)
{
    __shared__ float rl[ROUTE_LDS_FLOATS(NPL)];
    route_body<NPL>(c, logits, bias, T, blockIdx.x, threadIdx.x, ids, wout, pair_tok, pair_exp, pair_w,
                    tok_pairs, nullptr, nullptr, err, rl);
}

extern "C" int whip_route(const whip_route_cfg *c, const float *logits, const float *bias, int T,
                          int32_t *ids, float *w, int32_t *pair_tok, int32_t *pair_exp,
                          float *pair_w, int32_t *tok_pairs, int *err, hipStream_t s)
{
    if (c->E > MAXE || c->E <= 0 || c->K <= 0 || c->K > 64 || c->K > c->E) return (int)hipErrorInvalidValue;
    if (c->n_group > 1 && (c->n_group > 64 || c->E % c->n_group || c->topk_group < 1))
        return (int)hipErrorInvalidValue;
    if (T <= 0) return (int)hipSuccess;
    const int E = c->E;
#define ROUTE(N) hipLaunchKernelGGL(k_route<N>, dim3(T), dim3(64), 0, s, *c, logits, bias, T, ids, w, \
                                    pair_tok, pair_exp, pair_w, tok_pairs, err)
    if (E <= 64) ROUTE(1);
    else if (E <= 128) ROUTE(2);
    else if (E <= 256) ROUTE(4);
    else if (E <= 512) ROUTE(8);
    else ROUTE(16);
#undef ROUTE
    return (int)hipGetLastError();
}

// Pairs of a chunk in (expert, token) order — the order moe_chunk reads
// experts in (src/model.c:7193-7197) — and each token's pairs in ascending
// expert order, its combine order (src/model.c:7230-7250).  Keys carry the
// selection slot as the last tie-break so every position is written once.
// The pairs' experts are staged in LDS first (at most PAIRS_LDS of them;
// beyond that they are read from global memory): a pair's position is a
// count over all pairs, and one global round trip per comparison made this
// launch cost more than the routing at 64 and more pairs.  The count reads
// four experts per LDS access, several accesses in flight (a loop that
// waits on each read took 19 us at 256 pairs), and four threads share each
// pair's count; the staged list is padded to a multiple of four with a
// value no expert id reaches.
#define PAIRS_LDS 4096
#define PAIRS_THREADS 1024
__global__ void __launch_bounds__(PAIRS_THREADS)
k_pairs(const int32_t *__restrict__ ids, const float *__restrict__ w, int T, int K, int E,
        int32_t *__restrict__ pair_tok, int32_t *__restrict__ pair_exp, float *__restrict__ pair_w,
        int32_t *__restrict__ tok_pairs)
{
    __shared__ __attribute__((aligned(16))) int se[PAIRS_LDS + 4];
    const int P = T * K;
    const bool staged = P <= PAIRS_LDS;
    if (staged) {
        for (int q = threadIdx.x; q < P; q += blockDim.x) se[q] = ids[q] < 0 ? E : ids[q];
        if (threadIdx.x < 4) se[P + threadIdx.x] = 0x7fffffff;
        __syncthreads();
    }
    auto exp_of = [&](int q) { return staged ? se[q] : (ids[q] < 0 ? E : ids[q]); };
    // four threads per pair (part 0-3 of four adjacent lanes), each counting
    // every fourth group of four entries; the parts meet by two shuffles
    const int part = threadIdx.x & 3;
    for (int q0 = 0; q0 < P; q0 += PAIRS_THREADS / 4) {   // uniform
        const int q = q0 + (int)(threadIdx.x >> 2);
        const bool live = q < P;
        const int qc = live ? q : 0;
        const int e = exp_of(qc);
        // pairs before q: a lower expert, or the same expert at an earlier
        // (token, slot), i.e. an earlier flat index
        int pos = 0;
        if (staged) {
            const int4 *s4 = (const int4 *)se;
            const int n4 = (P + 3) >> 2;
#pragma unroll 4
            for (int i = part; i < n4; i += 4) {
                const int4 v = s4[i];
                const int b = 4 * i;
                pos += (v.x < e) | ((v.x == e) & (b < qc));
                pos += (v.y < e) | ((v.y == e) & (b + 1 < qc));
                pos += (v.z < e) | ((v.z == e) & (b + 2 < qc));
                pos += (v.w < e) | ((v.w == e) & (b + 3 < qc));
            }
        } else {
            for (int q2 = part; q2 < P; q2 += 4) {
                const int e2 = exp_of(q2);
                pos += (e2 < e) || (e2 == e && q2 < qc);
            }
        }
        pos += __shfl_xor(pos, 1, 4);
        pos += __shfl_xor(pos, 2, 4);
        if (live && part == 0) {
            const int t = q / K, j = q % K;
            int rk = 0;
            for (int j2 = 0; j2 < K; j2++) {
                const int e2 = exp_of(t * K + j2);
                rk += (e2 < e) || (e2 == e && j2 < j);
            }
            pair_tok[pos] = t;
            pair_exp[pos] = e;
            pair_w[pos] = w[q];
            tok_pairs[t * K + rk] = pos;
        }
    }
}

extern "C" int whip_pairs(const int32_t *ids, const float *w, int T, int K, int E,
                            int32_t *pair_tok, int32_t *pair_exp, float *pair_w,
                            int32_t *tok_pairs, hipStream_t s)
{
    hipLaunchKernelGGL(k_pairs, dim3(1), dim3(PAIRS_THREADS), 0, s, ids, w, T, K, E, pair_tok, pair_exp,
                       pair_w, tok_pairs);
    return (int)hipGetLastError();
}
