// SPDX-License-Identifier: Apache-2.0
//
// gemv.hip — trunk matrix-vector products for the MoE layer: the router
// logits and the shared expert (F32, Q8G int8 + f16 group scale, Q4G two
// signed nibbles per byte, low first, minus 8; tools/convert.py:893-924).
//
// One wavefront per output row; each lane streams 16-byte chunks of the
// row (coalesced 128-bit loads) and keeps a partial per token; a chunk
// never straddles a quantisation group, so its group scale multiplies the
// chunk's partial once.  Up to TB tokens share every weight load; larger
// batches take further passes over the (L2-resident) row.
#include "common.h"
#include "launch.h"

#define TB 4

template <int FMT>
__device__ __forceinline__ void decode_chunk(const uint8_t *row, int k, float *w);

template <> __device__ __forceinline__ void decode_chunk<0>(const uint8_t *row, int k, float *w)
{
    const float4 v = *(const float4 *)(row + (size_t)k * 16);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
}

template <> __device__ __forceinline__ void decode_chunk<2>(const uint8_t *row, int k, float *w)
{
    const uint4 v = *(const uint4 *)(row + (size_t)k * 16);
    const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 16; i++) w[i] = (float)(int8_t)((u[i >> 2] >> ((i & 3) * 8)) & 0xff);
}

template <> __device__ __forceinline__ void decode_chunk<3>(const uint8_t *row, int k, float *w)
{
    const uint4 v = *(const uint4 *)(row + (size_t)k * 16);
    const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const uint32_t b = (u[i >> 2] >> ((i & 3) * 8)) & 0xff;
        w[2 * i] = (float)((int)(b & 15) - 8);
        w[2 * i + 1] = (float)((int)(b >> 4) - 8);
    }
}

template <int FMT>
__global__ void __launch_bounds__(256)
k_gemv(const uint8_t *__restrict__ W0, const uint16_t *__restrict__ S0, size_t rb0,
       const uint8_t *__restrict__ W1, const uint16_t *__restrict__ S1, size_t rb1,
       int rows, int cols, int group, const float *__restrict__ x, int x_ld, int T,
       float *__restrict__ y0, float *__restrict__ y1, int y_ld)
{
    constexpr int NE = FMT == 0 ? 4 : FMT == 2 ? 16 : 32;   // elements per 16 B chunk
    const int which = blockIdx.y;
    const uint8_t *W = which ? W1 : W0;
    const uint16_t *S = which ? S1 : S0;
    const size_t rowbytes = which ? rb1 : rb0;
    float *y = which ? y1 : y0;
    const int r = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    const int ng = FMT == 0 ? 1 : (cols + group - 1) / group;
    const int padded = FMT == 0 ? cols : ng * group;
    const int nchunk = (padded + NE - 1) / NE;
    const uint8_t *row = W + (size_t)r * rowbytes;
    const uint16_t *sr = FMT == 0 ? nullptr : S + (size_t)r * ng;

    for (int t0 = 0; t0 < T; t0 += TB) {
        const int tn = min(TB, T - t0);
        float acc[TB] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int k = lane; k < nchunk; k += 64) {
            float w[NE];
            decode_chunk<FMT>(row, k, w);
            const int e0 = k * NE;
            const float sc = FMT == 0 ? 1.0f : wh_f16_scale(sr[e0 / group]);
#pragma unroll
            for (int t = 0; t < TB; t++) {
                if (t >= tn) break;
                const float *xt = x + (size_t)(t0 + t) * x_ld + e0;
                float part = 0.0f;
                if (e0 + NE <= cols) {
#pragma unroll
                    for (int i = 0; i < NE; i += 4) {
                        const float4 xv = *(const float4 *)(xt + i);
                        part = __fmaf_rn(w[i], xv.x, part);
                        part = __fmaf_rn(w[i + 1], xv.y, part);
                        part = __fmaf_rn(w[i + 2], xv.z, part);
                        part = __fmaf_rn(w[i + 3], xv.w, part);
                    }
                } else {
                    for (int i = 0; i < NE && e0 + i < cols; i++) part = __fmaf_rn(w[i], xt[i], part);
                }
                acc[t] = __fmaf_rn(sc, part, acc[t]);
            }
        }
#pragma unroll
        for (int t = 0; t < TB; t++) {
            if (t >= tn) break;
            const float v = wave_sum(acc[t]);
            if (lane == 0) y[(size_t)(t0 + t) * y_ld + r] = v;
        }
    }
}

extern "C" int whip_gemv(const whip_mat *A, const whip_mat *B, const float *x, int x_ld, int T,
                         float *y0, float *y1, int y_ld, hipStream_t s)
{
    if (B && (B->fmt != A->fmt || B->rows != A->rows || B->cols != A->cols || B->group != A->group))
        return (int)hipErrorInvalidValue;
    if (A->fmt == 0 && (A->cols % 4 || A->rowbytes % 16)) return (int)hipErrorInvalidValue;
    if (A->fmt != 0 && (A->group % 32 || A->rowbytes % 16)) return (int)hipErrorInvalidValue;
    if (x_ld % 4) return (int)hipErrorInvalidValue;
    dim3 grid((A->rows + 3) / 4, B ? 2 : 1);
    const uint8_t *w1 = B ? (const uint8_t *)B->q : nullptr;
    const uint16_t *s1 = B ? B->qs : nullptr;
    const size_t rb1 = B ? B->rowbytes : 0;
#define GEMV_LAUNCH(F)                                                                       \
    hipLaunchKernelGGL(k_gemv<F>, grid, dim3(256), 0, s, (const uint8_t *)A->q, A->qs,       \
                       A->rowbytes, w1, s1, rb1, A->rows, A->cols, A->group, x, x_ld, T, y0, \
                       y1, y_ld)
    switch (A->fmt) {
    case 0: GEMV_LAUNCH(0); break;
    case 2: GEMV_LAUNCH(2); break;
    case 3: GEMV_LAUNCH(3); break;
    default: return (int)hipErrorInvalidValue;
    }
#undef GEMV_LAUNCH
    return (int)hipGetLastError();
}

__global__ void k_bf16_to_f32(const uint16_t *__restrict__ x, float *__restrict__ y, size_t n)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = wh_bf16(x[i]);
}

extern "C" int whip_bf16_to_f32(const uint16_t *x, float *y, size_t n, hipStream_t s)
{
    hipLaunchKernelGGL(k_bf16_to_f32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, y, n);
    return (int)hipGetLastError();
}
