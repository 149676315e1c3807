// SPDX-License-Identifier: Apache-2.0
//
// synth.hip — synthetic expert records generated and encoded on the device
// (include/waste_hip_synth.h).
//
// One wavefront per matrix row: lanes own the row's 8-wide vectors
// v = lane, lane + 64, ...; pass 1 generates the row's N(0, std) weights
// and takes max|w| across the wave (the row scale, stored as f16); pass 2
// regenerates them, divides by the scale and encodes each vector stage by
// stage against the kind's books (in LDS; every lane reads the same entry
// at once, a broadcast): nearest entry by squared L2 summed over the 8
// dims in order, first minimum wins, then the residual (src/vq.c:50-96).
#include <hip/hip_fp16.h>
#include "common.h"
#include "launch.h"
#include "waste_abi.h"

__device__ __forceinline__ uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

// Two N(0,1) values for column pair c2 of row r (Box-Muller on a hash).
__device__ __forceinline__ float2 gauss2(uint64_t key, int r, int c2)
{
    const uint64_t h = mix64(key ^ ((uint64_t)r * 0x9E3779B97F4A7C15ULL) ^
                             ((uint64_t)c2 * 0xD1B54A32D192ED03ULL));
    const float u1 = ((uint32_t)(h >> 40) + 0.5f) * (1.0f / 16777216.0f);
    const float u2 = ((uint32_t)(h & 0xffffff) + 0.5f) * (1.0f / 16777216.0f);
    const float rad = sqrtf(-2.0f * logf(u1));
    float s, c;
    sincosf(6.283185307f * u2, &s, &c);
    return make_float2(rad * c, rad * s);
}

__global__ void __launch_bounds__(256)
k_synth(uint64_t seed, int layer, int H, int I, int cb_base, const float *__restrict__ books,
        int e0, uint8_t *__restrict__ dst, size_t rec_bytes, float stdv, float *__restrict__ raw)
{
    __shared__ float cbk[3 * 256 * 8];
    const int kind = blockIdx.y, e = e0 + blockIdx.z;
    const int M = kind == 2 ? H : I, N = kind == 2 ? I : H, nv = N / 8;
    const int lane = threadIdx.x & 63;
    for (int i = threadIdx.x; i < 3 * 256 * 8; i += blockDim.x) cbk[i] = books[(size_t)kind * 3 * 256 * 8 + i];
    __syncthreads();
    uint8_t *rec = dst + (size_t)blockIdx.z * rec_bytes;
    const size_t gu = (size_t)I * (H / 8) * 3, dn = (size_t)H * (I / 8) * 3;
    const size_t off = kind == 0 ? 48 : kind == 1 ? 48 + gu : 48 + 2 * gu;
    const size_t sc_off = 48 + 2 * gu + dn;
    if (blockIdx.x == 0 && kind == 0 && threadIdx.x == 0) {
        waste_expert_hdr h;
        h.magic = WASTE_MAGIC_EXPERT; h.layer = (uint16_t)layer; h.expert_id = (uint16_t)e;
        h.fmt = WQ_VQ3R; h.flags = 0; h.codebook_id = (uint16_t)cb_base; h.lowrank_id = 0;
        h.reserved0 = 0; h.rec_4k_blocks = (uint32_t)(rec_bytes / 4096);
        h.gate_off = 48; h.up_off = (uint32_t)(48 + gu); h.down_off = (uint32_t)(48 + 2 * gu);
        h.chan_corr_off = (uint32_t)sc_off; h.crc32 = 0; h.reserved1[0] = h.reserved1[1] = 0;
        const uint32_t *src = (const uint32_t *)&h;
        for (int i = 0; i < 12; i++) ((uint32_t *)rec)[i] = src[i];
    }
    const uint64_t key = mix64(seed * 0x100000001B3ULL + (uint64_t)e * 3 + kind + 1);
    for (int r = blockIdx.x * 4 + (threadIdx.x >> 6); r < M; r += gridDim.x * 4) {

    float amax = 0.0f;
    for (int v = lane; v < nv; v += 64)
        for (int j = 0; j < 8; j += 2) {
            const float2 g = gauss2(key, r, (v * 8 + j) >> 1);
            amax = fmaxf(amax, fmaxf(fabsf(g.x * stdv), fabsf(g.y * stdv)));
        }
    for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    const float scale = fmaxf(amax, 1e-8f);
    if (lane == 0) {
        const __half hs = __float2half_rn(scale);
        ((uint16_t *)(rec + sc_off))[(kind == 0 ? 0 : kind == 1 ? I : 2 * I) + r] = __half_as_ushort(hs);
    }
    uint8_t *ix = rec + off + (size_t)(r >> 6) * nv * 192 + (r & 63) * 3;
    for (int v = lane; v < nv; v += 64) {
        float x[8];
        for (int j = 0; j < 8; j += 2) {
            const float2 g = gauss2(key, r, (v * 8 + j) >> 1);
            x[j] = __fdiv_rn(__fmul_rn(g.x, stdv), scale);
            x[j + 1] = __fdiv_rn(__fmul_rn(g.y, stdv), scale);
        }
        if (raw && kind == 0 && blockIdx.z == 0)
            for (int j = 0; j < 8; j++) raw[(size_t)r * N + v * 8 + j] = x[j];
        for (int s = 0; s < 3; s++) {
            const float *C = cbk + s * 256 * 8;
            int best = 0;
            float bestd = __int_as_float(0x7f800000);
            for (int c = 0; c < 256; c++) {
                float d = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float t = __fsub_rn(x[j], C[c * 8 + j]);
                    d = __fadd_rn(d, __fmul_rn(t, t));
                }
                if (d < bestd) { bestd = d; best = c; }
            }
            ix[(size_t)v * 192 + s] = (uint8_t)best;
#pragma unroll
            for (int j = 0; j < 8; j++) x[j] = __fsub_rn(x[j], C[best * 8 + j]);
        }
    }
    }
}

extern "C" int whip_synth_records(uint64_t seed, int layer, int H, int I, int cb_base,
                                  const float *books, int e0, int n, uint8_t *dst, size_t rec_bytes,
                                  float stdv, float *raw, hipStream_t s)
{
    if (hipMemsetAsync(dst, 0, (size_t)n * rec_bytes, s) != hipSuccess) return -1;
    const int maxm = H > I ? H : I;
    const int gx = (maxm + 3) / 4 < 64 ? (maxm + 3) / 4 : 64;
    hipLaunchKernelGGL(k_synth, dim3(gx, 3, n), dim3(256), 0, s, seed, layer, H, I,
                       cb_base, books, e0, dst, rec_bytes, stdv, raw);
    return (int)hipGetLastError();
}
