// SPDX-License-Identifier: Apache-2.0
//
// vq_tile.h — the positions-across-lanes VQ3R tile: index loads, the
// conflict-free table lookups and the transpose-reduce, and the table build
// on the matrix cores.  Shared by the apply kernels and the one-launch decode.
#pragma once
#include "common.h"
#include "bf16_split.h"

// ---- positions across lanes ------------------------------------------------
// The same products with the lanes laid across positions instead of rows.
// In the kernel above every lane of a wavefront reads the same position's
// table at its own random code, so the 64 reads of one LDS instruction land
// on random banks and the instruction replays about five times.  Here lane
// (v, h) owns position v of a 32-position chunk and row half h of a 64-row
// block: it reads only position v's tables, and the tables are laid out
// [code][64 slots] with stage 0 in slots 0-31, stage 1 in slots 32-63
// (table A) and stage 2 twice (table B), so a lookup's bank is its slot.
// Row half 1 swaps each row's stage-0 and stage-1 index bytes once per tile;
// in every lookup the two halves then read different slot halves and all
// 64 lanes hit 64 different banks.  A lookup's address is one byte permute:
// the code into byte 1 of a per-lane base that holds the slot (byte 0) and
// the table (byte 2).
//
// Each lane ends a tile with its position's contribution to its 32 rows; a
// transpose-reduce across the 32 lanes of its half (a lane swap at offset
// 16, then offsets 8, mirror-4, 1, 2, each halving the registers kept)
// leaves every lane one row's sum over the chunk.  A workgroup owns a run
// of tiles (64 rows x 32 positions) in table order and rebuilds the tables
// when the run crosses from one (kind, chunk[, pair]) to the next.
#define PW 32
#define LT 1024
#define LW (LT / 64)
#define LUT_B 16384                 // floats: table B after table A

typedef const uint4 WH_GLOBAL g_uint4;
typedef float acc16 __attribute__((ext_vector_type(16)));

struct tile_buf { uint4 q[6]; };

__device__ __forceinline__ void load_tile(tile_buf &b, g_u8 *base, uint32_t loff)
{
#pragma unroll
    for (int i = 0; i < 6; i++) b.q[i] = *(g_uint4 *)(base + loff + 16 * i);
}

// one tile: 32 rows of this lane's half at its position, then the reduce.
// The buffer is consumed in place (row half 1's byte swap overwrites it).
//
// The three table reads of rows j and 16 + j (o[st] and o[3 + st]).
__device__ __forceinline__ void lookup6(const char *L, const uint32_t *d, int j, uint32_t bA0, uint32_t bA1,
                                        uint32_t bB, float *o)
{
#pragma unroll
    for (int st = 0; st < 3; st++) {
        const uint32_t base = st == 0 ? bA0 : st == 1 ? bA1 : bB;
        const int b0 = 3 * j + st, b1 = 3 * (16 + j) + st;
        o[st] = *(const float *)(L + __builtin_amdgcn_perm(d[b0 >> 2], base, 0x03020000u | ((4u + (b0 & 3)) << 8)));
        o[3 + st] =
            *(const float *)(L + __builtin_amdgcn_perm(d[b1 >> 2], base, 0x03020000u | ((4u + (b1 & 3)) << 8)));
    }
}

__device__ __forceinline__ float tile_sum(tile_buf &b, const float *smem, uint32_t bA0, uint32_t bA1,
                                          uint32_t bB, uint32_t s0, uint32_t s1, uint32_t s2, int lane)
{
    uint32_t d[24];
#pragma unroll
    for (int i = 0; i < 6; i++) { d[4 * i] = b.q[i].x; d[4 * i + 1] = b.q[i].y; d[4 * i + 2] = b.q[i].z; d[4 * i + 3] = b.q[i].w; }
    // half 1: stage-0 and stage-1 bytes of every row swap places
#pragma unroll
    for (int g = 0; g < 8; g++) {
        const uint32_t x0 = d[3 * g], x1 = d[3 * g + 1], x2 = d[3 * g + 2];
        d[3 * g] = __builtin_amdgcn_perm(x1, x0, s0);
        d[3 * g + 1] = __builtin_amdgcn_perm(x1, x0, s1);
        d[3 * g + 2] = __builtin_amdgcn_perm(x2, x2, s2);
    }
    const char *L = (const char *)smem;
    // rows j and 16 + j, folded at once by the first reduce step (a lane
    // swap at offset 16): e[j] is row j on lanes 0-15, row 16 + j on 16-31.
    // Software-pipelined: the reads of step j + 1 go out before step j's
    // are summed, so twelve reads are in flight at each wait instead of
    // the compiler's own eight-read bursts, each summed as soon as it is
    // sent (the scheduling barriers keep the order).
    float e[16];
    float t[2][6];
    lookup6(L, d, 0, bA0, bA1, bB, t[0]);
#pragma unroll
    for (int j = 0; j < 16; j++) {
        if (j + 1 < 16) lookup6(L, d, j + 1, bA0, bA1, bB, t[(j + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
        const float *c = t[j & 1];
        const float lo = (c[0] + c[1]) + c[2], hi = (c[3] + c[4]) + c[5];
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
        e[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
        __builtin_amdgcn_sched_barrier(0);
    }
    const bool b3 = (lane >> 3) & 1, b2 = (lane >> 2) & 1, b0 = lane & 1, b1 = (lane >> 1) & 1;
    float f[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const float keep = b3 ? e[8 + j] : e[j], send = b3 ? e[j] : e[8 + j];
        f[j] = keep + __uint_as_float(dpp32<0x128>(__float_as_uint(send)));
    }
    float g4[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float keep = b2 ? f[4 + j] : f[j], send = b2 ? f[j] : f[4 + j];
        g4[j] = keep + __uint_as_float(dpp32<0x141>(__float_as_uint(send)));
    }
    float g2[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const float keep = b0 ? g4[2 + j] : g4[j], send = b0 ? g4[j] : g4[2 + j];
        g2[j] = keep + __uint_as_float(dpp32<0xB1>(__float_as_uint(send)));
    }
    const float keep = b1 ? g2[1] : g2[0], send = b1 ? g2[0] : g2[1];
    return keep + __uint_as_float(dpp32<0x4E>(__float_as_uint(send)));
}

// A chunk's tables from one kind's three books (sbook: [stage][dim][code]
// fp32 in LDS, visible to the workgroup) and x at this lane's position
// (x0, and x1, x2 when three: its 8 values as bf16 pieces), on the bf16
// matrix cores.  A book value is an fp16 (11 significant bits), so
// hi = its top 8 bits and lo = the rest (at most 3 bits) are exact bf16
// values with hi + lo == value; x is one exact bf16 piece (bf16
// activations) or three (fp32, bf16_split.h).  One
// v_mfma_f32_32x32x16_bf16 takes K = 16 as (hi of dims 0-7 | lo of dims
// 0-7) against (the x piece's dims 0-7, twice): every product is exact in
// fp32 and only the fp32 sums round, as in an fp32 dot product.
//
// A product is 32 rows x 32 positions.  Its rows are chosen so that the two
// half-waves of the output write the two slot halves of the same codes:
// table A products take row m = (stage (m/4)%2, code c0 + 4(m/8) + m%4), so
// output register r of lane (v, h) is stage h of code c0 + r at position v,
// slot 32h + v; table B products take stage 2 in both halves (its two
// copies).  Every LDS write of a wavefront then covers 64 consecutive
// words, one per bank.  16 products of 16 codes for each table.  The caller
// synchronises after.
__device__ __forceinline__ void table_mfma(float *smem, const float *sbook, uint4 x0, uint4 x1, uint4 x2, bool three,
                                           int wv, int lane)
{
    const int m = lane & 31, h = lane >> 5;
    for (int tile = wv; tile < 32; tile += LW) {     // uniform per wavefront
        const bool tb = tile >= 16;
        const int c0 = (tile & 15) * 16;
        const int st = tb ? 2 : (m >> 2) & 1, code = c0 + (m >> 3) * 4 + (m & 3);
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t q[2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const float f = sbook[(st * 8 + 2 * i + j) * 256 + code];
                const uint32_t hi = __float_as_uint(f) & 0xffff0000u;
                q[j] = h ? __float_as_uint(__fsub_rn(f, __uint_as_float(hi))) >> 16 : hi >> 16;
            }
            w[i] = q[0] | (q[1] << 16);
        }
        const bf16x8 A = as_b8(make_uint4(w[0], w[1], w[2], w[3]));
        acc16 acc;
#pragma unroll
        for (int r = 0; r < 16; r++) acc[r] = 0.0f;
        if (three) {                                 // uniform; the smallest pieces first
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, as_b8(x2), acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, as_b8(x1), acc, 0, 0, 0);
        }
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, as_b8(x0), acc, 0, 0, 0);
        float *row = smem + (tb ? LUT_B : 0) + c0 * 64 + 32 * h + m;
#pragma unroll
        for (int r = 0; r < 16; r++) row[r * 64] = acc[r];
    }
}

// A workgroup's tiles in table order: t -> (pair, kind, chunk, row block).
// span: classes (kind, chunk), each over every pair's row blocks; else
// classes (pair, kind, chunk), each over one pair's row blocks.
struct tile_map {
    int span, nch, kinds, nb, tpc;
    __device__ __forceinline__ void at(int t, int &p, int &kind, int &chunk, int &rb) const
    {
        const int cls = t / tpc, within = t - cls * tpc;
        if (span) { kind = cls / nch; chunk = cls - kind * nch; p = within / nb; rb = within - p * nb; }
        else { p = cls / (kinds * nch); const int r = cls - p * kinds * nch; kind = r / nch; chunk = r - kind * nch; rb = within; }
    }
};

// A wavefront's position in the tile order, advanced without division: the
// tile index t and its (pair, kind, chunk, row block).  A division by a value
// known only at run time is tens of scalar instructions, and the sixteen
// wavefronts of a workgroup share one scalar unit; a cursor starts from one
// decode, done by a lane of the first wavefront in the prologue, and then
// only adds and compares.
struct tile_cur {
    int t, p, kind, chunk, rb;
    __device__ __forceinline__ void step(const tile_map &tm, int P, int n)
    {
        t += n;
        rb += n;
        while (rb >= tm.nb) {                        // uniform
            rb -= tm.nb;
            if (tm.span) {
                if (++p == P) { p = 0; if (++chunk == tm.nch) { chunk = 0; ++kind; } }
            } else if (++chunk == tm.nch) {
                chunk = 0;
                if (++kind == tm.kinds) { kind = 0; ++p; }
            }
        }
    }
};
