// SPDX-License-Identifier: Apache-2.0
//
// vq_tile.h — the positions-across-lanes VQ3R tile: index loads, the
// conflict-free table lookups and the transpose-reduce, and the table build
// on the matrix cores.  Shared by the apply kernels and the one-launch decode.
#pragma once
#include "common.h"

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
__device__ __forceinline__ float lookup3(const char *L, const uint32_t *d, int j, uint32_t bA0,
                                         uint32_t bA1, uint32_t bB)
{
    float t[3];
#pragma unroll
    for (int st = 0; st < 3; st++) {
        const int byte = 3 * j + st;
        const uint32_t base = st == 0 ? bA0 : st == 1 ? bA1 : bB;
        const uint32_t a = __builtin_amdgcn_perm(d[byte >> 2], base, 0x03020000u | ((4u + (byte & 3)) << 8));
        t[st] = *(const float *)(L + a);
    }
    return (t[0] + t[1]) + t[2];
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
    // swap at offset 16): e[j] is row j on lanes 0-15, row 16 + j on 16-31
    float e[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const float lo = lookup3(L, d, j, bA0, bA1, bB), hi = lookup3(L, d, 16 + j, bA0, bA1, bB);
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
        e[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
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

// A chunk's tables from one kind's three books (sbook: [stage][dim][code] in
// LDS, visible to the workgroup) and x at this lane's position v (xv[8]):
// 24 products of 32 codes x 32 positions on the matrix cores
// (books[code][dim] x x[dim][position]), fp32 throughout.  Table A holds
// stage 0 in slots 0-31 and stage 1 in slots 32-63, table B stage 2 twice;
// a lane's slot is its position.  The caller synchronises after.
__device__ __forceinline__ void table_mfma(float *smem, const float *sbook, const float *xv, int wv, int v, int h)
{
    float xb[4];                                     // B operand: x[position v][dim 2i + h]
#pragma unroll
    for (int i = 0; i < 4; i++) xb[i] = h ? xv[2 * i + 1] : xv[2 * i];
    for (int tile = wv; tile < 24; tile += LW) {     // uniform per wavefront
        const int st = tile >> 3, c0 = (tile & 7) * 32;
        acc16 acc;
#pragma unroll
        for (int r = 0; r < 16; r++) acc[r] = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float av = sbook[(st * 8 + 2 * i + h) * 256 + c0 + v];
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av, xb[i], acc, 0, 0, 0);
        }
        // acc[r]: code c0 + 8(r/4) + 4h + r%4, position v
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int c = c0 + (r >> 2) * 8 + 4 * h + (r & 3);
            if (st < 2) smem[c * 64 + 32 * st + v] = acc[r];
            else { smem[LUT_B + c * 64 + v] = acc[r]; smem[LUT_B + c * 64 + 32 + v] = acc[r]; }
        }
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
