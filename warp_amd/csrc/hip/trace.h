// SPDX-License-Identifier: Apache-2.0
//
// trace.h — optional constant-clock timeline of the batch-1 decode kernels
// (WH_TRACE, off in the library build).  Each translation unit that
// includes it holds its own buffer, [kernel][workgroup % 256][slot] of
// 100 MHz wall-clock stamps, read and cleared by the reader it names with
// WT_READER.  WT(k, i): the first lane of every wavefront stamps slot i of
// its workgroup (later writers win).  WT_SPAN(k, end): one pair of slots
// per kernel, the start of workgroup 0 and the latest end over every
// workgroup since the last read.
#pragma once

#ifdef WH_TRACE
#define WT_SLOTS 24
#define WT_ROWS (4 * 256)
__device__ uint64_t wt_buf[WT_ROWS * WT_SLOTS];
#define WT(k, i)                                                                                       \
    do {                                                                                               \
        if ((threadIdx.x & 63) == 0) wt_buf[((k) * 256 + (blockIdx.x & 255)) * WT_SLOTS + (i)] = wall_clock64(); \
    } while (0)
#define WT_SPAN(k, end)                                                                                \
    do {                                                                                               \
        if (threadIdx.x == 0) {                                                                        \
            const unsigned long long t_ = wall_clock64();                                              \
            if (end) atomicMax((unsigned long long *)&wt_buf[(k) * 256 * WT_SLOTS + 23], t_);          \
            else if (blockIdx.x == 0) wt_buf[(k) * 256 * WT_SLOTS + 22] = t_;                          \
        }                                                                                              \
    } while (0)
// WT_KEEP(i) keeps a stamp in a register and WT_PUT(k, i) stores it at the
// end, so that no wait in between covers a trace store
#define WT_DECL uint64_t wt_keep_[8] = {0, 0, 0, 0, 0, 0, 0, 0}
#define WT_KEEP(i) (wt_keep_[(i)] = wall_clock64())
#define WT_PUT(k, i)                                                                                   \
    do {                                                                                               \
        if ((threadIdx.x & 63) == 0) wt_buf[((k) * 256 + (blockIdx.x & 255)) * WT_SLOTS + (i)] = wt_keep_[(i)]; \
    } while (0)
#define WT_PUTAT(k, row, i) (wt_buf[((k) * 256 + (row)) * WT_SLOTS + (i)] = wt_keep_[(i)])
// WT_L(i): thread 0 keeps a stamp in LDS (no memory counter touched);
// WT_LPUT(k, row) stores the kept stamps to row `row` of kernel k
__shared__ uint64_t wt_lds_[16];
#define WT_L(i) do { if (threadIdx.x == 0) wt_lds_[(i)] = wall_clock64(); } while (0)
#define WT_LPUT(k, row)                                                                                \
    do {                                                                                               \
        if (threadIdx.x == 0)                                                                          \
            for (int q_ = 0; q_ < 16; q_++) wt_buf[((k) * 256 + (row)) * WT_SLOTS + q_] = wt_lds_[q_]; \
    } while (0)
#define WT_READER(name)                                                                                \
    extern "C" int name(uint64_t *host)                                                                \
    {                                                                                                  \
        hipError_t e = hipMemcpyFromSymbol(host, HIP_SYMBOL(wt_buf), sizeof wt_buf, 0, hipMemcpyDeviceToHost); \
        if (e != hipSuccess) return (int)e;                                                            \
        static uint64_t zero[WT_ROWS * WT_SLOTS];                                                      \
        return (int)hipMemcpyToSymbol(HIP_SYMBOL(wt_buf), zero, sizeof zero, 0, hipMemcpyHostToDevice); \
    }
#else
#define WT(k, i) do { } while (0)
#define WT_SPAN(k, end) do { } while (0)
#define WT_DECL do { } while (0)
#define WT_KEEP(i) do { } while (0)
#define WT_PUT(k, i) do { } while (0)
#define WT_PUTAT(k, row, i) do { } while (0)
#define WT_L(i) do { } while (0)
#define WT_LPUT(k, row) do { } while (0)
#define WT_READER(name)
#endif
