// SPDX-License-Identifier: Apache-2.0
//
// table.hip — the layer's record table, updated in stream order.
//
// An expert cache hands the layer device records between its router and its
// experts.  Writing the table from the host would need a copy the host waits
// on; here the new entries travel as kernel arguments and one wavefront
// writes them, so the update lands exactly where the stream reaches it.
// Each record's header is checked first, as record_check does
// (src/model.c:3645-3692, the checksum aside, which needs the payload on
// the host): a record that fails stays unbound and raises bit 8 of the
// layer's error word.
#include "common.h"
#include "launch.h"
#include "waste_abi.h"

__global__ void __launch_bounds__(64)
k_bind(const uint8_t **__restrict__ recs, whip_bind_args a, int *__restrict__ err)
{
    const int l = threadIdx.x;
    if (l >= a.n) return;
    const int e = a.expert[l];
    const uint8_t *r = a.rec[l];
    if (!r) {
        recs[e] = nullptr;
        return;
    }
    const uint4 *h4 = (const uint4 *)r;
    const uint4 q0 = h4[0], q1 = h4[1], q2 = h4[2];
    // bytes  0-15: magic | layer, expert | fmt, flags, codebook | lowrank, reserved
    // bytes 16-31: rec_4k_blocks | gate_off | up_off | down_off
    // bytes 32-47: chan_corr_off | crc32 | reserved
    const uint32_t magic = q0.x, layer = q0.y & 0xffffu, eid = q0.y >> 16;
    const uint32_t fmt = q0.z & 0xffu, cb = q0.z >> 16, lowrank = q0.w & 0xffffu;
    const bool ok = magic == WASTE_MAGIC_EXPERT && layer == a.layer && eid == (uint32_t)e &&
                    fmt == a.fmt && lowrank == 0 && q1.x == a.rec_4k_blocks && q1.y == 48u &&
                    q1.z == a.off_up && q1.w == a.off_down && q2.x == a.off_sc &&
                    (a.cb < 0 || cb == (uint32_t)a.cb) && (long)cb >= (long)a.book0 &&
                    (long)cb + (long)a.nbk <= (long)a.n_books;
    recs[e] = ok ? r : nullptr;
    if (!ok) atomicOr(err, 8);
}

extern "C" int whip_bind(const uint8_t **recs, const whip_bind_args *a, int *err, hipStream_t s)
{
    if (a->n <= 0) return (int)hipSuccess;
    if (a->n > WHIP_BIND_MAX) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_bind, dim3(1), dim3(64), 0, s, recs, *a, err);
    return (int)hipGetLastError();
}

// Clears bits of the layer's error word in stream order (after the
// kernels that may have raised them, before the ones that may raise them
// again), so a host that reads the word and retries needs no copy.
__global__ void __launch_bounds__(64) k_err_clear(int *__restrict__ err, int mask)
{
    if (threadIdx.x == 0) atomicAnd(err, ~mask);
}

extern "C" int whip_err_clear(int *err, int mask, hipStream_t s)
{
    hipLaunchKernelGGL(k_err_clear, dim3(1), dim3(64), 0, s, err, mask);
    return (int)hipGetLastError();
}
