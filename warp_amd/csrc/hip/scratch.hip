// SPDX-License-Identifier: Apache-2.0
//
// scratch.hip — the library's static device scratch area, for the one entry
// point that must not allocate (waste_hip_moe_forward_static).
//
// `scratch` is a file-scope device array: every GPU the library runs on holds
// its own copy, at its own address, until the process ends.  Host code never
// passes the array's name to a kernel or a copy (on the host that name is a
// stand-in, not a device address); it asks whip_scratch for the current
// device's address, which hipGetSymbolAddress gives once per device.
//
// The area keeps what the last call left in it.  Its first
// WHIP_SCRATCH_HEAD bytes hold state that must start at zero (the routing
// exchange's tag word and tagged logits, the routing launch's block
// counter).  A device variable without an initializer is zero-filled when
// the code object loads, and every launch leaves that state as valid for
// the next (the counter back at zero, the tags only growing), so no call
// clears it: a first call captured into a graph, or made on any stream,
// needs nothing done before it.
#include <hip/hip_runtime.h>
#include <mutex>

#include "launch.h"

static __device__ __align__(256) unsigned char scratch[WHIP_SCRATCH_BYTES];

#define SCRATCH_DEVS 64
static std::mutex g_mu;
static void *g_ptr[SCRATCH_DEVS];

extern "C" int whip_scratch(void **ptr)
{
    *ptr = nullptr;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= SCRATCH_DEVS) return (int)hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (!p || (uintptr_t)p % 256) return (int)hipErrorInvalidSymbol;
        g_ptr[dev] = p;
    }
    *ptr = g_ptr[dev];
    return 0;
}

__global__ void __launch_bounds__(256) k_zero_words(uint32_t *__restrict__ p, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) p[i] = 0u;
}

extern "C" int whip_zero(void *p, size_t bytes, hipStream_t s)
{
    if (bytes % 4 || (uintptr_t)p % 4) return (int)hipErrorInvalidValue;
    const size_t n = bytes / 4;
    if (!n) return 0;
    const unsigned blocks = (unsigned)((n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024);
    hipLaunchKernelGGL(k_zero_words, dim3(blocks), dim3(256), 0, s, (uint32_t *)p, n);
    return (int)hipGetLastError();
}
