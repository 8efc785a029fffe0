// phase_trace.h -- workgroup-0 phase timestamps for latency studies.
// Compiled only into a -DMANTLE_PHASE_TRACE build, never into the product.
// Every translation unit has its own buffer (100 MHz wall clock stamps, 8 per
// launch); MANTLE_PHASE_READER defines the host function that copies it out.
#pragma once

#include <hip/hip_runtime.h>

#ifdef MANTLE_PHASE_TRACE
namespace mantle {
static __device__ unsigned long long g_phase[8192 * 8];
static __device__ unsigned int g_phase_n;
}  // namespace mantle
#define PHASE_SLOT()                                                            \
    unsigned phase_slot_ = 0;                                                   \
    if (blockIdx.x == 0 && threadIdx.x == 0) phase_slot_ = atomicAdd(&::mantle::g_phase_n, 1u) & 8191u
#define PHASE(k)                                                                \
    do {                                                                        \
        if (blockIdx.x == 0 && threadIdx.x == 0)                                \
            ::mantle::g_phase[phase_slot_ * 8 + (k)] = wall_clock64();          \
    } while (0)
// Stamp once `val` has arrived (the empty asm makes the wave wait for it).
#define PHASE_AFTER(k, val)                                                     \
    do {                                                                        \
        asm volatile("" ::"v"(val));                                            \
        PHASE(k);                                                               \
    } while (0)
#define MANTLE_PHASE_READER(fn)                                                                          \
    int fn(unsigned long long* out, int max_slots, unsigned* n) {                                        \
        hipError_t e = hipMemcpyFromSymbol(n, HIP_SYMBOL(::mantle::g_phase_n), sizeof(unsigned));         \
        if (e != hipSuccess) return e;                                                                   \
        const int k = (int)(*n < (unsigned)max_slots ? *n : (unsigned)max_slots);                        \
        if (k == 0) return 0;                                                                            \
        return hipMemcpyFromSymbol(out, HIP_SYMBOL(::mantle::g_phase), sizeof(unsigned long long) * 8 * k); \
    }
#else
#define PHASE_SLOT() (void)0
#define PHASE(k) (void)0
#define PHASE_AFTER(k, val) (void)0
#endif
