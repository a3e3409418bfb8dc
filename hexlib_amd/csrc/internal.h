// Host-side internals shared by every translation unit of libhexlib_gpu.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hexlib_gpu.h"

namespace hx {

// The stream every per-kernel API call enqueues on.
hipStream_t stream();
// Records the first failing launch status until hexlib_gpu_take_error().
void note(hipError_t e);
// Per-thread flag: while set (a DRYRUN invoke), API functions validate their
// arguments and return without touching the GPU.
bool dry_run();
void set_dry_run(bool on);

// Allocates the largest split-K workspace recorded by dry runs (hipMalloc,
// outside any capture). 0 on success.
int prepare_workspace();

inline bool aligned(const void *p, uintptr_t a) {
    return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

inline unsigned blocks_for(long long work, int per_block, unsigned cap = 1u << 20) {
    long long b = (work + per_block - 1) / per_block;
    if (b < 1) b = 1;
    if (b > (long long) cap) b = cap;
    return (unsigned) b;
}

}  // namespace hx

// Records, during a dry run, the split-K workspace a launch would need.
void hx_reserve_workspace(size_t bytes);

// Every launch goes through here: skipped under a dry run, error recorded.
#define HX_LAUNCH(kernel, grid, block, lds, ...)                                  \
    do {                                                                        \
        if (hx::dry_run()) break;                                               \
        hipLaunchKernelGGL((kernel), (grid), (block), (lds), hx::stream(),       \
                           __VA_ARGS__);                                        \
        hx::note(hipGetLastError());                                            \
    } while (0)
