// Host-side internals shared by every translation unit of libhexlib_gpu.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hexlib_gpu.h"

namespace hx {

// The stream every per-kernel API call enqueues on: the calling host thread's
// (hexlib_gpu_set_stream sets it for that thread only).
hipStream_t stream();
// Records this thread's first failing launch status until
// hexlib_gpu_take_error() (per host thread, like the stream).
void note(hipError_t e);
// Per-thread flag: while set (a DRYRUN invoke), API functions validate their
// arguments and return without touching the GPU.
bool dry_run();
void set_dry_run(bool on);

// Device scratch of one owner: the split-K workspace, grow-only per device.
// Each session owns one, so sessions driven from different threads never
// share partial results; direct per-kernel calls use the process default one
// (calls that overlap in time on different streams then share it and must
// not split K concurrently). While a session's invoke runs, its scratch is
// the calling thread's current one.
struct Scratch;
Scratch *scratch_new();
// Frees every buffer the scratch ever held; the owner's work must be done.
void scratch_free(Scratch *s);
Scratch *current_scratch();
void set_current_scratch(Scratch *s);   // nullptr: the process default

// The split-K workspace of at least `bytes` on the current device, from the
// current scratch, or nullptr when it cannot be had without an allocation
// during stream capture (the caller then runs without split-K) -- or, under a
// FixedWorkspace, when it does not fit that buffer (refused() then says so).
float *workspace(size_t bytes);
// Dry runs record the largest workspace a validated blob will need ...
void reserve_workspace(size_t bytes);
// ... and this allocates it in the current scratch (hipMalloc, outside any
// capture). 0 on success.
int prepare_workspace();

// For the calling thread while alive: workspace() hands out `ptr` (capacity
// `cap` bytes) and never allocates; a larger request is refused.
struct FixedWorkspace {
    FixedWorkspace(float *ptr, size_t cap);
    ~FixedWorkspace();
    static bool refused();
};

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


// Every launch goes through here: skipped under a dry run, error recorded.
#define HX_LAUNCH(kernel, grid, block, lds, ...)                                  \
    do {                                                                        \
        if (hx::dry_run()) break;                                               \
        hipLaunchKernelGGL((kernel), (grid), (block), (lds), hx::stream(),       \
                           __VA_ARGS__);                                        \
        hx::note(hipGetLastError());                                            \
    } while (0)
