// dkz_internal.hpp -- host-side plumbing shared by the op sources: the current
// stream, argument checks, the launch helper with sync-after-launch, and the
// per-device reduction scratch. Not part of the ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dkz_ops.h"

namespace dkz {

// Stream every op and copy is issued on (the null stream by default).
hipStream_t current_stream();

// Records "what failed" for dkz_last_error_context on this host thread.
void set_error_context(const char *fmt, ...);

// Called right after a kernel launch: reports a launch error, and under
// sync-after-launch waits for the kernel and reports its fault. `name` and the
// launch shape go into the error context (gpu.zig:445-462).
int after_launch(const char *name, dim3 grid, dim3 block);

// Whether sync-after-launch is on (DARKNET_GPU_SYNC, dkz_set_sync_after_launch).
bool sync_after_launch();

// The one-launch batch-norm passes (batchnorm.hip) wait for the other
// workgroups of their channel for a bounded time; one that gives up writes
// NaN results, leaves the state that outlives the call alone and records its
// kernel in a device word. take_barrier_timeout reads that word on the
// current device (synchronously) and clears it: 0 when it was clear, else
// hipErrorLaunchTimeOut with the kernel named in the error context.
// Called by dkz_synchronize and dkz_copy_to_host (where the reference's
// kernel faults surface) and, under sync-after-launch, right after the pass.
int take_barrier_timeout();

// Producer-to-consumer reuse of the 256 MB Infinity Cache. Every kernel
// launch advances a count (after_launch); the elementwise and broadcast ops
// record the range each launch wrote (note_output). recently_written(p, n)
// tells whether [p, p + n) lies in a range written by one of the last
// kRecentLaunches launches and is at most kRecentMaxBytes: the cache then
// likely holds it, and a single-stream reduction reads it with ordinary
// loads (which find it there and leave it for the op after); otherwise with
// nontemporal loads, which stream data from HBM faster but leave the cache
// without it. A hint only: results do not depend on it. Process-wide (the
// reference drives one device from one host thread).
constexpr uint64_t kRecentLaunches = 2;
constexpr uint64_t kRecentMaxBytes = 192ull << 20;
void note_output(const void *p, uint64_t bytes);
bool recently_written(const void *p, uint64_t bytes);

// Makes the batch-norm passes' occupancy and kernel-attribute lookups for
// the current device now (dkz_init), so no op makes one for the first time
// inside a graph capture.
void batchnorm_prewarm();

template <typename Kernel, typename... Args>
inline int launch(const char *name, Kernel kernel, dim3 grid, dim3 block, Args... args) {
    (void)hipGetLastError();  // a stale error from the caller's own calls is not ours
    hipLaunchKernelGGL(kernel, grid, block, 0, current_stream(), args...);
    return after_launch(name, grid, block);
}

// Devices the library keeps per-device state for (ordinals 0..63).
constexpr int kMaxDevices = 64;

// Scratch of the current device, allocated once by dkz_init (or on first
// use) and zeroed then: the f64 partial sums one split channel reduction
// hands from its first launch to its second, the partial tiles of a split-K
// gemm, and one 64-bit counter slot per channel for the reductions whose
// workgroups count themselves in to find the channel's last (reduce.hip).
// Every user writes all the
// partials and tiles it then reads; the slots start at zero and every user
// leaves them at zero.
struct Scratch {
    double *partials;
    float *gemm;
    uint64_t gemm_floats;
    uint64_t *slots;
};
constexpr uint32_t kScratchPartials = 1u << 18;    // channels * chunks (2 MiB of f64)
#ifndef DKZ_SCRATCH_GEMM_LOG2
#define DKZ_SCRATCH_GEMM_LOG2 25
#endif
constexpr uint64_t kScratchGemmFloats = 1ull << DKZ_SCRATCH_GEMM_LOG2;  // split-K partial tiles (128 MiB)
constexpr uint32_t kScratchSlots = 1u << 16;         // 64-bit counter slots (512 KiB)
// A split reduction's per-channel counters and f64 partials sit
// kCounterStride / kPartialStride elements apart, so that no two share a
// 128-byte line: atomics and write-through stores to one line are
// serialised at the memory side.
#ifndef DKZ_SPLIT_CSTRIDE
#define DKZ_SPLIT_CSTRIDE 32
#endif
#ifndef DKZ_SPLIT_PSTRIDE
#define DKZ_SPLIT_PSTRIDE 16
#endif
constexpr uint32_t kCounterStride = DKZ_SPLIT_CSTRIDE;
constexpr uint32_t kPartialStride = DKZ_SPLIT_PSTRIDE;
int device_scratch(Scratch *out);

// While one of these lives, device_scratch() on this host thread returns
// *s instead of the library's allocated scratch (and allocates nothing): the
// no-allocation entry point runs the regular code with its static scratch.
class ScratchOverride {
  public:
    explicit ScratchOverride(const Scratch *s);
    ~ScratchOverride();
    ScratchOverride(const ScratchOverride &) = delete;
    ScratchOverride &operator=(const ScratchOverride &) = delete;

  private:
    const Scratch *prev_;
};

// Per-device set-up of the static scratch of the no-allocation entry point
// (noalloc.hip): looks its address up once for the current device `dev`.
int static_scratch_setup(int dev);

// Largest element count any op indexes with 32-bit arithmetic, as the
// reference's kernels do (int global_index(), darknet_kernels.hip:40-42).
constexpr uint64_t kMaxElems = 0x7fffffffull;

inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

inline uint32_t div_up(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

}  // namespace dkz

#define DKZ_REQUIRE(cond)                                                    \
    do {                                                                     \
        if (!(cond)) {                                                       \
            ::dkz::set_error_context("%s: invalid argument (%s)", __func__, #cond); \
            return (int)hipErrorInvalidValue;                                \
        }                                                                    \
    } while (0)

#define DKZ_TRY(expr)                    \
    do {                                 \
        const int dkz_rc_ = (expr);      \
        if (dkz_rc_ != 0) return dkz_rc_; \
    } while (0)
