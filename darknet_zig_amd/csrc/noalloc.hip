// noalloc.hip -- dkz_batchnorm_backward_noalloc: the batch-norm backward
// step (dkz_batchnorm_backward, batchnorm.hip) for callers that cannot
// allocate device memory -- code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc. It runs the same kernels with the
// same launch geometry (so its results are the regular entry point's, bit
// for bit), but every byte of scratch they use lives in `scratch` below, a
// file-scope device array, instead of the library's allocated scratch:
//   * kScratchPartials f64 partial sums (2 MiB): what a split reduction
//     hands from its partial pass to its finalisation. Every call writes all
//     the partials it then reads.
//   * kScratchSlots 64-bit counter slots (512 KiB): the workgroups of a split
//     channel reduction count themselves in their channel's slot to find the
//     last one, and those of a one-launch pass post their sums on lines
//     after the channel counters, so the slots must be zero when a call
//     starts. Every kernel leaves them at zero; each call clears them all
//     first anyway (a small kernel, not a memset, so the call can be captured
//     in a graph).
// Nothing here calls hipMalloc, hipFree or an allocating library routine.
// Each GPU holds its own copy of the array until the process ends; every
// call on a GPU shares it, so calls that overlap on one GPU (two streams,
// two host threads) race and must not be issued.
//
// The array's name is a host-side stand-in on the host: its device address,
// per device, comes from hipGetSymbolAddress (static_scratch_setup, called
// by dkz_init and by the first call on a device) and only that address is
// handed to kernels.
#include <mutex>

#include "dkz_device.hpp"
#include "dkz_internal.hpp"

namespace dkz {
namespace {

constexpr size_t kPartialsBytes = (size_t)kScratchPartials * sizeof(double);
constexpr size_t kSlotsBytes = (size_t)kScratchSlots * sizeof(uint64_t);
constexpr size_t kStaticScratchBytes = kPartialsBytes + kSlotsBytes;
static_assert(kPartialsBytes % 256 == 0, "slots stay 256-byte aligned");

static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

std::mutex g_setup_mutex;
void *g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device

__global__ __launch_bounds__(kBlock) void zero_slots_kernel(uint64_t *slots, uint32_t n) {
    const uint32_t i = blockIdx.x * kBlock + threadIdx.x;
    if (i < n) slots[i] = 0;
}

}  // namespace

int static_scratch_setup(int dev) {
    if (dev < 0 || dev >= kMaxDevices) return (int)hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_setup_mutex);
    if (g_scratch_ptr[dev] != nullptr) return 0;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
        set_error_context("looking up the static scratch of device %d: %s", dev, hipGetErrorString(e));
        return e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol;
    }
    g_scratch_ptr[dev] = p;
    return 0;
}

}  // namespace dkz

using namespace dkz;

extern "C" {

int dkz_batchnorm_backward_noalloc(int batch, int filters, int spatial, int activation, const float *output,
                                   float *delta, const float *x, const float *x_norm, const float *mean,
                                   const float *variance, const float *scales, float *bias_updates,
                                   float *scale_updates, float *mean_delta, float *variance_delta) {
    DKZ_REQUIRE(batch >= 0 && filters >= 0 && spatial >= 0);
    if (filters == 0) return 0;
    // Every split the kernels choose fits the array (pick_split sizes the
    // partials to kScratchPartials); the slots cover every channel a split
    // channel reduction counts in (reduce.hip).
    if ((uint64_t)batch * (uint64_t)filters * (uint64_t)spatial > kMaxElems) {
        set_error_context("%s: %d x %d x %d elements exceed the 2^31-1 the static scratch path supports", __func__,
                          batch, filters, spatial);
        return (int)hipErrorInvalidValue;
    }
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    DKZ_TRY(static_scratch_setup(dev));
    unsigned char *base = static_cast<unsigned char *>(g_scratch_ptr[dev]);
    const Scratch sc{reinterpret_cast<double *>(base), nullptr, 0,
                     reinterpret_cast<uint64_t *>(base + kPartialsBytes)};
    DKZ_TRY(launch("batchnorm_backward_noalloc_zero_slots", zero_slots_kernel, dim3(div_up(kScratchSlots, kBlock)),
                   dim3(kBlock), sc.slots, kScratchSlots));
    const ScratchOverride use(&sc);
    return dkz_batchnorm_backward(batch, filters, spatial, activation, output, delta, x, x_norm, mean, variance,
                                  scales, bias_updates, scale_updates, mean_delta, variance_delta);
}

}  // extern "C"
