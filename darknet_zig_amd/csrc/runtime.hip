// runtime.hip -- device and memory glue of the C ABI. Replaces the HIP backend
// interface of src/hip/hip.zig:60-135 and the device/memory half of
// src/gpu.zig (init 259-347, alloc/free/push/pull/sync 362-410).
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <mutex>

#include "dkz_internal.hpp"

namespace dkz {
namespace {

struct DeviceState {
    void *scratch = nullptr;
};

DeviceState g_devices[kMaxDevices];
std::mutex g_mutex;
// The stream and the sync-after-launch switch are process-wide, as gpu.zig's
// are (gpu.zig:178, hip.zig:134); atomics, so that a host thread setting them
// while another issues ops is a well-defined (if unordered) change.
std::atomic<hipStream_t> g_stream{nullptr};
std::atomic<bool> g_sync_after_launch{false};
// note_output / recently_written: the last few written ranges, each with
// the launch count just after the launch that wrote it.
struct WrittenRange {
    uintptr_t lo = 0, hi = 0;
    uint64_t at = 0;
};
std::atomic<uint64_t> g_launches{0};
std::mutex g_written_mutex;
WrittenRange g_written[4];
unsigned g_written_next = 0;
thread_local char g_context[512] = "";
thread_local const Scratch *t_scratch_override = nullptr;

bool env_flag(const char *name) {
    const char *v = getenv(name);
    return v != nullptr && v[0] != '\0' && v[0] != '0';
}

constexpr size_t kScratchBytes =
    kScratchPartials * sizeof(double) + kScratchGemmFloats * sizeof(float) + kScratchSlots * sizeof(uint64_t);

int ensure_scratch(int dev) {
    std::lock_guard<std::mutex> lock(g_mutex);
    if (g_devices[dev].scratch != nullptr) return 0;
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, kScratchBytes);
    if (e != hipSuccess) {
        set_error_context("allocating the scratch (%zu bytes)", kScratchBytes);
        return (int)e;
    }
    e = hipMemset(p, 0, kScratchBytes);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        (void)hipFree(p);
        set_error_context("zeroing the scratch");
        return (int)e;
    }
    g_devices[dev].scratch = p;
    return 0;
}

}  // namespace

hipStream_t current_stream() { return g_stream.load(std::memory_order_relaxed); }

bool sync_after_launch() { return g_sync_after_launch.load(std::memory_order_relaxed); }

void set_error_context(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_context, sizeof g_context, fmt, ap);
    va_end(ap);
}

void note_output(const void *p, uint64_t bytes) {
    if (p == nullptr || bytes == 0) return;
    std::lock_guard<std::mutex> lock(g_written_mutex);
    WrittenRange &w = g_written[g_written_next++ % 4];
    w.lo = (uintptr_t)p;
    w.hi = (uintptr_t)p + bytes;
    w.at = g_launches.load(std::memory_order_relaxed);
}

bool recently_written(const void *p, uint64_t bytes) {
    if (p == nullptr || bytes == 0 || bytes > kRecentMaxBytes) return false;
    const uintptr_t lo = (uintptr_t)p, hi = lo + bytes;
    const uint64_t now = g_launches.load(std::memory_order_relaxed);
    std::lock_guard<std::mutex> lock(g_written_mutex);
    for (const WrittenRange &w : g_written)
        if (w.hi > w.lo && lo >= w.lo && hi <= w.hi && now - w.at <= kRecentLaunches) return true;
    return false;
}

int after_launch(const char *name, dim3 grid, dim3 block) {
    g_launches.fetch_add(1, std::memory_order_relaxed);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error_context("HIP: launching %s <<<(%u,%u),(%u,%u)>>> failed: %s", name, grid.x, grid.y,
                          block.x, block.y, hipGetErrorString(e));
        return (int)e;
    }
    if (sync_after_launch()) {
        e = hipStreamSynchronize(current_stream());
        if (e != hipSuccess) {
            set_error_context("HIP: %s <<<(%u,%u),(%u,%u)>>> faulted: %s", name, grid.x, grid.y,
                              block.x, block.y, hipGetErrorString(e));
            return (int)e;
        }
    }
    return 0;
}

ScratchOverride::ScratchOverride(const Scratch *s) : prev_(t_scratch_override) { t_scratch_override = s; }

ScratchOverride::~ScratchOverride() { t_scratch_override = prev_; }

int device_scratch(Scratch *out) {
    if (t_scratch_override != nullptr) {
        *out = *t_scratch_override;
        return 0;
    }
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kMaxDevices) return (int)hipErrorInvalidDevice;
    if (g_devices[dev].scratch == nullptr) DKZ_TRY(ensure_scratch(dev));
    out->partials = static_cast<double *>(g_devices[dev].scratch);
    out->gemm = reinterpret_cast<float *>(out->partials + kScratchPartials);
    out->gemm_floats = kScratchGemmFloats;
    out->slots = reinterpret_cast<uint64_t *>(out->gemm + kScratchGemmFloats);
    return 0;
}

}  // namespace dkz

using namespace dkz;

extern "C" {

int dkz_device_count(int *count) {
    DKZ_REQUIRE(count != nullptr);
    return (int)hipGetDeviceCount(count);
}

int dkz_init(int device) {
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) {
        set_error_context("querying device count");
        return (int)e;
    }
    if (device < 0 || device >= count || device >= 64) {
        set_error_context("Requested GPU %d but only %d HIP device(s) present", device, count);
        return (int)hipErrorInvalidDevice;
    }
    e = hipSetDevice(device);
    if (e != hipSuccess) {
        set_error_context("selecting the device");
        return (int)e;
    }
    if (env_flag("DARKNET_GPU_SYNC") || env_flag("DARKNET_HIP_SYNC")) g_sync_after_launch = true;
    DKZ_TRY(ensure_scratch(device));
    DKZ_TRY(static_scratch_setup(device));
    batchnorm_prewarm();
    return 0;
}

int dkz_device_name(int device, char *buf, int len) {
    DKZ_REQUIRE(buf != nullptr && len > 0);
    buf[0] = '\0';
    hipDevice_t dev;
    hipError_t e = hipDeviceGet(&dev, device);
    if (e != hipSuccess) return (int)e;
    e = hipDeviceGetName(buf, len - 1 > 0 ? len - 1 : 1, dev);
    if (e != hipSuccess) return (int)e;
    if (buf[0] == '\0') {
        // Some boxes report no marketing name; the architecture name is there.
        hipDeviceProp_t prop;
        e = hipGetDeviceProperties(&prop, device);
        if (e != hipSuccess) return (int)e;
        snprintf(buf, (size_t)len, "%s", prop.gcnArchName);
    }
    return 0;
}

int dkz_mem_info(size_t *free_bytes, size_t *total_bytes) {
    DKZ_REQUIRE(free_bytes != nullptr && total_bytes != nullptr);
    return (int)hipMemGetInfo(free_bytes, total_bytes);
}

int dkz_malloc(void **ptr, size_t bytes) {
    DKZ_REQUIRE(ptr != nullptr);
    *ptr = nullptr;
    if (bytes == 0) return 0;
    hipError_t e = hipMalloc(ptr, bytes);
    if (e != hipSuccess) {
        set_error_context("device allocation of %zu bytes", bytes);
        *ptr = nullptr;
        return (int)e;
    }
    e = hipMemsetAsync(*ptr, 0, bytes, current_stream());
    if (e == hipSuccess) e = hipStreamSynchronize(current_stream());
    if (e != hipSuccess) {
        set_error_context("zeroing device memory");
        (void)hipFree(*ptr);
        *ptr = nullptr;
    }
    return (int)e;
}

int dkz_free(void *ptr) {
    if (ptr == nullptr) return 0;
    return (int)hipFree(ptr);
}

int dkz_memset_zero(void *ptr, size_t bytes) {
    if (bytes == 0) return 0;
    DKZ_REQUIRE(ptr != nullptr);
    return (int)hipMemsetAsync(ptr, 0, bytes, current_stream());
}

int dkz_copy_to_device(void *dst, const void *src, size_t bytes) {
    if (bytes == 0) return 0;
    DKZ_REQUIRE(dst != nullptr && src != nullptr);
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, current_stream());
    if (e == hipSuccess) e = hipStreamSynchronize(current_stream());
    if (e != hipSuccess) set_error_context("copy host to device");
    return (int)e;
}

int dkz_copy_to_host(void *dst, const void *src, size_t bytes) {
    if (bytes == 0) return 0;
    DKZ_REQUIRE(dst != nullptr && src != nullptr);
    const hipStream_t s = current_stream();
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        set_error_context("copy device to host");
        return (int)e;
    }
    return take_barrier_timeout();
}

int dkz_synchronize(void) {
    hipError_t e = hipStreamSynchronize(current_stream());
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        set_error_context("device synchronise");
        return (int)e;
    }
    return take_barrier_timeout();
}

const char *dkz_error_string(int err) { return hipGetErrorString((hipError_t)err); }

void dkz_set_sync_after_launch(int on) { g_sync_after_launch.store(on != 0); }

int dkz_get_sync_after_launch(void) { return sync_after_launch() ? 1 : 0; }

const char *dkz_last_error_context(void) { return g_context; }

int dkz_set_stream(void *stream) {
    g_stream.store(static_cast<hipStream_t>(stream));
    return 0;
}

void *dkz_get_stream(void) { return current_stream(); }

}  // extern "C"
