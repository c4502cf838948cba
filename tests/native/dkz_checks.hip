// dkz_checks.hip -- test-only helpers that exercise the product's device
// header (darknet_zig_amd/csrc/dkz_device.hpp) directly:
//
//   * chk_fastdiv: the launch-constant division, run on the host;
//   * chk_xcd_run_block: the workgroup renumbering that keeps runs of
//     logical blocks on one XCD, run on the host;
//   * chk_exp2f_tab: the expf table entries, for the high-precision check;
//   * chk_expf_host_mismatches: expf_libm compiled for the host, compared
//     with the C library's expf over a range of float bit patterns;
//   * chk_expf_hash_host / chk_expf_hash_device: an order-independent hash of
//     expf over a bit-pattern range, from the C library (host) and from
//     expf_libm running on the GPU, so the two can be compared without moving
//     2^32 results;
//   * chk_expf_cw / chk_expf_cw_max_err / chk_expf_cw_hash_*: the same for
//     expf_cw, softmax's exp: its host build against exp in double (the
//     largest error in ulps over a bit-pattern range), and the hash of its
//     host build against its device build (they must agree bit for bit).
//
// Built by tests/native/build.py into tests/native/libdkz_checks.so.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <thread>
#include <vector>

#include "dkz_device.hpp"

namespace {

inline uint32_t bits_of(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

// NaN results are compared as one canonical NaN: the libraries agree on
// NaN-ness, not on payload bits.
__host__ __device__ inline uint32_t canon(uint32_t u) {
    return ((u & 0x7fffffffu) > 0x7f800000u) ? 0x7fc00000u : u;
}

__host__ __device__ inline uint64_t mix(uint64_t i, uint32_t r) {
    uint64_t z = (i * 0x9e3779b97f4a7c15ull) ^ ((uint64_t)r * 0xbf58476d1ce4e5b9ull);
    z ^= z >> 31;
    z *= 0x94d049bb133111ebull;
    return z ^ (z >> 29);
}

template <class F>
uint64_t parallel_sum(uint64_t lo, uint64_t hi, int threads, F f) {
    if (threads < 1) threads = 1;
    std::vector<uint64_t> part(threads, 0);
    std::vector<std::thread> pool;
    for (int t = 0; t < threads; ++t) {
        pool.emplace_back([&, t] {
            const uint64_t a = lo + (hi - lo) * t / threads, b = lo + (hi - lo) * (t + 1) / threads;
            uint64_t s = 0;
            for (uint64_t i = a; i < b; ++i) s += f(i);
            part[t] = s;
        });
    }
    for (auto &th : pool) th.join();
    uint64_t s = 0;
    for (uint64_t v : part) s += v;
    return s;
}

template <class F>
uint64_t parallel_max(uint64_t lo, uint64_t hi, int threads, F f) {
    if (threads < 1) threads = 1;
    std::vector<uint64_t> part(threads, 0);
    std::vector<std::thread> pool;
    for (int t = 0; t < threads; ++t) {
        pool.emplace_back([&, t] {
            const uint64_t a = lo + (hi - lo) * t / threads, b = lo + (hi - lo) * (t + 1) / threads;
            uint64_t m = 0;
            for (uint64_t i = a; i < b; ++i) {
                const uint64_t v = f(i);
                m = v > m ? v : m;
            }
            part[t] = m;
        });
    }
    for (auto &th : pool) th.join();
    uint64_t m = 0;
    for (uint64_t v : part) m = v > m ? v : m;
    return m;
}

// |expf_cw(x) - exp(x)| in 1/1024 ulps of the float nearest exp(x) (the ulp
// of a subnormal being 2^-149), exp(x) evaluated in double; 0 for NaN inputs
// when the result is NaN.
uint64_t expf_cw_err(uint64_t i) {
    float x;
    const uint32_t u = (uint32_t)i;
    memcpy(&x, &u, 4);
    const float y = dkz::expf_cw(x);
    if (x != x) return y != y ? 0u : ~0ull;
    const double e = exp((double)x);
    const float ef = (float)e;
    if (isinf(ef) || isinf(y)) return (isinf(ef) && isinf(y)) ? 0u : ~0ull;
    int ex = 0;
    frexp(e, &ex);
    const double ulp = ldexp(1.0, (ex - 24 < -149) ? -149 : ex - 24);
    return (uint64_t)(fabs((double)y - e) / ulp * 1024.0);
}

__global__ void expf_cw_hash_kernel(uint64_t lo, uint64_t hi, unsigned long long *out) {
    uint64_t s = 0;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = lo + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < hi; i += stride) {
        const uint32_t u = (uint32_t)i;
        float x;
        __builtin_memcpy(&x, &u, 4);
        const float r = dkz::expf_cw(x);
        uint32_t rb;
        __builtin_memcpy(&rb, &r, 4);
        s += mix(i, canon(rb));
    }
    atomicAdd(out, (unsigned long long)s);
}

__global__ void expf_hash_kernel(uint64_t lo, uint64_t hi, unsigned long long *out) {
    uint64_t s = 0;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = lo + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < hi; i += stride) {
        const uint32_t u = (uint32_t)i;
        float x;
        __builtin_memcpy(&x, &u, 4);
        const float r = dkz::expf_libm(x);
        uint32_t rb;
        __builtin_memcpy(&rb, &r, 4);
        s += mix(i, canon(rb));
    }
    atomicAdd(out, (unsigned long long)s);
}

}  // namespace

extern "C" {

uint32_t chk_fastdiv(uint32_t n, uint32_t d) { return dkz::fdiv(n, dkz::make_fastdiv(d)); }

uint32_t chk_xcd_run_block(uint32_t b, uint32_t grid, uint32_t r) { return dkz::xcd_run_block(b, grid, r); }

uint64_t chk_exp2f_tab(uint32_t i) { return dkz::exp2f_tab(i); }

float chk_expf_restated(float x) { return dkz::expf_libm(x); }

uint64_t chk_expf_host_mismatches(uint64_t lo, uint64_t hi, int threads) {
    return parallel_sum(lo, hi, threads, [](uint64_t i) -> uint64_t {
        float x;
        const uint32_t u = (uint32_t)i;
        memcpy(&x, &u, 4);
        return canon(bits_of(dkz::expf_libm(x))) != canon(bits_of(expf(x))) ? 1u : 0u;
    });
}

uint64_t chk_expf_hash_host(uint64_t lo, uint64_t hi, int threads) {
    return parallel_sum(lo, hi, threads, [](uint64_t i) -> uint64_t {
        float x;
        const uint32_t u = (uint32_t)i;
        memcpy(&x, &u, 4);
        return mix(i, canon(bits_of(expf(x))));
    });
}

float chk_expf_cw(float x) { return dkz::expf_cw(x); }

uint64_t chk_expf_cw_max_err(uint64_t lo, uint64_t hi, int threads) {
    return parallel_max(lo, hi, threads, expf_cw_err);
}

uint64_t chk_expf_cw_hash_host(uint64_t lo, uint64_t hi, int threads) {
    return parallel_sum(lo, hi, threads, [](uint64_t i) -> uint64_t {
        float x;
        const uint32_t u = (uint32_t)i;
        memcpy(&x, &u, 4);
        return mix(i, canon(bits_of(dkz::expf_cw(x))));
    });
}

// Returns a hipError_t; *hash receives the device-side hash of expf_cw.
int chk_expf_cw_hash_device(uint64_t lo, uint64_t hi, uint64_t *hash) {
    unsigned long long *d = nullptr;
    hipError_t e = hipMalloc(&d, sizeof *d);
    if (e != hipSuccess) return (int)e;
    e = hipMemset(d, 0, sizeof *d);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(expf_cw_hash_kernel, dim3(8192), dim3(256), 0, nullptr, lo, hi, d);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    unsigned long long h = 0;
    if (e == hipSuccess) e = hipMemcpy(&h, d, sizeof h, hipMemcpyDeviceToHost);
    (void)hipFree(d);
    *hash = h;
    return (int)e;
}

// Returns a hipError_t; *hash receives the device-side hash.
int chk_expf_hash_device(uint64_t lo, uint64_t hi, uint64_t *hash) {
    unsigned long long *d = nullptr;
    hipError_t e = hipMalloc(&d, sizeof *d);
    if (e != hipSuccess) return (int)e;
    e = hipMemset(d, 0, sizeof *d);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(expf_hash_kernel, dim3(8192), dim3(256), 0, nullptr, lo, hi, d);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    unsigned long long h = 0;
    if (e == hipSuccess) e = hipMemcpy(&h, d, sizeof h, hipMemcpyDeviceToHost);
    (void)hipFree(d);
    *hash = h;
    return (int)e;
}

}  // extern "C"
