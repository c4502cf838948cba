// softmax.hip -- grouped softmax (src/gpu.zig:614-629, CPU twin
// blas.zig:213-242).
//
// Group (b, g) holds n elements `stride` apart starting at
// b*batch_offset + g*group_offset. Per group the CPU twin takes the max
// (starting from -FLT_MAX), writes e_i = exp(x_i/T - max/T), sums the e_i
// left to right in f32 and divides. Every step except that sum is exact or
// elementwise, and exp is the host-identical expf_libm, so the kernels below
// reproduce the twin bit for bit wherever they keep the sequential sum:
//
//  * contiguous groups (stride 1) with 32 < n <= kSeqMax: one workgroup per
//    group; max by wave64 DPP + LDS, the exps in parallel into LDS, one lane
//    adds them in order, then all lanes divide. Bit-exact.
//  * contiguous groups with n > kSeqMax: the same, but the sum is an f64
//    tree (within 1e-5 relative of the twin) because the row no longer fits
//    in LDS.
//  * strided groups (spatial softmax) or n <= 32: one lane per group runs the
//    twin's three loops; adjacent lanes are adjacent groups, so with
//    group_offset 1 the loads coalesce. Bit-exact.
#include <float.h>

#include "dkz_device.hpp"
#include "dkz_internal.hpp"

namespace dkz {
namespace {

constexpr uint32_t kSeqMax = 8192;  // floats staged in LDS (32 KiB)

struct Groups {
    uint32_t n, groups, batch_offset, group_offset, stride;
    float temp;
    FastDiv div_groups;
};

__device__ __forceinline__ uint32_t group_base(uint32_t r, const Groups &G) {
    const uint32_t b = fdiv(r, G.div_groups);
    const uint32_t g = r - b * G.groups;
    return b * G.batch_offset + g * G.group_offset;
}

template <bool SEQ>
__global__ __launch_bounds__(kBlock) void softmax_block_kernel(const float *in, float *out, Groups G) {
    extern __shared__ float4 e_lds4[];  // n floats when SEQ; float4 keeps it 16-byte aligned
    float *e_lds = reinterpret_cast<float *>(e_lds4);
    __shared__ float red_f[kBlock / kWave];
    __shared__ double red_d[kBlock / kWave];
    __shared__ float sum_sh;
    const uint32_t off = group_base(blockIdx.x, G);
    const float *x = in + off;
    float *y = out + off;
    const uint32_t n = G.n;

    float mx = -FLT_MAX;
    for (uint32_t i = threadIdx.x; i < n; i += kBlock) mx = fmaxf(mx, x[i]);
    mx = block_max(mx, red_f);
    const float mt = mx / G.temp;

    float sum;
    if constexpr (SEQ) {
        for (uint32_t i = threadIdx.x; i < n; i += kBlock) e_lds[i] = expf_libm(x[i] / G.temp - mt);
        __syncthreads();
        if (threadIdx.x == 0) {
            // The one sequential part: 8 LDS reads in flight ahead of the adds.
            float s = 0.0f;
            uint32_t i = 0;
            for (; i + 32 <= n; i += 32) {
                float4 v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] = e_lds4[(i >> 2) + u];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    s += v[u].x;
                    s += v[u].y;
                    s += v[u].z;
                    s += v[u].w;
                }
            }
            for (; i < n; ++i) s += e_lds[i];
            sum_sh = s;
        }
        __syncthreads();
        sum = sum_sh;
        for (uint32_t i = threadIdx.x; i < n; i += kBlock) y[i] = e_lds[i] / sum;
    } else {
        double acc = 0.0;
        for (uint32_t i = threadIdx.x; i < n; i += kBlock) {
            const float e = expf_libm(x[i] / G.temp - mt);
            y[i] = e;
            acc += (double)e;
        }
        sum = (float)block_sum(acc, red_d);
        for (uint32_t i = threadIdx.x; i < n; i += kBlock) y[i] = y[i] / sum;
    }
}

// One lane per group: blas.zig:213-223 verbatim.
__global__ __launch_bounds__(kBlock) void softmax_lane_kernel(const float *in, float *out, Groups G,
                                                              uint32_t rows) {
    const uint32_t r = blockIdx.x * kBlock + threadIdx.x;
    if (r >= rows) return;
    const uint32_t off = group_base(r, G);
    const float *x = in + off;
    float *y = out + off;
    const uint32_t n = G.n, st = G.stride;
    float mx = -FLT_MAX;
    for (uint32_t i = 0; i < n; ++i) mx = fmaxf(mx, x[i * st]);
    const float mt = mx / G.temp;
    float s = 0.0f;
    for (uint32_t i = 0; i < n; ++i) {
        const float e = expf_libm(x[i * st] / G.temp - mt);
        s += e;
        y[i * st] = e;
    }
    for (uint32_t i = 0; i < n; ++i) y[i * st] = y[i * st] / s;
}

}  // namespace
}  // namespace dkz

using namespace dkz;

extern "C" {

int dkz_softmax(const float *input, int n, int batch, int batch_offset, int groups, int group_offset,
                int stride, float temp, float *output) {
    DKZ_REQUIRE(n >= 0 && batch >= 0 && batch_offset >= 0 && groups >= 0 && group_offset >= 0 && stride >= 0);
    const uint64_t rows64 = (uint64_t)batch * (uint64_t)groups;
    if (rows64 == 0 || n == 0) return 0;  // gpu.zig:625 launches batch*groups lanes
    DKZ_REQUIRE(input && output);
    // Highest element touched must stay in 32-bit range.
    const uint64_t last = (uint64_t)(batch - 1) * batch_offset + (uint64_t)(groups - 1) * group_offset +
                          (uint64_t)(n - 1) * stride;
    DKZ_REQUIRE(last <= kMaxElems && rows64 <= kMaxElems);
    const uint32_t rows = (uint32_t)rows64;
    const Groups G{(uint32_t)n,      (uint32_t)groups, (uint32_t)batch_offset, (uint32_t)group_offset,
                   (uint32_t)stride, temp,             make_fastdiv((uint32_t)groups)};
    if (stride == 1 && n > 32) {
        (void)hipGetLastError();
        if ((uint32_t)n <= kSeqMax) {
            hipLaunchKernelGGL(softmax_block_kernel<true>, dim3(rows), dim3(kBlock), (size_t)n * sizeof(float),
                               current_stream(), input, output, G);
        } else {
            hipLaunchKernelGGL(softmax_block_kernel<false>, dim3(rows), dim3(kBlock), 0, current_stream(), input,
                               output, G);
        }
        return after_launch("softmax", dim3(rows), dim3(kBlock));
    }
    return launch("softmax_lane", softmax_lane_kernel, dim3(div_up(rows, kBlock)), dim3(kBlock), input, output,
                  G, rows);
}

}  // extern "C"
