// softmax.hip -- grouped softmax (src/gpu.zig:614-629, CPU twin
// blas.zig:213-242), and the softmax layer's forward step with its
// cross-entropy loss fused in (layers/misc.zig:63-76).
//
// Group (b, g) holds n elements `stride` apart starting at
// b*batch_offset + g*group_offset. Per group the CPU twin takes the max
// (starting from -FLT_MAX), forms e_i = exp(x_i/T - max/T), sums the e_i left
// to right in f32 and divides. The contract for softmax is 1e-5 relative per
// element, so the contiguous-group kernels below (stride 1, n > 32) keep the
// twin's max and its exp argument x_i/T - max/T bit for bit but evaluate exp
// with expf_cw (under one ulp), add the exps as a tree (pairwise in f32
// within a lane, then in f64 across lanes by DPP/LDS butterflies:
// deterministic, and far closer to the exact sum than a sequential f32 one)
// and scale by one rounded reciprocal; every p is within 1e-6 relative of
// the exact softmax of the twin's arguments:
//
//  * n <= kSegMaxN (2048) with many groups: a segment of L = 4..64 lanes per
//    group, the group held in registers (16 or 32 floats a lane, read once in
//    float4s when aligned), max and sum over the segment by DPP; from 4096
//    groups each segment takes two groups in turn, the second's loads issued
//    before the first is worked on.
//  * n <= kWgMaxN (32768), or few groups: one workgroup (64..1024 lanes) per
//    group, held in registers, max and sum by DPP within waves and LDS
//    across them.
//  * longer groups: one workgroup per group, three passes over x (max; sum;
//    exps scaled and stored).
//
// Strided groups (the spatial softmax, elements `stride` apart) and groups
// of at most 32 elements keep the twin's sequential sum and the
// host-libm-identical expf_libm, and are bit-exact:
//
//  * side-by-side strided groups (group_offset 1) with n <= kTileMaxN: a
//    workgroup stages T = 8..64 consecutive groups in LDS; all its lanes
//    share the loads, exps and divides, and lane g < T takes group g's max
//    and sum.
//  * other strided groups, or n <= 32: one lane per group runs the twin's
//    three loops, eight loads at a time.
//
// dkz_softmax_layer_forward runs the layer's two calls (softmax, then
// softmax_x_ent over the whole batch) as one pass for contiguous groups
// longer than 32: the loss and delta are formed from each probability as it
// is stored, with softmax_x_ent's expressions.
#include <float.h>

#include "dkz_device.hpp"
#include "dkz_hints.hpp"
#include "dkz_internal.hpp"

namespace dkz {
namespace {

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

// The cross-entropy step of the softmax layer (layers/misc.zig:70-75,
// blas.zig:247-252), fused into the softmax pass: delta = t - p and
// loss = t != 0 ? -log(p) : 0 on the probabilities just stored.
struct Xent {
    const float *truth;
    float *delta;
    float *loss;
};

__device__ __forceinline__ void xent1(float p, float t, float &d, float &l) {
    l = (t != 0.0f) ? -logf(p) : 0.0f;
    d = t - p;
}

__device__ __forceinline__ float xent_loss(float p, float t) { return (t != 0.0f) ? -logf(p) : 0.0f; }

// A lane's share of one group, M = 4K floats held in registers. Slot m is
// element at(m): with float4 access (V4) lane j of P lanes holds float4s
// j, j+P, ..., otherwise elements j, j+P, j+2P, ...
template <int K, bool V4>
struct RowSlice {
    static constexpr int M = 4 * K;
    float v[M];
    uint32_t j, P;

    __device__ __forceinline__ uint32_t at(int m) const {
        return V4 ? 4 * (j + (uint32_t)(m >> 2) * P) + (uint32_t)(m & 3) : j + (uint32_t)m * P;
    }

    // Whether slot m lies inside a group of n elements (with float4 access n
    // is a multiple of 4, so a float4 is inside or outside as a whole).
    __device__ __forceinline__ bool inside(int m, uint32_t n) const {
        return V4 ? 4 * (j + (uint32_t)(m >> 2) * P) < n : j + (uint32_t)m * P < n;
    }

    // Slots past n (or of a dead group) read as `fill`. NT: nontemporal loads.
    template <bool NT = false>
    __device__ __forceinline__ void load(const float *p, uint32_t n, bool live, float fill) {
        if constexpr (V4) {
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const uint32_t q = j + (uint32_t)k * P;
                float4 a = make_float4(fill, fill, fill, fill);
                if (live && 4 * q < n) a = ld4<NT>(p, q);
                v[4 * k] = a.x;
                v[4 * k + 1] = a.y;
                v[4 * k + 2] = a.z;
                v[4 * k + 3] = a.w;
            }
        } else {
#pragma unroll
            for (int m = 0; m < M; ++m) v[m] = (live && inside(m, n)) ? ld1<NT>(p, at(m)) : fill;
        }
    }

    __device__ __forceinline__ float max() const {
        float mx = v[0];
#pragma unroll
        for (int m = 1; m < M; ++m) mx = fmaxf(mx, v[m]);
        return mx;
    }

    // v[m] <- exp(v[m]/T - mt) for the slots inside the group (0 elsewhere);
    // returns their sum, added pairwise in f32 (error below 2^-21 relative
    // for 32 terms) and widened to f64 for the cross-lane sum -- or NaN when
    // an argument is NaN (a NaN logit, or +inf's inf - inf), which makes the
    // whole group NaN as the twin's NaN sum does. The twin's argument
    // x/T - max/T is formed exactly as the twin forms it (x/1 is x, so T == 1
    // skips the divides).
    __device__ __forceinline__ double exps(uint32_t n, bool live, float temp, float mt) {
        bool nan = false;
        if (temp == 1.0f) {
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float a = v[m] - mt;
                const bool in = live && inside(m, n);
                nan |= in && a != a;
                v[m] = expf_cw_num(in ? a : -__builtin_inff());  // exp(-inf) = 0 outside the group
            }
        } else {
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float a = v[m] / temp - mt;
                const bool in = live && inside(m, n);
                nan |= in && a != a;
                v[m] = expf_cw_num(in ? a : -__builtin_inff());
            }
        }
        float t[M];
#pragma unroll
        for (int m = 0; m < M; ++m) t[m] = v[m];
#pragma unroll
        for (int w = M / 2; w >= 1; w /= 2) {
#pragma unroll
            for (int m = 0; m < w; ++m) t[m] = t[m] + t[m + w];
        }
        return nan ? (double)__builtin_nanf("") : (double)t[0];
    }

    // p = e * inv into `out`; with XENT also delta and loss, from the truth
    // held in `tr` (EARLY) or read from `truth` here. The losses' logs run
    // only in waves where some lane holds a nonzero truth (with one-hot
    // truth, most waves store zeros).
    template <bool XENT, bool EARLY = true, int HS = 0>
    __device__ __forceinline__ void store(float *out, uint32_t n, bool live, float inv, const RowSlice &tr,
                                          const float *truth, float *delta, float *loss) {
        constexpr bool kNtP = (HS & 2) != 0, kNtT = (HS & 4) != 0, kNtDL = (HS & 8) != 0;
        float t[XENT ? M : 1];
        bool any = false;
        if constexpr (XENT) {
#pragma unroll
            for (int m = 0; m < M; ++m) {
                if constexpr (EARLY) t[m] = tr.v[m];
                else t[m] = (live && inside(m, n)) ? ld1<kNtT>(truth, at(m)) : 0.0f;
                any |= t[m] != 0.0f;
            }
        }
#pragma unroll
        for (int m = 0; m < M; ++m) v[m] = v[m] * inv;
        if constexpr (V4) {
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const uint32_t q = j + (uint32_t)k * P;
                if (!(live && 4 * q < n)) continue;
                st4<kNtP>(out, q, make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]));
                if constexpr (XENT)
                    st4<kNtDL>(delta, q, make_float4(t[4 * k] - v[4 * k], t[4 * k + 1] - v[4 * k + 1],
                                                     t[4 * k + 2] - v[4 * k + 2], t[4 * k + 3] - v[4 * k + 3]));
            }
        } else {
#pragma unroll
            for (int m = 0; m < M; ++m) {
                if (!(live && inside(m, n))) continue;
                st1<kNtP>(out, at(m), v[m]);
                if constexpr (XENT) st1<kNtDL>(delta, at(m), t[m] - v[m]);
            }
        }
        if constexpr (XENT) {
            float l[M];
            if (__ballot(any) != 0) {
#pragma unroll
                for (int m = 0; m < M; ++m) l[m] = xent_loss(v[m], t[m]);
            } else {
#pragma unroll
                for (int m = 0; m < M; ++m) l[m] = 0.0f;
            }
            if constexpr (V4) {
#pragma unroll
                for (int k = 0; k < K; ++k) {
                    const uint32_t q = j + (uint32_t)k * P;
                    if (live && 4 * q < n)
                        st4<kNtDL>(loss, q, make_float4(l[4 * k], l[4 * k + 1], l[4 * k + 2], l[4 * k + 3]));
                }
            } else {
#pragma unroll
                for (int m = 0; m < M; ++m)
                    if (live && inside(m, n)) st1<kNtDL>(loss, at(m), l[m]);
            }
        }
    }
};

// Segments of L lanes, one group each; blockDim.x / L groups a workgroup.
// The group's truth is read with its logits (XENT), so the loss costs no
// second memory round trip.
template <int L, int K, bool V4, bool XENT>
__global__ __launch_bounds__(kBlock) void softmax_seg_kernel(const float *in, float *out, Groups G, uint32_t rows,
                                                             Xent xe) {
    constexpr int HS = XENT ? DKZ_HINT_SOFTMAX_XENT : DKZ_HINT_SOFTMAX;
    const uint32_t t = threadIdx.x;
    const uint32_t r = blockIdx.x * (blockDim.x / L) + t / L;
    const bool live = r < rows;  // the same for the whole segment
    const uint32_t off = group_base(live ? r : 0u, G), n = G.n;
    RowSlice<K, V4> x;
    x.j = t & (L - 1);
    x.P = L;
    x.template load<(HS & 1) != 0>(in + off, n, live, -FLT_MAX);
    RowSlice<K, V4> tr;  // the truth (XENT only)
    if constexpr (XENT) {
        tr.j = x.j;
        tr.P = L;
        tr.template load<(HS & 4) != 0>(xe.truth + off, n, live, 0.0f);
    }
    const float mx = seg_max<L>(x.max());
    const double s = seg_sum<L>(x.exps(n, live, G.temp, mx / G.temp));
    const float inv = (float)(1.0 / s);
    if constexpr (XENT) {
        x.template store<true, true, HS>(out + off, n, live, inv, tr, nullptr, xe.delta + off, xe.loss + off);
    } else {
        x.template store<false, true, HS>(out + off, n, live, inv, x, nullptr, nullptr, nullptr);
    }
}

// The segment kernel as a grid-stride loop: each segment takes groups
// r, r + R, r + 2R, ... (R = segments in the grid) and loads the next
// group before working on the current one, so each wave's reads and writes
// alternate over the kernel instead of all reads landing first.
template <int L, int K, bool V4>
__global__ __launch_bounds__(kBlock) void softmax_seg_stream_kernel(const float *in, float *out, Groups G,
                                                                    uint32_t rows) {
    constexpr int HS = DKZ_HINT_SOFTMAX;
    const uint32_t t = threadIdx.x;
    const uint32_t per_block = blockDim.x / L;
    const uint32_t stride = gridDim.x * per_block;
    uint32_t r = blockIdx.x * per_block + t / L;
    const uint32_t n = G.n;
    RowSlice<K, V4> cur, nxt;
    cur.j = nxt.j = t & (L - 1);
    cur.P = nxt.P = L;
    bool live = r < rows;
    uint32_t off = group_base(live ? r : 0u, G);
    cur.template load<(HS & 1) != 0>(in + off, n, live, -FLT_MAX);
    // every segment of the grid runs the same number of iterations, so the
    // whole wave stays active for the DPP reductions
    const uint32_t iters = (rows + stride - 1) / stride;
    for (uint32_t it = 0; it < iters; ++it) {
        const uint32_t rn = r + stride;
        const bool live_n = rn < rows;
        const uint32_t off_n = group_base(live_n ? rn : 0u, G);
        if (it + 1 < iters) nxt.template load<(HS & 1) != 0>(in + off_n, n, live_n, -FLT_MAX);
        const float mx = seg_max<L>(cur.max());
        const double s = seg_sum<L>(cur.exps(n, live, G.temp, mx / G.temp));
        const float inv = (float)(1.0 / s);
        cur.template store<false, true, HS>(out + off, n, live, inv, cur, nullptr, nullptr, nullptr);
#pragma unroll
        for (int m = 0; m < RowSlice<K, V4>::M; ++m) cur.v[m] = nxt.v[m];
        r = rn;
        live = live_n;
        off = off_n;
    }
}

// One workgroup (blockDim.x = 64..1024 lanes) per group.
template <int K, bool V4, bool XENT>
__global__ __launch_bounds__(1024) void softmax_wg_kernel(const float *in, float *out, Groups G, Xent xe) {
    __shared__ float red_f[16];
    __shared__ double red_d[16];
    const uint32_t t = threadIdx.x, nw = blockDim.x / kWave, w = t / kWave;
    const uint32_t off = group_base(blockIdx.x, G), n = G.n;
    constexpr int HS = XENT ? DKZ_HINT_SOFTMAX_XENT : DKZ_HINT_SOFTMAX;
    RowSlice<K, V4> x;
    x.j = t;
    x.P = blockDim.x;
    x.template load<(HS & 1) != 0>(in + off, n, true, -FLT_MAX);
    // The truth is read with the logits when it fits in registers beside
    // them (K <= 4), otherwise as the results are stored.
    constexpr bool kEarly = K <= 4;
    RowSlice<K, V4> tr;  // the truth (XENT and kEarly only)
    if constexpr (XENT && kEarly) {
        tr.j = t;
        tr.P = blockDim.x;
        tr.template load<(HS & 4) != 0>(xe.truth + off, n, true, 0.0f);
    }
    float mx = wave_max(x.max());
    if ((t & (kWave - 1)) == 0) red_f[w] = mx;
    __syncthreads();
    mx = red_f[0];
    for (uint32_t i = 1; i < nw; ++i) mx = fmaxf(mx, red_f[i]);
    double s = wave_sum(x.exps(n, true, G.temp, mx / G.temp));
    if ((t & (kWave - 1)) == 0) red_d[w] = s;
    __syncthreads();
    s = red_d[0];
    for (uint32_t i = 1; i < nw; ++i) s += red_d[i];
    const float inv = (float)(1.0 / s);
    if constexpr (XENT) {
        x.template store<true, kEarly, HS>(out + off, n, true, inv, tr, xe.truth + off, xe.delta + off,
                                           xe.loss + off);
    } else {
        x.template store<false, true, HS>(out + off, n, true, inv, x, nullptr, nullptr, nullptr);
    }
}

// Groups longer than a workgroup holds in registers: one workgroup of
// kBigBlock lanes per group, three passes over x (the max; the sum of the
// exps; the exps scaled and stored, with the loss when XENT), eight elements
// a lane in flight per step.
constexpr uint32_t kBigBlock = 1024;

template <bool XENT>
__global__ __launch_bounds__(kBigBlock) void softmax_big_kernel(const float *in, float *out, Groups G, Xent xe) {
    __shared__ float red_f[kBigBlock / kWave];
    __shared__ double red_d[kBigBlock / kWave];
    constexpr uint32_t kU = 8;
    const uint32_t t = threadIdx.x, w = t / kWave, n = G.n;
    const uint32_t off = group_base(blockIdx.x, G);
    const float *x = in + off;
    float mx = -FLT_MAX;
    for (uint32_t i0 = t; i0 < n; i0 += kBigBlock * kU) {
        float v[kU];
#pragma unroll
        for (uint32_t u = 0; u < kU; ++u) v[u] = i0 + u * kBigBlock < n ? x[i0 + u * kBigBlock] : -FLT_MAX;
#pragma unroll
        for (uint32_t u = 0; u < kU; ++u) mx = fmaxf(mx, v[u]);
    }
    mx = wave_max(mx);
    if ((t & (kWave - 1)) == 0) red_f[w] = mx;
    __syncthreads();
    mx = red_f[0];
    for (uint32_t i = 1; i < kBigBlock / kWave; ++i) mx = fmaxf(mx, red_f[i]);
    const float mt = mx / G.temp;
    double s = 0.0;
    for (uint32_t i0 = t; i0 < n; i0 += kBigBlock * kU) {
        float v[kU];
#pragma unroll
        for (uint32_t u = 0; u < kU; ++u) v[u] = i0 + u * kBigBlock < n ? x[i0 + u * kBigBlock] : 0.0f;
#pragma unroll
        for (uint32_t u = 0; u < kU; ++u)
            if (i0 + u * kBigBlock < n) s += (double)expf_cw(v[u] / G.temp - mt);
    }
    s = wave_sum(s);
    if ((t & (kWave - 1)) == 0) red_d[w] = s;
    __syncthreads();
    s = red_d[0];
    for (uint32_t i = 1; i < kBigBlock / kWave; ++i) s += red_d[i];
    const float inv = (float)(1.0 / s);
    for (uint32_t i0 = t; i0 < n; i0 += kBigBlock * kU) {
        float v[kU];
#pragma unroll
        for (uint32_t u = 0; u < kU; ++u) v[u] = i0 + u * kBigBlock < n ? x[i0 + u * kBigBlock] : 0.0f;
#pragma unroll
        for (uint32_t u = 0; u < kU; ++u) {
            const uint32_t i = i0 + u * kBigBlock;
            if (i >= n) continue;
            const float p = expf_cw(v[u] / G.temp - mt) * inv;
            out[off + i] = p;
            if constexpr (XENT) xent1(p, xe.truth[off + i], xe.delta[off + i], xe.loss[off + i]);
        }
    }
}

// Segment path: groups of up to kSegMaxN elements, L lanes each.
constexpr uint32_t kSegMaxN = 2048;
// Groups below which one workgroup per group is used even for short groups
// (more waves per group to spread a small launch over the CUs).
#ifndef DKZ_SOFTMAX_SEG_MIN_ROWS
#define DKZ_SOFTMAX_SEG_MIN_ROWS 1024
#endif
// Workgroup path: up to 1024 lanes x 32 floats.
constexpr uint32_t kWgMaxN = 32768;

// Groups per segment of the grid-stride kernel for many groups (>= 4096):
// measured cold at [8192,1000], 12.9 us one group per segment, 12.4 two,
// 13.8 four; 0 turns it off.
#ifndef DKZ_SOFTMAX_STREAM
#define DKZ_SOFTMAX_STREAM 2
#endif

template <int L, int K>
int launch_seg(const float *input, float *output, const Groups &G, uint32_t rows, bool v4, const Xent *xe) {
    if (DKZ_SOFTMAX_STREAM > 0 && !xe && rows >= 4096) {
        // DKZ_SOFTMAX_STREAM groups a segment on average
        const uint32_t per_block = (uint32_t)(kBlock / L);
        const dim3 grid(div_up(rows, per_block * DKZ_SOFTMAX_STREAM));
        void (*k)(const float *, float *, Groups, uint32_t) =
            v4 ? softmax_seg_stream_kernel<L, K, true> : softmax_seg_stream_kernel<L, K, false>;
        (void)hipGetLastError();
        hipLaunchKernelGGL(k, grid, dim3(kBlock), 0, current_stream(), input, output, G, rows);
        return after_launch("softmax_seg_stream", grid, dim3(kBlock));
    }
    // Four segments' waves a workgroup when that still gives >= 512
    // workgroups, else one wave (small launches reach more CUs).
    const uint32_t per_wave = (uint32_t)(kWave / L);
    const uint32_t block = (uint64_t)rows >= 512ull * 4 * per_wave ? (uint32_t)kBlock : (uint32_t)kWave;
    const dim3 grid(div_up(rows, block / L));
    const Xent x = xe ? *xe : Xent{nullptr, nullptr, nullptr};
    void (*k)(const float *, float *, Groups, uint32_t, Xent);
    if (xe) k = v4 ? softmax_seg_kernel<L, K, true, true> : softmax_seg_kernel<L, K, false, true>;
    else k = v4 ? softmax_seg_kernel<L, K, true, false> : softmax_seg_kernel<L, K, false, false>;
    (void)hipGetLastError();
    hipLaunchKernelGGL(k, grid, dim3(block), 0, current_stream(), input, output, G, rows, x);
    return after_launch(xe ? "softmax_xent_seg" : "softmax_seg", grid, dim3(block));
}

template <int K>
int launch_wg(const float *input, float *output, const Groups &G, uint32_t rows, uint32_t block, bool v4,
              const Xent *xe) {
    const Xent x = xe ? *xe : Xent{nullptr, nullptr, nullptr};
    void (*k)(const float *, float *, Groups, Xent);
    if (xe) k = v4 ? softmax_wg_kernel<K, true, true> : softmax_wg_kernel<K, false, true>;
    else k = v4 ? softmax_wg_kernel<K, true, false> : softmax_wg_kernel<K, false, false>;
    (void)hipGetLastError();
    hipLaunchKernelGGL(k, dim3(rows), dim3(block), 0, current_stream(), input, output, G, x);
    return after_launch(xe ? "softmax_xent_wg" : "softmax_wg", dim3(rows), dim3(block));
}

// Contiguous groups (stride 1) of more than 32 elements.
int softmax_contiguous(const float *input, float *output, const Groups &G, uint32_t rows, bool v4,
                       const Xent *xe) {
    const uint32_t n = G.n;
    if (n <= kSegMaxN && rows >= DKZ_SOFTMAX_SEG_MIN_ROWS) {
        if (n <= 64) return launch_seg<4, 4>(input, output, G, rows, v4, xe);
        if (n <= 128) return launch_seg<8, 4>(input, output, G, rows, v4, xe);
        if (n <= 256) return launch_seg<16, 4>(input, output, G, rows, v4, xe);
        if (n <= 512) return launch_seg<32, 4>(input, output, G, rows, v4, xe);
        if (n <= 1024) return launch_seg<64, 4>(input, output, G, rows, v4, xe);
        return launch_seg<64, 8>(input, output, G, rows, v4, xe);
    }
    if (n <= kWgMaxN) {
        // Lanes for about four floats each (64..1024), then 4K floats a lane.
        uint32_t block = kWave;
        while (block < 1024 && 4 * block < n) block *= 2;
        const uint32_t per_lane = (n + block - 1) / block;
        if (per_lane <= 4) return launch_wg<1>(input, output, G, rows, block, v4, xe);
        if (per_lane <= 8) return launch_wg<2>(input, output, G, rows, block, v4, xe);
        if (per_lane <= 16) return launch_wg<4>(input, output, G, rows, block, v4, xe);
        return launch_wg<8>(input, output, G, rows, block, v4, xe);
    }
    const Xent x = xe ? *xe : Xent{nullptr, nullptr, nullptr};
    if (xe)
        return launch("softmax_xent_big", softmax_big_kernel<true>, dim3(rows), dim3(kBigBlock), input, output, G, x);
    return launch("softmax_big", softmax_big_kernel<false>, dim3(rows), dim3(kBigBlock), input, output, G, x);
}

constexpr uint32_t kTileMaxN = 128;
// Workgroups a strided-softmax launch aims for: tiles of T = 64, 32, 16 or 8
// rows, the widest that still gives this many (a [64,85,13,13] spatial
// softmax has 10816 rows: 169 tiles of 64 leave most CUs idle).
#ifndef DKZ_SOFTMAX_TILE_MIN_WGS
#define DKZ_SOFTMAX_TILE_MIN_WGS 512
#endif

// Runs of 128 / T consecutive tiles (512 bytes of each element row) go to
// one XCD (xcd_run_block): a tile's runs rarely start on a 128-byte line, so
// neighbouring tiles share lines, which that XCD's L2 then fetches once.
// Rows r0 .. r0+T-1 (group r = b*groups + g); tile[i*T + l] holds element i
// of row r0 + l. Side-by-side groups make element i of the T rows T
// consecutive floats, so the loads are T-float runs.
template <uint32_t T>
__global__ __launch_bounds__(kBlock) void softmax_tile_kernel(const float *in, float *out, Groups G, uint32_t rows) {
    __shared__ float tile[kTileMaxN * T];
    __shared__ uint32_t base_sh[T];
    __shared__ float mt_sh[T], sum_sh[T];
    const uint32_t r0 = xcd_run_block(blockIdx.x, gridDim.x, T >= 128 ? 1u : 128u / T) * T;
    const uint32_t nr = rows - r0 < T ? rows - r0 : T;
    const uint32_t n = G.n, st = G.stride, total = n * T;
    const uint32_t t = threadIdx.x;
    if (t < T) base_sh[t] = t < nr ? group_base(r0 + t, G) : 0u;
    __syncthreads();
    // Eight loads per lane in flight: element i of row l for q = i*T + l.
    for (uint32_t q0 = t; q0 < total; q0 += kBlock * 8) {
        float v[8];
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u) {
            const uint32_t q = q0 + u * kBlock, l = q & (T - 1);
            v[u] = q < total && l < nr ? in[base_sh[l] + (q / T) * st] : 0.0f;
        }
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u)
            if (q0 + u * kBlock < total) tile[q0 + u * kBlock] = v[u];
    }
    __syncthreads();
    // The row lanes' max and sum read eight LDS entries ahead of folding them
    // (in element order), so each pass waits on LDS once per eight elements.
    if (t < nr) {
        float mx = -FLT_MAX;
        uint32_t i = 0;
        for (; i + 8 <= n; i += 8) {
            float v[8];
#pragma unroll
            for (uint32_t k = 0; k < 8; ++k) v[k] = tile[(i + k) * T + t];
#pragma unroll
            for (uint32_t k = 0; k < 8; ++k) mx = fmaxf(mx, v[k]);
        }
        for (; i < n; ++i) mx = fmaxf(mx, tile[i * T + t]);
        mt_sh[t] = mx / G.temp;
    }
    __syncthreads();
    for (uint32_t q = t; q < total; q += kBlock) {
        const uint32_t l = q & (T - 1);
        if (l < nr) tile[q] = expf_libm(tile[q] / G.temp - mt_sh[l]);
    }
    __syncthreads();
    if (t < nr) {
        float s = 0.0f;
        uint32_t i = 0;
        for (; i + 8 <= n; i += 8) {
            float v[8];
#pragma unroll
            for (uint32_t k = 0; k < 8; ++k) v[k] = tile[(i + k) * T + t];
#pragma unroll
            for (uint32_t k = 0; k < 8; ++k) s += v[k];
        }
        for (; i < n; ++i) s += tile[i * T + t];
        sum_sh[t] = s;
    }
    __syncthreads();
    for (uint32_t q = t; q < total; q += kBlock) {
        const uint32_t l = q & (T - 1);
        if (l < nr) out[base_sh[l] + (q / T) * st] = tile[q] / sum_sh[l];
    }
}

int softmax_tiles(const float *input, float *output, const Groups &G, uint32_t rows) {
    if (div_up(rows, 64u) >= DKZ_SOFTMAX_TILE_MIN_WGS)
        return launch("softmax_tile", softmax_tile_kernel<64>, dim3(div_up(rows, 64u)), dim3(kBlock), input, output,
                      G, rows);
    if (div_up(rows, 32u) >= DKZ_SOFTMAX_TILE_MIN_WGS)
        return launch("softmax_tile", softmax_tile_kernel<32>, dim3(div_up(rows, 32u)), dim3(kBlock), input, output,
                      G, rows);
    if (div_up(rows, 16u) >= DKZ_SOFTMAX_TILE_MIN_WGS)
        return launch("softmax_tile", softmax_tile_kernel<16>, dim3(div_up(rows, 16u)), dim3(kBlock), input, output,
                      G, rows);
    return launch("softmax_tile", softmax_tile_kernel<8>, dim3(div_up(rows, 8u)), dim3(kBlock), input, output, G,
                  rows);
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
    // Each loop takes its loads eight at a time, ahead of the arithmetic,
    // which stays in element order.
    constexpr uint32_t kB = 8;
    float mx = -FLT_MAX;
    uint32_t i = 0;
    for (; i + kB <= n; i += kB) {
        float v[kB];
#pragma unroll
        for (uint32_t k = 0; k < kB; ++k) v[k] = x[(i + k) * st];
#pragma unroll
        for (uint32_t k = 0; k < kB; ++k) mx = fmaxf(mx, v[k]);
    }
    for (; i < n; ++i) mx = fmaxf(mx, x[i * st]);
    const float mt = mx / G.temp;
    float s = 0.0f;
    for (i = 0; i + kB <= n; i += kB) {
        float v[kB];
#pragma unroll
        for (uint32_t k = 0; k < kB; ++k) v[k] = x[(i + k) * st];
#pragma unroll
        for (uint32_t k = 0; k < kB; ++k) {
            const float e = expf_libm(v[k] / G.temp - mt);
            s += e;
            y[(i + k) * st] = e;
        }
    }
    for (; i < n; ++i) {
        const float e = expf_libm(x[i * st] / G.temp - mt);
        s += e;
        y[i * st] = e;
    }
    for (i = 0; i + kB <= n; i += kB) {
        float v[kB];
#pragma unroll
        for (uint32_t k = 0; k < kB; ++k) v[k] = y[(i + k) * st];
#pragma unroll
        for (uint32_t k = 0; k < kB; ++k) y[(i + k) * st] = v[k] / s;
    }
    for (; i < n; ++i) y[i * st] = y[i * st] / s;
}

int softmax_run(const float *input, int n, int batch, int batch_offset, int groups, int group_offset, int stride,
                float temp, float *output, const Xent *xe) {
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
    if (!(stride == 1 && n > 32)) {
        DKZ_REQUIRE(xe == nullptr);
        if (group_offset == 1 && stride > 1 && (uint32_t)n <= kTileMaxN) return softmax_tiles(input, output, G, rows);
        return launch("softmax_lane", softmax_lane_kernel, dim3(div_up(rows, kBlock)), dim3(kBlock), input, output,
                      G, rows);
    }
    bool v4 = n % 4 == 0 && batch_offset % 4 == 0 && group_offset % 4 == 0 && aligned16(input) && aligned16(output);
    if (xe) v4 = v4 && aligned16(xe->truth) && aligned16(xe->delta) && aligned16(xe->loss);
    return softmax_contiguous(input, output, G, rows, v4, xe);
}

}  // namespace
}  // namespace dkz

using namespace dkz;

extern "C" {

int dkz_softmax(const float *input, int n, int batch, int batch_offset, int groups, int group_offset,
                int stride, float temp, float *output) {
    return softmax_run(input, n, batch, batch_offset, groups, group_offset, stride, temp, output, nullptr);
}

int dkz_softmax_layer_forward(int batch, int inputs, int groups, float temp, const float *input,
                              const float *truth, float *output, float *delta, float *loss) {
    DKZ_REQUIRE(inputs >= 0 && groups >= 0 && batch >= 0);
    if (groups == 0 || batch == 0 || inputs == 0) return 0;
    DKZ_REQUIRE(inputs % groups == 0);  // misc.zig:20
    const int per_group = inputs / groups;
    if (truth == nullptr)  // misc.zig:66: no truth, no loss
        return softmax_run(input, per_group, batch, inputs, groups, per_group, 1, temp, output, nullptr);
    DKZ_REQUIRE(delta != nullptr && loss != nullptr);
    if (per_group > 32) {
        const Xent xe{truth, delta, loss};
        return softmax_run(input, per_group, batch, inputs, groups, per_group, 1, temp, output, &xe);
    }
    // Short groups take the one-lane-per-group kernel; the loss is its own pass.
    DKZ_TRY(softmax_run(input, per_group, batch, inputs, groups, per_group, 1, temp, output, nullptr));
    DKZ_REQUIRE((uint64_t)batch * inputs <= kMaxElems);
    return dkz_softmax_cross_entropy(batch * inputs, output, truth, delta, loss);
}

}  // extern "C"
