// reduce.hip -- per-channel reductions over N*H*W (mean, variance, mean_delta,
// variance_delta, backward_bias, backward_scale: src/gpu.zig:539-590) and the
// per-row reduction of global average pooling (gpu.zig:761-763).
//
// Channel reductions:
//   * The grid is filters x K workgroups; workgroup (f, k) owns the k-th
//     contiguous chunk of channel f's batch*spatial elements. K is picked from
//     the shape only, so a shape always reduces in the same order on any GPU.
//   * Each lane computes the CPU twin's per-element term in f32 -- x, (x-m)^2,
//     delta*x_norm, delta*(x-m), rounded exactly as blas.zig rounds them -- and
//     accumulates it in f64. A chunk is then summed by wave64 DPP reductions
//     and a 4-entry LDS step (dkz_device.hpp).
//   * K (chan_split) aims at ~1024 workgroups in all, so the grid covers the
//     256 CUs several times whatever the channel count. K == 1 (channels
//     alone enough): the workgroup, 1024 threads wide for long channels,
//     finalises its channel itself. 128..255 long channels: two 1024-thread
//     workgroups each, meeting through one atomic exchange
//     (chan_pair_kernel). Otherwise K > 1: one launch in which the last
//     workgroup of each channel to finish adds the channel's K f64 partials
//     in index order and finalises (chan_split_kernel: coherent atomic
//     stores and a per-channel counter, no fence, nothing waits). The result
//     is deterministic, and it is the exact sum to within f64 rounding, so
//     its distance to the CPU twin's sequential f32 sum is that sum's own
//     rounding error.
//   * The finalisation repeats blas.zig's f32 arithmetic on the f32-rounded
//     total: sum * (1/(B*S)), sum * (-1/sqrt(v+1e-5)), updates[f] += sum, ...
#include "dkz_channel.hpp"
#include "dkz_hints.hpp"

namespace dkz {
namespace {

#ifndef DKZ_CHAN_UNROLL
#define DKZ_CHAN_UNROLL 4
#endif
constexpr int kUnroll = DKZ_CHAN_UNROLL;
// Float4s in flight per lane for single-input sums. Measured on MI355X: 8 or
// 16 instead of 4 took config 1's mean from 6.0 to 7.0 us and config 2's
// backward_bias from 18.7 to 19.2 / 20.1 us, so single-input sums keep 4.
#ifndef DKZ_CHAN_UNROLL1
#define DKZ_CHAN_UNROLL1 DKZ_CHAN_UNROLL
#endif
#ifndef DKZ_CHAN_KMAJOR
#define DKZ_CHAN_KMAJOR 1
#endif
// Elements in flight per lane for channels whose spatial size is not a
// multiple of 4 (read an element at a time).
#ifndef DKZ_CHAN_SCALAR_W
#define DKZ_CHAN_SCALAR_W 8
#endif

template <class Term>
__device__ __forceinline__ double term4(const Term &t, float4 a, float4 b) {
    return ((double)t(a.x, b.x) + (double)t(a.y, b.y)) + ((double)t(a.z, b.z) + (double)t(a.w, b.w));
}

// Sum of this workgroup's chunk of channel f (all threads return it).
// T::at(f) gives the per-element term of channel f; p1 is read only when TWO.
// H: bit 0 / bit 1 = nontemporal loads of p0 / p1 (dkz_hints.hpp).
template <class T, bool TWO, bool VEC, int H, int BS>
__device__ __forceinline__ double chunk_sum(const T &t, const float *p0, const float *p1, const RedGeom &g,
                                            uint32_t f, uint32_t k, double *lds) {
    const uint32_t j0 = k * g.chunk;
    const uint32_t j1 = min(j0 + g.chunk, g.chan_len);
    const uint32_t fbase = f * g.spatial;
    const auto term = t.at(f);
    double acc0 = 0.0, acc1 = 0.0;
    if constexpr (VEC) {
        constexpr uint32_t kStep = 4 * BS;
        constexpr int kU = TWO ? kUnroll : DKZ_CHAN_UNROLL1;
        uint32_t j = j0 + 4 * threadIdx.x;
        for (; j + kStep * (kU - 1) < j1; j += kStep * kU) {
            float4 a[kU], b[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                const uint32_t v = chan_addr(fbase, j + u * kStep, g) >> 2;
                a[u] = ld4<(H & 1) != 0>(p0, v);
                if constexpr (TWO) b[u] = ld4<(H & 2) != 0>(p1, v);
                else b[u] = a[u];
            }
#pragma unroll
            for (int u = 0; u < kU; u += 2) {
                acc0 += term4(term, a[u], b[u]);
                acc1 += term4(term, a[u + 1], b[u + 1]);
            }
        }
        if constexpr (!TWO) {
            // the last (at most kU - 1) float4s, loaded together: those past
            // the chunk read the lane's next float4 again and are not added
            // ([64,512,14,14] mean 8.5 -> 7.9 us, [32,256,28,28] 8.1 -> 7.3;
            // two-input sums measured 0.5-1% slower this way and keep the
            // loop)
            if (j < j1) {
                float4 a[kU - 1];
#pragma unroll
                for (int u = 0; u < kU - 1; ++u) {
                    const uint32_t ju = j + u * kStep;
                    a[u] = ld4<(H & 1) != 0>(p0, chan_addr(fbase, ju < j1 ? ju : j, g) >> 2);
                }
#pragma unroll
                for (int u = 0; u < kU - 1; ++u)
                    if (j + u * kStep < j1) acc0 += term4(term, a[u], a[u]);
            }
        } else {
            for (; j < j1; j += kStep) {
                const uint32_t v = chan_addr(fbase, j, g) >> 2;
                acc0 += term4(term, ld4<(H & 1) != 0>(p0, v), ld4<(H & 2) != 0>(p1, v));
            }
        }
    } else {
        // An element at a time (spatial not a multiple of 4), W a lane in
        // flight: the loads past the chunk read the lane's first element
        // again and are not added, so each lane still adds its elements in
        // index order. With one load a round trip [64,1024,13,13]'s mean took
        // 22.9 us, with 4 a lane 11.5, with 8 11.0 ([64,256,19,19] 15.4 /
        // 8.4 / 7.6; 16 no better).
        constexpr int W = DKZ_CHAN_SCALAR_W;
        for (uint32_t j = j0 + threadIdx.x; j < j1; j += W * BS) {
            float a[W], b[W];
#pragma unroll
            for (int u = 0; u < W; ++u) {
                const uint32_t ju = j + u * BS;
                const uint32_t e = chan_addr(fbase, ju < j1 ? ju : j, g);
                a[u] = p0[e];
                b[u] = TWO ? p1[e] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < W; ++u)
                if (j + u * BS < j1) acc0 += (double)term(a[u], b[u]);
        }
    }
    return block_sum<BS>(acc0 + acc1, lds);
}

// K == 1: one workgroup of BS threads per channel, finalised in place.
template <class T, class Fin, bool TWO, bool VEC, int H, int BS>
__global__ __launch_bounds__(BS) void chan_reduce_kernel(T t, Fin fin, const float *p0, const float *p1, RedGeom g) {
    __shared__ double lds[BS / kWave];
    const float pre = threadIdx.x == 0 ? fin.pre(blockIdx.x) : 0.0f;
    const double total = chunk_sum<T, TWO, VEC, H, BS>(t, p0, p1, g, blockIdx.x, 0, lds);
    if (threadIdx.x == 0) fin(blockIdx.x, total, pre);
}

// K > 1, one launch: workgroup (f, k) stores its f64 partial at
// partials[f*K + k] with an agent-scope atomic store, which is written
// through to the memory side where every XCD's L2 sees it (gfx950's L2s are
// not coherent with each other for ordinary stores), waits for that store to
// complete, and then counts itself in channel f's counter with an
// agent-scope atomic add. The workgroup that brings the counter to K is the
// channel's last: it empties the counter for the next launch, reads the K
// partials with agent-scope atomic loads (which bypass its own L2) and adds
// them in index order over one wave, exactly as the two-launch finalisation
// does, then finalises. No fence: a release/acquire fence at agent scope
// writes back and invalidates the whole L2 of the XCD. Nothing waits on
// another workgroup, so any grid size is safe, and the sum's order is fixed
// by the shape alone (deterministic).
template <class T, class Fin, bool TWO, bool VEC, int H, int BS>
__global__ __launch_bounds__(BS) void chan_split_kernel(T t, Fin fin, const float *p0, const float *p1, RedGeom g,
                                                        double *partials, uint64_t *counters) {
    __shared__ double lds[BS / kWave];
    __shared__ uint32_t last_sh;
    uint32_t f, k;
    if constexpr (DKZ_CHAN_KMAJOR != 0) {
        // consecutive workgroups: the same chunk of consecutive channels, so
        // the grid sweeps the tensor in address order
        k = fdiv(blockIdx.x, g.div_filters);
        f = blockIdx.x - k * g.div_filters.d;
    } else {
        f = fdiv(blockIdx.x, g.div_k);
        k = blockIdx.x - f * g.K;
    }
    const uint32_t slot = f * g.K + k;
    const double total = chunk_sum<T, TWO, VEC, H, BS>(t, p0, p1, g, f, k, lds);
    if (threadIdx.x == 0) {
        __hip_atomic_store(&partials[(uint64_t)slot * kPartialStride], total, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        const uint64_t before = __hip_atomic_fetch_add(&counters[(uint64_t)f * kCounterStride], 1ull,
                                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_sh = before == (uint64_t)(g.K - 1) ? 1u : 0u;
    }
    __syncthreads();
    if (last_sh == 0 || threadIdx.x >= kWave) return;
    const float pre = fin.pre(f);
    const double *p = partials + (uint64_t)f * g.K * kPartialStride;
    double s = 0.0;
    for (uint32_t i = threadIdx.x; i < g.K; i += kWave)
        s += __hip_atomic_load(&p[(uint64_t)i * kPartialStride], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s = wave_sum(s);
    if (threadIdx.x == 0) {
        __hip_atomic_store(&counters[(uint64_t)f * kCounterStride], 0ull, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        fin(f, s, pre);
    }
}

// Two workgroups per channel, one launch, for 128..255 channels of at least
// 32 Ki elements and at most DKZ_PAIR_MAX_BYTES (250 MB) to read: 1024-thread
// workgroups, every CU streaming, and the two halves meet in channel f's
// counter slot (zero when empty): each swaps its partial in with one
// agent-scope atomic exchange, which returns what the slot held. The one
// that gets the other's partial back adds the two (f64 addition is
// commutative, so the sum does not depend on which finished first), empties
// the slot and finalises. One memory round trip at the end instead of the
// split kernel's three (store and wait, count, read the partials). Config
// 2, cold: backward_bias / mean_delta 19.9 -> 18.5 us, backward_scale /
// variance_delta 34.4 / 33.8 -> 33.5 / 32.5 us, the backward chain 6584 ->
// 6680 GB/s. A partial travels as its bits XOR kMeetKey (dkz_channel.hpp),
// so a stored partial is never zero.
#ifndef DKZ_CHAN_PAIR
#define DKZ_CHAN_PAIR 1
#endif
#ifndef DKZ_PAIR_MAX_BYTES
#define DKZ_PAIR_MAX_BYTES 250000000ull
#endif

template <class T, class Fin, bool TWO, bool VEC, int H, int BS>
__global__ __launch_bounds__(BS) void chan_pair_kernel(T t, Fin fin, const float *p0, const float *p1, RedGeom g,
                                                       uint64_t *slots) {
    __shared__ double lds[BS / kWave];
    const uint32_t f = blockIdx.x >> 1, k = blockIdx.x & 1;
    const float pre = threadIdx.x == 0 ? fin.pre(f) : 0.0f;
    const double s = chunk_sum<T, TWO, VEC, H, BS>(t, p0, p1, g, f, k, lds);
    if (threadIdx.x == 0) {
        uint64_t *slot = &slots[(uint64_t)f * kCounterStride];
        const uint64_t mine = __builtin_bit_cast(uint64_t, s) ^ kMeetKey;
        const uint64_t held = __hip_atomic_exchange(slot, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (held != 0) {
            __hip_atomic_store(slot, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            fin(f, s + __builtin_bit_cast(double, held ^ kMeetKey), pre);
        }
    }
}

// Workgroups per channel of a per-op reduction: about DKZ_CHAN_TARGET_WGS
// workgroups in all (four per CU), each owning at least DKZ_CHAN_MIN_CHUNK
// elements; one per channel when the channels alone are that many. From the
// shape only, so a shape always reduces in the same order. Measured on
// MI355X with chunk-major order: 2048 / 4096 workgroups gave config 2's
// backward_bias 19.0 / 25.8 us against 18.8, config 1's mean 6.4 against
// 5.9 us (every extra workgroup adds an atomic on its channel's counter).
#ifndef DKZ_CHAN_TARGET_WGS
#define DKZ_CHAN_TARGET_WGS 1024
#endif
#ifndef DKZ_CHAN_MIN_CHUNK
#define DKZ_CHAN_MIN_CHUNK 2048
#endif
// Threads a split workgroup. Measured at config 1 (mean / variance, graph
// replay, cold): 256 threads with ~1024 workgroups 5.96 / 5.98 us; 512 x 512
// 6.10 / 6.17, 512 x 256 6.23 / 6.35, 1024 x 256 6.45 / 6.40, 1024 x 512
// 6.56 / 6.68, 256 x 256 7.00 / 7.13.
#ifndef DKZ_CHAN_SPLIT_BS
#define DKZ_CHAN_SPLIT_BS 256
#endif
// K > 1 only when filters < DKZ_CHAN_TARGET_WGS, so a padded counter per
// channel always fits the scratch's slots.
static_assert((uint64_t)DKZ_CHAN_TARGET_WGS * DKZ_SPLIT_CSTRIDE <= kScratchSlots, "one counter per split channel");
inline uint32_t chan_split(uint32_t filters, uint32_t chan_len) {
    uint32_t k = div_up(DKZ_CHAN_TARGET_WGS, filters);
    const uint32_t kmax = chan_len / DKZ_CHAN_MIN_CHUNK > 1 ? chan_len / DKZ_CHAN_MIN_CHUNK : 1;
    if (k > kmax) k = kmax;
    while (k > 1 && (uint64_t)filters * k * kPartialStride > kScratchPartials) --k;
    return k < 1 ? 1 : k;
}

template <int H, class T, class Fin, bool TWO>
int run_chan_reduce(const char *name, const T &t, const Fin &fin, const float *p0, const float *p1,
                    int batch, int filters, int spatial) {
    const uint64_t chan_len64 = (uint64_t)batch * (uint64_t)spatial;
    DKZ_REQUIRE(chan_len64 * (uint64_t)filters <= kMaxElems);
    const uint32_t F = (uint32_t)filters, S = (uint32_t)spatial, L = (uint32_t)chan_len64;
    const bool vec = S % 4 == 0 && aligned16(p0) && (!TWO || aligned16(p1));
    const uint64_t bytes = (uint64_t)4 * (TWO ? 2 : 1) * F * L;
    if (DKZ_CHAN_PAIR && F >= 128 && F < 256 && L >= 32 * kWideBlock && bytes <= DKZ_PAIR_MAX_BYTES) {
        const RedGeom g2 = make_red_geom(F, S, L, 2, vec);
        if (g2.K == 2) {
            Scratch sc{nullptr};
            DKZ_TRY(device_scratch(&sc));
            const dim3 block(kWideBlock);
            if (vec)
                return launch(name, chan_pair_kernel<T, Fin, TWO, true, H, kWideBlock>, dim3(2 * F), block, t, fin,
                              p0, p1, g2, sc.slots);
            return launch(name, chan_pair_kernel<T, Fin, TWO, false, H, kWideBlock>, dim3(2 * F), block, t, fin, p0,
                          p1, g2, sc.slots);
        }
    }
    const RedGeom g = make_red_geom(F, S, L, chan_split(F, L), vec);
    const uint32_t K = g.K;
    if (K == 1) {
        if (L >= 16 * kWideBlock) {
            const dim3 block(kWideBlock);
            if (vec) return launch(name, chan_reduce_kernel<T, Fin, TWO, true, H, kWideBlock>, dim3(F), block, t, fin, p0, p1, g);
            return launch(name, chan_reduce_kernel<T, Fin, TWO, false, H, kWideBlock>, dim3(F), block, t, fin, p0, p1, g);
        }
        const dim3 block(kBlock);
        if (vec) return launch(name, chan_reduce_kernel<T, Fin, TWO, true, H, kBlock>, dim3(F), block, t, fin, p0, p1, g);
        return launch(name, chan_reduce_kernel<T, Fin, TWO, false, H, kBlock>, dim3(F), block, t, fin, p0, p1, g);
    }
    constexpr int BS = DKZ_CHAN_SPLIT_BS;
    const dim3 block(BS);
    Scratch sc{nullptr};
    DKZ_TRY(device_scratch(&sc));
    if (vec)
        return launch(name, chan_split_kernel<T, Fin, TWO, true, H, BS>, dim3(F * K), block, t, fin, p0, p1, g,
                      sc.partials, sc.slots);
    return launch(name, chan_split_kernel<T, Fin, TWO, false, H, BS>, dim3(F * K), block, t, fin, p0, p1, g,
                  sc.partials, sc.slots);
}

// ---- per-element terms (f32, rounded as the CPU twin rounds them) ---------

struct Value {  // sum += v (blas.zig:78, 112, 153)
    __device__ float operator()(float v, float) const { return v; }
};
struct SumValue {
    __device__ Value at(uint32_t) const { return {}; }
};

struct SqDev {  // d = v - m; sum += d*d (blas.zig:128-131)
    float m;
    __device__ float operator()(float v, float) const {
        const float d = v - m;
        return d * d;
    }
};
struct SumSqDev {
    const float *mean;
    __device__ SqDev at(uint32_t f) const { return {mean[f]}; }
};

struct Prod {  // sum += dv * xv (blas.zig:96), p0 = delta, p1 = x_norm
    __device__ float operator()(float d, float x) const { return d * x; }
};
struct SumProd {
    __device__ Prod at(uint32_t) const { return {}; }
};

struct ProdDev {  // sum += dv * (xv - m) (blas.zig:174), p0 = delta, p1 = x
    float m;
    __device__ float operator()(float d, float x) const { return d * (x - m); }
};
struct SumProdDev {
    const float *mean;
    __device__ ProdDev at(uint32_t f) const { return {mean[f]}; }
};

// ---- finalisations ----------------------------------------------------------

// Each finaliser reads what it needs of channel f besides the sum (pre) before
// the sum is formed, so that load overlaps the partial sums' loads.
struct FinScale {  // out[f] = sum * scale_f (blas.zig:114, 133)
    float *out;
    float scale;
    __device__ float pre(uint32_t) const { return 0.0f; }
    __device__ void operator()(uint32_t f, double s, float) const { out[f] = (float)s * scale; }
};
struct FinMeanDelta {  // blas.zig:155
    float *out;
    const float *variance;
    __device__ float pre(uint32_t f) const { return variance[f]; }
    __device__ void operator()(uint32_t f, double s, float v) const {
        out[f] = (float)s * (-1.0f / sqrtf(v + 1e-5f));
    }
};
struct FinVarianceDelta {  // blas.zig:176: (sum * -0.5) * pow(v + 1e-5, -1.5)
    float *out;
    const float *variance;
    __device__ float pre(uint32_t f) const { return variance[f]; }
    __device__ void operator()(uint32_t f, double s, float v) const {
        out[f] = ((float)s * -0.5f) * pow_m1p5(v + 1e-5f);
    }
};
struct FinAccumulate {  // updates[f] += sum (blas.zig:79, 98)
    float *updates;
    __device__ float pre(uint32_t f) const { return updates[f]; }
    __device__ void operator()(uint32_t f, double s, float u) const { updates[f] = u + (float)s; }
};

// backward_bias with spatial == 1 (gpu.zig:540-543, a connected layer's
// [batch, filters] delta): the twin adds the batch's rows into the update one
// after another in f32 (blas.zig:73-82). Here a workgroup of kConnWaves
// waves owns 64 consecutive filters (a wave's lanes read 256 contiguous
// bytes of a row); wave w adds rows w, w + kConnWaves, ... in f64, eight
// rows' loads in flight, and the first wave adds the waves' sums in wave
// order and rounds u + sum once. Deterministic, and the correctly rounded
// f32 of the update's exact value to within f64 rounding, so at least as
// close to it as the twin's sequential sum.
constexpr uint32_t kConnWaves = 16;
__global__ __launch_bounds__(kConnWaves * kWave) void backward_bias_conn_kernel(float *updates, const float *delta,
                                                                               uint32_t batch, uint32_t filters) {
    constexpr uint32_t kRows = 8;
    __shared__ double part[kConnWaves][kWave];
    const uint32_t l = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    const uint32_t f = blockIdx.x * kWave + l;
    const bool live = f < filters;
    // Lanes past the last filter read the last filter's column and drop it,
    // so every load is unconditional and a lane's eight stay in flight
    // together (a conditional load would be waited on before the next).
    const uint32_t fc = live ? f : filters - 1;
    double acc = 0.0;
    uint32_t b = w;
    for (; b + (kRows - 1) * kConnWaves < batch; b += kRows * kConnWaves) {
        float v[kRows];
#pragma unroll
        for (uint32_t k = 0; k < kRows; ++k) v[k] = delta[(b + k * kConnWaves) * filters + fc];
#pragma unroll
        for (uint32_t k = 0; k < kRows; ++k) acc += (double)v[k];
    }
    for (; b < batch; b += kConnWaves) acc += (double)delta[b * filters + fc];
    part[w][l] = live ? acc : 0.0;
    __syncthreads();
    if (w == 0 && live) {
        double s = part[0][l];
#pragma unroll
        for (uint32_t i = 1; i < kConnWaves; ++i) s += part[i][l];
        updates[f] = (float)((double)updates[f] + s);
    }
}

// ---- global average pooling forward: one wave per row ----------------------

template <bool VEC>
__global__ __launch_bounds__(kBlock) void avgpool_rows_kernel(const float *x, float *out, uint32_t rows,
                                                              uint32_t S, float denom) {
    const uint32_t row = blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
    if (row >= rows) return;  // whole waves leave together
    const uint32_t l = threadIdx.x & (kWave - 1);
    double acc = 0.0;
    if constexpr (VEC) {
        const uint32_t S4 = S >> 2;
        const uint32_t v0 = row * S4;
        // Four float4s a lane in flight, those past the row masked: they add
        // +0.0, which leaves the sum as it is (it starts at +0.0), so every
        // lane still adds its float4s in index order. A loop whose bound
        // left out the lanes without four whole float4s (at 784 elements a
        // row, 60 of 64) made them read theirs one round trip at a time:
        // config 5 72.4 -> 59.5 us.
        const float4 zero = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (uint32_t i = l; i < S4; i += 4 * kWave) {
            float4 a[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t iu = i + u * kWave;
                a[u] = iu < S4 ? ld4<(DKZ_HINT_AVGPOOL_FWD & 1) != 0>(x, v0 + iu) : zero;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) acc += term4(Value{}, a[u], a[u]);
        }
    } else {
        // the same, an element at a time: four loads a lane in flight, the
        // masked ones adding +0.0, each lane's elements in index order
        const uint32_t e0 = row * S;
        for (uint32_t i = l; i < S; i += 4 * kWave) {
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t iu = i + u * kWave;
                v[u] = iu < S ? x[e0 + iu] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) acc += (double)v[u];
        }
    }
    acc = wave_sum(acc);
    if (l == 0) out[row] = (float)acc / denom;  // pooling.zig:155: sum / denom
}

// Rows of at most 4L elements (L = 4 .. 32): L lanes a row, 64 / L rows a
// wave, each lane adding elements l, l + L, l + 2L, l + 3L of its row in
// f64 (all four loads in flight, the ones past the row masked, adding
// +0.0), then a butterfly over the row's L lanes; rounded once and divided
// as avgpool_rows_kernel does. With a wave a row, a 7x7 plane left 15 of 64
// lanes idle and paid a whole wave's reduction per 49 elements.
template <int L>
__global__ __launch_bounds__(kBlock) void avgpool_seg_kernel(const float *x, float *out, uint32_t rows, uint32_t S,
                                                             float denom) {
    const uint32_t lane = threadIdx.x & (kWave - 1), l = lane % L;
    const uint32_t row = (blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave) * (kWave / L) + lane / L;
    double acc = 0.0;
    if (row < rows) {
        const uint32_t e0 = row * S;
        for (uint32_t i = l; i < S; i += 4 * L) {
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t iu = i + u * L;
                v[u] = iu < S ? x[e0 + iu] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) acc += (double)v[u];
        }
    }
    acc = seg_sum<L>(acc);  // the whole wave: rows past the end add zeros
    if (row < rows && l == 0) out[row] = (float)acc / denom;
}

}  // namespace
}  // namespace dkz

using namespace dkz;

#define DKZ_REQUIRE_SHAPE(b, f, s) DKZ_REQUIRE((b) >= 0 && (f) >= 0 && (s) >= 0)

extern "C" {

int dkz_mean(const float *x, int batch, int filters, int spatial, float *out) {
    DKZ_REQUIRE_SHAPE(batch, filters, spatial);
    if (filters == 0) return 0;
    DKZ_REQUIRE(out && (x || (uint64_t)batch * spatial == 0));
    const float scale = 1.0f / (float)((uint64_t)batch * (uint64_t)spatial);  // blas.zig:107
    return run_chan_reduce<DKZ_HINT_MEAN, SumValue, FinScale, false>("mean", SumValue{}, FinScale{out, scale}, x, nullptr,
                                                      batch, filters, spatial);
}

int dkz_variance(const float *x, const float *mean, int batch, int filters, int spatial, float *out) {
    DKZ_REQUIRE_SHAPE(batch, filters, spatial);
    if (filters == 0) return 0;
    DKZ_REQUIRE(out && mean && (x || (uint64_t)batch * spatial == 0));
    // blas.zig:122, usize arithmetic: batch*spatial - 1 wraps when the product is 0.
    const float scale = 1.0f / (float)((uint64_t)batch * (uint64_t)spatial - 1u);
    return run_chan_reduce<DKZ_HINT_VARIANCE, SumSqDev, FinScale, false>("variance", SumSqDev{mean}, FinScale{out, scale}, x,
                                                      nullptr, batch, filters, spatial);
}

int dkz_mean_delta(const float *delta, const float *variance, int batch, int filters, int spatial,
                   float *out) {
    DKZ_REQUIRE_SHAPE(batch, filters, spatial);
    if (filters == 0) return 0;
    DKZ_REQUIRE(out && variance && (delta || (uint64_t)batch * spatial == 0));
    const FinMeanDelta fin{out, variance};
    if (recently_written(delta, 4ull * (uint64_t)batch * (uint64_t)filters * (uint64_t)spatial))
        return run_chan_reduce<DKZ_HINT_MEAN_DELTA, SumValue, FinMeanDelta, false>("mean_delta", SumValue{}, fin,
                                                                                   delta, nullptr, batch, filters,
                                                                                   spatial);
    return run_chan_reduce<DKZ_HINT_MEAN_DELTA_COLD, SumValue, FinMeanDelta, false>("mean_delta", SumValue{}, fin,
                                                                                    delta, nullptr, batch, filters,
                                                                                    spatial);
}

int dkz_variance_delta(const float *x, const float *delta, const float *mean, const float *variance,
                       int batch, int filters, int spatial, float *out) {
    DKZ_REQUIRE_SHAPE(batch, filters, spatial);
    if (filters == 0) return 0;
    DKZ_REQUIRE(out && mean && variance && ((x && delta) || (uint64_t)batch * spatial == 0));
    return run_chan_reduce<DKZ_HINT_VARIANCE_DELTA, SumProdDev, FinVarianceDelta, true>("variance_delta", SumProdDev{mean},
                                                               FinVarianceDelta{out, variance}, delta, x,
                                                               batch, filters, spatial);
}

int dkz_backward_bias(float *bias_updates, const float *delta, int batch, int filters, int spatial) {
    DKZ_REQUIRE_SHAPE(batch, filters, spatial);
    // blas.zig:73-82 adds one row sum per batch item: nothing at all when batch == 0.
    if (filters == 0 || batch == 0) return 0;
    DKZ_REQUIRE(bias_updates && (delta || spatial == 0));
    if (spatial == 1) {
        DKZ_REQUIRE((uint64_t)batch * (uint64_t)filters <= kMaxElems);
        return launch("backward_bias_conn", backward_bias_conn_kernel, dim3(div_up((uint32_t)filters, kWave)),
                      dim3(kConnWaves * kWave), bias_updates, delta, (uint32_t)batch, (uint32_t)filters);
    }
    const FinAccumulate fin{bias_updates};
    if (recently_written(delta, 4ull * (uint64_t)batch * (uint64_t)filters * (uint64_t)spatial))
        return run_chan_reduce<DKZ_HINT_BACKWARD_BIAS, SumValue, FinAccumulate, false>("backward_bias", SumValue{},
                                                                                       fin, delta, nullptr, batch,
                                                                                       filters, spatial);
    return run_chan_reduce<DKZ_HINT_BACKWARD_BIAS_COLD, SumValue, FinAccumulate, false>(
        "backward_bias", SumValue{}, fin, delta, nullptr, batch, filters, spatial);
}

int dkz_backward_scale(const float *x_norm, const float *delta, int batch, int filters, int spatial,
                       float *scale_updates) {
    DKZ_REQUIRE_SHAPE(batch, filters, spatial);
    if (filters == 0) return 0;
    DKZ_REQUIRE(scale_updates && ((x_norm && delta) || (uint64_t)batch * spatial == 0));
    return run_chan_reduce<DKZ_HINT_BACKWARD_SCALE, SumProd, FinAccumulate, true>("backward_scale", SumProd{},
                                                         FinAccumulate{scale_updates}, delta, x_norm, batch,
                                                         filters, spatial);
}

int dkz_forward_avgpool(int n, int w, int h, int c, const float *input, float *output) {
    DKZ_REQUIRE(n >= 0 && w >= 0 && h >= 0 && c >= 0);
    if (n == 0) return 0;
    const uint64_t S = (uint64_t)w * (uint64_t)h;
    DKZ_REQUIRE(S * (uint64_t)n <= kMaxElems);
    DKZ_REQUIRE(output && (input || S == 0));
    const float denom = (float)S;  // pooling.zig:148
    const uint32_t rows = (uint32_t)n;
    if (S <= 128) {  // short rows: L lanes a row, L the least of 4, 8, 16, 32 with 4L >= S
        const uint32_t per_wg = (kBlock / kWave) * (kWave / (S <= 16 ? 4 : S <= 32 ? 8 : S <= 64 ? 16 : 32));
        const dim3 g(div_up(rows, per_wg)), b(kBlock);
        const uint32_t s = (uint32_t)S;
        if (S <= 16) return launch("forward_avgpool", avgpool_seg_kernel<4>, g, b, input, output, rows, s, denom);
        if (S <= 32) return launch("forward_avgpool", avgpool_seg_kernel<8>, g, b, input, output, rows, s, denom);
        if (S <= 64) return launch("forward_avgpool", avgpool_seg_kernel<16>, g, b, input, output, rows, s, denom);
        return launch("forward_avgpool", avgpool_seg_kernel<32>, g, b, input, output, rows, s, denom);
    }
    const dim3 grid(div_up(rows, kBlock / kWave)), block(kBlock);
    if (S % 4 == 0 && aligned16(input))
        return launch("forward_avgpool", avgpool_rows_kernel<true>, grid, block, input, output, rows,
                      (uint32_t)S, denom);
    return launch("forward_avgpool", avgpool_rows_kernel<false>, grid, block, input, output, rows, (uint32_t)S,
                  denom);
}

}  // extern "C"
