// batchnorm.hip -- the batch-norm layer step as fused passes over the tensor.
//
// The reference issues the layer as a sequence of per-op launches, each
// streaming the whole tensor (layers/batchnorm.zig:129-174, plus the
// activation of convolutional.zig:269 and its gradient at :280):
//   forward (train):  copy->x, mean, variance, 4 x EMA, normalize,
//                     copy->x_norm, scale_bias, add_bias, activate
//                     = 56 bytes/element with the copies;
//   backward:         gradient, backward_bias, backward_scale, scale_bias,
//                     mean_delta, variance_delta, normalize_delta
//                     = 56 bytes/element.
// Here each direction is, in general, one reduction pass, a tiny
// per-channel finalise, and one apply pass:
//   forward:  stats (read input: 4 B/elem) -> finalise (mean, variance, EMA)
//             -> apply (read input; write x, x_norm, output: 16 B/elem);
//   backward: sums (read y, delta, x_norm, x: 16 B/elem) -> finalise
//             (bias/scale updates, mean_delta, variance_delta) -> apply
//             (read y, delta, x; write delta: 16 B/elem).
// When every workgroup of the grid fits the GPU at once, each direction is
// one launch instead (bn_fwd_coop_kernel, bn_bwd_coop_kernel,
// bn_bwd_reg_kernel): a workgroup keeps its chunk (or, for the largest
// tensors, part of it) in registers and LDS, the channel's workgroups meet
// at a barrier, and the apply step runs on what they hold: 16 B/elem
// forward, 20 backward (plus 12 for any part read again).
// Element results are the per-op sequence's, bit for bit, given the same
// per-channel values: every element expression below is the one of the
// corresponding op (broadcast.hip, elementwise.hip), in the same order.
//
// Forward statistics. The per-op path makes two passes (mean, then the sum
// of squared deviations from it). The fused pass reads the input once and
// accumulates, in f64, s1 = sum(x - c) and s2 = sum((x - c)^2) about a
// per-channel shift c = the channel's first element (x - c is exact in f64).
// Then sum(x) = n*c + s1, and the sum of squared deviations from any f32
// mean m is s2 - s1^2/n + n*(c + s1/n - m)^2. Shifting by a sample of the
// channel keeps the cancellation in s2 - s1^2/n to the factor
// 1 + ((c - mean)/stddev)^2, so the result stays within a few f64 ulps of the
// exact sum unless c is an outlier by ~10^4 standard deviations. The twin
// (blas.zig:121-135) sums f32-rounded (x - m)^2 terms sequentially in f32, so
// the two agree to within the twin's own rounding error.
//
// The fast path needs spatial % 4 == 0, 16-byte aligned tensors and a
// non-empty tensor; any other call runs the per-op sequence, which handles
// every shape (and edge case) exactly as the individual entry points do.
#include <atomic>
#include <cstdlib>
#include <type_traits>

#include "dkz_channel.hpp"
#include "dkz_hints.hpp"

namespace dkz {
namespace {

constexpr int kUnroll = 4;
constexpr float kMomentum = 0.99f;          // rolling_momentum, batchnorm.zig:16 (f32)
constexpr float kAlpha = 1.0f - kMomentum;  // batchnorm.zig:141: an f32 subtraction, exact

template <int NS>
struct Sums {
    double s[NS];
};

// f(std::integral_constant<int, I>) for I = B, B + S, ... < E: a loop whose
// index is a compile-time constant in each step (so arrays indexed by it
// stay in registers, however long the body).
template <int B, int E, int S, class F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + S, E, S>(f);
    }
}

// Workgroup of a reduction pass: chunk k of channel f. KMAJOR: consecutive
// workgroups take the same chunk of consecutive channels, so the grid
// sweeps the tensor roughly in address order; otherwise consecutive chunks
// of one channel.
// Launch shape of the reduction passes, measured on MI355X (config 2
// backward, config 1 forward):
//  * the backward sums grid is chunk-major (workgroup i takes chunk i / F of
//    channel i % F): 138 us against 147 us channel-major; the forward
//    statistics grid is channel-major: 23.6 us against 25.2 us;
//  * about 8192 workgroups of >= 4096 elements (partials permitting): 138 us
//    against 142 us with 2048 (a smoother tail);
//  * two float4s of each of the four streams in flight per lane (1 or 4:
//    no difference).
#ifndef DKZ_BN_KMAJOR
#define DKZ_BN_KMAJOR 1
#endif
#ifndef DKZ_BN_STATS_KMAJOR
#define DKZ_BN_STATS_KMAJOR 0
#endif
#ifndef DKZ_BN_SUMS_UNROLL
#define DKZ_BN_SUMS_UNROLL 2
#endif
#ifndef DKZ_BN_SPLIT_TARGET
#define DKZ_BN_SPLIT_TARGET 8192
#endif
#ifndef DKZ_BN_MIN_CHUNK
#define DKZ_BN_MIN_CHUNK 4096
#endif
template <bool KMAJOR>
__device__ __forceinline__ void red_coords(const RedGeom &g, uint32_t &f, uint32_t &k) {
    if constexpr (KMAJOR) {
        k = fdiv(blockIdx.x, g.div_filters);
        f = blockIdx.x - k * g.div_filters.d;
    } else {
        f = fdiv(blockIdx.x, g.div_k);
        k = blockIdx.x - f * g.K;
    }
}

// NS sums over a BS-thread workgroup; the result is valid in wave 0. Each
// wave's sums go through LDS (lds holds NS * BS/64 doubles) and wave 0 adds
// them with one more DPP reduction, so the order is fixed by the shape.
template <int NS, int BS>
__device__ __forceinline__ Sums<NS> block_sums(const double (&a)[NS], double *lds) {
    constexpr int W = BS / kWave;
    const int w = threadIdx.x / kWave, l = threadIdx.x & (kWave - 1);
    Sums<NS> r;
#pragma unroll
    for (int q = 0; q < NS; ++q) {
        const double v = wave_sum(a[q]);
        if (l == 0) lds[q * W + w] = v;
    }
    __syncthreads();
    if (w == 0) {
#pragma unroll
        for (int q = 0; q < NS; ++q) r.s[q] = wave_sum(l < W ? lds[q * W + l] : 0.0);
    }
    return r;
}

// Partial sums of workgroup (f, k) go to partials[(q*F + f)*K + k].
template <int NS, int BS>
__device__ __forceinline__ void store_partials(const Sums<NS> &r, const RedGeom &g, uint32_t f, uint32_t k,
                                               double *partials) {
    if (threadIdx.x == 0) {
        const uint32_t F = g.div_filters.d;
#pragma unroll
        for (int q = 0; q < NS; ++q) partials[((uint32_t)q * F + f) * g.K + k] = r.s[q];
    }
}

// Second launch: one wave per channel adds its K partials of each sum in
// index order, then finalises.
template <int NS, class Fin>
__global__ __launch_bounds__(kBlock) void bn_finalize_kernel(Fin fin, const double *partials, uint32_t F,
                                                             uint32_t K) {
    const uint32_t f = blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
    if (f >= F) return;  // whole waves leave together
    const uint32_t l = threadIdx.x & (kWave - 1);
    Sums<NS> r;
#pragma unroll
    for (int q = 0; q < NS; ++q) {
        const double *p = partials + ((uint64_t)q * F + f) * K;
        double s = 0.0;
        for (uint32_t i = l; i < K; i += kWave) s += p[i];
        r.s[q] = wave_sum(s);
    }
    if (l == 0) fin(f, r);
}

// ---- forward ----------------------------------------------------------------

// mean, variance and the rolling averages of channel f from s1 = sum(x - c),
// s2 = sum((x - c)^2) over its n elements, c = the channel's first element.
// The split statistics pass stores c beside the partials (shift[f]): the
// apply pass may overwrite the input in place before every workgroup has
// finalised.
struct FwdFin {
    const double *shift;
    float *mean, *variance, *rolling_mean, *rolling_variance;
    double n;
    float mean_scale;  // 1/(B*S) in f32 (blas.zig:107)
    float var_scale;   // 1/(B*S - 1) in f32 (blas.zig:122)
    __device__ void stats(const Sums<2> &r, double c, float &m, float &v) const {
        const double s1 = r.s[0], s2 = r.s[1];
        m = (float)(n * c + s1) * mean_scale;  // blas.zig:114: sum * (1/(B*S))
        const double dm = (c + s1 / n) - (double)m;
        double m2 = s2 - s1 * (s1 / n);
        m2 = m2 > 0.0 ? m2 : 0.0;
        v = (float)(m2 + n * dm * dm) * var_scale;  // blas.zig:133
    }
    // met == false (a one-launch pass whose channel barrier gave up): the
    // batch statistics are written (NaN) but the rolling averages, which
    // carry over to the next call, are left as they were.
    __device__ void write(uint32_t f, float m, float v, bool met = true) const {
        mean[f] = m;
        variance[f] = v;
        if (!met) return;
        // batchnorm.zig:140-143: scal(0.99) then axpy(1 - 0.99) -- axpy is an fma (blas.zig:22)
        rolling_mean[f] = __builtin_fmaf(kAlpha, m, rolling_mean[f] * kMomentum);
        rolling_variance[f] = __builtin_fmaf(kAlpha, v, rolling_variance[f] * kMomentum);
    }
    __device__ void operator()(uint32_t f, const Sums<2> &r) const {  // after a split pass
        float m, v;
        stats(r, shift[f], m, v);
        write(f, m, v);
    }
};

__device__ __forceinline__ void acc_shifted(float4 v, double c, double &a1, double &a2) {
    const double d0 = (double)v.x - c, d1 = (double)v.y - c, d2 = (double)v.z - c, d3 = (double)v.w - c;
    a1 += (d0 + d1) + (d2 + d3);
    a2 += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
}

// FIN: the channel is one workgroup (K == 1), which finalises it itself.
template <int H, int BS, bool FIN>
__global__ __launch_bounds__(BS) void bn_stats_kernel(const float *input, RedGeom g, FwdFin fin, double *partials) {
    __shared__ double lds[2 * (BS / kWave)];
    uint32_t f, k;
    red_coords<DKZ_BN_STATS_KMAJOR != 0>(g, f, k);
    const uint32_t j0 = k * g.chunk;
    const uint32_t j1 = min(j0 + g.chunk, g.chan_len);
    const uint32_t fbase = f * g.spatial;
    const double c = (double)input[fbase];
    double a[2] = {0.0, 0.0}, b[2] = {0.0, 0.0};
    constexpr uint32_t kStep = 4 * BS;
    uint32_t j = j0 + 4 * threadIdx.x;
    for (; j + kStep * (kUnroll - 1) < j1; j += kStep * kUnroll) {
        float4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) v[u] = ld4<(H & 1) != 0>(input, chan_addr(fbase, j + u * kStep, g) >> 2);
#pragma unroll
        for (int u = 0; u < kUnroll; u += 2) {
            acc_shifted(v[u], c, a[0], a[1]);
            acc_shifted(v[u + 1], c, b[0], b[1]);
        }
    }
    for (; j < j1; j += kStep) acc_shifted(ld4<(H & 1) != 0>(input, chan_addr(fbase, j, g) >> 2), c, a[0], a[1]);
    const double t[2] = {a[0] + b[0], a[1] + b[1]};
    const Sums<2> r = block_sums<2, BS>(t, lds);
    if constexpr (FIN) {
        if (threadIdx.x == 0) {
            float m, v;
            fin.stats(r, c, m, v);
            fin.write(f, m, v);
        }
    } else {
        store_partials<2, BS>(r, g, f, k, partials);
        if (k == 0 && threadIdx.x == 0) partials[2u * g.div_filters.d * g.K + f] = c;  // = fin.shift[f]
    }
}

struct FwdParams {
    const float *mean, *variance, *scales, *biases;
};

// What the forward apply pass needs of channel f.
struct FwdChan {
    float m, inv, gam, bet;
};

__device__ __forceinline__ FwdChan fwd_chan(float m, float v, float gam, float bet) {
    return {m, 1.0f / (sqrtf(v) + 1e-6f), gam, bet};  // blas.zig:141-143
}

// x_norm = (input - m) * inv (blas.zig:137-146); output = act(x_norm * scale
// + bias) (blas.zig:63-71, 53-61; activations.zig:107-125).
template <int A>
__device__ __forceinline__ void fwd_elem(float4 v, const FwdChan &c, float4 &xn, float4 &o) {
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        const float t = (lane(v, l) - c.m) * c.inv;
        lane(xn, l) = t;
        lane(o, l) = activate<A>(t * c.gam + c.bet);
    }
}

// Whether the apply pass finalises its own channels (saves the finalize
// launch: config 1 forward 23.6 -> 20.9 us, config 2 backward 140.7 ->
// 139.1 us) when the split reduction leaves partials.
#ifndef DKZ_BN_DEFER_FWD
#define DKZ_BN_DEFER_FWD 1
#endif
#ifndef DKZ_BN_DEFER_BWD
#define DKZ_BN_DEFER_BWD 1
#endif
// ... while a channel has at most this many partials: every apply workgroup
// adds its channels' K partials itself, so with few channels split many
// ways that is K loads per workgroup and the separate finalize launch is
// cheaper. Measured (two passes, graph replay, backward / forward):
// [2,1,60M] 1815 / 1233 us deferred (K 8192), 769 / 513 not; [4,3,12M]
// 1253 / 675 against 788 / 552; [16,64,43264] (K 128) 231 against 220.
#ifndef DKZ_BN_DEFER_MAX_K
#define DKZ_BN_DEFER_MAX_K 16
#endif
// Elements of one apply workgroup, and how many channel rows it may span
// and still finalise its channels itself.
#ifndef DKZ_BN_APPLY_UNROLL
#define DKZ_BN_APPLY_UNROLL 4  // 2 or 8 float4s per stream per lane: slower (config 2: +1 / +7 us)
#endif
constexpr int kApplyUnroll = DKZ_BN_APPLY_UNROLL;
constexpr uint32_t kTile = kBlock * kApplyUnroll * 4;
constexpr uint32_t kSlots = 16;

// The rows [r0, r0 + nrows) of this workgroup's tile of n elements.
__device__ __forceinline__ void tile_rows(const ChanGeom &g, uint32_t n, uint32_t &e0, uint32_t &r0,
                                          uint32_t &nrows) {
    e0 = blockIdx.x * kTile;
    const uint32_t e1 = min(e0 + kTile, n) - 1;
    r0 = fdiv(e0, g.spatial);
    nrows = fdiv(e1, g.spatial) - r0 + 1;
}

// Adds channel f's K partials of each of NS sums, in index order, over one
// wave (all lanes return the sums). The same code as bn_finalize_kernel,
// so every workgroup that does this gets the same bits.
template <int NS>
__device__ __forceinline__ Sums<NS> wave_partials(const double *partials, uint32_t F, uint32_t K, uint32_t f) {
    const uint32_t l = threadIdx.x & (kWave - 1);
    Sums<NS> r;
#pragma unroll
    for (int q = 0; q < NS; ++q) {
        const double *p = partials + ((uint64_t)q * F + f) * K;
        double s = 0.0;
        for (uint32_t i = l; i < K; i += kWave) s += p[i];
        r.s[q] = wave_sum(s);
    }
    return r;
}

// Forward apply: x = input, x_norm (TRAIN), output.
// FIN: the statistics are still K partials per channel; the workgroup adds
// them for the (at most kSlots) rows of its tile itself, and the workgroup
// whose tile holds a channel's first element writes that channel's mean,
// variance and rolling averages, exactly once. Otherwise they are read
// from p (normalised with the batch statistics, or with the rolling ones
// when !TRAIN).
// H: bit 0 = input load, bit 1 = x store, bit 2 = x_norm store, bit 3 = output store.
template <int A, bool TRAIN, int H, bool FIN>
__global__ __launch_bounds__(kBlock) void bn_fwd_apply_kernel(const float *input, float *output, float *x,
                                                              float *x_norm, FwdParams p, ChanGeom g, uint32_t n,
                                                              FwdFin fin, const double *partials, uint32_t K) {
    constexpr bool kNtIn = (H & 1) != 0, kNtX = (H & 2) != 0, kNtXn = (H & 4) != 0, kNtOut = (H & 8) != 0;
    __shared__ FwdChan slot[kSlots];
    const uint32_t nv = n >> 2;
    const uint32_t base = blockIdx.x * (kBlock * kApplyUnroll) + threadIdx.x;
    const bool full = base + (kApplyUnroll - 1) * kBlock < nv;
    float4 v[kApplyUnroll];
#pragma unroll
    for (int u = 0; u < kApplyUnroll; ++u) {
        const uint32_t i = base + u * kBlock;
        if (full || i < nv) v[u] = ld4<kNtIn>(input, i);
    }
    uint32_t r0 = 0;
    if constexpr (FIN) {
        uint32_t e0, nrows;
        tile_rows(g, n, e0, r0, nrows);
        for (uint32_t s = threadIdx.x / kWave; s < nrows; s += kBlock / kWave) {
            const uint32_t r = r0 + s;
            const uint32_t f = r - fdiv(r, g.filters) * g.filters.d;
            const Sums<2> sums = wave_partials<2>(partials, g.filters.d, K, f);
            if ((threadIdx.x & (kWave - 1)) == 0) {
                float m, var;
                fin.stats(sums, fin.shift[f], m, var);
                slot[s] = fwd_chan(m, var, p.scales[f], p.biases[f]);
                // row r == f is channel f's first row (b = 0); several slots
                // may hold one channel when the tile spans more than F rows
                if (r == f && f * g.spatial.d >= e0) fin.write(f, m, var);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < kApplyUnroll; ++u) {
        const uint32_t i = base + u * kBlock;
        if (!(full || i < nv)) continue;
        const uint32_t r = fdiv(i << 2, g.spatial);
        FwdChan c;
        if constexpr (FIN) {
            c = slot[r - r0];
        } else {
            const uint32_t f = r - fdiv(r, g.filters) * g.filters.d;
            c = fwd_chan(p.mean[f], p.variance[f], p.scales[f], p.biases[f]);
        }
        float4 xn, o;
        fwd_elem<A>(v[u], c, xn, o);
        st4<kNtX>(x, i, v[u]);
        if constexpr (TRAIN) st4<kNtXn>(x_norm, i, xn);
        st4<kNtOut>(output, i, o);
    }
}

// ---- one-launch forward --------------------------------------------------------

// The K workgroups of one channel meet here: each posts its NS partial sums
// and waits until all K have posted, then adds them (channel_meet, called
// by wave 0 of the workgroup; the caller's __syncthreads follow).
//   * Workgroup k's sums go to its own posting line (line f*K + k after the
//     F channel counters; kMeetLine, kMeetKey: dkz_channel.hpp).
//   * Wave 0 then reads the channel's other lines with coherent loads until
//     every value is non-zero and adds the K partials of each sum in index
//     order -- lane l adds lines l, l + 64, ..., then a wave sum -- so every
//     workgroup of the channel gets the same bits. The workgroup's own line
//     is taken from its registers.
//   * The last workgroup to have read (a count in the channel's counter
//     slot) clears the K lines and the count, so the next launch starts from
//     zero.
// The last workgroup to post pays one memory round trip (its poll) after
// its sums are formed; the others see its post one round trip after it
// lands. Measured at config 1 (per-workgroup s_memrealtime stamps), the
// counter-and-generation barrier this replaces (arrive, release, observe,
// then read the partials) took 2.7 us from the last arrival to the sums.
//
// A channel's workgroups have consecutive indices and the hardware
// dispatches workgroups in index order, so the lowest channel not yet done
// always has all its workgroups resident or about to be, and completes: no
// deadlock for any grid size as long as K workgroups fit the GPU at once.
// The wait is bounded anyway (kSpinMax polls with a short sleep between
// them), so every wave ends even if that assumption failed; the meeting
// then returns false and the workgroup's results are NaN, not sums of
// partials some of which were never posted. Such a workgroup adds nothing
// to the state that outlives the call (rolling averages, bias and scale
// updates) and records its kernel in barrier_timeout, which the host turns
// into an error status (take_barrier_timeout: dkz_synchronize, or the op
// itself under sync-after-launch). It still counts itself as having read,
// and the late workgroups find every partial posted and finish the
// protocol, leaving the slots clear for the next launch.
constexpr uint32_t kSpinMax = 1u << 20;

// Slots a one-launch pass over F channels of K workgroups needs: the
// channel counters, then one posting line per workgroup.
inline uint64_t meet_slots(uint64_t F, uint64_t K) { return F * kCounterStride + F * K * kMeetLine; }

// Which one-launch pass last gave up at a channel meeting on this device
// (0: none since the host last looked). Written by the kernels with a
// vector atomic store, read and cleared by take_barrier_timeout.
__device__ uint32_t barrier_timeout;

__device__ __forceinline__ void note_timeout(uint32_t met, uint32_t which) {
    if (met == 0) __hip_atomic_store(&barrier_timeout, which, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The meeting's spin limit: kSpinMax, or $DKZ_BARRIER_SPIN_LIMIT, read at
// each launch (a test sets 0 to force time-outs and check that they turn
// into NaN results and an error status).
inline uint32_t barrier_spin_limit() {
    const char *e = getenv("DKZ_BARRIER_SPIN_LIMIT");
    return e != nullptr && *e != '\0' ? (uint32_t)strtoul(e, nullptr, 10) : kSpinMax;
}

// Called by all 64 lanes of wave 0 with this workgroup's sums in r (the
// same in every lane, as block_sums leaves them); returns with the
// channel's totals in r (NaN if the wait ran out) and whether it met. The
// workgroup must call channel_leave once it no longer needs the lines.
template <int NS>
__device__ __forceinline__ bool channel_meet(uint64_t *slots, uint32_t F, uint32_t K, uint32_t f, uint32_t k,
                                             Sums<NS> &r, uint32_t spin) {
    const uint32_t l = threadIdx.x & (kWave - 1);
    const uint64_t *const lines = slots + (uint64_t)F * kCounterStride + (uint64_t)f * K * kMeetLine;
    uint64_t own[NS];
#pragma unroll
    for (int q = 0; q < NS; ++q) own[q] = __builtin_bit_cast(uint64_t, r.s[q]) ^ kMeetKey;
    if (l < (uint32_t)NS) {
        uint64_t v = own[0];
#pragma unroll
        for (int q = 1; q < NS; ++q) v = l == (uint32_t)q ? own[q] : v;
        __hip_atomic_store(const_cast<uint64_t *>(&lines[(uint64_t)k * kMeetLine + l]), v, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    double acc[NS];
    bool met = false;
    for (uint32_t it = 0;; ++it) {
        bool have = true;
#pragma unroll
        for (int q = 0; q < NS; ++q) acc[q] = 0.0;
        for (uint32_t i = l; i < K; i += kWave) {
            // a lane's NS loads of one line are issued together
            uint64_t u[NS];
            if (i == k) {
#pragma unroll
                for (int q = 0; q < NS; ++q) u[q] = own[q];
            } else {
#pragma unroll
                for (int q = 0; q < NS; ++q)
                    u[q] = __hip_atomic_load(&lines[(uint64_t)i * kMeetLine + q], __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
            }
#pragma unroll
            for (int q = 0; q < NS; ++q) {
                have = have && u[q] != 0;
                acc[q] += __builtin_bit_cast(double, u[q] ^ kMeetKey);
            }
        }
        if (__all(have)) {
            met = true;
            break;
        }
        if (it >= spin) break;
        __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int q = 0; q < NS; ++q) r.s[q] = met ? wave_sum(acc[q]) : __builtin_nan("");
    return met;
}

// Called by all 64 lanes of wave 0 at the end of the workgroup, after
// channel_meet: counts the workgroup as done with the channel's lines; the
// last of the K clears them and the count (off the path to the outputs:
// the other waves' stores drain meanwhile).
template <int NS>
__device__ __forceinline__ void channel_leave(uint64_t *slots, uint32_t F, uint32_t K, uint32_t f) {
    const uint32_t l = threadIdx.x & (kWave - 1);
    uint64_t *const count = slots + (uint64_t)f * kCounterStride;
    uint64_t *const lines = slots + (uint64_t)F * kCounterStride + (uint64_t)f * K * kMeetLine;
    uint64_t before = 0;
    if (l == 0) before = __hip_atomic_fetch_add(count, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    before = __shfl(before, 0);
    if (before == (uint64_t)(K - 1)) {
        for (uint32_t i = l; i < K * (uint32_t)NS; i += kWave)
            __hip_atomic_store(&lines[(uint64_t)(i / NS) * kMeetLine + i % NS], 0ull, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        if (l == 0) __hip_atomic_store(count, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Workgroups of kCoopBS threads holding kCoopU float4s a lane: a workgroup
// owns at most kCoopBS * 4 * kCoopU elements of one channel. Measured at
// config 1 (graph replay, cold): 1024 x 4 (8 workgroups a channel, one a
// CU) 15.2-15.3 us; 256 x 8 16.2-16.4; 512 x 4 / 512 x 8 15.5-15.7;
// 1024 x 2 / x 3 / x 6 / x 8 15.8 / 17.7 / 16.3 / 17.6; 128 x 16 18.4;
// 256 x 4 / x 16 17.6 / 18.0. Shapes whose grid at 1024 x 4 does not fit
// the GPU at once try 256 x 8 (smaller workgroups fit more of them).
#ifndef DKZ_BN_COOP_BS
#define DKZ_BN_COOP_BS 1024
#endif
#ifndef DKZ_BN_COOP_U
#define DKZ_BN_COOP_U 4
#endif
#ifndef DKZ_BN_COOP_BS2
#define DKZ_BN_COOP_BS2 256
#endif
#ifndef DKZ_BN_COOP_U2
#define DKZ_BN_COOP_U2 8
#endif
constexpr int kCoopBS = DKZ_BN_COOP_BS, kCoopU = DKZ_BN_COOP_U;
constexpr int kCoopBS2 = DKZ_BN_COOP_BS2, kCoopU2 = DKZ_BN_COOP_U2;
// Where the one-launch forward with 1024- or 256-thread workgroups stores x
// (the input's copy): 0 as each float4 arrives, 1 after the channel meeting
// with x_norm and the output, 2 from the workgroup's other waves while its
// first wave meets the channel (the first wave's own after the meeting).
// Measured at config 1 (graph replay, cold): 13.8-13.9 / 14.0 / 13.2 us;
// the register-holding variant (config 2's shape) stores x at once: there 2
// took 70.6 to 74.4 us.
#ifndef DKZ_BN_COOP_X_STORE
#define DKZ_BN_COOP_X_STORE 2
#endif
// The register-resident variant: 512 threads (two waves a SIMD, up to 256
// registers a lane) holding 49 float4s a lane, so one workgroup a CU covers
// 100352 elements (half of a config-2 channel).
constexpr int kRegBlock = 512, kRegU = 49;
// float4s of input a lane loads at once past its held chunk
constexpr int kFwdExtraG = 4;

// Forward (train) in one launch: workgroup (f, k) -- channel-major, k
// fastest -- loads chunk k of channel f into registers once, adds its f64
// shifted sums (as bn_stats_kernel), posts them, waits at the channel
// barrier, adds the channel's K partials, forms mean, variance (and, in
// workgroup k == 0, the rolling averages) exactly as the split statistics
// path does, and writes x, x_norm and the output from the registers. The
// input is read once: 16 bytes an element instead of 20. BS threads a
// workgroup, U float4s a lane: (kCoopBS, kCoopU) for small tensors, and
// (kRegBlock, kRegU) -- one 512-thread workgroup a CU, 196 floats a lane --
// for tensors that fill the register file (config 2's 103 MB over 256 CUs).
template <int A, int H, int BS, int U, bool EXTRA = false>
__global__ __launch_bounds__(BS) void bn_fwd_coop_kernel(const float *input, float *output, float *x,
                                                         float *x_norm, FwdParams p, RedGeom g, FwdFin fin,
                                                         uint64_t *slots, uint32_t spin) {
    constexpr bool kNtIn = (H & 1) != 0, kNtX = (H & 2) != 0, kNtXn = (H & 4) != 0, kNtOut = (H & 8) != 0;
    constexpr int kXMode = U > kCoopU2 ? 0 : DKZ_BN_COOP_X_STORE;  // the register-holding variant stores x at once
    __shared__ double lds[2 * (BS / kWave)];
    __shared__ FwdChan chan_sh;
    const uint32_t f = fdiv(blockIdx.x, g.div_k);
    const uint32_t k = blockIdx.x - f * g.K;
    const uint32_t F = g.div_filters.d;
    const uint32_t j0 = k * g.chunk;
    const uint32_t j1 = min(j0 + g.chunk, g.chan_len);
    const uint32_t fbase = f * g.spatial;
    const double c = (double)input[fbase];
    // float4 u of the lane is element jb + u*4*BS of the channel. Its
    // address is recomputed in each phase from a copy of jb the compiler
    // cannot see through, so it keeps no U addresses alive across phases
    // (at U = 49 they would push the data out of registers).
    const auto phase_base = [&]() {
        uint32_t jb = j0 + 4 * threadIdx.x;
        asm volatile("" : "+v"(jb));
        return jb;
    };
    float4 v[U];
    {
        const uint32_t jb = phase_base();
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t j = jb + (uint32_t)u * (4 * BS);
            if (j < j1) v[u] = ld4<kNtIn>(input, chan_addr(fbase, j, g) >> 2);
        }
    }
    double a[2] = {0.0, 0.0};
    {
        const uint32_t jb = phase_base();
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t j = jb + (uint32_t)u * (4 * BS);
            if (j >= j1) continue;
            acc_shifted(v[u], c, a[0], a[1]);
            // x (the input copy) needs no statistics: its stores drain while
            // the channel meets
            if constexpr (kXMode == 0) st4<kNtX>(x, chan_addr(fbase, j, g) >> 2, v[u]);
        }
    }
    if constexpr (EXTRA) {
        // chunks longer than U float4s a lane (tensors larger than the GPU
        // holds at once): the rest is read here, cached, and again after
        // the barrier
        for (uint32_t u0 = U;; u0 += kFwdExtraG) {
            const uint32_t jb = phase_base();
            if (jb + u0 * (4 * BS) >= j1) break;
            float4 w[kFwdExtraG];
#pragma unroll
            for (int q = 0; q < kFwdExtraG; ++q) {
                const uint32_t j = jb + (u0 + q) * (4 * BS);
                if (j < j1) w[q] = ld4<false>(input, chan_addr(fbase, j, g) >> 2);
            }
#pragma unroll
            for (int q = 0; q < kFwdExtraG; ++q) {
                const uint32_t j = jb + (u0 + q) * (4 * BS);
                if (j >= j1) continue;
                acc_shifted(w[q], c, a[0], a[1]);
                st4<kNtX>(x, chan_addr(fbase, j, g) >> 2, w[q]);
            }
        }
    }
    Sums<2> sums = block_sums<2, BS>(a, lds);
    if constexpr (kXMode == 2) {
        // the other waves store x while wave 0 meets the channel (wave 0's
        // stores would hold its polls back: they count in the same vmcnt)
        if (threadIdx.x >= kWave) {
            const uint32_t jb = phase_base();
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t j = jb + (uint32_t)u * (4 * BS);
                if (j < j1) st4<kNtX>(x, chan_addr(fbase, j, g) >> 2, v[u]);
            }
        }
    }
    if (threadIdx.x < kWave) {
        const uint32_t met = channel_meet<2>(slots, F, g.K, f, k, sums, spin) ? 1u : 0u;
        if (threadIdx.x == 0) {
            float m, var;
            fin.stats(sums, c, m, var);
            chan_sh = fwd_chan(m, var, p.scales[f], p.biases[f]);
            if (k == 0) fin.write(f, m, var, met != 0);
            note_timeout(met, kTimeoutFwdCoop);
        }
    }
    __syncthreads();
    const FwdChan ch = chan_sh;
    const uint32_t jb = phase_base();
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t j = jb + (uint32_t)u * (4 * BS);
        if (j >= j1) continue;
        const uint32_t at = chan_addr(fbase, j, g) >> 2;
        float4 xn, o;
        fwd_elem<A>(v[u], ch, xn, o);
        if constexpr (kXMode == 1) st4<kNtX>(x, at, v[u]);
        if constexpr (kXMode == 2) {
            if (threadIdx.x < kWave) st4<kNtX>(x, at, v[u]);
        }
        st4<kNtXn>(x_norm, at, xn);
        st4<kNtOut>(output, at, o);
    }
    if constexpr (EXTRA) {
        for (uint32_t u0 = U;; u0 += kFwdExtraG) {
            const uint32_t jb2 = phase_base();
            if (jb2 + u0 * (4 * BS) >= j1) break;
            float4 w[kFwdExtraG];
#pragma unroll
            for (int q = 0; q < kFwdExtraG; ++q) {
                const uint32_t j = jb2 + (u0 + q) * (4 * BS);
                if (j < j1) w[q] = ld4<true>(input, chan_addr(fbase, j, g) >> 2);
            }
#pragma unroll
            for (int q = 0; q < kFwdExtraG; ++q) {
                const uint32_t j = jb2 + (u0 + q) * (4 * BS);
                if (j >= j1) continue;
                const uint32_t at = chan_addr(fbase, j, g) >> 2;
                float4 xn, o;
                fwd_elem<A>(w[q], ch, xn, o);
                st4<kNtXn>(x_norm, at, xn);
                st4<kNtOut>(output, at, o);
            }
        }
    }
    if (threadIdx.x < kWave) channel_leave<2>(slots, F, g.K, f);
}

// ---- backward -----------------------------------------------------------------

// Per channel: s0 = sum(d1), s1 = sum(d1 * x_norm), s2 = sum(d2),
// s3 = sum(d2 * (x - m)), where d1 = delta * gradient(y) (activations.zig:
// 127-143) and d2 = d1 * scale (the scale_bias on delta, batchnorm.zig:165).
struct BwdFin {
    const float *variance;
    float *bias_updates, *scale_updates, *mean_delta, *variance_delta;
    __device__ void values(uint32_t f, const Sums<4> &r, float &md, float &vd) const {
        const float v = variance[f];
        md = (float)r.s[2] * (-1.0f / sqrtf(v + 1e-5f));            // blas.zig:155
        vd = ((float)r.s[3] * -0.5f) * pow_m1p5(v + 1e-5f);          // blas.zig:176
    }
    // met == false (a one-launch pass whose channel barrier gave up):
    // mean_delta and variance_delta are written (NaN), but nothing is added
    // to the updates, which accumulate across calls.
    __device__ void write(uint32_t f, const Sums<4> &r, float md, float vd, bool met = true) const {
        if (met) {
            bias_updates[f] = bias_updates[f] + (float)r.s[0];   // blas.zig:79
            scale_updates[f] = scale_updates[f] + (float)r.s[1]; // blas.zig:98
        }
        mean_delta[f] = md;
        variance_delta[f] = vd;
    }
    __device__ void operator()(uint32_t f, const Sums<4> &r) const {
        float md, vd;
        values(f, r, md, vd);
        write(f, r, md, vd);
    }
};

template <int A>
__device__ __forceinline__ float grad_delta(float d, float y) {
    if constexpr (A == kLinear) return d;  // activations.zig:129: linear leaves delta alone
    else return d * gradient<A>(y);
}

template <int A>
__device__ __forceinline__ void acc_bwd(float4 y, float4 d, float4 xn, float4 x, float m, float gam,
                                        double (&a)[4]) {
    double t[4][4];
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        const float d1 = grad_delta<A>(lane(d, l), lane(y, l));
        const float d2 = d1 * gam;
        t[0][l] = (double)d1;
        t[1][l] = (double)(d1 * lane(xn, l));         // blas.zig:96
        t[2][l] = (double)d2;
        t[3][l] = (double)(d2 * (lane(x, l) - m));    // blas.zig:174
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) a[q] += (t[q][0] + t[q][1]) + (t[q][2] + t[q][3]);
}

// H: bit 0 = y, bit 1 = delta, bit 2 = x_norm, bit 3 = x loads.
template <int A, int H, int BS, bool FIN>
__global__ __launch_bounds__(BS) void bn_bwd_sums_kernel(const float *y, const float *delta, const float *x_norm,
                                                         const float *x, const float *mean, const float *scales,
                                                         RedGeom g, BwdFin fin, double *partials) {
    constexpr bool kLin = A == kLinear;
    __shared__ double lds[4 * (BS / kWave)];
    uint32_t f, k;
    red_coords<DKZ_BN_KMAJOR != 0>(g, f, k);
    const uint32_t j0 = k * g.chunk;
    const uint32_t j1 = min(j0 + g.chunk, g.chan_len);
    const uint32_t fbase = f * g.spatial;
    const float m = mean[f], gam = scales[f];
    double a[4] = {0.0, 0.0, 0.0, 0.0};
    constexpr int kU = DKZ_BN_SUMS_UNROLL;  // four streams: kU float4s each in flight per lane
    constexpr uint32_t kStep = 4 * BS;
    uint32_t j = j0 + 4 * threadIdx.x;
    for (; j + kStep * (kU - 1) < j1; j += kStep * kU) {
        float4 vy[kU], vd[kU], vn[kU], vx[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const uint32_t i = chan_addr(fbase, j + u * kStep, g) >> 2;
            vd[u] = ld4<(H & 2) != 0>(delta, i);
            if constexpr (!kLin) vy[u] = ld4<(H & 1) != 0>(y, i);
            else vy[u] = vd[u];
            vn[u] = ld4<(H & 4) != 0>(x_norm, i);
            vx[u] = ld4<(H & 8) != 0>(x, i);
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) acc_bwd<A>(vy[u], vd[u], vn[u], vx[u], m, gam, a);
    }
    for (; j < j1; j += kStep) {
        const uint32_t i = chan_addr(fbase, j, g) >> 2;
        const float4 vd = ld4<(H & 2) != 0>(delta, i);
        const float4 vy = kLin ? vd : ld4<(H & 1) != 0>(y, i);
        acc_bwd<A>(vy, vd, ld4<(H & 4) != 0>(x_norm, i), ld4<(H & 8) != 0>(x, i), m, gam, a);
    }
    const Sums<4> r = block_sums<4, BS>(a, lds);
    if constexpr (FIN) {
        if (threadIdx.x == 0) fin(f, r);
    } else {
        store_partials<4, BS>(r, g, f, k, partials);
    }
}

struct BwdParams {
    const float *mean, *variance, *mean_delta, *variance_delta, *scales;
    float denom;  // f32(spatial * batch), blas.zig:191
};

// What the backward apply pass needs of channel f.
struct BwdChan {
    float m, inv, vd2, mdn, gam;
};

__device__ __forceinline__ BwdChan bwd_chan(const BwdParams &p, uint32_t f, float md, float vd) {
    return {p.mean[f], 1.0f / sqrtf(p.variance[f] + 1e-5f), vd * 2.0f, md / p.denom, p.scales[f]};
}

// delta = d2 * inv + ((vd * 2) * (x - m)) / N + md / N (blas.zig:180-204) on
// d2 = delta * gradient(y) * scale.
template <int A>
__device__ __forceinline__ float4 bwd_elem(float4 y, float4 d, float4 x, const BwdChan &c, float denom) {
    float4 o;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        const float d2 = grad_delta<A>(lane(d, l), lane(y, l)) * c.gam;
        lane(o, l) = (d2 * c.inv + (c.vd2 * (lane(x, l) - c.m)) / denom) + c.mdn;
    }
    return o;
}

// Backward apply. FIN as in the forward apply: the workgroup adds the
// partials of its tile's channels itself, and the workgroup holding a
// channel's first element writes its updates, mean_delta and variance_delta.
// H: bit 0 = y, bit 1 = delta, bit 2 = x loads, bit 3 = delta store.
template <int A, int H, bool FIN>
__global__ __launch_bounds__(kBlock) void bn_bwd_apply_kernel(const float *y, float *delta, const float *x,
                                                              BwdParams p, ChanGeom g, uint32_t n, BwdFin fin,
                                                              const double *partials, uint32_t K) {
    constexpr bool kLin = A == kLinear;
    constexpr bool kNtY = (H & 1) != 0, kNtD = (H & 2) != 0, kNtX = (H & 4) != 0, kNtOut = (H & 8) != 0;
    __shared__ BwdChan slot[kSlots];
    const uint32_t nv = n >> 2;
    const uint32_t base = blockIdx.x * (kBlock * kApplyUnroll) + threadIdx.x;
    const bool full = base + (kApplyUnroll - 1) * kBlock < nv;
    float4 vy[kApplyUnroll], vd[kApplyUnroll], vx[kApplyUnroll];
#pragma unroll
    for (int u = 0; u < kApplyUnroll; ++u) {
        const uint32_t i = base + u * kBlock;
        if (full || i < nv) {
            vd[u] = ld4<kNtD>(delta, i);
            if constexpr (!kLin) vy[u] = ld4<kNtY>(y, i);
            else vy[u] = vd[u];
            vx[u] = ld4<kNtX>(x, i);
        }
    }
    uint32_t r0 = 0;
    if constexpr (FIN) {
        uint32_t e0, nrows;
        tile_rows(g, n, e0, r0, nrows);
        for (uint32_t s = threadIdx.x / kWave; s < nrows; s += kBlock / kWave) {
            const uint32_t r = r0 + s;
            const uint32_t f = r - fdiv(r, g.filters) * g.filters.d;
            const Sums<4> sums = wave_partials<4>(partials, g.filters.d, K, f);
            if ((threadIdx.x & (kWave - 1)) == 0) {
                float md, vdl;
                fin.values(f, sums, md, vdl);
                slot[s] = bwd_chan(p, f, md, vdl);
                if (r == f && f * g.spatial.d >= e0) fin.write(f, sums, md, vdl);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < kApplyUnroll; ++u) {
        const uint32_t i = base + u * kBlock;
        if (!(full || i < nv)) continue;
        const uint32_t r = fdiv(i << 2, g.spatial);
        BwdChan c;
        if constexpr (FIN) {
            c = slot[r - r0];
        } else {
            const uint32_t f = r - fdiv(r, g.filters) * g.filters.d;
            c = bwd_chan(p, f, p.mean_delta[f], p.variance_delta[f]);
        }
        st4<kNtOut>(delta, i, bwd_elem<A>(vy[u], vd[u], vx[u], c, p.denom));
    }
}

// ---- one-launch backward -------------------------------------------------------

// Backward in one launch (the shape of bn_fwd_coop_kernel): workgroup (f, k)
// loads chunk k of channel f of y, delta, x_norm and x once, forms the four
// f64 sums of bn_bwd_sums_kernel, posts them, waits at the channel barrier,
// adds the channel's K partials, finalises exactly as the two-pass path
// (workgroup k == 0 writing the updates, mean_delta and variance_delta) and
// writes normalize_delta's result from the y, delta and x it holds: 20 bytes
// an element instead of 32.
// BS threads a workgroup, U float4s of each input a lane. Measured at
// config 1's shape (graph replay, cold): 1024 x 4 (8 workgroups a channel,
// one a CU) 20.0 us; 512 x 4 20.4; 256 x 8 21.2; 256 x 4 22.3; 1024 x 2 and
// 512 x 2 (grids that do not fit at once: two passes) 27.5. Shapes whose grid
// at 1024 x 4 does not fit the GPU at once try 256 x 4.
#ifndef DKZ_BN_BWD_COOP_BS
#define DKZ_BN_BWD_COOP_BS 1024
#endif
#ifndef DKZ_BN_BWD_COOP_U
#define DKZ_BN_BWD_COOP_U 4
#endif
#ifndef DKZ_BN_BWD_COOP_BS2
#define DKZ_BN_BWD_COOP_BS2 256
#endif
#ifndef DKZ_BN_BWD_COOP_U2
#define DKZ_BN_BWD_COOP_U2 4
#endif
constexpr int kBwdCoopBS = DKZ_BN_BWD_COOP_BS, kBwdCoopU = DKZ_BN_BWD_COOP_U;
// bn_bwd_reg_kernel: 512 threads (one workgroup a CU), 49 float4s of each
// input a lane (a workgroup covers 100352 elements, half a config-2
// channel), loading G float4s of each input at once. Of the two terms
// normalize_delta needs, d2 (delta * gradient(y) * scale: two inputs) is
// held for all 49 -- RD in registers, the other 49 - RD in LDS -- and
// x - mean for the first LX in LDS; the other 49 - LX read x again after the
// meeting (4 bytes an element instead of y, delta and x). LDS: (49 - RD +
// LX) float4s a lane, 144 KiB of the CU's 160 at RD 42, LX 11. Measured at
// config 2 (graph replay, cold): two passes 128 us; holding both terms of
// 30 float4s (21 in registers, 9 in LDS) and reading y, delta and x of the
// other 19 again 93.8-94.5 us; registers only, both terms, 22 / 20 / 16 /
// 12 float4s 104.5 / 105.5 / 110 / 113 us; this layout 88.9 us with GX 8
// x loads in flight after the meeting (GX 4 / 2: 89.6 / 91.7 us), the
// first PRE of them issued before the meeting (DKZ_BN_BWD_REG_PRE). RD 42
// takes up to 240 registers a lane and no scratch with G 2 (G 4 spills, and
// a build that spilled takes the two passes: 126 us).
#ifndef DKZ_BN_BWD_REG
#define DKZ_BN_BWD_REG 1
#endif
#ifndef DKZ_BN_BWD_REG_RD
#define DKZ_BN_BWD_REG_RD 42
#endif
#ifndef DKZ_BN_BWD_REG_LX
#define DKZ_BN_BWD_REG_LX 11
#endif
#ifndef DKZ_BN_BWD_REG_G
#define DKZ_BN_BWD_REG_G 2
#endif
// x loads in flight a lane after the meeting
#ifndef DKZ_BN_BWD_REG_GX
#define DKZ_BN_BWD_REG_GX 8
#endif
// x float4s a lane of the part read again that are loaded before the block's
// sums and the meeting, so that they are in flight while the workgroup waits
// (config 2, A/B on one box: 91.2 -> 90.5 us with 8, 90.6 with 4; 16 spills)
#ifndef DKZ_BN_BWD_REG_PRE
#define DKZ_BN_BWD_REG_PRE 8
#endif
// The output is formed from the last float4 of the chunk to the first, so x
// read again comes back newest first, while the Infinity Cache still holds
// it from the sums phase (config 2's counter bytes: 1.1125 -> 1.105 of the
// algorithmic bytes, 468.8 -> 465.0 MB read a launch; time unchanged).
#ifndef DKZ_BN_BWD_REG_DESC
#define DKZ_BN_BWD_REG_DESC 1
#endif
// Tensors larger than the GPU holds at once take this kernel while a
// workgroup's chunk is at most this many times what it holds (its share of
// re-read bytes grows with the chunk), two passes beyond.
#ifndef DKZ_BN_BWD_REG_MAX_CHUNKS
#define DKZ_BN_BWD_REG_MAX_CHUNKS 4
#endif
constexpr int kBwdRegBS = 512, kBwdRegU = 49, kBwdRegRD = DKZ_BN_BWD_REG_RD, kBwdRegLX = DKZ_BN_BWD_REG_LX;
static_assert(kBwdRegRD <= kBwdRegU && kBwdRegLX <= kBwdRegU, "held float4s within the chunk");
static_assert((size_t)(kBwdRegU - kBwdRegRD + kBwdRegLX) * kBwdRegBS * 16 <= 144 * 1024, "LDS of one CU");
constexpr int kBwdCoopBS2 = DKZ_BN_BWD_COOP_BS2, kBwdCoopU2 = DKZ_BN_BWD_COOP_U2;

template <int A, int H, int BS, int U>
__global__ __launch_bounds__(BS) void bn_bwd_coop_kernel(const float *y, float *delta, const float *x_norm,
                                                         const float *x, BwdParams p, RedGeom g, BwdFin fin,
                                                         uint64_t *slots, uint32_t spin) {
    constexpr bool kLin = A == kLinear;
    constexpr bool kNtY = (H & 1) != 0, kNtD = (H & 2) != 0, kNtXn = (H & 4) != 0, kNtX = (H & 8) != 0;
    constexpr bool kNtOut = (H & 16) != 0;
    __shared__ double lds[4 * (BS / kWave)];
    __shared__ BwdChan chan_sh;
    const uint32_t f = fdiv(blockIdx.x, g.div_k);
    const uint32_t k = blockIdx.x - f * g.K;
    const uint32_t F = g.div_filters.d;
    const uint32_t j0 = k * g.chunk;
    const uint32_t j1 = min(j0 + g.chunk, g.chan_len);
    const uint32_t fbase = f * g.spatial;
    const float m = p.mean[f], gam = p.scales[f];
    // Held through the barrier: d2 = delta * gradient(y) * scale and x - mean,
    // the two terms normalize_delta needs besides per-channel values, each
    // formed exactly as bwd_elem forms it.
    float4 d2[U], xm[U];
    uint32_t at[U];
    double a[4] = {0.0, 0.0, 0.0, 0.0};
    {
        float4 vy[U], vd[U], vx[U], vn[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t j = j0 + 4 * threadIdx.x + (uint32_t)u * (4 * BS);
            at[u] = j < j1 ? chan_addr(fbase, j, g) >> 2 : 0xffffffffu;
            if (j < j1) {
                vd[u] = ld4<kNtD>(delta, at[u]);
                if constexpr (!kLin) vy[u] = ld4<kNtY>(y, at[u]);
                else vy[u] = vd[u];
                vn[u] = ld4<kNtXn>(x_norm, at[u]);
                vx[u] = ld4<kNtX>(x, at[u]);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (at[u] == 0xffffffffu) continue;
            acc_bwd<A>(vy[u], vd[u], vn[u], vx[u], m, gam, a);
#pragma unroll
            for (int l = 0; l < 4; ++l) {
                lane(d2[u], l) = grad_delta<A>(lane(vd[u], l), lane(vy[u], l)) * gam;
                lane(xm[u], l) = lane(vx[u], l) - m;
            }
        }
    }
    Sums<4> sums = block_sums<4, BS>(a, lds);
    if (threadIdx.x < kWave) {
        const uint32_t met = channel_meet<4>(slots, F, g.K, f, k, sums, spin) ? 1u : 0u;
        if (threadIdx.x == 0) {
            float md, vdl;
            fin.values(f, sums, md, vdl);
            chan_sh = bwd_chan(p, f, md, vdl);
            if (k == 0) fin.write(f, sums, md, vdl, met != 0);
            note_timeout(met, kTimeoutBwdCoop);
        }
    }
    __syncthreads();
    const BwdChan ch = chan_sh;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        if (at[u] == 0xffffffffu) continue;
        float4 o;
#pragma unroll
        for (int l = 0; l < 4; ++l)  // bwd_elem's expression on the held terms
            lane(o, l) = (lane(d2[u], l) * ch.inv + (ch.vd2 * lane(xm[u], l)) / p.denom) + ch.mdn;
        st4<kNtOut>(delta, at[u], o);
    }
    if (threadIdx.x < kWave) channel_leave<4>(slots, F, g.K, f);
}

// The one-launch backward for tensors too large for bn_bwd_coop_kernel's
// grid to fit the GPU at once (config 2's): one 512-thread workgroup a CU,
// U float4s of each input a lane. The sums pass over the chunk keeps d2 for
// all U float4s (RD in registers, the rest in LDS) and x - mean for the
// first LX (LDS); after the channel meeting the output is formed from those
// and, past LX, from x read again, last float4 first. The sums pass reads
// that part of x with ordinary loads, so the second read -- newest first --
// may find it in the Infinity Cache, and everything else nontemporally; the
// first PRE float4s of the second read are issued before the meeting.
// Bytes: 16 an element read once, 4 written,
// plus 4 for x read again past LX -- instead of the two passes' 16 + 12 + 4
// for every element. Chunks longer than U float4s a lane (tensors larger
// than the GPU holds at once) read y, delta and x of the rest again.
template <int A, int H, int BS, int U, int RD, int LX>
__global__ __launch_bounds__(BS) void bn_bwd_reg_kernel(const float *y, float *delta, const float *x_norm,
                                                        const float *x, BwdParams p, RedGeom g, BwdFin fin,
                                                        uint64_t *slots, uint32_t spin) {
    constexpr bool kLin = A == kLinear;
    constexpr bool kNtOut = (H & 16) != 0;
    constexpr int G = DKZ_BN_BWD_REG_G;   // float4s of each input a lane loads at once
    constexpr int GX = DKZ_BN_BWD_REG_GX; // x loads in flight after the meeting
    constexpr int LD = U - RD;            // d2 float4s held in LDS
    constexpr int PX = DKZ_BN_BWD_REG_PRE < U - LX ? DKZ_BN_BWD_REG_PRE : U - LX;  // x loaded before the meeting
    constexpr bool kDesc = DKZ_BN_BWD_REG_DESC != 0;  // output formed last float4 first
    constexpr int P0 = kDesc ? U - PX : LX;           // first of the PX float4s loaded before the meeting
    __shared__ double lds[4 * (BS / kWave)];
    __shared__ float4 held_d2[(LD > 0 ? LD : 1) * BS];  // float4 RD + i of lane t at [i * BS + t]
    __shared__ float4 held_xm[(LX > 0 ? LX : 1) * BS];  // float4 i of lane t at [i * BS + t]
    __shared__ BwdChan chan_sh;
    const uint32_t f = fdiv(blockIdx.x, g.div_k);
    const uint32_t k = blockIdx.x - f * g.K;
    const uint32_t F = g.div_filters.d;
    const uint32_t j0 = k * g.chunk;
    const uint32_t j1 = min(j0 + g.chunk, g.chan_len);
    const uint32_t fbase = f * g.spatial;
    const float m = p.mean[f], gam = p.scales[f];
    // float4 u of the lane is element jb + u*4*BS of the channel; jb is
    // recomputed in each phase from a copy the compiler cannot see through,
    // so no per-float4 address stays live across phases.
    const auto phase_base = [&]() {
        uint32_t jb = j0 + 4 * threadIdx.x;
        asm volatile("" : "+v"(jb));
        return jb;
    };
    float4 d2[RD > 0 ? RD : 1];
    double a[4] = {0.0, 0.0, 0.0, 0.0};
    // sums over the held part, keeping d2 (and x - m for u < LX); the steps
    // are generated at compile time, so every index into d2 is a constant
    // and the array stays in registers
    static_for<0, U, G>([&](auto step) {
        constexpr int u0 = decltype(step)::value;
        constexpr int n = U - u0 < G ? U - u0 : G;
        const uint32_t jb = phase_base();
        float4 vy[G], vd[G], vn[G], vx[G];
#pragma unroll
        for (int v = 0; v < n; ++v) {
            const uint32_t j = jb + (uint32_t)(u0 + v) * (4 * BS);
            if (j < j1) {
                const uint32_t at = chan_addr(fbase, j, g) >> 2;
                vd[v] = ld4<true>(delta, at);
                if constexpr (!kLin) vy[v] = ld4<true>(y, at);
                else vy[v] = vd[v];
                vn[v] = ld4<true>(x_norm, at);
                // x past LX is read again after the meeting: cached
                vx[v] = u0 + v < LX ? ld4<true>(x, at) : ld4<false>(x, at);
            }
        }
        static_for<0, n, 1>([&](auto vc) {
            constexpr int v = decltype(vc)::value, u = u0 + v;
            const uint32_t j = jb + (uint32_t)u * (4 * BS);
            if (j >= j1) return;
            acc_bwd<A>(vy[v], vd[v], vn[v], vx[v], m, gam, a);
            float4 t2;
#pragma unroll
            for (int l = 0; l < 4; ++l) lane(t2, l) = grad_delta<A>(lane(vd[v], l), lane(vy[v], l)) * gam;
            if constexpr (u < RD) d2[u] = t2;
            else held_d2[(u - RD) * BS + threadIdx.x] = t2;
            if constexpr (u < LX) {
                float4 tm;
#pragma unroll
                for (int l = 0; l < 4; ++l) lane(tm, l) = lane(vx[v], l) - m;
                held_xm[u * BS + threadIdx.x] = tm;
            }
        });
    });
    // chunks longer than U float4s a lane (tensors larger than the GPU
    // holds at once): the rest is read here, cached, and again after the
    // meeting
    for (uint32_t u0 = U;; u0 += G) {
        const uint32_t jb = phase_base();
        if (jb + u0 * (4 * BS) >= j1) break;
        float4 vy[G], vd[G], vn[G], vx[G];
#pragma unroll
        for (int v = 0; v < G; ++v) {
            const uint32_t j = jb + (u0 + v) * (4 * BS);
            if (j < j1) {
                const uint32_t at = chan_addr(fbase, j, g) >> 2;
                vd[v] = ld4<false>(delta, at);
                if constexpr (!kLin) vy[v] = ld4<false>(y, at);
                else vy[v] = vd[v];
                vn[v] = ld4<true>(x_norm, at);
                vx[v] = ld4<false>(x, at);
            }
        }
#pragma unroll
        for (int v = 0; v < G; ++v) {
            const uint32_t j = jb + (u0 + v) * (4 * BS);
            if (j < j1) acc_bwd<A>(vy[v], vd[v], vn[v], vx[v], m, gam, a);
        }
    }
    // the first PX float4s of the x read again (in the order the output is
    // formed), loaded now so they are in flight during the block's sums and
    // the meeting
    float4 px[PX > 0 ? PX : 1];
    {
        const uint32_t jb = phase_base();
        static_for<0, PX, 1>([&](auto vc) {
            constexpr int v = decltype(vc)::value;
            const uint32_t j = jb + (uint32_t)(P0 + v) * (4 * BS);
            if (j < j1) px[v] = ld4<true>(x, chan_addr(fbase, j, g) >> 2);
        });
    }
    Sums<4> sums = block_sums<4, BS>(a, lds);
    if (threadIdx.x < kWave) {
        const uint32_t met = channel_meet<4>(slots, F, g.K, f, k, sums, spin) ? 1u : 0u;
        if (threadIdx.x == 0) {
            float md, vdl;
            fin.values(f, sums, md, vdl);
            chan_sh = bwd_chan(p, f, md, vdl);
            if (k == 0) fin.write(f, sums, md, vdl, met != 0);
            note_timeout(met, kTimeoutBwdReg);
        }
    }
    __syncthreads();
    const BwdChan ch = chan_sh;
    // the held part, last float4 first (kDesc): d2 from registers or LDS,
    // x - m from LDS or x read again
    static_for<0, U, GX>([&](auto step) {
        constexpr int u0 = decltype(step)::value;
        constexpr int n = U - u0 < GX ? U - u0 : GX;
        const uint32_t jb = phase_base();
        float4 vx[GX];
        static_for<0, n, 1>([&](auto vc) {
            constexpr int v = decltype(vc)::value, u = kDesc ? U - 1 - (u0 + v) : u0 + v;
            const uint32_t j = jb + (uint32_t)u * (4 * BS);
            if constexpr (u >= LX && (u < P0 || u >= P0 + PX)) {
                if (j < j1) vx[v] = ld4<true>(x, chan_addr(fbase, j, g) >> 2);
            }
        });
        static_for<0, n, 1>([&](auto vc) {
            constexpr int v = decltype(vc)::value, u = kDesc ? U - 1 - (u0 + v) : u0 + v;
            const uint32_t j = jb + (uint32_t)u * (4 * BS);
            if (j >= j1) return;
            float4 t2, tm;
            if constexpr (u < RD) t2 = d2[u];
            else t2 = held_d2[(u - RD) * BS + threadIdx.x];
            if constexpr (u < LX) {
                tm = held_xm[u * BS + threadIdx.x];
            } else if constexpr (u >= P0 && u < P0 + PX) {
#pragma unroll
                for (int l = 0; l < 4; ++l) lane(tm, l) = lane(px[u - P0], l) - ch.m;
            } else {
#pragma unroll
                for (int l = 0; l < 4; ++l) lane(tm, l) = lane(vx[v], l) - ch.m;
            }
            float4 o;
#pragma unroll
            for (int l = 0; l < 4; ++l) lane(o, l) = (lane(t2, l) * ch.inv + (ch.vd2 * lane(tm, l)) / p.denom) + ch.mdn;
            st4<kNtOut>(delta, chan_addr(fbase, j, g) >> 2, o);
        });
    });
    for (uint32_t u0 = U;; u0 += G) {
        const uint32_t jb = phase_base();
        if (jb + u0 * (4 * BS) >= j1) break;
        float4 vy[G], vd[G], vx[G];
#pragma unroll
        for (int v = 0; v < G; ++v) {
            const uint32_t j = jb + (u0 + v) * (4 * BS);
            if (j < j1) {
                const uint32_t at = chan_addr(fbase, j, g) >> 2;
                vd[v] = ld4<true>(delta, at);
                if constexpr (!kLin) vy[v] = ld4<true>(y, at);
                else vy[v] = vd[v];
                vx[v] = ld4<true>(x, at);
            }
        }
#pragma unroll
        for (int v = 0; v < G; ++v) {
            const uint32_t j = jb + (u0 + v) * (4 * BS);
            if (j < j1) st4<kNtOut>(delta, chan_addr(fbase, j, g) >> 2, bwd_elem<A>(vy[v], vd[v], vx[v], ch, p.denom));
        }
    }
    if (threadIdx.x < kWave) channel_leave<4>(slots, F, g.K, f);
}

// ---- host ---------------------------------------------------------------------

// The one-launch forward, for channels split over at most 256 workgroups
// (a channel's workgroups must fit the GPU at once).
#ifndef DKZ_BN_FWD_COOP
#define DKZ_BN_FWD_COOP 1
#endif
// ... and at most this many workgroups in all (and no more than the GPU
// holds at once, resident_workgroups), so that the whole grid is resident at
// once (otherwise workgroups waiting at their barrier hold CUs that later
// channels need: config 2's shape, 6272 workgroups, took 105 us against 97
// for the two passes; the backward with 2048 workgroups at 4 waves per SIMD
// 38.6 against 27.8).
#ifndef DKZ_BN_COOP_MAX_WGS
#define DKZ_BN_COOP_MAX_WGS 2048
#endif
#ifndef DKZ_BN_BWD_COOP
#define DKZ_BN_BWD_COOP 1
#endif
#ifndef DKZ_BN_FWD_COOP_REG
#define DKZ_BN_FWD_COOP_REG 1
#endif
// The register-resident forward also runs on tensors larger than the GPU
// holds at once -- as many workgroups a channel as fit, each reading again
// the part of its chunk it cannot hold -- while a chunk is at most this many
// times what a workgroup holds. Measured against the two passes (graph
// replay): [16,64,208,208] (1.7 times) 151.6 -> 131.4 us, [32,128,112,112]
// (2.0) 178.4 -> 155.8; [4,3,6M] (2.8) 291 -> 303, [2,1,50M] (3.9) 434 -> 478.
#ifndef DKZ_BN_FWD_REG_MAX_CHUNKS
#define DKZ_BN_FWD_REG_MAX_CHUNKS 2
#endif

// Workgroups of Kernel (BS threads) the GPU holds at once: HIP's occupancy
// for the kernel's registers and LDS times the CU count, looked up once per
// kernel and device. A one-launch pass runs only when its whole grid fits,
// so no workgroup waits at its channel barrier for one that is not yet
// resident.
// The lookups are HIP queries, not stream work; dkz_init makes them all
// once (batchnorm_prewarm) so that no op makes one for the first time inside
// a graph capture. The caches are atomics: two host threads that race to
// fill one store the same value.
template <auto Kernel, int BS>
uint32_t resident_workgroups() {
    static std::atomic<uint32_t> cache[kMaxDevices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
    uint32_t v = cache[dev].load(std::memory_order_relaxed);
    if (v == 0) {
        int per_cu = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, Kernel, BS, 0) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return 0;
        v = (uint32_t)(per_cu > 0 ? per_cu : 0) * (uint32_t)(cus > 0 ? cus : 0);
        cache[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

// Whether Kernel keeps everything in registers (no private scratch), looked
// up once: the register-resident pass is only worth it without spills (the
// exp-based activations' tanh, for one, spills at 49 float4s a lane).
template <auto Kernel>
bool no_spills() {
    static std::atomic<int> cached{-1};  // -1 unknown, 0 spills, 1 none
    int v = cached.load(std::memory_order_relaxed);
    if (v < 0) {
        hipFuncAttributes attr{};
        v = hipFuncGetAttributes(&attr, reinterpret_cast<const void *>(Kernel)) == hipSuccess &&
                    attr.localSizeBytes == 0
                ? 1
                : 0;
        cached.store(v, std::memory_order_relaxed);
    }
    return v == 1;
}

struct Shape {
    uint32_t B, F, S, n;
};

struct FwdArgs {
    Shape sh;
    bool train;
    const float *input;
    float *output, *x, *x_norm, *mean, *variance, *rolling_mean, *rolling_variance;
    const float *scales, *biases;
};

struct BwdArgs {
    Shape sh;
    const float *y;
    float *delta;
    const float *x, *x_norm, *mean, *variance, *scales;
    float *bias_updates, *scale_updates, *mean_delta, *variance_delta;
};

// Split of a reduction pass over the channels of a shape.
template <int NS>
RedGeom sums_geom(const Shape &sh, uint32_t streams) {
    const uint32_t L = sh.B * sh.S;
    return make_red_geom(sh.F, sh.S, L,
                         pick_split(sh.F, L, streams, NS, DKZ_BN_SPLIT_TARGET, DKZ_BN_MIN_CHUNK), true);
}

// An apply workgroup's tile spans at most kSlots rows, so it can finalise
// its own channels.
inline bool tile_fits_slots(uint32_t S) { return (kTile - 1) / S + 2 <= kSlots; }

// Launches a reduction pass. K == 1: one workgroup per channel finalises it
// (1024 threads for long channels). K > 1: partial sums into the scratch,
// then the finalize launch -- unless `defer`, when the apply pass finalises
// and *partials receives the scratch.
template <int NS, class Fin, class KWide, class KFin, class KPart, class... Args>
int run_sums(const char *name, const RedGeom &g, const Shape &sh, const Fin &fin, bool defer,
             const double **partials, KWide kwide, KFin kfin, KPart kpart, Args... args) {
    *partials = nullptr;
    if (g.K == 1) {
        if (g.chan_len >= 16 * kWideBlock)
            return launch(name, kwide, dim3(sh.F), dim3(kWideBlock), args..., g, fin, (double *)nullptr);
        return launch(name, kfin, dim3(sh.F), dim3(kBlock), args..., g, fin, (double *)nullptr);
    }
    Scratch sc{nullptr};
    DKZ_TRY(device_scratch(&sc));
    DKZ_TRY(launch(name, kpart, dim3(sh.F * g.K), dim3(kBlock), args..., g, fin, sc.partials));
    if (defer) {
        *partials = sc.partials;
        return 0;
    }
    return launch(name, bn_finalize_kernel<NS, Fin>, dim3(div_up(sh.F, kBlock / kWave)), dim3(kBlock), fin,
                  (const double *)sc.partials, sh.F, g.K);
}

// The one-launch forward with BS-thread workgroups holding U float4s a
// lane, when its whole grid fits the GPU at once (and, for CHECK_SPILLS,
// when the kernel keeps its chunk in registers): launches it and returns
// true with its status in *rc; otherwise returns false, launching nothing.
template <int A, int BS, int U, bool CHECK_SPILLS, bool EXTRA = false>
bool fwd_coop(const FwdArgs &a, uint64_t L, int *rc) {
    constexpr auto kernel = bn_fwd_coop_kernel<A, DKZ_HINT_BN_FWD_COOP, BS, U, EXTRA>;
    constexpr uint64_t chunk = (uint64_t)BS * 4 * U;
    const Shape &sh = a.sh;
    uint64_t K = div_up(L, chunk);
    if constexpr (EXTRA) {
        // only for tensors whose held chunks do not all fit: as many
        // workgroups a channel as fit, each reading again what it cannot
        // hold, while that is at most DKZ_BN_FWD_REG_MAX_CHUNKS times what it
        // holds
        if (!no_spills<kernel>()) return false;
        const uint64_t res = resident_workgroups<kernel, BS>();
        if ((uint64_t)sh.F * K <= res) return false;
        K = res / sh.F;
        if (K == 0 || div_up(L, K) > (uint64_t)DKZ_BN_FWD_REG_MAX_CHUNKS * chunk) return false;
    }
    const uint64_t wgs = (uint64_t)sh.F * K;
    if (K > 256 || wgs > DKZ_BN_COOP_MAX_WGS || meet_slots(sh.F, K) > kScratchSlots) return false;
    if constexpr (CHECK_SPILLS) {
        if (!no_spills<kernel>()) return false;
    }
    if (wgs > resident_workgroups<kernel, BS>()) return false;
    const RedGeom gc = make_red_geom(sh.F, sh.S, (uint32_t)L, (uint32_t)K, true);
    Scratch sc{nullptr};
    *rc = device_scratch(&sc);
    if (*rc != 0) return true;
    const FwdFin fin{nullptr, a.mean, a.variance, a.rolling_mean, a.rolling_variance,
                     (double)L, 1.0f / (float)L, 1.0f / (float)(L - 1u)};
    const FwdParams p{a.mean, a.variance, a.scales, a.biases};
    *rc = launch("batchnorm_forward", kernel, dim3(sh.F * gc.K), dim3(BS), a.input, a.output, a.x, a.x_norm, p, gc,
                 fin, sc.slots, barrier_spin_limit());
    if (*rc == 0 && sync_after_launch()) *rc = take_barrier_timeout();
    return true;
}

// $DKZ_BN_TWO_PASS=1 (read at each call) skips the one-launch passes, so
// the tests reach the two-pass path at any shape.
inline bool two_pass_forced() {
    const char *e = getenv("DKZ_BN_TWO_PASS");
    return e != nullptr && e[0] == '1';
}

template <int A>
int bn_forward_fused(const FwdArgs &a) {
    constexpr int H = DKZ_HINT_BN_FWD_APPLY;
    const Shape &sh = a.sh;
    const ChanGeom cg{make_fastdiv(sh.S), make_fastdiv(sh.F)};
    const dim3 grid(div_up(sh.n, kTile)), block(kBlock);
    const uint64_t L = (uint64_t)sh.B * sh.S;
    // shift: after the 2*F*K partials of a split pass (two sums + one shift
    // per channel fit the scratch: pick_split is asked for 3 per chunk)
    const RedGeom g = sums_geom<3>(sh, 1);
    Scratch sc{nullptr};
    if (a.train && g.K > 1) DKZ_TRY(device_scratch(&sc));
    const FwdFin fin{sc.partials ? sc.partials + 2u * sh.F * g.K : nullptr, a.mean, a.variance, a.rolling_mean,
                     a.rolling_variance, (double)L, 1.0f / (float)L, 1.0f / (float)(L - 1u)};
    if (!a.train) {
        const FwdParams p{a.rolling_mean, a.rolling_variance, a.scales, a.biases};
        return launch("batchnorm_forward_apply", bn_fwd_apply_kernel<A, false, H, false>, grid, block, a.input,
                      a.output, a.x, a.x_norm, p, cg, sh.n, fin, (const double *)nullptr, 0u);
    }
    int rc = 0;
    const bool one_launch = !two_pass_forced();
    if (DKZ_BN_FWD_COOP && one_launch && (fwd_coop<A, kCoopBS, kCoopU, false>(a, L, &rc) ||
                                          fwd_coop<A, kCoopBS2, kCoopU2, false>(a, L, &rc)))
        return rc;
    // the same with one 512-thread workgroup a CU holding 196 floats a lane,
    // for tensors that fill the register file
    if (DKZ_BN_FWD_COOP_REG && one_launch &&
        (fwd_coop<A, kRegBlock, kRegU, true>(a, L, &rc) || fwd_coop<A, kRegBlock, kRegU, true, true>(a, L, &rc)))
        return rc;
    const bool defer = DKZ_BN_DEFER_FWD && g.K > 1 && g.K <= DKZ_BN_DEFER_MAX_K && tile_fits_slots(sh.S);
    const double *partials = nullptr;
    DKZ_TRY(run_sums<2>("batchnorm_forward_stats", g, sh, fin, defer, &partials,
                        bn_stats_kernel<DKZ_HINT_BN_STATS, kWideBlock, true>,
                        bn_stats_kernel<DKZ_HINT_BN_STATS, kBlock, true>,
                        bn_stats_kernel<DKZ_HINT_BN_STATS, kBlock, false>, a.input));
    const FwdParams p{a.mean, a.variance, a.scales, a.biases};
    if (defer)
        return launch("batchnorm_forward_apply", bn_fwd_apply_kernel<A, true, H, true>, grid, block, a.input,
                      a.output, a.x, a.x_norm, p, cg, sh.n, fin, partials, g.K);
    return launch("batchnorm_forward_apply", bn_fwd_apply_kernel<A, true, H, false>, grid, block, a.input,
                  a.output, a.x, a.x_norm, p, cg, sh.n, fin, (const double *)nullptr, 0u);
}

// The one-launch backward with BS-thread workgroups holding U float4s of
// each input a lane, when its whole grid fits the GPU at once: launches it
// and returns true with its status in *rc; otherwise returns false,
// launching nothing.
template <int A, int BS, int U>
bool bwd_coop(const BwdArgs &a, uint64_t L, const BwdFin &fin, int *rc) {
    constexpr auto kernel = bn_bwd_coop_kernel<A, DKZ_HINT_BN_BWD_COOP, BS, U>;
    const Shape &sh = a.sh;
    const uint64_t K = div_up(L, (uint64_t)BS * 4 * U), wgs = (uint64_t)sh.F * K;
    if (K > 256 || wgs > DKZ_BN_COOP_MAX_WGS || meet_slots(sh.F, K) > kScratchSlots ||
        wgs > resident_workgroups<kernel, BS>())
        return false;
    const RedGeom gc = make_red_geom(sh.F, sh.S, (uint32_t)L, (uint32_t)K, true);
    Scratch sc{nullptr};
    *rc = device_scratch(&sc);
    if (*rc != 0) return true;
    const BwdParams p{a.mean, a.variance, a.mean_delta, a.variance_delta, a.scales,
                      (float)((uint64_t)sh.S * (uint64_t)sh.B)};
    *rc = launch("batchnorm_backward", kernel, dim3(sh.F * gc.K), dim3(BS), a.y, a.delta, a.x_norm, a.x, p, gc, fin,
                 sc.slots, barrier_spin_limit());
    if (*rc == 0 && sync_after_launch()) *rc = take_barrier_timeout();
    return true;
}

// bn_bwd_reg_kernel under the same rules as bwd_coop, and only when the
// kernel keeps its held part in registers (no scratch).
template <int A>
bool bwd_reg(const BwdArgs &a, uint64_t L, const BwdFin &fin, int *rc) {
    constexpr auto kernel = bn_bwd_reg_kernel<A, DKZ_HINT_BN_BWD_COOP, kBwdRegBS, kBwdRegU, kBwdRegRD, kBwdRegLX>;
    const Shape &sh = a.sh;
    constexpr uint64_t kCap = (uint64_t)kBwdRegBS * 4 * kBwdRegU;  // 100352
    if (!no_spills<kernel>()) return false;
    const uint64_t res = resident_workgroups<kernel, kBwdRegBS>();
    uint64_t K = div_up(L, kCap);
    if ((uint64_t)sh.F * K > res) {
        // more than the GPU holds at once: as many workgroups a channel as
        // fit, each re-reading what it cannot hold -- while that is at most
        // DKZ_BN_BWD_REG_MAX_CHUNKS times what it holds
        K = res / sh.F;
        if (K == 0 || div_up(L, K) > (uint64_t)DKZ_BN_BWD_REG_MAX_CHUNKS * kCap) return false;
    }
    const uint64_t wgs = (uint64_t)sh.F * K;
    if (K > 256 || wgs > DKZ_BN_COOP_MAX_WGS || meet_slots(sh.F, K) > kScratchSlots || wgs > res) return false;
    const RedGeom gc = make_red_geom(sh.F, sh.S, (uint32_t)L, (uint32_t)K, true);
    Scratch sc{nullptr};
    *rc = device_scratch(&sc);
    if (*rc != 0) return true;
    const BwdParams p{a.mean, a.variance, a.mean_delta, a.variance_delta, a.scales,
                      (float)((uint64_t)sh.S * (uint64_t)sh.B)};
    *rc = launch("batchnorm_backward", kernel, dim3(sh.F * gc.K), dim3(kBwdRegBS), a.y, a.delta, a.x_norm, a.x, p,
                 gc, fin, sc.slots, barrier_spin_limit());
    if (*rc == 0 && sync_after_launch()) *rc = take_barrier_timeout();
    return true;
}

template <int A>
int bn_backward_fused(const BwdArgs &a) {
    constexpr int H = DKZ_HINT_BN_BWD_APPLY;
    const Shape &sh = a.sh;
    const BwdFin fin{a.variance, a.bias_updates, a.scale_updates, a.mean_delta, a.variance_delta};
    const uint64_t L = (uint64_t)sh.B * sh.S;
    int rc = 0;
    const bool one_launch = !two_pass_forced();
    if (DKZ_BN_BWD_COOP && one_launch && (bwd_coop<A, kBwdCoopBS, kBwdCoopU>(a, L, fin, &rc) ||
                                          bwd_coop<A, kBwdCoopBS2, kBwdCoopU2>(a, L, fin, &rc)))
        return rc;
    if (DKZ_BN_BWD_REG && one_launch && bwd_reg<A>(a, L, fin, &rc)) return rc;
    const RedGeom g = sums_geom<4>(sh, A == kLinear ? 3 : 4);
    const bool defer = DKZ_BN_DEFER_BWD && g.K > 1 && g.K <= DKZ_BN_DEFER_MAX_K && tile_fits_slots(sh.S);
    const double *partials = nullptr;
    constexpr int HS = DKZ_HINT_BN_BWD_SUMS;
    DKZ_TRY(run_sums<4>("batchnorm_backward_sums", g, sh, fin, defer, &partials,
                        bn_bwd_sums_kernel<A, HS, kWideBlock, true>, bn_bwd_sums_kernel<A, HS, kBlock, true>,
                        bn_bwd_sums_kernel<A, HS, kBlock, false>, a.y, (const float *)a.delta, a.x_norm, a.x,
                        a.mean, a.scales));
    const ChanGeom cg{make_fastdiv(sh.S), make_fastdiv(sh.F)};
    const BwdParams p{a.mean, a.variance, a.mean_delta, a.variance_delta, a.scales,
                      (float)((uint64_t)sh.S * (uint64_t)sh.B)};
    const dim3 grid(div_up(sh.n, kTile)), block(kBlock);
    if (defer)
        return launch("batchnorm_backward_apply", bn_bwd_apply_kernel<A, H, true>, grid, block, a.y, a.delta, a.x,
                      p, cg, sh.n, fin, partials, g.K);
    return launch("batchnorm_backward_apply", bn_bwd_apply_kernel<A, H, false>, grid, block, a.y, a.delta, a.x, p,
                  cg, sh.n, fin, (const double *)nullptr, 0u);
}

// Every occupancy and attribute lookup the one-launch passes of activation
// A make, made ahead (fwd_coop, bwd_coop and bwd_reg ask the same ones).
template <int A>
void prewarm() {
    constexpr int HF = DKZ_HINT_BN_FWD_COOP, HB = DKZ_HINT_BN_BWD_COOP;
    (void)resident_workgroups<bn_fwd_coop_kernel<A, HF, kCoopBS, kCoopU>, kCoopBS>();
    (void)resident_workgroups<bn_fwd_coop_kernel<A, HF, kCoopBS2, kCoopU2>, kCoopBS2>();
    (void)no_spills<bn_fwd_coop_kernel<A, HF, kRegBlock, kRegU>>();
    (void)resident_workgroups<bn_fwd_coop_kernel<A, HF, kRegBlock, kRegU>, kRegBlock>();
    (void)no_spills<bn_fwd_coop_kernel<A, HF, kRegBlock, kRegU, true>>();
    (void)resident_workgroups<bn_fwd_coop_kernel<A, HF, kRegBlock, kRegU, true>, kRegBlock>();
    (void)resident_workgroups<bn_bwd_coop_kernel<A, HB, kBwdCoopBS, kBwdCoopU>, kBwdCoopBS>();
    (void)resident_workgroups<bn_bwd_coop_kernel<A, HB, kBwdCoopBS2, kBwdCoopU2>, kBwdCoopBS2>();
    constexpr auto reg = bn_bwd_reg_kernel<A, HB, kBwdRegBS, kBwdRegU, kBwdRegRD, kBwdRegLX>;
    (void)no_spills<reg>();
    (void)resident_workgroups<reg, kBwdRegBS>();
}

typedef int (*FwdFn)(const FwdArgs &);
typedef int (*BwdFn)(const BwdArgs &);
typedef void (*PrewarmFn)();
template <int... As>
struct BnTables {
    static constexpr FwdFn fwd[] = {bn_forward_fused<As>...};
    static constexpr BwdFn bwd[] = {bn_backward_fused<As>...};
    static constexpr PrewarmFn prewarm[] = {dkz::prewarm<As>...};
};
using Tables = BnTables<0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13>;

}  // namespace

void batchnorm_prewarm() {
    for (const PrewarmFn fn : Tables::prewarm) fn();
}

int take_barrier_timeout() {
    uint32_t which = 0;
    hipError_t e = hipMemcpyFromSymbol(&which, HIP_SYMBOL(barrier_timeout), sizeof which, 0, hipMemcpyDeviceToHost);
    if (e != hipSuccess) {
        set_error_context("reading the channel-barrier time-out flag");
        return (int)e;
    }
    if (which == 0) return 0;
    const uint32_t zero = 0;
    e = hipMemcpyToSymbol(HIP_SYMBOL(barrier_timeout), &zero, sizeof zero, 0, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        set_error_context("clearing the channel-barrier time-out flag");
        return (int)e;
    }
    static const char *const kernels[] = {"?", "batchnorm_forward (bn_fwd_coop_kernel)",
                                          "batchnorm_backward (bn_bwd_coop_kernel)",
                                          "batchnorm_backward (bn_bwd_reg_kernel)"};
    set_error_context("HIP: %s: a channel meeting gave up waiting for the channel's other workgroups; those "
                      "workgroups' outputs are NaN, rolling averages and bias/scale updates were left unchanged",
                      kernels[which < 4 ? which : 0]);
    return (int)hipErrorLaunchTimeOut;
}

}  // namespace dkz

using namespace dkz;

extern "C" {

int dkz_batchnorm_forward(int batch, int filters, int spatial, int activation, int train, const float *input,
                          float *output, float *x, float *x_norm, float *mean, float *variance,
                          float *rolling_mean, float *rolling_variance, const float *scales,
                          const float *biases) {
    DKZ_REQUIRE(batch >= 0 && filters >= 0 && spatial >= 0);
    DKZ_REQUIRE(activation >= 0 && activation < kActCount);
    const uint64_t n64 = (uint64_t)batch * (uint64_t)filters * (uint64_t)spatial;
    DKZ_REQUIRE(n64 <= kMaxElems);
    if (filters == 0) return 0;
    DKZ_REQUIRE(scales && biases && rolling_mean && rolling_variance);
    DKZ_REQUIRE(!train || (mean && variance));
    DKZ_REQUIRE(n64 == 0 || (input && output && x && (!train || x_norm)));
    const int n = (int)n64;
    const bool fast = n64 > 0 && spatial % 4 == 0 && aligned16(input) && aligned16(output) && aligned16(x) &&
                      (!train || aligned16(x_norm));
    if (fast) {
        const FwdArgs a{{(uint32_t)batch, (uint32_t)filters, (uint32_t)spatial, (uint32_t)n},
                        train != 0, input, output, x, x_norm, mean, variance, rolling_mean, rolling_variance,
                        scales, biases};
        return Tables::fwd[activation](a);
    }
    // The per-op sequence of batchnorm.zig:129-153 and convolutional.zig:269.
    if (input != output) DKZ_TRY(dkz_copy(n, input, output));
    DKZ_TRY(dkz_copy(n, output, x));
    if (train) {
        DKZ_TRY(dkz_mean(output, batch, filters, spatial, mean));
        DKZ_TRY(dkz_variance(output, mean, batch, filters, spatial, variance));
        DKZ_TRY(dkz_scal(filters, kMomentum, rolling_mean));
        DKZ_TRY(dkz_axpy(filters, kAlpha, mean, rolling_mean));
        DKZ_TRY(dkz_scal(filters, kMomentum, rolling_variance));
        DKZ_TRY(dkz_axpy(filters, kAlpha, variance, rolling_variance));
        DKZ_TRY(dkz_normalize(output, mean, variance, batch, filters, spatial));
        DKZ_TRY(dkz_copy(n, output, x_norm));
    } else {
        DKZ_TRY(dkz_normalize(output, rolling_mean, rolling_variance, batch, filters, spatial));
    }
    DKZ_TRY(dkz_scale_bias(output, scales, batch, filters, spatial));
    DKZ_TRY(dkz_add_bias(output, biases, batch, filters, spatial));
    return dkz_activate_array(output, n, activation);
}

int dkz_batchnorm_backward(int batch, int filters, int spatial, int activation, const float *output,
                           float *delta, const float *x, const float *x_norm, const float *mean,
                           const float *variance, const float *scales, float *bias_updates,
                           float *scale_updates, float *mean_delta, float *variance_delta) {
    DKZ_REQUIRE(batch >= 0 && filters >= 0 && spatial >= 0);
    DKZ_REQUIRE(activation >= 0 && activation < kActCount);
    const uint64_t n64 = (uint64_t)batch * (uint64_t)filters * (uint64_t)spatial;
    DKZ_REQUIRE(n64 <= kMaxElems);
    if (filters == 0) return 0;
    DKZ_REQUIRE(mean && variance && scales && bias_updates && scale_updates && mean_delta && variance_delta);
    DKZ_REQUIRE(n64 == 0 || (delta && x && x_norm && (activation == kLinear || output)));
    const int n = (int)n64;
    const bool fast = n64 > 0 && spatial % 4 == 0 && aligned16(delta) && aligned16(x) && aligned16(x_norm) &&
                      (activation == kLinear || aligned16(output));
    if (fast) {
        const BwdArgs a{{(uint32_t)batch, (uint32_t)filters, (uint32_t)spatial, (uint32_t)n},
                        output, delta, x, x_norm, mean, variance, scales,
                        bias_updates, scale_updates, mean_delta, variance_delta};
        return Tables::bwd[activation](a);
    }
    // convolutional.zig:280 and the per-op sequence of batchnorm.zig:155-174.
    DKZ_TRY(dkz_gradient_array(output, n, activation, delta));
    DKZ_TRY(dkz_backward_bias(bias_updates, delta, batch, filters, spatial));
    DKZ_TRY(dkz_backward_scale(x_norm, delta, batch, filters, spatial, scale_updates));
    DKZ_TRY(dkz_scale_bias(delta, scales, batch, filters, spatial));
    DKZ_TRY(dkz_mean_delta(delta, variance, batch, filters, spatial, mean_delta));
    DKZ_TRY(dkz_variance_delta(x, delta, mean, variance, batch, filters, spatial, variance_delta));
    return dkz_normalize_delta(x, mean, variance, mean_delta, variance_delta, batch, filters, spatial, delta);
}

}  // extern "C"
