// dkz_channel.hpp -- geometry of per-channel work on a [batch, filters,
// spatial] (NCHW) tensor, shared by the broadcast ops, the channel reductions
// and the fused batch-norm passes.
//
// Element e belongs to row r = e / spatial and channel f = r % filters
// (blas.zig:51). Element j of channel f's batch*spatial elements lives at
// ((b*F + f)*S + s) = f*S + j + b*(F-1)*S with b = j / S.
#pragma once

#include "dkz_device.hpp"
#include "dkz_internal.hpp"

namespace dkz {

// ---- broadcasts: which channel (or row) an element belongs to ---------------

struct ChanGeom {
    FastDiv spatial;
    FastDiv filters;
};

// ROWWISE: the constant is per row r (backward_avgpool), not per channel.
template <bool ROWWISE>
__device__ __forceinline__ uint32_t channel_of(uint32_t e, const ChanGeom &g) {
    const uint32_t r = fdiv(e, g.spatial);
    if constexpr (ROWWISE) return r;
    else return r - fdiv(r, g.filters) * g.filters.d;
}

// ---- reductions: which elements a workgroup of a channel owns ---------------

struct RedGeom {
    uint32_t spatial;
    uint32_t chan_len;   // batch * spatial
    uint32_t chunk;      // elements per workgroup (multiple of 4 on the float4 path)
    uint32_t K;          // workgroups per channel
    uint32_t row_extra;  // (filters - 1) * spatial
    FastDiv div_k;
    FastDiv div_spatial;
    FastDiv div_filters;
};

__device__ __forceinline__ uint32_t chan_addr(uint32_t fbase, uint32_t j, const RedGeom &g) {
    return fbase + j + fdiv(j, g.div_spatial) * g.row_extra;
}

// Widest workgroup of a one-launch channel reduction.
constexpr uint32_t kWideBlock = 1024;

// One-launch reductions hand f64 partial sums between workgroups through
// the scratch's slots as the bits XOR kMeetKey, so a posted value is never
// zero (the slots are zero when a launch starts, and every kernel that
// posts leaves them zero): kMeetKey is a NaN payload no sum produces (a NaN
// reaching a sum carries an f32 payload whose low 29 bits are zero). The
// batch-norm passes give each workgroup its own 128-byte posting line
// (kMeetLine 64-bit slots).
constexpr uint64_t kMeetKey = 0xFFF8DEADBEEF0001ull;
constexpr uint32_t kMeetLine = 16;

// What a one-launch batch-norm pass that gave up waiting for the other
// workgroups of its channel writes to the device's time-out flag
// (take_barrier_timeout names it).
enum : uint32_t { kTimeoutFwdCoop = 1, kTimeoutBwdCoop = 2, kTimeoutBwdReg = 3 };

// How a channel reduction is split, from the shape only (so a shape always
// reduces in the same order on any GPU). A workgroup streams at most
// ~43 GB/s, so one 1024-thread workgroup per channel reaches ~5.5 TB/s with
// 128 channels and ~6.4 TB/s with 256; splitting each channel over ~2048
// workgroups reaches ~6.4 TB/s but costs a second (finalize) launch of
// ~4 us. Hence:
//  * filters >= 256, or filters >= 128 with at most 160 MB to read: one
//    workgroup per channel and one launch (1024 threads for long channels);
//  * otherwise about 2048 workgroups of >= 4096 elements, then the finalize
//    launch. `sums` f64 partials per workgroup must fit the scratch.
#ifndef DKZ_ONE_LAUNCH_MAX_BYTES
#define DKZ_ONE_LAUNCH_MAX_BYTES 160000000ull
#endif
inline uint32_t pick_split(uint32_t filters, uint32_t chan_len, uint32_t streams, uint32_t sums = 1,
                           uint32_t target = 2048, uint32_t min_chunk = 4096) {
    const uint64_t bytes = (uint64_t)4 * streams * filters * chan_len;
    if (filters >= 256 || (filters >= 128 && bytes <= DKZ_ONE_LAUNCH_MAX_BYTES)) return 1;
    uint32_t k = div_up(target, filters);
    const uint32_t kmax = chan_len / min_chunk > 1 ? chan_len / min_chunk : 1;
    if (k > kmax) k = kmax;
    while (k > 1 && (uint64_t)filters * k * sums > kScratchPartials) --k;
    return k < 1 ? 1 : k;
}

// Geometry for splitting each channel of L = batch*spatial elements over K
// workgroups. `vec`: chunks are whole float4s. K may shrink so that no
// workgroup is left empty.
inline RedGeom make_red_geom(uint32_t F, uint32_t S, uint32_t L, uint32_t K, bool vec) {
    uint32_t chunk = L == 0 ? 0 : div_up(L, K);
    if (vec) chunk = (chunk + 3) & ~3u;
    K = chunk > 0 ? div_up(L, chunk) : 1;
    return RedGeom{S, L, chunk, K, (F - 1) * S, make_fastdiv(K), make_fastdiv(S == 0 ? 1 : S),
                   make_fastdiv(F == 0 ? 1 : F)};
}

}  // namespace dkz
