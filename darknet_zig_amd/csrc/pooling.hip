// pooling.hip -- max pooling forward/backward (src/gpu.zig:725-759, CPU twin
// layers/pooling.zig:59-103). Global average pooling lives in reduce.hip
// (forward) and broadcast.hip (backward).
//
// Forward: out_w = (in_w + pad - size)/stride + 1 (pooling.zig:33-34), the
// window starts at -pad/2, out-of-range taps are skipped, and the first
// maximum under strict '>' wins, starting from -FLT_MAX with index -1. The
// index is the absolute flat index into the batched input.
//
// Backward: the twin scatters prev_delta[idx[o]] += delta[o] over ascending o.
// With stride 1 each input element gathers instead: it visits the outputs
// whose window covers it in ascending o and adds delta[o] whenever idx[o]
// names it. With stride >= 2 (a quarter as many outputs as inputs, or fewer)
// each output lane takes its argmax t, and the lowest output naming t adds all
// of t's contributions. Either way an element with several contributors
// receives them in the twin's order, each element is written by one lane, and
// the result is bit-exact with no atomics. Elements with no contributor are
// not written (0 + -0 would otherwise flip a sign).
//
// From 256 planes the generic shapes go through LDS. Windows of 4 and more
// take a separable forward, several planes a workgroup: a row pass keeps
// each input row's first window maximum and its column, a column pass the
// first of those over the window's rows (2*size taps an output instead of
// size^2, the same first maximum; with stride 1 and sizes 4 to 13, prefix
// and suffix maxima over blocks of `size` make it a few selects an output).
// Smaller windows take one workgroup a plane, every window scanned from the
// plane in LDS. The stride-1 backward stages the indexes and deltas of
// several planes a workgroup before its gather (from windows of 5, for the
// inputs some output names alone); with stride >= 2 one workgroup a plane
// stages the plane of prev_delta with them, updates it in LDS and writes it
// back whole.
//
// Size 2, stride 2, offset 0 with in_w % 4 == 0 and even in_h -- the shape of
// a darknet [maxpool] size=2 stride=2 layer -- has a fast path: each lane owns
// two adjacent outputs and their 2x4 input patch, read and written as two
// float4s (outputs and indexes as float2/int2), all with streaming hints.
#include <float.h>

#include <algorithm>

#include "dkz_device.hpp"
#include "dkz_hints.hpp"
#include "dkz_internal.hpp"

namespace dkz {
namespace {

struct PoolGeom {
    uint32_t h, w, c, oh, ow, size, stride, half_pad;  // window offset is -half_pad
    FastDiv div_w, div_h, div_ow, div_oh, div_size, div_stride;
};

// The generic kernels visit a window's taps (forward) or an element's
// candidate outputs (backward) in batches of TB -- 4 when the window (or the
// candidate set) is at most 2x2, else 9, a whole 3x3 window: a batch's loads
// are all issued before any of them is used.

// ---- generic ----------------------------------------------------------------

// The forward through one workgroup per plane when the plane fits in LDS
// (build-time switch, for measurement).
#ifndef DKZ_POOL_PLANE
#define DKZ_POOL_PLANE 1
#endif
// Floats of LDS a plane workgroup may take (12288: 48 KiB).
#ifndef DKZ_POOL_PLANE_MAX
#define DKZ_POOL_PLANE_MAX 12288
#endif
static_assert(DKZ_POOL_PLANE_MAX * sizeof(float) <= 65536, "a workgroup's dynamic LDS is at most 64 KiB");
// The plane kernels run one workgroup per plane: below this many planes the
// grid would leave most CUs idle, and the per-output kernels (hundreds of
// workgroups) run instead. Measured 3x3/s2 forward / backward, plane path
// against per-output kernels: [1,32,56,56] 4.9 / 9.7 against 2.9 / 4.4 us,
// [1,128,56,56] 5.5 / 9.9 against 3.5 / 5.3, [1,64,104,104] forward 13.9
// against 4.1.
// The 3x3 stride-2 kernels (build-time switch, for measurement).
#ifndef DKZ_POOL_3S2
#define DKZ_POOL_3S2 1
#endif
#ifndef DKZ_POOL_PLANE_MIN
#define DKZ_POOL_PLANE_MIN 256
#endif
#ifndef DKZ_POOL_PLANE_UNROLL
#define DKZ_POOL_PLANE_UNROLL 1
#endif
// The several-planes-a-workgroup kernels (build-time switches, for
// measurement): the separable forward for windows of at least
// DKZ_POOL_SEP_MIN_SIZE, the stride-1 gather backward for windows of at
// least DKZ_POOL_GATHER_MIN_DIM. Measured on [64,512,19,19] stride 1,
// forward / backward us against one workgroup a plane: size 5 120.6 / 162.8
// -> 89.8 / 138.2, size 13 461.9 / 544.6 -> 120.0 / 465.3; the separable
// forward lost on 2x2/s1 [64,512,26,26] (53.4 -> 90.5) and 3x3/s1
// [64,128,56,56] (90.6 -> 120.1), the gather without runs (below) on 2x2/s1
// [64,256,13,13] (17.0 -> 20.3).
#ifndef DKZ_POOL_SEP
#define DKZ_POOL_SEP 1
#endif
#ifndef DKZ_POOL_SEP_MIN_SIZE
#define DKZ_POOL_SEP_MIN_SIZE 4
#endif
#ifndef DKZ_POOL_S1_GATHER
#define DKZ_POOL_S1_GATHER 1
#endif
// Stride-1 windows of 4, 5, 9 and 13 through the separable forward with
// runs of outputs a lane and the window size compiled in. Measured on
// [64,512,19,19], us: size 4 54.0 -> 44.1, 5 89.6 -> 48.0, 9 94.4 -> 61.0,
// 13 121.4 -> 73.7; runs of 2 or 8 outputs were 7-23% slower than 4. The
// same kernel for 2x2 and 3x3 lost to one workgroup a plane except on
// planes of a few hundred elements (3x3/s1 [64,512,19,19] 64.4 -> 40.7,
// 2x2/s1 [64,512,26,26] 54.8 -> 68.3, 3x3/s1 [64,128,56,56] 90.2 -> 99.3).
#ifndef DKZ_POOL_SEP_RUN
#define DKZ_POOL_SEP_RUN 1
#endif
// Stride-1 windows of 4 to 13 through blocks of `size` outputs a lane with
// prefix and suffix maxima (for 4, 5, 9 and 13 instead of runs of 4). Measured on [64,512,19,19], us: size
// 4 43.8 -> 42.3, 5 47.7 -> 43.7, 9 61.9 -> 61.2 (a 19-wide line is two
// full blocks of 9 and one of 1), 13 76.3 -> 53.2.
#ifndef DKZ_POOL_BLOCKS
#define DKZ_POOL_BLOCKS 1
#endif
// The stride-1 gather from windows of DKZ_POOL_GATHER_MIN_DIM; windows of
// 2, 3, 4, 5, 9 and 13 with runs of inputs a lane and the window size
// compiled in. Measured, us: [64,512,19,19] size 5 137.1 -> 61.0, 9 283.8
// -> 132.8, 13 463.5 -> 254.4, 3x3/s1 [64,128,56,56] 155.3 -> 100.6, and
// for 2x2 against one lane an input over global memory [64,256,13,13] 16.7
// -> 14.6, [64,512,26,26] 117.0 -> 66.7; runs of 2 or 8 inputs were
// 2-63% slower than 4.
#ifndef DKZ_POOL_GATHER_MIN_DIM
#define DKZ_POOL_GATHER_MIN_DIM 2
#endif
#ifndef DKZ_POOL_RUN_GATHER
#define DKZ_POOL_RUN_GATHER 1
#endif
// The stride-1 backward through its targets only (the inputs some output
// names), from windows of DKZ_POOL_TARGETS_MIN_DIM. Measured against the
// gather with runs, us: [64,512,19,19] size 5 61.3 -> 53.1, 9 133.9 ->
// 80.2, 13 257.6 -> 121.4; it lost at size 4 (50.6 -> 53.1), 3 (42.1 ->
// 48.2) and 2 ([64,512,26,26] 67.4 -> 93.0), where most inputs are targets.
// Then a lane a target with consecutive targets on consecutive lanes and
// the candidates' deltas loaded with their indexes (a select, no branch):
// size 5 51.6-53.0, 9 66.8, 13 83.1; the targets spread over a workgroup's
// four waves instead cost VALU issue (13: 106.3). From size 4 or 3 it tied
// (48.2 against 49.3) and lost (46.3 against 41.7).
#ifndef DKZ_POOL_S1_TARGETS
#define DKZ_POOL_S1_TARGETS 1
#endif
#ifndef DKZ_POOL_TARGETS_MIN_DIM
#define DKZ_POOL_TARGETS_MIN_DIM 5
#endif
// Elements (input plane elements) a workgroup of those kernels aims at, and
// the fewest workgroups their grid keeps when there are enough planes.
#ifndef DKZ_POOL_SEP_TARGET
#define DKZ_POOL_SEP_TARGET 2048
#endif
#ifndef DKZ_POOL_SEP_MIN_GROUPS
#define DKZ_POOL_SEP_MIN_GROUPS 512
#endif

// Candidate outputs of input (y, x) -- those whose window covers it: rows
// i with i*stride + n - half_pad == y for some n in [0, size), i.e. rows
// [ilo, ihi], and likewise columns [jlo, jhi].
__device__ __forceinline__ void pool_candidates(uint32_t y, uint32_t x, const PoolGeom &g, int &ilo, int &ihi,
                                                int &jlo, int &jhi) {
    const int yp = (int)(y + g.half_pad), xp = (int)(x + g.half_pad);
    const int s = (int)g.stride, sz = (int)g.size;
    ilo = yp - sz + 1 <= 0 ? 0 : (int)fdiv((uint32_t)(yp - sz + s), g.div_stride);  // ceil((yp-sz+1)/s)
    jlo = xp - sz + 1 <= 0 ? 0 : (int)fdiv((uint32_t)(xp - sz + s), g.div_stride);
    ihi = min((int)fdiv((uint32_t)yp, g.div_stride), (int)g.oh - 1);
    jhi = min((int)fdiv((uint32_t)xp, g.div_stride), (int)g.ow - 1);
}

template <int TB>
__global__ __launch_bounds__(kBlock) void maxpool_fwd_kernel(const float *in, float *out, int *idx, PoolGeom g,
                                                             uint32_t out_n) {
    const uint32_t o = blockIdx.x * kBlock + threadIdx.x;
    if (o >= out_n) return;
    uint32_t t = fdiv(o, g.div_ow);
    const uint32_t j = o - t * g.ow;
    uint32_t t2 = fdiv(t, g.div_oh);
    const uint32_t i = t - t2 * g.oh;
    const uint32_t plane = t2;  // k + b*c
    float mx = -FLT_MAX;
    int mi = -1;
    // Taps in the twin's order (window row n, then column m); those outside
    // the input are skipped.
    const uint32_t taps = g.size * g.size;
    for (uint32_t t0 = 0; t0 < taps; t0 += TB) {
        float v[TB];
        uint32_t at[TB];
        bool ok[TB];
#pragma unroll
        for (int u = 0; u < TB; ++u) {
            const uint32_t tap = t0 + u;
            const uint32_t n = fdiv(tap, g.div_size), m = tap - n * g.size;
            const int ch = (int)(i * g.stride + n) - (int)g.half_pad;
            const int cw = (int)(j * g.stride + m) - (int)g.half_pad;
            ok[u] = tap < taps && ch >= 0 && ch < (int)g.h && cw >= 0 && cw < (int)g.w;
            at[u] = (uint32_t)cw + g.w * ((uint32_t)ch + g.h * plane);
            v[u] = ok[u] ? in[at[u]] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < TB; ++u) {
            if (ok[u] && v[u] > mx) {
                mx = v[u];
                mi = (int)at[u];
            }
        }
    }
    out[o] = mx;
    idx[o] = mi;
}

// Forward, one workgroup per input plane (h*w floats, at most
// kPlaneMaxFloats): the plane is read once into LDS (float4s when VEC: the
// planes are 16-byte aligned), then each lane scans its outputs' windows
// from LDS in the twin's order.
constexpr uint32_t kPlaneMaxFloats = DKZ_POOL_PLANE_MAX;

// Copies n 4-byte elements from global memory into LDS, R vectors of four
// (VEC: src and dst 16-byte aligned) or 4R elements a lane at a time: every
// load of a batch (addresses clamped into the array) is issued before the
// first LDS write, so that a workgroup waits out the memory latency once a
// batch rather than once an element. Arrays of at most one element (or
// vector) a lane take a single guarded load.
template <typename T, typename T4, bool VEC, int BS, int R = 4>
__device__ __forceinline__ void stage_to_lds(T *dst, const T *src, uint32_t n) {
    if constexpr (VEC) {
        const uint32_t n4 = n / 4;
        const T4 *s4 = reinterpret_cast<const T4 *>(src);
        T4 *d4 = reinterpret_cast<T4 *>(dst);
        if (n4 <= BS) {
            if (threadIdx.x < n4) d4[threadIdx.x] = s4[threadIdx.x];
        } else {
            for (uint32_t b = threadIdx.x; b < n4; b += R * BS) {
                T4 t[R];
#pragma unroll
                for (int k = 0; k < R; ++k) t[k] = s4[min(b + (uint32_t)(k * BS), n4 - 1)];
#pragma unroll
                for (int k = 0; k < R; ++k)
                    if (b + (uint32_t)(k * BS) < n4) d4[b + k * BS] = t[k];
            }
        }
        for (uint32_t q = n4 * 4 + threadIdx.x; q < n; q += BS) dst[q] = src[q];
    } else if (n <= BS) {
        if (threadIdx.x < n) dst[threadIdx.x] = src[threadIdx.x];
    } else {
        for (uint32_t b = threadIdx.x; b < n; b += 4 * R * BS) {
            T t[4 * R];
#pragma unroll
            for (int k = 0; k < 4 * R; ++k) t[k] = src[min(b + (uint32_t)(k * BS), n - 1)];
#pragma unroll
            for (int k = 0; k < 4 * R; ++k)
                if (b + (uint32_t)(k * BS) < n) dst[b + k * BS] = t[k];
        }
    }
}

// The same for an output plane's indexes and deltas (n each), both arrays'
// loads of a batch issued together.
template <int BS, int R = 2>
__device__ __forceinline__ void stage_pair_to_lds(int *il, float *dl, const int *idx, const float *delta,
                                                  uint32_t n) {
    if (n <= BS) {
        if (threadIdx.x < n) {
            il[threadIdx.x] = idx[threadIdx.x];
            dl[threadIdx.x] = delta[threadIdx.x];
        }
        return;
    }
    for (uint32_t b = threadIdx.x; b < n; b += 4 * R * BS) {
        int ti[4 * R];
        float td[4 * R];
#pragma unroll
        for (int k = 0; k < 4 * R; ++k) {
            const uint32_t q = min(b + (uint32_t)(k * BS), n - 1);
            ti[k] = idx[q];
            td[k] = delta[q];
        }
#pragma unroll
        for (int k = 0; k < 4 * R; ++k) {
            if (b + (uint32_t)(k * BS) < n) {
                il[b + k * BS] = ti[k];
                dl[b + k * BS] = td[k];
            }
        }
    }
}

// S > 0: the window is S x S (its taps unrolled, all reads issued first);
// S == 0: g.size.
template <bool VEC, int S>
__global__ __launch_bounds__(kBlock) void maxpool_plane_fwd_kernel(const float *in, float *out, int *idx, PoolGeom g) {
    extern __shared__ float4 plane_lds4[];
    float *pl = reinterpret_cast<float *>(plane_lds4);
    const uint32_t plane = blockIdx.x, hw = g.h * g.w, ohw = g.oh * g.ow;
    stage_to_lds<float, float4, VEC, kBlock>(pl, in + (size_t)plane * hw, hw);
    __syncthreads();
    for (uint32_t o = threadIdx.x; o < ohw; o += kBlock) {
        const uint32_t i = fdiv(o, g.div_ow), j = o - i * g.ow;
        const int ch0 = (int)(i * g.stride) - (int)g.half_pad, cw0 = (int)(j * g.stride) - (int)g.half_pad;
        float mx = -FLT_MAX;
        int mi = -1;
        if constexpr (S > 0) {
            float v[S * S];
            bool ok[S * S];
#pragma unroll
            for (int n = 0; n < S; ++n)
#pragma unroll
                for (int m = 0; m < S; ++m) {
                    const int ch = ch0 + n, cw = cw0 + m;
                    ok[n * S + m] = ch >= 0 && ch < (int)g.h && cw >= 0 && cw < (int)g.w;
                    v[n * S + m] = ok[n * S + m] ? pl[(uint32_t)ch * g.w + (uint32_t)cw] : 0.0f;
                }
#pragma unroll
            for (int t = 0; t < S * S; ++t) {
                if (ok[t] && v[t] > mx) {
                    mx = v[t];
                    mi = (int)(plane * hw + (uint32_t)(ch0 + t / S) * g.w + (uint32_t)(cw0 + t % S));
                }
            }
            out[(size_t)plane * ohw + o] = mx;
            idx[(size_t)plane * ohw + o] = mi;
            continue;
        }
        for (uint32_t n = 0; n < g.size; ++n) {
            const int ch = ch0 + (int)n;
            if (ch < 0 || ch >= (int)g.h) continue;
            const float *row = pl + (uint32_t)ch * g.w;
            for (uint32_t m = 0; m < g.size; ++m) {
                const int cw = cw0 + (int)m;
                if (cw < 0 || cw >= (int)g.w) continue;
                const float v = row[cw];
                if (v > mx) {
                    mx = v;
                    mi = (int)(plane * hw + (uint32_t)ch * g.w + (uint32_t)cw);
                }
            }
        }
        out[(size_t)plane * ohw + o] = mx;
        idx[(size_t)plane * ohw + o] = mi;
    }
}

template <int TB>
__global__ __launch_bounds__(kBlock) void maxpool_bwd_kernel(const float *delta, float *prev, const int *idx,
                                                             PoolGeom g, uint32_t in_n) {
    const uint32_t e = blockIdx.x * kBlock + threadIdx.x;
    if (e >= in_n) return;
    uint32_t t = fdiv(e, g.div_w);
    const uint32_t x = e - t * g.w;
    const uint32_t t2 = fdiv(t, g.div_h);
    const uint32_t y = t - t2 * g.h;
    const uint32_t plane = t2;
    int ilo, ihi, jlo, jhi;
    pool_candidates(y, x, g, ilo, ihi, jlo, jhi);
    if (ilo > ihi || jlo > jhi) return;
    // Candidates in ascending o (row i, then column j): a batch's indexes are
    // loaded together, then the deltas of those that name e -- and, at the
    // first hit, e's own value -- then the deltas are added in order.
    const uint32_t cnt = (uint32_t)(ihi - ilo + 1) * (uint32_t)(jhi - jlo + 1);
    int ci = ilo, cj = jlo;
    float v = 0.0f;
    bool touched = false;
    for (uint32_t c0 = 0; c0 < cnt; c0 += TB) {
        uint32_t o[TB];
        bool hit[TB];
        float d[TB];
#pragma unroll
        for (int u = 0; u < TB; ++u) {
            const bool ok = c0 + u < cnt;
            o[u] = (uint32_t)cj + g.ow * ((uint32_t)ci + g.oh * plane);
            hit[u] = ok && idx[o[u]] == (int)e;
            if (++cj > jhi) {
                cj = jlo;
                ++ci;
            }
        }
        bool any = false;
#pragma unroll
        for (int u = 0; u < TB; ++u) any = any || hit[u];
        if (any && !touched) v = prev[e];
#pragma unroll
        for (int u = 0; u < TB; ++u) d[u] = hit[u] ? delta[o[u]] : 0.0f;
#pragma unroll
        for (int u = 0; u < TB; ++u) {
            if (hit[u]) {
                touched = true;
                v += d[u];
            }
        }
    }
    if (touched) prev[e] = v;
}

// Backward with stride 1 and windows wider than 2, one workgroup per plane
// (oh*ow outputs, at most kPlaneMaxFloats / 2): the plane's indexes and deltas are read once into
// LDS, then each lane gathers for its inputs -- consecutive across lanes --
// exactly as maxpool_bwd_kernel does, from LDS.
__global__ __launch_bounds__(kBlock) void maxpool_plane_bwd_kernel(const float *delta, float *prev, const int *idx,
                                                                   PoolGeom g) {
    extern __shared__ float4 plane_lds4[];
    const uint32_t plane = blockIdx.x, hw = g.h * g.w, ohw = g.oh * g.ow;
    int *il = reinterpret_cast<int *>(plane_lds4);
    float *dl = reinterpret_cast<float *>(plane_lds4) + ohw;
    stage_pair_to_lds<kBlock>(il, dl, idx + (size_t)plane * ohw, delta + (size_t)plane * ohw, ohw);
    __syncthreads();
    for (uint32_t el = threadIdx.x; el < hw; el += kBlock) {
        const uint32_t y = fdiv(el, g.div_w), x = el - y * g.w;
        int ilo, ihi, jlo, jhi;
        pool_candidates(y, x, g, ilo, ihi, jlo, jhi);
        const uint32_t e = plane * hw + el;
        float v = 0.0f;
        bool touched = false;
        for (int ci = ilo; ci <= ihi; ++ci) {
            for (int cj = jlo; cj <= jhi; ++cj) {
                const uint32_t o = (uint32_t)ci * g.ow + (uint32_t)cj;
                if (il[o] != (int)e) continue;
                if (!touched) v = prev[e];
                touched = true;
                v += dl[o];
            }
        }
        if (touched) prev[e] = v;
    }
}

// ---- several planes a workgroup ----------------------------------------------

// The kernels below take P consecutive planes a workgroup (the last one may
// take fewer), so that planes of a few hundred elements still give every
// lane of a 256-lane workgroup several elements: the planes of one
// workgroup are contiguous in memory, read and written as one run.
constexpr uint32_t kSepBS = 256;

// Separable forward. The workgroup's planes are read into LDS once. A row
// pass takes, for every input row y and output column j, the first maximum
// under strict '>' of the window's columns in that row (value and column;
// -FLT_MAX and -1 when no tap beats -FLT_MAX); a column pass takes, for
// every output, the first of those row maxima over the window's rows under
// the same rule. The twin's scan (window rows, then columns, strict '>',
// from -FLT_MAX) ends on the first tap in row-major order of the window's
// largest values (NaNs never win; -0 and +0 tie), and that tap is the
// first row whose row maximum is one of them, at that row's first column
// holding one: the same value and index. h*ow + oh*ow window scans of
// `size` taps each, against oh*ow scans of size^2. Taps are visited in
// batches of 4 whose loads (clamped into the row) are all issued first.
// VEC: the workgroups' first planes start 16-byte aligned.
template <bool VEC>
__global__ __launch_bounds__(kSepBS) void maxpool_sep_fwd_kernel(const float *in, float *out, int *idx, PoolGeom g,
                                                                 uint32_t planes, uint32_t P) {
    extern __shared__ float4 plane_lds4[];
    const uint32_t plane0 = blockIdx.x * P, np = min(P, planes - plane0);
    const uint32_t hw = g.h * g.w, ohw = g.oh * g.ow;
    float *pl = reinterpret_cast<float *>(plane_lds4);
    float *rmax = pl + P * hw;                               // [P*h][ow]
    int *rarg = reinterpret_cast<int *>(rmax + P * g.h * g.ow);  // [P*h][ow]
    stage_to_lds<float, float4, VEC, kSepBS>(pl, in + (size_t)plane0 * hw, np * hw);
    __syncthreads();
    const int sz = (int)g.size, w = (int)g.w, h = (int)g.h;
    for (uint32_t r = threadIdx.x; r < np * g.h * g.ow; r += kSepBS) {
        const uint32_t q = fdiv(r, g.div_ow), j = r - q * g.ow;  // q = p*h + y
        const int c0 = (int)(j * g.stride) - (int)g.half_pad;
        const int lo = max(c0, 0), n = min(c0 + sz, w) - lo;  // taps [lo, lo + n)
        const float *row = pl + q * g.w;
        float mx = -FLT_MAX;
        int a = -1;
        for (int m0 = 0; m0 < n; m0 += 4) {
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = row[lo + min(m0 + u, n - 1)];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if (m0 + u < n && v[u] > mx) {
                    mx = v[u];
                    a = lo + m0 + u;
                }
            }
        }
        rmax[r] = mx;
        rarg[r] = a;
    }
    __syncthreads();
    const size_t out0 = (size_t)plane0 * ohw;
    for (uint32_t o = threadIdx.x; o < np * ohw; o += kSepBS) {
        const uint32_t q = fdiv(o, g.div_ow), j = o - q * g.ow;  // q = p*oh + i
        const uint32_t p = fdiv(q, g.div_oh), i = q - p * g.oh;
        const int r0 = (int)(i * g.stride) - (int)g.half_pad;
        const int lo = max(r0, 0), n = min(r0 + sz, h) - lo;  // rows [lo, lo + n)
        const float *col = rmax + p * g.h * g.ow + j;
        float mx = -FLT_MAX;
        int best = -1;
        for (int m0 = 0; m0 < n; m0 += 4) {
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = col[(uint32_t)(lo + min(m0 + u, n - 1)) * g.ow];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if (m0 + u < n && v[u] > mx) {
                    mx = v[u];
                    best = lo + m0 + u;
                }
            }
        }
        // a row maximum above -FLT_MAX has a column
        const int a = best < 0 ? -1 : rarg[(p * g.h + (uint32_t)best) * g.ow + j];
        out[out0 + o] = mx;
        idx[out0 + o] = best < 0 ? -1 : (int)((plane0 + p) * hw + (uint32_t)best * g.w + (uint32_t)a);
    }
}

// The separable forward for stride 1 and an S x S window known at compile
// time, each lane taking a run of kRun consecutive outputs: in the row pass
// kRun outputs of one input row from the kRun + S - 1 input values they
// span, in the column pass kRun outputs of one output column from the
// kRun + S - 1 row maxima they span, each value read from LDS once a run
// instead of once a window. Taps outside the input read as -FLT_MAX, which
// never beats the -FLT_MAX start under strict '>' -- the same as skipping
// them. Each output's window is scanned on its own in the twin's order, so
// the results are those of maxpool_sep_fwd_kernel.
constexpr int kRun = 4;

template <bool VEC, int S>
__global__ __launch_bounds__(kSepBS) void maxpool_sep_run_fwd_kernel(const float *in, float *out, int *idx,
                                                                     PoolGeom g, uint32_t planes, uint32_t P,
                                                                     FastDiv div_ow_runs, FastDiv div_oh_runs) {
    extern __shared__ float4 plane_lds4[];
    constexpr int T = kRun + S - 1;
    const uint32_t plane0 = blockIdx.x * P, np = min(P, planes - plane0);
    const uint32_t hw = g.h * g.w, ohw = g.oh * g.ow;
    const uint32_t ow_runs = (g.ow + kRun - 1) / kRun, oh_runs = (g.oh + kRun - 1) / kRun;
    float *pl = reinterpret_cast<float *>(plane_lds4);
    float *rmax = pl + P * hw;                                   // [P*h][ow]
    int *rarg = reinterpret_cast<int *>(rmax + P * g.h * g.ow);  // [P*h][ow]
    stage_to_lds<float, float4, VEC, kSepBS>(pl, in + (size_t)plane0 * hw, np * hw);
    __syncthreads();
    const int w = (int)g.w, h = (int)g.h, hp = (int)g.half_pad;
    for (uint32_t r = threadIdx.x; r < np * g.h * ow_runs; r += kSepBS) {
        const uint32_t q = fdiv(r, div_ow_runs), j0 = (r - q * ow_runs) * kRun;  // q = p*h + y
        const int c0 = (int)j0 - hp;
        const float *row = pl + q * g.w;
        float v[T];
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int c = c0 + t;
            const float x = row[min(max(c, 0), w - 1)];
            v[t] = c >= 0 && c < w ? x : -FLT_MAX;
        }
#pragma unroll
        for (int k = 0; k < kRun; ++k) {
            float mx = -FLT_MAX;
            int a = -1;
#pragma unroll
            for (int m = 0; m < S; ++m) {
                if (v[k + m] > mx) {
                    mx = v[k + m];
                    a = k + m;
                }
            }
            if (j0 + k < g.ow) {
                rmax[q * g.ow + j0 + k] = mx;
                rarg[q * g.ow + j0 + k] = a < 0 ? -1 : c0 + a;
            }
        }
    }
    __syncthreads();
    for (uint32_t r = threadIdx.x; r < np * oh_runs * g.ow; r += kSepBS) {
        const uint32_t q = fdiv(r, g.div_ow), j = r - q * g.ow;  // q = p*oh_runs + run
        const uint32_t p = fdiv(q, div_oh_runs), i0 = (q - p * oh_runs) * kRun;
        const int r0 = (int)i0 - hp;
        const float *col = rmax + p * g.h * g.ow + j;
        float v[T];
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int ch = r0 + t;
            const float x = col[(uint32_t)min(max(ch, 0), h - 1) * g.ow];
            v[t] = ch >= 0 && ch < h ? x : -FLT_MAX;
        }
        const size_t o_plane = (size_t)(plane0 + p) * ohw;
#pragma unroll
        for (int k = 0; k < kRun; ++k) {
            float mx = -FLT_MAX;
            int best = -1;
#pragma unroll
            for (int m = 0; m < S; ++m) {
                if (v[k + m] > mx) {
                    mx = v[k + m];
                    best = k + m;
                }
            }
            if (i0 + k < g.oh) {
                // a row that won is inside the input and has a column
                const uint32_t ch = best < 0 ? 0u : (uint32_t)(r0 + best);
                const int a = rarg[(p * g.h + ch) * g.ow + j];
                out[o_plane + (i0 + k) * g.ow + j] = mx;
                idx[o_plane + (i0 + k) * g.ow + j] =
                    best < 0 ? -1 : (int)((plane0 + p) * hw + ch * g.w + (uint32_t)a);
            }
        }
    }
}

// The separable forward for stride 1 and an S x S window known at compile
// time, each lane taking a block of S consecutive outputs of a line (an
// input row in the row pass, an output column in the column pass) from the
// 2S values from the block's first window start: the suffix maxima of the
// first S values and the prefix maxima of the next S, so that the window
// starting k into the block is the suffix from k joined with the prefix up
// to k - 1 -- about three selects a value and three an output, whatever S
// (van Herk's and Gil and Werman's sliding maximum). The twin's first
// maximum is kept: the suffix scan (right to left) moves to an equal value
// once it holds one, the prefix scan (left to right) only to a greater one,
// and the join takes the prefix part, which lies after the suffix part,
// only when it is greater. Taps outside the input read as -FLT_MAX, which
// is never taken: the suffix scan moves to an equal value only once it holds
// a tap, and NaNs compare false.
template <int S>
struct BlockMax {
    float sv[S], pv[S];
    int si[S], pi[S];  // offsets into the 2S values, -1 for none

    __device__ __forceinline__ void scan(const float (&v)[2 * S]) {
        float m = -FLT_MAX;
        int a = -1;
#pragma unroll
        for (int k = S - 1; k >= 0; --k) {
            if (v[k] > m || (v[k] == m && a >= 0)) {
                m = v[k];
                a = k;
            }
            sv[k] = m;
            si[k] = a;
        }
        m = -FLT_MAX;
        a = -1;
#pragma unroll
        for (int k = 0; k < S; ++k) {
            if (v[S + k] > m) {
                m = v[S + k];
                a = S + k;
            }
            pv[k] = m;
            pi[k] = a;
        }
    }
    // the window starting k into the block
    __device__ __forceinline__ void window(int k, float &m, int &a) const {
        m = sv[k];
        a = si[k];
        if (k >= 1 && pv[k - 1] > m) {
            m = pv[k - 1];
            a = pi[k - 1];
        }
    }
};

template <bool VEC, int S>
__global__ __launch_bounds__(kSepBS) void maxpool_sep_block_fwd_kernel(const float *in, float *out, int *idx,
                                                                       PoolGeom g, uint32_t planes, uint32_t P,
                                                                       FastDiv div_ow_blocks, FastDiv div_oh_blocks) {
    extern __shared__ float4 plane_lds4[];
    const uint32_t plane0 = blockIdx.x * P, np = min(P, planes - plane0);
    const uint32_t hw = g.h * g.w, ohw = g.oh * g.ow;
    const uint32_t ow_blocks = (g.ow + S - 1) / S, oh_blocks = (g.oh + S - 1) / S;
    float *pl = reinterpret_cast<float *>(plane_lds4);
    float *rmax = pl + P * hw;                                   // [P*h][ow]
    int *rarg = reinterpret_cast<int *>(rmax + P * g.h * g.ow);  // [P*h][ow]
    stage_to_lds<float, float4, VEC, kSepBS>(pl, in + (size_t)plane0 * hw, np * hw);
    __syncthreads();
    const int w = (int)g.w, h = (int)g.h, hp = (int)g.half_pad;
    for (uint32_t r = threadIdx.x; r < np * g.h * ow_blocks; r += kSepBS) {
        const uint32_t q = fdiv(r, div_ow_blocks), j0 = (r - q * ow_blocks) * S;  // q = p*h + y
        const int c0 = (int)j0 - hp;
        const float *row = pl + q * g.w;
        float v[2 * S];
#pragma unroll
        for (int t = 0; t < 2 * S; ++t) {
            const int c = c0 + t;
            const float x = row[min(max(c, 0), w - 1)];
            v[t] = c >= 0 && c < w ? x : -FLT_MAX;
        }
        BlockMax<S> bm;
        bm.scan(v);
#pragma unroll
        for (int k = 0; k < S; ++k) {
            if (j0 + k < g.ow) {
                float m;
                int a;
                bm.window(k, m, a);
                rmax[q * g.ow + j0 + k] = m;
                rarg[q * g.ow + j0 + k] = a < 0 ? -1 : c0 + a;
            }
        }
    }
    __syncthreads();
    for (uint32_t r = threadIdx.x; r < np * oh_blocks * g.ow; r += kSepBS) {
        const uint32_t q = fdiv(r, g.div_ow), j = r - q * g.ow;  // q = p*oh_blocks + block
        const uint32_t p = fdiv(q, div_oh_blocks), i0 = (q - p * oh_blocks) * S;
        const int r0 = (int)i0 - hp;
        const float *col = rmax + p * g.h * g.ow + j;
        float v[2 * S];
#pragma unroll
        for (int t = 0; t < 2 * S; ++t) {
            const int ch = r0 + t;
            const float x = col[(uint32_t)min(max(ch, 0), h - 1) * g.ow];
            v[t] = ch >= 0 && ch < h ? x : -FLT_MAX;
        }
        BlockMax<S> bm;
        bm.scan(v);
        const size_t o_plane = (size_t)(plane0 + p) * ohw;
#pragma unroll
        for (int k = 0; k < S; ++k) {
            if (i0 + k < g.oh) {
                float m;
                int best;
                bm.window(k, m, best);
                // a row that won is inside the input and has a column
                const uint32_t ch = best < 0 ? 0u : (uint32_t)(r0 + best);
                const int a = rarg[(p * g.h + ch) * g.ow + j];
                out[o_plane + (i0 + k) * g.ow + j] = m;
                idx[o_plane + (i0 + k) * g.ow + j] =
                    best < 0 ? -1 : (int)((plane0 + p) * hw + ch * g.w + (uint32_t)a);
            }
        }
    }
}

// Backward with stride 1, P planes a workgroup: the planes' indexes and
// deltas are read into LDS once, then each lane gathers for its inputs --
// consecutive across lanes -- as maxpool_bwd_kernel does (candidate outputs
// in ascending order, delta added whenever the index names the input), a
// window row at a time, the indexes of 4 candidates loaded together.
// prev_delta is read for every input, a lane's next 8 inputs' loads issued
// together (the first batch before the barrier), and written only where
// some output names the input.
__global__ __launch_bounds__(kSepBS) void maxpool_s1_gather_kernel(const float *delta, float *prev, const int *idx,
                                                                   PoolGeom g, uint32_t planes, uint32_t P) {
    extern __shared__ float4 plane_lds4[];
    const uint32_t plane0 = blockIdx.x * P, np = min(P, planes - plane0);
    const uint32_t hw = g.h * g.w, ohw = g.oh * g.ow;
    int *il = reinterpret_cast<int *>(plane_lds4);  // [P][oh][ow]
    float *dl = reinterpret_cast<float *>(plane_lds4) + P * ohw;
    const size_t o0 = (size_t)plane0 * ohw;
    stage_pair_to_lds<kSepBS>(il, dl, idx + o0, delta + o0, np * ohw);
    const uint32_t e0 = plane0 * hw, n_el = np * hw;
    // prev_delta of the lane's next kPrev inputs, loaded together; the
    // first batch's loads are in flight across the barrier
    constexpr int kPrev = 8;
    float pv[kPrev];
#pragma unroll
    for (int k = 0; k < kPrev; ++k) pv[k] = prev[e0 + min(threadIdx.x + (uint32_t)(k * kSepBS), n_el - 1)];
    __syncthreads();
#pragma unroll 1
    for (uint32_t el = threadIdx.x, k = 0; el < n_el; el += kSepBS) {
        float v = pv[0];
#pragma unroll
        for (int u = 0; u + 1 < kPrev; ++u) pv[u] = pv[u + 1];
        if (++k == kPrev) {
            k = 0;
#pragma unroll
            for (int u = 0; u < kPrev; ++u)
                pv[u] = prev[e0 + min(el + (uint32_t)((u + 1) * kSepBS), n_el - 1)];
        }
        const uint32_t q = fdiv(el, g.div_w), x = el - q * g.w;  // q = p*h + y
        const uint32_t p = fdiv(q, g.div_h), y = q - p * g.h;
        const int e = (int)(e0 + el);
        int ilo, ihi, jlo, jhi;
        pool_candidates(y, x, g, ilo, ihi, jlo, jhi);
        const int n = jhi - jlo + 1;
        bool touched = false;
        for (int ci = ilo; ci <= ihi; ++ci) {
            const uint32_t rb = p * ohw + (uint32_t)ci * g.ow + (uint32_t)jlo;
            for (int m0 = 0; m0 < n; m0 += 4) {
                int ix[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) ix[u] = il[rb + (uint32_t)min(m0 + u, n - 1)];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    if (m0 + u < n && ix[u] == e) {
                        v += dl[rb + (uint32_t)(m0 + u)];
                        touched = true;
                    }
                }
            }
        }
        if (touched) prev[e] = v;
    }
}

// The stride-1 backward through the inputs that some output names ("targets"),
// P planes a workgroup: the planes' indexes and deltas are staged in LDS,
// each output marks its index in an LDS array of the planes' inputs (an
// exchange, so that exactly one marker appends the input to a list of
// targets), and a lane a target then gathers as maxpool_s1_gather_kernel
// does -- candidate outputs in ascending order, each delta whose index
// names the target added to its prev_delta. Inputs that no output names are
// neither read nor written; with large windows they are nearly all of them
// (a 13x13 window's maximum is shared by many outputs), so the size^2
// candidate checks run for a few inputs a plane instead of every one. Which
// lane takes which target varies from run to run; what each target receives,
// and in which order, does not.
// TB: candidates of a window row whose indexes and deltas are loaded
// together (the host takes 4 or 8, whichever loads fewer for the window's
// width, 8 on a tie).
template <int TB>
__global__ __launch_bounds__(kSepBS) void maxpool_s1_target_gather_kernel(const float *delta, float *prev,
                                                                          const int *idx, PoolGeom g,
                                                                          uint32_t planes, uint32_t P) {
    extern __shared__ float4 plane_lds4[];
    __shared__ uint32_t n_targets;
    const uint32_t plane0 = blockIdx.x * P, np = min(P, planes - plane0);
    const uint32_t hw = g.h * g.w, ohw = g.oh * g.ow, n_el = np * hw, n_out = np * ohw;
    int *il = reinterpret_cast<int *>(plane_lds4);                   // [P][oh][ow]
    float *dl = reinterpret_cast<float *>(plane_lds4) + P * ohw;     // [P][oh][ow]
    uint32_t *mark = reinterpret_cast<uint32_t *>(dl + P * ohw);     // [P][h][w]
    uint32_t *list = mark + P * hw;                                  // the targets, plane-relative
    const size_t o0 = (size_t)plane0 * ohw;
    const uint32_t e0 = plane0 * hw;
    for (uint32_t q = threadIdx.x; q < n_el; q += kSepBS) mark[q] = 0u;
    if (threadIdx.x == 0) n_targets = 0u;
    stage_pair_to_lds<kSepBS>(il, dl, idx + o0, delta + o0, n_out);
    __syncthreads();
    for (uint32_t o = threadIdx.x; o < n_out; o += kSepBS) {
        const int tv = il[o];
        // consecutive outputs often name one input: the first of such a run
        // marks it (fewer exchanges on one LDS word; [64,512,19,19] size 13
        // 86.0 -> 77.0 us, 9 67.8 -> 62.6)
        if (o > 0 && il[o - 1] == tv) continue;
        const int64_t t = (int64_t)tv - (int64_t)e0;  // -1 and other planes' inputs fall outside
        if (t >= 0 && t < (int64_t)n_el && atomicExch(&mark[t], 1u) == 0u) list[atomicAdd(&n_targets, 1u)] = (uint32_t)t;
    }
    __syncthreads();
    const uint32_t nt = n_targets;
    // consecutive lanes take consecutive targets: a workgroup's few targets
    // fill as few waves as they can, whose candidate scans then cost the
    // least VALU issue
    for (uint32_t k = threadIdx.x; k < nt; k += kSepBS) {
        const uint32_t el = list[k];
        const uint32_t q = fdiv(el, g.div_w), x = el - q * g.w;  // q = p*h + y
        const uint32_t p = fdiv(q, g.div_h), y = q - p * g.h;
        const int e = (int)(e0 + el);
        float v = prev[e];
        int ilo, ihi, jlo, jhi;
        pool_candidates(y, x, g, ilo, ihi, jlo, jhi);
        const int n = jhi - jlo + 1;
        for (int ci = ilo; ci <= ihi; ++ci) {
            const uint32_t rb = p * ohw + (uint32_t)ci * g.ow + (uint32_t)jlo;
            for (int m0 = 0; m0 < n; m0 += TB) {
                int ix[TB];
                float d[TB];
#pragma unroll
                for (int u = 0; u < TB; ++u) {
                    const uint32_t c = rb + (uint32_t)min(m0 + u, n - 1);
                    ix[u] = il[c];
                    d[u] = dl[c];
                }
#pragma unroll
                for (int u = 0; u < TB; ++u) v = m0 + u < n && ix[u] == e ? v + d[u] : v;
            }
        }
        prev[e] = v;  // a target: some output names it
    }
}

// The stride-1 gather for an S x S window known at compile time, each lane
// taking a run of kRunG consecutive inputs of one row: for each candidate
// output row (ascending) the kRunG + S - 1 candidate columns' indexes and
// deltas are read from LDS once for the run, and each input adds, in
// ascending column order, the deltas whose index names it -- selected, not
// branched on, so a candidate costs a compare, an add and a select. The
// order of the adds is maxpool_s1_gather_kernel's (the twin's), and an
// input is written only where some output names it. prev_delta of the
// lane's next run is loaded while the current one gathers.
constexpr int kRunG = 4;

template <int S>
__global__ __launch_bounds__(kSepBS) void maxpool_s1_run_gather_kernel(const float *delta, float *prev,
                                                                       const int *idx, PoolGeom g, uint32_t planes,
                                                                       uint32_t P, FastDiv div_w_runs) {
    extern __shared__ float4 plane_lds4[];
    constexpr int T = kRunG + S - 1;
    const uint32_t plane0 = blockIdx.x * P, np = min(P, planes - plane0);
    const uint32_t hw = g.h * g.w, ohw = g.oh * g.ow, w_runs = (g.w + kRunG - 1) / kRunG;
    int *il = reinterpret_cast<int *>(plane_lds4);  // [P][oh][ow]
    float *dl = reinterpret_cast<float *>(plane_lds4) + P * ohw;
    const size_t o0 = (size_t)plane0 * ohw;
    stage_pair_to_lds<kSepBS>(il, dl, idx + o0, delta + o0, np * ohw);
    const uint32_t e0 = plane0 * hw, n_el = np * hw, n_runs = np * g.h * w_runs;
    const int hp = (int)g.half_pad, oh = (int)g.oh, ow = (int)g.ow;
    // the lane's first run's prev_delta, in flight across the barrier
    auto run_elems = [&](uint32_t r, uint32_t *el) {
        const uint32_t q = fdiv(r, div_w_runs), x0 = (r - q * w_runs) * kRunG;  // q = p*h + y
#pragma unroll
        for (int k = 0; k < kRunG; ++k) el[k] = q * g.w + x0 + k;  // x0 + k may pass the row's end
    };
    float pn[kRunG];
    {
        const uint32_t r = min(threadIdx.x, n_runs - 1);
        uint32_t el[kRunG];
        run_elems(r, el);
#pragma unroll
        for (int k = 0; k < kRunG; ++k) pn[k] = prev[e0 + min(el[k], n_el - 1)];
    }
    __syncthreads();
#pragma unroll 1
    for (uint32_t r = threadIdx.x; r < n_runs; r += kSepBS) {
        float v[kRunG];
#pragma unroll
        for (int k = 0; k < kRunG; ++k) v[k] = pn[k];
        {
            uint32_t el[kRunG];
            run_elems(min(r + kSepBS, n_runs - 1), el);
#pragma unroll
            for (int k = 0; k < kRunG; ++k) pn[k] = prev[e0 + min(el[k], n_el - 1)];
        }
        const uint32_t q = fdiv(r, div_w_runs), x0 = (r - q * w_runs) * kRunG;
        const uint32_t p = fdiv(q, g.div_h), y = q - p * g.h;
        const int jb = (int)x0 + hp - S + 1;  // candidate column of t = 0
        const int ilo = max((int)y + hp - S + 1, 0), ihi = min((int)y + hp, oh - 1);
        int e[kRunG];
#pragma unroll
        for (int k = 0; k < kRunG; ++k) e[k] = (int)(e0 + q * g.w + x0 + k);
        bool touched[kRunG];
#pragma unroll
        for (int k = 0; k < kRunG; ++k) touched[k] = false;
        for (int ci = ilo; ci <= ihi; ++ci) {
            const int *irow = il + p * ohw + (uint32_t)ci * g.ow;
            const float *drow = dl + p * ohw + (uint32_t)ci * g.ow;
            int ix[T];
            float d[T];
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const int j = jb + t;
                const uint32_t jc = (uint32_t)min(max(j, 0), ow - 1);
                ix[t] = j >= 0 && j < ow ? irow[jc] : -1;  // -1 names no input
                d[t] = drow[jc];
            }
#pragma unroll
            for (int k = 0; k < kRunG; ++k) {
#pragma unroll
                for (int m = 0; m < S; ++m) {
                    const bool hit = ix[k + m] == e[k];
                    v[k] = hit ? v[k] + d[k + m] : v[k];
                    touched[k] = touched[k] || hit;
                }
            }
        }
#pragma unroll
        for (int k = 0; k < kRunG; ++k)
            if (touched[k] && x0 + k < g.w) prev[e[k]] = v[k];
    }
}

// Backward, one lane per output (stride >= 2, where outputs are a quarter of
// the inputs or fewer): output o names input t = idx[o]. Of the outputs that
// name t, the lowest o -- the first to add into t in the twin's ascending
// scatter -- adds all of them in order, so each touched input is written by
// exactly one lane and untouched inputs are not visited. A lane finds out
// whether it is that output from the indexes of t's candidate outputs below o.
template <int TB>
__global__ __launch_bounds__(kBlock) void maxpool_bwd_out_kernel(const float *delta, float *prev, const int *idx,
                                                                 PoolGeom g, uint32_t out_n, uint32_t in_n) {
    const uint32_t o = blockIdx.x * kBlock + threadIdx.x;
    if (o >= out_n) return;
    const int tv = idx[o];
    if (tv < 0 || (uint32_t)tv >= in_n) return;  // -1: no tap of o's window was taken
    const uint32_t t = (uint32_t)tv;
    const uint32_t q = fdiv(t, g.div_w);
    const uint32_t x = t - q * g.w;
    const uint32_t plane = fdiv(q, g.div_h);
    const uint32_t y = q - plane * g.h;
    int ilo, ihi, jlo, jhi;
    pool_candidates(y, x, g, ilo, ihi, jlo, jhi);
    if (ilo > ihi || jlo > jhi) return;
    const uint32_t cnt = (uint32_t)(ihi - ilo + 1) * (uint32_t)(jhi - jlo + 1);
    const float p0 = prev[t];
    float v = 0.0f;
    bool mine = false;
    int ci = ilo, cj = jlo;
    for (uint32_t c0 = 0; c0 < cnt; c0 += TB) {
        uint32_t oc[TB];
        int ix[TB];
        bool ok[TB];
#pragma unroll
        for (int u = 0; u < TB; ++u) {
            ok[u] = c0 + u < cnt;
            oc[u] = (uint32_t)cj + g.ow * ((uint32_t)ci + g.oh * plane);
            ix[u] = ok[u] && oc[u] != o ? idx[oc[u]] : tv;
            if (++cj > jhi) {
                cj = jlo;
                ++ci;
            }
        }
        float d[TB];
#pragma unroll
        for (int u = 0; u < TB; ++u) d[u] = ok[u] && oc[u] >= o && ix[u] == tv ? delta[oc[u]] : 0.0f;
#pragma unroll
        for (int u = 0; u < TB; ++u) {
            if (!ok[u] || ix[u] != tv) continue;
            if (oc[u] < o) return;  // a lower output adds into t first
            if (oc[u] == o) {
                v = p0 + d[u];
                mine = true;
            } else if (mine) {
                v += d[u];
            }
        }
    }
    if (mine) prev[t] = v;
}

// Backward with stride >= 2, one workgroup per plane (h*w inputs plus oh*ow
// outputs within kPlaneMaxFloats): the plane of prev_delta and the outputs'
// indexes and deltas are read into LDS, each output lane applies
// maxpool_bwd_out_kernel's rule there (the lowest output naming an input
// adds all of that input's deltas in order, so every touched element has
// one writer), and the plane is written back whole (untouched elements keep
// their bits). VEC: the prev_delta planes are 16-byte aligned.
template <bool VEC>
__global__ __launch_bounds__(kBlock) void maxpool_plane_bwd_out_kernel(const float *delta, float *prev, const int *idx,
                                                                       PoolGeom g) {
    extern __shared__ float4 plane_lds4[];
    const uint32_t plane = blockIdx.x, hw = g.h * g.w, ohw = g.oh * g.ow;
    float *pl = reinterpret_cast<float *>(plane_lds4);
    int *il = reinterpret_cast<int *>(pl + hw);
    float *dl = pl + hw + ohw;
    float *dst = prev + (size_t)plane * hw;
    stage_to_lds<float, float4, VEC, kBlock>(pl, dst, hw);
    stage_pair_to_lds<kBlock>(il, dl, idx + (size_t)plane * ohw, delta + (size_t)plane * ohw, ohw);
    __syncthreads();
    const int base = (int)(plane * hw);
    for (uint32_t o = threadIdx.x; o < ohw; o += kBlock) {
        const int tv = il[o] - base;
        if (tv < 0 || (uint32_t)tv >= hw) continue;  // -1, or outside this plane
        const uint32_t t = (uint32_t)tv;
        const uint32_t y = fdiv(t, g.div_w), x = t - y * g.w;
        int ilo, ihi, jlo, jhi;
        pool_candidates(y, x, g, ilo, ihi, jlo, jhi);
        bool mine = false, lower = false;
        float v = 0.0f;
        for (int ci = ilo; ci <= ihi && !lower; ++ci) {
            for (int cj = jlo; cj <= jhi; ++cj) {
                const uint32_t oc = (uint32_t)ci * g.ow + (uint32_t)cj;
                if (il[oc] != il[o]) continue;
                if (oc < o) {
                    lower = true;  // a lower output adds into t first
                    break;
                }
                if (oc == o) {
                    v = pl[t] + dl[oc];
                    mine = true;
                } else if (mine) {
                    v += dl[oc];
                }
            }
        }
        if (mine && !lower) pl[t] = v;
    }
    __syncthreads();
    if constexpr (VEC) {
        for (uint32_t q = threadIdx.x; q < hw / 4; q += kBlock) reinterpret_cast<float4 *>(dst)[q] = plane_lds4[q];
    } else {
        for (uint32_t q = threadIdx.x; q < hw; q += kBlock) dst[q] = pl[q];
    }
}

// ---- 2x2, stride 2, offset 0 ------------------------------------------------

__device__ __forceinline__ void max_tap(float val, int index, float &mx, int &mi) {
    if (val > mx) {
        mx = val;
        mi = index;
    }
}

// q indexes output pairs; ow is even so a pair never straddles a row.
// Nontemporal accesses per DKZ_HINT_MAXPOOL_FWD / _BWD (dkz_hints.hpp).
constexpr int kHf = DKZ_HINT_MAXPOOL_FWD, kHb = DKZ_HINT_MAXPOOL_BWD;
constexpr int kH3f = DKZ_HINT_MAXPOOL3_FWD, kH3b = DKZ_HINT_MAXPOOL3_BWD;

__global__ __launch_bounds__(kBlock) void maxpool2_fwd_kernel(const float *in, float *out, int *idx,
                                                              PoolGeom g, uint32_t pairs) {
    const uint32_t q = blockIdx.x * kBlock + threadIdx.x;
    if (q >= pairs) return;
    const uint32_t o = 2 * q;
    const uint32_t t = fdiv(o, g.div_ow);
    const uint32_t j = o - t * g.ow;
    const uint32_t plane = fdiv(t, g.div_oh);
    const uint32_t i = t - plane * g.oh;
    const uint32_t r0 = (plane * g.h + 2 * i) * g.w + 2 * j;  // first tap of output j
    const uint32_t r1 = r0 + g.w;
    const float4 a = ld4<(kHf & 1) != 0>(in, r0 >> 2);
    const float4 b = ld4<(kHf & 1) != 0>(in, r1 >> 2);
    float m0 = -FLT_MAX, m1 = -FLT_MAX;
    int i0 = -1, i1 = -1;
    max_tap(a.x, (int)r0, m0, i0);
    max_tap(a.y, (int)r0 + 1, m0, i0);
    max_tap(b.x, (int)r1, m0, i0);
    max_tap(b.y, (int)r1 + 1, m0, i0);
    max_tap(a.z, (int)r0 + 2, m1, i1);
    max_tap(a.w, (int)r0 + 3, m1, i1);
    max_tap(b.z, (int)r1 + 2, m1, i1);
    max_tap(b.w, (int)r1 + 3, m1, i1);
    st2<(kHf & 2) != 0>(out, q, make_float2(m0, m1));
    st2i<(kHf & 4) != 0>(idx, q, make_int2(i0, i1));
}

__device__ __forceinline__ float add_if(float p, int want, int have, float d) {
    return have == want ? p + d : p;
}

__global__ __launch_bounds__(kBlock) void maxpool2_bwd_kernel(const float *delta, float *prev, const int *idx,
                                                              PoolGeom g, uint32_t pairs) {
    const uint32_t q = blockIdx.x * kBlock + threadIdx.x;
    if (q >= pairs) return;
    const uint32_t o = 2 * q;
    const uint32_t t = fdiv(o, g.div_ow);
    const uint32_t j = o - t * g.ow;
    const uint32_t plane = fdiv(t, g.div_oh);
    const uint32_t i = t - plane * g.oh;
    const uint32_t r0 = (plane * g.h + 2 * i) * g.w + 2 * j;
    const uint32_t r1 = r0 + g.w;
    const float2 d = ld2<(kHb & 1) != 0>(delta, q);
    const int2 k = ld2i<(kHb & 1) != 0>(idx, q);
    float4 a = ld4<(kHb & 2) != 0>(prev, r0 >> 2);
    float4 b = ld4<(kHb & 2) != 0>(prev, r1 >> 2);
    // Each input of the patch has exactly one candidate output: j for the
    // first two columns, j+1 for the last two.
    a.x = add_if(a.x, (int)r0, k.x, d.x);
    a.y = add_if(a.y, (int)r0 + 1, k.x, d.x);
    b.x = add_if(b.x, (int)r1, k.x, d.x);
    b.y = add_if(b.y, (int)r1 + 1, k.x, d.x);
    a.z = add_if(a.z, (int)r0 + 2, k.y, d.y);
    a.w = add_if(a.w, (int)r0 + 3, k.y, d.y);
    b.z = add_if(b.z, (int)r1 + 2, k.y, d.y);
    b.w = add_if(b.w, (int)r1 + 3, k.y, d.y);
    st4<(kHb & 4) != 0>(prev, r0 >> 2, a);
    st4<(kHb & 4) != 0>(prev, r1 >> 2, b);
}

// ---- 3x3, stride 2, window offset -P0 (P0 = pad/2 = 0 or 1) -----------------
//
// For ow % 4 == 0 and w == 2*ow (darknet's size=3 stride=2 layer with pad 1
// or 2 on a width that is a multiple of 8).
//
// Forward: a lane owns outputs x0..x0+3 (x0 = 4*xq) of output row y; their
// windows span the 9 input columns 2*x0 - P0 .. 2*x0 - P0 + 8 of input rows
// 2y - P0 .. 2y - P0 + 2, read per row as two aligned float4s (columns
// 2*x0 .. 2*x0 + 7) and the one column beside them. Columns and rows outside
// the input read a clamped in-range address and count as -FLT_MAX, which
// strict '>' never takes: the twin's scan (rows outer, columns inner) and its
// first-maximum index, bit for bit.
template <int P0>
__global__ __launch_bounds__(kBlock) void maxpool3s2_fwd_kernel(const float *in, float *out, int *idx, PoolGeom g,
                                                                FastDiv div_qw, uint32_t lanes) {
    const uint32_t q = blockIdx.x * kBlock + threadIdx.x;
    if (q >= lanes) return;
    const uint32_t t = fdiv(q, div_qw);  // plane * oh + y
    const uint32_t xq = q - t * (g.ow >> 2);
    const uint32_t plane = fdiv(t, g.div_oh);
    const uint32_t y = t - plane * g.oh;
    const uint32_t c0 = 8 * xq;                      // first column of the float4 pair
    const int ce = P0 == 1 ? (int)c0 - 1 : (int)c0 + 8;  // the column beside them
    const bool ce_ok = ce >= 0 && ce < (int)g.w;
    float v[3][9];
    int rowi[3];
#pragma unroll
    for (int kh = 0; kh < 3; ++kh) {
        const int r = 2 * (int)y - P0 + kh;
        const bool r_ok = r >= 0 && r < (int)g.h;
        const uint32_t rc = r_ok ? (uint32_t)r : 0u;
        const uint32_t base = (plane * g.h + rc) * g.w;
        rowi[kh] = (int)base;
        const float4 a = ld4<(kH3f & 1) != 0>(in, (base + c0) >> 2);
        const float4 b = ld4<(kH3f & 1) != 0>(in, (base + c0 + 4) >> 2);
        const float e = in[base + (ce_ok ? (uint32_t)ce : c0)];
        const float lo = -FLT_MAX;
        // local column k is input column 2*x0 - P0 + k
        float *row = v[kh];
        if (P0 == 1) {
            row[0] = r_ok && ce_ok ? e : lo;
            row[1] = r_ok ? a.x : lo; row[2] = r_ok ? a.y : lo; row[3] = r_ok ? a.z : lo; row[4] = r_ok ? a.w : lo;
            row[5] = r_ok ? b.x : lo; row[6] = r_ok ? b.y : lo; row[7] = r_ok ? b.z : lo; row[8] = r_ok ? b.w : lo;
        } else {
            row[0] = r_ok ? a.x : lo; row[1] = r_ok ? a.y : lo; row[2] = r_ok ? a.z : lo; row[3] = r_ok ? a.w : lo;
            row[4] = r_ok ? b.x : lo; row[5] = r_ok ? b.y : lo; row[6] = r_ok ? b.z : lo; row[7] = r_ok ? b.w : lo;
            row[8] = r_ok && ce_ok ? e : lo;
        }
    }
    const int col0 = (int)c0 - P0;
    float m[4];
    int mi[4];
#pragma unroll
    for (int o = 0; o < 4; ++o) {
        m[o] = -FLT_MAX;
        mi[o] = -1;
#pragma unroll
        for (int kh = 0; kh < 3; ++kh)
#pragma unroll
            for (int kw = 0; kw < 3; ++kw) max_tap(v[kh][2 * o + kw], rowi[kh] + col0 + 2 * o + kw, m[o], mi[o]);
    }
    const uint32_t ov = (t * g.ow + 4 * xq) >> 2;
    st4<(kH3f & 2) != 0>(out, ov, make_float4(m[0], m[1], m[2], m[3]));
    reinterpret_cast<int4 *>(idx)[ov] = make_int4(mi[0], mi[1], mi[2], mi[3]);
}

// Backward: a lane owns input columns 8*q8 .. 8*q8 + 7 of input row r. The
// outputs whose windows can hold them are rows y_a <= y_b (the one or two
// with 2y - P0 <= r <= 2y - P0 + 2) and columns 4*q8 - 1 + P0 .. 4*q8 + 3 + P0,
// read as an aligned float4/int4 at column 4*q8 and one beside it. Each input
// adds the deltas of the candidates naming it in ascending output order (row
// y_a's columns ascending, then row y_b's): the twin's order, bit for bit.
// Every input is written by its lane alone; those no output names keep their
// value.
template <int P0>
__global__ __launch_bounds__(kBlock) void maxpool3s2_bwd_kernel(const float *delta, float *prev, const int *idx,
                                                                PoolGeom g, FastDiv div_q8, uint32_t lanes) {
    const uint32_t q = blockIdx.x * kBlock + threadIdx.x;
    if (q >= lanes) return;
    const uint32_t t = fdiv(q, div_q8);  // plane * h + r
    const uint32_t q8 = q - t * (g.w >> 3);
    const uint32_t plane = fdiv(t, g.div_h);
    const int r = (int)(t - plane * g.h);
    const uint32_t ib = t * g.w + 8 * q8;  // absolute index of the lane's first input
    float4 pa = ld4<(kH3b & 2) != 0>(prev, ib >> 2);
    float4 pb = ld4<(kH3b & 2) != 0>(prev, (ib >> 2) + 1);
    // candidate output rows
    const int yb = (r + P0) >> 1;
    const int ya = r + P0 >= 1 ? (r + P0 - 1) >> 1 : 0;
    const int oh = (int)g.oh, ow = (int)g.ow;
    const int xe = P0 == 1 ? 4 * (int)q8 + 4 : 4 * (int)q8 - 1;  // the column beside the aligned four
    const bool xe_ok = xe >= 0 && xe < ow;
    float d[2][5];
    int k[2][5];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const int y = s == 0 ? ya : yb;
        const bool y_ok = y < oh && (s == 0 || yb != ya);
        const uint32_t orow = (plane * g.oh + (uint32_t)(y_ok ? y : 0)) * g.ow;
        const uint32_t ov = (orow + 4 * q8) >> 2;
        const float4 dd = ld4<(kH3b & 1) != 0>(delta, ov);
        const int4 kk = reinterpret_cast<const int4 *>(idx)[ov];
        const float de = delta[orow + (xe_ok ? (uint32_t)xe : 4 * q8)];
        const int ke = idx[orow + (xe_ok ? (uint32_t)xe : 4 * q8)];
        // slot j is candidate column xe (P0 == 0: j = 0; P0 == 1: j = 4) or 4*q8 + (j - (1 - P0))
        const int off = 1 - P0;
        d[s][off + 0] = dd.x; d[s][off + 1] = dd.y; d[s][off + 2] = dd.z; d[s][off + 3] = dd.w;
        k[s][off + 0] = y_ok ? kk.x : -1; k[s][off + 1] = y_ok ? kk.y : -1;
        k[s][off + 2] = y_ok ? kk.z : -1; k[s][off + 3] = y_ok ? kk.w : -1;
        d[s][P0 == 1 ? 4 : 0] = de;
        k[s][P0 == 1 ? 4 : 0] = y_ok && xe_ok ? ke : -1;
    }
    float p[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int want = (int)ib + e;
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int j = 0; j < 5; ++j) p[e] = add_if(p[e], want, k[s][j], d[s][j]);
    }
    st4<(kH3b & 4) != 0>(prev, ib >> 2, make_float4(p[0], p[1], p[2], p[3]));
    st4<(kH3b & 4) != 0>(prev, (ib >> 2) + 1, make_float4(p[4], p[5], p[6], p[7]));
}

// Whether the 3x3/s2 kernels take a shape (see above); pad/2 is P0.
bool pool3s2_shape(const PoolGeom &g, bool backward) {
    (void)backward;  // w == 2*ow with ow % 4 == 0 makes w a multiple of 8, as both need
    return g.size == 3 && g.stride == 2 && g.half_pad <= 1 && g.ow % 4 == 0 && 2 * g.ow == g.w && g.h > 0 &&
           g.oh > 0;
}

// Planes a workgroup of the several-planes kernels takes: about
// DKZ_POOL_SEP_TARGET input elements (hw each), at most what fits in
// kPlaneMaxFloats of LDS (lds_floats each), and few enough to leave
// DKZ_POOL_SEP_MIN_GROUPS workgroups where the planes allow. 0: a plane
// alone does not fit.
uint32_t sep_planes(uint64_t planes, uint64_t hw, uint64_t lds_floats) {
    if (hw == 0 || lds_floats == 0 || lds_floats > kPlaneMaxFloats) return 0;
    uint64_t p = std::max<uint64_t>(1, DKZ_POOL_SEP_TARGET / hw);
    p = std::min<uint64_t>(p, kPlaneMaxFloats / lds_floats);
    p = std::min<uint64_t>(p, std::max<uint64_t>(1, planes / DKZ_POOL_SEP_MIN_GROUPS));
    return (uint32_t)p;
}

// maxpool_sep_block_fwd_kernel for a window size of 4 to 13.
template <bool VEC>
auto block_fwd_kernel(uint32_t size) -> decltype(&maxpool_sep_block_fwd_kernel<VEC, 4>) {
    switch (size) {
    case 4: return maxpool_sep_block_fwd_kernel<VEC, 4>;
    case 5: return maxpool_sep_block_fwd_kernel<VEC, 5>;
    case 6: return maxpool_sep_block_fwd_kernel<VEC, 6>;
    case 7: return maxpool_sep_block_fwd_kernel<VEC, 7>;
    case 8: return maxpool_sep_block_fwd_kernel<VEC, 8>;
    case 9: return maxpool_sep_block_fwd_kernel<VEC, 9>;
    case 10: return maxpool_sep_block_fwd_kernel<VEC, 10>;
    case 11: return maxpool_sep_block_fwd_kernel<VEC, 11>;
    case 12: return maxpool_sep_block_fwd_kernel<VEC, 12>;
    default: return maxpool_sep_block_fwd_kernel<VEC, 13>;
    }
}

// Validates the gpu.zig arguments and derives the geometry. `n` is out_n
// (forward) or in_n (backward); the batch follows from it.
int pool_geometry(int in_h, int in_w, int in_c, int stride, int size, int pad, PoolGeom *g, uint64_t *planes,
                  bool *fast) {
    DKZ_REQUIRE(in_h >= 0 && in_w >= 0 && in_c >= 0 && pad >= 0);
    DKZ_REQUIRE(stride >= 1 && size >= 1);
    DKZ_REQUIRE((uint64_t)size * (uint64_t)size <= kMaxElems - 16);  // taps counted below 2^31
    DKZ_REQUIRE((int64_t)in_w + pad >= size && (int64_t)in_h + pad >= size);  // pooling.zig:33-34
    g->h = (uint32_t)in_h;
    g->w = (uint32_t)in_w;
    g->c = (uint32_t)in_c;
    g->size = (uint32_t)size;
    g->stride = (uint32_t)stride;
    g->half_pad = (uint32_t)(pad / 2);
    g->ow = (uint32_t)((in_w + pad - size) / stride + 1);
    g->oh = (uint32_t)((in_h + pad - size) / stride + 1);
    g->div_w = make_fastdiv(g->w ? g->w : 1);
    g->div_h = make_fastdiv(g->h ? g->h : 1);
    g->div_ow = make_fastdiv(g->ow);
    g->div_oh = make_fastdiv(g->oh);
    g->div_size = make_fastdiv(g->size);
    g->div_stride = make_fastdiv(g->stride);
    *planes = 0;
    *fast = size == 2 && stride == 2 && pad / 2 == 0 && in_w % 4 == 0 && in_h % 2 == 0 && in_w > 0 && in_h > 0;
    return 0;
}

}  // namespace
}  // namespace dkz

using namespace dkz;

extern "C" {

int dkz_forward_maxpool(int out_n, int in_h, int in_w, int in_c, int stride, int size, int pad,
                        const float *input, float *output, int *indexes) {
    DKZ_REQUIRE(out_n >= 0);
    if (out_n == 0) return 0;
    PoolGeom g;
    uint64_t planes;
    bool fast;
    DKZ_TRY(pool_geometry(in_h, in_w, in_c, stride, size, pad, &g, &planes, &fast));
    const uint64_t per_plane = (uint64_t)g.oh * g.ow;
    DKZ_REQUIRE(per_plane > 0 && (uint64_t)out_n % per_plane == 0);
    planes = (uint64_t)out_n / per_plane;  // c * batch
    DKZ_REQUIRE(planes * g.h * g.w <= kMaxElems);
    DKZ_REQUIRE(input && output && indexes);
    if (fast && aligned16(input) && ((uintptr_t)output & 7u) == 0 && ((uintptr_t)indexes & 7u) == 0) {
        const uint32_t pairs = (uint32_t)out_n / 2;
        return launch("forward_maxpool_2x2", maxpool2_fwd_kernel, dim3(div_up(pairs, kBlock)), dim3(kBlock),
                      input, output, indexes, g, pairs);
    }
    if (DKZ_POOL_3S2 && pool3s2_shape(g, false) && aligned16(input) && aligned16(output) && aligned16(indexes)) {
        const uint32_t lanes = (uint32_t)out_n / 4;
        const FastDiv dq = make_fastdiv(g.ow / 4);
        if (g.half_pad == 1)
            return launch("forward_maxpool_3x3s2", maxpool3s2_fwd_kernel<1>, dim3(div_up(lanes, kBlock)), dim3(kBlock),
                          input, output, indexes, g, dq, lanes);
        return launch("forward_maxpool_3x3s2", maxpool3s2_fwd_kernel<0>, dim3(div_up(lanes, kBlock)), dim3(kBlock),
                      input, output, indexes, g, dq, lanes);
    }
    const uint64_t hw = (uint64_t)g.h * g.w;
    const bool runs = DKZ_POOL_SEP_RUN && g.stride == 1 && (g.size == 4 || g.size == 5 || g.size == 9 || g.size == 13);
    const bool blocks = DKZ_POOL_BLOCKS && g.stride == 1 && g.size >= 4 && g.size <= 13;
    if (DKZ_POOL_SEP && g.size >= DKZ_POOL_SEP_MIN_SIZE && planes >= DKZ_POOL_PLANE_MIN) {
        const uint64_t lds_floats = hw + 2ull * g.h * g.ow;
        const uint32_t P = sep_planes(planes, hw, lds_floats);
        if (P > 0) {
            const dim3 grid((uint32_t)div_up(planes, (uint64_t)P)), block(kSepBS);
            const bool vec = aligned16(input) && ((uint64_t)P * hw) % 4 == 0;
            const size_t lds = (size_t)(P * lds_floats * sizeof(float));
            (void)hipGetLastError();
            if (blocks) {
                const FastDiv dob = make_fastdiv(div_up(g.ow, g.size)), dohb = make_fastdiv(div_up(g.oh, g.size));
                const auto k = vec ? block_fwd_kernel<true>(g.size) : block_fwd_kernel<false>(g.size);
                hipLaunchKernelGGL(k, grid, block, lds, current_stream(), input, output, indexes, g, (uint32_t)planes,
                                   P, dob, dohb);
                return after_launch("forward_maxpool_separable", grid, block);
            }
            if (runs) {
                const FastDiv dor = make_fastdiv(div_up(g.ow, kRun)), dohr = make_fastdiv(div_up(g.oh, kRun));
                auto k = vec ? maxpool_sep_run_fwd_kernel<true, 4> : maxpool_sep_run_fwd_kernel<false, 4>;
                if (g.size == 5) k = vec ? maxpool_sep_run_fwd_kernel<true, 5> : maxpool_sep_run_fwd_kernel<false, 5>;
                if (g.size == 9) k = vec ? maxpool_sep_run_fwd_kernel<true, 9> : maxpool_sep_run_fwd_kernel<false, 9>;
                if (g.size == 13) k = vec ? maxpool_sep_run_fwd_kernel<true, 13> : maxpool_sep_run_fwd_kernel<false, 13>;
                hipLaunchKernelGGL(k, grid, block, lds, current_stream(), input, output, indexes, g, (uint32_t)planes,
                                   P, dor, dohr);
                return after_launch("forward_maxpool_separable", grid, block);
            }
            hipLaunchKernelGGL(vec ? maxpool_sep_fwd_kernel<true> : maxpool_sep_fwd_kernel<false>, grid, block,
                               lds, current_stream(), input, output, indexes, g,
                               (uint32_t)planes, P);
            return after_launch("forward_maxpool_separable", grid, block);
        }
    }
    if (DKZ_POOL_PLANE && hw > 0 && hw <= kPlaneMaxFloats && planes >= DKZ_POOL_PLANE_MIN) {
        const dim3 pgrid((uint32_t)planes), block(kBlock);
        const size_t lds = (size_t)hw * sizeof(float);
        const bool vec = aligned16(input) && hw % 4 == 0;
        (void)hipGetLastError();
        auto k = vec ? maxpool_plane_fwd_kernel<true, 0> : maxpool_plane_fwd_kernel<false, 0>;
        if (DKZ_POOL_PLANE_UNROLL && g.size == 3) k = vec ? maxpool_plane_fwd_kernel<true, 3> : maxpool_plane_fwd_kernel<false, 3>;
        if (DKZ_POOL_PLANE_UNROLL && g.size == 2) k = vec ? maxpool_plane_fwd_kernel<true, 2> : maxpool_plane_fwd_kernel<false, 2>;
        hipLaunchKernelGGL(k, pgrid, block, lds, current_stream(), input, output, indexes, g);
        return after_launch("forward_maxpool_plane", pgrid, block);
    }
    const dim3 grid(div_up((uint32_t)out_n, kBlock));
    if (g.size <= 2)
        return launch("forward_maxpool", maxpool_fwd_kernel<4>, grid, dim3(kBlock), input, output, indexes, g,
                      (uint32_t)out_n);
    return launch("forward_maxpool", maxpool_fwd_kernel<9>, grid, dim3(kBlock), input, output, indexes, g,
                  (uint32_t)out_n);
}

int dkz_backward_maxpool(int in_n, int in_h, int in_w, int in_c, int stride, int size, int pad,
                         const float *delta, float *prev_delta, const int *indexes) {
    DKZ_REQUIRE(in_n >= 0);
    if (in_n == 0) return 0;
    PoolGeom g;
    uint64_t planes;
    bool fast;
    DKZ_TRY(pool_geometry(in_h, in_w, in_c, stride, size, pad, &g, &planes, &fast));
    const uint64_t per_plane = (uint64_t)g.h * g.w;
    DKZ_REQUIRE(per_plane > 0 && (uint64_t)in_n % per_plane == 0);
    planes = (uint64_t)in_n / per_plane;
    DKZ_REQUIRE(planes * g.oh * g.ow <= kMaxElems);
    DKZ_REQUIRE(delta && prev_delta && indexes);
    if (fast && aligned16(prev_delta) && ((uintptr_t)delta & 7u) == 0 && ((uintptr_t)indexes & 7u) == 0) {
        const uint32_t pairs = (uint32_t)(planes * g.oh * g.ow / 2);
        return launch("backward_maxpool_2x2", maxpool2_bwd_kernel, dim3(div_up(pairs, kBlock)), dim3(kBlock),
                      delta, prev_delta, indexes, g, pairs);
    }
    if (DKZ_POOL_3S2 && pool3s2_shape(g, true) && aligned16(prev_delta) && aligned16(delta) && aligned16(indexes)) {
        const uint32_t lanes = (uint32_t)(in_n / 8);
        const FastDiv dq = make_fastdiv(g.w / 8);
        if (g.half_pad == 1)
            return launch("backward_maxpool_3x3s2", maxpool3s2_bwd_kernel<1>, dim3(div_up(lanes, kBlock)),
                          dim3(kBlock), delta, prev_delta, indexes, g, dq, lanes);
        return launch("backward_maxpool_3x3s2", maxpool3s2_bwd_kernel<0>, dim3(div_up(lanes, kBlock)), dim3(kBlock),
                      delta, prev_delta, indexes, g, dq, lanes);
    }
    // Outputs whose window covers one input, per dimension: at most ceil(size / stride).
    const uint32_t per_dim = (g.size + g.stride - 1) / g.stride;
    const uint64_t ohw = (uint64_t)g.oh * g.ow;
    if (DKZ_POOL_PLANE && g.stride >= 2 && per_plane + 2 * ohw <= kPlaneMaxFloats && planes >= DKZ_POOL_PLANE_MIN) {
        const dim3 pgrid((uint32_t)planes), block(kBlock);
        const size_t lds = (size_t)(per_plane + 2 * ohw) * sizeof(float);
        const bool vec = aligned16(prev_delta) && per_plane % 4 == 0;
        (void)hipGetLastError();
        hipLaunchKernelGGL(vec ? maxpool_plane_bwd_out_kernel<true> : maxpool_plane_bwd_out_kernel<false>, pgrid,
                           block, lds, current_stream(), delta, prev_delta, indexes, g);
        return after_launch("backward_maxpool_plane", pgrid, block);
    }
    if (g.stride >= 2) {
        const uint32_t out_n = (uint32_t)(planes * g.oh * g.ow);
        const dim3 ogrid(div_up(out_n, kBlock));
        if (per_dim <= 2)
            return launch("backward_maxpool", maxpool_bwd_out_kernel<4>, ogrid, dim3(kBlock), delta, prev_delta,
                          indexes, g, out_n, (uint32_t)in_n);
        return launch("backward_maxpool", maxpool_bwd_out_kernel<9>, ogrid, dim3(kBlock), delta, prev_delta,
                      indexes, g, out_n, (uint32_t)in_n);
    }
    if (DKZ_POOL_S1_TARGETS && per_dim >= DKZ_POOL_TARGETS_MIN_DIM && planes >= DKZ_POOL_PLANE_MIN) {
        const uint32_t P = sep_planes(planes, per_plane, 2 * ohw + 2 * per_plane);
        if (P > 0) {
            const dim3 grid((uint32_t)div_up(planes, (uint64_t)P)), block(kSepBS);
            (void)hipGetLastError();
            const uint32_t w8 = div_up(g.size, 8) * 8, w4 = div_up(g.size, 4) * 4;
            hipLaunchKernelGGL(w8 <= w4 ? maxpool_s1_target_gather_kernel<8> : maxpool_s1_target_gather_kernel<4>,
                               grid, block,
                               (size_t)(P * (2 * ohw + 2 * per_plane) * sizeof(float)), current_stream(), delta,
                               prev_delta, indexes, g, (uint32_t)planes, P);
            return after_launch("backward_maxpool_targets", grid, block);
        }
    }
    if (DKZ_POOL_S1_GATHER && per_dim >= DKZ_POOL_GATHER_MIN_DIM && planes >= DKZ_POOL_PLANE_MIN) {
        const uint32_t P = sep_planes(planes, per_plane, 2 * ohw);
        if (P > 0) {
            const dim3 grid((uint32_t)div_up(planes, (uint64_t)P)), block(kSepBS);
            const size_t lds = (size_t)(P * 2 * ohw * sizeof(float));
            (void)hipGetLastError();
            if (DKZ_POOL_RUN_GATHER && (g.size == 2 || g.size == 3 || g.size == 4 || g.size == 5 || g.size == 9 ||
                                        g.size == 13)) {
                const FastDiv dwr = make_fastdiv(div_up(g.w, kRunG));
                auto k = maxpool_s1_run_gather_kernel<3>;
                if (g.size == 2) k = maxpool_s1_run_gather_kernel<2>;
                if (g.size == 4) k = maxpool_s1_run_gather_kernel<4>;
                if (g.size == 5) k = maxpool_s1_run_gather_kernel<5>;
                if (g.size == 9) k = maxpool_s1_run_gather_kernel<9>;
                if (g.size == 13) k = maxpool_s1_run_gather_kernel<13>;
                hipLaunchKernelGGL(k, grid, block, lds, current_stream(), delta, prev_delta, indexes, g,
                                   (uint32_t)planes, P, dwr);
                return after_launch("backward_maxpool_gather", grid, block);
            }
            hipLaunchKernelGGL(maxpool_s1_gather_kernel, grid, block, lds, current_stream(), delta, prev_delta,
                               indexes, g, (uint32_t)planes, P);
            return after_launch("backward_maxpool_gather", grid, block);
        }
    }
    // Otherwise through LDS when more than 2x2 outputs can cover an input
    // (2x2 windows measured faster with the batched loads of
    // maxpool_bwd_kernel).
    if (DKZ_POOL_PLANE && per_dim > 2 && ohw <= kPlaneMaxFloats / 2 && planes >= DKZ_POOL_PLANE_MIN) {
        const dim3 pgrid((uint32_t)planes), block(kBlock);
        (void)hipGetLastError();
        hipLaunchKernelGGL(maxpool_plane_bwd_kernel, pgrid, block, (size_t)ohw * 8, current_stream(), delta,
                           prev_delta, indexes, g);
        return after_launch("backward_maxpool_plane", pgrid, block);
    }
    const dim3 grid(div_up((uint32_t)in_n, kBlock));
    if (per_dim <= 2)
        return launch("backward_maxpool", maxpool_bwd_kernel<4>, grid, dim3(kBlock), delta, prev_delta, indexes, g,
                      (uint32_t)in_n);
    return launch("backward_maxpool", maxpool_bwd_kernel<9>, grid, dim3(kBlock), delta, prev_delta, indexes, g,
                  (uint32_t)in_n);
}

}  // extern "C"
