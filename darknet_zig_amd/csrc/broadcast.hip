// broadcast.hip -- ops that combine every element of an NCHW tensor with a
// per-channel (or per-row) constant: add_bias, scale_bias, normalize,
// normalize_delta (src/gpu.zig:527-537, 573-608) and backward_avgpool
// (gpu.zig:765-767).
//
// Element e of a [batch, filters, spatial] tensor belongs to row r = e / spatial
// and channel f = r % filters (blas.zig:51); both divisions are multiply-high
// by launch constants. The tensor streams through in float4s exactly as in
// elementwise.hip; when spatial % 4 == 0 a float4 never straddles a row, so
// its channel constants are looked up (and derived, e.g. normalize's
// reciprocal) once per float4.
#include "dkz_channel.hpp"
#include "dkz_hints.hpp"

namespace dkz {
namespace {

// float4s per lane per stream, by tensor size: large tensors stream best
// with one (config-2 chain, scale_bias and normalize_delta: 1 -> 6590 GB/s,
// 2 -> 6550, 3 -> 6489, 4 -> 6510), the ~33 MB tensors of config 1 with four
// (normalize 0.63 of peak against 0.57 with one).
#ifndef DKZ_BCAST_UNROLL_LARGE
#define DKZ_BCAST_UNROLL_LARGE 1
#endif
#ifndef DKZ_BCAST_UNROLL_SMALL
#define DKZ_BCAST_UNROLL_SMALL 4
#endif
// Threads a workgroup below the large-tensor threshold. Measured at config 1
// (graph replay, cold): 512 threads took normalize / scale_bias / add_bias /
// leaky 2-3% faster but the copy 3% slower and config 3's softmax_x_ent
// 2.9 -> 3.5 us (half the workgroups); 1024 threads lost 3-8% on all and
// doubled softmax_x_ent. 256 stays.
#ifndef DKZ_BCAST_BS_SMALL
#define DKZ_BCAST_BS_SMALL 256
#endif
#ifndef DKZ_BCAST_LARGE_FLOAT4S
#define DKZ_BCAST_LARGE_FLOAT4S (1u << 22)  // 16 Mi elements
#endif

template <class Op, bool TWO, bool ROWWISE, bool S4>
__device__ __forceinline__ float4 bcast_vec(const Op &op, uint32_t v, float4 io, float4 a,
                                            const ChanGeom &g) {
    if constexpr (S4) {
        const auto p = op.param(channel_of<ROWWISE>(v << 2, g));
        io.x = op(io.x, a.x, p);
        io.y = op(io.y, a.y, p);
        io.z = op(io.z, a.z, p);
        io.w = op(io.w, a.w, p);
    } else {
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const auto p = op.param(channel_of<ROWWISE>((v << 2) + l, g));
            lane(io, l) = op(lane(io, l), lane(a, l), p);
        }
    }
    return io;
}

// H: bit 0 = nontemporal io loads, bit 1 = io stores, bit 2 = loads of a.
template <class Op, bool TWO, bool ROWWISE, bool S4, int H, int kUnroll, int BS = kBlock>
__global__ __launch_bounds__(BS) void bcast_vec_kernel(Op op, float *io, const float *a, ChanGeom g, uint32_t n) {
    constexpr bool kNtIo = (H & 1) != 0, kNtOut = (H & 2) != 0, kNtA = (H & 4) != 0;
    const uint32_t nv = n >> 2;
    const uint32_t base = blockIdx.x * (BS * kUnroll) + threadIdx.x;
    if (base + (kUnroll - 1) * BS < nv) {
        float4 x[kUnroll], y[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            x[u] = ld4<kNtIo>(io, base + u * BS);
            if constexpr (TWO) y[u] = ld4<kNtA>(a, base + u * BS);
            else y[u] = x[u];
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u)
            st4<kNtOut>(io, base + u * BS, bcast_vec<Op, TWO, ROWWISE, S4>(op, base + u * BS, x[u], y[u], g));
    } else {
        for (int u = 0; u < kUnroll; ++u) {
            const uint32_t v = base + u * BS;
            if (v < nv) {
                const float4 x = ld4<kNtIo>(io, v);
                const float4 y = TWO ? ld4<kNtA>(a, v) : x;
                st4<kNtOut>(io, v, bcast_vec<Op, TWO, ROWWISE, S4>(op, v, x, y, g));
            }
        }
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 3u)) {
        const uint32_t e = (nv << 2) + threadIdx.x;
        io[e] = op(io[e], TWO ? a[e] : 0.0f, op.param(channel_of<ROWWISE>(e, g)));
    }
}

template <class Op, bool TWO, bool ROWWISE>
__global__ __launch_bounds__(kBlock) void bcast_scalar_kernel(Op op, float *io, const float *a,
                                                              ChanGeom g, uint32_t n) {
    for (uint32_t e = blockIdx.x * kBlock + threadIdx.x; e < n; e += gridDim.x * kBlock)
        io[e] = op(io[e], TWO ? a[e] : 0.0f, op.param(channel_of<ROWWISE>(e, g)));
}

// filters, spatial already validated as non-negative ints; n64 the
// element count (batch * filters * spatial), at most kMaxElems.
template <int H, class Op, bool TWO, bool ROWWISE = false>
int launch_bcast(const char *name, const Op &op, float *io, const float *a, int filters, int spatial, uint64_t n64) {
    const uint32_t n = (uint32_t)n64;
    const ChanGeom g{make_fastdiv((uint32_t)spatial), make_fastdiv((uint32_t)filters)};
    if (aligned16(io) && (!TWO || aligned16(a))) {
        const uint32_t nv = n >> 2;
        const bool large = nv >= DKZ_BCAST_LARGE_FLOAT4S;
        constexpr int kU = DKZ_BCAST_UNROLL_LARGE, kUs = DKZ_BCAST_UNROLL_SMALL, kBs = DKZ_BCAST_BS_SMALL;
        if (large) {
            const dim3 grid(div_up(nv, (uint64_t)kBlock * kU));
            if (spatial % 4 == 0)
                return launch(name, bcast_vec_kernel<Op, TWO, ROWWISE, true, H, kU>, grid, dim3(kBlock), op, io, a,
                              g, n);
            return launch(name, bcast_vec_kernel<Op, TWO, ROWWISE, false, H, kU>, grid, dim3(kBlock), op, io, a, g,
                          n);
        }
        const dim3 grid(nv == 0 ? 1u : div_up(nv, (uint64_t)kBs * kUs));
        if (spatial % 4 == 0)
            return launch(name, bcast_vec_kernel<Op, TWO, ROWWISE, true, H, kUs, kBs>, grid, dim3(kBs), op, io, a, g,
                          n);
        return launch(name, bcast_vec_kernel<Op, TWO, ROWWISE, false, H, kUs, kBs>, grid, dim3(kBs), op, io, a, g,
                      n);
    }
    const uint32_t grid = div_up(n, kBlock) < 65536u ? div_up(n, kBlock) : 65536u;
    return launch(name, bcast_scalar_kernel<Op, TWO, ROWWISE>, dim3(grid), dim3(kBlock), op, io, a, g, n);
}

// Launches the op and records what it wrote (note_output).
template <int H, class Op, bool TWO, bool ROWWISE = false>
int run_bcast(const char *name, const Op &op, float *io, const float *a, int batch, int filters,
              int spatial) {
    const uint64_t n64 = (uint64_t)batch * (uint64_t)filters * (uint64_t)spatial;
    if (n64 == 0) return 0;
    DKZ_REQUIRE(n64 <= kMaxElems);
    DKZ_TRY((launch_bcast<H, Op, TWO, ROWWISE>(name, op, io, a, filters, spatial, n64)));
    note_output(io, 4 * n64);
    return 0;
}

// ---- ops ------------------------------------------------------------------

struct AddBiasOp {  // blas.zig:53-61
    const float *biases;
    __device__ float param(uint32_t f) const { return biases[f]; }
    __device__ float operator()(float v, float, float b) const { return v + b; }
};

struct ScaleBiasOp {  // blas.zig:63-71
    const float *scales;
    __device__ float param(uint32_t f) const { return scales[f]; }
    __device__ float operator()(float v, float, float s) const { return v * s; }
};

struct NormParam {
    float m, inv;
};
struct NormalizeOp {  // blas.zig:137-146
    const float *mean, *variance;
    __device__ NormParam param(uint32_t f) const {
        return {mean[f], 1.0f / (sqrtf(variance[f]) + 1e-6f)};
    }
    __device__ float operator()(float v, float, NormParam p) const { return (v - p.m) * p.inv; }
};

struct NormDeltaParam {
    float m, inv, vd2, md_over_n;
};
// blas.zig:180-204: dv*inv + vd*2*(xv-m)/denom + md/denom, left to right.
// vd*2 is exact, and md/denom is the same value for every element of f.
struct NormalizeDeltaOp {
    const float *mean, *variance, *mean_delta, *variance_delta;
    float denom;
    __device__ NormDeltaParam param(uint32_t f) const {
        return {mean[f], 1.0f / sqrtf(variance[f] + 1e-5f), variance_delta[f] * 2.0f, mean_delta[f] / denom};
    }
    __device__ float operator()(float dv, float xv, NormDeltaParam p) const {
        return (dv * p.inv + (p.vd2 * (xv - p.m)) / denom) + p.md_over_n;
    }
};

struct AvgpoolBackOp {  // pooling.zig:160-172: d = out_delta[r] / S, added to the row
    const float *out_delta;
    float denom;
    __device__ float param(uint32_t r) const { return out_delta[r] / denom; }
    __device__ float operator()(float v, float, float d) const { return v + d; }
};

}  // namespace
}  // namespace dkz

using namespace dkz;

#define DKZ_REQUIRE_SHAPE(b, f, s) DKZ_REQUIRE((b) >= 0 && (f) >= 0 && (s) >= 0)
#define DKZ_EMPTY(b, f, s) ((b) == 0 || (f) == 0 || (s) == 0)

extern "C" {

int dkz_add_bias(float *output, const float *biases, int batch, int filters, int spatial) {
    DKZ_REQUIRE_SHAPE(batch, filters, spatial);
    if (DKZ_EMPTY(batch, filters, spatial)) return 0;
    DKZ_REQUIRE(output && biases);
    return run_bcast<DKZ_HINT_ADD_BIAS, AddBiasOp, false>("add_bias", AddBiasOp{biases}, output, nullptr, batch, filters,
                                       spatial);
}

int dkz_scale_bias(float *output, const float *scales, int batch, int filters, int spatial) {
    DKZ_REQUIRE_SHAPE(batch, filters, spatial);
    if (DKZ_EMPTY(batch, filters, spatial)) return 0;
    DKZ_REQUIRE(output && scales);
    if ((uint64_t)batch * filters * spatial * sizeof(float) < DKZ_SCALE_BIAS_SMALL_BYTES)
        return run_bcast<DKZ_HINT_SCALE_BIAS_SMALL, ScaleBiasOp, false>("scale_bias", ScaleBiasOp{scales}, output,
                                                                        nullptr, batch, filters, spatial);
    return run_bcast<DKZ_HINT_SCALE_BIAS, ScaleBiasOp, false>("scale_bias", ScaleBiasOp{scales}, output, nullptr, batch,
                                         filters, spatial);
}

int dkz_normalize(float *x, const float *mean, const float *variance, int batch, int filters,
                  int spatial) {
    DKZ_REQUIRE_SHAPE(batch, filters, spatial);
    if (DKZ_EMPTY(batch, filters, spatial)) return 0;
    DKZ_REQUIRE(x && mean && variance);
    return run_bcast<DKZ_HINT_NORMALIZE, NormalizeOp, false>("normalize", NormalizeOp{mean, variance}, x, nullptr, batch,
                                         filters, spatial);
}

int dkz_normalize_delta(const float *x, const float *mean, const float *variance,
                        const float *mean_delta, const float *variance_delta, int batch, int filters,
                        int spatial, float *delta) {
    DKZ_REQUIRE_SHAPE(batch, filters, spatial);
    if (DKZ_EMPTY(batch, filters, spatial)) return 0;
    DKZ_REQUIRE(x && mean && variance && mean_delta && variance_delta && delta);
    const float denom = (float)((uint64_t)spatial * (uint64_t)batch);  // blas.zig:191
    const NormalizeDeltaOp op{mean, variance, mean_delta, variance_delta, denom};
    return run_bcast<DKZ_HINT_NORMALIZE_DELTA, NormalizeDeltaOp, true>("normalize_delta", op, delta, x, batch, filters, spatial);
}

int dkz_backward_avgpool(int n, int w, int h, int c, float *in_delta, const float *out_delta) {
    DKZ_REQUIRE(n >= 0 && w >= 0 && h >= 0 && c >= 0);
    const uint64_t spatial = (uint64_t)w * (uint64_t)h;
    if (n == 0 || spatial == 0) return 0;
    DKZ_REQUIRE(spatial <= kMaxElems);
    DKZ_REQUIRE(in_delta && out_delta);
    const AvgpoolBackOp op{out_delta, (float)spatial};
    return run_bcast<DKZ_HINT_AVGPOOL_BWD, AvgpoolBackOp, false, true>("backward_avgpool", op, in_delta, nullptr, n, 1,
                                                 (int)spatial);
}

}  // extern "C"
