// elementwise.hip -- the streaming elementwise ops of src/gpu.zig:483-521 and
// 631-645 (fill, copy, axpy, scal, mul, constrain, activate, gradient,
// softmax cross-entropy, l2, l1, smooth L1).
//
// One kernel shape serves all of them: each thread moves kUnroll float4s per
// stream, issuing every load before the first store, so a wave keeps
// kUnroll * 16 bytes per lane and stream in flight. The last n % 4 elements
// go to the first threads of block 0. Streams that are not 16-byte aligned
// (a Buf.offset() view, gpu.zig:128-133) take a one-element-per-thread
// grid-stride kernel with the same arithmetic.
#include "dkz_device.hpp"
#include "dkz_hints.hpp"
#include "dkz_internal.hpp"

namespace dkz {
namespace {

constexpr int kUnroll = 4;

// NI input streams, NO output streams; an output may be one of the inputs.
template <int NI, int NO>
struct Streams {
    const float *in[NI > 0 ? NI : 1];
    float *out[NO];
};

template <int NI, int NO, class Op>
__device__ __forceinline__ void apply_one(const Op &op, const Streams<NI, NO> &s, uint32_t i) {
    float a[NI > 0 ? NI : 1];
    float r[NO];
#pragma unroll
    for (int k = 0; k < NI; ++k) a[k] = s.in[k][i];
    op(a, r);
#pragma unroll
    for (int k = 0; k < NO; ++k) s.out[k][i] = r[k];
}

// H: bit k marks input stream k for nontemporal loads, bit 4 the outputs'
// stores (dkz_hints.hpp).
template <int H>
__device__ __forceinline__ float4 ld4_in(int k, const float *p, uint32_t v) {
    return ((H >> k) & 1) ? ld4<true>(p, v) : ld4<false>(p, v);
}

template <int NI, int NO, int H, class Op>
__device__ __forceinline__ void apply_vec(const Op &op, const Streams<NI, NO> &s, uint32_t v,
                                          const float4 (&in)[NI > 0 ? NI : 1]) {
    float4 out[NO];
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        float a[NI > 0 ? NI : 1];
        float r[NO];
#pragma unroll
        for (int k = 0; k < NI; ++k) a[k] = lane(in[k], l);
        op(a, r);
#pragma unroll
        for (int k = 0; k < NO; ++k) lane(out[k], l) = r[k];
    }
#pragma unroll
    for (int k = 0; k < NO; ++k) st4<(H & 16) != 0>(s.out[k], v, out[k]);
}

template <int NI, int NO, int H, class Op>
__global__ __launch_bounds__(kBlock) void ew_vec_kernel(Op op, Streams<NI, NO> s, uint32_t n) {
    const uint32_t nv = n >> 2;
    const uint32_t base = blockIdx.x * (kBlock * kUnroll) + threadIdx.x;
    if (base + (kUnroll - 1) * kBlock < nv) {
        // Whole tile in range: every load is issued before the first store.
        float4 in[kUnroll][NI > 0 ? NI : 1];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u)
#pragma unroll
            for (int k = 0; k < NI; ++k) in[u][k] = ld4_in<H>(k, s.in[k], base + u * kBlock);
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) apply_vec<NI, NO, H>(op, s, base + u * kBlock, in[u]);
    } else {
        for (int u = 0; u < kUnroll; ++u) {
            const uint32_t v = base + u * kBlock;
            if (v < nv) {
                float4 in[NI > 0 ? NI : 1];
#pragma unroll
                for (int k = 0; k < NI; ++k) in[k] = ld4_in<H>(k, s.in[k], v);
                apply_vec<NI, NO, H>(op, s, v, in);
            }
        }
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 3u)) apply_one<NI, NO>(op, s, (nv << 2) + threadIdx.x);
}

template <int NI, int NO, class Op>
__global__ __launch_bounds__(kBlock) void ew_scalar_kernel(Op op, Streams<NI, NO> s, uint32_t n) {
    for (uint32_t i = blockIdx.x * kBlock + threadIdx.x; i < n; i += gridDim.x * kBlock)
        apply_one<NI, NO>(op, s, i);
}

template <int H, int NI, int NO, class Op>
int run_ew(const char *name, const Op &op, const Streams<NI, NO> &s, int n) {
    if (n == 0) return 0;
    bool vec = true;
    for (int k = 0; k < NI; ++k) vec = vec && aligned16(s.in[k]);
    for (int k = 0; k < NO; ++k) vec = vec && aligned16(s.out[k]);
    const uint32_t un = (uint32_t)n;
    if (vec) {
        const uint32_t nv = un >> 2;
        const uint32_t grid = nv == 0 ? 1u : div_up(nv, (uint64_t)kBlock * kUnroll);
        return launch(name, ew_vec_kernel<NI, NO, H, Op>, dim3(grid), dim3(kBlock), op, s, un);
    }
    const uint32_t grid = div_up(un, kBlock) < 65536u ? div_up(un, kBlock) : 65536u;
    return launch(name, ew_scalar_kernel<NI, NO, Op>, dim3(grid), dim3(kBlock), op, s, un);
}

// ---- ops (CPU twins: blas.zig:13-46, activations.zig:107-143) -------------

struct FillOp {  // blas.zig:13
    float alpha;
    __device__ void operator()(const float (&)[1], float (&r)[1]) const { r[0] = alpha; }
};
struct CopyOp {  // blas.zig:17
    __device__ void operator()(const float (&a)[1], float (&r)[1]) const { r[0] = a[0]; }
};
struct AxpyOp {  // blas.zig:21, contracted: one rounding
    float alpha;
    __device__ void operator()(const float (&a)[2], float (&r)[1]) const {
        r[0] = __builtin_fmaf(alpha, a[0], a[1]);
    }
};
struct ScalOp {  // blas.zig:26
    float alpha;
    __device__ void operator()(const float (&a)[1], float (&r)[1]) const { r[0] = a[0] * alpha; }
};
struct MulOp {  // blas.zig:31: y *= x
    __device__ void operator()(const float (&a)[2], float (&r)[1]) const { r[0] = a[1] * a[0]; }
};
struct ConstrainOp {  // blas.zig:44: @max(-alpha, @min(v, alpha))
    float alpha;
    __device__ void operator()(const float (&a)[1], float (&r)[1]) const {
        r[0] = fmaxf(-alpha, fminf(a[0], alpha));
    }
};
template <int A>
struct ActivateOp {  // activations.zig:107-125
    __device__ void operator()(const float (&a)[1], float (&r)[1]) const { r[0] = activate<A>(a[0]); }
};
template <int A>
struct GradientOp {  // activations.zig:127-143: delta *= gradient(y); in = {y, delta}
    __device__ void operator()(const float (&a)[2], float (&r)[1]) const {
        r[0] = a[1] * gradient<A>(a[0]);
    }
};
// blas.zig:247-252; in = {pred, truth}, out = {delta, err}
struct SoftmaxXentOp {
    __device__ void operator()(const float (&a)[2], float (&r)[2]) const {
        const float p = a[0], t = a[1];
        r[1] = (t != 0.0f) ? -logf(p) : 0.0f;
        r[0] = t - p;
    }
};
struct L2Op {  // blas.zig:254-260
    __device__ void operator()(const float (&a)[2], float (&r)[2]) const {
        const float diff = a[1] - a[0];
        r[1] = diff * diff;
        r[0] = diff;
    }
};
struct L1Op {  // blas.zig:262-268
    __device__ void operator()(const float (&a)[2], float (&r)[2]) const {
        const float diff = a[1] - a[0];
        r[1] = fabsf(diff);
        r[0] = diff > 0.0f ? 1.0f : -1.0f;
    }
};
struct SmoothL1Op {  // blas.zig:270-282
    __device__ void operator()(const float (&a)[2], float (&r)[2]) const {
        const float diff = a[1] - a[0];
        const float ad = fabsf(diff);
        if (ad < 1.0f) {
            r[1] = diff * diff;
            r[0] = diff;
        } else {
            r[1] = 2.0f * ad - 1.0f;
            r[0] = diff < 0.0f ? 1.0f : -1.0f;
        }
    }
};

template <int A>
int activate_dispatch(float *x, int n) {
    Streams<1, 1> s{{x}, {x}};
    return run_ew<DKZ_HINT_ACTIVATE>("activate_array", ActivateOp<A>{}, s, n);
}

template <int A>
int gradient_dispatch(const float *y, int n, float *delta) {
    Streams<2, 1> s{{y, delta}, {delta}};
    return run_ew<DKZ_HINT_GRADIENT>("gradient_array", GradientOp<A>{}, s, n);
}

typedef int (*ActFn)(float *, int);
typedef int (*GradFn)(const float *, int, float *);

template <int... As>
struct ActTables {
    static constexpr ActFn act[] = {activate_dispatch<As>...};
    static constexpr GradFn grad[] = {gradient_dispatch<As>...};
};
using Tables = ActTables<0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13>;

template <class Op>
int run_loss(const char *name, int n, const float *pred, const float *truth, float *delta, float *err) {
    DKZ_REQUIRE(n >= 0);
    if (n == 0) return 0;
    DKZ_REQUIRE(pred && truth && delta && err);
    Streams<2, 2> s{{pred, truth}, {delta, err}};
    return run_ew<DKZ_HINT_LOSS>(name, Op{}, s, n);
}

}  // namespace
}  // namespace dkz

using namespace dkz;

extern "C" {

int dkz_fill(float *x, int n, float alpha) {
    DKZ_REQUIRE(n >= 0);
    if (n == 0) return 0;
    DKZ_REQUIRE(x != nullptr);
    Streams<0, 1> s{{nullptr}, {x}};
    return run_ew<DKZ_HINT_FILL>("fill", FillOp{alpha}, s, n);
}

int dkz_copy(int n, const float *x, float *y) {
    DKZ_REQUIRE(n >= 0);
    if (n == 0) return 0;
    DKZ_REQUIRE(x != nullptr && y != nullptr);
    Streams<1, 1> s{{x}, {y}};
    return run_ew<DKZ_HINT_COPY>("copy", CopyOp{}, s, n);
}

int dkz_axpy(int n, float alpha, const float *x, float *y) {
    DKZ_REQUIRE(n >= 0);
    if (n == 0) return 0;
    DKZ_REQUIRE(x != nullptr && y != nullptr);
    Streams<2, 1> s{{x, y}, {y}};
    return run_ew<DKZ_HINT_AXPY>("axpy", AxpyOp{alpha}, s, n);
}

int dkz_scal(int n, float alpha, float *x) {
    DKZ_REQUIRE(n >= 0);
    if (n == 0) return 0;
    DKZ_REQUIRE(x != nullptr);
    Streams<1, 1> s{{x}, {x}};
    return run_ew<DKZ_HINT_SCAL>("scal", ScalOp{alpha}, s, n);
}

int dkz_mul(int n, const float *x, float *y) {
    DKZ_REQUIRE(n >= 0);
    if (n == 0) return 0;
    DKZ_REQUIRE(x != nullptr && y != nullptr);
    Streams<2, 1> s{{x, y}, {y}};
    return run_ew<DKZ_HINT_MUL>("mul", MulOp{}, s, n);
}

int dkz_constrain(int n, float alpha, float *x) {
    DKZ_REQUIRE(n >= 0);
    if (n == 0) return 0;
    DKZ_REQUIRE(x != nullptr);
    Streams<1, 1> s{{x}, {x}};
    return run_ew<DKZ_HINT_CONSTRAIN>("constrain", ConstrainOp{alpha}, s, n);
}

int dkz_activate_array(float *x, int n, int a) {
    DKZ_REQUIRE(n >= 0);
    DKZ_REQUIRE(a >= 0 && a < kActCount);
    if (n == 0 || a == kLinear) return 0;  // activations.zig:111: linear is a no-op
    DKZ_REQUIRE(x != nullptr);
    return Tables::act[a](x, n);
}

int dkz_gradient_array(const float *x, int n, int a, float *delta) {
    DKZ_REQUIRE(n >= 0);
    DKZ_REQUIRE(a >= 0 && a < kActCount);
    if (n == 0 || a == kLinear) return 0;  // activations.zig:129: linear is a no-op
    DKZ_REQUIRE(x != nullptr && delta != nullptr);
    return Tables::grad[a](x, n, delta);
}

int dkz_softmax_cross_entropy(int n, const float *pred, const float *truth, float *delta, float *err) {
    return run_loss<SoftmaxXentOp>("softmax_x_ent", n, pred, truth, delta, err);
}

int dkz_l2(int n, const float *pred, const float *truth, float *delta, float *err) {
    return run_loss<L2Op>("l2", n, pred, truth, delta, err);
}

int dkz_l1(int n, const float *pred, const float *truth, float *delta, float *err) {
    return run_loss<L1Op>("l1", n, pred, truth, delta, err);
}

int dkz_smooth_l1(int n, const float *pred, const float *truth, float *delta, float *err) {
    return run_loss<SmoothL1Op>("smooth_l1", n, pred, truth, delta, err);
}

}  // extern "C"
