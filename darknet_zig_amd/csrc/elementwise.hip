// elementwise.hip -- the streaming elementwise ops of src/gpu.zig:483-521,
// 631-645, 769 and 804-830 (fill, copy, axpy, scal, mul, add_scalar,
// constrain, rand_uniform, activate, gradient, softmax cross-entropy, l2, l1,
// smooth L1, dropout, and the Adam update as one pass).
//
// One kernel shape serves all of them: each thread moves kUnroll float4s per
// stream (2 or 4, by tensor size), issuing every load before the first
// store, so a wave keeps kUnroll * 16 bytes per lane and stream in flight.
// The last n % 4 elements go to the first threads of block 0. Streams that are not 16-byte aligned
// (a Buf.offset() view, gpu.zig:128-133) take a one-element-per-thread
// grid-stride kernel with the same arithmetic.
#include "dkz_device.hpp"
#include "dkz_hints.hpp"
#include "dkz_internal.hpp"

namespace dkz {
namespace {

// float4s per lane per stream, by tensor size. Large tensors: 2 (config-2
// gradient 45.5 us against 46.0 with 4; rand_uniform over 103 M floats 66.6
// against 71.9 us). The ~16 M-element tensors of config 1 and the per-channel
// vectors: 4 (the config-1 layer sequence, copies and EMA included, 55.8 us
// against 70.8 with 2).
#ifndef DKZ_EW_UNROLL_LARGE
#define DKZ_EW_UNROLL_LARGE 2
#endif
#ifndef DKZ_EW_UNROLL_SMALL
#define DKZ_EW_UNROLL_SMALL 4
#endif
// Threads a workgroup below the large-tensor threshold. Measured at config 1
// (graph replay, cold): 512 threads took normalize / scale_bias / add_bias /
// leaky 2-3% faster but the copy 3% slower and config 3's softmax_x_ent
// 2.9 -> 3.5 us (half the workgroups); 1024 threads lost 3-8% on all and
// doubled softmax_x_ent. 256 stays.
#ifndef DKZ_EW_BS_SMALL
#define DKZ_EW_BS_SMALL 256
#endif
#ifndef DKZ_EW_LARGE_FLOAT4S
#define DKZ_EW_LARGE_FLOAT4S (1u << 22)  // 16 Mi elements
#endif

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

template <int NI, int NO, int H, class Op, int kUnroll, int BS = kBlock>
__global__ __launch_bounds__(BS) void ew_vec_kernel(Op op, Streams<NI, NO> s, uint32_t n) {
    const uint32_t nv = n >> 2;
    const uint32_t base = blockIdx.x * (BS * kUnroll) + threadIdx.x;
    if (base + (kUnroll - 1) * BS < nv) {
        // Whole tile in range: every load is issued before the first store.
        float4 in[kUnroll][NI > 0 ? NI : 1];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u)
#pragma unroll
            for (int k = 0; k < NI; ++k) in[u][k] = ld4_in<H>(k, s.in[k], base + u * BS);
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) apply_vec<NI, NO, H>(op, s, base + u * BS, in[u]);
    } else {
        for (int u = 0; u < kUnroll; ++u) {
            const uint32_t v = base + u * BS;
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
int launch_ew(const char *name, const Op &op, const Streams<NI, NO> &s, int n) {
    bool vec = true;
    for (int k = 0; k < NI; ++k) vec = vec && aligned16(s.in[k]);
    for (int k = 0; k < NO; ++k) vec = vec && aligned16(s.out[k]);
    const uint32_t un = (uint32_t)n;
    if (vec) {
        const uint32_t nv = un >> 2;
        if (nv >= DKZ_EW_LARGE_FLOAT4S)
            return launch(name, ew_vec_kernel<NI, NO, H, Op, DKZ_EW_UNROLL_LARGE>,
                          dim3(div_up(nv, (uint64_t)kBlock * DKZ_EW_UNROLL_LARGE)), dim3(kBlock), op, s, un);
        constexpr int kBs = DKZ_EW_BS_SMALL;
        const uint32_t grid = nv == 0 ? 1u : div_up(nv, (uint64_t)kBs * DKZ_EW_UNROLL_SMALL);
        return launch(name, ew_vec_kernel<NI, NO, H, Op, DKZ_EW_UNROLL_SMALL, kBs>, dim3(grid), dim3(kBs), op, s, un);
    }
    const uint32_t grid = div_up(un, kBlock) < 65536u ? div_up(un, kBlock) : 65536u;
    return launch(name, ew_scalar_kernel<NI, NO, Op>, dim3(grid), dim3(kBlock), op, s, un);
}

// Launches the op and records what it wrote (note_output).
template <int H, int NI, int NO, class Op>
int run_ew(const char *name, const Op &op, const Streams<NI, NO> &s, int n) {
    if (n == 0) return 0;
    DKZ_TRY(launch_ew<H>(name, op, s, n));
    for (int k = 0; k < NO; ++k) note_output(s.out[k], 4ull * (uint32_t)n);
    return 0;
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
struct AddScalarOp {  // darknet_kernels.hip:150-153
    float alpha;
    __device__ void operator()(const float (&a)[1], float (&r)[1]) const { r[0] = a[0] + alpha; }
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

// layers/misc.zig:105-127: in = {x, rand}
struct DropoutOp {
    float prob, scale;
    __device__ void operator()(const float (&a)[2], float (&r)[1]) const {
        r[0] = (a[1] < prob) ? 0.0f : a[0] * scale;
    }
};

// gpu.zig:804-830 adamUpdate as one pass; in = out = {w, d, m, v}. Each
// element goes through the wrapper's launches in their order -- scal(b1, m),
// scal(b2, v), axpy(-decay*batch, w, d), axpy(1-b1, d, m), mul(d, d),
// axpy(1-b2, d, v), the adam_kernel step (darknet_kernels.hip:588-595),
// fill(d, 0) -- with the same roundings (axpy contracted, everything else
// one rounding per operation), so the result equals the eight-launch
// sequence bit for bit. c1 and c2 are the bias corrections 1 - b^t.
struct AdamOp {
    float b1, b2, neg_decay_batch, one_m_b1, one_m_b2, c1, c2, rate, eps;
    __device__ void operator()(const float (&a)[4], float (&r)[4]) const {
        const float m = a[2] * b1;
        const float v = a[3] * b2;
        const float d = __builtin_fmaf(neg_decay_batch, a[0], a[1]);
        const float m2 = __builtin_fmaf(one_m_b1, d, m);
        const float dd = d * d;
        const float v2 = __builtin_fmaf(one_m_b2, dd, v);
        const float mhat = m2 / c1;
        const float vhat = v2 / c2;
        r[0] = a[0] + rate * mhat / (sqrtf(vhat) + eps);
        r[1] = 0.0f;
        r[2] = m2;
        r[3] = v2;
    }
};

// darknet_kernels.hip:168-183: element i of a rand_uniform draw is the top 24
// bits of hash(seed ^ hash(i)), scaled into [0, 1) (every value exact). The
// hash is Wellons' "lowbias32".
__device__ __forceinline__ uint32_t hash_u32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}
__device__ __forceinline__ float uniform_at(uint32_t seed, uint32_t i) {
    return (float)(hash_u32(seed ^ hash_u32(i)) >> 8) * (1.0f / 16777216.0f);
}

template <bool NT, int kUnroll>
__global__ __launch_bounds__(kBlock) void rand_vec_kernel(float *x, uint32_t seed, uint32_t n) {
    const uint32_t nv = n >> 2;
    const uint32_t base = blockIdx.x * (kBlock * kUnroll) + threadIdx.x;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const uint32_t v = base + u * kBlock;
        if (v < nv) {
            const uint32_t e = v << 2;
            st4<NT>(x, v, make_float4(uniform_at(seed, e), uniform_at(seed, e + 1), uniform_at(seed, e + 2),
                                      uniform_at(seed, e + 3)));
        }
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 3u)) {
        const uint32_t e = (nv << 2) + threadIdx.x;
        x[e] = uniform_at(seed, e);
    }
}

__global__ __launch_bounds__(kBlock) void rand_scalar_kernel(float *x, uint32_t seed, uint32_t n) {
    for (uint32_t i = blockIdx.x * kBlock + threadIdx.x; i < n; i += gridDim.x * kBlock) x[i] = uniform_at(seed, i);
}

inline bool disjoint(const float *a, const float *b, int n) { return a + n <= b || b + n <= a; }

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
    if ((uint64_t)n * sizeof(float) < DKZ_COPY_SMALL_BYTES)
        return run_ew<DKZ_HINT_COPY_SMALL>("copy", CopyOp{}, s, n);
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

int dkz_add_scalar(int n, float alpha, float *x) {
    DKZ_REQUIRE(n >= 0);
    if (n == 0) return 0;
    DKZ_REQUIRE(x != nullptr);
    Streams<1, 1> s{{x}, {x}};
    return run_ew<DKZ_HINT_ADD_SCALAR>("add_scalar", AddScalarOp{alpha}, s, n);
}

int dkz_rand_uniform(int n, float *x, unsigned int seed) {
    DKZ_REQUIRE(n >= 0);
    if (n == 0) return 0;
    DKZ_REQUIRE(x != nullptr);
    const uint32_t un = (uint32_t)n;
    if (aligned16(x)) {
        const uint32_t nv = un >> 2;
        constexpr bool kNt = (DKZ_HINT_RAND_UNIFORM & 16) != 0;
        if (nv >= DKZ_EW_LARGE_FLOAT4S)
            return launch("rand_uniform", rand_vec_kernel<kNt, DKZ_EW_UNROLL_LARGE>,
                          dim3(div_up(nv, (uint64_t)kBlock * DKZ_EW_UNROLL_LARGE)), dim3(kBlock), x, (uint32_t)seed, un);
        const uint32_t grid = nv == 0 ? 1u : div_up(nv, (uint64_t)kBlock * DKZ_EW_UNROLL_SMALL);
        return launch("rand_uniform", rand_vec_kernel<kNt, DKZ_EW_UNROLL_SMALL>, dim3(grid), dim3(kBlock), x,
                      (uint32_t)seed, un);
    }
    const uint32_t grid = div_up(un, kBlock) < 65536u ? div_up(un, kBlock) : 65536u;
    return launch("rand_uniform", rand_scalar_kernel, dim3(grid), dim3(kBlock), x, (uint32_t)seed, un);
}

int dkz_dropout(float *input, int size, const float *rand, float prob, float scale) {
    DKZ_REQUIRE(size >= 0);
    if (size == 0) return 0;
    DKZ_REQUIRE(input != nullptr && rand != nullptr);
    Streams<2, 1> s{{input, rand}, {input}};
    if ((uint64_t)size * sizeof(float) >= DKZ_DROPOUT_LARGE_BYTES)
        return run_ew<DKZ_HINT_DROPOUT_LARGE>("dropout", DropoutOp{prob, scale}, s, size);
    return run_ew<DKZ_HINT_DROPOUT>("dropout", DropoutOp{prob, scale}, s, size);
}

int dkz_adam_update(float *w, float *d, float *m, float *v, float b1, float b2, float eps, float decay,
                    float rate, int n, int batch, int t) {
    DKZ_REQUIRE(n >= 0 && batch >= 0);
    if (n == 0) return 0;
    DKZ_REQUIRE(w && d && m && v);
    DKZ_REQUIRE(disjoint(w, d, n) && disjoint(w, m, n) && disjoint(w, v, n) && disjoint(d, m, n) &&
                disjoint(d, v, n) && disjoint(m, v, n));
    // The wrapper's scalar arguments, formed in f32 as gpu.zig:819-825 forms
    // them; the bias corrections as adam_kernel forms them (powf of the step
    // count converted to float), here once on the host.
    AdamOp op;
    op.b1 = b1;
    op.b2 = b2;
    op.neg_decay_batch = -decay * (float)batch;
    op.one_m_b1 = 1.0f - b1;
    op.one_m_b2 = 1.0f - b2;
    op.c1 = 1.0f - powf(b1, (float)t);
    op.c2 = 1.0f - powf(b2, (float)t);
    op.rate = rate;
    op.eps = eps;
    Streams<4, 4> s{{w, d, m, v}, {w, d, m, v}};
    return run_ew<DKZ_HINT_ADAM>("adam_update", op, s, n);
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
