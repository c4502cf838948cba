// dkz_device.hpp -- device helpers shared by the gfx950 kernels: division by a
// launch constant, wave64 reductions, the host-libm-identical expf, and the
// activation functions of src/activations.zig.
//
// Every kernel source is compiled with -ffp-contract=off, correctly rounded
// fp32 division and square root, and fp32 denormals preserved, so a plain
// float expression here rounds exactly like the same expression in the Zig
// CPU twin (strict float mode). Fused multiply-adds appear only where they
// are written out with __builtin_fma / __builtin_fmaf.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dkz {

constexpr int kBlock = 256;  // four wave64s per workgroup
constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Unsigned division by a divisor fixed for the whole launch.
//
// For d >= 2, with l = ceil(log2 d), p = 31 + l and m = ceil(2^p / d), the
// quotient of any n < 2^31 is (n * m) >> p: writing m = (2^p + e)/d with
// 0 <= e < d, n*m/2^p = n/d + n*e/(d*2^p) and n*e < 2^31 * 2^l = 2^p keeps
// the error term below 1/d, so it never carries past the next integer. m is
// below 2^32 because d > 2^(l-1) (or m = 2^31 when d = 2^l).
// ---------------------------------------------------------------------------
struct FastDiv {
    uint32_t d;
    uint32_t mul;  // 0 encodes d == 1
    uint32_t shr;
};

__host__ __device__ inline FastDiv make_fastdiv(uint32_t d) {
    FastDiv f{d, 0u, 0u};
    if (d > 1) {
        uint32_t l = 0;
        while ((1ull << l) < d) ++l;
        const uint32_t p = 31 + l;
        f.mul = (uint32_t)(((1ull << p) + d - 1) / d);
        f.shr = p - 32;
    }
    return f;
}

__host__ __device__ __forceinline__ uint32_t umulhi32(uint32_t a, uint32_t b) {
    return (uint32_t)(((uint64_t)a * (uint64_t)b) >> 32);
}

// Requires n < 2^31.
__host__ __device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv &f) {
    return f.mul ? (umulhi32(n, f.mul) >> f.shr) : n;
}

// ---------------------------------------------------------------------------
// Global accesses of the tensors: 128-bit (and 64-bit) loads and stores, with
// or without the nontemporal hint (NT). Which operand of which op carries the
// hint is decided per op in dkz_hints.hpp. Small per-channel vectors use
// ordinary loads.
// ---------------------------------------------------------------------------
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

template <bool NT>
__device__ __forceinline__ float4 ld4(const float *p, uint32_t v) {
    if constexpr (NT) {
        const f32x4 r = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p) + v);
        return make_float4(r.x, r.y, r.z, r.w);
    } else {
        return reinterpret_cast<const float4 *>(p)[v];
    }
}
template <bool NT>
__device__ __forceinline__ void st4(float *p, uint32_t v, float4 x) {
    if constexpr (NT) {
        const f32x4 w = {x.x, x.y, x.z, x.w};
        __builtin_nontemporal_store(w, reinterpret_cast<f32x4 *>(p) + v);
    } else {
        reinterpret_cast<float4 *>(p)[v] = x;
    }
}
template <bool NT>
__device__ __forceinline__ float2 ld2(const float *p, uint32_t v) {
    if constexpr (NT) {
        const f32x2 r = __builtin_nontemporal_load(reinterpret_cast<const f32x2 *>(p) + v);
        return make_float2(r.x, r.y);
    } else {
        return reinterpret_cast<const float2 *>(p)[v];
    }
}
template <bool NT>
__device__ __forceinline__ void st2(float *p, uint32_t v, float2 x) {
    if constexpr (NT) {
        const f32x2 w = {x.x, x.y};
        __builtin_nontemporal_store(w, reinterpret_cast<f32x2 *>(p) + v);
    } else {
        reinterpret_cast<float2 *>(p)[v] = x;
    }
}
template <bool NT>
__device__ __forceinline__ int2 ld2i(const int *p, uint32_t v) {
    if constexpr (NT) {
        const i32x2 r = __builtin_nontemporal_load(reinterpret_cast<const i32x2 *>(p) + v);
        return make_int2(r.x, r.y);
    } else {
        return reinterpret_cast<const int2 *>(p)[v];
    }
}
template <bool NT>
__device__ __forceinline__ void st2i(int *p, uint32_t v, int2 x) {
    if constexpr (NT) {
        const i32x2 w = {x.x, x.y};
        __builtin_nontemporal_store(w, reinterpret_cast<i32x2 *>(p) + v);
    } else {
        reinterpret_cast<int2 *>(p)[v] = x;
    }
}

template <bool NT>
__device__ __forceinline__ float ld1(const float *p, uint32_t i) {
    if constexpr (NT) return __builtin_nontemporal_load(p + i);
    else return p[i];
}
template <bool NT>
__device__ __forceinline__ void st1(float *p, uint32_t i, float x) {
    if constexpr (NT) __builtin_nontemporal_store(x, p + i);
    else p[i] = x;
}

// Workgroups are dispatched to the 8 XCDs in turn (workgroup b to XCD b % 8),
// each with its own L2. xcd_run_block(b, grid, R) renumbers them so that the
// logical blocks R*i .. R*i + R - 1 run on one XCD (physical blocks b,
// b + 8, ..., b + 8(R-1)): neighbouring blocks whose data share 128-byte lines
// then fetch each shared line once. A bijection on [0, grid); blocks past the
// last whole group of 8R keep their index.
__host__ __device__ __forceinline__ uint32_t xcd_run_block(uint32_t b, uint32_t grid, uint32_t R) {
    if (b >= grid / (8 * R) * (8 * R)) return b;
    return R * ((b / (8 * R)) * 8 + (b & 7)) + (b / 8) % R;
}

__device__ __forceinline__ float &lane(float4 &v, int k) {
    return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w;
}
__device__ __forceinline__ float lane(const float4 &v, int k) {
    return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w;
}

// ---------------------------------------------------------------------------
// Wave64 reductions. The first four steps are DPP moves inside each 16-lane
// row (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror,
// row_mirror); each step adds a lane's value to its partner's, and the two
// partners compute the same sum with the operands swapped, so after them every
// lane of a row holds that row's sum bit for bit. The four row sums are then
// read from lanes 0, 16, 32, 48 and added in a fixed order. The result is the
// same in every lane and depends only on the data, never on timing.
// Call with the whole wave active.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const uint64_t u = (uint64_t)__double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xf, 0xf, false);
    return __longlong_as_double((long long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo));
}

__device__ __forceinline__ double readlane_d(double v, int l) {
    const uint64_t u = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // row_half_mirror
constexpr int kDppMirror = 0x140;     // row_mirror

__device__ __forceinline__ double wave_sum(double v) {
    v += dpp_d<kDppXor1>(v);
    v += dpp_d<kDppXor2>(v);
    v += dpp_d<kDppHalfMirror>(v);
    v += dpp_d<kDppMirror>(v);
    return (readlane_d(v, 0) + readlane_d(v, 16)) + (readlane_d(v, 32) + readlane_d(v, 48));
}

// Maximum under fmaxf semantics (a NaN operand is ignored), as Zig's @max.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<kDppXor1>(v));
    v = fmaxf(v, dpp_f<kDppXor2>(v));
    v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
    v = fmaxf(v, dpp_f<kDppMirror>(v));
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// Reductions over a segment of L consecutive lanes (L = 4, 8, 16, 32, 64;
// the whole wave active). Butterfly steps: DPP quad permutes and row mirrors
// inside 16-lane rows, then lane swaps across rows. Partners combine the same
// two operands, so every lane of the segment ends with the same bits.
template <int L>
__device__ __forceinline__ float seg_max(float v) {
    if constexpr (L == kWave) {
        return wave_max(v);
    } else {
        v = fmaxf(v, dpp_f<kDppXor1>(v));
        v = fmaxf(v, dpp_f<kDppXor2>(v));
        if constexpr (L >= 8) v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
        if constexpr (L >= 16) v = fmaxf(v, dpp_f<kDppMirror>(v));
        if constexpr (L >= 32) v = fmaxf(v, __shfl_xor(v, 16));
        return v;
    }
}

template <int L>
__device__ __forceinline__ double seg_sum(double v) {
    if constexpr (L == kWave) {
        return wave_sum(v);
    } else {
        v += dpp_d<kDppXor1>(v);
        v += dpp_d<kDppXor2>(v);
        if constexpr (L >= 8) v += dpp_d<kDppHalfMirror>(v);
        if constexpr (L >= 16) v += dpp_d<kDppMirror>(v);
        if constexpr (L >= 32) v += __shfl_xor(v, 16);
        return v;
    }
}

// Sum over a BS-thread workgroup; every thread returns the same value, added
// over the waves in index order. `lds` holds BS/64 doubles. Contains barriers:
// call from all threads.
template <int BS = kBlock>
__device__ __forceinline__ double block_sum(double v, double *lds) {
    v = wave_sum(v);
    const int w = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) lds[w] = v;
    __syncthreads();
    double t = lds[0];
#pragma unroll
    for (int i = 1; i < BS / kWave; ++i) t += lds[i];
    __syncthreads();
    return t;
}

__device__ __forceinline__ float block_max(float v, float *lds) {
    v = wave_max(v);
    const int w = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) lds[w] = v;
    __syncthreads();
    const float t = fmaxf(fmaxf(lds[0], lds[1]), fmaxf(lds[2], lds[3]));
    __syncthreads();
    return t;
}

// ---------------------------------------------------------------------------
// expf, bit-identical to the host C library's (glibc 2.35 on x86-64 with FMA,
// which is what the Zig twins' @exp binds to). The method is the published
// one of ARM optimized-routines (Szabolcs Nagy, 2017), used by glibc since
// 2.28: with N = 32, x*N/ln2 = k + r, exp(x) = 2^(k/N) * 2^(r/N), 2^(k/N) read
// from a 32-entry table and scaled by the exponent bits, 2^(r/N) a cubic in r,
// all in double and rounded to float once. The table entry i is the bit
// pattern of 2^(i/32) rounded to double, minus i << 47; the range reduction is
// fused exactly as the FMA build of the library fuses it. Agreement with the
// host expf is checked over all 2^32 inputs by the test suite.
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ uint64_t exp2f_tab(uint32_t i) {
    constexpr uint64_t kTab[32] = {
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
    };
    return kTab[i];
}

__host__ __device__ __forceinline__ float expf_libm(float x) {
    constexpr double kInvLn2N = 0x1.71547652b82fep+0 * 32;
    constexpr double kShift = 0x1.8p+52;
    constexpr double kC0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / 32;
    uint32_t ux;
    __builtin_memcpy(&ux, &x, 4);
    const uint32_t ax = ux & 0x7fffffffu;
    if (ax >= 0x42b00000u) {  // |x| >= 88 or NaN
        if (ux == 0xff800000u) return 0.0f;
        if (ax >= 0x7f800000u) return x + x;
        if (x > 0x1.62e42ep6f) return __builtin_inff();  // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double xd = (double)x;
    double kd = __builtin_fma(kInvLn2N, xd, kShift);
    uint64_t ki;
    __builtin_memcpy(&ki, &kd, 8);
    kd -= kShift;
    const double r = __builtin_fma(kInvLn2N, xd, -kd);
    const uint64_t t = exp2f_tab((uint32_t)(ki % 32)) + (ki << 47);
    double s;
    __builtin_memcpy(&s, &t, 8);
    const double z = __builtin_fma(kC0, r, kC1);
    const double r2 = r * r;
    double y = __builtin_fma(kC2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    return (float)(y * s);
}

// ---------------------------------------------------------------------------
// exp for softmax, whose contract is 1e-5 relative per element (not bit
// equality with the host libm): under one ulp at a third of expf_libm's cost
// and without its per-lane table reads.
//
// Cody & Waite's reduction: k = rint(x/ln2), r = x - k*ln2 with ln2 split into
// a head of 16 significant bits (k*head is exact for |k| <= 2^8) and a tail,
// so |r| <= ln2/2 up to an error far below ulp(r). exp(r) = 1 + r + r^2 q(r)
// with q of degree 4, evaluated in Horner form: the coefficients are a
// minimax fit (Lawson-reweighted least squares over 4000 Chebyshev nodes of
// [-ln2/2, ln2/2], relative error of exp weighted) rounded to f32, 3.8e-9
// relative before rounding. 2^k is applied by ldexp, which rounds a subnormal
// result once. x is clamped to [-104, 89] first (exp(-104) rounds to 0 and
// exp(89) overflows to +inf, so the clamp changes no result). Only
// IEEE-exact operations (min, max, multiply, fma, rint, ldexp), so the host
// build of this function gives the device's bits, and its accuracy is
// checked on the host over every float input.
//
// expf_cw_num requires x not NaN (softmax detects a NaN argument once per
// group instead of per element); expf_cw passes NaN through.
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ float expf_cw_num(float x) {
    constexpr float kLog2e = (float)1.4426950408889634;  // 1/ln2
    constexpr float kLn2Hi = 0x1.62e4p-1f;               // ln2 to 16 bits
    constexpr float kLn2Lo = (float)(0.6931471805599453 - (double)kLn2Hi);
    constexpr float q0 = 0x1.fffffcp-2f, q1 = 0x1.555492p-3f, q2 = 0x1.5558f2p-5f;
    constexpr float q3 = 0x1.1239d4p-7f, q4 = 0x1.6a244cp-10f;
#if defined(__HIP_DEVICE_COMPILE__)
    const float xc = __builtin_amdgcn_fmed3f(x, -104.0f, 89.0f);  // the same clamp for x not NaN
#else
    const float xc = __builtin_fminf(__builtin_fmaxf(x, -104.0f), 89.0f);
#endif
    const float k = __builtin_rintf(xc * kLog2e);
    float r = __builtin_fmaf(k, -kLn2Hi, xc);
    r = __builtin_fmaf(k, -kLn2Lo, r);
    float p = __builtin_fmaf(q4, r, q3);
    p = __builtin_fmaf(p, r, q2);
    p = __builtin_fmaf(p, r, q1);
    p = __builtin_fmaf(p, r, q0);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_ldexpf(p, (int)k);
}

__host__ __device__ __forceinline__ float expf_cw(float x) {
    const float y = expf_cw_num(x);
    return x != x ? x : y;
}

// v^-1.5 as 1/(v*sqrt(v)) in f64, rounded once: the factor of variance_delta.
// std.math.pow(f32, v, -1.5) (blas.zig:176) goes through f32 exp and log and
// lands within a few ulps of it.
__device__ __forceinline__ float pow_m1p5(float v) {
    const double d = (double)v;
    return (float)(1.0 / (d * sqrt(d)));
}

// ---------------------------------------------------------------------------
// Activations (src/activations.zig:11-27 codes, 58-104 maths). Selects, not
// multiplies, where the Zig code selects; literals are the f32 roundings of
// the Zig comptime values (1.0507 * 1.6732 folds to 1.75803124f).
// ---------------------------------------------------------------------------
enum Act : int {
    kLogistic = 0, kRelu = 1, kRelie = 2, kLinear = 3, kRamp = 4, kTanh = 5, kPlse = 6,
    kLeaky = 7, kElu = 8, kLoggy = 9, kStair = 10, kHardtan = 11, kLhtan = 12, kSelu = 13,
    kActCount = 14
};

template <int A>
__device__ __forceinline__ float activate(float x) {
    if constexpr (A == kLinear) return x;
    else if constexpr (A == kLogistic) return 1.0f / (1.0f + expf_libm(-x));
    else if constexpr (A == kLoggy) return 2.0f / (1.0f + expf_libm(-x)) - 1.0f;
    else if constexpr (A == kRelu) return x > 0.0f ? x : 0.0f;
    else if constexpr (A == kElu) return x >= 0.0f ? x : expf_libm(x) - 1.0f;
    else if constexpr (A == kSelu) return x >= 0.0f ? 1.0507f * x : 1.75803124f * (expf_libm(x) - 1.0f);
    else if constexpr (A == kRelie) return x > 0.0f ? x : 0.01f * x;
    else if constexpr (A == kRamp) return (x > 0.0f ? x : 0.0f) + 0.1f * x;
    else if constexpr (A == kLeaky) return x > 0.0f ? x : 0.1f * x;
    else if constexpr (A == kTanh) {
        const float e = expf_libm(2.0f * x);
        return (e - 1.0f) / (e + 1.0f);
    } else if constexpr (A == kPlse) {
        return x < -4.0f ? 0.01f * (x + 4.0f) : x > 4.0f ? 0.01f * (x - 4.0f) + 1.0f : 0.125f * x + 0.5f;
    } else if constexpr (A == kStair) {
        // @rem(@intFromFloat(floor(x)), 2) == 0, decided on the float itself:
        // an integer-valued n is even exactly when n/2 is an integer.
        const float n = floorf(x);
        const float h = n * 0.5f;
        return floorf(h) == h ? floorf(x / 2.0f) : (x - n) + floorf(x / 2.0f);
    } else if constexpr (A == kHardtan) return fmaxf(-1.0f, fminf(x, 1.0f));
    else if constexpr (A == kLhtan) {
        return x < 0.0f ? 0.001f * x : x > 1.0f ? 0.001f * (x - 1.0f) + 1.0f : x;
    } else return x;
}

template <int A>
__device__ __forceinline__ float gradient(float y) {
    if constexpr (A == kLinear) return 1.0f;
    else if constexpr (A == kLogistic) return (1.0f - y) * y;
    else if constexpr (A == kLoggy) {
        const float t = (y + 1.0f) / 2.0f;
        return (2.0f * (1.0f - t)) * t;
    } else if constexpr (A == kRelu) return y > 0.0f ? 1.0f : 0.0f;
    else if constexpr (A == kElu) return y >= 0.0f ? 1.0f : y + 1.0f;
    else if constexpr (A == kSelu) return y >= 0.0f ? 1.0507f : y + 1.75803124f;
    else if constexpr (A == kRelie) return y > 0.0f ? 1.0f : 0.01f;
    else if constexpr (A == kRamp) return (y > 0.0f ? 1.0f : 0.0f) + 0.1f;
    else if constexpr (A == kLeaky) return y > 0.0f ? 1.0f : 0.1f;
    else if constexpr (A == kTanh) return 1.0f - y * y;
    else if constexpr (A == kPlse) return (y < 0.0f || y > 1.0f) ? 0.01f : 0.125f;
    else if constexpr (A == kStair) return floorf(y) == y ? 0.0f : 1.0f;
    else if constexpr (A == kHardtan) return (y > -1.0f && y < 1.0f) ? 1.0f : 0.0f;
    else if constexpr (A == kLhtan) return (y > 0.0f && y < 1.0f) ? 1.0f : 0.001f;
    else return 1.0f;
}

}  // namespace dkz
