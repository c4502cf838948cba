// softmax.hip -- grouped softmax (src/gpu.zig:614-629, CPU twin
// blas.zig:213-242), and the softmax layer's forward step with its
// cross-entropy loss fused in (layers/misc.zig:63-76).
//
// Group (b, g) holds n elements `stride` apart starting at
// b*batch_offset + g*group_offset. Per group the CPU twin takes the max
// (starting from -FLT_MAX), writes e_i = exp(x_i/T - max/T), sums the e_i
// left to right in f32 and divides. Every step except that sum is exact or
// elementwise, and exp is the host-identical expf_libm, so the kernels below
// reproduce the twin bit for bit wherever they keep the sequential sum:
//
//  * contiguous groups (stride 1) with 32 < n <= kSeqMax: one workgroup per
//    group; the row is read once into LDS (in float4s when aligned), max by
//    wave64 DPP + LDS, the exps in parallel in place, one lane adds them in
//    order, then all lanes divide. Bit-exact.
//  * many contiguous groups (at least kRowsMin) with 32 < n <= kRowsMaxN (256):
//    a workgroup stages kRows groups in LDS (odd row pitch, so lanes walking
//    columns of different rows use different banks); all its lanes share the
//    loads, exps and divides, and lane r of the first wave runs group r's max
//    and its sequential sum, so kRows sums advance per instruction. Bit-exact.
//  * many contiguous groups (at least DKZ_SOFTMAX_WIDE_MIN) with
//    kRowsMaxN < n <= kWideMaxN (1024): 2, 4 or 8 groups a workgroup held
//    in registers; maxes and exps on all lanes, then lane l of the first
//    wave adds group l's exps in order from LDS. Bit-exact.
//  * contiguous groups with n > kSeqMax: one workgroup per group, the row
//    not staged, and the sum an f64 tree (within 1e-5 relative of the twin)
//    because the row no longer fits in LDS.
//  * strided groups that sit side by side (group_offset 1, the spatial
//    softmax over the classes of each position) with n <= kTileMaxN: a
//    workgroup stages 64 consecutive groups in LDS; all its lanes share the
//    loads, exps and divides, and lane g < 64 takes group g's max and its
//    sequential sum. Bit-exact.
//  * other strided groups, or n <= 32: one lane per group runs the twin's
//    three loops, eight loads at a time. Bit-exact.
//
// dkz_softmax_layer_forward runs the layer's two calls (softmax, then
// softmax_x_ent over the whole batch) as one pass where the block kernels
// apply: the loss and delta are formed from each probability as it is
// stored, with softmax_x_ent's expressions.
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

__device__ __forceinline__ void read32(const float4 *lds, uint32_t batch, float4 (&v)[8]) {
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = lds[batch * 8 + u];
}

// s plus the 32 values, one at a time, left to right.
__device__ __forceinline__ float add32(float s, const float4 (&v)[8]) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        s += v[u].x;
        s += v[u].y;
        s += v[u].z;
        s += v[u].w;
    }
    return s;
}

// V4: the row is 16-byte aligned and n % 4 == 0 (every pointer too), so it
// moves in float4s.
template <bool SEQ, bool XENT, bool V4>
__global__ __launch_bounds__(kBlock) void softmax_block_kernel(const float *in, float *out, Groups G, Xent xe) {
    extern __shared__ float4 e_lds4[];  // n floats when SEQ; float4 keeps it 16-byte aligned
    float *e_lds = reinterpret_cast<float *>(e_lds4);
    __shared__ float red_f[kBlock / kWave];
    __shared__ double red_d[kBlock / kWave];
    __shared__ float sum_sh;
    const uint32_t off = group_base(blockIdx.x, G);
    const float *x = in + off;
    float *y = out + off;
    const uint32_t n = G.n, nv = n >> 2;

    float mx = -FLT_MAX;
    float sum;
    if constexpr (SEQ) {
        // The row is read once, into LDS; the max is order-free.
        if constexpr (V4) {
            for (uint32_t v = threadIdx.x; v < nv; v += kBlock) {
                const float4 a = ld4<false>(x, v);
                e_lds4[v] = a;
                mx = fmaxf(mx, fmaxf(fmaxf(a.x, a.y), fmaxf(a.z, a.w)));
            }
        } else {
            for (uint32_t i = threadIdx.x; i < n; i += kBlock) {
                const float a = x[i];
                e_lds[i] = a;
                mx = fmaxf(mx, a);
            }
        }
        mx = block_max(mx, red_f);
        const float mt = mx / G.temp;
        // Each lane turns the entries it loaded into exps, in place.
        if constexpr (V4) {
            for (uint32_t v = threadIdx.x; v < nv; v += kBlock) {
                float4 a = e_lds4[v];
                a.x = expf_libm(a.x / G.temp - mt);
                a.y = expf_libm(a.y / G.temp - mt);
                a.z = expf_libm(a.z / G.temp - mt);
                a.w = expf_libm(a.w / G.temp - mt);
                e_lds4[v] = a;
            }
        } else {
            for (uint32_t i = threadIdx.x; i < n; i += kBlock) e_lds[i] = expf_libm(e_lds[i] / G.temp - mt);
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            // The one sequential part, in batches of 32 exps: the LDS reads of
            // the next batch are in flight while this one is added.
            float s = 0.0f;
            const uint32_t nb = n >> 5;
            float4 va[8], vb[8];
            if (nb > 0) read32(e_lds4, 0, va);
            for (uint32_t b = 0; b < nb;) {
                if (b + 1 < nb) read32(e_lds4, b + 1, vb);
                s = add32(s, va);
                if (++b >= nb) break;
                if (b + 1 < nb) read32(e_lds4, b + 1, va);
                s = add32(s, vb);
                ++b;
            }
            for (uint32_t i = nb << 5; i < n; ++i) s += e_lds[i];
            sum_sh = s;
        }
        __syncthreads();
        sum = sum_sh;
        if constexpr (V4) {
            for (uint32_t v = threadIdx.x; v < nv; v += kBlock) {
                const float4 e = e_lds4[v];
                const float4 p = make_float4(e.x / sum, e.y / sum, e.z / sum, e.w / sum);
                st4<false>(y, v, p);
                if constexpr (XENT) {
                    const float4 t = ld4<false>(xe.truth + off, v);
                    float4 d, l;
                    xent1(p.x, t.x, d.x, l.x);
                    xent1(p.y, t.y, d.y, l.y);
                    xent1(p.z, t.z, d.z, l.z);
                    xent1(p.w, t.w, d.w, l.w);
                    st4<false>(xe.delta + off, v, d);
                    st4<false>(xe.loss + off, v, l);
                }
            }
        } else {
            for (uint32_t i = threadIdx.x; i < n; i += kBlock) {
                const float p = e_lds[i] / sum;
                y[i] = p;
                if constexpr (XENT) xent1(p, xe.truth[off + i], xe.delta[off + i], xe.loss[off + i]);
            }
        }
    } else {
        for (uint32_t i = threadIdx.x; i < n; i += kBlock) mx = fmaxf(mx, x[i]);
        mx = block_max(mx, red_f);
        const float mt = mx / G.temp;
        double acc = 0.0;
        for (uint32_t i = threadIdx.x; i < n; i += kBlock) {
            const float e = expf_libm(x[i] / G.temp - mt);
            y[i] = e;
            acc += (double)e;
        }
        sum = (float)block_sum(acc, red_d);
        for (uint32_t i = threadIdx.x; i < n; i += kBlock) {
            const float p = y[i] / sum;
            y[i] = p;
            if constexpr (XENT) xent1(p, xe.truth[off + i], xe.delta[off + i], xe.loss[off + i]);
        }
    }
}

constexpr uint32_t kRows = 16;
// Up to 256 elements a row (16 KiB of LDS a workgroup): measured against the
// one-workgroup-per-row kernel, [16384,100] 28.7 -> 9.6 us and [8192,256]
// 18.0 -> 14.8 us, while rows of 1000 were slower (64 KiB a workgroup leaves
// two per CU, too few loads in flight).
constexpr uint32_t kRowsMaxN = 256;
constexpr uint32_t kRowsMin = 4096;

// op(...op(op(acc, row[0]), row[1])..., row[n-1]): one lane's sequential fold
// of an LDS row, with the reads of the next 16 elements in flight while the
// current 16 are folded.
template <class Op>
__device__ __forceinline__ float row_fold(const float *row, uint32_t n, float acc, Op op) {
    constexpr uint32_t kB = 16;
    const uint32_t nb = n / kB;
    float a[kB], b[kB];
    if (nb > 0) {
#pragma unroll
        for (uint32_t u = 0; u < kB; ++u) a[u] = row[u];
    }
    for (uint32_t j = 0; j < nb;) {
        if (j + 1 < nb) {
#pragma unroll
            for (uint32_t u = 0; u < kB; ++u) b[u] = row[(j + 1) * kB + u];
        }
#pragma unroll
        for (uint32_t u = 0; u < kB; ++u) acc = op(acc, a[u]);
        if (++j >= nb) break;
        if (j + 1 < nb) {
#pragma unroll
            for (uint32_t u = 0; u < kB; ++u) a[u] = row[(j + 1) * kB + u];
        }
#pragma unroll
        for (uint32_t u = 0; u < kB; ++u) acc = op(acc, b[u]);
        ++j;
    }
    for (uint32_t i = nb * kB; i < n; ++i) acc = op(acc, row[i]);
    return acc;
}

struct MaxOp {
    __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
struct AddOp {
    __device__ float operator()(float a, float b) const { return a + b; }
};

// Groups r0 .. r0+kRows-1, contiguous (stride 1); tile[l*pitch + i] holds
// element i of group r0 + l.
__global__ __launch_bounds__(kBlock) void softmax_rows_kernel(const float *in, float *out, Groups G, FastDiv div_n,
                                                              uint32_t pitch, uint32_t rows) {
    extern __shared__ float tile[];
    __shared__ uint32_t base_sh[kRows];
    __shared__ float mt_sh[kRows], sum_sh[kRows];
    const uint32_t r0 = blockIdx.x * kRows;
    const uint32_t nr = rows - r0 < kRows ? rows - r0 : kRows;
    const uint32_t n = G.n, total = nr * n, t = threadIdx.x;
    if (t < kRows) base_sh[t] = t < nr ? group_base(r0 + t, G) : 0u;
    __syncthreads();
    // Eight loads per lane in flight: element i of row l for q = l*n + i.
    for (uint32_t q0 = t; q0 < total; q0 += kBlock * 8) {
        float v[8];
        uint32_t at[8];
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u) {
            const uint32_t q = q0 + u * kBlock;
            const uint32_t l = fdiv(q, div_n), i = q - l * n;
            at[u] = l * pitch + i;
            v[u] = q < total ? in[base_sh[q < total ? l : 0] + i] : 0.0f;
        }
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u)
            if (q0 + u * kBlock < total) tile[at[u]] = v[u];
    }
    __syncthreads();
    if (t < nr) mt_sh[t] = row_fold(tile + t * pitch, n, -FLT_MAX, MaxOp{}) / G.temp;
    __syncthreads();
    for (uint32_t q = t; q < total; q += kBlock) {
        const uint32_t l = fdiv(q, div_n), i = q - l * n;
        float &e = tile[l * pitch + i];
        e = expf_libm(e / G.temp - mt_sh[l]);
    }
    __syncthreads();
    if (t < nr) sum_sh[t] = row_fold(tile + t * pitch, n, 0.0f, AddOp{});
    __syncthreads();
    for (uint32_t q = t; q < total; q += kBlock) {
        const uint32_t l = fdiv(q, div_n), i = q - l * n;
        out[base_sh[l] + i] = tile[l * pitch + i] / sum_sh[l];
    }
}

// Many contiguous groups of kRowsMaxN < n <= kWideMaxN: R groups a
// workgroup (R * 1028 floats of LDS at most), held in registers -- lane t holds elements 4t..4t+3 (V4) or
// t, t+256, t+512, t+768 of each -- so the maxes (wave64 DPP + LDS) and the
// exps run on all lanes; the exps then go to LDS (row pitch a multiple of 4
// but not of 32) where lane l < R of the first wave adds group l's in order,
// so R sequential sums advance per instruction, and all lanes divide their
// registers by the sums. Bit-exact.
// Groups a workgroup: about 1024 workgroups (fewer leave the loads, the
// VALU-heavy exps and divides and the stores of the workgroups in lock step;
// more repeat the per-workgroup barriers and sums): measured at n = 1000,
// 2048 groups 16.8 -> 12.4 us (R = 2), 4096 24.5 -> 17.5 (R = 4), 8192
// 41.5 -> 28.9 and 16384 80 -> 50.5 (R = 8); below 2048 groups the
// one-workgroup-per-group kernel is as fast.
#ifndef DKZ_SOFTMAX_WIDE_MIN
#define DKZ_SOFTMAX_WIDE_MIN 2048
#endif
constexpr uint32_t kWideMaxN = 4 * kBlock;

template <int R, bool V4, bool XENT>
__global__ __launch_bounds__(kBlock) void softmax_wide_kernel(const float *in, float *out, Groups G, uint32_t rows,
                                                              uint32_t pitch, Xent xe) {
    extern __shared__ float4 wide_lds4[];  // R rows of `pitch` floats
    float *tile = reinterpret_cast<float *>(wide_lds4);
    __shared__ float red[R][kBlock / kWave];
    __shared__ float sum_sh[R];
    const uint32_t t = threadIdx.x, n = G.n, r0 = blockIdx.x * R;
    const uint32_t nr = rows - r0 < (uint32_t)R ? rows - r0 : (uint32_t)R;
    const int wave = (int)(t / kWave);
    // Element j of this lane's four in a group (V4: 4t + j; else t + 256j).
    auto at = [&](int j) -> uint32_t { return V4 ? 4 * t + (uint32_t)j : t + (uint32_t)j * kBlock; };

    float v[R][4];
    uint32_t base[R];
#pragma unroll
    for (int l = 0; l < R; ++l) base[l] = group_base(r0 + ((uint32_t)l < nr ? (uint32_t)l : 0u), G);
#pragma unroll
    for (int l = 0; l < R; ++l) {
        const bool live = (uint32_t)l < nr;
        if constexpr (V4) {
            float4 a = make_float4(-FLT_MAX, -FLT_MAX, -FLT_MAX, -FLT_MAX);
            if (live && 4 * t < n) a = ld4<false>(in + base[l], t);
            v[l][0] = a.x;
            v[l][1] = a.y;
            v[l][2] = a.z;
            v[l][3] = a.w;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) v[l][j] = live && at(j) < n ? in[base[l] + at(j)] : -FLT_MAX;
        }
    }
#pragma unroll
    for (int l = 0; l < R; ++l) {
        const float m = wave_max(fmaxf(fmaxf(v[l][0], v[l][1]), fmaxf(v[l][2], v[l][3])));
        if ((t & (kWave - 1)) == 0) red[l][wave] = m;
    }
    __syncthreads();
#pragma unroll
    for (int l = 0; l < R; ++l) {
        const float mt = fmaxf(fmaxf(red[l][0], red[l][1]), fmaxf(red[l][2], red[l][3])) / G.temp;
        float *row = tile + l * pitch;
        if constexpr (V4) {
            if (4 * t < n) {
#pragma unroll
                for (int j = 0; j < 4; ++j) v[l][j] = expf_libm(v[l][j] / G.temp - mt);
                reinterpret_cast<float4 *>(row)[t] = make_float4(v[l][0], v[l][1], v[l][2], v[l][3]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (at(j) < n) {
                    v[l][j] = expf_libm(v[l][j] / G.temp - mt);
                    row[at(j)] = v[l][j];
                }
            }
        }
    }
    __syncthreads();
    if (t < nr) {
        // Group t's exps left to right, 32 at a time, the next 32's LDS reads
        // in flight while these are added.
        const float4 *row4 = reinterpret_cast<const float4 *>(tile + t * pitch);
        float s = 0.0f;
        const uint32_t nb = n >> 5;
        float4 va[8], vb[8];
        if (nb > 0) read32(row4, 0, va);
        for (uint32_t b = 0; b < nb;) {
            if (b + 1 < nb) read32(row4, b + 1, vb);
            s = add32(s, va);
            if (++b >= nb) break;
            if (b + 1 < nb) read32(row4, b + 1, va);
            s = add32(s, vb);
            ++b;
        }
        for (uint32_t i = nb << 5; i < n; ++i) s += tile[t * pitch + i];
        sum_sh[t] = s;
    }
    __syncthreads();
#pragma unroll
    for (int l = 0; l < R; ++l) {
        if ((uint32_t)l >= nr) break;
        const float sum = sum_sh[l];
        const uint32_t off = base[l];
        if constexpr (V4) {
            if (4 * t < n) {
                const float4 p = make_float4(v[l][0] / sum, v[l][1] / sum, v[l][2] / sum, v[l][3] / sum);
                st4<false>(out + off, t, p);
                if constexpr (XENT) {
                    const float4 tr = ld4<false>(xe.truth + off, t);
                    float4 d, ls;
                    xent1(p.x, tr.x, d.x, ls.x);
                    xent1(p.y, tr.y, d.y, ls.y);
                    xent1(p.z, tr.z, d.z, ls.z);
                    xent1(p.w, tr.w, d.w, ls.w);
                    st4<false>(xe.delta + off, t, d);
                    st4<false>(xe.loss + off, t, ls);
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (at(j) < n) {
                    const float p = v[l][j] / sum;
                    out[off + at(j)] = p;
                    if constexpr (XENT) xent1(p, xe.truth[off + at(j)], xe.delta[off + at(j)], xe.loss[off + at(j)]);
                }
            }
        }
    }
}

template <int R>
int launch_wide(const float *input, float *output, const Groups &G, uint32_t rows, bool v4, const Xent *xe) {
    const uint32_t n4 = (G.n + 3) & ~3u;
    const uint32_t pitch = n4 % 32 == 0 ? n4 + 4 : n4;  // a multiple of 4, not of 32
    const size_t lds = (size_t)R * pitch * sizeof(float);
    const Xent x = xe ? *xe : Xent{nullptr, nullptr, nullptr};
    void (*k)(const float *, float *, Groups, uint32_t, uint32_t, Xent);
    if (xe) k = v4 ? softmax_wide_kernel<R, true, true> : softmax_wide_kernel<R, false, true>;
    else k = v4 ? softmax_wide_kernel<R, true, false> : softmax_wide_kernel<R, false, false>;
    const dim3 grid(div_up(rows, (uint32_t)R));
    (void)hipGetLastError();
    hipLaunchKernelGGL(k, grid, dim3(kBlock), lds, current_stream(), input, output, G, rows, pitch, x);
    return after_launch(xe ? "softmax_xent_wide" : "softmax_wide", grid, dim3(kBlock));
}

constexpr uint32_t kTileRows = 64;
constexpr uint32_t kTileMaxN = 128;

// Rows r0 .. r0+63 (group r = b*groups + g); tile[i*64 + l] holds element i of
// row r0 + l.
__global__ __launch_bounds__(kBlock) void softmax_tile_kernel(const float *in, float *out, Groups G, uint32_t rows) {
    __shared__ float tile[kTileMaxN * kTileRows];
    __shared__ uint32_t base_sh[kTileRows];
    __shared__ float mt_sh[kTileRows], sum_sh[kTileRows];
    const uint32_t r0 = blockIdx.x * kTileRows;
    const uint32_t nr = rows - r0 < kTileRows ? rows - r0 : kTileRows;
    const uint32_t n = G.n, st = G.stride, total = n * kTileRows;
    const uint32_t t = threadIdx.x;
    if (t < kTileRows) base_sh[t] = t < nr ? group_base(r0 + t, G) : 0u;
    __syncthreads();
    // Eight loads per lane in flight: element i of row l for q = i*64 + l.
    for (uint32_t q0 = t; q0 < total; q0 += kBlock * 8) {
        float v[8];
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u) {
            const uint32_t q = q0 + u * kBlock, l = q & (kTileRows - 1);
            v[u] = q < total && l < nr ? in[base_sh[l] + (q / kTileRows) * st] : 0.0f;
        }
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u)
            if (q0 + u * kBlock < total) tile[q0 + u * kBlock] = v[u];
    }
    __syncthreads();
    if (t < nr) {
        float mx = -FLT_MAX;
        for (uint32_t i = 0; i < n; ++i) mx = fmaxf(mx, tile[i * kTileRows + t]);
        mt_sh[t] = mx / G.temp;
    }
    __syncthreads();
    for (uint32_t q = t; q < total; q += kBlock) {
        const uint32_t l = q & (kTileRows - 1);
        if (l < nr) tile[q] = expf_libm(tile[q] / G.temp - mt_sh[l]);
    }
    __syncthreads();
    if (t < nr) {
        float s = 0.0f;
        for (uint32_t i = 0; i < n; ++i) s += tile[i * kTileRows + t];
        sum_sh[t] = s;
    }
    __syncthreads();
    for (uint32_t q = t; q < total; q += kBlock) {
        const uint32_t l = q & (kTileRows - 1);
        if (l < nr) out[base_sh[l] + (q / kTileRows) * st] = tile[q] / sum_sh[l];
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
        if (group_offset == 1 && stride > 1 && (uint32_t)n <= kTileMaxN)
            return launch("softmax_tile", softmax_tile_kernel, dim3(div_up(rows, kTileRows)), dim3(kBlock), input,
                          output, G, rows);
        return launch("softmax_lane", softmax_lane_kernel, dim3(div_up(rows, kBlock)), dim3(kBlock), input, output,
                      G, rows);
    }
    if (!xe && rows >= kRowsMin && (uint32_t)n <= kRowsMaxN) {
        const uint32_t pitch = (uint32_t)n | 1u;  // odd: the rows' columns fall in distinct banks
        const size_t lds = (size_t)kRows * pitch * sizeof(float);
        (void)hipGetLastError();
        hipLaunchKernelGGL(softmax_rows_kernel, dim3(div_up(rows, kRows)), dim3(kBlock), lds, current_stream(),
                           input, output, G, make_fastdiv((uint32_t)n), pitch, rows);
        return after_launch("softmax_rows", dim3(div_up(rows, kRows)), dim3(kBlock));
    }
    const bool seq = (uint32_t)n <= kSeqMax;
    bool v4 = n % 4 == 0 && batch_offset % 4 == 0 && group_offset % 4 == 0 && aligned16(input) && aligned16(output);
    if (xe) v4 = v4 && aligned16(xe->truth) && aligned16(xe->delta) && aligned16(xe->loss);
    if (rows >= DKZ_SOFTMAX_WIDE_MIN && (uint32_t)n > kRowsMaxN && (uint32_t)n <= kWideMaxN) {
        if (rows >= 8192) return launch_wide<8>(input, output, G, rows, v4, xe);
        if (rows >= 4096) return launch_wide<4>(input, output, G, rows, v4, xe);
        return launch_wide<2>(input, output, G, rows, v4, xe);
    }
    const Xent x = xe ? *xe : Xent{nullptr, nullptr, nullptr};
    const size_t lds = seq ? (size_t)n * sizeof(float) : 0;
    void (*k)(const float *, float *, Groups, Xent);
    if (seq) {
        if (xe) k = v4 ? softmax_block_kernel<true, true, true> : softmax_block_kernel<true, true, false>;
        else k = v4 ? softmax_block_kernel<true, false, true> : softmax_block_kernel<true, false, false>;
    } else {
        k = xe ? softmax_block_kernel<false, true, false> : softmax_block_kernel<false, false, false>;
    }
    (void)hipGetLastError();
    hipLaunchKernelGGL(k, dim3(rows), dim3(kBlock), lds, current_stream(), input, output, G, x);
    return after_launch(xe ? "softmax_xent" : "softmax", dim3(rows), dim3(kBlock));
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
