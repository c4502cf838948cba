// im2col.hip -- the convolution lowering of src/gpu.zig:651-669 (im2col,
// col2im), CPU twins src/im2col.zig:13-83.
//
// The column buffer has channels*ksize*ksize rows of height_col*width_col;
// row c holds, for every output position (h, w), the input tap
// (c_im, h*stride - pad + kh, w*stride - pad + kw) with c = (c_im*ksize + kh)*ksize + kw,
// or 0 where the tap falls in the padding.
//
// im2col: the column buffer is the large, contiguous stream, so a lane owns
// float4s of it (kUnroll per lane, all gathers issued before the stores),
// decomposes a float4's first flat index with multiply-high divisions and
// steps the coordinates to the next three. The input taps are gathers that
// the caches serve: each input element feeds up to ksize^2 rows.
//
// col2im: a lane owns image elements and gathers their contributions, so
// every image element is written once and no atomics are needed. The CPU twin
// adds contributions in column order; for one image element those come from
// distinct rows c, i.e. in ascending (kh, kw), which is the order used here,
// starting from the image's current value -- the result is bit-exact.
#include "dkz_device.hpp"
#include "dkz_hints.hpp"
#include "dkz_internal.hpp"

namespace dkz {
namespace {

// Float4s of the column buffer per lane. A [128,56,56] k3 image takes, with
// cached stores, 7.4-7.8 us at 1 or 2, 8.1-8.5 at 4, 9.0 at 8; with
// nontemporal stores 6.6 at 4 and 5.9-6.2 at 2.
#ifndef DKZ_IM2COL_UNROLL
#define DKZ_IM2COL_UNROLL 2
#endif
constexpr int kUnroll = DKZ_IM2COL_UNROLL;

struct ColGeom {
    uint32_t H, W, Ho, Wo, k, s, p;
    FastDiv div_plane;  // Ho*Wo
    FastDiv div_wo;
    FastDiv div_k;
    FastDiv div_w;
    FastDiv div_h;
    FastDiv div_s;
};

__device__ __forceinline__ float im2col_at(const float *__restrict__ im, uint32_t e, const ColGeom &g) {
    const uint32_t row = fdiv(e, g.div_plane);
    const uint32_t pix = e - row * g.div_plane.d;
    const uint32_t h = fdiv(pix, g.div_wo);
    const uint32_t w = pix - h * g.Wo;
    const uint32_t t = fdiv(row, g.div_k);
    const uint32_t kw = row - t * g.k;
    const uint32_t c_im = fdiv(t, g.div_k);
    const uint32_t kh = t - c_im * g.k;
    const uint32_t y = h * g.s + kh - g.p;  // wraps above H when the tap is in the top padding
    const uint32_t x = w * g.s + kw - g.p;
    if (y >= g.H || x >= g.W) return 0.0f;
    return im[(c_im * g.H + y) * g.W + x];
}

// Column coordinates of flat element e, stepped one element at a time so a
// float4 costs one decomposition.
struct ColPos {
    uint32_t w, h, kw, kh, c;
};

__device__ __forceinline__ ColPos col_pos(uint32_t e, const ColGeom &g) {
    ColPos q;
    const uint32_t row = fdiv(e, g.div_plane);
    const uint32_t pix = e - row * g.div_plane.d;
    q.h = fdiv(pix, g.div_wo);
    q.w = pix - q.h * g.Wo;
    const uint32_t t = fdiv(row, g.div_k);
    q.kw = row - t * g.k;
    q.c = fdiv(t, g.div_k);
    q.kh = t - q.c * g.k;
    return q;
}

__device__ __forceinline__ void col_next(ColPos &q, const ColGeom &g) {
    if (++q.w == g.Wo) {
        q.w = 0;
        if (++q.h == g.Ho) {
            q.h = 0;
            if (++q.kw == g.k) {
                q.kw = 0;
                if (++q.kh == g.k) {
                    q.kh = 0;
                    ++q.c;
                }
            }
        }
    }
}

__device__ __forceinline__ float col_tap(const float *__restrict__ im, const ColPos &q, const ColGeom &g) {
    const uint32_t y = q.h * g.s + q.kh - g.p;  // wraps above H in the top padding
    const uint32_t x = q.w * g.s + q.kw - g.p;
    if (y >= g.H || x >= g.W) return 0.0f;
    return im[(q.c * g.H + y) * g.W + x];
}

// Workgroups are dealt to the 8 XCDs round robin; block b takes logical
// block xcd_block(b), so that XCD x writes the x-th eighth of the column
// buffer and its L2 fetches only the input channels of that eighth (with
// consecutive blocks every XCD fetched every channel: a [128,56,56] k3
// image took 5.0 us and read its input several times over, now 4.5 us). A
// bijection on [0, nb): the first 8 * (nb / 8) blocks are permuted, the
// rest keep their index.
#ifndef DKZ_IM2COL_XCD
#define DKZ_IM2COL_XCD 1
#endif
__device__ __forceinline__ uint32_t xcd_block(uint32_t b, uint32_t nb) {
    if (!DKZ_IM2COL_XCD) return b;
    const uint32_t per = nb / 8;
    return b < per * 8 ? (b % 8) * per + b / 8 : b;
}

#ifndef DKZ_IM2COL_S1_CLAMP
#define DKZ_IM2COL_S1_CLAMP 1
#endif

template <bool NT>
__global__ __launch_bounds__(kBlock) void im2col_vec_kernel(const float *__restrict__ im, float *__restrict__ col,
                                                            ColGeom g, uint32_t n) {
    const uint32_t nv = n >> 2;
    const uint32_t base = xcd_block(blockIdx.x, gridDim.x) * (kBlock * kUnroll) + threadIdx.x;
    float4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const uint32_t q4 = base + u * kBlock;
        if (q4 < nv) {
            ColPos q = col_pos(q4 << 2, g);
            v[u].x = col_tap(im, q, g);
            col_next(q, g);
            v[u].y = col_tap(im, q, g);
            col_next(q, g);
            v[u].z = col_tap(im, q, g);
            col_next(q, g);
            v[u].w = col_tap(im, q, g);
        }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const uint32_t q4 = base + u * kBlock;
        if (q4 < nv) st4<NT>(col, q4, v[u]);
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 3u)) {
        const uint32_t e = (nv << 2) + threadIdx.x;
        col[e] = im2col_at(im, e, g);
    }
}

// Stride 1 with W % 4 == 0 and Wo % 4 == 0: a column float4 (four outputs
// of one output row) holds input elements x0 .. x0+3 of one input row, x0 =
// w + kw - pad. They come from the aligned float4 at or below x0 and, unless
// x0 is itself aligned, the next one -- two 16-byte loads instead of four
// gathers. A block outside its row is not loaded and reads as zeros, which is
// exactly the padding (the row holds whole blocks, as W % 4 == 0).
__device__ __forceinline__ float pick(const float4 &a, const float4 &b, int i) {
    switch (i) {
        case 0: return a.x;
        case 1: return a.y;
        case 2: return a.z;
        case 3: return a.w;
        case 4: return b.x;
        case 5: return b.y;
        case 6: return b.z;
        default: return b.w;
    }
}

template <bool NT>
__global__ __launch_bounds__(kBlock) void im2col_s1_kernel(const float *__restrict__ im, float *__restrict__ col,
                                                           ColGeom g, uint32_t nv) {
    const uint32_t base = xcd_block(blockIdx.x, gridDim.x) * (kBlock * kUnroll) + threadIdx.x;
    const float4 zero = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#if DKZ_IM2COL_S1_CLAMP
    // Every load is issued before the first is used: a block outside its
    // row (or a float4 past the column's end) loads an in-range block --
    // the row clamped into the image, the block into the row -- and is then
    // replaced by zeros, so no load waits on a branch.
    float4 a[kUnroll], b[kUnroll];
    uint32_t use[kUnroll];  // bit 0: a inside the row, bit 1: b, bits 2..3: x0 mod 4
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const uint32_t q4 = base + u * kBlock;
        const ColPos q = col_pos((q4 < nv ? q4 : 0u) << 2, g);
        const int y = (int)(q.h + q.kh) - (int)g.p;
        const bool yin = y >= 0 && y < (int)g.H;
        const int yc = y < 0 ? 0 : (y >= (int)g.H ? (int)g.H - 1 : y);
        const int x0 = (int)(q.w + q.kw) - (int)g.p;
        const int sh = x0 & 3;  // x0 mod 4, also for x0 < 0
        const int xa = x0 - sh;  // aligned start of the first block
        const int xb = xa + 4;
        const int wl = (int)g.W - 4;  // last block start (W % 4 == 0, W > 0)
        const bool ain = yin && xa >= 0 && xa <= wl;
        const bool bin = yin && sh != 0 && xb >= 0 && xb <= wl;
        const int xac = xa < 0 ? 0 : (xa > wl ? wl : xa);
        const int xbc = sh == 0 ? xac : (xb < 0 ? 0 : (xb > wl ? wl : xb));
        const uint32_t row4 = ((q.c * g.H + (uint32_t)yc) * g.W) >> 2;
        a[u] = ld4<false>(im, row4 + (uint32_t)(xac >> 2));
        b[u] = ld4<false>(im, row4 + (uint32_t)(xbc >> 2));
        use[u] = (ain ? 1u : 0u) | (bin ? 2u : 0u) | ((uint32_t)sh << 2);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const uint32_t q4 = base + u * kBlock;
        if (q4 >= nv) continue;
        const float4 va = (use[u] & 1u) ? a[u] : zero;
        const float4 vb = (use[u] & 2u) ? b[u] : zero;
        const int sh = (int)(use[u] >> 2);
        st4<NT>(col, q4, make_float4(pick(va, vb, sh), pick(va, vb, sh + 1), pick(va, vb, sh + 2),
                                     pick(va, vb, sh + 3)));
    }
#else
    float4 out[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const uint32_t q4 = base + u * kBlock;
        out[u] = zero;
        if (q4 >= nv) continue;
        const ColPos q = col_pos(q4 << 2, g);
        const int y = (int)(q.h + q.kh) - (int)g.p;
        if (y < 0 || y >= (int)g.H) continue;
        const int x0 = (int)(q.w + q.kw) - (int)g.p;
        const int sh = x0 & 3;  // x0 mod 4, also for x0 < 0
        const int xa = x0 - sh;  // aligned start of the first block
        const int xb = xa + 4;
        const uint32_t row4 = ((q.c * g.H + (uint32_t)y) * g.W) >> 2;
        // A block is loaded only when it lies within the row: 0 <= start < W.
        const float4 a = xa >= 0 && xa < (int)g.W ? ld4<false>(im, row4 + (uint32_t)(xa >> 2)) : zero;
        const float4 b = sh != 0 && xb >= 0 && xb < (int)g.W ? ld4<false>(im, row4 + (uint32_t)(xb >> 2)) : zero;
        out[u] = make_float4(pick(a, b, sh), pick(a, b, sh + 1), pick(a, b, sh + 2), pick(a, b, sh + 3));
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const uint32_t q4 = base + u * kBlock;
        if (q4 < nv) st4<NT>(col, q4, out[u]);
    }
#endif
}

__global__ __launch_bounds__(kBlock) void im2col_scalar_kernel(const float *__restrict__ im, float *__restrict__ col,
                                                               ColGeom g, uint32_t n) {
    for (uint32_t e = blockIdx.x * kBlock + threadIdx.x; e < n; e += gridDim.x * kBlock) col[e] = im2col_at(im, e, g);
}

// Image element e = (c, y, x): its value plus every column entry that im2col
// took from it, in ascending (kh, kw). The taps are visited in batches of
// kTapBatch (a whole 3x3 window at once): a batch's loads are all issued
// before its adds, which then run in tap order and skip the taps that fall
// outside the column buffer. S1: stride 1, so output position
// (h, w) = (y + p - kh, x + p - kw) needs no division.
constexpr int kTapBatch = 9;

template <bool S1>
__device__ __forceinline__ float col2im_at(const float *__restrict__ col, float acc, uint32_t e, const ColGeom &g) {
    const uint32_t t = fdiv(e, g.div_w);
    const uint32_t x = e - t * g.W;
    const uint32_t c = fdiv(t, g.div_h);
    const uint32_t y = t - c * g.H;
    const uint32_t plane = g.div_plane.d;
    const uint32_t taps = g.k * g.k;
    for (uint32_t t0 = 0; t0 < taps; t0 += kTapBatch) {
        float v[kTapBatch];
        bool ok[kTapBatch];
#pragma unroll
        for (int u = 0; u < kTapBatch; ++u) {
            const uint32_t tap = t0 + u;
            const uint32_t kh = fdiv(tap, g.div_k);
            const uint32_t kw = tap - kh * g.k;
            const int hy = (int)(y + g.p) - (int)kh;  // h*stride for the output row that used this tap
            const int wx = (int)(x + g.p) - (int)kw;
            const uint32_t h = S1 ? (uint32_t)hy : fdiv((uint32_t)hy, g.div_s);
            const uint32_t w = S1 ? (uint32_t)wx : fdiv((uint32_t)wx, g.div_s);
            ok[u] = tap < taps && hy >= 0 && wx >= 0 && h < g.Ho && w < g.Wo &&
                    (S1 || (h * g.s == (uint32_t)hy && w * g.s == (uint32_t)wx));
            v[u] = ok[u] ? col[((c * g.k + kh) * g.k + kw) * plane + h * g.Wo + w] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kTapBatch; ++u) acc = ok[u] ? acc + v[u] : acc;
    }
    return acc;
}

template <bool S1>
__global__ __launch_bounds__(kBlock) void col2im_kernel(const float *__restrict__ col, float *__restrict__ im,
                                                        ColGeom g, uint32_t n) {
    const uint32_t e = blockIdx.x * kBlock + threadIdx.x;
    if (e < n) im[e] = col2im_at<S1>(col, im[e], e, g);
}

// gpu.zig:652-653: height_col = (height + 2*pad - ksize)/stride + 1 in usize.
int make_geom(int channels, int height, int width, int ksize, int stride, int pad, ColGeom *g, uint64_t *ncol,
              uint64_t *nim) {
    DKZ_REQUIRE(channels >= 0 && height >= 0 && width >= 0 && pad >= 0);
    DKZ_REQUIRE(ksize >= 1 && stride >= 1);
    DKZ_REQUIRE((int64_t)height + 2 * (int64_t)pad >= ksize && (int64_t)width + 2 * (int64_t)pad >= ksize);
    const uint64_t ho = ((uint64_t)height + 2 * (uint64_t)pad - ksize) / stride + 1;
    const uint64_t wo = ((uint64_t)width + 2 * (uint64_t)pad - ksize) / stride + 1;
    *ncol = (uint64_t)channels * ksize * ksize * ho * wo;
    *nim = (uint64_t)channels * height * width;
    DKZ_REQUIRE(*ncol <= kMaxElems && *nim <= kMaxElems);
    DKZ_REQUIRE(ho * stride + ksize + (uint64_t)height + 2 * (uint64_t)pad <= kMaxElems);
    g->H = (uint32_t)height;
    g->W = (uint32_t)width;
    g->Ho = (uint32_t)ho;
    g->Wo = (uint32_t)wo;
    g->k = (uint32_t)ksize;
    g->s = (uint32_t)stride;
    g->p = (uint32_t)pad;
    g->div_plane = make_fastdiv((uint32_t)(ho * wo));
    g->div_wo = make_fastdiv((uint32_t)wo);
    g->div_k = make_fastdiv((uint32_t)ksize);
    g->div_w = make_fastdiv(width > 0 ? (uint32_t)width : 1u);
    g->div_h = make_fastdiv(height > 0 ? (uint32_t)height : 1u);
    g->div_s = make_fastdiv((uint32_t)stride);
    return 0;
}

}  // namespace

}  // namespace dkz

using namespace dkz;

extern "C" {

int dkz_im2col(const float *im, int channels, int height, int width, int ksize, int stride, int pad, float *col) {
    ColGeom g;
    uint64_t ncol, nim;
    DKZ_TRY(make_geom(channels, height, width, ksize, stride, pad, &g, &ncol, &nim));
    if (ncol == 0) return 0;
    DKZ_REQUIRE(im != nullptr && col != nullptr);
    const uint32_t n = (uint32_t)ncol;
    if (stride == 1 && width % 4 == 0 && g.Wo % 4 == 0 && aligned16(im) && aligned16(col)) {
        const uint32_t nv = n >> 2;  // n % 4 == 0 as Wo % 4 == 0
        const uint32_t grid = div_up(nv, (uint64_t)kBlock * kUnroll);
        return launch("im2col_s1", im2col_s1_kernel<(DKZ_HINT_IM2COL & 2) != 0>, dim3(grid), dim3(kBlock), im, col,
                      g, nv);
    }
    if (aligned16(col)) {
        const uint32_t nv = n >> 2;
        const uint32_t grid = nv == 0 ? 1u : div_up(nv, (uint64_t)kBlock * kUnroll);
        return launch("im2col", im2col_vec_kernel<(DKZ_HINT_IM2COL & 2) != 0>, dim3(grid), dim3(kBlock), im, col,
                      g, n);
    }
    const uint32_t grid = div_up(n, kBlock) < 65536u ? div_up(n, kBlock) : 65536u;
    return launch("im2col", im2col_scalar_kernel, dim3(grid), dim3(kBlock), im, col, g, n);
}

int dkz_col2im(const float *col, int channels, int height, int width, int ksize, int stride, int pad, float *im) {
    ColGeom g;
    uint64_t ncol, nim;
    DKZ_TRY(make_geom(channels, height, width, ksize, stride, pad, &g, &ncol, &nim));
    if (nim == 0) return 0;
    DKZ_REQUIRE(im != nullptr && col != nullptr);
    const uint32_t n = (uint32_t)nim;
    if (stride == 1) return launch("col2im", col2im_kernel<true>, dim3(div_up(n, kBlock)), dim3(kBlock), col, im, g, n);
    return launch("col2im", col2im_kernel<false>, dim3(div_up(n, kBlock)), dim3(kBlock), col, im, g, n);
}

}  // extern "C"
