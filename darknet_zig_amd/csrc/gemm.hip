// gemm.hip -- C = alpha*op(A)*op(B) + beta*C, row-major (src/gpu.zig:671-719,
// CPU twin src/gemm.zig:47-278), on gfx950's fp32 matrix cores.
//
// A workgroup of four wave64s owns a BM x BN tile of C; each wave a
// (BM/2) x (BN/2) quarter of it, as (BM/64) x (BN/64) blocks of 32x32 that
// v_mfma_f32_32x32x2_f32 accumulates two k at a time (products exact, sums
// in fp32). K advances in slabs of 16: every thread loads its share of the
// next A and B slabs into registers while the waves run the current slab's
// MFMAs out of LDS; the registers then go to the other LDS buffer, so each
// slab costs one barrier.
//
// LDS keeps both slabs k-contiguous per row (As[i][k], Bs[j][k], rows padded
// to 20 words). Within a slab the sixteen k are dealt to the MFMAs so that
// MFMA s takes k = s from lanes 0-31 and k = 8 + s from lanes 32-63; a lane
// therefore needs eight consecutive k of its row, which two 128-bit LDS reads
// fetch (the 80-byte row pitch puts eight lanes' reads in distinct banks).
// The order in which the k of one output are summed changes; any order is as
// valid as the CPU twin's, which depends on its host's vector width.
//
// Global loads walk each operand's contiguous dimension in float4s (k for A
// row-major and B transposed -- stored to LDS as they are -- m or n for the
// other layouts, scattered to four LDS rows). Rows, columns and k past the
// matrix load as 0; a misaligned operand loads element by element.
//
// Small problems split K: the grid holds `splits` copies of the tile grid,
// each summing one range of K into a partial tile in the library's scratch,
// and a second kernel adds a tile's partials in split order and applies
// alpha and beta -- deterministic, no atomics. The epilogue follows
// gemm.zig:121-131 then :180-184: beta == 0 clears C (NaN included), beta == 1
// keeps it, anything else scales it; then C += alpha*acc.
//
// Workgroups take tiles in groups of 8 tile-rows, so that the tiles running
// at once share A and B panels, and neighbouring tile numbers are placed on
// one XCD (workgroups are dealt to the 8 XCDs round robin) so that they share
// its L2.
//
// The same kernel runs a convolutional layer's three per-image loops as one
// call each (dkz_convolution_forward, _weight_gradient, _data_gradient): its
// B operand is then an im2col gathered inside the slab loads (of the input,
// or of delta), the grid's second dimension runs over images and groups,
// and small images, strided data gradients and the weight gradient's long K
// get their own column orders, pixel mappings and splits (see ConvB and the
// entry points).
#include <algorithm>
#include <type_traits>
#include <vector>

#include "dkz_device.hpp"
#include "dkz_internal.hpp"

namespace dkz {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 16;
constexpr int kPitch = kBK + 4;  // LDS row pitch in words
constexpr int kGroupM = 8;
constexpr int kXcds = 8;

// Slabs in flight in the 64x64 kernel (build-time tunable).
#ifndef DKZ_GEMM_SMALL_PREFETCH
#define DKZ_GEMM_SMALL_PREFETCH 2
#endif

// Unchecked float4 loads for slabs wholly inside the matrix (build-time
// switch, for measurement).
#ifndef DKZ_GEMM_FULL_SLABS
#define DKZ_GEMM_FULL_SLABS 1
#endif

// Tiles wholly inside both operands take a loop without edge checks whose
// slab loads stay in flight (build-time switch, for measurement). Config 2's
// per-image convolution GEMMs 22.9 / 19.5 / 20.8 -> 21.0 / 18.3 / 19.8 us,
// 4096^3 109 -> 111 TFLOP/s, 8192x8192x4096 122 -> 126.
#ifndef DKZ_GEMM_FULL_TILES
#define DKZ_GEMM_FULL_TILES 1
#endif

// Workgroups per CU that a split-K grid aims for (build-time tunable).
#ifndef DKZ_GEMM_SPLIT_TARGET
#define DKZ_GEMM_SPLIT_TARGET 2
#endif

// The weight gradient: 128x128 tiles when filters per group fill them
// (DKZ_WGRAD_BIG), and with ksize 1 the workgroups per CU its K split aims
// for.
#ifndef DKZ_WGRAD_BIG
#define DKZ_WGRAD_BIG 1
#endif
#ifndef DKZ_WGRAD_TARGET_RAW
#define DKZ_WGRAD_TARGET_RAW 2
#endif
// The shortest K range of a weight-gradient split: below it the partial tiles
// the reduce reads cost more than the parallelism gains.
#ifndef DKZ_WGRAD_MIN_CHUNK
#define DKZ_WGRAD_MIN_CHUNK 512
#endif

// The B operand of a convolution taken straight from the image (implicit
// im2col): B[k][p] = im2col(image)[k][p] for k = (c, kh, kw) over a group's
// channels and p = (h, w) over the output positions (im2col.zig:13-49).
struct ConvB {
    uint32_t H, W, Wo, ksz, stride;
    int32_t pad, pad_x;  // rows and columns (negative: the window starts inside the image)
    FastDiv div_kk, div_k, div_wo;  // ksz*ksz, ksz, Wo
    uint32_t s1;    // stride 1, W % 4 == 0, Wo % 4 == 0, images 16-byte aligned
    uint32_t row4;  // Wo % 4 == 0: a float4's four positions share an output row
    // Weight gradient (k runs over image and position): positions per image,
    // and the element strides from one image to the next of delta (A) and of
    // the input (B); npos4: npos % 4 == 0, so no float4 spans two images.
    uint32_t npos;
    FastDiv div_npos;
    uint32_t a_img, b_img, npos4, a_vec, b_vec;  // a_vec / b_vec: delta / input 16-byte aligned
    // Products whose columns run over (image, position) (kSpan): C's element
    // stride from one image to the next; B's is b_img, the positions per
    // image npos.
    uint32_t c_img;
    // Products over one phase of a strided data gradient (kPhase): column j is
    // position (yq, xq) = (j / wp, j % wp) of the phase, i.e. input pixel
    // (ph_s*yq + ph_py, ph_s*xq + ph_px) of an image ph_w wide.
    FastDiv div_wp;
    uint32_t ph_s, ph_py, ph_px, ph_w;
};

// One phase of a strided data gradient in a launch that runs several (kPhase):
// its flipped taps (A, `k` = filters x taps per group), their window (ksz
// columns, kk = rows x columns) and pads over delta, and the phase's pixel
// offsets (py, px). Grid row y runs phase y / zrows over (image, group)
// y % zrows.
struct PhaseDesc {
    const float *a;
    uint32_t k, vec_a, ksz, py, px;
    int32_t pad, pad_x;
    FastDiv div_kk, div_k;
};
constexpr int kMaxPhases = 4;

struct GemmArgs {
    const float *a;
    const float *b;
    float *c;
    float *partial;  // splits > 1: [splits][m][n] partial tiles
    uint32_t m, n, k, lda, ldb, ldc;
    float alpha, beta;
    uint32_t tiles_m, tiles_n, splits, k_chunk;
    uint32_t vec_a, vec_b;  // operand 16-byte aligned with a leading dimension % 4 == 0
    // Batched launches (one workgroup row per matrix product, z = blockIdx.y):
    // A at a + (z % zgroups) * a_z, B at b + z * b_z, C at c + z * c_z.
    uint32_t zgroups, a_z, b_z, c_z;
    ConvB cv;  // implicit-im2col kernels only
    PhaseDesc ph[kMaxPhases];  // kPhase kernels only
    uint32_t zrows;
};

__device__ __forceinline__ void tile_of(uint32_t w, const GemmArgs &g, uint32_t &tm, uint32_t &tn, uint32_t &split) {
    const uint32_t tiles = g.tiles_m * g.tiles_n;
    const uint32_t total = tiles * g.splits;
    uint32_t t = w;
    if (total % kXcds == 0) t = (w % kXcds) * (total / kXcds) + w / kXcds;
    split = t / tiles;
    t -= split * tiles;
    const uint32_t per_group = kGroupM * g.tiles_n;
    const uint32_t first_m = (t / per_group) * kGroupM;
    const uint32_t gsize = g.tiles_m - first_m < (uint32_t)kGroupM ? g.tiles_m - first_m : (uint32_t)kGroupM;
    const uint32_t in_group = t % per_group;
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
}

// Four consecutive elements p[0..3] of a row (or column) starting at `idx`,
// where `avail` of them exist (0..4). vec: idx is a multiple of 4 and p is
// 16-byte aligned.
__device__ __forceinline__ float4 load4(const float *p, uint32_t idx, uint32_t avail, bool vec) {
    if (avail >= 4 && vec) return *reinterpret_cast<const float4 *>(p + idx);
    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (avail > 0) v.x = p[idx];
    if (avail > 1) v.y = p[idx + 1];
    if (avail > 2) v.z = p[idx + 2];
    if (avail > 3) v.w = p[idx + 3];
    return v;
}

// Element i (0..7) of the eight floats a, b.
__device__ __forceinline__ float pick8(const float4 &a, const float4 &b, int i) {
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

// One operand's slab loader. ROWK: the operand's rows run along the tile
// dimension with k contiguous (A row-major, B transposed); otherwise its rows
// run along k with the tile dimension contiguous. R rows of the tile.
template <int R, bool ROWK>
struct Slab {
    static constexpr int kLoads = R * kBK / 4 / kBlock;  // float4s per thread
    float4 v[kLoads];

    // rows: tile rows available (m - m0 or n - n0); k0/kmax: the slab's first
    // k and the end of this split's range.
    template <bool FULL = false>
    __device__ __forceinline__ void load(const float *p, uint32_t ld, uint32_t r0, uint32_t rows, uint32_t k0,
                                         uint32_t kend, bool vec, int tid) {
        // A whole slab inside the matrix (the usual case): every float4 is
        // there, so no per-element checks (a branch the whole workgroup
        // takes). FULL: the caller has checked that for every slab of the tile.
        if (FULL || (DKZ_GEMM_FULL_SLABS && vec && rows >= (uint32_t)R && kend - k0 >= (uint32_t)kBK)) {
#pragma unroll
            for (int l = 0; l < kLoads; ++l) {
                const int f = tid + l * kBlock;
                if constexpr (ROWK) {
                    const uint32_t r = f / (kBK / 4), q = f % (kBK / 4);
                    v[l] = *reinterpret_cast<const float4 *>(p + (r0 + r) * ld + k0 + 4 * q);
                } else {
                    const uint32_t kr = f % kBK, q = f / kBK;
                    v[l] = *reinterpret_cast<const float4 *>(p + (k0 + kr) * ld + r0 + 4 * q);
                }
            }
            return;
        }
#pragma unroll
        for (int l = 0; l < kLoads; ++l) {
            const int f = tid + l * kBlock;  // float4 number within the slab
            if constexpr (ROWK) {
                const uint32_t r = f / (kBK / 4), q = f % (kBK / 4);
                const uint32_t kk = k0 + 4 * q;
                const uint32_t avail = (r < rows && kk < kend) ? (kend - kk < 4 ? kend - kk : 4) : 0;
                v[l] = load4(p, (r0 + r) * ld + kk, avail, vec);
            } else {
                // k fastest across lanes: the transposing LDS stores below then
                // fall in distinct banks (row pitch 80 B: 16 lanes per k-run
                // cover 16 banks, the next 16 lanes start 16 banks further).
                const uint32_t kr = f % kBK, q = f / kBK;
                const uint32_t rr = 4 * q;
                const uint32_t avail = (k0 + kr < kend && rr < rows) ? (rows - rr < 4 ? rows - rr : 4) : 0;
                v[l] = load4(p, (k0 + kr) * ld + r0 + rr, avail, vec);
            }
        }
    }

    __device__ __forceinline__ void store(float *s, int tid) const {
#pragma unroll
        for (int l = 0; l < kLoads; ++l) {
            const int f = tid + l * kBlock;
            if constexpr (ROWK) {
                const int r = f / (kBK / 4), q = f % (kBK / 4);
                *reinterpret_cast<float4 *>(s + r * kPitch + 4 * q) = v[l];
            } else {
                const int kr = f % kBK, q = f / kBK;
                float *d = s + (4 * q) * kPitch + kr;
                d[0] = v[l].x;
                d[kPitch] = v[l].y;
                d[2 * kPitch] = v[l].z;
                d[3 * kPitch] = v[l].w;
            }
        }
    }
};

// Gather modes of the implicit im2col operand: kRaw reads the input itself as
// a k x npos matrix (what the layer multiplies by when ksize == 1), kGather
// takes each element's tap, kTwoBlock takes four positions of one output row
// (stride 1, W and Wo multiples of 4) from the aligned float4 at or below
// x0 = w + kw - pad and, unless x0 is aligned, the next one; a block outside
// its row reads as the padding's zeros. kRow (Wo a multiple of 4, any
// stride) takes four positions of one output row: the tap, the row and its
// bounds once, then four loads stride apart.
constexpr int kRaw = 0, kGather = 1, kTwoBlock = 2, kRow = 3;

// im2col(img)[kidx][p] (0 in the padding).
template <int MODE>
__device__ __forceinline__ float conv_col1(const float *img, const ConvB &cv, uint32_t kidx, uint32_t p) {
    if constexpr (MODE == kRaw) {
        return img[kidx * cv.npos + p];
    } else {
        const uint32_t c = fdiv(kidx, cv.div_kk), rem = kidx - c * cv.div_kk.d;
        const uint32_t kh = fdiv(rem, cv.div_k), kw = rem - kh * cv.ksz;
        const uint32_t h = fdiv(p, cv.div_wo), w = p - h * cv.Wo;
        const int y = (int)(h * cv.stride + kh) - cv.pad;
        const int x = (int)(w * cv.stride + kw) - cv.pad_x;
        return y >= 0 && y < (int)cv.H && x >= 0 && x < (int)cv.W ? img[(c * cv.H + (uint32_t)y) * cv.W + (uint32_t)x]
                                                                   : 0.0f;
    }
}

// im2col(img)[kidx][p0 .. p0+avail-1], zeros past avail. kTwoBlock needs
// avail == 4 and p0 % 4 == 0; kRaw loads a float4 when npos4 and avail == 4.
template <int MODE>
__device__ __forceinline__ float4 conv_col4(const float *img, const ConvB &cv, uint32_t kidx, uint32_t p0,
                                            uint32_t avail) {
    const float4 zero = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if constexpr (MODE == kTwoBlock) {
        const uint32_t c = fdiv(kidx, cv.div_kk), rem = kidx - c * cv.div_kk.d;
        const uint32_t kh = fdiv(rem, cv.div_k), kw = rem - kh * cv.ksz;
        const uint32_t h = fdiv(p0, cv.div_wo), w = p0 - h * cv.Wo;
        const int y = (int)(h + kh) - cv.pad;
        if (y < 0 || y >= (int)cv.H) return zero;
        const int x0 = (int)(w + kw) - cv.pad_x;
        const int sh = x0 & 3, xa = x0 - sh, xb = xa + 4;
        const uint32_t row4 = ((c * cv.H + (uint32_t)y) * cv.W) >> 2;
        const float4 a = xa >= 0 && xa < (int)cv.W ? ld4<false>(img, row4 + (uint32_t)(xa >> 2)) : zero;
        const float4 b = sh != 0 && xb >= 0 && xb < (int)cv.W ? ld4<false>(img, row4 + (uint32_t)(xb >> 2)) : zero;
        return make_float4(pick8(a, b, sh), pick8(a, b, sh + 1), pick8(a, b, sh + 2), pick8(a, b, sh + 3));
    } else if constexpr (MODE == kRow) {
        const uint32_t c = fdiv(kidx, cv.div_kk), rem = kidx - c * cv.div_kk.d;
        const uint32_t kh = fdiv(rem, cv.div_k), kw = rem - kh * cv.ksz;
        const uint32_t h = fdiv(p0, cv.div_wo), w = p0 - h * cv.Wo;
        const int y = (int)(h * cv.stride + kh) - cv.pad;
        if (y < 0 || y >= (int)cv.H) return zero;
        const float *row = img + (c * cv.H + (uint32_t)y) * cv.W;
        const int x0 = (int)(w * cv.stride + kw) - cv.pad_x;
        float4 out = zero;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int x = x0 + j * (int)cv.stride;
            if (x >= 0 && x < (int)cv.W) ::dkz::lane(out, j) = row[x];
        }
        return out;
    } else {
        if (MODE == kRaw && avail == 4 && cv.npos4 && cv.b_vec)
            return ld4<false>(img + kidx * cv.npos, p0 >> 2);
        float4 out = zero;
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j)
            if (j < avail) ::dkz::lane(out, j) = conv_col1<MODE>(img, cv, kidx, p0 + j);
        return out;
    }
}

// Columns q .. q+avail-1 of the im2col over (image, position) pairs, npos
// positions per image, images b_img apart: one image's conv_col4 when npos
// % 4 == 0 (!ODD; kTwoBlock needs it), else element by element, the tap
// decomposed once and (image, position) stepped along.
template <int MODE, bool ODD>
__device__ __forceinline__ float4 conv_span4(const float *img0, const ConvB &cv, uint32_t kidx, uint32_t q,
                                             uint32_t avail) {
    uint32_t i = fdiv(q, cv.div_npos), p = q - i * cv.npos;
    if constexpr (!ODD) return conv_col4<MODE>(img0 + (size_t)i * cv.b_img, cv, kidx, p, avail);
    static_assert(!ODD || (MODE != kTwoBlock && MODE != kRow), "row gathers need npos % 4 == 0");
    float4 out = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if constexpr (MODE == kRaw) {
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            if (j < avail) ::dkz::lane(out, j) = img0[(size_t)i * cv.b_img + kidx * cv.npos + p];
            if (++p == cv.npos) p = 0, ++i;
        }
    } else {
        const uint32_t c = fdiv(kidx, cv.div_kk), rem = kidx - c * cv.div_kk.d;
        const uint32_t kh = fdiv(rem, cv.div_k), kw = rem - kh * cv.ksz;
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            const uint32_t h = fdiv(p, cv.div_wo), w = p - h * cv.Wo;
            const int y = (int)(h * cv.stride + kh) - cv.pad;
            const int x = (int)(w * cv.stride + kw) - cv.pad_x;
            if (j < avail && y >= 0 && y < (int)cv.H && x >= 0 && x < (int)cv.W)
                ::dkz::lane(out, j) = img0[(size_t)i * cv.b_img + (c * cv.H + (uint32_t)y) * cv.W + (uint32_t)x];
            if (++p == cv.npos) p = 0, ++i;
        }
    }
    return out;
}

// The implicit im2col operand's slab. ROWK false: B of the forward product
// (rows along k = kidx, the positions contiguous). ROWK true: B of the weight
// gradient, transposed (rows along the tile dimension = kidx, k = image *
// npos + position). Same layouts and LDS stores as the ordinary slabs.
template <int R, bool ROWK, int MODE, int SPAN = 0>  // SPAN: 0 no, 1 npos % 4 == 0, 2 any npos
struct ConvSlab : Slab<R, ROWK> {
    using Slab<R, ROWK>::kLoads;
    using Slab<R, ROWK>::v;

    __device__ __forceinline__ void load_conv(const float *img0, const ConvB &cv, uint32_t r0, uint32_t rows,
                                              uint32_t k0, uint32_t kend, int tid) {
        const float4 zero = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int l = 0; l < kLoads; ++l) {
            const int f = tid + l * kBlock;
            float4 out = zero;
            if constexpr (!ROWK && SPAN == 0) {
                const uint32_t kr = f % kBK, rr = 4 * (f / kBK);
                const uint32_t kidx = k0 + kr;
                if (kidx < kend && rr < rows)
                    out = conv_col4<MODE>(img0, cv, kidx, r0 + rr, rows - rr < 4 ? rows - rr : 4);
            } else if constexpr (!ROWK) {
                const uint32_t kr = f % kBK, rr = 4 * (f / kBK);
                const uint32_t kidx = k0 + kr;
                if (kidx < kend && rr < rows)
                    out = conv_span4<MODE, SPAN == 2>(img0, cv, kidx, r0 + rr, rows - rr < 4 ? rows - rr : 4);
            } else {
                const uint32_t r = f / (kBK / 4), kk = k0 + 4 * (f % (kBK / 4));
                if (r < rows && kk < kend) {
                    // The four k are (image, position) pairs, like the
                    // columns of a spanning forward product.
                    const uint32_t kidx = r0 + r, avail = kend - kk < 4 ? kend - kk : 4;
                    if (cv.npos4) out = conv_span4<MODE, false>(img0, cv, kidx, kk, avail);
                    else if constexpr (MODE != kTwoBlock && MODE != kRow)
                        out = conv_span4<MODE, true>(img0, cv, kidx, kk, avail);
                }
            }
            v[l] = out;
        }
    }
};

// A of the weight gradient: delta, row f of the product holding filter f's
// deltas of every image in turn -- k = image * npos + position.
template <int R>
struct SegSlab : Slab<R, true> {
    using Slab<R, true>::kLoads;
    using Slab<R, true>::v;

    __device__ __forceinline__ void load_seg(const float *a0, const ConvB &cv, uint32_t r0, uint32_t rows,
                                             uint32_t k0, uint32_t kend, int tid) {
        const float4 zero = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int l = 0; l < kLoads; ++l) {
            const int f = tid + l * kBlock;
            const uint32_t r = f / (kBK / 4), kk = k0 + 4 * (f % (kBK / 4));
            float4 out = zero;
            if (r < rows && kk < kend) {
                const uint32_t row = r0 + r, avail = kend - kk < 4 ? kend - kk : 4;
                if (cv.npos4 && avail == 4 && cv.a_vec) {
                    const uint32_t i = fdiv(kk, cv.div_npos);
                    out = ld4<false>(a0 + (size_t)i * cv.a_img + row * cv.npos, (kk - i * cv.npos) >> 2);
                } else {
#pragma unroll
                    for (uint32_t j = 0; j < 4; ++j) {
                        if (j >= avail) break;
                        const uint32_t i = fdiv(kk + j, cv.div_npos);
                        ::dkz::lane(out, j) = a0[(size_t)i * cv.a_img + row * cv.npos + (kk + j - i * cv.npos)];
                    }
                }
            }
            v[l] = out;
        }
    }
};

// D: slabs in flight. The loads of slab s + D are issued while slab s is
// multiplied, from a ring of D register sets; the 128x128 kernel does four
// times the MFMAs per slab of the 64x64 one and runs with D = 1, the 64x64
// one -- used when few workgroups share a CU -- with DKZ_GEMM_SMALL_PREFETCH.
// IM: a convolution's operands. kFwd + mode: B of an NN product is the
// implicit im2col of the image; kWgrad + mode: the weight gradient, an NT
// product whose A is delta and whose B is the im2col, k running over image
// and position; kSpan + mode: as kFwd, but the columns run over (image,
// position) of every image, so small images fill whole tiles (kSpanOdd: the
// positions per image are not a multiple of 4); kPhase + mode: as kFwd, but
// column j goes to the pixel of one phase of a strided data gradient (see
// ConvB) (modes: kRaw, kGather, kTwoBlock). Each workgroup row z =
// blockIdx.y computes its own product (see GemmArgs).
constexpr int kImNone = -1, kFwd = 0, kWgrad = 8, kSpan = 16, kSpanOdd = 24, kPhase = 32, kPhaseSpan = 40,
              kPhaseSpanOdd = 48;

template <int BM, int BN, bool TA, bool TB, int D, int IM = kImNone>
__global__ __launch_bounds__(kBlock, 4) void gemm_mfma_kernel(GemmArgs g) {
    constexpr bool kWg = IM >= kWgrad && IM < kSpan;
    constexpr bool kPh = IM >= kPhase;
    constexpr bool kSp = (IM >= kSpan && IM < kPhase) || IM >= kPhaseSpan;
    constexpr int kSpanKind = !kSp ? 0 : ((IM >= kSpanOdd && IM < kPhase) || IM >= kPhaseSpanOdd) ? 2 : 1;
    constexpr int kMode = IM == kImNone ? 0 : IM % 8;
    static_assert(IM == kImNone || (!TA && TB == kWg), "forward: NN; weight gradient: NT");
    constexpr int WM = BM / 2, WN = BN / 2, TM = WM / 32, TN = WN / 32;
    // A wave with fewer than four 32x32 blocks spreads each block's MFMAs over
    // NC accumulators (MFMA q of a slab into accumulator q % NC), so that four
    // independent MFMAs are always in flight; they are added at the end.
    constexpr int NC = TM * TN >= 4 ? 1 : 4 / (TM * TN);
    __shared__ float As[2][BM * kPitch];
    __shared__ float Bs[2][BN * kPitch];

    uint32_t z = blockIdx.y;
    // A and the gather geometry; a phase row of a strided data gradient takes
    // its phase's taps, window and pixel offsets instead (fields picked with
    // constant indexes, so the kernel arguments stay where they are).
    const float *a_base = g.a;
    uint32_t k_all = g.k, k_chunk = g.k_chunk, lda = g.lda, a_z = g.a_z, vec_a = g.vec_a;
    ConvB cv = g.cv;
    if constexpr (kPh) {
        const uint32_t p = z / g.zrows;
        z -= p * g.zrows;
#define DKZ_PHASE_FIELD(f) (p == 0 ? g.ph[0].f : p == 1 ? g.ph[1].f : p == 2 ? g.ph[2].f : g.ph[3].f)
        a_base = DKZ_PHASE_FIELD(a);
        k_all = DKZ_PHASE_FIELD(k);
        vec_a = DKZ_PHASE_FIELD(vec_a);
        cv.ksz = DKZ_PHASE_FIELD(ksz);
        cv.pad = DKZ_PHASE_FIELD(pad);
        cv.pad_x = DKZ_PHASE_FIELD(pad_x);
        cv.div_kk = DKZ_PHASE_FIELD(div_kk);
        cv.div_k = DKZ_PHASE_FIELD(div_k);
        cv.ph_py = DKZ_PHASE_FIELD(py);
        cv.ph_px = DKZ_PHASE_FIELD(px);
#undef DKZ_PHASE_FIELD
        k_chunk = k_all;
        lda = k_all;
        a_z = g.m * k_all;
    }
    uint32_t tm, tn, split;
    tile_of(blockIdx.x, g, tm, tn, split);
    const float *ga = a_base + (size_t)(z % g.zgroups) * a_z;
    const float *gb = g.b + (size_t)z * g.b_z;
    float *gc = g.c + (size_t)z * g.c_z;
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t rows_a = g.m - m0, rows_b = g.n - n0;
    const uint32_t kbeg = split * k_chunk;
    const uint32_t kend = kbeg + k_chunk < k_all ? kbeg + k_chunk : k_all;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;
    const int half = lane >> 5, l32 = lane & 31;

    std::conditional_t<kWg, SegSlab<BM>, Slab<BM, !TA>> sa[D];
    std::conditional_t<IM != kImNone, ConvSlab<BN, kWg, kMode, kSpanKind>, Slab<BN, TB>> sb[D];
    auto load_a = [&](auto &slab, uint32_t k0, auto full) {
        if constexpr (kWg) slab.load_seg(ga, cv, m0, rows_a, k0, kend, tid);
        else slab.template load<decltype(full)::value>(ga, lda, m0, rows_a, k0, kend, vec_a, tid);
    };
    auto load_b = [&](auto &slab, uint32_t k0, auto full) {
        if constexpr (IM != kImNone) slab.load_conv(gb, cv, n0, rows_b, k0, kend, tid);
        else slab.template load<decltype(full)::value>(gb, g.ldb, n0, rows_b, k0, kend, g.vec_b, tid);
    };

    f32x16 acc[NC][TM][TN];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int ti = 0; ti < TM; ++ti)
#pragma unroll
            for (int tj = 0; tj < TN; ++tj)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[c][ti][tj][r] = 0.0f;

    const uint32_t steps = kend > kbeg ? (kend - kbeg + kBK - 1) / kBK : 0;
    // One slab's MFMAs out of LDS buffer `cur`.
    auto compute = [&](int cur) {
        float4 af[TM][2], bf[TN][2];
#pragma unroll
        for (int ti = 0; ti < TM; ++ti) {
            const float *p = As[cur] + (wm0 + ti * 32 + l32) * kPitch + 8 * half;
            af[ti][0] = *reinterpret_cast<const float4 *>(p);
            af[ti][1] = *reinterpret_cast<const float4 *>(p + 4);
        }
#pragma unroll
        for (int tj = 0; tj < TN; ++tj) {
            const float *p = Bs[cur] + (wn0 + tj * 32 + l32) * kPitch + 8 * half;
            bf[tj][0] = *reinterpret_cast<const float4 *>(p);
            bf[tj][1] = *reinterpret_cast<const float4 *>(p + 4);
        }
#pragma unroll
        for (int q = 0; q < 8; ++q)
#pragma unroll
            for (int ti = 0; ti < TM; ++ti)
#pragma unroll
                for (int tj = 0; tj < TN; ++tj)
                    acc[q % NC][ti][tj] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                        ::dkz::lane(af[ti][q >> 2], q & 3), ::dkz::lane(bf[tj][q >> 2], q & 3), acc[q % NC][ti][tj],
                        0, 0, 0);
    };
    // A tile wholly inside both operands (aligned, whole tile rows, a K range
    // of whole slabs) takes a loop without edge checks: every slab load is
    // one 128-bit load a float4, issued on every step (past the last slab
    // the last one again, unused), and the steady loop has no branch, so the
    // compiler waits only for the slab it stores while the next D - 1 stay in
    // flight. Other tiles check every element, and there the compiler waits
    // for every load in flight before a store.
    bool interior = false;
    if constexpr (IM == kImNone && DKZ_GEMM_FULL_TILES)
        interior = vec_a && g.vec_b && rows_a >= (uint32_t)BM && rows_b >= (uint32_t)BN && steps > 0 &&
                   (kend - kbeg) % kBK == 0;
    if (interior) {
        const std::true_type full{};
        const auto slab_k = [&](uint32_t x) { return kbeg + (x < steps ? x : steps - 1) * kBK; };
#pragma unroll
        for (int d = 0; d < D; ++d) {
            load_a(sa[d], slab_k(d), full);
            load_b(sb[d], slab_k(d), full);
        }
        sa[0].store(As[0], tid);
        sb[0].store(Bs[0], tid);
        load_a(sa[0], slab_k(D), full);
        load_b(sb[0], slab_k(D), full);
        __syncthreads();
        uint32_t s0 = 0;
        // steady state: every step stores slab s + 1 and loads slab s + 1 + D
        for (; s0 + D < steps; s0 += D) {
#pragma unroll
            for (int j = 0; j < D; ++j) {
                const uint32_t s = s0 + j;
                const int cur = s & 1;
                compute(cur);
                const int nx = (j + 1) % D;
                sa[nx].store(As[cur ^ 1], tid);
                sb[nx].store(Bs[cur ^ 1], tid);
                load_a(sa[nx], slab_k(s + 1 + D), full);
                load_b(sb[nx], slab_k(s + 1 + D), full);
                __syncthreads();
            }
        }
        // the last steps: every slab left is in its slot already
#pragma unroll
        for (int j = 0; j < D; ++j) {
            const uint32_t s = s0 + j;
            if (s < steps) {
                const int cur = s & 1;
                compute(cur);
                if (s + 1 < steps) {
                    const int nx = (j + 1) % D;
                    sa[nx].store(As[cur ^ 1], tid);
                    sb[nx].store(Bs[cur ^ 1], tid);
                }
                __syncthreads();
            }
        }
    } else {
        const std::false_type full{};
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if ((uint32_t)d < steps) {
                load_a(sa[d], kbeg + d * kBK, full);
                load_b(sb[d], kbeg + d * kBK, full);
            }
        }
        if (steps > 0) {
            sa[0].store(As[0], tid);
            sb[0].store(Bs[0], tid);
            // Slot 0 is free again: it takes slab D (slot X % D always holds slab X).
            if ((uint32_t)D < steps) {
                load_a(sa[0], kbeg + D * kBK, full);
                load_b(sb[0], kbeg + D * kBK, full);
            }
            __syncthreads();
        }
        for (uint32_t s0 = 0; s0 < steps; s0 += D) {
#pragma unroll
            for (int j = 0; j < D; ++j) {
                const uint32_t s = s0 + j;
                if (s >= steps) break;
                const int cur = s & 1;
                compute(cur);
                // Slab s + 1 (ring slot (j + 1) % D) goes to the other LDS buffer,
                // and its registers take the loads of slab s + 1 + D.
                const int nx = (j + 1) % D;
                if (s + 1 < steps) {
                    sa[nx].store(As[cur ^ 1], tid);
                    sb[nx].store(Bs[cur ^ 1], tid);
                    if (s + 1 + D < steps) {
                        load_a(sa[nx], kbeg + (s + 1 + D) * kBK, full);
                        load_b(sb[nx], kbeg + (s + 1 + D) * kBK, full);
                    }
                }
                __syncthreads();
            }
        }
    }

#pragma unroll
    for (int c = 1; c < NC; ++c)
#pragma unroll
        for (int ti = 0; ti < TM; ++ti)
#pragma unroll
            for (int tj = 0; tj < TN; ++tj) acc[0][ti][tj] += acc[c][ti][tj];

    // acc[0][ti][tj][r] is C(row, col) of the wave's block (ti, tj) with
    // row = 8*(r/4) + 4*(lane/32) + r%4 and col = lane%32.
#pragma unroll
    for (int ti = 0; ti < TM; ++ti)
#pragma unroll
        for (int tj = 0; tj < TN; ++tj) {
            const uint32_t j = n0 + wn0 + tj * 32 + l32;
            if (j >= g.n) continue;
            // Column j of C: position jp of image img (span), and with a
            // phase that position's pixel.
            float *cimg = gc;
            uint32_t jp = j;
            if constexpr (kSp) {
                const uint32_t img = fdiv(j, cv.div_npos);
                cimg = gc + (size_t)img * cv.c_img;
                jp = j - img * cv.npos;
            }
            float *ccol = cimg + jp;
            if constexpr (kPh) {
                const uint32_t yq = fdiv(jp, cv.div_wp), xq = jp - yq * cv.div_wp.d;
                ccol = cimg + (cv.ph_s * yq + cv.ph_py) * cv.ph_w + cv.ph_s * xq + cv.ph_px;
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t i = m0 + wm0 + ti * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
                if (i >= g.m) continue;
                if (g.splits > 1) {
                    g.partial[((size_t)split * g.m + i) * g.n + j] = acc[0][ti][tj][r];
                } else {
                    float *cp = ccol + i * g.ldc;
                    float cv = 0.0f;
                    if (g.beta != 0.0f) cv = (g.beta == 1.0f) ? *cp : *cp * g.beta;
                    *cp = cv + g.alpha * acc[0][ti][tj][r];
                }
            }
        }
}

// The split-K epilogue: C(i, j) = beta-applied C + alpha * (sum of the splits'
// partials in split order). V4: n % 4 == 0 and C's rows are float4-aligned,
// so a lane takes four consecutive columns of one row.
__device__ __forceinline__ float gemm_out(const float *cp, float s, const GemmArgs &g) {
    float cv = 0.0f;
    if (g.beta != 0.0f) cv = (g.beta == 1.0f) ? *cp : *cp * g.beta;
    return cv + g.alpha * s;
}

constexpr int kReduceBatch = 8;

template <bool V4>
__global__ __launch_bounds__(kBlock) void gemm_splitk_reduce_kernel(GemmArgs g) {
    const uint32_t mn = g.m * g.n;
    if constexpr (V4) {
        const uint32_t v = blockIdx.x * kBlock + threadIdx.x;
        if (v >= (mn >> 2)) return;
        const uint32_t e = v << 2, i = e / g.n, j = e - i * g.n;
        // Eight partials in flight at a time, added in split order; the
        // missing ones of the last batch are +0, which leaves the sum as is.
        float4 s = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (uint32_t t = 0; t < g.splits; t += kReduceBatch) {
            float4 p[kReduceBatch];
#pragma unroll
            for (int u = 0; u < kReduceBatch; ++u)
                p[u] = t + u < g.splits ? reinterpret_cast<const float4 *>(g.partial + (size_t)(t + u) * mn)[v]
                                        : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
            for (int u = 0; u < kReduceBatch; ++u) {
                s.x += p[u].x;
                s.y += p[u].y;
                s.z += p[u].z;
                s.w += p[u].w;
            }
        }
        float *cp = g.c + i * g.ldc + j;
        const float4 o = make_float4(gemm_out(cp, s.x, g), gemm_out(cp + 1, s.y, g), gemm_out(cp + 2, s.z, g),
                                     gemm_out(cp + 3, s.w, g));
        *reinterpret_cast<float4 *>(cp) = o;
    } else {
        const uint32_t e = blockIdx.x * kBlock + threadIdx.x;
        if (e >= mn) return;
        const uint32_t i = e / g.n, j = e - i * g.n;
        float s = 0.0f;
        for (uint32_t t = 0; t < g.splits; t += kReduceBatch) {
            float p[kReduceBatch];
#pragma unroll
            for (int u = 0; u < kReduceBatch; ++u) p[u] = t + u < g.splits ? g.partial[(size_t)(t + u) * mn + e] : 0.0f;
#pragma unroll
            for (int u = 0; u < kReduceBatch; ++u) s += p[u];
        }
        float *cp = g.c + i * g.ldc + j;
        *cp = gemm_out(cp, s, g);
    }
}

template <int BM, int BN, int D>
int launch_gemm(bool ta, bool tb, GemmArgs g) {
    const uint64_t total = (uint64_t)g.tiles_m * g.tiles_n * g.splits;
    DKZ_REQUIRE(total <= 0x7fffffffull);
    const dim3 grid((uint32_t)total), block(kBlock);
    if (!ta && !tb) return launch("gemm_nn", gemm_mfma_kernel<BM, BN, false, false, D>, grid, block, g);
    if (ta && !tb) return launch("gemm_tn", gemm_mfma_kernel<BM, BN, true, false, D>, grid, block, g);
    if (!ta && tb) return launch("gemm_nt", gemm_mfma_kernel<BM, BN, false, true, D>, grid, block, g);
    return launch("gemm_tt", gemm_mfma_kernel<BM, BN, true, true, D>, grid, block, g);
}

// A batched NN product over z = 0 .. zcount-1 (one grid row each); IM != kImNone:
// B is the implicit im2col of image z.
template <int BM, int BN, int D, int IM>
int launch_batched(const char *name, const GemmArgs &g, uint32_t zcount) {
    const dim3 grid(g.tiles_m * g.tiles_n, zcount);
    return launch(name, gemm_mfma_kernel<BM, BN, false, false, D, IM>, grid, dim3(kBlock), g);
}

// A batched TN product (A = weights, m x k stored k-major), no implicit
// operand: the data gradient of a 1x1 convolution.
template <int BM, int BN, int D>
int launch_batched_tn(const GemmArgs &g, uint32_t zcount) {
    const dim3 grid(g.tiles_m * g.tiles_n, zcount);
    return launch("convolution_data_gradient", gemm_mfma_kernel<BM, BN, true, false, D>, grid, dim3(kBlock), g);
}

// The data gradient's A: at[j][c][(f*ks + kh)*ks + kw] = w[j][f][c][ks-1-kh][ks-1-kw]
// for group j, channel c < cg and filter f < m -- the group's weights with
// channels as rows and the window flipped, so that the product with the
// implicit gather of delta is col2im(w^T x delta) (im2col.zig:51-79).
__global__ __launch_bounds__(kBlock) void flip_weights_kernel(const float *w, float *at, uint32_t kk, FastDiv div_kk,
                                                             FastDiv div_mkk, FastDiv div_cgmkk, uint32_t cg,
                                                             uint32_t total) {
    const uint32_t e = blockIdx.x * kBlock + threadIdx.x;
    if (e >= total) return;
    const uint32_t j = fdiv(e, div_cgmkk), r = e - j * div_cgmkk.d;
    const uint32_t c = fdiv(r, div_mkk), q = r - c * div_mkk.d;
    const uint32_t f = fdiv(q, div_kk), t = q - f * kk;
    at[e] = w[(size_t)j * div_cgmkk.d + (size_t)f * cg * kk + c * kk + (kk - 1 - t)];
}

// One phase's A of a strided data gradient: at[j][c][(f*na + a)*nb + b] =
// w[j][f][c][kh0 + s*(na-1-a)][kw0 + s*(nb-1-b)], the taps of the phase
// (kh = kh0 mod s, kw = kw0 mod s) with channels as rows, flipped.
struct PhaseTaps {
    uint32_t ks, s, kh0, kw0, na, nb, m, cg;
    FastDiv div_nb, div_nab, div_mnab, div_cgmnab;
};
__global__ __launch_bounds__(kBlock) void flip_phase_kernel(const float *w, float *at, PhaseTaps t, uint32_t total) {
    const uint32_t e = blockIdx.x * kBlock + threadIdx.x;
    if (e >= total) return;
    const uint32_t j = fdiv(e, t.div_cgmnab), r = e - j * t.div_cgmnab.d;
    const uint32_t c = fdiv(r, t.div_mnab), q = r - c * t.div_mnab.d;
    const uint32_t f = fdiv(q, t.div_nab), u = q - f * t.div_nab.d;
    const uint32_t a = fdiv(u, t.div_nb), b = u - a * t.nb;
    const uint32_t kh = t.kh0 + t.s * (t.na - 1 - a), kw = t.kw0 + t.s * (t.nb - 1 - b);
    const size_t kk = (size_t)t.ks * t.ks;
    at[e] = w[((size_t)j * t.m + f) * t.cg * kk + c * kk + kh * t.ks + kw];
}

template <int IM>
int launch_fwd(const char *name, const GemmArgs &g, uint32_t zcount, bool big) {
    if (big) return launch_batched<128, 128, 1, IM>(name, g, zcount);
    return launch_batched<64, 64, DKZ_GEMM_SMALL_PREFETCH, IM>(name, g, zcount);
}

// Columns over (image, position) of all `batch` images (kSpan), in 128x64
// tiles (64x64 below 128 rows): g holds one image's product per group
// (z = group); B and C advance b_img and c_img elements per image. Measured
// against per-image tiles: [64,512,14,14]->512 3x3 forward 1132 -> 975 us
// with 64x64 span tiles, 836 us with 128x64 ones (half the gathered B
// slabs per multiply-add), [64,1024,13,13]->1024 3324 -> 2642 -> 2536 us
// (data gradients alike), while with a fifth or less of the last tile empty
// ([64,256,28,28]->256, 26x26) the per-image 128x128 tiles stay 3-5% ahead;
// 128x128 tiles over (image, position) were slower than either (too few
// workgroups, and the per-tap gather spills). The 128x64 span kernels keep
// one slab in flight (two spill).
#ifndef DKZ_CONV_SPAN
#define DKZ_CONV_SPAN 1
#endif
#ifndef DKZ_SPAN_BM
#define DKZ_SPAN_BM 128
#endif

// Whether per-image column tiles of bn leave more than a fifth of their
// columns past the image's n positions.
inline bool span_pays(uint64_t n, uint64_t bn) {
    const uint64_t t = (uint64_t)div_up(n, bn) * bn;
    return (t - n) * 5 > t;
}

// Whether a batched convolution product of m rows and n positions per image
// runs as one span product: always with 128x64 span tiles (m >= 128), which
// measured ahead of per-image 128x128 tiles at every 3x3 size tried (2% at
// [64,128,56,56]->128, 6% at [64,256,28,28]->256, 13% at ->512, 30% at
// [64,256,26,26]->512, whose 1536 per-image tiles fill 1.5 rounds of
// workgroups) and for 1x1 forwards; below that when per-image tiles waste
// columns.
inline bool use_span(uint64_t batch, uint64_t m, uint64_t n, bool big) {
    if (!DKZ_CONV_SPAN || batch < 2) return false;
    return (DKZ_SPAN_BM == 128 && m >= 128) || span_pays(n, big ? 128 : 64);
}

// PH: `phases` phases of a strided data gradient per launch (kPhaseSpan, or
// kPhaseSpanOdd when the positions per image are not a multiple of 4; grid
// row = phase x group).
template <int MODE, bool PH = false>
int launch_span(const char *name, GemmArgs g, uint32_t batch, uint32_t groups, uint64_t b_img, uint64_t c_img,
                uint32_t phases = 1) {
    const uint32_t npos = g.n;
    g.n = batch * npos;
    g.tiles_m = div_up(g.m, 64);
    g.tiles_n = div_up(g.n, 64);
    g.cv.npos = npos;
    g.cv.div_npos = make_fastdiv(npos);
    g.cv.npos4 = npos % 4 == 0;
    g.cv.b_img = (uint32_t)b_img;
    g.cv.c_img = (uint32_t)c_img;
    g.zrows = groups;
    constexpr int D = DKZ_GEMM_SMALL_PREFETCH;
    if constexpr (PH) {
        DKZ_REQUIRE(phases >= 1 && phases <= (uint32_t)kMaxPhases);
        const bool big = DKZ_SPAN_BM == 128 && g.m >= 128;
        if (big) g.tiles_m = div_up(g.m, 128);
        if (npos % 4 == 0) {
            if (big) return launch_batched<128, 64, 1, kPhaseSpan + MODE>(name, g, phases * groups);
            return launch_batched<64, 64, D, kPhaseSpan + MODE>(name, g, phases * groups);
        }
        if constexpr (MODE == kTwoBlock || MODE == kRow) {
            DKZ_REQUIRE(npos % 4 == 0);  // row gathers are chosen only then
            return 0;
        } else {
            if (big) return launch_batched<128, 64, 1, kPhaseSpanOdd + MODE>(name, g, phases * groups);
            return launch_batched<64, 64, D, kPhaseSpanOdd + MODE>(name, g, phases * groups);
        }
    } else {
        if (DKZ_SPAN_BM == 128 && g.m >= 128) {
            g.tiles_m = div_up(g.m, 128);
            if (npos % 4 == 0) return launch_batched<128, 64, 1, kSpan + MODE>(name, g, groups);
            if constexpr (MODE != kTwoBlock && MODE != kRow)
                return launch_batched<128, 64, 1, kSpanOdd + MODE>(name, g, groups);
        }
        if (npos % 4 == 0) return launch_batched<64, 64, D, kSpan + MODE>(name, g, groups);
        if constexpr (MODE == kTwoBlock || MODE == kRow) {
            DKZ_REQUIRE(npos % 4 == 0);  // row gathers are chosen only then
            return 0;
        } else {
            return launch_batched<64, 64, D, kSpanOdd + MODE>(name, g, groups);
        }
    }
}

// The weight gradient's NT product (BM x BM tiles, K split into ranges),
// then the split-K reduce.
template <int BM, int IM>
int launch_wgrad(const GemmArgs &g) {
    const dim3 grid(g.tiles_m * g.tiles_n * g.splits);
    constexpr int D = BM == 128 ? 1 : DKZ_GEMM_SMALL_PREFETCH;
    DKZ_TRY(launch("convolution_weight_gradient", gemm_mfma_kernel<BM, BM, false, true, D, IM>, grid, dim3(kBlock), g));
    if (g.splits == 1) return 0;
    if (g.n % 4 == 0 && g.ldc % 4 == 0 && aligned16(g.c))
        return launch("convolution_weight_gradient", gemm_splitk_reduce_kernel<true>,
                      dim3(div_up((uint64_t)g.m * g.n / 4, kBlock)), dim3(kBlock), g);
    return launch("convolution_weight_gradient", gemm_splitk_reduce_kernel<false>,
                  dim3(div_up((uint64_t)g.m * g.n, kBlock)), dim3(kBlock), g);
}

template <int IM>
int launch_wgrad_tiles(const GemmArgs &g, bool big) {
    return big ? launch_wgrad<128, IM>(g) : launch_wgrad<64, IM>(g);
}

// Extent in elements of a rows x cols row-major view with leading dimension ld.
inline uint64_t extent(uint64_t rows, uint64_t cols, uint64_t ld) {
    return rows == 0 || cols == 0 ? 0 : (rows - 1) * ld + cols;
}

constexpr uint32_t kCus = 256;


}  // namespace
}  // namespace dkz

using namespace dkz;

extern "C" {

int dkz_gemm(int ta, int tb, int m, int n, int k, float alpha, const float *a, int lda, const float *b, int ldb,
             float beta, float *c, int ldc) {
    DKZ_REQUIRE(m >= 0 && n >= 0 && k >= 0 && lda >= 0 && ldb >= 0 && ldc >= 0);
    if (m == 0 || n == 0) return 0;  // gpu.zig:686
    DKZ_REQUIRE(c != nullptr && ldc >= n);
    DKZ_REQUIRE(extent(m, n, ldc) <= kMaxElems);
    if (k > 0) {
        DKZ_REQUIRE(a != nullptr && b != nullptr);
        DKZ_REQUIRE(lda >= (ta ? m : k) && ldb >= (tb ? k : n));
        DKZ_REQUIRE(extent(ta ? k : m, ta ? m : k, lda) + 3 <= kMaxElems);
        DKZ_REQUIRE(extent(tb ? n : k, tb ? k : n, ldb) + 3 <= kMaxElems);
    }
    GemmArgs g{};
    g.a = a;
    g.b = b;
    g.c = c;
    g.m = (uint32_t)m;
    g.n = (uint32_t)n;
    g.k = (uint32_t)k;
    g.lda = (uint32_t)lda;
    g.ldb = (uint32_t)ldb;
    g.ldc = (uint32_t)ldc;
    g.alpha = alpha;
    g.beta = beta;
    g.vec_a = aligned16(a) && lda % 4 == 0;
    g.vec_b = aligned16(b) && ldb % 4 == 0;
    g.splits = 1;
    g.k_chunk = (uint32_t)k;
    g.zgroups = 1;

    // 128x128 tiles when they give every CU two workgroups; 64x64 below, and
    // if even those leave CUs idle and K is long, split K (ranges of >= 128)
    // until about DKZ_GEMM_SPLIT_TARGET workgroups per CU, within the scratch.
    const uint64_t big = (uint64_t)div_up(m, 128) * div_up(n, 128);
    if (big >= 2 * kCus) {
        g.tiles_m = div_up(m, 128);
        g.tiles_n = div_up(n, 128);
        return launch_gemm<128, 128, 1>(ta != 0, tb != 0, g);
    }
    g.tiles_m = div_up(m, 64);
    g.tiles_n = div_up(n, 64);
    const uint64_t tiles = (uint64_t)g.tiles_m * g.tiles_n;
    uint64_t splits = 1;
    if (tiles < 2 * kCus && k >= 256) {
        splits = div_up((uint64_t)DKZ_GEMM_SPLIT_TARGET * kCus, tiles);
        const uint64_t by_k = (uint64_t)k / 128;
        if (splits > by_k) splits = by_k;
        Scratch sc;
        DKZ_TRY(device_scratch(&sc));
        const uint64_t cap = sc.gemm_floats / ((uint64_t)m * n);
        if (splits > cap) splits = cap;
    }
    if (splits > 1) {
        const uint32_t chunk = (uint32_t)((div_up(k, splits) + kBK - 1) / kBK * kBK);
        g.k_chunk = chunk;
        g.splits = div_up(k, chunk);
    }
    if (g.splits > 1) {
        Scratch sc;
        DKZ_TRY(device_scratch(&sc));
        g.partial = sc.gemm;
        DKZ_TRY((launch_gemm<64, 64, DKZ_GEMM_SMALL_PREFETCH>(ta != 0, tb != 0, g)));
        if (n % 4 == 0 && ldc % 4 == 0 && aligned16(c))
            return launch("gemm_splitk_reduce", gemm_splitk_reduce_kernel<true>,
                          dim3(div_up((uint64_t)m * n / 4, kBlock)), dim3(kBlock), g);
        return launch("gemm_splitk_reduce", gemm_splitk_reduce_kernel<false>, dim3(div_up((uint64_t)m * n, kBlock)),
                      dim3(kBlock), g);
    }
    return launch_gemm<64, 64, DKZ_GEMM_SMALL_PREFETCH>(ta != 0, tb != 0, g);
}

// convolutional.zig:240-260 in one launch: for image i and group j,
// output(i, j) (m x n, m = filters/groups, n = out_h*out_w) += weights(j)
// (m x k, k = ksize^2 * channels/groups) x im2col(input(i, j)) (k x n), with
// out_h = (height + 2*pad - ksize)/stride + 1 as outHeight computes it. The
// layer zero-fills the output first; this adds to it (beta = 1), as its gemm
// calls do. ksize 1 multiplies by the input itself (ldb = n), as the layer
// does. No workspace: the im2col operand is gathered inside the product.
int dkz_convolution_forward(int batch, int groups, int channels, int height, int width, int filters, int ksize,
                            int stride, int pad, const float *weights, const float *input, float *output) {
    DKZ_REQUIRE(batch >= 0 && groups >= 1 && groups <= 65535 && channels >= 0 && height >= 0 && width >= 0 &&
                filters >= 0);
    DKZ_REQUIRE(ksize >= 1 && stride >= 1 && pad >= 0);
    DKZ_REQUIRE(channels % groups == 0 && filters % groups == 0);
    DKZ_REQUIRE((int64_t)height + 2 * (int64_t)pad >= ksize && (int64_t)width + 2 * (int64_t)pad >= ksize);
    const uint64_t m = (uint64_t)filters / groups, cg = (uint64_t)channels / groups;
    const uint64_t ho = ((uint64_t)height + 2 * (uint64_t)pad - ksize) / stride + 1;
    const uint64_t wo = ((uint64_t)width + 2 * (uint64_t)pad - ksize) / stride + 1;
    const uint64_t n = ho * wo, k = (uint64_t)ksize * ksize * cg;
    const uint64_t zcount = (uint64_t)batch * groups, in_group = cg * height * width;
    if (zcount == 0 || m == 0 || n == 0 || k == 0) return 0;
    DKZ_REQUIRE(weights && input && output);
    DKZ_REQUIRE(zcount * m * n <= kMaxElems && zcount * in_group <= kMaxElems && (uint64_t)groups * m * k <= kMaxElems);
    DKZ_REQUIRE(ksize != 1 || n <= (uint64_t)height * width);  // the input is read as a k x n matrix
    GemmArgs g{};
    g.a = weights;
    g.b = input;
    g.c = output;
    g.m = (uint32_t)m;
    g.n = (uint32_t)n;
    g.k = (uint32_t)k;
    g.lda = (uint32_t)k;
    g.ldb = (uint32_t)n;
    g.ldc = (uint32_t)n;
    g.alpha = 1.0f;
    g.beta = 1.0f;
    g.splits = 1;
    g.k_chunk = (uint32_t)k;
    g.vec_a = aligned16(weights) && k % 4 == 0 && (m * k) % 4 == 0;
    g.vec_b = aligned16(input) && n % 4 == 0 && in_group % 4 == 0;
    g.zgroups = (uint32_t)groups;
    g.a_z = (uint32_t)(m * k);
    g.b_z = (uint32_t)in_group;
    g.c_z = (uint32_t)(m * n);
    const bool im = ksize != 1;
    if (im) {
        ConvB &cv = g.cv;
        cv.H = (uint32_t)height;
        cv.W = (uint32_t)width;
        cv.Wo = (uint32_t)wo;
        cv.ksz = (uint32_t)ksize;
        cv.stride = (uint32_t)stride;
        cv.pad = pad;
        cv.pad_x = pad;
        cv.div_kk = make_fastdiv((uint32_t)(ksize * ksize));
        cv.div_k = make_fastdiv((uint32_t)ksize);
        cv.div_wo = make_fastdiv((uint32_t)wo);
        cv.s1 = stride == 1 && width % 4 == 0 && wo % 4 == 0 && aligned16(input);
        cv.row4 = wo % 4 == 0;
    }
    // 128x128 tiles when m fills them and the whole batch gives every CU two
    // workgroups, else 64x64.
    const bool big = m >= 128 && (uint64_t)div_up(m, 128) * div_up(n, 128) * zcount >= 2 * kCus;
    g.tiles_m = (uint32_t)div_up(m, big ? 128 : 64);
    g.tiles_n = (uint32_t)div_up(n, big ? 128 : 64);
    // One product per group with columns over every image's positions (see
    // use_span), else one per (image, group).
    if (use_span(batch, m, n, big)) {
        constexpr const char *kName = "convolution_forward";
        const uint64_t b_img = (uint64_t)groups * in_group, c_img = (uint64_t)groups * m * n;
        g.cv.b_vec = g.vec_b;  // ksize 1: float4 rows of the input matrix
        if (!im) return launch_span<kRaw>(kName, g, (uint32_t)batch, (uint32_t)groups, b_img, c_img);
        if (g.cv.s1) return launch_span<kTwoBlock>(kName, g, (uint32_t)batch, (uint32_t)groups, b_img, c_img);
        if (g.cv.row4) return launch_span<kRow>(kName, g, (uint32_t)batch, (uint32_t)groups, b_img, c_img);
        return launch_span<kGather>(kName, g, (uint32_t)batch, (uint32_t)groups, b_img, c_img);
    }
    // At most 65535 grid rows per launch, whole images each (a multiple of
    // groups), so that every launch starts at group 0.
    const uint64_t chunk = 65535 - 65535 % (uint64_t)groups;
    for (uint64_t z0 = 0; z0 < zcount; z0 += chunk) {
        const uint32_t zc = (uint32_t)(zcount - z0 < chunk ? zcount - z0 : chunk);
        GemmArgs gz = g;
        gz.b = input + z0 * in_group;
        gz.c = output + z0 * m * n;
        constexpr int kS1 = kFwd + kTwoBlock, kGa = kFwd + kGather, kRw = kFwd + kRow;
        int e;
        if (!im) e = launch_fwd<kImNone>("convolution_forward", gz, zc, big);
        else if (g.cv.s1) e = launch_fwd<kS1>("convolution_forward", gz, zc, big);
        else if (g.cv.row4) e = launch_fwd<kRw>("convolution_forward", gz, zc, big);
        else e = launch_fwd<kGa>("convolution_forward", gz, zc, big);
        if (e != 0) return e;
    }
    return 0;
}

// convolutional.zig:299-305 (the data-gradient half of the per-image
// backward loop) in one call. For image i and group j, with m, n, k, the
// offsets and out_h, out_w as in dkz_convolution_forward and
// input_delta(i, j) = input_delta + (i*groups + j)*in_group:
//   ksize 1: input_delta(i, j), read as a k x n matrix as the layer reads it,
//            = weights(j)^T (k x m) x delta(i, j) (m x n) -- overwritten
//            (the layer's gemm with beta 0);
//   else:    input_delta(i, j) += col2im(weights(j)^T x delta(i, j)) -- the
//            layer's gemm into the workspace, then col2im, which adds.
// With stride 1 and pad < ksize the second is one product per image and
// group: input channels by input positions, k = (filter, tap) over the
// group's flipped weights (transposed once into the library's scratch) and
// delta gathered at each tap's output position, so col2im's adds join the
// product's sum. Otherwise the same per phase of the input pixels (y mod
// stride, x mod stride), each over its own taps. No workspace.
int dkz_convolution_data_gradient(int batch, int groups, int channels, int height, int width, int filters, int ksize,
                                  int stride, int pad, const float *weights, const float *delta,
                                  float *input_delta) {
    DKZ_REQUIRE(batch >= 0 && groups >= 1 && groups <= 65535 && channels >= 0 && height >= 0 && width >= 0 &&
                filters >= 0);
    DKZ_REQUIRE(ksize >= 1 && stride >= 1 && pad >= 0);
    DKZ_REQUIRE(channels % groups == 0 && filters % groups == 0);
    DKZ_REQUIRE((int64_t)height + 2 * (int64_t)pad >= ksize && (int64_t)width + 2 * (int64_t)pad >= ksize);
    const uint64_t m = (uint64_t)filters / groups, cg = (uint64_t)channels / groups;
    const uint64_t ho = ((uint64_t)height + 2 * (uint64_t)pad - ksize) / stride + 1;
    const uint64_t wo = ((uint64_t)width + 2 * (uint64_t)pad - ksize) / stride + 1;
    const uint64_t npos = ho * wo, kk = (uint64_t)ksize * ksize, kw = kk * cg;
    const uint64_t zcount = (uint64_t)batch * groups, in_group = cg * height * width;
    if (zcount == 0 || cg == 0 || npos == 0 || in_group == 0) return 0;
    DKZ_REQUIRE(weights && delta && input_delta);
    DKZ_REQUIRE(zcount * m * npos <= kMaxElems && zcount * in_group <= kMaxElems &&
                (uint64_t)groups * m * kw <= kMaxElems);
    DKZ_REQUIRE(ksize != 1 || npos <= (uint64_t)height * width);  // the k x n view stays inside the image
    const uint64_t chunk = 65535 - 65535 % (uint64_t)groups;
    GemmArgs g{};
    g.alpha = 1.0f;
    g.splits = 1;
    g.zgroups = (uint32_t)groups;
    g.b_z = (uint32_t)(m * npos);
    g.c_z = (uint32_t)in_group;
    if (ksize == 1) {
        // C(i, j) = A^T x B with A = weights(j) (m x cg, k-major), B = delta(i, j);
        // with m == 0 the sum is empty and beta 0 leaves zeros (gemm.zig:121-131).
        g.a = weights;
        g.m = (uint32_t)cg;
        g.n = (uint32_t)npos;
        g.k = (uint32_t)m;
        g.k_chunk = (uint32_t)m;
        g.lda = (uint32_t)cg;
        g.ldb = (uint32_t)npos;
        g.ldc = (uint32_t)npos;
        g.beta = 0.0f;
        g.a_z = (uint32_t)(m * cg);
        g.vec_a = aligned16(weights) && cg % 4 == 0;
        g.vec_b = aligned16(delta) && npos % 4 == 0 && (m * npos) % 4 == 0;
        const bool big = cg >= 128 && (uint64_t)div_up(cg, 128) * div_up(npos, 128) * zcount >= 2 * kCus;
        g.tiles_m = (uint32_t)div_up(cg, big ? 128 : 64);
        g.tiles_n = (uint32_t)div_up(npos, big ? 128 : 64);
        for (uint64_t z0 = 0; z0 < zcount; z0 += chunk) {
            const uint32_t zc = (uint32_t)(zcount - z0 < chunk ? zcount - z0 : chunk);
            GemmArgs gz = g;
            gz.b = delta + z0 * m * npos;
            gz.c = input_delta + z0 * in_group;
            DKZ_TRY(big ? (launch_batched_tn<128, 128, 1>(gz, zc))
                        : (launch_batched_tn<64, 64, DKZ_GEMM_SMALL_PREFETCH>(gz, zc)));
        }
        return 0;
    }
    if (m == 0) return 0;  // col2im adds an empty sum
    Scratch sc;
    DKZ_TRY(device_scratch(&sc));
    if (stride == 1 && pad <= ksize - 1) {
        // input_delta(i, j) += A x im2col(delta(i, j)) with A the group's
        // weights flipped and transposed (flip_weights_kernel, into the
        // scratch) and the im2col of delta (out_h x out_w, pad ksize-1-pad)
        // gathered inside the product: out_h + 2*(ksize-1-pad) - ksize + 1 =
        // height, and tap (kh, kw) of input position (y, x) reads delta at
        // (y + kh - (ksize-1-pad), ...), i.e. the layer's col2im term of tap
        // (ksize-1-kh, ksize-1-kw).
        const uint64_t at_floats = (uint64_t)groups * cg * m * kk;
        DKZ_REQUIRE(at_floats <= sc.gemm_floats);
        DKZ_TRY(launch("convolution_data_gradient", flip_weights_kernel, dim3(div_up(at_floats, kBlock)),
                       dim3(kBlock), weights, sc.gemm, (uint32_t)kk, make_fastdiv((uint32_t)kk),
                       make_fastdiv((uint32_t)(m * kk)), make_fastdiv((uint32_t)(cg * m * kk)), (uint32_t)cg,
                       (uint32_t)at_floats));
        const uint64_t n = (uint64_t)height * width, k = m * kk;
        g.a = sc.gemm;
        g.b = delta;
        g.c = input_delta;
        g.m = (uint32_t)cg;
        g.n = (uint32_t)n;
        g.k = (uint32_t)k;
        g.k_chunk = (uint32_t)k;
        g.lda = (uint32_t)k;
        g.ldb = (uint32_t)n;
        g.ldc = (uint32_t)n;
        g.beta = 1.0f;
        g.a_z = (uint32_t)(cg * k);
        g.vec_a = k % 4 == 0;  // the scratch is 256-byte aligned
        ConvB &cv = g.cv;
        cv.H = (uint32_t)ho;
        cv.W = (uint32_t)wo;
        cv.Wo = (uint32_t)width;
        cv.ksz = (uint32_t)ksize;
        cv.stride = 1;
        cv.pad = ksize - 1 - pad;
        cv.pad_x = ksize - 1 - pad;
        cv.div_kk = make_fastdiv((uint32_t)kk);
        cv.div_k = make_fastdiv((uint32_t)ksize);
        cv.div_wo = make_fastdiv((uint32_t)width);
        cv.s1 = width % 4 == 0 && wo % 4 == 0 && aligned16(delta);
        const bool big = cg >= 128 && (uint64_t)div_up(cg, 128) * div_up(n, 128) * zcount >= 2 * kCus;
        g.tiles_m = (uint32_t)div_up(cg, big ? 128 : 64);
        g.tiles_n = (uint32_t)div_up(n, big ? 128 : 64);
        constexpr int kS1 = kFwd + kTwoBlock, kGa = kFwd + kGather, kRw = kFwd + kRow;
        constexpr const char *kName = "convolution_data_gradient";
        cv.row4 = width % 4 == 0;
        if (use_span(batch, cg, n, big)) {
            const uint64_t b_img = (uint64_t)groups * m * npos, c_img = (uint64_t)groups * in_group;
            if (cv.s1) return launch_span<kTwoBlock>(kName, g, (uint32_t)batch, (uint32_t)groups, b_img, c_img);
            if (cv.row4) return launch_span<kRow>(kName, g, (uint32_t)batch, (uint32_t)groups, b_img, c_img);
            return launch_span<kGather>(kName, g, (uint32_t)batch, (uint32_t)groups, b_img, c_img);
        }
        for (uint64_t z0 = 0; z0 < zcount; z0 += chunk) {
            const uint32_t zc = (uint32_t)(zcount - z0 < chunk ? zcount - z0 : chunk);
            GemmArgs gz = g;
            gz.b = delta + z0 * m * npos;
            gz.c = input_delta + z0 * in_group;
            DKZ_TRY(cv.s1     ? launch_fwd<kS1>(kName, gz, zc, big)
                    : cv.row4 ? launch_fwd<kRw>(kName, gz, zc, big)
                              : launch_fwd<kGa>(kName, gz, zc, big));
        }
        return 0;
    }
    // Strided (or pad >= ksize): the im2col of delta would have holes between
    // the strided outputs. Input pixel (y, x) takes tap (kh, kw) only when
    // y + pad - kh is a multiple of stride, so the pixels split into stride^2
    // phases (y mod stride, x mod stride), each taking the taps kh = kh0 + s*a,
    // kw = kw0 + s*b with kh0 = (py + pad) mod s: per phase one product over
    // the phase's pixels whose A is those taps flipped (flip_phase_kernel) and
    // whose B is a stride-1 im2col of delta with window na x nb and pads
    // na-1-qy, nb-1-qx (qy = (py + pad - kh0) / s), written to the phase's
    // pixels. The same multiply-adds as the layer's gemm, no column buffer.
    const int s = stride;
    const uint64_t at_all = (uint64_t)groups * cg * m * kk;
    DKZ_REQUIRE(at_all <= sc.gemm_floats);
    // The phases that some tap reaches, most taps first (their workgroups
    // are the longest, so they start first).
    struct Phase {
        int py, px, kh0, kw0, na, nb, hp, wp, qy, qx;
    };
    std::vector<Phase> phases;
    for (int py = 0; py < s; ++py) {
        for (int px = 0; px < s; ++px) {
            Phase q{};
            q.py = py;
            q.px = px;
            q.kh0 = (py + pad) % s;
            q.kw0 = (px + pad) % s;
            q.na = q.kh0 < ksize ? (ksize - q.kh0 + s - 1) / s : 0;
            q.nb = q.kw0 < ksize ? (ksize - q.kw0 + s - 1) / s : 0;
            q.hp = py < height ? (height - py + s - 1) / s : 0;
            q.wp = px < width ? (width - px + s - 1) / s : 0;
            if (q.na == 0 || q.nb == 0 || q.hp == 0 || q.wp == 0) continue;  // no tap reaches these pixels
            q.qy = (py + pad - q.kh0) / s;
            q.qx = (px + pad - q.kw0) / s;
            phases.push_back(q);
        }
    }
    std::stable_sort(phases.begin(), phases.end(),
                     [](const Phase &x, const Phase &y) { return x.na * x.nb > y.na * y.nb; });
    // Phases share a launch (grid row = phase x (image, group)) when they
    // cover equal pixel grids, i.e. the stride divides the input, and a
    // launch's rows can hold every group of an image for each phase.
    const bool merge = height % s == 0 && width % s == 0 && (uint64_t)groups * kMaxPhases <= 65535;
    uint64_t at_off = 0;
    for (size_t i0 = 0; i0 < phases.size();) {
        const size_t cnt = merge ? std::min<size_t>(kMaxPhases, phases.size() - i0) : 1;
        const int hp = phases[i0].hp, wp = phases[i0].wp;
        const uint64_t n = (uint64_t)hp * wp;
        GemmArgs gp = g;
        for (size_t u = 0; u < cnt; ++u) {
            const Phase &q = phases[i0 + u];
            const uint64_t nab = (uint64_t)q.na * q.nb, k = m * nab;
            const uint64_t at_n = (uint64_t)groups * cg * k;
            PhaseTaps t{(uint32_t)ksize, (uint32_t)s, (uint32_t)q.kh0, (uint32_t)q.kw0, (uint32_t)q.na,
                        (uint32_t)q.nb, (uint32_t)m, (uint32_t)cg, make_fastdiv((uint32_t)q.nb),
                        make_fastdiv((uint32_t)nab), make_fastdiv((uint32_t)(m * nab)),
                        make_fastdiv((uint32_t)(cg * k))};
            float *at = sc.gemm + at_off;
            DKZ_TRY(launch("convolution_data_gradient", flip_phase_kernel, dim3(div_up(at_n, kBlock)), dim3(kBlock),
                           weights, at, t, (uint32_t)at_n));
            gp.ph[u] = PhaseDesc{at,
                                 (uint32_t)k,
                                 (uint32_t)(k % 4 == 0 && at_off % 4 == 0),
                                 (uint32_t)q.nb,
                                 (uint32_t)q.py,
                                 (uint32_t)q.px,
                                 q.na - 1 - q.qy,
                                 q.nb - 1 - q.qx,
                                 make_fastdiv((uint32_t)nab),
                                 make_fastdiv((uint32_t)q.nb)};
            at_off += at_n;
        }
        gp.a = gp.ph[0].a;
        gp.b = delta;
        gp.c = input_delta;
        gp.m = (uint32_t)cg;
        gp.n = (uint32_t)n;
        gp.k = gp.ph[0].k;
        gp.k_chunk = gp.k;
        gp.lda = gp.k;
        gp.ldb = (uint32_t)n;
        gp.ldc = (uint32_t)((uint64_t)height * width);
        gp.beta = 1.0f;
        gp.a_z = (uint32_t)(cg * gp.k);
        gp.vec_a = gp.ph[0].vec_a;
        ConvB &cv = gp.cv;
        cv.H = (uint32_t)ho;
        cv.W = (uint32_t)wo;
        cv.Wo = (uint32_t)wp;
        cv.stride = 1;
        cv.div_wo = make_fastdiv((uint32_t)wp);
        cv.s1 = wo % 4 == 0 && wp % 4 == 0 && aligned16(delta) && (m * npos) % 4 == 0;
        cv.row4 = wp % 4 == 0;
        cv.div_wp = make_fastdiv((uint32_t)wp);
        cv.ph_s = (uint32_t)s;
        cv.ph_w = (uint32_t)width;
        const bool big = cg >= 128 && (uint64_t)div_up(cg, 128) * div_up(n, 128) * zcount >= 2 * kCus;
        gp.tiles_m = (uint32_t)div_up(cg, big ? 128 : 64);
        gp.tiles_n = (uint32_t)div_up(n, big ? 128 : 64);
        constexpr int kPS1 = kPhase + kTwoBlock, kPGa = kPhase + kGather, kPRw = kPhase + kRow;
        constexpr const char *kName = "convolution_data_gradient";
        if (use_span(batch, cg, n, big)) {
            // Columns over (image, phase position) of every image.
            const uint64_t b_img = (uint64_t)groups * m * npos, c_img = (uint64_t)groups * in_group;
            const uint32_t b = (uint32_t)batch, gr = (uint32_t)groups, pc = (uint32_t)cnt;
            constexpr bool kPh = true;
            DKZ_TRY(cv.s1     ? (launch_span<kTwoBlock, kPh>(kName, gp, b, gr, b_img, c_img, pc))
                    : cv.row4 ? (launch_span<kRow, kPh>(kName, gp, b, gr, b_img, c_img, pc))
                              : (launch_span<kGather, kPh>(kName, gp, b, gr, b_img, c_img, pc)));
            i0 += cnt;
            continue;
        }
        // At most 65535 grid rows: cnt phases x zc (image, group) rows, whole
        // images each.
        const uint64_t rows = 65535 / cnt, zchunk = rows - rows % (uint64_t)groups;
        for (uint64_t z0 = 0; z0 < zcount; z0 += zchunk) {
            const uint32_t zc = (uint32_t)(zcount - z0 < zchunk ? zcount - z0 : zchunk);
            GemmArgs gz = gp;
            gz.b = delta + z0 * m * npos;
            gz.c = input_delta + z0 * in_group;
            gz.zrows = zc;
            const uint32_t zr = (uint32_t)(cnt * zc);
            DKZ_TRY(cv.s1     ? launch_fwd<kPS1>(kName, gz, zr, big)
                    : cv.row4 ? launch_fwd<kPRw>(kName, gz, zr, big)
                              : launch_fwd<kPGa>(kName, gz, zr, big));
        }
        i0 += cnt;
    }
    return 0;
}

// convolutional.zig:288-297 (the weight-gradient half of the per-image
// backward loop) in one product: for group j,
//     weight_updates(j) (m x k) += sum over images i of delta(i, j) (m x n) x im2col(input(i, j))^T (n x k)
// with the same m, n, k, offsets and ksize-1 reading of the input as
// dkz_convolution_forward, delta(i, j) = delta + (i*groups + j)*m*n and
// weight_updates(j) = weight_updates + j*m*k. One NT product per group whose
// k runs over (image, position), split into ranges of k that are added in
// order.
int dkz_convolution_weight_gradient(int batch, int groups, int channels, int height, int width, int filters,
                                    int ksize, int stride, int pad, const float *delta, const float *input,
                                    float *weight_updates) {
    DKZ_REQUIRE(batch >= 0 && groups >= 1 && channels >= 0 && height >= 0 && width >= 0 && filters >= 0);
    DKZ_REQUIRE(ksize >= 1 && stride >= 1 && pad >= 0);
    DKZ_REQUIRE(channels % groups == 0 && filters % groups == 0);
    DKZ_REQUIRE((int64_t)height + 2 * (int64_t)pad >= ksize && (int64_t)width + 2 * (int64_t)pad >= ksize);
    const uint64_t m = (uint64_t)filters / groups, cg = (uint64_t)channels / groups;
    const uint64_t ho = ((uint64_t)height + 2 * (uint64_t)pad - ksize) / stride + 1;
    const uint64_t wo = ((uint64_t)width + 2 * (uint64_t)pad - ksize) / stride + 1;
    const uint64_t npos = ho * wo, kw = (uint64_t)ksize * ksize * cg, in_group = cg * height * width;
    if (batch == 0 || m == 0 || kw == 0 || npos == 0) return 0;
    DKZ_REQUIRE(delta && input && weight_updates);
    const uint64_t images = (uint64_t)batch * groups;
    DKZ_REQUIRE(images * m * npos <= kMaxElems && images * in_group <= kMaxElems && (uint64_t)groups * m * kw <= kMaxElems);
    DKZ_REQUIRE((uint64_t)batch * npos <= kMaxElems);
    DKZ_REQUIRE(ksize != 1 || npos <= (uint64_t)height * width);  // the input is read as a k x n matrix
    GemmArgs g{};
    g.m = (uint32_t)m;
    g.n = (uint32_t)kw;
    g.k = (uint32_t)((uint64_t)batch * npos);
    g.ldc = (uint32_t)kw;
    g.alpha = 1.0f;
    g.beta = 1.0f;
    g.zgroups = 1;
    ConvB &cv = g.cv;
    cv.H = (uint32_t)height;
    cv.W = (uint32_t)width;
    cv.Wo = (uint32_t)wo;
    cv.ksz = (uint32_t)ksize;
    cv.stride = (uint32_t)stride;
    cv.pad = pad;
    cv.pad_x = pad;
    cv.div_kk = make_fastdiv((uint32_t)(ksize * ksize));
    cv.div_k = make_fastdiv((uint32_t)ksize);
    cv.div_wo = make_fastdiv((uint32_t)wo);
    cv.npos = (uint32_t)npos;
    cv.div_npos = make_fastdiv((uint32_t)npos);
    cv.a_img = (uint32_t)((uint64_t)groups * m * npos);
    cv.b_img = (uint32_t)((uint64_t)groups * in_group);
    cv.npos4 = npos % 4 == 0;
    cv.a_vec = aligned16(delta) && (m * npos) % 4 == 0;
    cv.b_vec = aligned16(input) && in_group % 4 == 0;
    const bool s1 = ksize != 1 && stride == 1 && width % 4 == 0 && wo % 4 == 0 && aligned16(input) &&
                    in_group % 4 == 0;
    cv.s1 = s1;
    const bool big = DKZ_WGRAD_BIG && m >= 128;
    g.tiles_m = (uint32_t)div_up(m, big ? 128 : 64);
    g.tiles_n = (uint32_t)div_up(kw, big ? 128 : 64);
    // Split K (image-major positions) into ranges of whole slabs, of at
    // least DKZ_WGRAD_MIN_CHUNK and within the scratch. The gathering kernels
    // run four workgroups per CU, so workgroups come in rounds of 4 * 256: the
    // split count is the smallest whose rounds are, within 2%, as full as the
    // best one's (a last round a tenth full leaves CUs idle for most of a
    // workgroup's time; measured at config 2's layer, 504 / 774 / 1008 /
    // 1512 workgroups 827 / 769 / 696 / 739 us; [64,512,14,14]->512 1152 ->
    // 1008 workgroups 758 -> 647 us, [64,1024,13,13]->1024 1152 -> 1728
    // 2949 -> 2558 us), and among those the smallest whose workgroup count is
    // a multiple of the XCD count, if any (the tile mapping then keeps each
    // range's tiles on one XCD, sharing its delta rows in L2: 999 instead of
    // 1008 workgroups cost 3% at config 2's layer).
    // With ksize 1, whose operands stream as plain float4s and whose partial
    // tiles weigh more, toward DKZ_WGRAD_TARGET_RAW workgroups per CU.
    const uint64_t tiles = (uint64_t)g.tiles_m * g.tiles_n;
    const uint64_t kt = (uint64_t)batch * npos;
    const uint64_t by_k = div_up(kt, (uint64_t)DKZ_WGRAD_MIN_CHUNK);
    Scratch sc;
    DKZ_TRY(device_scratch(&sc));
    const uint64_t cap = sc.gemm_floats / (m * kw);
    const uint64_t slots = (uint64_t)kCus * 4;
    uint64_t smax = by_k < cap ? by_k : cap;
    if (smax > 8 * slots / tiles + 1) smax = 8 * slots / tiles + 1;  // beyond eight rounds nothing changes
    if (smax < 1) smax = 1;
    auto chunk_of = [&](uint64_t s) { return div_up(div_up(kt, s), (uint64_t)kBK) * kBK; };
    uint64_t chunk = chunk_of(1);
    if (ksize == 1) {
        uint64_t want = div_up((uint64_t)DKZ_WGRAD_TARGET_RAW * kCus, tiles);
        if (want > smax) want = smax;
        chunk = chunk_of(want);
        for (uint64_t s = want; s > want / 2 && s > 1; --s) {
            if (div_up(kt, chunk_of(s)) * tiles % kXcds == 0) {
                chunk = chunk_of(s);
                break;
            }
        }
    } else {
        auto count = [&](uint64_t s) { return tiles * div_up(kt, chunk_of(s)); };
        auto fill = [&](uint64_t s) {
            const uint64_t w = count(s);
            return (double)w / (double)(div_up(w, slots) * slots);
        };
        double best = 0.0;
        for (uint64_t s = 1; s <= smax; ++s) best = fill(s) > best ? fill(s) : best;
        uint64_t pick = 0;
        for (uint64_t s = 1; s <= smax && pick == 0; ++s)
            if (fill(s) >= best - 0.02 && count(s) % kXcds == 0) pick = s;
        for (uint64_t s = 1; s <= smax && pick == 0; ++s)
            if (fill(s) >= best - 0.02) pick = s;
        chunk = chunk_of(pick);
    }
    g.splits = (uint32_t)div_up(kt, chunk);
    g.k_chunk = (uint32_t)chunk;
    g.partial = sc.gemm;
    constexpr int kWgRaw = kWgrad + kRaw, kWgGa = kWgrad + kGather, kWgS1 = kWgrad + kTwoBlock;
    constexpr int kWgRw = kWgrad + kRow;
    const bool row4 = ksize != 1 && wo % 4 == 0;
    for (int j = 0; j < groups; ++j) {
        GemmArgs gj = g;
        gj.a = delta + (uint64_t)j * m * npos;
        gj.b = input + (uint64_t)j * in_group;
        gj.c = weight_updates + (uint64_t)j * m * kw;
        if (ksize == 1) DKZ_TRY(launch_wgrad_tiles<kWgRaw>(gj, big));
        else if (s1) DKZ_TRY(launch_wgrad_tiles<kWgS1>(gj, big));
        else if (row4) DKZ_TRY(launch_wgrad_tiles<kWgRw>(gj, big));
        else DKZ_TRY(launch_wgrad_tiles<kWgGa>(gj, big));
    }
    return 0;
}

}  // extern "C"
