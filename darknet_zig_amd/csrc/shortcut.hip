// shortcut.hip -- residual add with resolution/channel mismatch
// (src/gpu.zig:773-800, CPU twin blas.zig:290-322).
//
// Over the overlapping region (b, k < minc, j < minh, i < minw):
//   out[i*sample + w2*(j*sample + h2*(k + c2*b))] =
//       s1*out[...] + s2*add[i*stride + w1*(j*stride + h1*(k + c1*b))]
// with stride = w1/w2 and sample = w2/w1, each at least 1, computed on the
// host exactly as gpu.zig:786-793 does. The map is one-to-one, so one lane per
// element is race-free; the two products are rounded before the sum (no fma).
//
// stride 2, sample 1 (a [shortcut] from a layer twice the resolution) has a
// fast path: a lane owns two adjacent outputs, reads them as a float2 and the
// four add values around their sources as one float4.
#include "dkz_device.hpp"
#include "dkz_hints.hpp"
#include "dkz_internal.hpp"

namespace dkz {
namespace {

struct ShortcutGeom {
    uint32_t minw, minh, minc, stride, sample, w1, h1, c1, w2, h2, c2;
    float s1, s2;
    FastDiv div_minw, div_minh, div_minc;
};

__device__ __forceinline__ void shortcut_coords(uint32_t id, const ShortcutGeom &g, uint32_t &i, uint32_t &j,
                                                uint32_t &k, uint32_t &b) {
    uint32_t t = fdiv(id, g.div_minw);
    i = id - t * g.minw;
    uint32_t t2 = fdiv(t, g.div_minh);
    j = t - t2 * g.minh;
    b = fdiv(t2, g.div_minc);
    k = t2 - b * g.minc;
}

__global__ __launch_bounds__(kBlock) void shortcut_kernel(const float *add, float *out, ShortcutGeom g,
                                                          uint32_t size) {
    const uint32_t id = blockIdx.x * kBlock + threadIdx.x;
    if (id >= size) return;
    uint32_t i, j, k, b;
    shortcut_coords(id, g, i, j, k, b);
    const uint32_t oi = i * g.sample + g.w2 * (j * g.sample + g.h2 * (k + g.c2 * b));
    const uint32_t ai = i * g.stride + g.w1 * (j * g.stride + g.h1 * (k + g.c1 * b));
    out[oi] = g.s1 * out[oi] + g.s2 * add[ai];
}

// id2 indexes output pairs (i even); minw is even so a pair shares (j, k, b).
__global__ __launch_bounds__(kBlock) void shortcut2_kernel(const float *add, float *out, ShortcutGeom g,
                                                           uint32_t pairs) {
    const uint32_t q = blockIdx.x * kBlock + threadIdx.x;
    if (q >= pairs) return;
    uint32_t i, j, k, b;
    shortcut_coords(2 * q, g, i, j, k, b);
    const uint32_t oi = i + g.w2 * (j + g.h2 * (k + g.c2 * b));
    const uint32_t ai = 2 * i + g.w1 * (2 * j + g.h1 * (k + g.c1 * b));
    constexpr int H = DKZ_HINT_SHORTCUT;  // bit 0: add loads, 1: out loads, 2: out stores
    float2 o = ld2<(H & 2) != 0>(out, oi >> 1);
    const float4 a = ld4<(H & 1) != 0>(add, ai >> 2);
    o.x = g.s1 * o.x + g.s2 * a.x;
    o.y = g.s1 * o.y + g.s2 * a.z;
    st2<(H & 4) != 0>(out, oi >> 1, o);
}

}  // namespace
}  // namespace dkz

using namespace dkz;

extern "C" {

int dkz_shortcut(int batch, int w1, int h1, int c1, const float *add, int w2, int h2, int c2, float s1, float s2,
                 float *out) {
    DKZ_REQUIRE(batch >= 0 && w1 >= 0 && h1 >= 0 && c1 >= 0 && w2 >= 0 && h2 >= 0 && c2 >= 0);
    const int minw = w1 < w2 ? w1 : w2, minh = h1 < h2 ? h1 : h2, minc = c1 < c2 ? c1 : c2;
    const uint64_t size = (uint64_t)batch * minw * minh * minc;  // gpu.zig:793
    if (size == 0) return 0;
    // gpu.zig:786-789: usize divisions, clamped to at least 1.
    int stride = w1 / w2, sample = w2 / w1;
    if (stride < 1) stride = 1;
    if (sample < 1) sample = 1;
    DKZ_REQUIRE(add && out);
    const uint64_t last_out = (uint64_t)(minw - 1) * sample +
                              (uint64_t)w2 * ((uint64_t)(minh - 1) * sample +
                                              (uint64_t)h2 * ((uint64_t)(minc - 1) + (uint64_t)c2 * (batch - 1)));
    const uint64_t last_add = (uint64_t)(minw - 1) * stride +
                              (uint64_t)w1 * ((uint64_t)(minh - 1) * stride +
                                              (uint64_t)h1 * ((uint64_t)(minc - 1) + (uint64_t)c1 * (batch - 1)));
    DKZ_REQUIRE(size <= kMaxElems && last_out <= kMaxElems && last_add + 3 <= kMaxElems);
    ShortcutGeom g{(uint32_t)minw,   (uint32_t)minh,   (uint32_t)minc, (uint32_t)stride, (uint32_t)sample,
                   (uint32_t)w1,     (uint32_t)h1,     (uint32_t)c1,   (uint32_t)w2,     (uint32_t)h2,
                   (uint32_t)c2,     s1,               s2,             make_fastdiv((uint32_t)minw),
                   make_fastdiv((uint32_t)minh),       make_fastdiv((uint32_t)minc)};
    const bool fast = stride == 2 && sample == 1 && minw % 2 == 0 && w2 % 2 == 0 && w1 % 4 == 0 &&
                      aligned16(add) && ((uintptr_t)out & 7u) == 0;
    if (fast) {
        const uint32_t pairs = (uint32_t)(size / 2);
        return launch("shortcut_s2", shortcut2_kernel, dim3(div_up(pairs, kBlock)), dim3(kBlock), add, out, g,
                      pairs);
    }
    return launch("shortcut", shortcut_kernel, dim3(div_up(size, kBlock)), dim3(kBlock), add, out, g,
                  (uint32_t)size);
}

}  // extern "C"
