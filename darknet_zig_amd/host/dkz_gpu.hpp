// dkz_gpu.hpp -- the host side of darknet-zig's GPU op layer (src/gpu.zig), in
// C++17 over the C ABI of libdkz (include/dkz_ops.h). Header only.
//
// Same names, argument order and meaning as gpu.zig's public functions, so a
// caller written against the reference reads the same here:
//
//   * Buf is gpu.zig's Buf (gpu.zig:117-134): a device pointer and a length in
//     4-byte elements; offset(n) is its pointer arithmetic.
//   * Sizes are size_t (Zig's usize); before the C ABI each passes through
//     ci(), which rejects a value that does not fit a C int as gpu.zig's
//     @intCast does (gpu.zig:416-418). Scalars are float; activation codes
//     are the ints of src/activations.zig:11-27.
//   * A failing call throws dkz::gpu::Error naming the call and, from the
//     library, the kernel and launch shape -- gpu.zig's must() panics with
//     the same information (gpu.zig:51-55, 444-464). Uncaught, it ends the
//     program as the panic does.
//   * Work is issued in call order, asynchronously; pull() and sync() wait
//     (gpu.zig:389-410, hip.zig:134).
//
// gpu.zig's backend selection, code-object search and kernel registry
// (gpu.zig:188-347) have no counterpart: the kernels live in libdkz.
#pragma once

#include <climits>
#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "dkz_ops.h"

namespace dkz {
namespace gpu {

class Error : public std::runtime_error {
   public:
    Error(int code, const std::string &what) : std::runtime_error(what), code_(code) {}
    int code() const { return code_; }

   private:
    int code_;
};

// gpu.zig:39: the backend's label as the reference prints it.
inline constexpr const char *backend_label = "HIP";

// gpu.zig:51-55 must(): a nonzero status ends the operation with a message.
inline void must(int err, const char *what) {
    if (err == 0) return;
    std::string msg = std::string(backend_label) + ": " + what + " failed: " + dkz_error_string(err);
    const char *ctx = dkz_last_error_context();
    if (ctx && ctx[0]) msg += std::string(" (") + ctx + ")";
    throw Error(err, msg);
}

// gpu.zig:416-418 ci(): usize -> c_int, checked.
inline int ci(size_t x) {
    if (x > (size_t)INT_MAX) throw Error(1, std::string(backend_label) + ": size " + std::to_string(x) +
                                                 " does not fit a C int");
    return (int)x;
}

// gpu.zig:117-134
struct Buf {
    void *ptr = nullptr;
    size_t len = 0;  // in 4-byte elements

    bool isNull() const { return ptr == nullptr; }
    Buf offset(size_t n) const {
        if (ptr == nullptr) return Buf{};
        if (n > len) throw Error(1, "Buf.offset past the end");
        return Buf{static_cast<char *>(ptr) + n * sizeof(float), len - n};
    }
    float *f() const { return static_cast<float *>(ptr); }
    int *i() const { return static_cast<int *>(ptr); }
};

// ---- device state (gpu.zig:141-183, 259-356) --------------------------------

// gpu.zig:32: this mirror is always built against libdkz (GPU support
// compiled in).
inline constexpr bool enabled = true;

inline int device_index = -1;

inline bool active() { return enabled && device_index >= 0; }

// gpu.zig:104-113: the GEMM a run uses, for a benchmark record -- the
// library's fp32 matrix-core kernel ("cpu" when no device is active) -- and
// the tile threshold the reference's blocked kernel was gated on, which the
// library does not have (0).
inline const char *gemmPolicy() { return active() ? "dkz-mfma" : "cpu"; }
inline unsigned long long gemmBlockMinTiles() { return 0; }

inline void setSyncAfterLaunch(bool on) { dkz_set_sync_after_launch(on ? 1 : 0); }

// gpu.zig:259-347: select the device; DARKNET_GPU_SYNC=1 turns on
// sync-after-launch (read by dkz_init).
inline void init(int index) {
    must(dkz_init(index), "selecting the device");
    device_index = index;
}

inline void sync() { must(dkz_synchronize(), "device synchronise"); }

inline void deinit() {  // gpu.zig:349-356
    if (!active()) return;
    sync();
    device_index = -1;
}

inline std::string deviceName() {  // gpu.zig:147-151
    if (!active()) return "CPU";
    char buf[256];
    must(dkz_device_name(device_index, buf, (int)sizeof buf), "querying the device name");
    return buf;
}

inline size_t deviceMemoryMib() {  // gpu.zig:153-155
    if (!active()) return 0;
    size_t free_b = 0, total = 0;
    must(dkz_mem_info(&free_b, &total), "querying device memory");
    return total >> 20;
}

// ---- memory (gpu.zig:362-410) ---------------------------------------------------

inline Buf alloc(size_t n) {
    if (n == 0) return Buf{};
    void *p = nullptr;
    must(dkz_malloc(&p, n * sizeof(float)), "device allocation");  // zero-filled, as gpu.zig:367
    return Buf{p, n};
}
inline Buf allocInts(size_t n) { return alloc(n); }

inline void free(Buf b) {
    if (b.ptr) must(dkz_free(b.ptr), "device free");
}

inline void push(Buf b, const float *host, size_t n) {
    if (n == 0 || b.ptr == nullptr) return;
    must(dkz_copy_to_device(b.ptr, host, n * sizeof(float)), "copy host to device");
}
inline void push(Buf b, const std::vector<float> &host) { push(b, host.data(), host.size()); }

inline void pull(Buf b, float *host, size_t n) {
    if (n == 0 || b.ptr == nullptr) return;
    must(dkz_copy_to_host(host, b.ptr, n * sizeof(float)), "copy device to host");
}
inline void pull(Buf b, std::vector<float> &host) { pull(b, host.data(), host.size()); }

inline void pullInts(Buf b, int32_t *host, size_t n) {
    if (n == 0 || b.ptr == nullptr) return;
    must(dkz_copy_to_host(host, b.ptr, n * sizeof(int32_t)), "copy device to host (ints)");
}
inline void pullInts(Buf b, std::vector<int32_t> &host) { pullInts(b, host.data(), host.size()); }

inline Buf make(const float *host, size_t n) {
    Buf b = alloc(n);
    push(b, host, n);
    return b;
}
inline Buf make(const std::vector<float> &host) { return make(host.data(), host.size()); }

// ---- elementwise (gpu.zig:483-521) ----------------------------------------------

inline void fill(Buf x, size_t n, float alpha) { must(dkz_fill(x.f(), ci(n), alpha), "fill"); }
inline void copy(size_t n, Buf x, Buf y) { must(dkz_copy(ci(n), x.f(), y.f()), "copy"); }
inline void axpy(size_t n, float alpha, Buf x, Buf y) { must(dkz_axpy(ci(n), alpha, x.f(), y.f()), "axpy"); }
inline void scal(size_t n, float alpha, Buf x) { must(dkz_scal(ci(n), alpha, x.f()), "scal"); }
inline void mul(size_t n, Buf x, Buf y) { must(dkz_mul(ci(n), x.f(), y.f()), "mul"); }
inline void addScalar(size_t n, float alpha, Buf x) { must(dkz_add_scalar(ci(n), alpha, x.f()), "add_scalar"); }
inline void constrainArray(size_t n, float alpha, Buf x) { must(dkz_constrain(ci(n), alpha, x.f()), "constrain"); }
inline void randUniform(size_t n, Buf x, uint32_t seed) {
    must(dkz_rand_uniform(ci(n), x.f(), seed), "rand_uniform");
}
inline void activateArray(Buf x, size_t n, int a) { must(dkz_activate_array(x.f(), ci(n), a), "activate_array"); }
inline void gradientArray(Buf x, size_t n, int a, Buf delta) {
    must(dkz_gradient_array(x.f(), ci(n), a, delta.f()), "gradient_array");
}

// ---- bias / scale (gpu.zig:527-555) ---------------------------------------------

inline void addBias(Buf output, Buf biases, size_t batch, size_t filters, size_t spatial) {
    must(dkz_add_bias(output.f(), biases.f(), ci(batch), ci(filters), ci(spatial)), "add_bias");
}
inline void scaleBias(Buf output, Buf scales, size_t batch, size_t filters, size_t spatial) {
    must(dkz_scale_bias(output.f(), scales.f(), ci(batch), ci(filters), ci(spatial)), "scale_bias");
}
inline void backwardBias(Buf bias_updates, Buf delta, size_t batch, size_t filters, size_t spatial) {
    must(dkz_backward_bias(bias_updates.f(), delta.f(), ci(batch), ci(filters), ci(spatial)), "backward_bias");
}
inline void backwardScale(Buf x_norm, Buf delta, size_t batch, size_t filters, size_t spatial, Buf scale_updates) {
    must(dkz_backward_scale(x_norm.f(), delta.f(), ci(batch), ci(filters), ci(spatial), scale_updates.f()),
         "backward_scale");
}

// ---- batch normalisation (gpu.zig:561-608) --------------------------------------

inline void mean(Buf x, size_t batch, size_t filters, size_t spatial, Buf out) {
    must(dkz_mean(x.f(), ci(batch), ci(filters), ci(spatial), out.f()), "mean");
}
inline void variance(Buf x, Buf mean_in, size_t batch, size_t filters, size_t spatial, Buf out) {
    must(dkz_variance(x.f(), mean_in.f(), ci(batch), ci(filters), ci(spatial), out.f()), "variance");
}
inline void normalize(Buf x, Buf mean_in, Buf variance_in, size_t batch, size_t filters, size_t spatial) {
    must(dkz_normalize(x.f(), mean_in.f(), variance_in.f(), ci(batch), ci(filters), ci(spatial)), "normalize");
}
inline void meanDelta(Buf delta, Buf variance_in, size_t batch, size_t filters, size_t spatial, Buf out) {
    must(dkz_mean_delta(delta.f(), variance_in.f(), ci(batch), ci(filters), ci(spatial), out.f()), "mean_delta");
}
inline void varianceDelta(Buf x, Buf delta, Buf mean_in, Buf variance_in, size_t batch, size_t filters,
                          size_t spatial, Buf out) {
    must(dkz_variance_delta(x.f(), delta.f(), mean_in.f(), variance_in.f(), ci(batch), ci(filters), ci(spatial),
                            out.f()),
         "variance_delta");
}
inline void normalizeDelta(Buf x, Buf mean_in, Buf variance_in, Buf mean_delta, Buf variance_delta, size_t batch,
                           size_t filters, size_t spatial, Buf delta) {
    must(dkz_normalize_delta(x.f(), mean_in.f(), variance_in.f(), mean_delta.f(), variance_delta.f(), ci(batch),
                             ci(filters), ci(spatial), delta.f()),
         "normalize_delta");
}

// ---- softmax and losses (gpu.zig:614-645) ---------------------------------------

inline void softmax(Buf input, size_t n, size_t batch, size_t batch_offset, size_t groups, size_t group_offset,
                    size_t stride, float temp, Buf output) {
    must(dkz_softmax(input.f(), ci(n), ci(batch), ci(batch_offset), ci(groups), ci(group_offset), ci(stride), temp,
                     output.f()),
         "softmax");
}
inline void softmaxCrossEntropy(size_t n, Buf pred, Buf truth, Buf delta, Buf err) {
    must(dkz_softmax_cross_entropy(ci(n), pred.f(), truth.f(), delta.f(), err.f()), "softmax_x_ent");
}
// No single gpu.zig counterpart: layers/misc.zig:63-76 (softmax, then the
// cross-entropy when truth is not null) as one call.
inline void softmaxLayerForward(size_t batch, size_t inputs, size_t groups, float temp, Buf input, Buf truth,
                                Buf output, Buf delta, Buf loss) {
    must(dkz_softmax_layer_forward(ci(batch), ci(inputs), ci(groups), temp, input.f(), truth.f(), output.f(),
                                   delta.f(), loss.f()),
         "softmax_layer_forward");
}
inline void l2(size_t n, Buf pred, Buf truth, Buf delta, Buf err) {
    must(dkz_l2(ci(n), pred.f(), truth.f(), delta.f(), err.f()), "l2");
}
inline void l1(size_t n, Buf pred, Buf truth, Buf delta, Buf err) {
    must(dkz_l1(ci(n), pred.f(), truth.f(), delta.f(), err.f()), "l1");
}
inline void smoothL1(size_t n, Buf pred, Buf truth, Buf delta, Buf err) {
    must(dkz_smooth_l1(ci(n), pred.f(), truth.f(), delta.f(), err.f()), "smooth_l1");
}

// ---- convolution helpers (gpu.zig:651-719) --------------------------------------

inline void im2col(Buf im, size_t channels, size_t height, size_t width, size_t ksize, size_t stride, size_t pad,
                   Buf col) {
    must(dkz_im2col(im.f(), ci(channels), ci(height), ci(width), ci(ksize), ci(stride), ci(pad), col.f()), "im2col");
}
inline void col2im(Buf col, size_t channels, size_t height, size_t width, size_t ksize, size_t stride, size_t pad,
                   Buf im) {
    must(dkz_col2im(col.f(), ci(channels), ci(height), ci(width), ci(ksize), ci(stride), ci(pad), im.f()), "col2im");
}
inline void gemm(bool ta, bool tb, size_t m, size_t n, size_t k, float alpha, Buf a, size_t lda, Buf b, size_t ldb,
                 float beta, Buf c, size_t ldc) {
    must(dkz_gemm(ta ? 1 : 0, tb ? 1 : 0, ci(m), ci(n), ci(k), alpha, a.f(), ci(lda), b.f(), ci(ldb), beta, c.f(),
                  ci(ldc)),
         "gemm");
}

// The per-image im2col + gemm loop of layers/convolutional.zig:240-260 in one call.
inline void convolutionForward(size_t batch, size_t groups, size_t channels, size_t height, size_t width,
                               size_t filters, size_t ksize, size_t stride, size_t pad, Buf weights, Buf input,
                               Buf output) {
    must(dkz_convolution_forward(ci(batch), ci(groups), ci(channels), ci(height), ci(width), ci(filters), ci(ksize),
                                 ci(stride), ci(pad), weights.f(), input.f(), output.f()),
         "convolution_forward");
}

// The weight-gradient gemms of layers/convolutional.zig:288-297 in one call.
inline void convolutionWeightGradient(size_t batch, size_t groups, size_t channels, size_t height, size_t width,
                                      size_t filters, size_t ksize, size_t stride, size_t pad, Buf delta, Buf input,
                                      Buf weight_updates) {
    must(dkz_convolution_weight_gradient(ci(batch), ci(groups), ci(channels), ci(height), ci(width), ci(filters),
                                         ci(ksize), ci(stride), ci(pad), delta.f(), input.f(), weight_updates.f()),
         "convolution_weight_gradient");
}

// The data-gradient gemms and col2im of layers/convolutional.zig:299-305 in one call.
inline void convolutionDataGradient(size_t batch, size_t groups, size_t channels, size_t height, size_t width,
                                    size_t filters, size_t ksize, size_t stride, size_t pad, Buf weights, Buf delta,
                                    Buf input_delta) {
    must(dkz_convolution_data_gradient(ci(batch), ci(groups), ci(channels), ci(height), ci(width), ci(filters),
                                       ci(ksize), ci(stride), ci(pad), weights.f(), delta.f(), input_delta.f()),
         "convolution_data_gradient");
}

// ---- pooling, dropout, shortcut, adam (gpu.zig:725-830) --------------------------

inline void forwardMaxpool(size_t out_n, size_t in_h, size_t in_w, size_t in_c, size_t stride, size_t size,
                           size_t pad, Buf input, Buf output, Buf indexes) {
    must(dkz_forward_maxpool(ci(out_n), ci(in_h), ci(in_w), ci(in_c), ci(stride), ci(size), ci(pad), input.f(),
                             output.f(), indexes.i()),
         "forward_maxpool");
}
inline void backwardMaxpool(size_t in_n, size_t in_h, size_t in_w, size_t in_c, size_t stride, size_t size,
                            size_t pad, Buf delta, Buf prev_delta, Buf indexes) {
    must(dkz_backward_maxpool(ci(in_n), ci(in_h), ci(in_w), ci(in_c), ci(stride), ci(size), ci(pad), delta.f(),
                              prev_delta.f(), indexes.i()),
         "backward_maxpool");
}
inline void forwardAvgpool(size_t n, size_t w, size_t h, size_t c, Buf input, Buf output) {
    must(dkz_forward_avgpool(ci(n), ci(w), ci(h), ci(c), input.f(), output.f()), "forward_avgpool");
}
inline void backwardAvgpool(size_t n, size_t w, size_t h, size_t c, Buf in_delta, Buf out_delta) {
    must(dkz_backward_avgpool(ci(n), ci(w), ci(h), ci(c), in_delta.f(), out_delta.f()), "backward_avgpool");
}
inline void dropout(Buf input, size_t size, Buf rand_buf, float prob, float scale) {
    must(dkz_dropout(input.f(), ci(size), rand_buf.f(), prob, scale), "dropout");
}
inline void shortcut(size_t batch, size_t w1, size_t h1, size_t c1, Buf add, size_t w2, size_t h2, size_t c2,
                     float s1, float s2, Buf out) {
    must(dkz_shortcut(ci(batch), ci(w1), ci(h1), ci(c1), add.f(), ci(w2), ci(h2), ci(c2), s1, s2, out.f()),
         "shortcut");
}
inline void adamUpdate(Buf w, Buf d, Buf m, Buf v, float b1, float b2, float eps, float decay, float rate, size_t n,
                       size_t batch, size_t t) {
    must(dkz_adam_update(w.f(), d.f(), m.f(), v.f(), b1, b2, eps, decay, rate, ci(n), ci(batch), ci(t)),
         "adam_update");
}

// ---- fused batch-norm layer passes (no single gpu.zig counterpart: each
// replaces the call sequence of layers/batchnorm.zig forwardGpu / backwardGpu
// with the activation calls of convolutional.zig:269 and :280) ------------------

inline void batchnormForward(size_t batch, size_t filters, size_t spatial, int activation, bool train, Buf input,
                             Buf output, Buf x, Buf x_norm, Buf mean_out, Buf variance_out, Buf rolling_mean,
                             Buf rolling_variance, Buf scales, Buf biases) {
    must(dkz_batchnorm_forward(ci(batch), ci(filters), ci(spatial), activation, train ? 1 : 0, input.f(), output.f(),
                               x.f(), x_norm.f(), mean_out.f(), variance_out.f(), rolling_mean.f(),
                               rolling_variance.f(), scales.f(), biases.f()),
         "batchnorm_forward");
}
inline void batchnormBackward(size_t batch, size_t filters, size_t spatial, int activation, Buf output, Buf delta,
                              Buf x, Buf x_norm, Buf mean_in, Buf variance_in, Buf scales, Buf bias_updates,
                              Buf scale_updates, Buf mean_delta, Buf variance_delta) {
    must(dkz_batchnorm_backward(ci(batch), ci(filters), ci(spatial), activation, output.f(), delta.f(), x.f(),
                                x_norm.f(), mean_in.f(), variance_in.f(), scales.f(), bias_updates.f(),
                                scale_updates.f(), mean_delta.f(), variance_delta.f()),
         "batchnorm_backward");
}

}  // namespace gpu
}  // namespace dkz
