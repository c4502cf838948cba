//! dkz.zig -- the C ABI of libdkz.so (include/dkz_ops.h) as Zig `extern fn`
//! declarations, every entry point in the header's order. This file replaces
//! the reference's HIP backend interface (src/hip/hip.zig:60-135) and the
//! kernel registry and launch helpers of src/gpu.zig (:188-257, :416-477):
//! gpu.zig's public wrappers (gpu.zig in this directory) call these instead.
//!
//! Types follow the header: int -> c_int, unsigned -> c_uint, float -> f32,
//! size_t -> usize; device buffers (float *, const float *) are
//! ?*anyopaque, the type of gpu.zig's Buf.ptr; host pointers keep their
//! element type. Every op returns a hipError_t value (0 on success).
//! tests/test_zig_binding.py checks these lines against the header.
//!
//! Link: exe.linkSystemLibrary("dkz") with libdkz.so's directory on the
//! library path, and exe.linkLibC().

/// hipError_t: 0 on success.
pub const Status = c_int;

pub extern fn dkz_init(device: c_int) Status;
pub extern fn dkz_device_count(count: *c_int) Status;
pub extern fn dkz_device_name(device: c_int, buf: [*]u8, len: c_int) Status;
pub extern fn dkz_mem_info(free_bytes: *usize, total_bytes: *usize) Status;
pub extern fn dkz_malloc(ptr: *?*anyopaque, bytes: usize) Status;
pub extern fn dkz_free(ptr: ?*anyopaque) Status;
pub extern fn dkz_memset_zero(ptr: ?*anyopaque, bytes: usize) Status;
pub extern fn dkz_copy_to_device(dst: ?*anyopaque, src: *const anyopaque, bytes: usize) Status;
pub extern fn dkz_copy_to_host(dst: *anyopaque, src: ?*const anyopaque, bytes: usize) Status;
pub extern fn dkz_synchronize() Status;
pub extern fn dkz_error_string(err: c_int) [*:0]const u8;
pub extern fn dkz_set_sync_after_launch(on: c_int) void;
pub extern fn dkz_get_sync_after_launch() c_int;
pub extern fn dkz_last_error_context() [*:0]const u8;
pub extern fn dkz_set_stream(stream: ?*anyopaque) Status;
pub extern fn dkz_get_stream() ?*anyopaque;
pub extern fn dkz_fill(x: ?*anyopaque, n: c_int, alpha: f32) Status;
pub extern fn dkz_copy(n: c_int, x: ?*anyopaque, y: ?*anyopaque) Status;
pub extern fn dkz_axpy(n: c_int, alpha: f32, x: ?*anyopaque, y: ?*anyopaque) Status;
pub extern fn dkz_scal(n: c_int, alpha: f32, x: ?*anyopaque) Status;
pub extern fn dkz_mul(n: c_int, x: ?*anyopaque, y: ?*anyopaque) Status;
pub extern fn dkz_add_scalar(n: c_int, alpha: f32, x: ?*anyopaque) Status;
pub extern fn dkz_constrain(n: c_int, alpha: f32, x: ?*anyopaque) Status;
pub extern fn dkz_rand_uniform(n: c_int, x: ?*anyopaque, seed: c_uint) Status;
pub extern fn dkz_activate_array(x: ?*anyopaque, n: c_int, a: c_int) Status;
pub extern fn dkz_gradient_array(x: ?*anyopaque, n: c_int, a: c_int, delta: ?*anyopaque) Status;
pub extern fn dkz_add_bias(output: ?*anyopaque, biases: ?*anyopaque, batch: c_int, filters: c_int, spatial: c_int) Status;
pub extern fn dkz_scale_bias(output: ?*anyopaque, scales: ?*anyopaque, batch: c_int, filters: c_int, spatial: c_int) Status;
pub extern fn dkz_backward_bias(bias_updates: ?*anyopaque, delta: ?*anyopaque, batch: c_int, filters: c_int, spatial: c_int) Status;
pub extern fn dkz_backward_scale(x_norm: ?*anyopaque, delta: ?*anyopaque, batch: c_int, filters: c_int, spatial: c_int, scale_updates: ?*anyopaque) Status;
pub extern fn dkz_mean(x: ?*anyopaque, batch: c_int, filters: c_int, spatial: c_int, out: ?*anyopaque) Status;
pub extern fn dkz_variance(x: ?*anyopaque, mean: ?*anyopaque, batch: c_int, filters: c_int, spatial: c_int, out: ?*anyopaque) Status;
pub extern fn dkz_normalize(x: ?*anyopaque, mean: ?*anyopaque, variance: ?*anyopaque, batch: c_int, filters: c_int, spatial: c_int) Status;
pub extern fn dkz_mean_delta(delta: ?*anyopaque, variance: ?*anyopaque, batch: c_int, filters: c_int, spatial: c_int, out: ?*anyopaque) Status;
pub extern fn dkz_variance_delta(x: ?*anyopaque, delta: ?*anyopaque, mean: ?*anyopaque, variance: ?*anyopaque, batch: c_int, filters: c_int, spatial: c_int, out: ?*anyopaque) Status;
pub extern fn dkz_normalize_delta(x: ?*anyopaque, mean: ?*anyopaque, variance: ?*anyopaque, mean_delta: ?*anyopaque, variance_delta: ?*anyopaque, batch: c_int, filters: c_int, spatial: c_int, delta: ?*anyopaque) Status;
pub extern fn dkz_softmax(input: ?*anyopaque, n: c_int, batch: c_int, batch_offset: c_int, groups: c_int, group_offset: c_int, stride: c_int, temp: f32, output: ?*anyopaque) Status;
pub extern fn dkz_softmax_layer_forward(batch: c_int, inputs: c_int, groups: c_int, temp: f32, input: ?*anyopaque, truth: ?*anyopaque, output: ?*anyopaque, delta: ?*anyopaque, loss: ?*anyopaque) Status;
pub extern fn dkz_softmax_cross_entropy(n: c_int, pred: ?*anyopaque, truth: ?*anyopaque, delta: ?*anyopaque, err: ?*anyopaque) Status;
pub extern fn dkz_l2(n: c_int, pred: ?*anyopaque, truth: ?*anyopaque, delta: ?*anyopaque, err: ?*anyopaque) Status;
pub extern fn dkz_l1(n: c_int, pred: ?*anyopaque, truth: ?*anyopaque, delta: ?*anyopaque, err: ?*anyopaque) Status;
pub extern fn dkz_smooth_l1(n: c_int, pred: ?*anyopaque, truth: ?*anyopaque, delta: ?*anyopaque, err: ?*anyopaque) Status;
pub extern fn dkz_forward_maxpool(out_n: c_int, in_h: c_int, in_w: c_int, in_c: c_int, stride: c_int, size: c_int, pad: c_int, input: ?*anyopaque, output: ?*anyopaque, indexes: ?*anyopaque) Status;
pub extern fn dkz_backward_maxpool(in_n: c_int, in_h: c_int, in_w: c_int, in_c: c_int, stride: c_int, size: c_int, pad: c_int, delta: ?*anyopaque, prev_delta: ?*anyopaque, indexes: ?*anyopaque) Status;
pub extern fn dkz_forward_avgpool(n: c_int, w: c_int, h: c_int, c: c_int, input: ?*anyopaque, output: ?*anyopaque) Status;
pub extern fn dkz_backward_avgpool(n: c_int, w: c_int, h: c_int, c: c_int, in_delta: ?*anyopaque, out_delta: ?*anyopaque) Status;
pub extern fn dkz_shortcut(batch: c_int, w1: c_int, h1: c_int, c1: c_int, add: ?*anyopaque, w2: c_int, h2: c_int, c2: c_int, s1: f32, s2: f32, out: ?*anyopaque) Status;
pub extern fn dkz_im2col(im: ?*anyopaque, channels: c_int, height: c_int, width: c_int, ksize: c_int, stride: c_int, pad: c_int, col: ?*anyopaque) Status;
pub extern fn dkz_col2im(col: ?*anyopaque, channels: c_int, height: c_int, width: c_int, ksize: c_int, stride: c_int, pad: c_int, im: ?*anyopaque) Status;
pub extern fn dkz_gemm(ta: c_int, tb: c_int, m: c_int, n: c_int, k: c_int, alpha: f32, a: ?*anyopaque, lda: c_int, b: ?*anyopaque, ldb: c_int, beta: f32, c: ?*anyopaque, ldc: c_int) Status;
pub extern fn dkz_convolution_forward(batch: c_int, groups: c_int, channels: c_int, height: c_int, width: c_int, filters: c_int, ksize: c_int, stride: c_int, pad: c_int, weights: ?*anyopaque, input: ?*anyopaque, output: ?*anyopaque) Status;
pub extern fn dkz_convolution_weight_gradient(batch: c_int, groups: c_int, channels: c_int, height: c_int, width: c_int, filters: c_int, ksize: c_int, stride: c_int, pad: c_int, delta: ?*anyopaque, input: ?*anyopaque, weight_updates: ?*anyopaque) Status;
pub extern fn dkz_convolution_data_gradient(batch: c_int, groups: c_int, channels: c_int, height: c_int, width: c_int, filters: c_int, ksize: c_int, stride: c_int, pad: c_int, weights: ?*anyopaque, delta: ?*anyopaque, input_delta: ?*anyopaque) Status;
pub extern fn dkz_dropout(input: ?*anyopaque, size: c_int, rand: ?*anyopaque, prob: f32, scale: f32) Status;
pub extern fn dkz_adam_update(w: ?*anyopaque, d: ?*anyopaque, m: ?*anyopaque, v: ?*anyopaque, b1: f32, b2: f32, eps: f32, decay: f32, rate: f32, n: c_int, batch: c_int, t: c_int) Status;
pub extern fn dkz_batchnorm_forward(batch: c_int, filters: c_int, spatial: c_int, activation: c_int, train: c_int, input: ?*anyopaque, output: ?*anyopaque, x: ?*anyopaque, x_norm: ?*anyopaque, mean: ?*anyopaque, variance: ?*anyopaque, rolling_mean: ?*anyopaque, rolling_variance: ?*anyopaque, scales: ?*anyopaque, biases: ?*anyopaque) Status;
pub extern fn dkz_batchnorm_backward(batch: c_int, filters: c_int, spatial: c_int, activation: c_int, output: ?*anyopaque, delta: ?*anyopaque, x: ?*anyopaque, x_norm: ?*anyopaque, mean: ?*anyopaque, variance: ?*anyopaque, scales: ?*anyopaque, bias_updates: ?*anyopaque, scale_updates: ?*anyopaque, mean_delta: ?*anyopaque, variance_delta: ?*anyopaque) Status;
pub extern fn dkz_batchnorm_backward_noalloc(batch: c_int, filters: c_int, spatial: c_int, activation: c_int, output: ?*anyopaque, delta: ?*anyopaque, x: ?*anyopaque, x_norm: ?*anyopaque, mean: ?*anyopaque, variance: ?*anyopaque, scales: ?*anyopaque, bias_updates: ?*anyopaque, scale_updates: ?*anyopaque, mean_delta: ?*anyopaque, variance_delta: ?*anyopaque) Status;
