//! gpu.zig -- the public API of the reference's src/gpu.zig, re-pointed at
//! libdkz.so's C ABI (dkz.zig): the build switch and backend label, the
//! device state (device_index, active, deviceName, deviceMemoryMib, the GEMM
//! policy a benchmark run records), init/deinit, Buf and the memory calls,
//! setSyncAfterLaunch, and the op wrappers of gpu.zig:483-830. Every public
//! name and signature the reference's callers use is the reference's
//! (tests/golden/gpu_zig_callers.json lists each one with its callers), so
//! the layers, network, parser, main, benchmark and gputest compile against
//! this file unchanged when it takes gpu.zig's place. Each op body is one
//! dkz_* call through must(), which panics with the reference's message
//! shape (gpu.zig:51-55) plus the library's context (the kernel and launch
//! shape that failed). The code-object lookup, the kernel registry,
//! launchDims/launch1d/launchPerFilter and the GEMM kernel choice are gone:
//! the library picks its own kernels and launch geometry.
//!
//! As in the reference, a build without -Dgpu (`enabled` false) references
//! no GPU symbol: every wrapper that would reach the library starts with
//! `if (!enabled) unreachable;` (gpu.zig:363, 390, 432), so nothing needs
//! to link against libdkz.so there.
//!
//! Sizes are usize as in the reference and cross the ABI as c_int (ci(),
//! gpu.zig:416-418); buffers cross as their device pointer.
const std = @import("std");
const build_options = @import("build_options");
const dkz = @import("dkz.zig");

/// gpu.zig:32: whether this build has GPU support (zig build -Dgpu=true).
pub const enabled = build_options.gpu;

/// gpu.zig:39: the backend's label in messages and benchmark records. The
/// library runs on HIP, so the reference's HIP label stands.
pub const backend_label = "HIP";

fn check(err: dkz.Status, what: []const u8) !void {
    if (err != 0) {
        std.debug.print("{s}: {s} failed: {s} {s}\n", .{
            backend_label, what, dkz.dkz_error_string(err), dkz.dkz_last_error_context(),
        });
        return error.GpuError;
    }
}

fn must(err: dkz.Status, what: []const u8) void {
    if (err != 0) std.debug.panic("{s}: {s} failed: {s} {s}", .{
        backend_label, what, dkz.dkz_error_string(err), dkz.dkz_last_error_context(),
    });
}

inline fn ci(x: usize) c_int {
    return @intCast(x);
}

/// gpu.zig:104-108: which GEMM a GPU run uses, for the benchmark to record.
/// The library has one, on the fp32 matrix cores; "cpu" when no device is
/// active, as in the reference.
pub fn gemmPolicy() []const u8 {
    if (!active()) return "cpu";
    return "dkz-mfma";
}

/// gpu.zig:111-113: the tile threshold the reference's register-blocked GEMM
/// was gated on. The library chooses its tiles from the shape alone, with no
/// such threshold: 0, as the reference reports when its gate is off.
pub fn gemmBlockMinTiles() u64 {
    return 0;
}

/// A device buffer: the reference's Buf (gpu.zig:117-133).
pub const Buf = struct {
    ptr: ?*anyopaque = null,
    /// Length in floats, not bytes.
    len: usize = 0,

    pub fn isNull(self: Buf) bool {
        return self.ptr == null;
    }

    /// A view starting `n` floats in, as darknet's pointer arithmetic on
    /// `float *` picks one image's slice of a batch.
    pub fn offset(self: Buf, n: usize) Buf {
        if (self.ptr == null) return .{};
        std.debug.assert(n <= self.len);
        const base: [*]u8 = @ptrCast(self.ptr.?);
        return .{ .ptr = @ptrCast(base + n * @sizeOf(f32)), .len = self.len - n };
    }
};

// ---------------------------------------------------------------------------
// state (gpu.zig:139-160)
// ---------------------------------------------------------------------------

/// -1 means "run on the CPU"; set by init, reset by deinit.
pub var device_index: i32 = -1;
/// Set by init, so a run can record which device produced its numbers.
var device_name_buf: [256]u8 = @splat(0);
var device_total_mib: usize = 0;

/// The selected device's name, or "CPU" when no device is active.
pub fn deviceName() []const u8 {
    if (!active()) return "CPU";
    return std.mem.sliceTo(&device_name_buf, 0);
}

/// Total memory of the selected device in MiB; 0 when running on the CPU.
pub fn deviceMemoryMib() usize {
    return if (active()) device_total_mib else 0;
}

pub fn active() bool {
    return enabled and device_index >= 0;
}

// ---------------------------------------------------------------------------
// device and memory (gpu.zig:181, 259-410)
// ---------------------------------------------------------------------------

/// Per-launch synchronisation on or off (gpu.zig:181-183); the library
/// then names a faulting kernel and its launch shape.
pub fn setSyncAfterLaunch(on: bool) void {
    if (!enabled) return;
    dkz.dkz_set_sync_after_launch(@intFromBool(on));
}

/// Selects GPU `index` and sets the library up (its per-device scratch);
/// DARKNET_GPU_SYNC / DARKNET_HIP_SYNC turn sync-after-launch on, and the
/// device's name and memory are recorded, as in gpu.zig:259-347. Prints the
/// device the way the reference does.
pub fn init(allocator: std.mem.Allocator, index: i32) !void {
    _ = allocator; // the reference used it for the code-object path; nothing to load here
    if (!enabled) {
        std.debug.print(
            \\This binary was built without GPU support.
            \\Rebuild with: zig build -Dgpu=true (and libdkz.so on the library path)
            \\
        , .{});
        return error.GpuNotCompiledIn;
    }
    var count: c_int = 0;
    try check(dkz.dkz_device_count(&count), "querying device count");
    if (index < 0 or index >= count) {
        std.debug.print("Requested GPU {d} but only {d} HIP device(s) present\n", .{ index, count });
        return error.NoSuchDevice;
    }
    try check(dkz.dkz_init(@intCast(index)), "initialising the device");
    device_name_buf = @splat(0);
    try check(dkz.dkz_device_name(@intCast(index), &device_name_buf, device_name_buf.len), "querying the device name");
    if (dkz.dkz_get_sync_after_launch() != 0) {
        std.debug.print("DARKNET_GPU_SYNC set: synchronising and checking after every kernel launch.\n", .{});
    }
    device_index = index;
    var free_b: usize = 0;
    var total_b: usize = 0;
    _ = dkz.dkz_mem_info(&free_b, &total_b);
    device_total_mib = total_b >> 20;
    std.debug.print("{s} device {d}: {s} ({d} MiB free / {d} MiB total)\n", .{
        backend_label, index, std.mem.sliceTo(&device_name_buf, 0), free_b >> 20, total_b >> 20,
    });
}

/// gpu.zig:349-356: back to the CPU. The library keeps its per-device
/// scratch until the process ends (there is no code object to unload).
pub fn deinit() void {
    if (!enabled) return;
    device_index = -1;
}

/// n floats of device memory, zero-filled (gpu.zig:362-369).
pub fn alloc(n: usize) Buf {
    if (!enabled) unreachable;
    if (n == 0) return .{};
    var ptr: ?*anyopaque = null;
    must(dkz.dkz_malloc(&ptr, n * @sizeOf(f32)), "device allocation");
    return .{ .ptr = ptr, .len = n };
}

/// Device buffer for n 32-bit ints (maxpool argmax indices).
pub fn allocInts(n: usize) Buf {
    return alloc(n);
}

/// Allocate and upload in one go.
pub fn make(host: []const f32) Buf {
    const b = alloc(host.len);
    push(b, host);
    return b;
}

pub fn free(b: Buf) void {
    if (!enabled) return;
    if (b.ptr) |p| must(dkz.dkz_free(p), "device free");
}

pub fn push(b: Buf, host: []const f32) void {
    if (!enabled) unreachable;
    if (host.len == 0 or b.ptr == null) return;
    must(dkz.dkz_copy_to_device(b.ptr, host.ptr, host.len * @sizeOf(f32)), "copy host to device");
}

pub fn pull(b: Buf, host: []f32) void {
    if (!enabled) unreachable;
    if (host.len == 0 or b.ptr == null) return;
    must(dkz.dkz_copy_to_host(host.ptr, b.ptr, host.len * @sizeOf(f32)), "copy device to host");
}

pub fn pullInts(b: Buf, host: []i32) void {
    if (!enabled) unreachable;
    if (host.len == 0 or b.ptr == null) return;
    must(dkz.dkz_copy_to_host(host.ptr, b.ptr, host.len * @sizeOf(i32)), "copy device to host (ints)");
}

pub fn sync() void {
    if (!enabled) return;
    must(dkz.dkz_synchronize(), "device synchronise");
}

// ---------------------------------------------------------------------------
// ops (gpu.zig:483-830), one dkz_* call each
// ---------------------------------------------------------------------------

pub fn fill(x: Buf, n: usize, alpha: f32) void {
    if (!enabled) unreachable;
    must(dkz.dkz_fill(x.ptr, ci(n), alpha), "fill");
}

pub fn copy(n: usize, x: Buf, y: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_copy(ci(n), x.ptr, y.ptr), "copy");
}

pub fn axpy(n: usize, alpha: f32, x: Buf, y: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_axpy(ci(n), alpha, x.ptr, y.ptr), "axpy");
}

pub fn scal(n: usize, alpha: f32, x: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_scal(ci(n), alpha, x.ptr), "scal");
}

pub fn mul(n: usize, x: Buf, y: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_mul(ci(n), x.ptr, y.ptr), "mul");
}

pub fn addScalar(n: usize, alpha: f32, x: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_add_scalar(ci(n), alpha, x.ptr), "add_scalar");
}

pub fn constrainArray(n: usize, alpha: f32, x: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_constrain(ci(n), alpha, x.ptr), "constrain");
}

pub fn randUniform(n: usize, x: Buf, seed: u32) void {
    if (!enabled) unreachable;
    must(dkz.dkz_rand_uniform(ci(n), x.ptr, seed), "rand_uniform");
}

pub fn activateArray(x: Buf, n: usize, a: c_int) void {
    if (!enabled) unreachable;
    must(dkz.dkz_activate_array(x.ptr, ci(n), a), "activate_array");
}

pub fn gradientArray(x: Buf, n: usize, a: c_int, delta: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_gradient_array(x.ptr, ci(n), a, delta.ptr), "gradient_array");
}

pub fn addBias(output: Buf, biases: Buf, batch: usize, filters: usize, spatial: usize) void {
    if (!enabled) unreachable;
    must(dkz.dkz_add_bias(output.ptr, biases.ptr, ci(batch), ci(filters), ci(spatial)), "add_bias");
}

pub fn scaleBias(output: Buf, scales: Buf, batch: usize, filters: usize, spatial: usize) void {
    if (!enabled) unreachable;
    must(dkz.dkz_scale_bias(output.ptr, scales.ptr, ci(batch), ci(filters), ci(spatial)), "scale_bias");
}

/// The spatial == 1 case of gpu.zig:540-548 is the library's too.
pub fn backwardBias(bias_updates: Buf, delta: Buf, batch: usize, filters: usize, spatial: usize) void {
    if (!enabled) unreachable;
    must(dkz.dkz_backward_bias(bias_updates.ptr, delta.ptr, ci(batch), ci(filters), ci(spatial)), "backward_bias");
}

pub fn backwardScale(x_norm: Buf, delta: Buf, batch: usize, filters: usize, spatial: usize, scale_updates: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_backward_scale(x_norm.ptr, delta.ptr, ci(batch), ci(filters), ci(spatial), scale_updates.ptr), "backward_scale");
}

pub fn mean(x: Buf, batch: usize, filters: usize, spatial: usize, out: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_mean(x.ptr, ci(batch), ci(filters), ci(spatial), out.ptr), "mean");
}

pub fn variance(x: Buf, mean_in: Buf, batch: usize, filters: usize, spatial: usize, out: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_variance(x.ptr, mean_in.ptr, ci(batch), ci(filters), ci(spatial), out.ptr), "variance");
}

pub fn normalize(x: Buf, mean_in: Buf, variance_in: Buf, batch: usize, filters: usize, spatial: usize) void {
    if (!enabled) unreachable;
    must(dkz.dkz_normalize(x.ptr, mean_in.ptr, variance_in.ptr, ci(batch), ci(filters), ci(spatial)), "normalize");
}

pub fn meanDelta(delta: Buf, variance_in: Buf, batch: usize, filters: usize, spatial: usize, out: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_mean_delta(delta.ptr, variance_in.ptr, ci(batch), ci(filters), ci(spatial), out.ptr), "mean_delta");
}

pub fn varianceDelta(x: Buf, delta: Buf, mean_in: Buf, variance_in: Buf, batch: usize, filters: usize, spatial: usize, out: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_variance_delta(x.ptr, delta.ptr, mean_in.ptr, variance_in.ptr, ci(batch), ci(filters), ci(spatial), out.ptr), "variance_delta");
}

pub fn normalizeDelta(
    x: Buf,
    mean_in: Buf,
    variance_in: Buf,
    mean_delta_in: Buf,
    variance_delta_in: Buf,
    batch: usize,
    filters: usize,
    spatial: usize,
    delta: Buf,
) void {
    if (!enabled) unreachable;
    must(dkz.dkz_normalize_delta(x.ptr, mean_in.ptr, variance_in.ptr, mean_delta_in.ptr, variance_delta_in.ptr, ci(batch), ci(filters), ci(spatial), delta.ptr), "normalize_delta");
}

pub fn softmax(
    input: Buf,
    n: usize,
    batch: usize,
    batch_offset: usize,
    groups: usize,
    group_offset: usize,
    stride: usize,
    temp: f32,
    output: Buf,
) void {
    if (!enabled) unreachable;
    must(dkz.dkz_softmax(input.ptr, ci(n), ci(batch), ci(batch_offset), ci(groups), ci(group_offset), ci(stride), temp, output.ptr), "softmax");
}

pub fn softmaxCrossEntropy(n: usize, pred: Buf, truth: Buf, delta: Buf, err: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_softmax_cross_entropy(ci(n), pred.ptr, truth.ptr, delta.ptr, err.ptr), "softmax_x_ent");
}

pub fn l2(n: usize, pred: Buf, truth: Buf, delta: Buf, err: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_l2(ci(n), pred.ptr, truth.ptr, delta.ptr, err.ptr), "l2");
}

pub fn l1(n: usize, pred: Buf, truth: Buf, delta: Buf, err: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_l1(ci(n), pred.ptr, truth.ptr, delta.ptr, err.ptr), "l1");
}

pub fn smoothL1(n: usize, pred: Buf, truth: Buf, delta: Buf, err: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_smooth_l1(ci(n), pred.ptr, truth.ptr, delta.ptr, err.ptr), "smooth_l1");
}

pub fn im2col(im: Buf, channels: usize, height: usize, width: usize, ksize: usize, stride: usize, pad: usize, col: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_im2col(im.ptr, ci(channels), ci(height), ci(width), ci(ksize), ci(stride), ci(pad), col.ptr), "im2col");
}

pub fn col2im(col: Buf, channels: usize, height: usize, width: usize, ksize: usize, stride: usize, pad: usize, im: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_col2im(col.ptr, ci(channels), ci(height), ci(width), ci(ksize), ci(stride), ci(pad), im.ptr), "col2im");
}

/// The tile policy of gpu.zig:686-718 is the library's own choice now.
pub fn gemm(
    ta: bool,
    tb: bool,
    m: usize,
    n: usize,
    k: usize,
    alpha: f32,
    a: Buf,
    lda: usize,
    b: Buf,
    ldb: usize,
    beta: f32,
    c: Buf,
    ldc: usize,
) void {
    if (!enabled) unreachable;
    must(dkz.dkz_gemm(@intFromBool(ta), @intFromBool(tb), ci(m), ci(n), ci(k), alpha, a.ptr, ci(lda), b.ptr, ci(ldb), beta, c.ptr, ci(ldc)), "gemm");
}

pub fn forwardMaxpool(
    out_n: usize,
    in_h: usize,
    in_w: usize,
    in_c: usize,
    stride: usize,
    size: usize,
    pad: usize,
    input: Buf,
    output: Buf,
    indexes: Buf,
) void {
    if (!enabled) unreachable;
    must(dkz.dkz_forward_maxpool(ci(out_n), ci(in_h), ci(in_w), ci(in_c), ci(stride), ci(size), ci(pad), input.ptr, output.ptr, indexes.ptr), "forward_maxpool");
}

pub fn backwardMaxpool(
    in_n: usize,
    in_h: usize,
    in_w: usize,
    in_c: usize,
    stride: usize,
    size: usize,
    pad: usize,
    delta: Buf,
    prev_delta: Buf,
    indexes: Buf,
) void {
    if (!enabled) unreachable;
    must(dkz.dkz_backward_maxpool(ci(in_n), ci(in_h), ci(in_w), ci(in_c), ci(stride), ci(size), ci(pad), delta.ptr, prev_delta.ptr, indexes.ptr), "backward_maxpool");
}

pub fn forwardAvgpool(n: usize, w: usize, h: usize, c: usize, input: Buf, output: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_forward_avgpool(ci(n), ci(w), ci(h), ci(c), input.ptr, output.ptr), "forward_avgpool");
}

pub fn backwardAvgpool(n: usize, w: usize, h: usize, c: usize, in_delta: Buf, out_delta: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_backward_avgpool(ci(n), ci(w), ci(h), ci(c), in_delta.ptr, out_delta.ptr), "backward_avgpool");
}

pub fn dropout(input: Buf, size: usize, rand_buf: Buf, prob: f32, scale: f32) void {
    if (!enabled) unreachable;
    must(dkz.dkz_dropout(input.ptr, ci(size), rand_buf.ptr, prob, scale), "dropout");
}

/// The stride/sample/min marshalling of gpu.zig:786-793 is the library's.
pub fn shortcut(
    batch: usize,
    w1: usize,
    h1: usize,
    c1: usize,
    add: Buf,
    w2: usize,
    h2: usize,
    c2: usize,
    s1: f32,
    s2: f32,
    out: Buf,
) void {
    if (!enabled) unreachable;
    must(dkz.dkz_shortcut(ci(batch), ci(w1), ci(h1), ci(c1), add.ptr, ci(w2), ci(h2), ci(c2), s1, s2, out.ptr), "shortcut");
}

/// gpu.zig:804-830's eight launches are one pass.
pub fn adamUpdate(
    w: Buf,
    d: Buf,
    m: Buf,
    v: Buf,
    b1: f32,
    b2: f32,
    eps: f32,
    decay: f32,
    rate: f32,
    n: usize,
    batch: usize,
    t: usize,
) void {
    if (!enabled) unreachable;
    must(dkz.dkz_adam_update(w.ptr, d.ptr, m.ptr, v.ptr, b1, b2, eps, decay, rate, ci(n), ci(batch), ci(t)), "adam_update");
}

// ---------------------------------------------------------------------------
// entry points with no single gpu.zig counterpart: a layer's call sequence
// as one call (layers/batchnorm.zig:129-174 with the activation of
// convolutional.zig:269/280; layers/misc.zig:63-76; convolutional.zig:249-305)
// ---------------------------------------------------------------------------

pub fn batchnormForward(batch: usize, filters: usize, spatial: usize, activation: c_int, train: bool, input: Buf, output: Buf, x: Buf, x_norm: Buf, mean_out: Buf, variance_out: Buf, rolling_mean: Buf, rolling_variance: Buf, scales: Buf, biases: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_batchnorm_forward(ci(batch), ci(filters), ci(spatial), activation, @intFromBool(train), input.ptr, output.ptr, x.ptr, x_norm.ptr, mean_out.ptr, variance_out.ptr, rolling_mean.ptr, rolling_variance.ptr, scales.ptr, biases.ptr), "batchnorm_forward");
}

pub fn batchnormBackward(batch: usize, filters: usize, spatial: usize, activation: c_int, output: Buf, delta: Buf, x: Buf, x_norm: Buf, mean_in: Buf, variance_in: Buf, scales: Buf, bias_updates: Buf, scale_updates: Buf, mean_delta: Buf, variance_delta: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_batchnorm_backward(ci(batch), ci(filters), ci(spatial), activation, output.ptr, delta.ptr, x.ptr, x_norm.ptr, mean_in.ptr, variance_in.ptr, scales.ptr, bias_updates.ptr, scale_updates.ptr, mean_delta.ptr, variance_delta.ptr), "batchnorm_backward");
}

pub fn softmaxLayerForward(batch: usize, inputs: usize, groups: usize, temp: f32, input: Buf, truth: Buf, output: Buf, delta: Buf, loss: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_softmax_layer_forward(ci(batch), ci(inputs), ci(groups), temp, input.ptr, truth.ptr, output.ptr, delta.ptr, loss.ptr), "softmax_layer_forward");
}

pub fn convolutionForward(batch: usize, groups: usize, channels: usize, height: usize, width: usize, filters: usize, ksize: usize, stride: usize, pad: usize, weights: Buf, input: Buf, output: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_convolution_forward(ci(batch), ci(groups), ci(channels), ci(height), ci(width), ci(filters), ci(ksize), ci(stride), ci(pad), weights.ptr, input.ptr, output.ptr), "convolution_forward");
}

pub fn convolutionWeightGradient(batch: usize, groups: usize, channels: usize, height: usize, width: usize, filters: usize, ksize: usize, stride: usize, pad: usize, delta: Buf, input: Buf, weight_updates: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_convolution_weight_gradient(ci(batch), ci(groups), ci(channels), ci(height), ci(width), ci(filters), ci(ksize), ci(stride), ci(pad), delta.ptr, input.ptr, weight_updates.ptr), "convolution_weight_gradient");
}

pub fn convolutionDataGradient(batch: usize, groups: usize, channels: usize, height: usize, width: usize, filters: usize, ksize: usize, stride: usize, pad: usize, weights: Buf, delta: Buf, input_delta: Buf) void {
    if (!enabled) unreachable;
    must(dkz.dkz_convolution_data_gradient(ci(batch), ci(groups), ci(channels), ci(height), ci(width), ci(filters), ci(ksize), ci(stride), ci(pad), weights.ptr, delta.ptr, input_delta.ptr), "convolution_data_gradient");
}
