"""Host-side mirror of darknet-zig's GPU op layer (src/gpu.zig) over libdkz.so.

Same names, argument order and meaning as the public functions of gpu.zig, so
code and tests written against the reference read the same here:

* `Buf` is gpu.zig's `Buf` (gpu.zig:117-134): a device pointer plus a length
  in 4-byte elements; `offset(n)` is its pointer arithmetic.
* Sizes are non-negative ints (gpu.zig passes usize and casts with ci(),
  gpu.zig:416-418); scalars are floats; activations are the int codes of
  src/activations.zig:11-27 (see `darknet_zig_amd.activations`).
* Every call goes straight to one C-ABI function. A nonzero status raises
  `GpuError` with the library's context text -- the Python form of gpu.zig's
  must()/panic (gpu.zig:51-55, 444-464).

Host arrays are numpy arrays (float32, or int32 for maxpool indexes).
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib


class GpuError(RuntimeError):
    """A nonzero status from libdkz (a hipError_t value)."""

    def __init__(self, code: int, what: str, context: str):
        self.code = code
        self.context = context
        super().__init__(f"{what}: {_lib.load().dkz_error_string(code).decode()} ({code}) {context}".rstrip())


def _must(code: int, what: str) -> None:
    if code != 0:
        ctx = _lib.load().dkz_last_error_context().decode(errors="replace")
        raise GpuError(code, what, ctx)


@dataclass(frozen=True)
class Buf:
    """A device-side array of 4-byte elements; ptr None means "no buffer"."""

    ptr: int | None = None
    len: int = 0

    def is_null(self) -> bool:
        return self.ptr is None

    def offset(self, n: int) -> "Buf":
        """A view starting n elements in (gpu.zig:128-133)."""
        if self.ptr is None:
            return Buf()
        assert 0 <= n <= self.len
        return Buf(self.ptr + 4 * n, self.len - n)


def _p(b: Buf | None):
    return None if b is None or b.ptr is None else C.c_void_p(b.ptr)


# ---------------------------------------------------------------------------
# device state (gpu.zig:259-356)
# ---------------------------------------------------------------------------


# gpu.zig:32, 39: this mirror always drives libdkz (GPU support compiled
# in); the backend's label as the reference prints it.
enabled = True
backend_label = "HIP"
# gpu.zig:141: -1 means "run on the CPU"; set by init, reset by deinit.
device_index = -1


def active() -> bool:  # gpu.zig:157-159
    return enabled and device_index >= 0


def deviceName() -> str:  # gpu.zig:147-151
    return device_name(device_index) if active() else "CPU"


def deviceMemoryMib() -> int:  # gpu.zig:153-155
    return mem_info()[1] >> 20 if active() else 0


def gemmPolicy() -> str:
    """gpu.zig:104-108: the GEMM a run uses (the library's fp32 matrix-core
    kernel), "cpu" when no device is active."""
    return "dkz-mfma" if active() else "cpu"


def gemmBlockMinTiles() -> int:
    """gpu.zig:111-113: the tile threshold of the reference's blocked GEMM;
    the library picks tiles from the shape alone, with no such gate: 0."""
    return 0


def deinit() -> None:  # gpu.zig:349-356
    global device_index
    device_index = -1


def device_count() -> int:
    n = C.c_int(0)
    _must(_lib.load().dkz_device_count(C.byref(n)), "querying device count")
    return n.value


def init(index: int = 0) -> None:
    global device_index
    _must(_lib.load().dkz_init(index), "initialising the device")
    device_index = index


def device_name(index: int = 0) -> str:
    buf = C.create_string_buffer(256)
    _must(_lib.load().dkz_device_name(index, buf, 256), "querying the device name")
    return buf.value.decode(errors="replace")


def mem_info() -> tuple[int, int]:
    free, total = C.c_size_t(0), C.c_size_t(0)
    _must(_lib.load().dkz_mem_info(C.byref(free), C.byref(total)), "querying memory")
    return free.value, total.value


def setSyncAfterLaunch(on: bool) -> None:  # gpu.zig:181
    _lib.load().dkz_set_sync_after_launch(1 if on else 0)


# ---------------------------------------------------------------------------
# memory (gpu.zig:362-410)
# ---------------------------------------------------------------------------


def alloc(n: int) -> Buf:
    """n zero-filled 4-byte elements; alloc(0) is the null Buf (gpu.zig:362-369)."""
    if n == 0:
        return Buf()
    p = C.c_void_p()
    _must(_lib.load().dkz_malloc(C.byref(p), 4 * n), "device allocation")
    return Buf(p.value, n)


def allocInts(n: int) -> Buf:  # gpu.zig:373
    return alloc(n)


def free(b: Buf) -> None:
    if b.ptr is not None:
        _must(_lib.load().dkz_free(C.c_void_p(b.ptr)), "device free")


def _host(a: np.ndarray) -> np.ndarray:
    if a.dtype not in (np.float32, np.int32) or not a.flags.c_contiguous:
        raise TypeError("host arrays must be C-contiguous float32 or int32")
    return a


def push(b: Buf, host: np.ndarray) -> None:  # gpu.zig:389-393
    host = _host(host)
    if host.size == 0 or b.ptr is None:
        return
    assert host.size <= b.len
    _must(_lib.load().dkz_copy_to_device(C.c_void_p(b.ptr), host.ctypes.data, 4 * host.size), "copy host to device")


def pull(b: Buf, host: np.ndarray) -> None:  # gpu.zig:395-399 (and pullInts, 401-405)
    host = _host(host)
    if host.size == 0 or b.ptr is None:
        return
    assert host.size <= b.len
    _must(_lib.load().dkz_copy_to_host(host.ctypes.data, C.c_void_p(b.ptr), 4 * host.size), "copy device to host")


pullInts = pull


def make(host: np.ndarray) -> Buf:  # gpu.zig:378-382
    b = alloc(host.size)
    push(b, np.ascontiguousarray(host))
    return b


def sync() -> None:  # gpu.zig:407-410
    _must(_lib.load().dkz_synchronize(), "device synchronise")


# ---------------------------------------------------------------------------
# elementwise ops (gpu.zig:483-521)
# ---------------------------------------------------------------------------


def fill(x: Buf, n: int, alpha: float) -> None:
    _must(_lib.load().dkz_fill(_p(x), n, alpha), "fill")


def copy(n: int, x: Buf, y: Buf) -> None:
    _must(_lib.load().dkz_copy(n, _p(x), _p(y)), "copy")


def axpy(n: int, alpha: float, x: Buf, y: Buf) -> None:
    _must(_lib.load().dkz_axpy(n, alpha, _p(x), _p(y)), "axpy")


def scal(n: int, alpha: float, x: Buf) -> None:
    _must(_lib.load().dkz_scal(n, alpha, _p(x)), "scal")


def mul(n: int, x: Buf, y: Buf) -> None:
    _must(_lib.load().dkz_mul(n, _p(x), _p(y)), "mul")


def addScalar(n: int, alpha: float, x: Buf) -> None:  # gpu.zig:503
    _must(_lib.load().dkz_add_scalar(n, alpha, _p(x)), "add_scalar")


def randUniform(n: int, x: Buf, seed: int) -> None:  # gpu.zig:511 (seed: u32)
    _must(_lib.load().dkz_rand_uniform(n, _p(x), seed & 0xFFFFFFFF), "rand_uniform")


def constrainArray(n: int, alpha: float, x: Buf) -> None:
    _must(_lib.load().dkz_constrain(n, alpha, _p(x)), "constrain")


def activateArray(x: Buf, n: int, a: int) -> None:
    _must(_lib.load().dkz_activate_array(_p(x), n, int(a)), "activate_array")


def gradientArray(x: Buf, n: int, a: int, delta: Buf) -> None:
    _must(_lib.load().dkz_gradient_array(_p(x), n, int(a), _p(delta)), "gradient_array")


# ---------------------------------------------------------------------------
# bias / scale (gpu.zig:527-555)
# ---------------------------------------------------------------------------


def addBias(output: Buf, biases: Buf, batch: int, filters: int, spatial: int) -> None:
    _must(_lib.load().dkz_add_bias(_p(output), _p(biases), batch, filters, spatial), "add_bias")


def scaleBias(output: Buf, scales: Buf, batch: int, filters: int, spatial: int) -> None:
    _must(_lib.load().dkz_scale_bias(_p(output), _p(scales), batch, filters, spatial), "scale_bias")


def backwardBias(bias_updates: Buf, delta: Buf, batch: int, filters: int, spatial: int) -> None:
    _must(_lib.load().dkz_backward_bias(_p(bias_updates), _p(delta), batch, filters, spatial), "backward_bias")


def backwardScale(x_norm: Buf, delta: Buf, batch: int, filters: int, spatial: int, scale_updates: Buf) -> None:
    _must(
        _lib.load().dkz_backward_scale(_p(x_norm), _p(delta), batch, filters, spatial, _p(scale_updates)),
        "backward_scale",
    )


# ---------------------------------------------------------------------------
# batch normalisation (gpu.zig:561-608)
# ---------------------------------------------------------------------------


def mean(x: Buf, batch: int, filters: int, spatial: int, out: Buf) -> None:
    _must(_lib.load().dkz_mean(_p(x), batch, filters, spatial, _p(out)), "mean")


def variance(x: Buf, mean_in: Buf, batch: int, filters: int, spatial: int, out: Buf) -> None:
    _must(_lib.load().dkz_variance(_p(x), _p(mean_in), batch, filters, spatial, _p(out)), "variance")


def normalize(x: Buf, mean_in: Buf, variance_in: Buf, batch: int, filters: int, spatial: int) -> None:
    _must(_lib.load().dkz_normalize(_p(x), _p(mean_in), _p(variance_in), batch, filters, spatial), "normalize")


def meanDelta(delta: Buf, variance_in: Buf, batch: int, filters: int, spatial: int, out: Buf) -> None:
    _must(_lib.load().dkz_mean_delta(_p(delta), _p(variance_in), batch, filters, spatial, _p(out)), "mean_delta")


def varianceDelta(
    x: Buf, delta: Buf, mean_in: Buf, variance_in: Buf, batch: int, filters: int, spatial: int, out: Buf
) -> None:
    _must(
        _lib.load().dkz_variance_delta(
            _p(x), _p(delta), _p(mean_in), _p(variance_in), batch, filters, spatial, _p(out)
        ),
        "variance_delta",
    )


def normalizeDelta(
    x: Buf,
    mean_in: Buf,
    variance_in: Buf,
    mean_delta_in: Buf,
    variance_delta_in: Buf,
    batch: int,
    filters: int,
    spatial: int,
    delta: Buf,
) -> None:
    _must(
        _lib.load().dkz_normalize_delta(
            _p(x), _p(mean_in), _p(variance_in), _p(mean_delta_in), _p(variance_delta_in), batch, filters, spatial,
            _p(delta),
        ),
        "normalize_delta",
    )


# ---------------------------------------------------------------------------
# softmax and losses (gpu.zig:614-645)
# ---------------------------------------------------------------------------


def softmax(
    input: Buf,
    n: int,
    batch: int,
    batch_offset: int,
    groups: int,
    group_offset: int,
    stride: int,
    temp: float,
    output: Buf,
) -> None:
    _must(
        _lib.load().dkz_softmax(_p(input), n, batch, batch_offset, groups, group_offset, stride, temp, _p(output)),
        "softmax",
    )


def softmaxLayerForward(
    batch: int, inputs: int, groups: int, temp: float, input: Buf, truth: Buf | None, output: Buf,
    delta: Buf | None, loss: Buf | None,
) -> None:
    """layers/misc.zig:63-76 (softmax, then the cross-entropy when truth is
    given) as one call; no single gpu.zig counterpart."""
    _must(_lib.load().dkz_softmax_layer_forward(batch, inputs, groups, temp, _p(input), _p(truth), _p(output),
                                                _p(delta), _p(loss)), "softmax_layer_forward")


def softmaxCrossEntropy(n: int, pred: Buf, truth: Buf, delta: Buf, err: Buf) -> None:
    _must(_lib.load().dkz_softmax_cross_entropy(n, _p(pred), _p(truth), _p(delta), _p(err)), "softmax_x_ent")


def l2(n: int, pred: Buf, truth: Buf, delta: Buf, err: Buf) -> None:
    _must(_lib.load().dkz_l2(n, _p(pred), _p(truth), _p(delta), _p(err)), "l2")


def l1(n: int, pred: Buf, truth: Buf, delta: Buf, err: Buf) -> None:
    _must(_lib.load().dkz_l1(n, _p(pred), _p(truth), _p(delta), _p(err)), "l1")


def smoothL1(n: int, pred: Buf, truth: Buf, delta: Buf, err: Buf) -> None:
    _must(_lib.load().dkz_smooth_l1(n, _p(pred), _p(truth), _p(delta), _p(err)), "smooth_l1")


# ---------------------------------------------------------------------------
# pooling and shortcut (gpu.zig:725-800)
# ---------------------------------------------------------------------------


def forwardMaxpool(
    out_n: int, in_h: int, in_w: int, in_c: int, stride: int, size: int, pad: int, input: Buf, output: Buf,
    indexes: Buf,
) -> None:
    _must(
        _lib.load().dkz_forward_maxpool(
            out_n, in_h, in_w, in_c, stride, size, pad, _p(input), _p(output), _p(indexes)
        ),
        "forward_maxpool",
    )


def backwardMaxpool(
    in_n: int, in_h: int, in_w: int, in_c: int, stride: int, size: int, pad: int, delta: Buf, prev_delta: Buf,
    indexes: Buf,
) -> None:
    _must(
        _lib.load().dkz_backward_maxpool(
            in_n, in_h, in_w, in_c, stride, size, pad, _p(delta), _p(prev_delta), _p(indexes)
        ),
        "backward_maxpool",
    )


def forwardAvgpool(n: int, w: int, h: int, c: int, input: Buf, output: Buf) -> None:
    _must(_lib.load().dkz_forward_avgpool(n, w, h, c, _p(input), _p(output)), "forward_avgpool")


def backwardAvgpool(n: int, w: int, h: int, c: int, in_delta: Buf, out_delta: Buf) -> None:
    _must(_lib.load().dkz_backward_avgpool(n, w, h, c, _p(in_delta), _p(out_delta)), "backward_avgpool")


def shortcut(
    batch: int, w1: int, h1: int, c1: int, add: Buf, w2: int, h2: int, c2: int, s1: float, s2: float, out: Buf
) -> None:
    _must(_lib.load().dkz_shortcut(batch, w1, h1, c1, _p(add), w2, h2, c2, s1, s2, _p(out)), "shortcut")


# ---------------------------------------------------------------------------
# convolution helpers (gpu.zig:651-669)
# ---------------------------------------------------------------------------


def im2col(im: Buf, channels: int, height: int, width: int, ksize: int, stride: int, pad: int, col: Buf) -> None:
    _must(_lib.load().dkz_im2col(_p(im), channels, height, width, ksize, stride, pad, _p(col)), "im2col")


def col2im(col: Buf, channels: int, height: int, width: int, ksize: int, stride: int, pad: int, im: Buf) -> None:
    _must(_lib.load().dkz_col2im(_p(col), channels, height, width, ksize, stride, pad, _p(im)), "col2im")


def gemm(
    ta: bool, tb: bool, m: int, n: int, k: int, alpha: float, a: Buf, lda: int, b: Buf, ldb: int, beta: float,
    c: Buf, ldc: int,
) -> None:  # gpu.zig:671-719
    _must(_lib.load().dkz_gemm(1 if ta else 0, 1 if tb else 0, m, n, k, alpha, _p(a), lda, _p(b), ldb, beta, _p(c),
                               ldc), "gemm")


def convolutionForward(
    batch: int, groups: int, channels: int, height: int, width: int, filters: int, ksize: int, stride: int,
    pad: int, weights: Buf, input: Buf, output: Buf,
) -> None:  # the per-image loop of layers/convolutional.zig:240-260 in one call
    _must(_lib.load().dkz_convolution_forward(batch, groups, channels, height, width, filters, ksize, stride, pad,
                                              _p(weights), _p(input), _p(output)), "convolution_forward")


def convolutionWeightGradient(
    batch: int, groups: int, channels: int, height: int, width: int, filters: int, ksize: int, stride: int,
    pad: int, delta: Buf, input: Buf, weight_updates: Buf,
) -> None:  # the weight-gradient gemms of layers/convolutional.zig:288-297 in one call
    _must(_lib.load().dkz_convolution_weight_gradient(batch, groups, channels, height, width, filters, ksize, stride,
                                                      pad, _p(delta), _p(input), _p(weight_updates)),
          "convolution_weight_gradient")


def convolutionDataGradient(
    batch: int, groups: int, channels: int, height: int, width: int, filters: int, ksize: int, stride: int,
    pad: int, weights: Buf, delta: Buf, input_delta: Buf,
) -> None:  # the data-gradient gemms and col2im of layers/convolutional.zig:299-305 in one call
    _must(_lib.load().dkz_convolution_data_gradient(batch, groups, channels, height, width, filters, ksize, stride,
                                                    pad, _p(weights), _p(delta), _p(input_delta)),
          "convolution_data_gradient")


def dropout(input: Buf, size: int, rand_buf: Buf, prob: float, scale: float) -> None:  # gpu.zig:769
    _must(_lib.load().dkz_dropout(_p(input), size, _p(rand_buf), prob, scale), "dropout")


def adamUpdate(
    w: Buf, d: Buf, m: Buf, v: Buf, b1: float, b2: float, eps: float, decay: float, rate: float, n: int,
    batch: int, t: int,
) -> None:  # gpu.zig:804-830
    _must(_lib.load().dkz_adam_update(_p(w), _p(d), _p(m), _p(v), b1, b2, eps, decay, rate, n, batch, t),
          "adam_update")


# ---- fused batch-norm layer passes (no single gpu.zig counterpart: each
# replaces the call sequence of layers/batchnorm.zig forwardGpu / backwardGpu
# together with the activation calls of convolutional.zig:269 and :280) ----


def batchnormForward(
    batch: int,
    filters: int,
    spatial: int,
    activation: int,
    train: bool,
    input: Buf,
    output: Buf,
    x: Buf,
    x_norm: Buf | None,
    mean: Buf | None,
    variance: Buf | None,
    rolling_mean: Buf,
    rolling_variance: Buf,
    scales: Buf,
    biases: Buf,
) -> None:
    _must(
        _lib.load().dkz_batchnorm_forward(
            batch, filters, spatial, int(activation), 1 if train else 0, _p(input), _p(output), _p(x),
            _p(x_norm), _p(mean), _p(variance), _p(rolling_mean), _p(rolling_variance), _p(scales), _p(biases),
        ),
        "batchnorm_forward",
    )


def batchnormBackward(
    batch: int,
    filters: int,
    spatial: int,
    activation: int,
    output: Buf | None,
    delta: Buf,
    x: Buf,
    x_norm: Buf,
    mean: Buf,
    variance: Buf,
    scales: Buf,
    bias_updates: Buf,
    scale_updates: Buf,
    mean_delta: Buf,
    variance_delta: Buf,
) -> None:
    _must(
        _lib.load().dkz_batchnorm_backward(
            batch, filters, spatial, int(activation), _p(output), _p(delta), _p(x), _p(x_norm), _p(mean),
            _p(variance), _p(scales), _p(bias_updates), _p(scale_updates), _p(mean_delta), _p(variance_delta),
        ),
        "batchnorm_backward",
    )
