"""numpy-facing wrapper of libdkz_oracle.so (oracle/dkz_oracle.c).

TEST INFRASTRUCTURE ONLY: the CPU twins used as the parity checker and as the
CPU baseline. Every function mirrors one in blas.zig / activations.zig /
layers/pooling.zig (see the C source for the citations). In-place functions
modify their numpy argument, exactly as the Zig twins modify their slice.
"""

from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "libdkz_oracle.so"

_f = C.c_float
_sz = C.c_size_t
_i = C.c_int
_P = C.c_void_p

_SIGS = {
    "ref_fill": (None, [_P, _sz, _f]),
    "ref_copy": (None, [_P, _P, _sz]),
    "ref_axpy": (None, [_f, _P, _P, _sz]),
    "ref_scal": (None, [_f, _P, _sz]),
    "ref_mul": (None, [_P, _P, _sz]),
    "ref_constrain_array": (None, [_f, _P, _sz]),
    "ref_add_bias": (None, [_P, _P, _sz, _sz, _sz]),
    "ref_scale_bias": (None, [_P, _P, _sz, _sz, _sz]),
    "ref_backward_bias": (None, [_P, _P, _sz, _sz, _sz]),
    "ref_backward_scale": (None, [_P, _P, _sz, _sz, _sz, _P]),
    "ref_mean": (None, [_P, _sz, _sz, _sz, _P]),
    "ref_variance": (None, [_P, _P, _sz, _sz, _sz, _P]),
    "ref_normalize": (None, [_P, _P, _P, _sz, _sz, _sz]),
    "ref_mean_delta": (None, [_P, _P, _sz, _sz, _sz, _P]),
    "ref_variance_delta": (None, [_P, _P, _P, _P, _sz, _sz, _sz, _P]),
    "ref_normalize_delta": (None, [_P, _P, _P, _P, _P, _sz, _sz, _sz, _P]),
    "ref_softmax_one": (None, [_P, _sz, _f, _sz, _P]),
    "ref_softmax": (None, [_P, _sz, _sz, _sz, _sz, _sz, _sz, _f, _P]),
    "ref_softmax_cross_entropy": (None, [_P, _P, _P, _P, _sz]),
    "ref_l2": (None, [_P, _P, _P, _P, _sz]),
    "ref_l1": (None, [_P, _P, _P, _P, _sz]),
    "ref_smooth_l1": (None, [_P, _P, _P, _P, _sz]),
    "ref_shortcut": (None, [_sz, _sz, _sz, _sz, _P, _sz, _sz, _sz, _f, _f, _P]),
    "ref_activate": (_f, [_f, _i]),
    "ref_gradient": (_f, [_f, _i]),
    "ref_activate_array": (None, [_P, _sz, _i]),
    "ref_gradient_array": (None, [_P, _sz, _i, _P]),
    "ref_maxpool_out_dim": (_sz, [_sz, _sz, _sz, _sz]),
    "ref_forward_maxpool": (None, [_sz, _sz, _sz, _sz, _sz, _sz, _sz, _P, _P, _P]),
    "ref_backward_maxpool": (None, [_sz, _P, _P, _P]),
    "ref_forward_avgpool": (None, [_sz, _sz, _sz, _sz, _P, _P]),
    "ref_backward_avgpool": (None, [_sz, _sz, _sz, _sz, _P, _P]),
    "ref_add_scalar": (None, [_f, _P, _sz]),
    "ref_hash_u32": (C.c_uint32, [C.c_uint32]),
    "ref_rand_uniform": (None, [_P, _sz, C.c_uint32]),
    "ref_rand_uniform_from": (None, [_P, _sz, C.c_uint32, _sz]),
    "ref_dropout": (None, [_P, _sz, _P, _f, _f]),
    "ref_adam_update": (None, [_P, _P, _P, _P, _f, _f, _f, _f, _f, _sz, _sz, _sz]),
    "ref_conv_out_dim": (_sz, [_sz, _sz, _sz, _sz]),
    "ref_im2col": (None, [_P, _sz, _sz, _sz, _sz, _sz, _sz, _P]),
    "ref_col2im": (None, [_P, _sz, _sz, _sz, _sz, _sz, _sz, _P]),
    "ref_gemm": (None, [_i, _i, _sz, _sz, _sz, _f, _P, _sz, _P, _sz, _f, _P, _sz]),
    "ref_pow_f32": (_f, [_f, _f]),
    "ref_expf": (_f, [_f]),
}

_LIB = None


def build() -> Path:
    """Compiles the oracle with its Makefile (always rebuilds)."""
    subprocess.run(["make", "-s", "-B", "-C", str(ORACLE_DIR)], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            build()
        lib_ = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(lib_, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = lib_
    return _LIB


def _ptr(a: np.ndarray) -> int:
    assert a.flags.c_contiguous and a.dtype in (np.float32, np.int32), a.dtype
    return a.ctypes.data


# ---- blas.zig:13-46 --------------------------------------------------------


def fill(x: np.ndarray, alpha: float) -> None:
    lib().ref_fill(_ptr(x), x.size, alpha)


def copy(src: np.ndarray, dst: np.ndarray) -> None:
    lib().ref_copy(_ptr(src), _ptr(dst), src.size)


def axpy(alpha: float, x: np.ndarray, y: np.ndarray) -> None:
    lib().ref_axpy(alpha, _ptr(x), _ptr(y), x.size)


def scal(alpha: float, x: np.ndarray) -> None:
    lib().ref_scal(alpha, _ptr(x), x.size)


def mul(x: np.ndarray, y: np.ndarray) -> None:
    lib().ref_mul(_ptr(x), _ptr(y), x.size)


def constrainArray(alpha: float, x: np.ndarray) -> None:
    lib().ref_constrain_array(alpha, _ptr(x), x.size)


# ---- blas.zig:53-204 -------------------------------------------------------


def addBias(output, biases, batch, filters, spatial) -> None:
    lib().ref_add_bias(_ptr(output), _ptr(biases), batch, filters, spatial)


def scaleBias(output, scales, batch, filters, spatial) -> None:
    lib().ref_scale_bias(_ptr(output), _ptr(scales), batch, filters, spatial)


def backwardBias(bias_updates, delta, batch, filters, spatial) -> None:
    lib().ref_backward_bias(_ptr(bias_updates), _ptr(delta), batch, filters, spatial)


def backwardScale(x_norm, delta, batch, filters, spatial, scale_updates) -> None:
    lib().ref_backward_scale(_ptr(x_norm), _ptr(delta), batch, filters, spatial, _ptr(scale_updates))


def mean(x, batch, filters, spatial, out) -> None:
    lib().ref_mean(_ptr(x), batch, filters, spatial, _ptr(out))


def variance(x, mean_in, batch, filters, spatial, out) -> None:
    lib().ref_variance(_ptr(x), _ptr(mean_in), batch, filters, spatial, _ptr(out))


def normalize(x, mean_in, variance_in, batch, filters, spatial) -> None:
    lib().ref_normalize(_ptr(x), _ptr(mean_in), _ptr(variance_in), batch, filters, spatial)


def meanDelta(delta, variance_in, batch, filters, spatial, out) -> None:
    lib().ref_mean_delta(_ptr(delta), _ptr(variance_in), batch, filters, spatial, _ptr(out))


def varianceDelta(x, delta, mean_in, variance_in, batch, filters, spatial, out) -> None:
    lib().ref_variance_delta(_ptr(x), _ptr(delta), _ptr(mean_in), _ptr(variance_in), batch, filters, spatial,
                             _ptr(out))


def normalizeDelta(x, mean_in, variance_in, mean_delta, variance_delta, batch, filters, spatial, delta) -> None:
    lib().ref_normalize_delta(_ptr(x), _ptr(mean_in), _ptr(variance_in), _ptr(mean_delta), _ptr(variance_delta),
                              batch, filters, spatial, _ptr(delta))


# ---- blas.zig:213-322 ------------------------------------------------------


def softmax(input, n, batch, batch_offset, groups, group_offset, stride, temp, output) -> None:
    lib().ref_softmax(_ptr(input), n, batch, batch_offset, groups, group_offset, stride, temp, _ptr(output))


def softmaxCrossEntropy(pred, truth, delta, err) -> None:
    lib().ref_softmax_cross_entropy(_ptr(pred), _ptr(truth), _ptr(delta), _ptr(err), pred.size)


def l2(pred, truth, delta, err) -> None:
    lib().ref_l2(_ptr(pred), _ptr(truth), _ptr(delta), _ptr(err), pred.size)


def l1(pred, truth, delta, err) -> None:
    lib().ref_l1(_ptr(pred), _ptr(truth), _ptr(delta), _ptr(err), pred.size)


def smoothL1(pred, truth, delta, err) -> None:
    lib().ref_smooth_l1(_ptr(pred), _ptr(truth), _ptr(delta), _ptr(err), pred.size)


def shortcut(batch, w1, h1, c1, add, w2, h2, c2, s1, s2, out) -> None:
    lib().ref_shortcut(batch, w1, h1, c1, _ptr(add), w2, h2, c2, s1, s2, _ptr(out))


# ---- activations.zig ---------------------------------------------------------


def activate(x: float, a: int) -> float:
    return lib().ref_activate(x, int(a))


def gradient(y: float, a: int) -> float:
    return lib().ref_gradient(y, int(a))


def activateArray(x: np.ndarray, a: int) -> None:
    lib().ref_activate_array(_ptr(x), x.size, int(a))


def gradientArray(y: np.ndarray, a: int, delta: np.ndarray) -> None:
    lib().ref_gradient_array(_ptr(y), y.size, int(a), _ptr(delta))


# ---- layers/pooling.zig -----------------------------------------------------


def maxpool_out_dim(in_dim, size, stride, pad) -> int:
    return lib().ref_maxpool_out_dim(in_dim, size, stride, pad)


def forwardMaxpool(batch, h, w, c, size, stride, pad, input, output, indexes) -> None:
    lib().ref_forward_maxpool(batch, h, w, c, size, stride, pad, _ptr(input), _ptr(output), _ptr(indexes))


def backwardMaxpool(indexes, delta, prev_delta) -> None:
    lib().ref_backward_maxpool(indexes.size, _ptr(indexes), _ptr(delta), _ptr(prev_delta))


def forwardAvgpool(batch, w, h, c, input, output) -> None:
    lib().ref_forward_avgpool(batch, w, h, c, _ptr(input), _ptr(output))


def backwardAvgpool(batch, w, h, c, out_delta, in_delta) -> None:
    lib().ref_backward_avgpool(batch, w, h, c, _ptr(out_delta), _ptr(in_delta))


# ---- the rest of gpu.zig's surface (kernel-defined ops, misc.zig dropout) ----


def addScalar(alpha: float, x: np.ndarray) -> None:
    lib().ref_add_scalar(alpha, _ptr(x), x.size)


def hash_u32(x: int) -> int:
    return lib().ref_hash_u32(x & 0xFFFFFFFF)


def randUniform(x: np.ndarray, seed: int, first: int = 0) -> None:
    """x = elements first .. first + x.size - 1 of the seed's sequence."""
    if first == 0:
        lib().ref_rand_uniform(_ptr(x), x.size, seed & 0xFFFFFFFF)
    else:
        lib().ref_rand_uniform_from(_ptr(x), x.size, seed & 0xFFFFFFFF, first)


def dropout(x: np.ndarray, rand: np.ndarray, prob: float, scale: float) -> None:
    lib().ref_dropout(_ptr(x), x.size, _ptr(rand), prob, scale)


def adamUpdate(w, d, m, v, b1, b2, eps, decay, rate, n, batch, t) -> None:
    lib().ref_adam_update(_ptr(w), _ptr(d), _ptr(m), _ptr(v), b1, b2, eps, decay, rate, n, batch, t)


# ---- im2col.zig ---------------------------------------------------------------


def conv_out_dim(size, ksize, stride, pad) -> int:
    return lib().ref_conv_out_dim(size, ksize, stride, pad)


def im2col(im, channels, height, width, ksize, stride, pad, col) -> None:
    lib().ref_im2col(_ptr(im), channels, height, width, ksize, stride, pad, _ptr(col))


def col2im(col, channels, height, width, ksize, stride, pad, im) -> None:
    lib().ref_col2im(_ptr(col), channels, height, width, ksize, stride, pad, _ptr(im))


# ---- gemm.zig ------------------------------------------------------------------


def gemm(ta, tb, m, n, k, alpha, a, lda, b, ldb, beta, c, ldc) -> None:
    lib().ref_gemm(int(bool(ta)), int(bool(tb)), m, n, k, alpha, _ptr(a), lda, _ptr(b), ldb, beta, _ptr(c), ldc)


def pow_f32(x: float, y: float) -> float:
    return lib().ref_pow_f32(x, y)


def expf(x: float) -> float:
    return lib().ref_expf(x)


# ---- layers/batchnorm.zig: the layer sequences over the twins above ---------

ROLLING_MOMENTUM = np.float32(0.99)  # batchnorm.zig:16, an f32 constant
EMA_ALPHA = np.float32(1) - ROLLING_MOMENTUM  # batchnorm.zig:87: 1 - rolling_momentum, in f32


def batchnormForward(batch, filters, spatial, activation, train, input, output, x, x_norm, mean_out, variance_out,
                     rolling_mean, rolling_variance, scales, biases) -> None:
    """layers/batchnorm.zig:74-99 (forward, CPU), then the activation the
    convolutional layer applies to its output (convolutional.zig:173).
    input is copied to output first unless it is the same array (the
    standalone batchnorm layer, batchnorm.zig:78)."""
    n = batch * filters * spatial
    if input is not output:
        copy(input[:n], output[:n])
    copy(output[:n], x[:n])
    if train:
        mean(output[:n], batch, filters, spatial, mean_out)
        variance(output[:n], mean_out, batch, filters, spatial, variance_out)
        scal(ROLLING_MOMENTUM, rolling_mean)
        axpy(EMA_ALPHA, mean_out, rolling_mean)
        scal(ROLLING_MOMENTUM, rolling_variance)
        axpy(EMA_ALPHA, variance_out, rolling_variance)
        normalize(output[:n], mean_out, variance_out, batch, filters, spatial)
        copy(output[:n], x_norm[:n])
    else:
        normalize(output[:n], rolling_mean, rolling_variance, batch, filters, spatial)
    scaleBias(output[:n], scales, batch, filters, spatial)
    addBias(output[:n], biases, batch, filters, spatial)
    activateArray(output[:n], activation)


def batchnormBackward(batch, filters, spatial, activation, output, delta, x, x_norm, mean_in, variance_in, scales,
                      bias_updates, scale_updates, mean_delta_out, variance_delta_out) -> None:
    """The activation gradient of convolutional.zig:184, then
    layers/batchnorm.zig:101-123 (backward, CPU). mean_in / variance_in are
    the statistics the forward normalised with (batchnorm.zig:108-109)."""
    n = batch * filters * spatial
    gradientArray(output[:n], activation, delta[:n])
    backwardBias(bias_updates, delta[:n], batch, filters, spatial)
    backwardScale(x_norm[:n], delta[:n], batch, filters, spatial, scale_updates)
    scaleBias(delta[:n], scales, batch, filters, spatial)
    meanDelta(delta[:n], variance_in, batch, filters, spatial, mean_delta_out)
    varianceDelta(x[:n], delta[:n], mean_in, variance_in, batch, filters, spatial, variance_delta_out)
    normalizeDelta(x[:n], mean_in, variance_in, mean_delta_out, variance_delta_out, batch, filters, spatial, delta[:n])
