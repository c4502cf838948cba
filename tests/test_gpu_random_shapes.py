"""A seeded sweep of random shapes through the GPU path, against the oracle,
at each op family's parity bar: the per-channel ops and the fused batch-norm
passes over random (batch, filters, spatial) -- every residue of spatial mod
4, filters on both sides of the one-launch/split thresholds, ragged last
chunks --, elementwise ops over random lengths and misaligned views, the
convolution lowering over random geometries, the GEMM over random shapes,
transposes and leading dimensions, the whole-batch convolution forward,
weight gradient and data gradient over random layers (groups, ksize, stride,
pad), and max pooling over random windows, strides, pads and plane counts. The shapes are drawn once from a fixed seed, so a failure names a
reproducible case."""

from __future__ import annotations

import numpy as np
import pytest

from darknet_zig_amd import gpu
from darknet_zig_amd.activations import Activation
from oracle import ref
from tests.helpers import assert_bitexact, assert_r5, chan_f32, chan_sum64, down, normal, rng, uniform, up
from tests.test_gpu_batchnorm_fused import _backward_case, _forward_case
from tests.test_gpu_convolution import _dgrad_reference as dgrad_reference
from tests.test_gpu_convolution import _reference as conv_reference
from tests.test_gpu_convolution import _wgrad_reference as wgrad_reference
from tests.test_gpu_gemm import check as gemm_check

pytestmark = pytest.mark.gpu

_R = np.random.default_rng(20240921)
CHANNEL_SHAPES = sorted({(int(_R.integers(1, 10)), int(_R.choice([1, 3, 17, 64, 127, 128, 129, 255, 256, 300])),
                          int(_R.integers(1, 700))) for _ in range(24)})
EW_SIZES = sorted({int(v) for v in _R.integers(1, 300000, 12)})
CONV = sorted({(int(_R.integers(1, 9)), int(_R.integers(3, 24)), int(_R.integers(3, 24)), int(_R.integers(1, 4)),
                int(_R.integers(1, 3)), int(_R.integers(0, 3))) for _ in range(12)})
GEMM = sorted({(bool(_R.integers(0, 2)), bool(_R.integers(0, 2)), int(_R.integers(1, 300)), int(_R.integers(1, 300)),
                int(_R.integers(0, 700))) for _ in range(16)})


def _layer():
    """batch, groups, channels, height, width, filters, ksize, stride, pad with
    the window inside the padded image."""
    while True:
        batch, groups, k = int(_R.integers(1, 7)), int(_R.integers(1, 4)), int(_R.choice([1, 1, 2, 3, 3, 5]))
        h, w, stride, pad = int(_R.integers(3, 21)), int(_R.integers(3, 21)), int(_R.integers(1, 4)), int(_R.integers(0, 4))
        if h + 2 * pad >= k and w + 2 * pad >= k:
            return (batch, groups, groups * int(_R.integers(1, 10)), h, w, groups * int(_R.integers(1, 41)), k, stride,
                    pad)


LAYERS = sorted({_layer() for _ in range(14)})


def _large_bn():
    """[batch, filters, spatial] of 3 to 26 M elements: the one-launch
    register-holding paths and, past what the GPU holds at once, the two
    passes."""
    f = int(_R.choice([1, 3, 17, 64, 128, 255]))
    s = 4 * int(_R.integers(256, 4096)) + int(_R.choice([0, 0, 0, 2]))
    b = max(1, int(_R.integers(3_000_000, 26_000_000)) // (f * s))
    return b, f, s


LARGE_BN = sorted({_large_bn() for _ in range(5)})

_P = np.random.default_rng(20261202)


def _pool():
    """batch, channels, height, width, size, stride, pad with the window
    inside the padded input; planes below 256 (per-output and per-input
    kernels), from 256 (planes in LDS, a plane a workgroup) and from 1024
    (several planes a workgroup), under about 2 M inputs."""
    while True:
        size, stride = int(_P.choice([1, 2, 2, 3, 3, 4, 5, 6, 7, 9, 13])), int(_P.choice([1, 1, 1, 2, 3]))
        h, w, pad = int(_P.integers(1, 41)), int(_P.integers(1, 41)), int(_P.integers(0, size + 3))
        if h + pad < size or w + pad < size:
            continue
        planes = int(_P.choice([int(_P.integers(1, 256)), int(_P.integers(256, 1024)), int(_P.integers(1024, 5000))]))
        if planes * h * w > 2_000_000:
            continue
        c = int(_P.choice([1, 3, 7, 16]))
        return max(1, planes // c), c, h, w, size, stride, pad


POOLS = sorted({_pool() for _ in range(28)})


@pytest.mark.parametrize("shape", CHANNEL_SHAPES, ids=str)
def test_channel_ops(dev, shape):
    B, F, S = shape
    n = B * F * S
    r = rng(B * 100003 + F * 1009 + S)
    x, delta, x_norm = normal(r, n, 0.2, 1.0), normal(r, n), normal(r, n)
    bias, scales = normal(r, F, 0, 0.1), uniform(r, F, 0.5, 1.5)
    m, v = np.empty(F, np.float32), np.empty(F, np.float32)
    ref.mean(x, B, F, S, m)
    ref.variance(x, m, B, F, S, v)
    x64, d64 = (a.astype(np.float64).reshape(B, F, S) for a in (x, delta))
    dx, dd, dxn, dm, dv, dbias, dscales = up(x), up(delta), up(x_norm), up(m), up(v), up(bias), up(scales)
    out = gpu.alloc(F)

    gpu.mean(dx, B, F, S, out)
    assert_r5(down(out, m), m, x64.sum(axis=(0, 2)) * np.float64(np.float32(1) / np.float32(B * S)), "mean")
    if B * S > 1:
        gpu.variance(dx, dm, B, F, S, out)
        diff = x - chan_f32(m, shape)
        dev64 = chan_sum64(diff * diff, shape)
        assert_r5(down(out, v), v, dev64 * np.float64(np.float32(1) / np.float32(B * S - 1)), "variance")
    upd0 = normal(r, F)
    cpu = upd0.copy()
    ref.backwardScale(x_norm, delta, B, F, S, cpu)
    du = up(upd0)
    gpu.backwardScale(dxn, dd, B, F, S, du)
    assert_r5(down(du, upd0), cpu, upd0 + chan_sum64(delta * x_norm, shape), "backward_scale")
    cpu = upd0.copy()
    ref.backwardBias(cpu, delta, B, F, S)
    gpu.push(du, upd0)
    gpu.backwardBias(du, dd, B, F, S)
    got = down(du, upd0)
    assert_r5(got, cpu, upd0 + d64.sum(axis=(0, 2)), "backward_bias" + (" (spatial 1)" if S == 1 else ""))
    md, vd = np.empty(F, np.float32), np.empty(F, np.float32)
    ref.meanDelta(delta, v, B, F, S, md)
    ref.varianceDelta(x, delta, m, v, B, F, S, vd)
    gpu.meanDelta(dd, dv, B, F, S, out)
    fac = (np.float32(-1.0) / np.sqrt(v + np.float32(1e-5))).astype(np.float64)
    assert_r5(down(out, md), md, d64.sum(axis=(0, 2)) * fac, "mean_delta")
    gpu.varianceDelta(dx, dd, dm, dv, B, F, S, out)
    vd64 = chan_sum64(delta * (x - chan_f32(m, shape)), shape) * -0.5 * \
        (v + np.float32(1e-5)).astype(np.float64) ** -1.5
    assert_r5(down(out, vd), vd, vd64, "variance_delta")

    # broadcasts, fed the twin's per-channel vectors: bit-exact
    for name, fn, cpu_fn in (
        ("add_bias", lambda b: gpu.addBias(b, dbias, B, F, S), lambda a: ref.addBias(a, bias, B, F, S)),
        ("scale_bias", lambda b: gpu.scaleBias(b, dscales, B, F, S), lambda a: ref.scaleBias(a, scales, B, F, S)),
        ("normalize", lambda b: gpu.normalize(b, dm, dv, B, F, S), lambda a: ref.normalize(a, m, v, B, F, S)),
    ):
        want = x.copy()
        cpu_fn(want)
        db = up(x)
        fn(db)
        assert_bitexact(down(db, x), want, name)
        gpu.free(db)
    want = delta.copy()
    ref.normalizeDelta(x, m, v, md, vd, B, F, S, want)
    dmd, dvd = up(md), up(vd)
    gpu.normalizeDelta(dx, dm, dv, dmd, dvd, B, F, S, dd)
    assert_bitexact(down(dd, delta), want, "normalize_delta")
    for b in (dx, dd, dxn, dm, dv, dbias, dscales, out, du, dmd, dvd):
        gpu.free(b)


@pytest.mark.parametrize("shape", CHANNEL_SHAPES, ids=str)
def test_fused_batchnorm(dev, shape):
    B, F, S = shape
    act = list(Activation)[(B + F + S) % len(Activation)]
    m, v = _forward_case(shape, act, True, (B + S) % 2 == 0, seed=B * 7 + F * 3 + S)
    _backward_case(shape, act, seed=B * 11 + F + S * 5)


@pytest.mark.parametrize("shape", LARGE_BN, ids=str)
def test_fused_batchnorm_large(dev, shape):
    B, F, S = shape
    act = list(Activation)[(B + F + S) % len(Activation)]
    _forward_case(shape, act, True, True, seed=B + F * 5 + S)
    _backward_case(shape, act, seed=B * 3 + F + S)


@pytest.mark.parametrize("n", EW_SIZES)
def test_elementwise(dev, n):
    r = rng(n)
    off = n % 4
    a, b = uniform(r, n, -3, 3), uniform(r, n, -3, 3)
    whole_a = up(np.concatenate([np.zeros(off, np.float32), a]))
    whole_b = up(np.concatenate([np.zeros(off, np.float32), b]))
    va, vb = whole_a.offset(off), whole_b.offset(off)
    act = list(Activation)[n % len(Activation)]
    cpu_y = a.copy()
    ref.activateArray(cpu_y, act)
    cpu_d = b.copy()
    ref.gradientArray(cpu_y, act, cpu_d)
    gpu.activateArray(va, n, act)
    gpu.gradientArray(va, n, act, vb)
    got = np.empty(n + off, np.float32)
    gpu.pull(whole_a, got)
    assert_bitexact(got[off:], cpu_y, f"activate {act.name}")
    gpu.pull(whole_b, got)
    assert_bitexact(got[off:], cpu_d, f"gradient {act.name}")
    cpu = cpu_d.copy()
    ref.axpy(-0.75, cpu_y, cpu)
    gpu.axpy(n, -0.75, va, vb)
    gpu.pull(whole_b, got)
    assert_bitexact(got[off:], cpu, "axpy")
    gpu.free(whole_a)
    gpu.free(whole_b)


@pytest.mark.parametrize("case", POOLS, ids=str)
def test_maxpool(dev, case):
    """Max pooling over random geometries, bit-exact: inputs drawn from 16
    levels (ties everywhere: the first maximum must win) with a NaN and a
    -inf, and deltas over six decades so that adding an input's deltas in
    another order changes the rounded result."""
    batch, c, h, w, size, stride, pad = case
    oh, ow = ref.maxpool_out_dim(h, size, stride, pad), ref.maxpool_out_dim(w, size, stride, pad)
    r = rng(sum(case))
    x = (np.floor(uniform(r, batch * c * h * w, 0, 16)) - 8).astype(np.float32)
    x[min(5, x.size - 1)] = np.nan
    x[min(11, x.size - 1)] = -np.inf
    out_n = batch * c * oh * ow
    out_c, idx_c = np.empty(out_n, np.float32), np.empty(out_n, np.int32)
    ref.forwardMaxpool(batch, h, w, c, size, stride, pad, x, out_c, idx_c)
    dx, dout, didx = up(x), gpu.alloc(out_n), gpu.allocInts(out_n)
    gpu.forwardMaxpool(out_n, h, w, c, stride, size, pad, dx, dout, didx)
    assert_bitexact(down(dout, out_c), out_c, f"maxpool fwd {case}")
    assert_bitexact(down(didx, idx_c), idx_c, f"maxpool idx {case}")
    delta = (normal(r, out_n) * np.float32(10.0) ** uniform(r, out_n, -3, 3)).astype(np.float32)
    prev = normal(r, x.size)
    prev_c = prev.copy()
    ref.backwardMaxpool(idx_c, delta, prev_c)
    dd, dprev = up(delta), up(prev)
    gpu.backwardMaxpool(x.size, h, w, c, stride, size, pad, dd, dprev, didx)
    assert_bitexact(down(dprev, prev), prev_c, f"maxpool bwd {case}")
    for b in (dx, dout, didx, dd, dprev):
        gpu.free(b)


@pytest.mark.parametrize("C,H,W,k,s,p", CONV)
def test_conv_lowering(dev, C, H, W, k, s, p):
    if H + 2 * p < k or W + 2 * p < k:
        pytest.skip("window larger than the padded image")
    r = rng(C * 1000 + H * 31 + W)
    im = uniform(r, C * H * W)
    ncol = C * k * k * ref.conv_out_dim(H, k, s, p) * ref.conv_out_dim(W, k, s, p)
    cpu_col = np.empty(ncol, np.float32)
    ref.im2col(im, C, H, W, k, s, p, cpu_col)
    dim, dcol = up(im), gpu.alloc(ncol)
    gpu.im2col(dim, C, H, W, k, s, p, dcol)
    assert_bitexact(down(dcol, cpu_col), cpu_col, "im2col")
    base = uniform(r, C * H * W)
    cpu_im = base.copy()
    ref.col2im(cpu_col, C, H, W, k, s, p, cpu_im)
    gpu.push(dim, base)
    gpu.col2im(dcol, C, H, W, k, s, p, dim)
    assert_bitexact(down(dim, base), cpu_im, "col2im")
    gpu.free(dim)
    gpu.free(dcol)


@pytest.mark.parametrize("ta,tb,m,n,k", GEMM)
def test_gemm(dev, ta, tb, m, n, k):
    gemm_check(ta, tb, m, n, k, 1.25 if k % 2 else -0.5, (0.0, 1.0, 0.5)[k % 3], seed=m + n + k,
               pad=(m % 3, n % 2, k % 4))


@pytest.mark.parametrize("case", LAYERS, ids=str)
def test_convolution_layer(dev, case):
    batch, groups, C, H, W, F, ks, s, p = case
    r = rng(sum(case) * 7 + 3)
    ho, wo = ref.conv_out_dim(H, ks, s, p), ref.conv_out_dim(W, ks, s, p)
    if ks == 1 and ho * wo > H * W:
        pytest.skip("ksize 1 with padding: the layer reads past the image as a k x n matrix")
    x = uniform(r, batch * C * H * W)
    w = uniform(r, F * (C // groups) * ks * ks)
    d = uniform(r, batch * F * ho * wo)
    out0, wu0 = uniform(r, batch * F * ho * wo), uniform(r, F * (C // groups) * ks * ks)
    dx, dw, dd, do, du = up(x), up(w), up(d), up(out0), up(wu0)
    want, bd, _ = conv_reference(case, x, w, out0)
    gpu.convolutionForward(batch, groups, C, H, W, F, ks, s, p, dw, dx, do)
    err = np.abs(down(do, out0).astype(np.float64) - want)
    assert (err <= bd).all(), f"forward {case}: max err/bound {float(np.max(err / np.maximum(bd, 1e-300))):.3g}"
    want, bd = wgrad_reference(case, x, d, wu0)
    gpu.convolutionWeightGradient(batch, groups, C, H, W, F, ks, s, p, dd, dx, du)
    err = np.abs(down(du, wu0).astype(np.float64) - want)
    assert (err <= bd).all(), f"weight gradient {case}: max err/bound {float(np.max(err / np.maximum(bd, 1e-300))):.3g}"
    im0 = uniform(r, batch * C * H * W)
    di = up(im0)
    want, bd = dgrad_reference(case, w, d, im0)
    gpu.convolutionDataGradient(batch, groups, C, H, W, F, ks, s, p, dw, dd, di)
    err = np.abs(down(di, im0).astype(np.float64) - want)
    assert (err <= bd).all(), f"data gradient {case}: max err/bound {float(np.max(err / np.maximum(bd, 1e-300))):.3g}"
    for b in (dx, dw, dd, do, du, di):
        gpu.free(b)
