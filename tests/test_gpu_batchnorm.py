"""GPU parity of the bias/scale broadcasts and the batch-norm reductions.

Broadcast ops (add_bias, scale_bias, normalize, normalize_delta) are fed the
CPU twin's per-channel vectors, so each op is checked in isolation and held
to bit-exactness. Reductions (mean, variance, mean_delta, variance_delta,
backward_bias, backward_scale) are held to the 1e-5 rule of tests/helpers.py
against an f64 evaluation of the same formula. Shapes: gputest's B4*F17*S53
(gputest.zig:157-160), odd and tiny shapes, spatial == 1 (connected layers),
and the benchmark configs 1 ([128,32,32,32]) and 2 ([64,128,56,56]) at full size.
"""

from __future__ import annotations

import numpy as np
import pytest

from darknet_zig_amd import gpu
from darknet_zig_amd.activations import Activation
from oracle import ref
from tests.helpers import assert_bitexact, assert_r5, chan_f32, chan_sum64, down, normal, rng, uniform, up

pytestmark = pytest.mark.gpu

SHAPES = [
    (4, 17, 53),      # gputest
    (1, 2, 4),        # blas.zig:334-346's known-answer shape
    (3, 5, 7),        # smoke_test.zig:276-308's bijection shape
    (2, 3, 1),        # spatial 1 (connected layer)
    (7, 1, 13),
    (5, 33, 196),     # spatial % 4 == 0, filters not a power of two
    (16, 64, 3136),   # K > 1 split path
    (8, 1024, 169),   # 13x13 planes: spatial % 4 != 0, one workgroup a channel
]
CONFIG1 = (128, 32, 1024)
CONFIG2 = (64, 128, 3136)


def _chan64(a: np.ndarray, shape) -> np.ndarray:
    B, F, S = shape
    return a.astype(np.float64).reshape(B, F, S)


def _stats(x: np.ndarray, shape):
    B, F, S = shape
    m = np.empty(F, np.float32)
    v = np.empty(F, np.float32)
    ref.mean(x, B, F, S, m)
    ref.variance(x, m, B, F, S, v)
    return m, v


@pytest.mark.parametrize("shape", SHAPES + [CONFIG1], ids=str)
def test_add_scale_bias(dev, shape):
    B, F, S = shape
    r = rng(sum(shape))
    x, bias, scales = normal(r, B * F * S), normal(r, F, 0, 0.1), uniform(r, F, 0.5, 1.5)
    for name, fn, cpu_fn, vec in (
        ("add_bias", gpu.addBias, ref.addBias, bias),
        ("scale_bias", gpu.scaleBias, ref.scaleBias, scales),
    ):
        cpu = x.copy()
        cpu_fn(cpu, vec, B, F, S)
        dx, dv = up(x), up(vec)
        fn(dx, dv, B, F, S)
        assert_bitexact(down(dx, x), cpu, f"{name} {shape}")
        # numpy broadcast pins the NCHW channel index independently of the twin
        want = x.reshape(B, F, S) + vec[None, :, None] if name == "add_bias" else x.reshape(B, F, S) * vec[None, :, None]
        assert_bitexact(cpu, want.astype(np.float32).ravel(), f"{name} numpy")
        gpu.free(dx)
        gpu.free(dv)


@pytest.mark.parametrize("shape", SHAPES + [CONFIG1], ids=str)
def test_mean_variance_normalize(dev, shape):
    B, F, S = shape
    r = rng(1000 + sum(shape))
    x = normal(r, B * F * S, 0.3, 1.0)
    m_cpu, v_cpu = _stats(x, shape)
    dx = up(x)
    dm, dvar = gpu.alloc(F), gpu.alloc(F)
    gpu.mean(dx, B, F, S, dm)
    m_gpu = down(dm, m_cpu)
    scale_m = np.float32(1.0) / np.float32(B * S)
    x64 = _chan64(x, shape)
    assert_r5(m_gpu, m_cpu, x64.sum(axis=(0, 2)) * np.float64(scale_m), f"mean {shape}")

    # variance on the CPU mean, so only the reduction differs
    dm_cpu = up(m_cpu)
    gpu.variance(dx, dm_cpu, B, F, S, dvar)
    v_gpu = down(dvar, v_cpu)
    if B * S > 1:
        scale_v = np.float32(1.0) / np.float32(B * S - 1)
        diff = x - chan_f32(m_cpu, shape)  # blas.zig:128-131: f32 difference, f32 square
        dev64 = chan_sum64(diff * diff, shape)
        assert_r5(v_gpu, v_cpu, dev64 * np.float64(scale_v), f"variance {shape}")

    # normalize with the CPU statistics: bit-exact
    cpu = x.copy()
    ref.normalize(cpu, m_cpu, v_cpu, B, F, S)
    dv_cpu = up(v_cpu)
    gpu.normalize(dx, dm_cpu, dv_cpu, B, F, S)
    assert_bitexact(down(dx, x), cpu, f"normalize {shape}")
    for b in (dx, dm, dvar, dm_cpu, dv_cpu):
        gpu.free(b)


@pytest.mark.parametrize("shape", SHAPES + [CONFIG2], ids=str)
def test_backward_reductions_and_normalize_delta(dev, shape):
    B, F, S = shape
    r = rng(2000 + sum(shape))
    x, delta, x_norm = normal(r, B * F * S), normal(r, B * F * S), normal(r, B * F * S)
    m, v = _stats(x, shape)
    x64, d64, xn64 = _chan64(x, shape), _chan64(delta, shape), _chan64(x_norm, shape)
    dx, dd, dxn, dm, dv = up(x), up(delta), up(x_norm), up(m), up(v)

    # backward_bias / backward_scale accumulate into nonzero updates
    upd0 = normal(r, F, 0, 1)
    for name, fn, cpu_fn, want64 in (
        ("backward_bias", lambda u: gpu.backwardBias(u, dd, B, F, S), lambda u: ref.backwardBias(u, delta, B, F, S),
         upd0.astype(np.float64) + d64.sum(axis=(0, 2))),
        ("backward_scale", lambda u: gpu.backwardScale(dxn, dd, B, F, S, u),
         lambda u: ref.backwardScale(x_norm, delta, B, F, S, u),
         upd0.astype(np.float64) + chan_sum64(delta * x_norm, shape)),  # f32 products, blas.zig:96
    ):
        cpu = upd0.copy()
        cpu_fn(cpu)
        du = up(upd0)
        fn(du)
        got = down(du, upd0)
        assert_r5(got, cpu, want64, f"{name} {shape}" + (" (spatial 1 path)" if S == 1 else ""))
        gpu.free(du)

    md_cpu, vd_cpu = np.empty(F, np.float32), np.empty(F, np.float32)
    ref.meanDelta(delta, v, B, F, S, md_cpu)
    ref.varianceDelta(x, delta, m, v, B, F, S, vd_cpu)
    dmd, dvd = gpu.alloc(F), gpu.alloc(F)
    gpu.meanDelta(dd, dv, B, F, S, dmd)
    gpu.varianceDelta(dx, dd, dm, dv, B, F, S, dvd)
    fac = np.float32(-1.0) / np.sqrt(v + np.float32(1e-5))
    assert_r5(down(dmd, md_cpu), md_cpu, d64.sum(axis=(0, 2)) * fac.astype(np.float64), f"mean_delta {shape}")
    v64 = (v + np.float32(1e-5)).astype(np.float64)
    vd64 = chan_sum64(delta * (x - chan_f32(m, shape)), shape) * -0.5 * v64**-1.5  # blas.zig:174
    assert_r5(down(dvd, vd_cpu), vd_cpu, vd64, f"variance_delta {shape}")

    # normalize_delta with the CPU per-channel inputs: bit-exact
    cpu = delta.copy()
    ref.normalizeDelta(x, m, v, md_cpu, vd_cpu, B, F, S, cpu)
    dmd_c, dvd_c = up(md_cpu), up(vd_cpu)
    gpu.normalizeDelta(dx, dm, dv, dmd_c, dvd_c, B, F, S, dd)
    assert_bitexact(down(dd, delta), cpu, f"normalize_delta {shape}")
    for b in (dx, dd, dxn, dm, dv, dmd, dvd, dmd_c, dvd_c):
        gpu.free(b)


@pytest.mark.parametrize("shape", [(256, 1000, 1), (1, 5, 1), (3, 70, 1), (129, 64, 1), (1000, 130, 1),
                                   (4099, 33, 1), (17, 2000, 1)], ids=str)
def test_backward_bias_connected(dev, shape):
    """backward_bias with spatial 1 (a connected layer's [batch, filters]
    delta, gpu.zig:540-543): the 1e-5 rule against the twin's sequential sum
    and the exact f64 update, with large and cancelling updates (the twin's
    update starts from a value the batch's deltas nearly cancel), and the
    same bits on a repeat. Shapes cover filters off a multiple of 64, a batch
    off a multiple of the 16 row-waves and of 8 rows a load round, one row,
    and several load rounds per wave."""
    B, F, S = shape
    r = rng(777 + B + F)
    delta = normal(r, B * F, 0, 1)
    d64 = delta.astype(np.float64).reshape(B, F)
    upd0 = normal(r, F, 0, 10)
    upd0[::3] = (-d64.sum(axis=0)[::3]).astype(np.float32)  # near-cancelling updates
    cpu = upd0.copy()
    ref.backwardBias(cpu, delta, B, F, S)
    dd, du = up(delta), up(upd0)
    gpu.backwardBias(du, dd, B, F, S)
    got = down(du, upd0)
    assert_r5(got, cpu, upd0.astype(np.float64) + d64.sum(axis=0), f"backward_bias {shape}")
    gpu.push(du, upd0)
    gpu.backwardBias(du, dd, B, F, S)
    assert_bitexact(down(du, upd0), got, f"backward_bias repeat {shape}")
    for b in (dd, du):
        gpu.free(b)


@pytest.mark.parametrize("shape", [CONFIG1, CONFIG2, (16, 64, 3136)], ids=str)
def test_reductions_deterministic(dev, shape):
    """Same input, same bits, every time: a split reduction's last workgroup
    per channel adds the partials in index order, whichever workgroup that
    is. 200 repeats of each op at shapes that split."""
    B, F, S = shape
    r = rng(9)
    x, d = normal(r, B * F * S), normal(r, B * F * S)
    m, v = _stats(x, shape)
    dx, dd, dm, dv, out = up(x), up(d), up(m), up(v), gpu.alloc(F)
    ops = {
        "mean": lambda: gpu.mean(dx, B, F, S, out),
        "variance": lambda: gpu.variance(dx, dm, B, F, S, out),
        "variance_delta": lambda: gpu.varianceDelta(dx, dd, dm, dv, B, F, S, out),
    }
    for name, op in ops.items():
        first = None
        for _ in range(200):
            op()
            got = down(out, np.empty(F, np.float32))
            if first is None:
                first = got
            else:
                assert_bitexact(got, first, f"{name} repeat {shape}")
    zero = up(np.zeros(F, np.float32))
    for _ in range(50):  # accumulate: each call adds the same bits
        gpu.backwardBias(zero, dd, B, F, S)
    single = up(np.zeros(F, np.float32))
    gpu.backwardBias(single, dd, B, F, S)
    s1 = down(single, np.empty(F, np.float32))
    want = np.zeros(F, np.float32)
    for _ in range(50):
        want = want + s1
    assert_bitexact(down(zero, want), want, f"backward_bias x50 {shape}")
    for b in (dx, dd, dm, dv, out, zero, single):
        gpu.free(b)


def _bn_forward_cpu(x, scales, biases, roll_m, roll_v, shape):
    """batchnorm.zig:74-99 (+ the conv layer's leaky activation,
    convolutional.zig:269) on the CPU twins."""
    B, F, S = shape
    out = x.copy()
    xs = out.copy()
    m, v = np.empty(F, np.float32), np.empty(F, np.float32)
    ref.mean(out, B, F, S, m)
    ref.variance(out, m, B, F, S, v)
    # batchnorm.zig:140-143 with its f32 constants: scal(rolling_momentum),
    # axpy(1 - rolling_momentum) -- 0.99f and 0.00999999f, not 0.01
    ref.scal(ref.ROLLING_MOMENTUM, roll_m)
    ref.axpy(ref.EMA_ALPHA, m, roll_m)
    ref.scal(ref.ROLLING_MOMENTUM, roll_v)
    ref.axpy(ref.EMA_ALPHA, v, roll_v)
    ref.normalize(out, m, v, B, F, S)
    x_norm = out.copy()
    ref.scaleBias(out, scales, B, F, S)
    ref.addBias(out, biases, B, F, S)
    ref.activateArray(out, Activation.leaky)
    return out, xs, x_norm, m, v


def test_bn_layer_forward_sequence(dev):
    """Config 1 as the layer runs it (batchnorm.zig:129-153 + activate): the
    reductions feed the broadcasts, so the chain is compared with a tolerance
    (gputest.zig:214-235 chains the same way at 1e-3)."""
    B, F, S = CONFIG1
    r = rng(1)
    x, scales, biases = normal(r, B * F * S), uniform(r, F, 0.5, 1.5), normal(r, F, 0, 0.1)
    rm0, rv0 = normal(r, F, 0, 0.1), uniform(r, F, 0.5, 1.5)
    rm, rv = rm0.copy(), rv0.copy()
    out_c, _, xn_c, m_c, v_c = _bn_forward_cpu(x, scales, biases, rm, rv, CONFIG1)

    n = B * F * S
    d_out, d_x, d_xn = up(x), gpu.alloc(n), gpu.alloc(n)
    d_m, d_v, d_rm, d_rv, d_s, d_b = gpu.alloc(F), gpu.alloc(F), up(rm0), up(rv0), up(scales), up(biases)
    gpu.copy(n, d_out, d_x)
    gpu.mean(d_out, B, F, S, d_m)
    gpu.variance(d_out, d_m, B, F, S, d_v)
    gpu.scal(F, float(ref.ROLLING_MOMENTUM), d_rm)
    gpu.axpy(F, float(ref.EMA_ALPHA), d_m, d_rm)
    gpu.scal(F, float(ref.ROLLING_MOMENTUM), d_rv)
    gpu.axpy(F, float(ref.EMA_ALPHA), d_v, d_rv)
    gpu.normalize(d_out, d_m, d_v, B, F, S)
    gpu.copy(n, d_out, d_xn)
    gpu.scaleBias(d_out, d_s, B, F, S)
    gpu.addBias(d_out, d_b, B, F, S)
    gpu.activateArray(d_out, n, Activation.leaky)
    np.testing.assert_allclose(down(d_out, x), out_c, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(down(d_xn, x), xn_c, rtol=1e-4, atol=1e-5)
    assert_bitexact(down(d_x, x), x, "x copy")
    np.testing.assert_allclose(down(d_rm, rm0), rm, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(down(d_rv, rv0), rv, rtol=1e-5, atol=1e-7)
    for b in (d_out, d_x, d_xn, d_m, d_v, d_rm, d_rv, d_s, d_b):
        gpu.free(b)


def test_bn_layer_backward_sequence(dev):
    """Config 2 as the layer runs it: gradient (leaky), then
    batchnorm.zig:155-174's backward_bias, backward_scale, scale_bias(delta),
    mean_delta, variance_delta, normalize_delta, against the CPU sequence
    (batchnorm.zig:101-123)."""
    B, F, S = CONFIG2
    n = B * F * S
    r = rng(2)
    y, delta, x, x_norm = normal(r, n), normal(r, n), normal(r, n), normal(r, n)
    ref.activateArray(y, Activation.leaky)
    scales = uniform(r, F, 0.5, 1.5)
    m, v = _stats(x, CONFIG2)
    bu0, su0 = np.zeros(F, np.float32), np.zeros(F, np.float32)

    d_c = delta.copy()
    bu, su = bu0.copy(), su0.copy()
    md, vd = np.empty(F, np.float32), np.empty(F, np.float32)
    ref.gradientArray(y, Activation.leaky, d_c)
    g64 = _chan64(d_c, CONFIG2)  # the gradient is bit-exact, so both sides reduce this
    bu64 = g64.sum(axis=(0, 2))
    su64 = chan_sum64(d_c * x_norm, CONFIG2)  # f32 products of the (bit-exact) gradient
    ref.backwardBias(bu, d_c, B, F, S)
    ref.backwardScale(x_norm, d_c, B, F, S, su)
    ref.scaleBias(d_c, scales, B, F, S)
    ref.meanDelta(d_c, v, B, F, S, md)
    ref.varianceDelta(x, d_c, m, v, B, F, S, vd)
    ref.normalizeDelta(x, m, v, md, vd, B, F, S, d_c)

    g_y, g_d, g_x, g_xn = up(y), up(delta), up(x), up(x_norm)
    g_m, g_v, g_s, g_bu, g_su, g_md, g_vd = up(m), up(v), up(scales), up(bu0), up(su0), gpu.alloc(F), gpu.alloc(F)
    gpu.gradientArray(g_y, n, Activation.leaky, g_d)
    gpu.backwardBias(g_bu, g_d, B, F, S)
    gpu.backwardScale(g_xn, g_d, B, F, S, g_su)
    gpu.scaleBias(g_d, g_s, B, F, S)
    gpu.meanDelta(g_d, g_v, B, F, S, g_md)
    gpu.varianceDelta(g_x, g_d, g_m, g_v, B, F, S, g_vd)
    gpu.normalizeDelta(g_x, g_m, g_v, g_md, g_vd, B, F, S, g_d)
    # The reductions in the chain follow the reduction rule; the final delta
    # carries their (tiny) differences through md/N and vd*2*(x-m)/N.
    assert_r5(down(g_bu, bu0), bu, bu64, "chain backward_bias")
    assert_r5(down(g_su, su0), su, su64, "chain backward_scale")
    np.testing.assert_allclose(down(g_d, delta), d_c, rtol=1e-4, atol=1e-5)
    for b in (g_y, g_d, g_x, g_xn, g_m, g_v, g_s, g_bu, g_su, g_md, g_vd):
        gpu.free(b)


def test_empty_channels(dev):
    """filters == 0 is a no-op; batch*spatial == 0 follows the twin's
    arithmetic (mean = 0 * (1/0) = NaN); backward_bias with batch 0 adds
    nothing."""
    out = up(np.array([5.0, -0.0], np.float32))
    gpu.mean(gpu.Buf(), 0, 2, 0, out)
    got = down(out, np.zeros(2, np.float32))
    assert np.isnan(got).all()
    gpu.backwardBias(out, gpu.Buf(), 0, 2, 3)
    gpu.mean(gpu.Buf(), 3, 0, 4, gpu.Buf())  # filters 0: nothing touched
    gpu.free(out)
