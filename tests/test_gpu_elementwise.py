"""GPU parity of the elementwise ops against the CPU twins (bit-exact).

Mirrors gputest.zig:86-154 (n = 4099, U(-1,1) inputs, seeded) and extends it
to every activation and gradient, fill/copy/mul/constrain, the losses, sizes
around the float4 tail, misaligned views (Buf.offset) and an SGD-sized vector.
"""

from __future__ import annotations

import numpy as np
import pytest

from darknet_zig_amd import gpu
from darknet_zig_amd.activations import Activation
from oracle import ref
from tests.helpers import assert_bitexact, down, normal, rng, uniform, up

pytestmark = pytest.mark.gpu

SIZES = [1, 3, 4, 5, 4099, 65536 + 7]

SPECIALS = np.array(
    [0.0, -0.0, 1.0, -1.0, 0.5, -0.5, 4.0, -4.0, 88.0, -88.0, 88.8, -103.9, -104.0, 1e-40, -1e-40,
     np.inf, -np.inf, np.nan, 3.4e38, -3.4e38, 1e-7, -1e-7, 0.999, 1.001, 2.5, -2.5],
    dtype=np.float32,
)


def _run_inplace(op, host: np.ndarray, offset: int = 0):
    """Uploads host at an element offset (a Buf.offset view) and runs op(buf)."""
    pad = np.zeros(offset, np.float32)
    whole = up(np.concatenate([pad, host]))
    view = whole.offset(offset)
    op(view)
    out = np.empty(host.size + offset, np.float32)
    gpu.pull(whole, out)
    gpu.free(whole)
    return out[offset:]


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("offset", [0, 1])
def test_axpy_scal(dev, n, offset):
    r = rng(20240921 + n)
    a, b = uniform(r, n), uniform(r, n)
    cpu = b.copy()
    ref.axpy(2.5, a, cpu)
    da = up(a)
    got = _run_inplace(lambda yb: gpu.axpy(n, 2.5, da, yb), b, offset)
    assert_bitexact(got, cpu, f"axpy n={n} off={offset}")
    cpu = a.copy()
    ref.scal(0.3, cpu)
    got = _run_inplace(lambda xb: gpu.scal(n, 0.3, xb), a, offset)
    assert_bitexact(got, cpu, f"scal n={n}")
    gpu.free(da)


def test_axpy_is_fused(dev):
    # One rounding: values where fma(a, x, y) != a*x + y in f32.
    a = np.float32(1.0 + 2.0**-12)
    x = np.full(1024, 1.0 + 2.0**-12, np.float32)
    y = np.full(1024, -(1.0 + 2.0**-11), np.float32)
    cpu = y.copy()
    ref.axpy(float(a), x, cpu)
    dx, dy = up(x), up(y)
    gpu.axpy(1024, float(a), dx, dy)
    got = down(dy, y)
    assert_bitexact(got, cpu, "axpy fma")
    assert got[0] != np.float32(a * x[0]) + y[0]  # the unfused value differs here
    gpu.free(dx)
    gpu.free(dy)


@pytest.mark.parametrize("n", SIZES)
def test_fill_copy_mul_constrain(dev, n):
    r = rng(7 + n)
    a, b = uniform(r, n, -3, 3), uniform(r, n, -3, 3)
    a[: min(n, 3)] = np.array([np.nan, -np.inf, np.inf], np.float32)[: min(n, 3)]

    x = up(a)
    gpu.fill(x, n, 0.75)
    assert_bitexact(down(x, a), np.full(n, 0.75, np.float32), "fill")
    gpu.free(x)

    x, y = up(a), gpu.alloc(n)
    gpu.copy(n, x, y)
    assert_bitexact(down(y, a), a, "copy")

    cpu = b.copy()
    ref.mul(a, cpu)
    yb = up(b)
    gpu.mul(n, x, yb)
    assert_bitexact(down(yb, b), cpu, "mul")

    cpu = a.copy()
    ref.constrainArray(1.5, cpu)
    gpu.constrainArray(n, 1.5, x)
    assert_bitexact(down(x, a), cpu, "constrain")
    for bb in (x, y, yb):
        gpu.free(bb)


def _act_inputs(a: Activation, n: int, seed: int) -> np.ndarray:
    r = rng(seed)
    x = np.concatenate([uniform(r, n, -6, 6), normal(r, n, 0, 30), SPECIALS])
    if a == Activation.stair:  # @intFromFloat is illegal behaviour on NaN/inf/huge
        x = x[np.isfinite(x) & (np.abs(x) < 2.0**62)]
    return np.ascontiguousarray(x)


@pytest.mark.parametrize("a", list(Activation), ids=lambda a: a.name)
def test_activate_array(dev, a):
    x = _act_inputs(a, 20000, 100 + int(a))
    cpu = x.copy()
    ref.activateArray(cpu, a)
    got = _run_inplace(lambda b: gpu.activateArray(b, x.size, a), x)
    assert_bitexact(got, cpu, f"activate {a.name}")


@pytest.mark.parametrize("a", list(Activation), ids=lambda a: a.name)
def test_gradient_array(dev, a):
    x = _act_inputs(a, 20000, 200 + int(a))
    y = x.copy()
    ref.activateArray(y, a)  # gradient() consumes activation outputs (gputest.zig:137-140)
    y = np.concatenate([y, x])  # and arbitrary values, to hit every branch
    delta = uniform(rng(300 + int(a)), y.size, -2, 2)
    cpu = delta.copy()
    ref.gradientArray(y, a, cpu)
    dy = up(y)
    got = _run_inplace(lambda d: gpu.gradientArray(dy, y.size, a, d), delta)
    assert_bitexact(got, cpu, f"gradient {a.name}")
    gpu.free(dy)


def test_logistic_dense_sweep(dev):
    # Every float32 in [-20, 20) with a stride of 3 ulps-ish: 2^24 inputs through
    # the ABI, checked bit for bit against the twin (which calls libm expf).
    lo, hi = np.float32(-20.0).view(np.int32), np.float32(20.0).view(np.int32)
    pos = np.arange(0, hi, 61, dtype=np.int32).view(np.float32)
    neg = -pos
    x = np.ascontiguousarray(np.concatenate([pos, neg]))
    for a in (Activation.logistic, Activation.tanh, Activation.elu):
        cpu = x.copy()
        ref.activateArray(cpu, a)
        got = _run_inplace(lambda b: gpu.activateArray(b, x.size, a), x)
        assert_bitexact(got, cpu, f"dense {a.name}")
    del lo


@pytest.mark.parametrize(
    "name, fn, cpu_fn",
    [
        ("softmax_x_ent", gpu.softmaxCrossEntropy, ref.softmaxCrossEntropy),
        ("l2", gpu.l2, ref.l2),
        ("l1", gpu.l1, ref.l1),
        ("smooth_l1", gpu.smoothL1, ref.smoothL1),
    ],
)
@pytest.mark.parametrize("n", [1, 4099, 256 * 1000])
def test_losses(dev, name, fn, cpu_fn, n):
    r = rng(400 + n)
    if name == "softmax_x_ent":
        pred = r.uniform(1e-6, 1.0, n).astype(np.float32)
        truth = (r.uniform(0, 1, n) < 0.1).astype(np.float32)
    else:
        pred, truth = uniform(r, n, -3, 3), uniform(r, n, -3, 3)
        truth[: min(n, 2)] = pred[: min(n, 2)]  # diff == 0 hits l1's -1 branch
    d_cpu, e_cpu = np.empty_like(pred), np.empty_like(pred)
    cpu_fn(pred, truth, d_cpu, e_cpu)
    dp, dt, dd, de = up(pred), up(truth), gpu.alloc(n), gpu.alloc(n)
    fn(n, dp, dt, dd, de)
    assert_bitexact(down(dd, pred), d_cpu, f"{name} delta")
    got_e = down(de, pred)
    if name == "softmax_x_ent":
        # err = -log(p) is a transcendental of a libm other than the host's:
        # within 1e-5 relative (one or two ulps).
        np.testing.assert_allclose(got_e, e_cpu, rtol=1e-5, atol=0)
    else:
        assert_bitexact(got_e, e_cpu, f"{name} err")
    for b in (dp, dt, dd, de):
        gpu.free(b)


def test_sgd_update_full_size(dev):
    """Config 4's SGD step over n = 25 000 000 floats, values ~N(0, 0.05):
    axpy(-decay*batch, w, dw), axpy(lr/batch, dw, w), scal(momentum, dw)
    (convolutional.zig:324-334)."""
    n = 25_000_000
    r = rng(4)
    w, dw = normal(r, n, 0, 0.05), normal(r, n, 0, 0.05)
    batch, lr, decay, momentum = 128, 0.1, 0.0005, 0.9
    cw, cdw = w.copy(), dw.copy()
    ref.axpy(-decay * batch, cw, cdw)
    ref.axpy(lr / batch, cdw, cw)
    ref.scal(momentum, cdw)
    gw, gdw = up(w), up(dw)
    gpu.axpy(n, -decay * batch, gw, gdw)
    gpu.axpy(n, lr / batch, gdw, gw)
    gpu.scal(n, momentum, gdw)
    assert_bitexact(down(gw, w), cw, "sgd w")
    assert_bitexact(down(gdw, dw), cdw, "sgd dw")
    gpu.free(gw)
    gpu.free(gdw)


def test_zero_sizes_are_noops(dev):
    b = up(np.array([1.0, 2.0], np.float32))
    gpu.axpy(0, 1.0, b, b)
    gpu.scal(0, 5.0, b)
    gpu.activateArray(b, 0, Activation.logistic)
    gpu.activateArray(b, 2, Activation.linear)
    assert down(b, np.zeros(2, np.float32)).tolist() == [1.0, 2.0]
    gpu.free(b)
