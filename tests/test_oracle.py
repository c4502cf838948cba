"""Pinning the CPU oracle (oracle/dkz_oracle.c) before it is trusted.

Each function of the C restatement is checked against something other than
its own formula: the reference's known answers (tests/golden/), exact
rational arithmetic, numpy's independent float32/float64 arithmetic on
reshaped arrays (which pins NCHW indexing and strides), closed forms and
invariants, finite differences, and brute force on tiny inputs -- chosen so a
dropped term, a wrong sign or index, or a transposed operand fails one of them.
"""

from __future__ import annotations

import json
import math
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

from darknet_zig_amd.activations import Activation
from oracle import ref

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())["cases"]
f32 = np.float32


def case(op):
    return next(c for c in GOLDEN if c["op"] == op)


def r(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------------------
# the reference's own known answers
# ---------------------------------------------------------------------------


def test_known_softmax():  # blas.zig:324-332
    c = case("softmax")
    a = c["args"]
    x = np.array(a["input"], np.float32)
    out = np.zeros_like(x)
    ref.softmax(x, a["n"], a["batch"], a["batch_offset"], a["groups"], a["group_offset"], a["stride"], a["temp"], out)
    assert abs(float(out.sum()) - c["expect"]["sum"]) <= c["expect"]["sum_abs_tol"]
    assert out[3] > out[0]


def test_known_mean_normalize():  # blas.zig:334-346
    c = case("mean_variance_normalize")
    a = c["args"]
    x = np.array(a["x"], np.float32)
    m, v = np.empty(2, np.float32), np.empty(2, np.float32)
    ref.mean(x, a["batch"], a["filters"], a["spatial"], m)
    np.testing.assert_allclose(m, c["expect"]["mean"], atol=c["expect"]["mean_abs_tol"])
    ref.variance(x, m, a["batch"], a["filters"], a["spatial"], v)
    ref.normalize(x, m, v, a["batch"], a["filters"], a["spatial"])
    assert abs(float(x[:4].sum())) <= c["expect"]["normalized_sum_abs_tol"]


def test_known_leaky():  # activations.zig:145-150
    c = case("leaky")
    for xin, want in zip(c["args"]["activate"], c["expect"]["activate"]):
        assert abs(ref.activate(xin, Activation.leaky) - want) <= c["expect"]["abs_tol"]
    for yin, want in zip(c["args"]["gradient"], c["expect"]["gradient"]):
        assert abs(ref.gradient(yin, Activation.leaky) - want) <= c["expect"]["abs_tol"]


def test_known_bn_rolling_ema():  # smoke_test.zig:229-274, via scal/axpy on C floats
    c = case("bn_rolling_ema")
    a = c["args"]
    n = a["batch"] * a["w"] * a["h"] * a["c"]
    x = r(31).uniform(*a["input_uniform"], n).astype(np.float32)
    m, v = np.empty(a["c"], np.float32), np.empty(a["c"], np.float32)
    ref.mean(x, a["batch"], a["c"], a["w"] * a["h"], m)
    ref.variance(x, m, a["batch"], a["c"], a["w"] * a["h"], v)
    rm, rv = np.zeros(a["c"], np.float32), np.zeros(a["c"], np.float32)
    for _ in range(a["steps"]):  # batchnorm.zig:86-89
        ref.scal(a["momentum"], rm)
        ref.axpy(1 - a["momentum"], m, rm)
        ref.scal(a["momentum"], rv)
        ref.axpy(1 - a["momentum"], v, rv)
    frac = 1.0 - ref.pow_f32(a["momentum"], a["steps"])
    lo, hi = c["expect"]["fraction_range"]
    assert lo < frac < hi
    np.testing.assert_allclose(rm, m * frac, rtol=c["expect"]["rel_tol"])
    np.testing.assert_allclose(rv, v * frac, rtol=c["expect"]["rel_tol"])


def test_known_nchw_bijection():  # smoke_test.zig:276-308, through add_bias
    c = case("nchw_bijection")
    B, F, S = c["args"]["batch"], c["args"]["n"], c["args"]["size"]
    out = np.zeros(B * F * S, np.float32)
    bias = np.ones(F, np.float32)
    ref.addBias(out, bias, B, F, S)
    assert np.all(out == c["expect"]["each_index_hit"])  # every element hit exactly once
    bias = np.arange(F, dtype=np.float32)
    out[:] = 0
    ref.addBias(out, bias, B, F, S)
    assert np.array_equal(out.reshape(B, F, S), np.broadcast_to(bias[None, :, None], (B, F, S)))


# ---------------------------------------------------------------------------
# elementwise: exact arithmetic
# ---------------------------------------------------------------------------


def round_f32(q: Fraction) -> float:
    """Round an exact rational to the nearest float32 (ties to even)."""
    if q == 0:
        return 0.0
    sign = -1 if q < 0 else 1
    q = abs(q)
    e = q.numerator.bit_length() - q.denominator.bit_length()
    if Fraction(2) ** e > q:
        e -= 1
    e = max(e, -126)  # subnormals share the minimum exponent
    scale = Fraction(2) ** (23 - e)
    m = q * scale
    fl = math.floor(m)
    rem = m - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    val = Fraction(fl) / scale
    if val >= Fraction(2) ** 128:
        return sign * math.inf
    return sign * float(val)


def test_axpy_single_rounding():
    # F1: blas.zig:21-24 under @setFloatMode(.optimized) contracts to one fma.
    g = r(1)
    a = f32(1.0 + 2.0**-12)
    x = np.concatenate([g.uniform(-2, 2, 2000), [1.0 + 2.0**-12] * 4]).astype(np.float32)
    y = np.concatenate([g.uniform(-2, 2, 2000), [-(1.0 + 2.0**-11)] * 4]).astype(np.float32)
    got = y.copy()
    ref.axpy(float(a), x, got)
    want = [round_f32(Fraction(float(a)) * Fraction(float(xi)) + Fraction(float(yi))) for xi, yi in zip(x, y)]
    assert np.array_equal(got, np.array(want, np.float32))
    two_roundings = (a * x + y).astype(np.float32)
    assert not np.array_equal(got, two_roundings)  # the unfused form is distinguishable


def test_scal_mul_fill_copy_constrain():
    g = r(2)
    x = g.normal(0, 3, 5000).astype(np.float32)
    y = g.normal(0, 3, 5000).astype(np.float32)
    t = x.copy()
    ref.scal(0.3, t)
    assert np.array_equal(t, x * f32(0.3))
    t = y.copy()
    ref.mul(x, t)
    assert np.array_equal(t, y * x)
    t = np.empty_like(x)
    ref.fill(t, -2.5)
    assert np.all(t == f32(-2.5))
    ref.copy(x, t)
    assert np.array_equal(t, x)
    x[:3] = [np.nan, np.inf, -np.inf]
    t = x.copy()
    ref.constrainArray(1.5, t)
    assert t[0] == f32(1.5)  # std.math.clamp: @min(NaN, a) = a, then @max(-a, a) = a
    assert t[1] == f32(1.5) and t[2] == f32(-1.5)
    assert np.array_equal(t[3:], np.clip(x[3:], -1.5, 1.5))


# ---------------------------------------------------------------------------
# bias / scale / batch-norm
# ---------------------------------------------------------------------------

SHAPES = [(1, 1, 1), (2, 3, 5), (4, 17, 53), (3, 8, 16)]


@pytest.mark.parametrize("shape", SHAPES)
def test_bias_broadcasts_match_numpy(shape):
    B, F, S = shape
    g = r(sum(shape))
    x = g.normal(0, 1, B * F * S).astype(np.float32)
    b = g.normal(0, 1, F).astype(np.float32)
    t = x.copy()
    ref.addBias(t, b, B, F, S)
    assert np.array_equal(t, (x.reshape(B, F, S) + b[None, :, None]).ravel())
    t = x.copy()
    ref.scaleBias(t, b, B, F, S)
    assert np.array_equal(t, (x.reshape(B, F, S) * b[None, :, None]).ravel())


@pytest.mark.parametrize("shape", SHAPES)
def test_channel_reductions_match_f64(shape):
    B, F, S = shape
    g = r(100 + sum(shape))
    # well-conditioned data so the twin's f32 sums sit within 1e-6 of f64
    x = g.uniform(1, 2, B * F * S).astype(np.float32)
    d = g.uniform(1, 2, B * F * S).astype(np.float32)
    x64, d64 = (a.astype(np.float64).reshape(B, F, S) for a in (x, d))
    m, v = np.empty(F, np.float32), np.empty(F, np.float32)
    ref.mean(x, B, F, S, m)
    np.testing.assert_allclose(m, x64.mean(axis=(0, 2)), rtol=1e-6)
    if B * S > 1:
        ref.variance(x, m, B, F, S, v)
        want = ((x64 - m.astype(np.float64)[None, :, None]) ** 2).sum(axis=(0, 2)) / (B * S - 1)
        np.testing.assert_allclose(v, want, rtol=2e-6)
    upd0 = g.normal(0, 1, F).astype(np.float32)
    u = upd0.copy()
    ref.backwardBias(u, d, B, F, S)
    np.testing.assert_allclose(u, upd0 + d64.sum(axis=(0, 2)), rtol=1e-6)
    u = upd0.copy()
    ref.backwardScale(x, d, B, F, S, u)
    np.testing.assert_allclose(u, upd0 + (x64 * d64).sum(axis=(0, 2)), rtol=1e-6)
    var = g.uniform(0.5, 2, F).astype(np.float32)
    md = np.empty(F, np.float32)
    ref.meanDelta(d, var, B, F, S, md)
    np.testing.assert_allclose(md, -d64.sum(axis=(0, 2)) / np.sqrt(var.astype(np.float64) + 1e-5), rtol=2e-6)


def test_backward_bias_order_brute_force():
    # blas.zig:73-82 adds one row sum per batch item, in order; emulate it with
    # numpy float32 scalars and compare bit for bit.
    B, F, S = 3, 2, 5
    d = r(7).normal(0, 10, B * F * S).astype(np.float32)
    upd = np.array([0.1, -0.3], np.float32)
    want = upd.copy()
    for b in range(B):
        for f in range(F):
            s = f32(0.0)
            for k in range(S):
                s = f32(s + d[(b * F + f) * S + k])
            want[f] = f32(want[f] + s)
    got = upd.copy()
    ref.backwardBias(got, d, B, F, S)
    assert np.array_equal(got, want)


def test_normalize_closed_form():
    B, F, S = 8, 3, 49
    x = r(8).normal(2, 3, B * F * S).astype(np.float32)
    m, v = np.empty(F, np.float32), np.empty(F, np.float32)
    ref.mean(x, B, F, S, m)
    ref.variance(x, m, B, F, S, v)
    ref.normalize(x, m, v, B, F, S)
    xn = x.astype(np.float64).reshape(B, F, S)
    n = B * S
    np.testing.assert_allclose(xn.mean(axis=(0, 2)), 0.0, atol=1e-5)
    # unbiased v in the denominator, biased second moment: (n-1)/n (the 1e-6 is negligible)
    np.testing.assert_allclose((xn**2).mean(axis=(0, 2)), (n - 1) / n, rtol=1e-4)


def test_bn_backward_is_the_gradient_of_normalisation():
    """mean_delta, variance_delta and normalize_delta together are dL/dx for
    L(x) = sum(dy * xhat(x)), xhat = (x - mu)/sqrt(var_biased + 1e-5), when fed
    the biased variance (blas.zig:148-204). Central differences in f64."""
    B, F, S = 2, 3, 5
    g = r(9)
    x = g.normal(0, 1, B * F * S).astype(np.float32)
    dy = g.normal(0, 1, B * F * S).astype(np.float32)
    x64 = x.astype(np.float64).reshape(B, F, S)
    mu = x64.mean(axis=(0, 2))
    varb = x64.var(axis=(0, 2))
    m32, v32 = mu.astype(np.float32), varb.astype(np.float32)
    md, vd = np.empty(F, np.float32), np.empty(F, np.float32)
    ref.meanDelta(dy, v32, B, F, S, md)
    ref.varianceDelta(x, dy, m32, v32, B, F, S, vd)
    dx = dy.copy()
    ref.normalizeDelta(x, m32, v32, md, vd, B, F, S, dx)

    def loss(xx):
        xx = xx.reshape(B, F, S)
        mu_ = xx.mean(axis=(0, 2), keepdims=True)
        var_ = xx.var(axis=(0, 2), keepdims=True)
        return float((dy.astype(np.float64).reshape(B, F, S) * (xx - mu_) / np.sqrt(var_ + 1e-5)).sum())

    h = 1e-5
    num = np.empty(x.size)
    base = x.astype(np.float64)
    for i in range(x.size):
        p, q = base.copy(), base.copy()
        p[i] += h
        q[i] -= h
        num[i] = (loss(p) - loss(q)) / (2 * h)
    np.testing.assert_allclose(dx, num, rtol=2e-3, atol=2e-4)


# ---------------------------------------------------------------------------
# softmax and losses
# ---------------------------------------------------------------------------


def test_softmax_against_f64_and_invariants():
    g = r(10)
    b, c = 6, 137
    x = g.normal(0, 4, b * c).astype(np.float32)
    out = np.zeros_like(x)
    ref.softmax(x, c, b, c, 1, c, 1, 1.0, out)
    x64 = x.astype(np.float64).reshape(b, c)
    e = np.exp(x64 - x64.max(axis=1, keepdims=True))
    np.testing.assert_allclose(out.reshape(b, c), e / e.sum(axis=1, keepdims=True), rtol=2e-6, atol=1e-12)
    out2 = np.zeros_like(x)
    ref.softmax(x * f32(0.5), c, b, c, 1, c, 1, 0.5, out2)  # x/T with T = 0.5 undoes the halving
    np.testing.assert_allclose(out2, out, rtol=1e-6, atol=1e-12)


def test_softmax_groups_and_stride():
    # spatial softmax over channels: group g of image b starts at b*c*s + g and
    # steps by s (blas.zig:225-242); numpy softmax over axis 1 of [b, c, s].
    b, c, s = 2, 7, 9
    x = r(11).normal(0, 2, b * c * s).astype(np.float32)
    out = np.zeros_like(x)
    ref.softmax(x, c, b, c * s, s, 1, s, 1.0, out)
    x64 = x.astype(np.float64).reshape(b, c, s)
    e = np.exp(x64 - x64.max(axis=1, keepdims=True))
    np.testing.assert_allclose(out.reshape(b, c, s), e / e.sum(axis=1, keepdims=True), rtol=2e-6)


def test_losses():
    p = np.array([0.25, 0.5, 1.0, 3.0, -2.0, 0.5], np.float32)
    t = np.array([1.0, 0.0, 1.0, 0.0, 0.0, 0.5], np.float32)
    d, e = np.empty_like(p), np.empty_like(p)
    ref.softmaxCrossEntropy(p, t, d, e)
    assert np.array_equal(d, t - p)
    with np.errstate(invalid="ignore"):
        want = np.where(t != 0, -np.log(p.astype(np.float64)), 0.0)
    np.testing.assert_allclose(e, want, rtol=1e-6)
    ref.l2(p, t, d, e)
    assert np.array_equal(d, t - p) and np.array_equal(e, (t - p) * (t - p))
    ref.l1(p, t, d, e)
    assert np.array_equal(e, np.abs(t - p))
    assert d.tolist() == [1.0, -1.0, -1.0, -1.0, 1.0, -1.0]  # diff == 0 gives -1 (blas.zig:266)
    ref.smoothL1(p, t, d, e)
    # |diff| < 1: (diff^2, diff); else (2|diff|-1, +1 if diff < 0 else -1) (blas.zig:270-282)
    assert e.tolist() == [0.5625, 0.25, 0.0, 5.0, 3.0, 0.0]
    assert d.tolist() == [0.75, -0.5, 0.0, 1.0, -1.0, 0.0]


# ---------------------------------------------------------------------------
# shortcut
# ---------------------------------------------------------------------------


@pytest.mark.parametrize(
    "batch, w1, h1, c1, w2, h2, c2",
    [(2, 8, 8, 4, 8, 8, 4), (2, 28, 28, 6, 14, 14, 9), (1, 7, 7, 3, 14, 14, 3), (2, 9, 9, 5, 4, 4, 2)],
)
def test_shortcut_matches_numpy_slicing(batch, w1, h1, c1, w2, h2, c2):
    g = r(w1 + c2)
    add = g.normal(0, 1, batch * c1 * h1 * w1).astype(np.float32)
    out = g.normal(0, 1, batch * c2 * h2 * w2).astype(np.float32)
    s1, s2 = 0.5, 2.0
    got = out.copy()
    ref.shortcut(batch, w1, h1, c1, add, w2, h2, c2, s1, s2, got)
    stride, sample = max(w1 // w2, 1), max(w2 // w1, 1)
    mw, mh, mc = min(w1, w2), min(h1, h2), min(c1, c2)
    A = add.reshape(batch, c1, h1, w1)[:, :mc, : mh * stride : stride, : mw * stride : stride]
    want = out.reshape(batch, c2, h2, w2).copy()
    O = want[:, :mc, : mh * sample : sample, : mw * sample : sample]
    want[:, :mc, : mh * sample : sample, : mw * sample : sample] = f32(s1) * O + f32(s2) * A
    assert np.array_equal(got, want.ravel())


# ---------------------------------------------------------------------------
# activations
# ---------------------------------------------------------------------------


def test_activation_special_values():
    L = Activation
    assert ref.activate(0.0, L.logistic) == 0.5
    assert math.copysign(1.0, ref.activate(-0.0, L.relu)) == 1.0  # a select: -0 -> +0
    assert ref.activate(2.5, L.stair) == 1.0 and ref.activate(3.5, L.stair) == 1.5
    assert ref.activate(-3.0, L.hardtan) == -1.0 and ref.activate(float("nan"), L.hardtan) == 1.0
    assert ref.activate(-5.0, L.plse) == f32(0.01) * f32(-1.0)
    assert ref.activate(2.0, L.lhtan) == f32(0.001) * f32(1.0) + f32(1.0)
    # selu's 1.0507 * 1.6732 is folded at comptime, then rounded to f32 once
    k = round_f32(Fraction("1.0507") * Fraction("1.6732"))
    assert ref.gradient(-1.0, L.selu) == f32(-1.0) + f32(k)
    assert f32(k) == f32(1.75803124)


SMOOTH = [Activation.logistic, Activation.loggy, Activation.tanh, Activation.elu, Activation.selu,
          Activation.leaky, Activation.relu, Activation.relie, Activation.ramp, Activation.plse,
          Activation.lhtan, Activation.hardtan, Activation.linear]


@pytest.mark.parametrize("a", SMOOTH, ids=lambda a: a.name)
def test_gradient_is_derivative_in_terms_of_output(a):
    """gradient(act(x)) ~ d act / dx away from kinks (activations.zig:3-7)."""
    xs = np.linspace(-3.7, 3.9, 61)
    kinks = {Activation.plse: [-4, 4], Activation.lhtan: [0, 1], Activation.hardtan: [-1, 1]}.get(a, [0])
    h = 1e-3
    for x in xs:
        if min(abs(x - k) for k in kinks) < 5 * h:
            continue
        y = ref.activate(float(x), a)
        num = (ref.activate(float(x + h), a) - ref.activate(float(x - h), a)) / (2 * h)
        assert abs(ref.gradient(y, a) - num) <= 5e-3 * max(1.0, abs(num)), (a.name, x)


# ---------------------------------------------------------------------------
# pooling
# ---------------------------------------------------------------------------


def maxpool_brute(x, batch, c, h, w, size, stride, pad):
    off = -(pad // 2)
    oh, ow = (h + pad - size) // stride + 1, (w + pad - size) // stride + 1
    out = np.empty((batch, c, oh, ow), np.float32)
    idx = np.empty((batch, c, oh, ow), np.int32)
    X = x.reshape(batch, c, h, w)
    for b in range(batch):
        for k in range(c):
            for i in range(oh):
                for j in range(ow):
                    best, bi = -np.finfo(np.float32).max, -1
                    for n in range(size):
                        for m in range(size):
                            y_, x_ = off + i * stride + n, off + j * stride + m
                            if 0 <= y_ < h and 0 <= x_ < w and X[b, k, y_, x_] > best:
                                best, bi = X[b, k, y_, x_], ((b * c + k) * h + y_) * w + x_
                    out[b, k, i, j], idx[b, k, i, j] = best, bi
    return out.ravel(), idx.ravel()


@pytest.mark.parametrize("case", [(2, 3, 6, 6, 2, 2, 1), (1, 2, 7, 5, 3, 2, 2), (1, 1, 5, 5, 3, 1, 2), (2, 2, 4, 4, 2, 2, 0)])
def test_maxpool_brute_force(case):
    batch, c, h, w, size, stride, pad = case
    g = r(sum(case))
    x = g.integers(-3, 4, batch * c * h * w).astype(np.float32)  # many ties
    x[0] = np.nan
    oh, ow = ref.maxpool_out_dim(h, size, stride, pad), ref.maxpool_out_dim(w, size, stride, pad)
    out, idx = np.empty(batch * c * oh * ow, np.float32), np.empty(batch * c * oh * ow, np.int32)
    ref.forwardMaxpool(batch, h, w, c, size, stride, pad, x, out, idx)
    bo, bi = maxpool_brute(x, batch, c, h, w, size, stride, pad)
    assert np.array_equal(out, bo) and np.array_equal(idx, bi)
    d = g.normal(0, 1, out.size).astype(np.float32)
    prev = np.zeros_like(x)
    ref.backwardMaxpool(idx, d, prev)
    want = np.zeros(x.size, np.float64)
    np.add.at(want, idx[idx >= 0], d[idx >= 0].astype(np.float64))
    np.testing.assert_allclose(prev, want, rtol=1e-6, atol=1e-6)


def test_maxpool_empty_window_index():
    # a window of all NaN never passes '>' against -FLT_MAX: index -1, value -FLT_MAX
    x = np.full(16, np.nan, np.float32)
    out, idx = np.empty(4, np.float32), np.empty(4, np.int32)
    ref.forwardMaxpool(1, 4, 4, 1, 2, 2, 0, x, out, idx)
    assert np.all(idx == -1) and np.all(out == -np.finfo(np.float32).max)


def test_avgpool():
    batch, c, h, w = 2, 3, 5, 4
    g = r(12)
    x = g.normal(0, 1, batch * c * h * w).astype(np.float32)
    out = np.empty(batch * c, np.float32)
    ref.forwardAvgpool(batch, w, h, c, x, out)
    np.testing.assert_allclose(out, x.astype(np.float64).reshape(batch * c, h * w).mean(axis=1), rtol=1e-5, atol=1e-7)
    od = g.normal(0, 1, batch * c).astype(np.float32)
    prev = np.zeros_like(x)
    ref.backwardAvgpool(batch, w, h, c, od, prev)
    assert np.array_equal(prev.reshape(batch * c, h * w), np.repeat((od / f32(h * w))[:, None], h * w, axis=1))


# ---------------------------------------------------------------------------
# std.math.pow (blas.zig:176) -- parity at the bit level is unpinned
# ---------------------------------------------------------------------------


def test_pow_closed_forms():
    assert ref.pow_f32(4.0, -1.5) == 0.125
    assert ref.pow_f32(0.25, -1.5) == 8.0
    assert ref.pow_f32(2.0, 10.0) == 1024.0
    assert ref.pow_f32(9.0, 0.5) == 3.0
    assert ref.pow_f32(5.0, 0.0) == 1.0 and ref.pow_f32(1.0, float("nan")) == 1.0
    assert math.isnan(ref.pow_f32(-2.0, 1.5))


def test_pow_m15_close_to_f64():
    v = r(13).uniform(1e-5, 50, 20000).astype(np.float32)
    got = np.array([ref.pow_f32(float(a), -1.5) for a in v], np.float32)
    want = v.astype(np.float64) ** -1.5
    assert np.max(np.abs(got - want) / want) < 4 * 2.0**-23
