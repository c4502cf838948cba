"""GPU parity of dkz_softmax_layer_forward, the softmax layer's forward step
(layers/misc.zig:63-76: softmax, then the cross-entropy loss when truth is
given) as one call, against the CPU twins run in the layer's order
(blas.zig:213-252): the probabilities and the delta bit-exact, the loss
(-log p) within 1e-5 of the twin or closer to f64 (the device log against the
host libm's).

Cases: config 3 ([256,1000], logits ~N(0,4), one-hot labels), grouped rows,
rows whose length is not a multiple of 4, short groups (the one-lane path
plus a separate loss pass), misaligned views, a temperature, no truth (no
loss), and label-smoothed (dense) truth.
"""

from __future__ import annotations

import numpy as np
import pytest

from darknet_zig_amd import gpu
from oracle import ref
from tests.helpers import assert_bitexact, assert_r5, down, normal, rng, up

pytestmark = pytest.mark.gpu


def _cpu(x, truth, batch, inputs, groups, temp):
    per = inputs // groups
    p = np.zeros_like(x)
    ref.softmax(x, per, batch, inputs, groups, per, 1, temp, p)
    if truth is None:
        return p, None, None
    d, e = np.empty_like(x), np.empty_like(x)
    ref.softmaxCrossEntropy(p, truth, d, e)
    return p, d, e


def _views(arrays, offset):
    """Uploads each array at an element offset; returns (whole, view) pairs."""
    out = []
    for a in arrays:
        w = up(np.concatenate([np.zeros(offset, np.float32), a]))
        out.append((w, w.offset(offset)))
    return out


def _run(x, truth, batch, inputs, groups, temp, offset=0):
    n = x.size
    bufs = _views([x, truth if truth is not None else np.zeros(n, np.float32), np.zeros(n, np.float32),
                   np.zeros(n, np.float32), np.zeros(n, np.float32)], offset)
    (wx, vx), (wt, vt), (wo, vo), (wd, vd), (we, ve) = bufs
    gpu.softmaxLayerForward(batch, inputs, groups, temp, vx, vt if truth is not None else None, vo,
                            vd if truth is not None else None, ve if truth is not None else None)
    res = []
    for w in (wo, wd, we):
        h = np.empty(n + offset, np.float32)
        gpu.pull(w, h)
        res.append(h[offset:])
    for w, _ in bufs:
        gpu.free(w)
    return res


def _check(x, truth, batch, inputs, groups, temp, offset=0, name=""):
    p_c, d_c, e_c = _cpu(x, truth, batch, inputs, groups, temp)
    p, d, e = _run(x, truth, batch, inputs, groups, temp, offset)
    assert_bitexact(p, p_c, f"p {name}")
    if truth is None:
        assert np.all(d == 0) and np.all(e == 0), "no truth: delta and loss untouched"
        return
    assert_bitexact(d, d_c, f"delta {name}")
    e64 = np.where(truth != 0, -np.log(p_c.astype(np.float64)), 0.0)
    assert_r5(e, e_c, e64, f"loss {name}")


def _one_hot(r, batch, classes):
    t = np.zeros(batch * classes, np.float32)
    t[np.arange(batch) * classes + r.integers(0, classes, batch)] = 1.0
    return t


def test_config3_one_pass(dev):
    batch, classes = 256, 1000
    r = rng(3)
    x = normal(r, batch * classes, 0, 4.0)
    _check(x, _one_hot(r, batch, classes), batch, classes, 1, 1.0, name="cfg3")


@pytest.mark.parametrize("batch,inputs,groups,temp", [
    (8, 137, 1, 1.0),  # gputest.zig:252-279's rows: not a multiple of 4
    (4, 1000, 4, 1.0),  # four groups of 250
    (3, 96, 3, 0.5),  # 32-long groups: the one-lane path, then a separate loss pass
    (5, 40, 2, 2.0),
    (2, 8192, 1, 1.0),  # the longest row staged in LDS
    (2, 12000, 1, 1.0),  # longer: the f64-sum path
    # at least 2048 rows of 257..1024 held in registers, 2, 4 or 8 a
    # workgroup, the last tile partial; float4 and per-element layouts
    (2051, 1000, 1, 1.0),
    (4096, 1000, 1, 1.0),
    (4101, 600, 2, 0.7),
    (4097, 777, 1, 1.0),
    (4100, 1024, 1, 1.0),
])
def test_shapes(dev, batch, inputs, groups, temp):
    r = rng(batch * inputs + groups)
    x = normal(r, batch * inputs, 0, 3.0)
    t = np.zeros(batch * inputs, np.float32)
    per = inputs // groups
    for b in range(batch):
        for g in range(groups):
            t[b * inputs + g * per + r.integers(0, per)] = 1.0
    if inputs > 8192:
        p_c, d_c, e_c = _cpu(x, t, batch, inputs, groups, temp)
        p, d, e = _run(x, t, batch, inputs, groups, temp)
        xr = x.astype(np.float64).reshape(batch, inputs) / temp
        ex = np.exp(xr - xr.max(axis=1, keepdims=True))
        assert_r5(p, p_c, (ex / ex.sum(axis=1, keepdims=True)).ravel(), "p long rows")
        np.testing.assert_array_equal(d, t - p)  # softmax_x_ent's delta on the stored p
        return
    _check(x, t, batch, inputs, groups, temp, name=f"{batch}x{inputs}/{groups}")


@pytest.mark.parametrize("offset,batch", [(1, 6), (2, 6), (1, 4100)])
def test_misaligned_views(dev, offset, batch):
    classes = 500
    r = rng(offset)
    x = normal(r, batch * classes, 0, 2.0)
    _check(x, _one_hot(r, batch, classes), batch, classes, 1, 1.0, offset, name=f"offset {offset}, {batch} rows")


def test_no_truth_is_softmax_only(dev):
    batch, classes = 16, 1000
    x = normal(rng(9), batch * classes, 0, 4.0)
    _check(x, None, batch, classes, 1, 1.0, name="no truth")


def test_label_smoothed_truth(dev):
    """misc.zig:186-188 smooths the truth in place (scal, add_scalar): every
    element has t != 0, so every loss element is -log(p)."""
    batch, classes = 32, 1000
    r = rng(10)
    x = normal(r, batch * classes, 0, 4.0)
    t = _one_hot(r, batch, classes)
    ref.scal(1 - 0.1, t)
    ref.addScalar(np.float32(0.1) / np.float32(classes), t)
    _check(x, t, batch, classes, 1, 1.0, name="smoothed")


def test_equals_the_two_calls(dev):
    """The fused call against gpu.softmax + gpu.softmaxCrossEntropy on the
    device, config 3."""
    batch, classes = 256, 1000
    r = rng(33)
    x = normal(r, batch * classes, 0, 4.0)
    t = _one_hot(r, batch, classes)
    n = x.size
    dx, dt = up(x), up(t)
    p1, d1, e1 = gpu.alloc(n), gpu.alloc(n), gpu.alloc(n)
    gpu.softmax(dx, classes, batch, classes, 1, classes, 1, 1.0, p1)
    gpu.softmaxCrossEntropy(n, p1, dt, d1, e1)
    p2, d2, e2 = gpu.alloc(n), gpu.alloc(n), gpu.alloc(n)
    gpu.softmaxLayerForward(batch, classes, 1, 1.0, dx, dt, p2, d2, e2)
    for a, b, name in ((p1, p2, "p"), (d1, d2, "delta"), (e1, e2, "loss")):
        assert_bitexact(down(b, x), down(a, x), f"fused vs two calls: {name}")
    for b in (dx, dt, p1, d1, e1, p2, d2, e2):
        gpu.free(b)
