"""GPU parity of dkz_softmax_layer_forward, the softmax layer's forward step
(layers/misc.zig:63-76: softmax, then the cross-entropy loss when truth is
given) as one call, against the CPU twins run in the layer's order
(blas.zig:213-252): the probabilities to the softmax rule (1e-5 of the twin,
1e-6 of the f64 softmax), the delta bit-exact given the same probabilities
(the twin's softmax_x_ent run on the device's p), the loss (-log p) within
1e-5 of the twin or closer to f64 (the device log against the host libm's).

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
from tests.helpers import assert_bitexact, assert_r5, assert_softmax, down, normal, rng, softmax_f64, up

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
    p_c, _, _ = _cpu(x, None, batch, inputs, groups, temp)
    p, d, e = _run(x, truth, batch, inputs, groups, temp, offset)
    per = inputs // groups
    p64 = softmax_f64(x, per, batch, inputs, groups, per, 1, temp)
    if per <= 32:
        assert_bitexact(p, p_c, f"p {name}")  # the one-lane kernel
    else:
        assert_softmax(p, p_c, p64, f"p {name}")
    if truth is None:
        assert np.all(d == 0) and np.all(e == 0), "no truth: delta and loss untouched"
        return
    d_c, e_c = np.empty_like(x), np.empty_like(x)
    ref.softmaxCrossEntropy(p, truth, d_c, e_c)  # the twin's loss step on the device's p
    assert_bitexact(d, d_c, f"delta {name}")
    e64 = np.where(truth != 0, -np.log(p.astype(np.float64)), 0.0)
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
    (2, 8192, 1, 1.0),  # one workgroup per group, in registers
    (2, 12000, 1, 1.0),
    (2, 33000, 1, 1.0),  # longer than a workgroup holds: three passes
    (3, 40002, 2, 0.7),
    # at least 1024 groups: segments of 4..64 lanes, the last workgroup
    # partial; float4 and per-element layouts
    (1024, 40, 1, 1.0),
    (1500, 240, 2, 1.0),
    (2051, 1000, 1, 1.0),
    (1030, 1800, 1, 1.0),
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


@pytest.mark.parametrize("batch, classes", [(256, 1000), (4096, 1000), (2000, 100), (3, 20000)])
def test_equals_the_two_calls(dev, batch, classes):
    """The fused call against gpu.softmax + gpu.softmaxCrossEntropy on the
    device (config 3, and the segment, workgroup and long-group kernels):
    identical bits."""
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
