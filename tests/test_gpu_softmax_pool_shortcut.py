"""GPU parity of softmax, max/avg pooling and the shortcut.

Softmax: contiguous groups longer than 32 (gputest.zig:252-279's 8x137,
config 3's [256,1000] with logits ~N(0,4), every kernel geometry) are held to
the 1e-5 rule against the twin, within 1e-6 of the f64 softmax of the twin's
own exp arguments, with rows summing to 1; groups of at most 32 and strided
groups (spatial softmax) keep the twin's sequential sum and are bit-exact.
Maxpool: output bit-exact, indexes bit-exact (IX), backward bit-exact.
Avgpool: forward within 1e-5 (row sums), backward bit-exact. Shortcut:
bit-exact on the same-shape, stride, upsample and channel-mismatch paths.
"""

from __future__ import annotations

import numpy as np
import pytest

from darknet_zig_amd import gpu
from oracle import ref
from tests.helpers import (assert_bitexact, assert_r5, assert_softmax, down, normal, rng, softmax_f64, uniform,
                           up)

pytestmark = pytest.mark.gpu


def _softmax_case(x, n, batch, batch_offset, groups, group_offset, stride, temp):
    cpu = np.zeros_like(x)
    ref.softmax(x, n, batch, batch_offset, groups, group_offset, stride, temp, cpu)
    dx, dout = up(x), up(np.zeros_like(x))
    gpu.softmax(dx, n, batch, batch_offset, groups, group_offset, stride, temp, dout)
    got = down(dout, x)
    gpu.free(dx)
    gpu.free(dout)
    return got, cpu


@pytest.mark.parametrize(
    "batch, classes, sigma, temp",
    [(8, 137, 1.0, 1.0), (256, 1000, 4.0, 1.0), (3, 33, 10.0, 0.5), (5, 8192, 2.0, 1.0), (4, 40, 1.0, 2.0),
     # one workgroup per group (fewer than 1024 groups): 64..1024 lanes,
     # 4..32 floats a lane, float4 or per-element layout
     (7, 2048, 3.0, 1.0), (2, 4097, 3.0, 1.0), (3, 16384, 2.0, 0.7), (2, 32768, 3.0, 1.0), (2, 30001, 2.0, 1.0),
     # more than 32768: three passes over the group
     (2, 40000, 3.0, 1.0), (1, 100003, 2.0, 1.3),
     # segments of 4, 8, 16, 32 and 64 lanes (at least 1024 groups), the last
     # workgroup partial; one or four segments' waves a workgroup
     (1024, 64, 2.0, 1.0), (5000, 37, 2.0, 0.7), (1100, 61, 3.0, 1.0), (4104, 100, 3.0, 1.0),
     (4096, 128, 4.0, 1.0), (4096, 256, 4.0, 1.0), (1031, 255, 4.0, 1.0), (2049, 500, 3.0, 1.0),
     (3000, 333, 2.0, 1.0), (4096, 257, 3.0, 1.0), (4096, 1000, 4.0, 1.0), (4100, 300, 3.0, 1.0),
     (4097, 777, 2.0, 0.7), (4100, 1024, 3.0, 1.0), (8195, 1021, 2.0, 1.0), (8200, 1000, 4.0, 1.0),
     (1030, 1500, 3.0, 1.0), (2048, 2048, 3.0, 1.0), (1025, 2047, 2.0, 1.0)],
)
def test_softmax_rows(dev, batch, classes, sigma, temp):
    x = normal(rng(classes + batch), batch * classes, 0, sigma)
    got, cpu = _softmax_case(x, classes, batch, classes, 1, classes, 1, temp)
    p64 = softmax_f64(x, classes, batch, classes, 1, classes, 1, temp)
    assert_softmax(got, cpu, p64, f"softmax {batch}x{classes}")
    np.testing.assert_allclose(got.reshape(batch, classes).sum(axis=1, dtype=np.float64), 1.0, rtol=2e-6)


@pytest.mark.parametrize("batch, classes, sigma, temp", [(17, 1, 1.0, 1.0), (4, 5, 1.0, 2.0), (300, 32, 3.0, 1.0),
                                                         (1500, 7, 2.0, 0.5)])
def test_softmax_short_rows_bitexact(dev, batch, classes, sigma, temp):
    """Groups of at most 32: one lane per group runs the twin's loops (with
    the host-libm-identical exp), bit for bit."""
    x = normal(rng(classes + batch), batch * classes, 0, sigma)
    got, cpu = _softmax_case(x, classes, batch, classes, 1, classes, 1, temp)
    assert_bitexact(got, cpu, f"softmax {batch}x{classes}")


@pytest.mark.parametrize("batch, batch_offset, groups, group_offset, n",
                         [(3, 1000, 4, 250, 250), (5, 1200, 2, 600, 500), (1100, 130, 2, 64, 60),
                          (2, 4100, 2, 2050, 2049), (1200, 203, 1, 0, 201)])
def test_softmax_grouped_and_gapped(dev, batch, batch_offset, groups, group_offset, n):
    """Contiguous groups inside a larger batch stride (gaps between groups
    must stay untouched) and several groups per batch item; odd offsets take
    the per-element layout."""
    size = (batch - 1) * batch_offset + (groups - 1) * group_offset + n
    r = rng(n + groups)
    x = normal(r, size, 0, 3.0)
    cpu = np.full(size, -7.0, np.float32)
    ref.softmax(x, n, batch, batch_offset, groups, group_offset, 1, 1.0, cpu)
    dx, dout = up(x), up(np.full(size, -7.0, np.float32))
    gpu.softmax(dx, n, batch, batch_offset, groups, group_offset, 1, 1.0, dout)
    got = down(dout, x)
    gpu.free(dx)
    gpu.free(dout)
    p64 = softmax_f64(x, n, batch, batch_offset, groups, group_offset, 1, 1.0)
    inside = ~np.isnan(p64)
    assert np.all(got[~inside] == -7.0), "elements outside the groups were written"
    assert_softmax(got[inside], cpu[inside], p64[inside], f"softmax groups {batch}x{groups}x{n}")


def test_softmax_special_values(dev):
    """Rows with -inf entries (probability 0), a NaN (the whole row NaN, as
    the twin's sum becomes NaN), +inf (NaN through inf - inf), all equal
    entries (uniform), and a huge spread (probabilities that underflow to
    subnormals and to zero)."""
    classes = 100
    rows = [np.zeros(classes, np.float32) for _ in range(6)]
    rows[0][::3] = -np.inf
    rows[1][:] = np.linspace(-3, 3, classes)
    rows[1][17] = np.nan
    rows[2][5] = np.inf
    rows[3][:] = 2.5
    rows[4][:] = np.linspace(-120, 0, classes)
    rows[5][:] = np.linspace(-1e30, 1e30, classes)
    batch = 1024  # the segment kernel; the rows repeat
    x = np.concatenate([rows[i % len(rows)] for i in range(batch)]).astype(np.float32)
    for b in (batch, 6):  # segment and workgroup kernels
        got, cpu = _softmax_case(x[:b * classes], classes, b, classes, 1, classes, 1, 1.0)
        nan_g, nan_c = np.isnan(got), np.isnan(cpu)
        np.testing.assert_array_equal(nan_g, nan_c)
        p64 = softmax_f64(x[:b * classes], classes, b, classes, 1, classes, 1, 1.0)
        assert_softmax(got[~nan_c], cpu[~nan_c], p64[~nan_c], f"special values ({b} rows)")
        assert np.all(got[~nan_c] >= 0)


@pytest.mark.parametrize("b, c, s", [(2, 11, 49), (3, 85, 169), (2, 128, 65), (2, 130, 13), (1, 1, 7),
                                     (64, 85, 169), (100, 20, 196), (256, 5, 169)])
def test_softmax_spatial_groups(dev, b, c, s):
    # Spatial softmax: groups = positions, elements `spatial` apart
    # (n = channels, batch_offset = c*s, groups = s, group_offset = 1, stride = s).
    # Up to 128 channels the groups go through the LDS tile kernel (8, 16, 32
    # or 64 groups per workgroup by the group count: the last three cases take
    # 16, 32 and 64; the last tile partial); above, one lane per group.
    x = normal(rng(11 + c + s), b * c * s, 0, 2.0)
    got, cpu = _softmax_case(x, c, b, c * s, s, 1, s, 1.0)
    assert_bitexact(got, cpu, f"spatial softmax {b}x{c}x{s}")
    np.testing.assert_allclose(got.reshape(b, c, s).sum(axis=1), 1.0, rtol=1e-5)


def test_softmax_then_xent_config3(dev):
    """Config 3: logits [256,1000] ~N(0,4), one-hot labels; p to the 1e-5
    rule, then softmax_x_ent's delta = t - p bit-exact given the same p,
    summing to 0 per row."""
    batch, classes = 256, 1000
    r = rng(3)
    x = normal(r, batch * classes, 0, 4.0)
    truth = np.zeros(batch * classes, np.float32)
    truth[np.arange(batch) * classes + r.integers(0, classes, batch)] = 1.0
    got, cpu = _softmax_case(x, classes, batch, classes, 1, classes, 1, 1.0)
    assert_softmax(got, cpu, softmax_f64(x, classes, batch, classes, 1, classes, 1, 1.0), "softmax cfg3")
    # softmax_x_ent on the device's probabilities, against the twin's on the same ones
    d_c, e_c = np.empty_like(x), np.empty_like(x)
    ref.softmaxCrossEntropy(got, truth, d_c, e_c)
    dp, dt, dd, de = up(got), up(truth), gpu.alloc(x.size), gpu.alloc(x.size)
    gpu.softmaxCrossEntropy(x.size, dp, dt, dd, de)
    d = down(dd, x)
    assert_bitexact(d, d_c, "xent delta")
    np.testing.assert_allclose(d.reshape(batch, classes).sum(axis=1), 0.0, atol=1e-5)
    e64 = np.where(truth != 0, -np.log(got.astype(np.float64)), 0.0)
    assert_r5(down(de, x), e_c, e64, "xent loss")
    for bb in (dp, dt, dd, de):
        gpu.free(bb)


MAXPOOL_CASES = [
    # batch, c, h, w, size, stride, pad
    (3, 6, 14, 14, 2, 2, 1),      # gputest.zig:393-399 (generic path: w % 4 != 0)
    (2, 3, 8, 8, 2, 2, 1),        # 2x2 fast path
    (2, 3, 8, 8, 2, 2, 0),        # fast path, pad 0
    (2, 4, 13, 13, 2, 2, 1),      # odd input: last column dropped
    (2, 3, 9, 11, 3, 2, 2),       # overlapping windows, several contributors
    (1, 2, 7, 7, 3, 1, 2),        # darknet size=3 stride=1 (default pad size-1)
    (2, 2, 6, 10, 5, 3, 4),
    (256, 512, 28, 28, 2, 2, 1),  # config 5
    # at least 256 planes: planes in LDS -- the separable forward and the stride-1
    # gather where a plane's rows fit, else one workgroup a plane:
    (8, 64, 56, 56, 3, 2, 2),     # generic forward, float4 loads
    (86, 3, 9, 9, 2, 1, 1),       # plane of 81 floats: element loads
    (86, 3, 9, 9, 3, 1, 2),       # stride-1 backward through LDS, odd plane
    (64, 4, 13, 13, 13, 1, 12),   # spatial pyramid pooling's 13x13 window
    (86, 3, 110, 110, 3, 2, 2),   # the largest planes held in LDS (12100 floats)
    (86, 3, 78, 78, 3, 1, 2),     # stride-1 backward: the largest output planes held in LDS (6084)
    # the same windows on fewer planes, or larger ones: per-output / per-input kernels
    (2, 3, 9, 9, 2, 1, 1),
    (2, 3, 9, 9, 3, 1, 2),
    (2, 4, 13, 13, 13, 1, 12),
    (2, 3, 110, 110, 3, 2, 2),
    (2, 3, 120, 120, 3, 2, 2),    # larger planes: one lane per output
    (2, 3, 78, 78, 3, 1, 2),
    (1, 2, 80, 80, 3, 1, 2),      # larger: one lane per input
    # 3x3 stride 2 with w == 2*ow, ow % 4 == 0: four outputs a lane forward,
    # eight inputs a lane backward, window offset -1 or 0
    (64, 128, 56, 56, 3, 2, 2),   # the bench's generic pool shape
    (2, 3, 16, 24, 3, 2, 1),      # offset 0
    (3, 5, 10, 8, 3, 2, 2),       # one lane per output row
    (2, 4, 7, 16, 3, 2, 2),       # odd height: the last window row clamped
    (2, 2, 9, 8, 3, 2, 1),        # offset 0, odd height
    (1, 1, 1, 8, 3, 2, 2),        # one input row: rows -1 and 1 outside
    (2, 3, 8, 12, 3, 2, 2),       # ow = 6: not a multiple of 4, the generic kernels
    # several planes a workgroup (separable forward for windows of 4 and more,
    # stride-1 gather backward for windows of 3 and more); the last workgroup
    # holds fewer planes
    (19, 79, 13, 13, 5, 1, 4),    # 2 planes a workgroup, 751 workgroups
    (37, 83, 9, 9, 5, 1, 4),      # 5 planes of 81 floats: element loads
    (37, 83, 9, 9, 3, 1, 2),      # the gather alone
    (3, 683, 13, 13, 4, 1, 3),    # 4 planes: float4 loads, the last plane's tail in elements
    (16, 64, 6, 6, 4, 1, 11),     # windows wholly outside the input: index -1
    (16, 64, 9, 11, 5, 2, 4),     # stride 2
    (32, 40, 11, 11, 7, 1, 6),    # a window size not compiled into the runs-a-lane kernels
    (16, 64, 15, 15, 6, 1, 5),    # the block forward at every compiled size: 6, 8, 10, 11, 12
    (16, 64, 15, 15, 8, 1, 7),
    (16, 64, 14, 14, 10, 1, 9),
    (16, 64, 15, 15, 11, 1, 10),
    (8, 64, 13, 13, 12, 1, 11),
    (4, 512, 13, 13, 2, 1, 1),    # a tiny-YOLO [maxpool] size=2 stride=1: the 2x2 gather, 4 planes a workgroup
    (2, 128, 60, 60, 7, 1, 6),    # planes too large for the targets-only backward: the gather without runs
    (2, 128, 60, 60, 5, 1, 4),    # the same with runs of inputs a lane
    (41, 50, 7, 7, 2, 1, 1),      # 2x2/s1 with the last workgroup's planes ragged
    (8, 512, 19, 19, 13, 1, 12),  # spatial pyramid pooling's 13x13 window, 5 planes a workgroup
    (8, 512, 19, 19, 9, 1, 8),
]


@pytest.mark.parametrize("case", MAXPOOL_CASES, ids=str)
def test_maxpool(dev, case):
    batch, c, h, w, size, stride, pad = case
    oh, ow = ref.maxpool_out_dim(h, size, stride, pad), ref.maxpool_out_dim(w, size, stride, pad)
    r = rng(sum(case))
    x = uniform(r, batch * c * h * w)
    if batch * c * h * w < 10000:
        x[::7] = np.float32(0.25)  # ties: the first maximum must win
        x[3] = np.nan
        x[5] = -np.inf
    out_n = batch * c * oh * ow
    out_c, idx_c = np.empty(out_n, np.float32), np.empty(out_n, np.int32)
    ref.forwardMaxpool(batch, h, w, c, size, stride, pad, x, out_c, idx_c)
    dx, dout, didx = up(x), gpu.alloc(out_n), gpu.allocInts(out_n)
    gpu.forwardMaxpool(out_n, h, w, c, stride, size, pad, dx, dout, didx)
    assert_bitexact(down(dout, out_c), out_c, f"maxpool fwd {case}")
    assert_bitexact(down(didx, idx_c), idx_c, f"maxpool idx {case}")

    delta = uniform(r, out_n)
    prev = uniform(r, x.size) if x.size < 10**6 else np.zeros_like(x)
    prev_c = prev.copy()
    ref.backwardMaxpool(idx_c, delta, prev_c)
    dd, dprev = up(delta), up(prev)
    gpu.backwardMaxpool(x.size, h, w, c, stride, size, pad, dd, dprev, didx)
    got = down(dprev, prev)
    assert_bitexact(got, prev_c, f"maxpool bwd {case}")
    if stride >= size:  # at most one contributor per input: the delta is conserved
        np.testing.assert_allclose(got.astype(np.float64).sum() - prev.astype(np.float64).sum(),
                                   delta[idx_c >= 0].astype(np.float64).sum(), rtol=1e-4, atol=1e-3)
    for b in (dx, dout, didx, dd, dprev):
        gpu.free(b)


def _shared_peaks(batch, c, h, w, size, stride, pad, seed):
    """Input whose large values sit on the rows and columns that two or more
    windows share: a peak above its neighbours is then the argmax of every
    window that holds it."""
    r = rng(seed)
    x = uniform(r, (batch, c, h, w), -1.0, 0.0)
    hp = pad // 2

    def shared(n, on):
        cover = np.zeros(n, int)
        for i in range(on):
            lo = i * stride - hp
            cover[max(lo, 0):max(min(lo + size, n), 0)] += 1
        return cover >= 2

    rows = shared(h, ref.maxpool_out_dim(h, size, stride, pad))
    cols = shared(w, ref.maxpool_out_dim(w, size, stride, pad))
    mask = rows[:, None] & cols[None, :]
    x[:, :, mask] = uniform(r, (batch, c, int(mask.sum())), 1.0, 2.0)
    return x.ravel()


@pytest.mark.parametrize("case", [(2, 3, 11, 13, 3, 2, 2), (2, 2, 12, 12, 5, 3, 4), (1, 2, 9, 9, 3, 1, 2),
                                  (2, 2, 10, 10, 4, 2, 2), (1, 2, 122, 122, 3, 2, 2), (86, 3, 11, 13, 3, 2, 2),
                                  (64, 4, 12, 12, 5, 3, 4), (86, 3, 9, 9, 3, 1, 2), (1, 2, 120, 120, 3, 2, 2),
                                  (2, 3, 16, 16, 3, 2, 2), (1, 2, 12, 24, 3, 2, 1), (128, 9, 9, 9, 3, 1, 2),
                                  (128, 9, 11, 11, 5, 1, 4), (41, 50, 7, 7, 4, 1, 3), (64, 20, 12, 12, 7, 1, 6),
                                  (41, 50, 7, 7, 2, 1, 1)], ids=str)
def test_maxpool_shared_argmax(dev, case):
    """Inputs that are the argmax of several outputs: the backward pass must
    add their deltas in ascending output order -- the output-per-lane kernel
    for stride >= 2 (few planes, or planes too large for LDS: 122x122), the
    plane-in-LDS kernels for at least 256 planes, the gather kernels for
    stride 1 (several planes a workgroup from 1024 planes), and the eight-inputs-a-lane 3x3/s2 kernel (120x120, 16x16,
    12x24 with offset 0)."""
    batch, c, h, w, size, stride, pad = case
    oh, ow = ref.maxpool_out_dim(h, size, stride, pad), ref.maxpool_out_dim(w, size, stride, pad)
    x = _shared_peaks(*case, seed=sum(case))
    out_n = batch * c * oh * ow
    out_c, idx_c = np.empty(out_n, np.float32), np.empty(out_n, np.int32)
    ref.forwardMaxpool(batch, h, w, c, size, stride, pad, x, out_c, idx_c)
    counts = np.bincount(idx_c[idx_c >= 0], minlength=x.size)
    assert counts.max() >= 2, "the case must have inputs with several contributors"
    dx, dout, didx = up(x), gpu.alloc(out_n), gpu.allocInts(out_n)
    gpu.forwardMaxpool(out_n, h, w, c, stride, size, pad, dx, dout, didx)
    assert_bitexact(down(didx, idx_c), idx_c, f"maxpool idx {case}")
    r = rng(sum(case))
    # magnitudes over six decades, so that adding a shared input's deltas in
    # another order changes the rounded result
    delta = (normal(r, out_n) * np.float32(10.0) ** uniform(r, out_n, -3, 3)).astype(np.float32)
    prev = normal(r, x.size)
    prev_c = prev.copy()
    ref.backwardMaxpool(idx_c, delta, prev_c)
    dd, dprev = up(delta), up(prev)
    gpu.backwardMaxpool(x.size, h, w, c, stride, size, pad, dd, dprev, didx)
    assert_bitexact(down(dprev, prev), prev_c, f"maxpool bwd shared argmax {case}")
    for b in (dx, dout, didx, dd, dprev):
        gpu.free(b)


# rows of 1, 30, 49, 110 elements take 4, 8, 16, 32 lanes a row; 169, 196, 323, 784 a wave a row
@pytest.mark.parametrize("batch, c, h, w", [(3, 6, 14, 14), (2, 5, 7, 7), (4, 3, 1, 1), (8, 64, 13, 13),
                                        (2, 3, 17, 19), (2, 4, 5, 6), (3, 10, 10, 11), (64, 1024, 7, 7),
                                        (256, 512, 28, 28)])
def test_avgpool(dev, batch, c, h, w):
    r = rng(batch * c + h)
    x = uniform(r, batch * c * h * w)
    n = batch * c
    out_c = np.empty(n, np.float32)
    ref.forwardAvgpool(batch, w, h, c, x, out_c)
    dx, dout = up(x), gpu.alloc(n)
    gpu.forwardAvgpool(n, w, h, c, dx, dout)
    x64 = x.astype(np.float64).reshape(n, h * w)
    assert_r5(down(dout, out_c), out_c, x64.sum(axis=1) / (h * w), f"avgpool fwd {(batch, c, h, w)}")

    od = uniform(r, n)
    prev = uniform(r, x.size)
    prev_c = prev.copy()
    ref.backwardAvgpool(batch, w, h, c, od, prev_c)
    dod, dprev = up(od), up(prev)
    gpu.backwardAvgpool(n, w, h, c, dprev, dod)
    assert_bitexact(down(dprev, prev), prev_c, f"avgpool bwd {(batch, c, h, w)}")
    for b in (dx, dout, dod, dprev):
        gpu.free(b)


SHORTCUT_CASES = [
    # batch, w1, h1, c1 (add), w2, h2, c2 (out), s1, s2
    (2, 8, 8, 4, 8, 8, 4, 1.0, 1.0),          # gputest.zig:453-480
    (64, 28, 28, 256, 14, 14, 512, 1.0, 1.0), # config 4: stride 2, channel mismatch
    (3, 14, 14, 8, 7, 7, 8, 0.5, 2.0),        # stride 2, odd output width (generic)
    (2, 7, 7, 6, 14, 14, 3, 1.0, -0.75),      # upsample: sample 2
    (2, 9, 9, 5, 4, 4, 5, 0.9, 1.1),          # w1/w2 = 2 with remainder
    (1, 5, 5, 3, 5, 5, 9, 2.0, 1.0),          # channel mismatch only
    # the stride-2 pair path: pair counts off the 1024-pair workgroup tile,
    # add with more channels than out, heights that do not halve exactly
    (3, 16, 16, 8, 8, 8, 8, 0.5, 2.0),        # 768 pairs: one partial tile
    (5, 12, 11, 7, 6, 5, 3, -1.0, 0.25),      # minc = c2, h1 = 2*h2 + 1
    (7, 28, 28, 33, 14, 14, 40, 1.0, 1.0),    # 22638 pairs, ragged last tile
    (1, 4, 4, 1, 2, 2, 1, 1.0, 1.0),          # a single pair
]


@pytest.mark.parametrize("case", SHORTCUT_CASES, ids=str)
def test_shortcut(dev, case):
    batch, w1, h1, c1, w2, h2, c2, s1, s2 = case
    r = rng(sum(case[:7]))
    add, out = normal(r, batch * c1 * h1 * w1, 0, 0.05), normal(r, batch * c2 * h2 * w2, 0, 0.05)
    cpu = out.copy()
    ref.shortcut(batch, w1, h1, c1, add, w2, h2, c2, s1, s2, cpu)
    da, do = up(add), up(out)
    gpu.shortcut(batch, w1, h1, c1, da, w2, h2, c2, s1, s2, do)
    assert_bitexact(down(do, out), cpu, f"shortcut {case}")
    if case[1:4] == case[4:7] and s1 == s2 == 1.0:  # same shape: exact addition
        assert_bitexact(cpu, (out + add).astype(np.float32), "shortcut == add")
    gpu.free(da)
    gpu.free(do)
