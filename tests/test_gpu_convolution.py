"""dkz_convolution_forward, dkz_convolution_weight_gradient and
dkz_convolution_data_gradient: the per-image im2col + gemm (+ col2im) loops
of a convolutional layer's forward (layers/convolutional.zig:240-260),
weight gradient (:288-297) and data gradient (:299-305) as single products,
the im2col operand (of the input, or of delta) gathered inside them.

Reference per image i and group j: the oracle's im2col of the image (a copy,
bit-exact) times the group's weights in f64, added to the output's previous
contents. Tolerance per element as for dkz_gemm: Higham's bound
gamma_(k+3) * (sum_p |w_p col_p| + |out0|). For ksize 1 the layer multiplies
by the input itself, read as a k x n matrix; so does the entry point, also
where that reading is the layer's own (stride 2 with ksize 1)."""

from __future__ import annotations

import numpy as np
import pytest

from darknet_zig_amd import gpu
from oracle import ref
from tests.helpers import col2im64, down, rng, up

pytestmark = pytest.mark.gpu

U = 2.0 ** -24

CASES = [
    # batch, groups, channels, height, width, filters, ksize, stride, pad
    (2, 1, 16, 16, 16, 32, 3, 1, 1),   # stride 1, widths % 4 == 0: two-block gathers
    (3, 2, 8, 10, 12, 6, 3, 2, 1),     # groups, stride 2: per-element gathers
    (2, 1, 4, 9, 9, 5, 1, 1, 0),       # ksize 1: the input is the operand
    (1, 1, 3, 8, 8, 4, 1, 2, 0),       # ksize 1, stride 2: the layer's own reading of the input
    (4, 1, 32, 28, 28, 64, 3, 1, 1),   # 64x64 tiles
    (24, 1, 16, 56, 56, 128, 3, 1, 1),  # 128x128 tiles (600 of them), config 2's image size
    (64, 1, 4, 64, 64, 16, 3, 2, 1),   # 64x64 tiles (1024), per-element gathers
    (2, 1, 3, 8, 8, 4, 5, 1, 4),       # pad 4: whole blocks outside a row
    (2, 3, 9, 7, 5, 6, 3, 1, 2),       # three groups, odd widths
    (1, 1, 1, 3, 4, 1, 3, 1, 1),       # one channel, one filter
    # small images (over a fifth of the last column tile empty): 64x64 tiles
    # whose columns run over every image's positions -- two-block, per-tap,
    # odd positions per image, ksize 1
    (6, 1, 8, 12, 12, 16, 3, 1, 1),
    (8, 1, 16, 14, 14, 32, 3, 1, 1),
    (5, 1, 8, 9, 9, 24, 3, 1, 1),
    (4, 1, 8, 12, 12, 16, 1, 1, 0),
    (3, 2, 6, 7, 7, 10, 1, 1, 0),
    (64, 1, 8, 14, 14, 512, 3, 1, 1),  # 512 filters (128x128 tiles per image would leave 23% empty)
    (64, 1, 8, 13, 13, 512, 3, 1, 1),  # the same, 169 positions per image
    (4, 1, 8, 13, 13, 24, 3, 1, 1),    # 169 positions, 64x64 tiles per image (12% empty): per image
    # stride 2, even and odd windows, per image and over (image, position)
    (2, 1, 8, 16, 16, 16, 3, 2, 1),
    (2, 1, 4, 16, 16, 8, 2, 2, 0),
    (2, 1, 4, 16, 16, 8, 5, 2, 2),
    (6, 1, 8, 24, 24, 16, 3, 2, 1),    # ... over (image, position) columns
]


def _reference(case, x, w, out0):
    batch, groups, C, H, W, F, ks, s, p = case
    cg, m = C // groups, F // groups
    ho, wo = ref.conv_out_dim(H, ks, s, p), ref.conv_out_dim(W, ks, s, p)
    n, k = ho * wo, ks * ks * cg
    in_group = cg * H * W
    want = out0.astype(np.float64).copy()
    bound = np.abs(out0.astype(np.float64))
    for i in range(batch):
        for j in range(groups):
            z = i * groups + j
            img = x[z * in_group:(z + 1) * in_group]
            if ks == 1:
                col = img[: k * n].reshape(k, n)
            else:
                col = np.empty(k * n, np.float32)
                ref.im2col(img, cg, H, W, ks, s, p, col)
                col = col.reshape(k, n)
            wj = w[j * m * k:(j + 1) * m * k].reshape(m, k).astype(np.float64)
            sl = slice(z * m * n, (z + 1) * m * n)
            want[sl] += (wj @ col.astype(np.float64)).ravel()
            bound[sl] += (np.abs(wj) @ np.abs(col.astype(np.float64))).ravel()
    g = (k + 3) * U / (1 - (k + 3) * U)
    return want, g * bound, (m, n, k)


@pytest.mark.parametrize("case", CASES, ids=str)
def test_convolution_forward(dev, case):
    batch, groups, C, H, W, F, ks, s, p = case
    r = rng(sum(case))
    x = r.uniform(-1, 1, batch * C * H * W).astype(np.float32)
    w = r.uniform(-1, 1, F * (C // groups) * ks * ks).astype(np.float32)
    ho, wo = ref.conv_out_dim(H, ks, s, p), ref.conv_out_dim(W, ks, s, p)
    out0 = r.uniform(-1, 1, batch * F * ho * wo).astype(np.float32)
    want, bd, (m, n, k) = _reference(case, x, w, out0)
    dx, dw, do = up(x), up(w), up(out0)
    gpu.convolutionForward(batch, groups, C, H, W, F, ks, s, p, dw, dx, do)
    got = down(do, out0).astype(np.float64)
    err = np.abs(got - want)
    bad = ~(err <= bd)
    assert not bad.any(), (f"convolution {case}: {int(bad.sum())} beyond the fp32 bound; "
                           f"max err/bound {float(np.max(err / np.maximum(bd, 1e-300))):.3g}")
    for b in (dx, dw, do):
        gpu.free(b)


def test_convolution_forward_matches_per_image_calls(dev):
    """The same layer through the per-image calls the reference makes
    (im2col into a workspace, then gemm with beta 1): both within the bound of
    the f64 product, and identical wherever the products are exact (integer
    inputs)."""
    case = (3, 1, 8, 12, 12, 16, 3, 1, 1)
    batch, groups, C, H, W, F, ks, s, p = case
    r = rng(5)
    x = r.integers(-3, 4, batch * C * H * W).astype(np.float32)
    w = r.integers(-3, 4, F * C * ks * ks).astype(np.float32)
    n, k = H * W, ks * ks * C
    dx, dw = up(x), up(w)
    fused, loop = gpu.alloc(batch * F * n), gpu.alloc(batch * F * n)
    gpu.convolutionForward(batch, groups, C, H, W, F, ks, s, p, dw, dx, fused)
    ws = gpu.alloc(k * n)
    for i in range(batch):
        gpu.im2col(dx.offset(i * C * H * W), C, H, W, ks, s, p, ws)
        gpu.gemm(False, False, F, n, k, 1.0, dw, k, ws, n, 1.0, loop.offset(i * F * n), n)
    a, b = down(fused, np.empty(batch * F * n, np.float32)), down(loop, np.empty(batch * F * n, np.float32))
    assert np.array_equal(a, b)  # integer-valued: every order is exact
    for buf in (dx, dw, fused, loop, ws):
        gpu.free(buf)


def test_convolution_forward_rejects_bad_groups(dev):
    from darknet_zig_amd import _lib
    lib = _lib.load()
    buf = gpu.alloc(64)
    # channels not a multiple of groups, and a window larger than the padded image
    assert lib.dkz_convolution_forward(1, 2, 3, 4, 4, 2, 3, 1, 1, buf.ptr, buf.ptr, buf.ptr) != 0
    assert lib.dkz_convolution_forward(1, 1, 1, 2, 2, 1, 5, 1, 0, buf.ptr, buf.ptr, buf.ptr) != 0
    assert lib.dkz_convolution_forward(0, 1, 1, 2, 2, 1, 1, 1, 0, None, None, None) == 0  # empty batch
    gpu.free(buf)


WG_CASES = [
    # batch, groups, channels, height, width, filters, ksize, stride, pad
    (2, 1, 16, 16, 16, 32, 3, 1, 1),   # stride 1, widths % 4 == 0: two-block gathers
    (3, 2, 8, 10, 12, 6, 3, 2, 1),     # groups, stride 2: per-element gathers
    (2, 1, 4, 9, 9, 5, 1, 1, 0),       # ksize 1: the input itself (81 positions: float4s span images)
    (1, 1, 3, 8, 8, 4, 1, 2, 0),       # ksize 1, stride 2: the layer's own reading of the input
    (5, 1, 8, 7, 7, 16, 3, 1, 1),      # 49 positions: per-element loads across image boundaries
    (64, 1, 16, 28, 28, 32, 3, 1, 1),  # many images: the product split over image ranges
    (2, 3, 9, 7, 5, 6, 3, 1, 2),       # three groups, odd widths
    (3, 1, 8, 16, 16, 16, 3, 2, 1),    # stride 2
    (2, 2, 8, 16, 16, 8, 5, 2, 2),     # the same, 5x5, groups
    (4, 1, 8, 20, 20, 96, 3, 1, 1),    # 96 filters: 64x64 tiles, a partial row tile
    (4, 1, 16, 24, 24, 128, 3, 1, 1),  # 128x128 tiles
    (3, 1, 8, 17, 17, 160, 3, 2, 1),   # 128x128 tiles, stride 2, a partial row tile
    (4, 1, 32, 16, 16, 128, 1, 1, 0),  # 128x128 tiles, ksize 1
]


def _wgrad_reference(case, x, d, wu0):
    batch, groups, C, H, W, F, ks, s, p = case
    cg, m = C // groups, F // groups
    ho, wo = ref.conv_out_dim(H, ks, s, p), ref.conv_out_dim(W, ks, s, p)
    n, k = ho * wo, ks * ks * cg
    in_group = cg * H * W
    want = wu0.astype(np.float64).copy()
    bound = np.abs(wu0.astype(np.float64))
    for i in range(batch):
        for j in range(groups):
            z = i * groups + j
            img = x[z * in_group:(z + 1) * in_group]
            if ks == 1:
                col = img[: k * n].reshape(k, n)
            else:
                col = np.empty(k * n, np.float32)
                ref.im2col(img, cg, H, W, ks, s, p, col)
                col = col.reshape(k, n)
            dz = d[z * m * n:(z + 1) * m * n].reshape(m, n).astype(np.float64)
            sl = slice(j * m * k, (j + 1) * m * k)
            want[sl] += (dz @ col.astype(np.float64).T).ravel()
            bound[sl] += (np.abs(dz) @ np.abs(col.astype(np.float64)).T).ravel()
    kt = batch * n  # every image's positions are one sum
    g = (kt + 3) * U / (1 - (kt + 3) * U)
    return want, g * bound


@pytest.mark.parametrize("case", WG_CASES, ids=str)
def test_convolution_weight_gradient(dev, case):
    batch, groups, C, H, W, F, ks, s, p = case
    r = rng(sum(case) + 1)
    ho, wo = ref.conv_out_dim(H, ks, s, p), ref.conv_out_dim(W, ks, s, p)
    x = r.uniform(-1, 1, batch * C * H * W).astype(np.float32)
    d = r.uniform(-1, 1, batch * F * ho * wo).astype(np.float32)
    wu0 = r.uniform(-1, 1, F * (C // groups) * ks * ks).astype(np.float32)
    want, bd = _wgrad_reference(case, x, d, wu0)
    dx, dd, dw = up(x), up(d), up(wu0)
    gpu.convolutionWeightGradient(batch, groups, C, H, W, F, ks, s, p, dd, dx, dw)
    got = down(dw, wu0).astype(np.float64)
    err = np.abs(got - want)
    bad = ~(err <= bd)
    assert not bad.any(), (f"weight gradient {case}: {int(bad.sum())} beyond the fp32 bound; "
                           f"max err/bound {float(np.max(err / np.maximum(bd, 1e-300))):.3g}")
    for b in (dx, dd, dw):
        gpu.free(b)


def test_convolution_weight_gradient_matches_per_image_calls(dev):
    """The layer's per-image calls (im2col, then gemm(false, true, ..., beta 1)
    into the shared weight_updates) and the one product agree exactly on
    integer-valued inputs, where every summation order is exact."""
    case = (6, 1, 8, 12, 12, 16, 3, 1, 1)
    batch, groups, C, H, W, F, ks, s, p = case
    r = rng(9)
    x = r.integers(-3, 4, batch * C * H * W).astype(np.float32)
    d = r.integers(-3, 4, batch * F * H * W).astype(np.float32)
    n, k = H * W, ks * ks * C
    dx, dd = up(x), up(d)
    fused, loop = gpu.alloc(F * k), gpu.alloc(F * k)
    gpu.convolutionWeightGradient(batch, groups, C, H, W, F, ks, s, p, dd, dx, fused)
    ws = gpu.alloc(k * n)
    for i in range(batch):
        gpu.im2col(dx.offset(i * C * H * W), C, H, W, ks, s, p, ws)
        gpu.gemm(False, True, F, k, n, 1.0, dd.offset(i * F * n), n, ws, n, 1.0, loop, k)
    a, b = down(fused, np.empty(F * k, np.float32)), down(loop, np.empty(F * k, np.float32))
    assert np.array_equal(a, b)
    for buf in (dx, dd, fused, loop, ws):
        gpu.free(buf)


DG_CASES = [
    # batch, groups, channels, height, width, filters, ksize, stride, pad
    (2, 1, 16, 16, 16, 32, 3, 1, 1),    # stride 1, pad < ksize, widths % 4 == 0: two-block gathers of delta
    (3, 1, 5, 9, 11, 7, 3, 1, 1),       # stride 1, odd widths: per-element gathers
    (3, 2, 8, 10, 12, 6, 3, 2, 1),      # groups, stride 2: gemm into the scratch, then col2im
    (2, 1, 3, 8, 8, 4, 5, 1, 4),        # pad >= ksize: the same with stride 1
    (2, 1, 4, 13, 13, 6, 2, 2, 0),      # even window, stride 2
    (10, 1, 64, 160, 160, 8, 3, 2, 1),  # stride 2, two runs of images through the scratch (9 fit)
    (2, 3, 9, 7, 5, 6, 3, 1, 2),        # three groups, odd widths
    (4, 1, 16, 24, 24, 128, 3, 1, 1),   # 128 filters: k = 1152
    (24, 1, 128, 56, 56, 8, 3, 1, 1),   # 128 input channels: 128x128 tiles (600 of them)
    (6, 1, 8, 12, 12, 16, 3, 1, 1),     # small images: columns over every image's positions, two-block
    (64, 1, 512, 14, 14, 8, 3, 1, 1),   # the same for 512 channels, per-tap gathers
    (7, 2, 6, 9, 9, 8, 3, 1, 1),        # 81 positions per image, groups
    (2, 1, 4, 9, 9, 5, 1, 1, 0),        # ksize 1: overwritten (beta 0)
    (1, 1, 3, 8, 8, 4, 1, 2, 0),        # ksize 1, stride 2: the k x n view, a prefix of the image
    (3, 2, 6, 5, 7, 10, 1, 1, 0),       # ksize 1, groups
    (2, 1, 6, 12, 12, 5, 3, 3, 1),      # stride 3: nine one-tap phases, launched four, four and one at a time
    (2, 2, 10, 12, 10, 6, 5, 3, 2),     # stride 3, window 5 (phases of 4, 2 and 1 taps), width 10: one per launch
    (3, 1, 5, 15, 15, 7, 5, 3, 1),      # stride 3, window 5, merged phases of unequal tap counts
    (96, 1, 128, 56, 56, 8, 3, 2, 1),   # stride 2, 128 input channels: four phases per launch over every image
    (8, 1, 16, 12, 12, 8, 3, 2, 1),     # stride 2, 6x6 phases: columns over (image, phase position), 64x64 tiles
    (4, 1, 128, 16, 16, 8, 3, 2, 0),    # the same in 128x64 tiles, phase rows of 8 (row gathers), delta rows of 7
    (4, 1, 128, 12, 12, 8, 3, 2, 1),    # 128x64 tiles, phase rows of 6 (per-element gathers)
    (4, 2, 256, 12, 12, 8, 3, 2, 1),    # the same with two groups
    (4, 1, 128, 14, 14, 8, 3, 2, 1),    # 7x7 phases (49 positions per image) over every image, 128x64 tiles
    (8, 1, 16, 14, 14, 8, 3, 2, 1),     # the same in 64x64 tiles
]


def _dgrad_reference(case, w, d, im0):
    batch, groups, C, H, W, F, ks, s, p = case
    cg, m = C // groups, F // groups
    ho, wo = ref.conv_out_dim(H, ks, s, p), ref.conv_out_dim(W, ks, s, p)
    n, k = ho * wo, ks * ks * cg
    in_group = cg * H * W
    want = im0.astype(np.float64).copy()
    bound = np.abs(want)
    for i in range(batch):
        for j in range(groups):
            z = i * groups + j
            wj = w[j * m * k:(j + 1) * m * k].reshape(m, k).astype(np.float64)
            dz = d[z * m * n:(z + 1) * m * n].reshape(m, n).astype(np.float64)
            col, acol = wj.T @ dz, np.abs(wj).T @ np.abs(dz)
            sl = slice(z * in_group, (z + 1) * in_group)
            if ks == 1:  # the layer's beta-0 gemm straight into the image, as a k x n matrix
                want[z * in_group:z * in_group + k * n] = col.ravel()
                bound[z * in_group:z * in_group + k * n] = acol.ravel()
            else:
                want[sl] += col2im64(col, cg, H, W, ks, s, p)
                bound[sl] += col2im64(acol, cg, H, W, ks, s, p)
    terms = m * ks * ks + 1  # every product of every tap, plus the image's value
    g = (terms + 3) * U / (1 - (terms + 3) * U)
    return want, g * bound


@pytest.mark.parametrize("case", DG_CASES, ids=str)
def test_convolution_data_gradient(dev, case):
    batch, groups, C, H, W, F, ks, s, p = case
    r = rng(sum(case) + 2)
    ho, wo = ref.conv_out_dim(H, ks, s, p), ref.conv_out_dim(W, ks, s, p)
    w = r.uniform(-1, 1, F * (C // groups) * ks * ks).astype(np.float32)
    d = r.uniform(-1, 1, batch * F * ho * wo).astype(np.float32)
    im0 = r.uniform(-1, 1, batch * C * H * W).astype(np.float32)
    want, bd = _dgrad_reference(case, w, d, im0)
    dw, dd, di = up(w), up(d), up(im0)
    gpu.convolutionDataGradient(batch, groups, C, H, W, F, ks, s, p, dw, dd, di)
    got = down(di, im0).astype(np.float64)
    err = np.abs(got - want)
    bad = ~(err <= bd)
    assert not bad.any(), (f"data gradient {case}: {int(bad.sum())} beyond the fp32 bound; "
                           f"max err/bound {float(np.max(err / np.maximum(bd, 1e-300))):.3g}")
    for b in (dw, dd, di):
        gpu.free(b)


@pytest.mark.parametrize("case", [(5, 1, 8, 12, 12, 16, 3, 1, 1), (4, 2, 6, 11, 9, 8, 3, 2, 1),
                                  (3, 1, 8, 10, 10, 12, 1, 1, 0)], ids=str)
def test_convolution_data_gradient_matches_per_image_calls(dev, case):
    """The layer's per-image calls (gemm(true, false, ..., beta 0) into the
    workspace, then col2im into the image; for ksize 1 the gemm straight into
    the image) and the one call agree exactly on integer-valued inputs, where
    every summation order is exact."""
    batch, groups, C, H, W, F, ks, s, p = case
    cg, m = C // groups, F // groups
    ho, wo = ref.conv_out_dim(H, ks, s, p), ref.conv_out_dim(W, ks, s, p)
    n, k, in_group = ho * wo, ks * ks * cg, cg * H * W
    r = rng(sum(case))
    w = r.integers(-3, 4, F * k).astype(np.float32)
    d = r.integers(-3, 4, batch * F * n).astype(np.float32)
    im0 = r.integers(-3, 4, batch * C * H * W).astype(np.float32)
    dw, dd = up(w), up(d)
    fused, loop = up(im0), up(im0)
    gpu.convolutionDataGradient(batch, groups, C, H, W, F, ks, s, p, dw, dd, fused)
    ws = gpu.alloc(k * n)
    for i in range(batch):
        for j in range(groups):
            z = i * groups + j
            dst = loop.offset(z * in_group) if ks == 1 else ws
            gpu.gemm(True, False, k, n, m, 1.0, dw.offset(j * m * k), k, dd.offset(z * m * n), n, 0.0, dst, n)
            if ks != 1:
                gpu.col2im(ws, cg, H, W, ks, s, p, loop.offset(z * in_group))
    a, b = down(fused, im0), down(loop, im0)
    assert np.array_equal(a, b)
    for buf in (dw, dd, fused, loop, ws):
        gpu.free(buf)
