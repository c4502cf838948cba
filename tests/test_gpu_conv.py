"""GPU parity of the convolution lowering (gpu.zig:651-669) against the CPU
twins in im2col.zig: im2col bit-exact (a copy), col2im bit-exact (each image
element adds its contributions in the twin's column order).

gputest.zig:302-345's case (5 channels, 13x11, 3x3, stride 2, pad 1) plus
shapes around the float4 tail, 1x1 kernels, strides larger than the kernel,
pads larger than half the kernel, misaligned views and a full layer-sized
image.
"""

from __future__ import annotations

import numpy as np
import pytest

from darknet_zig_amd import gpu
from oracle import ref
from tests.helpers import assert_bitexact, down, rng, uniform, up

pytestmark = pytest.mark.gpu

SHAPES = [
    (5, 13, 11, 3, 2, 1),  # gputest.zig:303-308
    (1, 3, 3, 2, 1, 0),  # im2col.zig:87-95
    (3, 7, 5, 3, 1, 1),
    (4, 9, 9, 3, 2, 1),
    (2, 6, 6, 1, 1, 0),
    (5, 13, 11, 5, 3, 2),
    (3, 8, 8, 2, 2, 0),
    (2, 5, 5, 3, 1, 2),
    (7, 10, 9, 1, 3, 0),  # stride past the kernel: taps are skipped
    (3, 4, 4, 4, 1, 3),  # pad 3 with a 4-wide kernel
    (64, 28, 28, 3, 1, 1),
    (128, 56, 56, 3, 1, 1),  # config 2's layer, one image
    # stride 1 with W and the output width multiples of 4 (two aligned
    # 16-byte loads per column float4), pads that push whole blocks out of a row
    (1, 6, 8, 5, 1, 4),
    (2, 4, 8, 3, 1, 5),
    (1, 4, 12, 9, 1, 4),
    (2, 3, 4, 1, 1, 6),
    (3, 5, 16, 5, 1, 2),
]


def _col_len(C, H, W, k, s, p):
    return C * k * k * ref.conv_out_dim(H, k, s, p) * ref.conv_out_dim(W, k, s, p)


@pytest.mark.parametrize("C,H,W,k,s,p", SHAPES)
def test_im2col_col2im(dev, C, H, W, k, s, p):
    r = rng(C * 1000 + H * 10 + k)
    im = uniform(r, C * H * W)
    ncol = _col_len(C, H, W, k, s, p)
    cpu_col = np.empty(ncol, np.float32)
    ref.im2col(im, C, H, W, k, s, p, cpu_col)
    dim = up(im)
    dcol = up(np.full(ncol, np.nan, np.float32))
    gpu.im2col(dim, C, H, W, k, s, p, dcol)
    assert_bitexact(down(dcol, cpu_col), cpu_col, f"im2col {C,H,W,k,s,p}")

    # col2im accumulates into a nonzero image, from an independent column buffer
    col = uniform(r, ncol)
    base = uniform(r, C * H * W)
    cpu_im = base.copy()
    ref.col2im(col, C, H, W, k, s, p, cpu_im)
    dcol2, dim2 = up(col), up(base)
    gpu.col2im(dcol2, C, H, W, k, s, p, dim2)
    assert_bitexact(down(dim2, cpu_im), cpu_im, f"col2im {C,H,W,k,s,p}")
    for b in (dim, dcol, dcol2, dim2):
        gpu.free(b)


@pytest.mark.parametrize("offset", [1, 2, 3])
def test_im2col_misaligned_views(dev, offset):
    C, H, W, k, s, p = 3, 9, 7, 3, 1, 1
    r = rng(offset)
    im = uniform(r, C * H * W)
    ncol = _col_len(C, H, W, k, s, p)
    cpu_col = np.empty(ncol, np.float32)
    ref.im2col(im, C, H, W, k, s, p, cpu_col)
    whole_im = up(np.concatenate([np.zeros(offset, np.float32), im]))
    whole_col = gpu.alloc(ncol + offset)
    gpu.im2col(whole_im.offset(offset), C, H, W, k, s, p, whole_col.offset(offset))
    out = np.empty(ncol + offset, np.float32)
    gpu.pull(whole_col, out)
    assert_bitexact(out[offset:], cpu_col, f"im2col offset {offset}")
    gpu.free(whole_im)
    gpu.free(whole_col)


def test_col2im_of_im2col_counts_window_coverage(dev):
    """With an all-ones image, col2im(im2col(1)) counts how many windows
    cover each pixel (the im2col.zig:97-104 identity, at a real size)."""
    C, H, W, k, s, p = 16, 30, 30, 3, 1, 1
    ones = np.ones(C * H * W, np.float32)
    ncol = _col_len(C, H, W, k, s, p)
    dim, dcol, dout = up(ones), gpu.alloc(ncol), gpu.alloc(C * H * W)
    gpu.im2col(dim, C, H, W, k, s, p, dcol)
    gpu.col2im(dcol, C, H, W, k, s, p, dout)
    got = down(dout, ones).reshape(C, H, W)
    cover = np.full((H, W), 9, np.float32)
    cover[0, :] -= 3
    cover[-1, :] -= 3
    cover[:, 0] -= 3
    cover[:, -1] -= 3
    cover[[0, 0, -1, -1], [0, -1, 0, -1]] += 1
    np.testing.assert_array_equal(got, np.broadcast_to(cover, (C, H, W)))
    for b in (dim, dcol, dout):
        gpu.free(b)
