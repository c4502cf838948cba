"""The f64 col2im the convolution data-gradient tests build their expected
values with, pinned against the oracle's col2im (the twin's f32 loop,
im2col.zig:51-79): on integer-valued columns every sum is exact in both, so
they agree exactly, padding, strides, even and odd windows included."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import ref
from tests.helpers import col2im64, rng


@pytest.mark.parametrize("c,h,w,k,s,p", [(3, 8, 8, 3, 1, 1), (2, 9, 11, 3, 2, 1), (4, 7, 5, 5, 1, 4),
                                         (2, 13, 13, 2, 2, 0), (1, 6, 6, 1, 1, 0), (3, 10, 7, 4, 3, 2)])
def test_col2im64_matches_the_oracle(c, h, w, k, s, p):
    ho, wo = ref.conv_out_dim(h, k, s, p), ref.conv_out_dim(w, k, s, p)
    r = rng(c * 100 + h * 10 + w)
    col = r.integers(-50, 51, c * k * k * ho * wo).astype(np.float32)
    base = r.integers(-50, 51, c * h * w).astype(np.float32)
    im = base.copy()
    ref.col2im(col, c, h, w, k, s, p, im)
    np.testing.assert_array_equal(base.astype(np.float64) + col2im64(col, c, h, w, k, s, p), im.astype(np.float64))
