"""Maximum sizes. Every kernel indexes with 32-bit integers, as the
reference's do (darknet_kernels.hip's `int global_index()`), so one tensor
holds at most 2^31 - 1 elements; larger shapes are refused on the host
(tests/test_abi.py). These tests run the ops at that limit -- tensors of
8 GiB, generated on the device -- and check the elements whose indices lie at
the top of the range (and at the bottom) against the oracle on the same
elements, bit-exact for elementwise and index results, and the channel
reductions against the oracle and f64 sums of the whole downloaded tensor
(the 1e-5 rule).

  * elementwise (rand_uniform, copy, axpy, leaky, scal) at n = 2^31 - 1: the
    last three elements are the n % 4 tail that block 0 handles;
  * mean and variance at [2, 3, 357913940] (2^31 - 8 elements, each channel
    split over many workgroups) and mean at [1, 1024, 2097148] (one
    workgroup per channel);
  * softmax over [2147483, 1000] (the grid-stride segment kernel);
  * 2x2/s2 max pooling forward and backward, global average pooling forward
    and backward at [63, 512, 256, 256] (2^31 - 2^25 inputs; argmax indexes
    up to 2113929215);
  * stride-1 max pooling (sizes 13 and 7) at [11618, 512, 19, 19].
"""

from __future__ import annotations

import numpy as np
import pytest

from darknet_zig_amd import gpu
from darknet_zig_amd.activations import Activation
from oracle import ref
from tests.helpers import assert_bitexact, assert_r5, assert_softmax, softmax_f64

pytestmark = pytest.mark.gpu

N_MAX = 2**31 - 1
EDGE = 4099  # elements checked at each end: a ragged count, so the tail's float4 split varies


def _pull(b: gpu.Buf, first: int, n: int, dtype=np.float32) -> np.ndarray:
    out = np.empty(n, dtype)
    gpu.pull(b.offset(first), out)
    return out


def _ends(n: int) -> tuple[tuple[int, int], ...]:
    return ((0, EDGE), (n - EDGE, EDGE))


def test_elementwise_at_max_elements(dev):
    print("elementwise at n = 2^31 - 1", flush=True)
    x, y = gpu.alloc(N_MAX), gpu.alloc(N_MAX)
    try:
        gpu.randUniform(N_MAX, x, 0x5EED)
        xs = {}
        for first, n in _ends(N_MAX):
            want = np.empty(n, np.float32)
            ref.randUniform(want, 0x5EED, first)
            xs[first] = _pull(x, first, n)
            assert_bitexact(xs[first], want, f"rand_uniform [{first}, {first + n})")
        gpu.copy(N_MAX, x, y)
        for first, n in _ends(N_MAX):
            assert_bitexact(_pull(y, first, n), xs[first], f"copy [{first}, {first + n})")
        gpu.fill(y, N_MAX, 0.375)
        gpu.axpy(N_MAX, -1.5, x, y)
        gpu.activateArray(y, N_MAX, int(Activation.leaky))
        gpu.scal(N_MAX, 3.0, y)
        for first, n in _ends(N_MAX):
            want = np.full(n, 0.375, np.float32)
            ref.axpy(-1.5, xs[first], want)
            ref.activateArray(want, int(Activation.leaky))
            ref.scal(3.0, want)
            assert_bitexact(_pull(y, first, n), want, f"fill, axpy, leaky, scal [{first}, {first + n})")
    finally:
        gpu.free(x)
        gpu.free(y)


def _plane_sums64(x: np.ndarray, shape, term=None) -> np.ndarray:
    """Per-channel f64 sums over a [B, F, S] tensor without an f64 copy of it:
    each (b, f) row summed in chunks, `term` (f32, as the twin rounds it)
    applied per chunk."""
    B, F, S = shape
    out = np.zeros(F)
    step = 1 << 25
    for b in range(B):
        for f in range(F):
            row = x[(b * F + f) * S:(b * F + f + 1) * S]
            for s0 in range(0, S, step):
                c = row[s0:s0 + step]
                out[f] += np.add.reduce(term(c, f) if term else c, dtype=np.float64)
    return out


def test_split_channel_reductions_at_max_elements(dev):
    B, F, S = shape = (2, 3, 357913940)
    n = B * F * S
    print(f"mean and variance at {shape}: {n} elements", flush=True)
    x, dm, dv = gpu.alloc(n), gpu.alloc(F), gpu.alloc(F)
    try:
        gpu.randUniform(n, x, 77)
        gpu.scal(n, 4.0, x)
        gpu.mean(x, B, F, S, dm)
        m_gpu = _pull(dm, 0, F)
        gpu.variance(x, dm, B, F, S, dv)
        v_gpu = _pull(dv, 0, F)
        xh = _pull(x, 0, n)
    finally:
        for b in (x, dm, dv):
            gpu.free(b)
    m_cpu, v_cpu = np.empty(F, np.float32), np.empty(F, np.float32)
    ref.mean(xh, B, F, S, m_cpu)
    ref.variance(xh, m_gpu, B, F, S, v_cpu)  # the device's mean on both sides
    scale_m = np.float32(1.0) / np.float32(B * S)
    scale_v = np.float32(1.0) / np.float32(B * S - 1)
    m64 = _plane_sums64(xh, shape) * np.float64(scale_m)
    # blas.zig:128-131: the f32 difference, squared in f32
    v64 = _plane_sums64(xh, shape, lambda c, f: np.square(c - m_gpu[f])) * np.float64(scale_v)
    assert_r5(m_gpu, m_cpu, m64, f"mean {shape}")
    assert_r5(v_gpu, v_cpu, v64, f"variance {shape}")
    # the data are U(0, 4): every channel's mean and variance near 2 and 4/3
    np.testing.assert_allclose(m_gpu, 2.0, rtol=1e-3)
    np.testing.assert_allclose(v_gpu, 4.0 / 3.0, rtol=1e-3)


def test_per_channel_reduction_at_max_elements(dev):
    B, F, S = shape = (1, 1024, 2097148)
    n = B * F * S
    print(f"mean at {shape}: {n} elements", flush=True)
    x, dm = gpu.alloc(n), gpu.alloc(F)
    try:
        gpu.randUniform(n, x, 78)
        gpu.mean(x, B, F, S, dm)
        m_gpu = _pull(dm, 0, F)
        for f in (0, 1, F - 2, F - 1):
            xf = _pull(x, f * S, S)
            m_cpu = np.empty(1, np.float32)
            ref.mean(xf, 1, 1, S, m_cpu)
            m64 = np.add.reduce(xf, dtype=np.float64) * np.float64(np.float32(1.0) / np.float32(S))
            assert_r5(m_gpu[f:f + 1], m_cpu, np.array([m64]), f"mean {shape} channel {f}")
    finally:
        gpu.free(x)
        gpu.free(dm)


def test_softmax_rows_at_max_elements(dev):
    rows, classes = 2147483, 1000
    n = rows * classes
    print(f"softmax over [{rows}, {classes}]: {n} elements", flush=True)
    x, out = gpu.alloc(n), gpu.alloc(n)
    try:
        gpu.randUniform(n, x, 79)
        gpu.scal(n, 16.0, x)
        gpu.softmax(x, classes, rows, classes, 1, classes, 1, 1.0, out)
        for r0 in (0, rows - 64):
            xs = _pull(x, r0 * classes, 64 * classes)
            got = _pull(out, r0 * classes, 64 * classes)
            cpu = np.empty_like(xs)
            ref.softmax(xs, classes, 64, classes, 1, classes, 1, 1.0, cpu)
            assert_softmax(got, cpu, softmax_f64(xs, classes, 64, classes, 1, classes, 1, 1.0),
                           f"softmax rows [{r0}, {r0 + 64})")
    finally:
        gpu.free(x)
        gpu.free(out)


def test_pooling_at_max_elements(dev):
    B, C, H, W = 63, 512, 256, 256
    planes, hw, ohw = B * C, H * W, (H // 2) * (W // 2)
    n_in, n_out = planes * hw, planes * ohw
    print(f"max and average pooling at [{B}, {C}, {H}, {W}]: {n_in} inputs", flush=True)
    x, out, idx = gpu.alloc(n_in), gpu.alloc(n_out), gpu.allocInts(n_out)
    d, prev = gpu.alloc(n_out), gpu.alloc(n_in)
    avg, od = gpu.alloc(planes), gpu.alloc(planes)
    try:
        gpu.randUniform(n_in, x, 80)
        gpu.forwardMaxpool(n_out, H, W, C, 2, 2, 0, x, out, idx)
        gpu.randUniform(n_out, d, 81)
        gpu.backwardMaxpool(n_in, H, W, C, 2, 2, 0, d, prev, idx)
        gpu.forwardAvgpool(planes, W, H, C, x, avg)
        gpu.randUniform(planes, od, 82)
        gpu.backwardAvgpool(planes, W, H, C, prev, od)  # adds onto the max-pool backward's result
        avg_g, od_h = _pull(avg, 0, planes), _pull(od, 0, planes)
        for p in (0, 1, planes - 2, planes - 1):
            xp = _pull(x, p * hw, hw)
            o_c, i_c = np.empty(ohw, np.float32), np.empty(ohw, np.int32)
            ref.forwardMaxpool(1, H, W, 1, 2, 2, 0, xp, o_c, i_c)  # indexes within the plane
            assert_bitexact(_pull(out, p * ohw, ohw), o_c, f"maxpool fwd plane {p}")
            i_g = _pull(idx, p * ohw, ohw, np.int32)
            assert_bitexact(i_g, i_c + np.int32(p * hw), f"maxpool idx plane {p}")
            prev_c = np.zeros(hw, np.float32)
            ref.backwardMaxpool(i_c, _pull(d, p * ohw, ohw), prev_c)
            ref.backwardAvgpool(1, W, H, 1, od_h[p:p + 1], prev_c)
            assert_bitexact(_pull(prev, p * hw, hw), prev_c, f"maxpool + avgpool bwd plane {p}")
            a_c = np.empty(1, np.float32)
            ref.forwardAvgpool(1, W, H, 1, xp, a_c)
            assert_r5(avg_g[p:p + 1], a_c, np.array([np.add.reduce(xp, dtype=np.float64) / hw]),
                      f"avgpool fwd plane {p}")
    finally:
        for b in (x, out, idx, d, prev, avg, od):
            gpu.free(b)


@pytest.mark.parametrize("size", [13, 7])
def test_stride1_pooling_at_max_elements(dev, size):
    """Spatial pyramid pooling's stride-1 windows at [11618, 512, 19, 19]
    (2147378176 inputs): size 13 through the separable forward with runs
    of outputs a lane and the gather with runs of inputs a lane, size 7
    through the separable forward and the gather without them; the first
    and last planes against the oracle, bit-exact."""
    B, C, H, W = 11618, 512, 19, 19
    pad = size - 1
    planes, hw = B * C, H * W
    ohw = ref.maxpool_out_dim(H, size, 1, pad) * ref.maxpool_out_dim(W, size, 1, pad)
    n_in, n_out = planes * hw, planes * ohw
    assert n_in <= N_MAX
    print(f"stride-1 max pooling, size {size}, at [{B}, {C}, {H}, {W}]: {n_in} inputs", flush=True)
    x, out, idx = gpu.alloc(n_in), gpu.alloc(n_out), gpu.allocInts(n_out)
    d, prev = gpu.alloc(n_out), gpu.alloc(n_in)
    try:
        gpu.randUniform(n_in, x, 90 + size)
        gpu.forwardMaxpool(n_out, H, W, C, 1, size, pad, x, out, idx)
        gpu.randUniform(n_out, d, 91 + size)
        gpu.backwardMaxpool(n_in, H, W, C, 1, size, pad, d, prev, idx)
        for p in (0, 1, planes - 2, planes - 1):
            xp = _pull(x, p * hw, hw)
            o_c, i_c = np.empty(ohw, np.float32), np.empty(ohw, np.int32)
            ref.forwardMaxpool(1, H, W, 1, size, 1, pad, xp, o_c, i_c)  # indexes within the plane
            assert_bitexact(_pull(out, p * ohw, ohw), o_c, f"maxpool fwd plane {p}")
            assert_bitexact(_pull(idx, p * ohw, ohw, np.int32), i_c + np.int32(p * hw), f"maxpool idx plane {p}")
            prev_c = np.zeros(hw, np.float32)
            ref.backwardMaxpool(i_c, _pull(d, p * ohw, ohw), prev_c)
            assert_bitexact(_pull(prev, p * hw, hw), prev_c, f"maxpool bwd plane {p}")
    finally:
        for b in (x, out, idx, d, prev):
            gpu.free(b)
