"""Channel reductions split over several workgroups per channel run as one
launch: each workgroup writes its f64 partial with a coherent (agent-scope)
store and counts itself in its channel's counter, and the last to arrive adds
the channel's partials and finalises, then empties the counter. Each op is
launched many times back to back on fresh data, with no synchronisation in
between, so a partial read before it was visible, a counter not emptied for
the next launch, or a channel finalised twice would show as a wrong sum.
Shapes: 128 channels split 16 ways, config 1's 32 channels split 64 ways,
1000 channels split 3 ways with a ragged last chunk, and per-element loads
(spatial not a multiple of 4)."""

from __future__ import annotations

import numpy as np
import pytest

from darknet_zig_amd import _lib, gpu
from oracle import ref
from tests.helpers import assert_r5, chan_f32, chan_sum64, down, normal, rng, up

pytestmark = pytest.mark.gpu

SHAPES = [(4, 128, 16384), (128, 32, 1024), (3, 1000, 2100), (5, 64, 4099)]
ROUNDS = 30


@pytest.fixture
def quiet(dev):
    lib = _lib.load()
    before = lib.dkz_get_sync_after_launch()
    lib.dkz_set_sync_after_launch(0)
    yield lib
    lib.dkz_set_sync_after_launch(before)
    gpu.sync()


@pytest.mark.parametrize("shape", SHAPES, ids=str)
def test_split_reductions_back_to_back(quiet, shape):
    B, F, S = shape
    n = B * F * S
    r = rng(77)
    xs = [normal(r, n, 0.1 * k, 1.0) for k in range(ROUNDS)]
    var = (np.abs(normal(r, F)) + np.float32(0.5)).astype(np.float32)
    bufs = [up(x) for x in xs]
    dvar = up(var)
    outs = {name: [gpu.alloc(F) for _ in range(ROUNDS)] for name in ("mean", "bias", "md")}
    for k in range(ROUNDS):
        gpu.mean(bufs[k], B, F, S, outs["mean"][k])
        gpu.backwardBias(outs["bias"][k], bufs[k], B, F, S)
        gpu.meanDelta(bufs[k], dvar, B, F, S, outs["md"][k])
    gpu.sync()
    fac = (np.float32(-1.0) / np.sqrt(var + np.float32(1e-5))).astype(np.float64)
    for k in range(ROUNDS):
        s64 = xs[k].astype(np.float64).reshape(B, F, S).sum(axis=(0, 2))
        m_twin = np.empty(F, np.float32)
        ref.mean(xs[k], B, F, S, m_twin)
        scale = np.float64(np.float32(1) / np.float32(B * S))
        assert_r5(down(outs["mean"][k], m_twin), m_twin, s64 * scale, f"mean round {k}")
        b_twin = np.zeros(F, np.float32)
        ref.backwardBias(b_twin, xs[k], B, F, S)
        assert_r5(down(outs["bias"][k], b_twin), b_twin, s64, f"backward_bias round {k}")
        md_twin = np.empty(F, np.float32)
        ref.meanDelta(xs[k], var, B, F, S, md_twin)
        assert_r5(down(outs["md"][k], md_twin), md_twin, s64 * fac, f"mean_delta round {k}")
    for b in bufs + [dvar] + [o for v in outs.values() for o in v]:
        gpu.free(b)


@pytest.mark.parametrize("shape", SHAPES, ids=str)
def test_split_variance_matches_per_round(quiet, shape):
    B, F, S = shape
    n = B * F * S
    r = rng(78)
    for k in range(10):
        x = normal(r, n, 0.5, 2.0)
        m = np.empty(F, np.float32)
        ref.mean(x, B, F, S, m)
        v = np.empty(F, np.float32)
        ref.variance(x, m, B, F, S, v)
        dx, dm, out = up(x), up(m), gpu.alloc(F)
        gpu.variance(dx, dm, B, F, S, out)
        diff = x - chan_f32(m, shape)
        want = chan_sum64(diff * diff, shape) * np.float64(np.float32(1) / np.float32(B * S - 1))
        assert_r5(down(out, v), v, want, f"variance round {k}")
        for b in (dx, dm, out):
            gpu.free(b)
