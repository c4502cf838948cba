"""GPU parity of the fused batch-norm layer entry points
(dkz_batchnorm_forward / dkz_batchnorm_backward) against the CPU twins run
as the layer runs them (oracle.ref.batchnormForward / batchnormBackward:
layers/batchnorm.zig:74-123 with the activation calls of
convolutional.zig:173 and :184).

The per-channel values (mean, variance, the bias/scale updates, mean_delta,
variance_delta) are reductions and follow the 1e-5 rule of tests/helpers.py
against f64 evaluations. Every element result is then held to bit-exactness
against the twins fed the GPU's own per-channel values: the fused passes
must repeat the per-op element arithmetic exactly. Shapes cover the fused
fast path (spatial % 4 == 0) with split (K > 1) and one-workgroup-per-channel
reductions, and the per-op fallback (spatial % 4 != 0, spatial == 1).
"""

from __future__ import annotations

import numpy as np
import pytest

from darknet_zig_amd import _lib, gpu
from darknet_zig_amd.activations import Activation
from oracle import ref
from tests.helpers import assert_bitexact, assert_r5, down, normal, rng, uniform, up

pytestmark = pytest.mark.gpu

FAST = [
    (4, 17, 52),      # split reduction, small
    (5, 33, 196),
    (3, 128, 64),     # filters 128, few bytes: one 256-thread workgroup per channel
    (4, 256, 4096),   # filters 256, long channels: one 1024-thread workgroup per channel
    (2, 8, 20000),    # few channels, long: split with a ragged last chunk
    (16, 5, 600),     # split; an apply tile spans up to 8 rows, channels repeat within it
    (8, 6, 1536),     # split; apply tiles finalise their own channels
    (128, 32, 1024),  # benchmark config 1
    (8, 700, 1024),   # 700 channels: more 1024-thread workgroups than fit at once, so 256-thread ones
    (4, 300, 1024),   # 300 one-workgroup channels: the backward's 1024-thread grid does not fit, 256 does
]
FALLBACK = [
    (4, 17, 53),      # gputest's shape: spatial % 4 != 0
    (3, 5, 7),
    (6, 10, 1),       # spatial 1 (a connected layer)
]
CONFIG2 = (64, 128, 3136)


def _chan64(a, shape):
    B, F, S = shape
    return a.astype(np.float64).reshape(B, F, S)


def _free(*bufs):
    for b in bufs:
        gpu.free(b)


def _forward_case(shape, act, train, inplace, seed):
    B, F, S = shape
    n = B * F * S
    r = rng(seed)
    inp = normal(r, n, 0.25, 1.0)
    scales, biases = uniform(r, F, 0.5, 1.5), normal(r, F, 0, 0.1)
    rm0, rv0 = normal(r, F, 0, 0.1), uniform(r, F, 0.5, 1.5)
    sentinel = np.full(F, 7.0, np.float32)

    d_in = up(inp)
    d_out = d_in if inplace else gpu.alloc(n)
    d_x, d_xn = gpu.alloc(n), up(np.full(n, 3.0, np.float32))
    d_m, d_v, d_rm, d_rv = up(sentinel), up(sentinel), up(rm0), up(rv0)
    d_s, d_b = up(scales), up(biases)
    gpu.batchnormForward(B, F, S, act, train, d_in, d_out, d_x, d_xn, d_m, d_v, d_rm, d_rv, d_s, d_b)
    out, x, xn = down(d_out, inp), down(d_x, inp), down(d_xn, inp)
    g_m, g_v, g_rm, g_rv = down(d_m, sentinel), down(d_v, sentinel), down(d_rm, rm0), down(d_rv, rv0)
    _free(d_in, d_x, d_xn, d_m, d_v, d_rm, d_rv, d_s, d_b, *([] if inplace else [d_out]))

    assert_bitexact(x, inp, f"x {shape}")
    if train:
        # the twins' statistics, and f64 evaluations of the same formulas
        c_m, c_v = np.empty(F, np.float32), np.empty(F, np.float32)
        ref.mean(inp, B, F, S, c_m)
        ref.variance(inp, c_m, B, F, S, c_v)
        x64 = _chan64(inp, shape)
        assert_r5(g_m, c_m, x64.sum(axis=(0, 2)) * np.float64(np.float32(1) / np.float32(B * S)), f"mean {shape}")
        if B * S > 1:
            # the fused statistics sum exact (x - c) terms in f64 (not the twin's
            # f32-rounded (x - m)^2), so their f64 reference is the exact one
            dev64 = ((x64 - c_m.astype(np.float64)[None, :, None]) ** 2).sum(axis=(0, 2))
            assert_r5(g_v, c_v, dev64 * np.float64(np.float32(1) / np.float32(B * S - 1)), f"variance {shape}")
        # the rolling averages from the GPU statistics: scal then axpy, bit-exact
        want_rm, want_rv = rm0.copy(), rv0.copy()
        ref.scal(ref.ROLLING_MOMENTUM, want_rm)
        ref.axpy(ref.EMA_ALPHA, g_m, want_rm)
        ref.scal(ref.ROLLING_MOMENTUM, want_rv)
        ref.axpy(ref.EMA_ALPHA, g_v, want_rv)
        assert_bitexact(g_rm, want_rm, f"rolling_mean {shape}")
        assert_bitexact(g_rv, want_rv, f"rolling_variance {shape}")
        stat_m, stat_v = g_m, g_v
    else:
        assert_bitexact(g_m, sentinel, "mean untouched in inference")
        assert_bitexact(g_v, sentinel, "variance untouched in inference")
        assert_bitexact(g_rm, rm0, "rolling_mean untouched in inference")
        assert_bitexact(g_rv, rv0, "rolling_variance untouched in inference")
        stat_m, stat_v = rm0, rv0
    # element results: the twins on the statistics the GPU normalised with
    want = inp.copy()
    ref.normalize(want, stat_m, stat_v, B, F, S)
    if train:
        assert_bitexact(xn, want, f"x_norm {shape} act={act}")
    else:
        assert_bitexact(xn, np.full(n, 3.0, np.float32), "x_norm untouched in inference")
    ref.scaleBias(want, scales, B, F, S)
    ref.addBias(want, biases, B, F, S)
    ref.activateArray(want, act)
    assert_bitexact(out, want, f"output {shape} act={act}")
    return stat_m, stat_v


@pytest.mark.parametrize("shape", FAST + FALLBACK, ids=str)
def test_forward_train(dev, shape):
    _forward_case(shape, Activation.leaky, True, inplace=True, seed=sum(shape))


# Too many workgroups for the small one-launch forward, few enough for the
# register-resident one (a 512-thread workgroup a CU, up to 100352 elements
# of a channel each): config 2's shape (two per channel), one per channel
# (K = 1), and four per channel with a ragged last chunk.
REGISTER = [(64, 128, 3136), (32, 256, 3136), (100, 64, 4000),
            (4, 1, 6422528),   # one channel over all 256 workgroups
            (2, 3, 1338368)]   # the backward's 27 workgroups a channel, the last chunk ragged


@pytest.mark.parametrize("shape", REGISTER, ids=str)
def test_forward_train_register_resident(dev, shape):
    _forward_case(shape, Activation.leaky, True, inplace=True, seed=sum(shape) + 1)


@pytest.mark.parametrize("act", [Activation.tanh, Activation.linear, Activation.logistic], ids=lambda a: a.name)
def test_forward_register_resident_activations(dev, act):
    """At config 2's shape an activation whose register-resident kernel would
    spill (tanh) takes the two-pass path instead; either way the results are
    the twins'."""
    _forward_case(CONFIG2, act, True, inplace=True, seed=300 + int(act))


@pytest.mark.parametrize("shape", [(4, 17, 52), (4, 17, 53)], ids=str)
def test_forward_standalone_layer_copies_input(dev, shape):
    """input != output: the standalone batchnorm layer (batchnorm.zig:78)."""
    _forward_case(shape, Activation.linear, True, inplace=False, seed=11)


@pytest.mark.parametrize("shape", [(4, 17, 52), (4, 17, 53), (128, 32, 1024)], ids=str)
def test_forward_inference(dev, shape):
    _forward_case(shape, Activation.leaky, False, inplace=True, seed=12)


@pytest.mark.parametrize("act", list(Activation), ids=lambda a: a.name)
def test_forward_every_activation(dev, act):
    _forward_case((4, 12, 64), act, True, inplace=True, seed=100 + int(act))
    _forward_case((8, 6, 1536), act, True, inplace=True, seed=150 + int(act))


def test_forward_matches_oracle_layer_sequence(dev):
    """The whole oracle layer sequence at config 1, compared end to end: the
    statistics by the 1e-5 rule, everything downstream of them to 1e-4
    (they carry the statistics' last-bit differences)."""
    B, F, S = 128, 32, 1024
    n = B * F * S
    r = rng(21)
    inp = normal(r, n)
    scales, biases = uniform(r, F, 0.5, 1.5), normal(r, F, 0, 0.1)
    rm0, rv0 = normal(r, F, 0, 0.1), uniform(r, F, 0.5, 1.5)
    c_out, c_x, c_xn = inp.copy(), np.empty(n, np.float32), np.empty(n, np.float32)
    c_m, c_v, c_rm, c_rv = np.empty(F, np.float32), np.empty(F, np.float32), rm0.copy(), rv0.copy()
    ref.batchnormForward(B, F, S, Activation.leaky, True, c_out, c_out, c_x, c_xn, c_m, c_v, c_rm, c_rv, scales,
                         biases)
    d_io, d_x, d_xn = up(inp), gpu.alloc(n), gpu.alloc(n)
    d_m, d_v, d_rm, d_rv, d_s, d_b = gpu.alloc(F), gpu.alloc(F), up(rm0), up(rv0), up(scales), up(biases)
    gpu.batchnormForward(B, F, S, Activation.leaky, True, d_io, d_io, d_x, d_xn, d_m, d_v, d_rm, d_rv, d_s, d_b)
    np.testing.assert_allclose(down(d_io, inp), c_out, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(down(d_xn, inp), c_xn, rtol=1e-4, atol=1e-5)
    assert_bitexact(down(d_x, inp), c_x, "x")
    np.testing.assert_allclose(down(d_rm, rm0), c_rm, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(down(d_rv, rv0), c_rv, rtol=1e-5, atol=1e-7)
    _free(d_io, d_x, d_xn, d_m, d_v, d_rm, d_rv, d_s, d_b)


def _backward_case(shape, act, seed, with_y=True):
    B, F, S = shape
    n = B * F * S
    r = rng(seed)
    y, delta, x = normal(r, n), normal(r, n), normal(r, n, 0.2, 1.0)
    ref.activateArray(y, act)  # y is an activation output, as gradient() expects
    scales = uniform(r, F, 0.5, 1.5)
    m, v = np.empty(F, np.float32), np.empty(F, np.float32)
    ref.mean(x, B, F, S, m)
    ref.variance(x, m, B, F, S, v)
    x_norm = x.copy()
    ref.normalize(x_norm, m, v, B, F, S)
    bu0, su0 = normal(r, F, 0, 1), normal(r, F, 0, 1)

    # the twins' layer sequence
    c_d, c_bu, c_su = delta.copy(), bu0.copy(), su0.copy()
    c_md, c_vd = np.empty(F, np.float32), np.empty(F, np.float32)
    ref.batchnormBackward(B, F, S, act, y, c_d, x, x_norm, m, v, scales, c_bu, c_su, c_md, c_vd)

    d_y = up(y) if with_y else gpu.Buf()
    d_d, d_x, d_xn, d_m, d_v, d_s = up(delta), up(x), up(x_norm), up(m), up(v), up(scales)
    d_bu, d_su, d_md, d_vd = up(bu0), up(su0), gpu.alloc(F), gpu.alloc(F)
    gpu.batchnormBackward(B, F, S, act, d_y, d_d, d_x, d_xn, d_m, d_v, d_s, d_bu, d_su, d_md, d_vd)
    g_d, g_bu, g_su = down(d_d, delta), down(d_bu, bu0), down(d_su, su0)
    g_md, g_vd = down(d_md, c_md), down(d_vd, c_vd)
    _free(*[b for b in (d_y, d_d, d_x, d_xn, d_m, d_v, d_s, d_bu, d_su, d_md, d_vd) if not b.is_null()])

    # f64 evaluations on the (bit-exact) per-element terms
    d1 = delta.copy()
    ref.gradientArray(y, act, d1)
    d2 = d1.copy()
    ref.scaleBias(d2, scales, B, F, S)
    d1_64, d2_64 = _chan64(d1, shape), _chan64(d2, shape)
    prod = _chan64(d1 * x_norm, shape)  # f32 products, as blas.zig:96 rounds them
    dev = _chan64(d2 * (x - np.repeat(np.tile(m, B), S)), shape)  # blas.zig:174
    assert_r5(g_bu, c_bu, bu0.astype(np.float64) + d1_64.sum(axis=(0, 2)), f"bias_updates {shape} {act.name}")
    assert_r5(g_su, c_su, su0.astype(np.float64) + prod.sum(axis=(0, 2)), f"scale_updates {shape} {act.name}")
    fac = (np.float32(-1.0) / np.sqrt(v + np.float32(1e-5))).astype(np.float64)
    assert_r5(g_md, c_md, d2_64.sum(axis=(0, 2)) * fac, f"mean_delta {shape} {act.name}")
    v64 = (v + np.float32(1e-5)).astype(np.float64)
    assert_r5(g_vd, c_vd, dev.sum(axis=(0, 2)) * -0.5 * v64**-1.5, f"variance_delta {shape} {act.name}")
    # delta: normalize_delta of the twin's d2 with the GPU's mean_delta / variance_delta
    want = d2.copy()
    ref.normalizeDelta(x, m, v, g_md, g_vd, B, F, S, want)
    assert_bitexact(g_d, want, f"delta {shape} {act.name}")
    return g_d, c_d


@pytest.mark.parametrize("shape", FAST + FALLBACK + [CONFIG2], ids=str)
def test_backward(dev, shape):
    g_d, c_d = _backward_case(shape, Activation.leaky, seed=40 + sum(shape))
    np.testing.assert_allclose(g_d, c_d, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("act", list(Activation), ids=lambda a: a.name)
def test_backward_every_activation(dev, act):
    _backward_case((4, 12, 64), act, seed=200 + int(act))
    _backward_case((8, 6, 1536), act, seed=250 + int(act))


@pytest.mark.parametrize("shape", REGISTER, ids=str)
def test_backward_register_holding(dev, shape):
    """Grids too large for the one-launch kernel: one 512-thread workgroup a
    CU holding part of its chunk's terms in registers and reading the rest
    again after the channel barrier."""
    g_d, c_d = _backward_case(shape, Activation.leaky, seed=60 + sum(shape))
    np.testing.assert_allclose(g_d, c_d, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("shape", [(16, 64, 43264), (4, 3, 6000000)], ids=str)
def test_register_holding_rereads(dev, shape):
    """Tensors larger than the GPU holds at once: as many 512-thread
    workgroups a channel as fit, each holding part of its chunk and reading
    the rest again (a [16,64,208,208] layer: 1.7 times what a workgroup
    holds, both directions; 3 channels of 24 M: 2.8 times, the backward --
    the forward takes two passes there)."""
    _forward_case(shape, Activation.leaky, True, inplace=True, seed=69 + sum(shape))
    g_d, c_d = _backward_case(shape, Activation.leaky, seed=70 + sum(shape))
    np.testing.assert_allclose(g_d, c_d, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("act", [Activation.tanh, Activation.linear, Activation.logistic, Activation.selu],
                         ids=lambda a: a.name)
def test_backward_register_holding_activations(dev, act):
    _backward_case(CONFIG2, act, seed=350 + int(act))


HIP_ERROR_LAUNCH_TIMEOUT = 702  # hipErrorLaunchTimeOut


def _expect_timeout(kernel: str, sync_after_launch: bool, call):
    """Runs `call` (one fused op) and returns once its barrier time-out has
    been reported: by the op itself under sync-after-launch, else by the
    next gpu.sync(). Either way the status is hipErrorLaunchTimeOut, the
    context names `kernel`, and the report clears the flag (the next sync
    is clean)."""
    before = bool(_lib.load().dkz_get_sync_after_launch())
    gpu.setSyncAfterLaunch(sync_after_launch)
    try:
        if sync_after_launch:
            with pytest.raises(gpu.GpuError) as ei:
                call()
        else:
            call()
            with pytest.raises(gpu.GpuError) as ei:
                gpu.sync()
    finally:
        gpu.setSyncAfterLaunch(before)
    assert ei.value.code == HIP_ERROR_LAUNCH_TIMEOUT, ei.value
    assert kernel in ei.value.context, ei.value.context
    gpu.sync()  # reported once


@pytest.mark.parametrize("sync_after_launch", [False, True], ids=["at_sync", "sync_after_launch"])
@pytest.mark.parametrize("bwd_shape", [(128, 32, 1024), CONFIG2], ids=str)
def test_barrier_time_out_gives_nan(dev, monkeypatch, bwd_shape, sync_after_launch):
    """The one-launch passes' channel barrier waits a bounded time. Forced to
    give up at once (DKZ_BARRIER_SPIN_LIMIT=0, read at each launch), every
    workgroup but the last of its channel finds the barrier unmet and writes
    NaN rather than results from partial sums that were not all posted. The
    call then surfaces as hipErrorLaunchTimeOut naming the kernel (the op's
    own status under sync-after-launch, else the next sync), and the state
    that outlives the call is never poisoned: each channel's rolling
    averages and bias/scale updates are either left as they were (the
    channel's finalising workgroup timed out) or hold the right update (it
    met its channel), never NaN. The barrier's slots are left ready, so the
    next call is right again. Every kernel still exits normally: the spin
    limit only shortens its own wait."""
    B, F, S = 128, 32, 1024  # config 1: the forward splits each channel 8 ways
    n = B * F * S
    r = rng(77)
    x = normal(r, n)
    d_s, d_b = up(uniform(r, F, 0.5, 1.5)), up(normal(r, F, 0, 0.1))
    rm0, rv0 = normal(r, F, 0, 0.1), uniform(r, F, 0.5, 1.5)

    def forward(spin_limit):
        d_in, d_out, d_x, d_xn = up(x), gpu.alloc(n), gpu.alloc(n), gpu.alloc(n)
        d_m, d_v, d_rm, d_rv = gpu.alloc(F), gpu.alloc(F), up(rm0), up(rv0)

        def call():
            gpu.batchnormForward(B, F, S, Activation.leaky, True, d_in, d_out, d_x, d_xn, d_m, d_v, d_rm, d_rv,
                                 d_s, d_b)
        if spin_limit is None:
            call()
        else:
            monkeypatch.setenv("DKZ_BARRIER_SPIN_LIMIT", spin_limit)
            _expect_timeout("bn_fwd_coop_kernel", sync_after_launch, call)
            monkeypatch.delenv("DKZ_BARRIER_SPIN_LIMIT")
        got = down(d_out, x), down(d_rm, rm0), down(d_rv, rv0)
        _free(d_in, d_out, d_x, d_xn, d_m, d_v, d_rm, d_rv)
        return got

    out, rm, rv = forward("0")
    _, rm_ok, rv_ok = forward(None)
    assert np.isnan(out).any(), "a timed-out forward barrier left no NaN"
    for got, before, right, what in ((rm, rm0, rm_ok, "rolling_mean"), (rv, rv0, rv_ok, "rolling_variance")):
        assert np.isfinite(got).all(), what
        assert np.all((got == before) | (got == right)), what
    _free(d_s, d_b)

    Bb, Fb, Sb = bwd_shape
    nb = Bb * Fb * Sb
    y, delta, xb, xn = normal(r, nb), normal(r, nb), normal(r, nb), normal(r, nb)
    m, v, s = normal(r, Fb, 0, 0.1), uniform(r, Fb, 0.5, 1.5), uniform(r, Fb, 0.5, 1.5)
    bu0, su0 = normal(r, Fb), normal(r, Fb)
    kernel = "bn_bwd_reg_kernel" if bwd_shape == CONFIG2 else "bn_bwd_coop_kernel"

    def backward(spin_limit):
        d_y, d_d, d_xb, d_xnb, d_m, d_v, d_s = up(y), up(delta), up(xb), up(xn), up(m), up(v), up(s)
        d_bu, d_su, d_md, d_vd = up(bu0), up(su0), gpu.alloc(Fb), gpu.alloc(Fb)

        def call():
            gpu.batchnormBackward(Bb, Fb, Sb, Activation.leaky, d_y, d_d, d_xb, d_xnb, d_m, d_v, d_s, d_bu, d_su,
                                  d_md, d_vd)
        if spin_limit is None:
            call()
        else:
            monkeypatch.setenv("DKZ_BARRIER_SPIN_LIMIT", spin_limit)
            _expect_timeout(kernel, sync_after_launch, call)
            monkeypatch.delenv("DKZ_BARRIER_SPIN_LIMIT")
        got = down(d_d, delta), down(d_bu, bu0), down(d_su, su0)
        _free(d_y, d_d, d_xb, d_xnb, d_m, d_v, d_s, d_bu, d_su, d_md, d_vd)
        return got

    got, bu, su = backward("0")
    _, bu_ok, su_ok = backward(None)
    assert np.isnan(got).any(), "a timed-out backward barrier left no NaN"
    for g, before, right, what in ((bu, bu0, bu_ok, "bias_updates"), (su, su0, su_ok, "scale_updates")):
        assert np.isfinite(g).all(), what
        assert np.all((g == before) | (g == right)), what

    _forward_case((B, F, S), Activation.leaky, True, inplace=True, seed=78)
    _backward_case(bwd_shape, Activation.leaky, seed=79)


@pytest.mark.parametrize("shape", [(128, 32, 1024), (4, 17, 10000), (8, 512, 1024), CONFIG2, (2, 1, 1000000)],
                         ids=str)
def test_two_passes(dev, monkeypatch, shape):
    """The two-pass forward and backward (what larger tensors take), forced
    at shapes the one-launch kernels would otherwise run: channels split 32,
    49 and 488 ways (their partials added by a separate finalize launch), 9
    ways (added by each apply workgroup itself) and not at all."""
    monkeypatch.setenv("DKZ_BN_TWO_PASS", "1")
    _forward_case(shape, Activation.leaky, True, inplace=True, seed=90 + sum(shape))
    g_d, c_d = _backward_case(shape, Activation.leaky, seed=91 + sum(shape))
    np.testing.assert_allclose(g_d, c_d, rtol=1e-4, atol=1e-5)


def test_backward_linear_needs_no_output(dev):
    _backward_case((4, 12, 64), Activation.linear, seed=300, with_y=False)
    _backward_case((4, 12, 63), Activation.linear, seed=301, with_y=False)


def test_fused_deterministic(dev):
    """Repeated calls on the same inputs give the same bits (fixed split and
    summation order), at config 2 for the backward and config 1 forward."""
    B, F, S = CONFIG2
    n = B * F * S
    r = rng(5)
    y, delta, x, xn = normal(r, n), normal(r, n), normal(r, n), normal(r, n)
    m, v, s = normal(r, F, 0, 0.1), uniform(r, F, 0.5, 1.5), uniform(r, F, 0.5, 1.5)
    d_y, d_x, d_xn, d_m, d_v, d_s = up(y), up(x), up(xn), up(m), up(v), up(s)
    d_d = gpu.alloc(n)
    outs = [gpu.alloc(F) for _ in range(4)]
    first = None
    for _ in range(10):
        gpu.push(d_d, delta)
        for o in outs[:2]:
            gpu.fill(o, F, 0.0)
        gpu.batchnormBackward(B, F, S, Activation.leaky, d_y, d_d, d_x, d_xn, d_m, d_v, d_s, *outs)
        got = [down(o, m) for o in outs] + [down(d_d, delta)]
        if first is None:
            first = got
        else:
            for i, (a, b) in enumerate(zip(got, first)):
                assert_bitexact(a, b, f"backward repeat output {i}")
    _free(d_y, d_x, d_xn, d_m, d_v, d_s, d_d, *outs)

    B, F, S = 128, 32, 1024
    n = B * F * S
    inp = normal(r, n)
    d_in, d_out, d_x, d_xn = up(inp), gpu.alloc(n), gpu.alloc(n), gpu.alloc(n)
    d_s, d_b = up(uniform(r, F, 0.5, 1.5)), up(normal(r, F, 0, 0.1))
    stats = [gpu.alloc(F) for _ in range(4)]
    first = None
    for _ in range(10):
        gpu.fill(stats[2], F, 0.0)
        gpu.fill(stats[3], F, 1.0)
        gpu.batchnormForward(B, F, S, Activation.leaky, True, d_in, d_out, d_x, d_xn, *stats, d_s, d_b)
        got = [down(b, np.empty(F, np.float32)) for b in stats] + [down(d_out, inp)]
        if first is None:
            first = got
        else:
            for i, (a, b) in enumerate(zip(got, first)):
                assert_bitexact(a, b, f"forward repeat output {i}")
    _free(d_in, d_out, d_x, d_xn, d_s, d_b, *stats)


def test_empty_batch_follows_the_sequence(dev):
    """batch == 0 takes the per-op sequence: mean = 0 * (1/0) = NaN, variance
    0, the rolling averages move toward them (blas.zig:106-135); the backward
    adds nothing to the updates (blas.zig:73-82)."""
    F = 3
    d_m, d_v, d_rm, d_rv = gpu.alloc(F), gpu.alloc(F), up(np.ones(F, np.float32)), up(np.ones(F, np.float32))
    d_s, d_b = up(np.ones(F, np.float32)), up(np.zeros(F, np.float32))
    e = gpu.Buf()
    gpu.batchnormForward(0, F, 16, Activation.leaky, True, e, e, e, e, d_m, d_v, d_rm, d_rv, d_s, d_b)
    assert np.isnan(down(d_m, np.empty(F, np.float32))).all()
    assert_bitexact(down(d_v, np.empty(F, np.float32)), np.zeros(F, np.float32), "variance of nothing")
    c_rv = np.ones(F, np.float32)
    ref.scal(ref.ROLLING_MOMENTUM, c_rv)
    ref.axpy(ref.EMA_ALPHA, np.zeros(F, np.float32), c_rv)
    assert_bitexact(down(d_rv, c_rv), c_rv, "rolling_variance toward 0")
    d_bu = up(np.full(F, 2.0, np.float32))
    d_md, d_vd = gpu.alloc(F), gpu.alloc(F)
    gpu.batchnormBackward(0, F, 16, Activation.leaky, e, e, e, e, d_m, d_v, d_s, d_bu, d_b, d_md, d_vd)
    assert_bitexact(down(d_bu, np.empty(F, np.float32)), np.full(F, 2.0, np.float32), "no batch, no update")
    _free(d_m, d_v, d_rm, d_rv, d_s, d_b, d_bu, d_md, d_vd)


@pytest.mark.parametrize("shape, rounds", [((16, 24, 1024), 30), ((64, 128, 3136), 6)], ids=str)
def test_forward_back_to_back(dev, shape, rounds):
    """Channels split over several workgroups meet at a per-channel barrier
    inside one launch (the one-launch forward: 4 workgroups a channel at
    [16,24,1024], 2 register-resident ones at config 2's shape). Calls on
    different inputs issued back to back with no synchronisation
    (sync-after-launch off): a barrier counter not emptied, or partials read
    before they were visible, would show in a later call's statistics."""
    from darknet_zig_amd import _lib

    lib = _lib.load()
    before = lib.dkz_get_sync_after_launch()
    lib.dkz_set_sync_after_launch(0)
    try:
        B, F, S = shape
        n = B * F * S
        r = rng(123)
        xs = [normal(r, n, 0.3 * k, 1.0 + 0.1 * k) for k in range(rounds)]
        scales, biases = uniform(r, F, 0.5, 1.5), normal(r, F, 0, 0.1)
        d_s, d_b = up(scales), up(biases)
        bufs = []
        for k in range(rounds):
            d = dict(inp=up(xs[k]), out=gpu.alloc(n), x=gpu.alloc(n), xn=gpu.alloc(n), m=gpu.alloc(F),
                     v=gpu.alloc(F), rm=gpu.alloc(F), rv=gpu.alloc(F))
            bufs.append(d)
        for d in bufs:
            gpu.batchnormForward(B, F, S, Activation.leaky, True, d["inp"], d["out"], d["x"], d["xn"], d["m"], d["v"],
                                 d["rm"], d["rv"], d_s, d_b)
        gpu.sync()
        for k, d in enumerate(bufs):
            c_m, c_v = np.empty(F, np.float32), np.empty(F, np.float32)
            ref.mean(xs[k], B, F, S, c_m)
            ref.variance(xs[k], c_m, B, F, S, c_v)
            x64 = _chan64(xs[k], (B, F, S))
            g_m, g_v = down(d["m"], c_m), down(d["v"], c_v)
            assert_r5(g_m, c_m, x64.sum(axis=(0, 2)) * np.float64(np.float32(1) / np.float32(B * S)), f"mean {k}")
            dev64 = ((x64 - c_m.astype(np.float64)[None, :, None]) ** 2).sum(axis=(0, 2))
            assert_r5(g_v, c_v, dev64 * np.float64(np.float32(1) / np.float32(B * S - 1)), f"variance {k}")
            want = xs[k].copy()
            ref.normalize(want, g_m, g_v, B, F, S)
            assert_bitexact(down(d["xn"], xs[k]), want, f"x_norm {k}")
        for d in bufs:
            _free(*d.values())
        _free(d_s, d_b)
    finally:
        lib.dkz_set_sync_after_launch(before)
