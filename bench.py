#!/usr/bin/env python3
"""Benchmark of the gfx950 tensor-op layer on BASELINE.json's workload.

Headline (the one JSON line on stdout): configs[1], the batch-norm backward
layer step of darknet-zig at [64,128,56,56] fp32 -- gradient (leaky),
backward_bias, backward_scale, scale_bias(delta), mean_delta, variance_delta,
normalize_delta (convolutional.zig:280-286 + batchnorm.zig:155-174), run
through the C ABI exactly as the layer issues it. One step = one such pass
over one batch; inputs are resident in HBM and rotate over three buffer sets
(1.2 GB) so no step starts from data the 256 MB Infinity Cache still holds.

  value        algorithmic bytes of the 7-op chain x steps / wall time of the
               timed region (HIP events on the library's stream), in GB/s
  roofline     the chain's longest kernel: its algorithmic bytes / its mean
               duration from per-kernel HIP events over the same steps (less
               the event-pair overhead: the per-step excess of the event-timed
               steps over the clean ones, spread over the 7 pairs), against
               MI355X's 8 TB/s HBM peak; traffic from the committed counter
               summary profiles/traffic_bn_backward.txt
  per_op       every op of BASELINE.json's five configs timed on its own,
               cold (rotated buffers, >= 512 MB per rotation), in GB/s and as
               a fraction of 8 TB/s: sustained (back-to-back launches, the
               per-launch time of a stream of such calls) and single-launch
               (an event pair around each launch); plus rand_uniform/dropout,
               the one-pass Adam update, im2col/col2im, and shapes off the
               configs' fast paths (a 3x3/s2 max pool, a spatial softmax, a
               connected layer's bias gradient)
  gemm         dkz_gemm at config 2's convolution shapes and a large square,
               and config 2's convolutional layer forward, weight gradient
               and data gradient over the batch (the per-image loops against
               dkz_convolution_forward / _weight_gradient / _data_gradient),
               TFLOP/s
               against the 157.3 TFLOP/s fp32 matrix-core peak
  fused_bwd    the same step through dkz_batchnorm_backward (one reduction
               pass and one apply pass, 32 B/elem instead of 56)
  bn_act_gelem_s  config 1 elements / config 1 forward time and config 2
               elements / config 2 backward time: per-op (chained, and the sum
               of single-op times), the whole per-op layer forward with its
               copies and EMA, and the fused entry points
  cpu_baseline the CPU twins' C restatement (oracle/) on the same inputs on
               this host, one thread, median of 3 full config-2 chains

Algorithmic bytes count every logical fp32/int32 element read or written once
(4 B); per-channel vectors of C floats are not counted.

--per-op-traffic runs each per-op row's first three launches once between two
marker dispatches (after one untimed pass over all its rotations) and prints
the rows, for
rocprofv3 FETCH_SIZE/WRITE_SIZE runs and a kernel trace to attribute HBM
traffic and kernel time per row (profiles/traffic_per_op.md);
--copy-calibration runs the known-size copy that scales those counters.
"""

from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_GBS = 8000.0  # MI355X HBM3E, AMD public spec
METRIC = "achieved HBM GB/s (% of MI355X peak) per op; BN+act fwd+bwd GElem/s"


# ---------------------------------------------------------------------------
# HIP events (the library issues on the null stream unless told otherwise)
# ---------------------------------------------------------------------------


class Hip:
    def __init__(self):
        self.lib = C.CDLL("libamdhip64.so")
        for name, args in {
            "hipEventCreate": [C.POINTER(C.c_void_p)],
            "hipEventRecord": [C.c_void_p, C.c_void_p],
            "hipEventSynchronize": [C.c_void_p],
            "hipEventElapsedTime": [C.POINTER(C.c_float), C.c_void_p, C.c_void_p],
            "hipEventDestroy": [C.c_void_p],
            "hipDeviceSynchronize": [],
        }.items():
            fn = getattr(self.lib, name)
            fn.argtypes = args
            fn.restype = C.c_int

    def event(self) -> C.c_void_p:
        e = C.c_void_p()
        assert self.lib.hipEventCreate(C.byref(e)) == 0
        return e

    def record(self, e, stream) -> None:
        assert self.lib.hipEventRecord(e, stream) == 0

    def ms(self, a, b) -> float:
        assert self.lib.hipEventSynchronize(b) == 0
        out = C.c_float()
        assert self.lib.hipEventElapsedTime(C.byref(out), a, b) == 0
        return float(out.value)

    def sync(self) -> None:
        assert self.lib.hipDeviceSynchronize() == 0


# ---------------------------------------------------------------------------
# workloads
# ---------------------------------------------------------------------------


def gen(seed: int):
    return np.random.default_rng(seed)


class Device:
    """Device buffers of one run, uploaded once and freed at exit."""

    def __init__(self, gpu):
        self.gpu = gpu
        self.bufs = []

    def up(self, a: np.ndarray):
        b = self.gpu.make(np.ascontiguousarray(a))
        self.bufs.append(b)
        return b

    def zeros(self, n: int):
        b = self.gpu.alloc(n)
        self.bufs.append(b)
        return b

    def clone(self, b, n: int, k: int):
        """k copies of b made on the device (copy kernel)."""
        out = [b]
        for _ in range(k - 1):
            c = self.zeros(n)
            self.gpu.copy(n, b, c)
            out.append(c)
        return out

    def free(self):
        for b in self.bufs:
            self.gpu.free(b)
        self.bufs = []


def rotations(bytes_per_set: int, min_total: int = 512 << 20, lo: int = 2) -> int:
    return max(lo, -(-min_total // max(bytes_per_set, 1)))


def config2_host(seed=2):
    B, F, S = 64, 128, 56 * 56
    n = B * F * S
    r = gen(seed)
    y = r.normal(0, 1, n).astype(np.float32)
    y = np.where(y > 0, y, np.float32(0.1) * y).astype(np.float32)  # leaky output
    delta = r.normal(0, 1, n).astype(np.float32)
    x = r.normal(0, 1, n).astype(np.float32)
    x_norm = r.normal(0, 1, n).astype(np.float32)
    scales = r.uniform(0.5, 1.5, F).astype(np.float32)
    xm = x.reshape(B, F, S).astype(np.float64)
    mean = xm.mean(axis=(0, 2)).astype(np.float32)
    var = xm.var(axis=(0, 2), ddof=1).astype(np.float32)
    return dict(B=B, F=F, S=S, n=n, y=y, delta=delta, x=x, x_norm=x_norm, scales=scales, mean=mean, var=var)


def config2_chain_ops(gpu, d, h):
    """The 7 ops of one BN backward step on device set d; (name, bytes, fn)."""
    from darknet_zig_amd.activations import Activation

    B, F, S, n = h["B"], h["F"], h["S"], h["n"]
    E = 4 * n
    return [
        ("gradient_array(leaky)", 3 * E, lambda: gpu.gradientArray(d["y"], n, Activation.leaky, d["delta"])),
        ("backward_bias", E, lambda: gpu.backwardBias(d["bu"], d["delta"], B, F, S)),
        ("backward_scale", 2 * E, lambda: gpu.backwardScale(d["x_norm"], d["delta"], B, F, S, d["su"])),
        ("scale_bias(delta)", 2 * E, lambda: gpu.scaleBias(d["delta"], d["scales"], B, F, S)),
        ("mean_delta", E, lambda: gpu.meanDelta(d["delta"], d["var"], B, F, S, d["md"])),
        ("variance_delta", 2 * E, lambda: gpu.varianceDelta(d["x"], d["delta"], d["mean"], d["var"], B, F, S, d["vd"])),
        ("normalize_delta", 3 * E,
         lambda: gpu.normalizeDelta(d["x"], d["mean"], d["var"], d["md"], d["vd"], B, F, S, d["delta"])),
    ]


def fused_backward(gpu, d, h):
    """The same layer step through the fused entry point (one reduction pass
    over y, delta, x_norm, x; one apply pass over y, delta, x): 32 B/elem."""
    from darknet_zig_amd.activations import Activation

    gpu.batchnormBackward(h["B"], h["F"], h["S"], Activation.leaky, d["y"], d["delta"], d["x"], d["x_norm"],
                          d["mean"], d["var"], d["scales"], d["bu"], d["su"], d["md"], d["vd"])


def upload_config2(dev, h, sets: int):
    F, n = h["F"], h["n"]
    big = {k: dev.up(h[k]) for k in ("y", "delta", "x", "x_norm")}
    small = {k: dev.up(h[k]) for k in ("scales", "mean", "var")}
    out = []
    clones = {k: dev.clone(v, n, sets) for k, v in big.items()}
    for s in range(sets):
        d = {k: clones[k][s] for k in big}
        d.update(small)
        d.update(bu=dev.zeros(F), su=dev.zeros(F), md=dev.zeros(F), vd=dev.zeros(F))
        out.append(d)
    return out


# ---------------------------------------------------------------------------
# timing
# ---------------------------------------------------------------------------


def time_chain(hip, stream, chains, steps, warmup):
    """Clean timed region: `steps` chain passes, events only at its ends."""
    for k in range(warmup):
        for _, _, fn in chains[k % len(chains)]:
            fn()
    hip.sync()
    a, b = hip.event(), hip.event()
    hip.record(a, stream)
    for k in range(steps):
        for _, _, fn in chains[k % len(chains)]:
            fn()
    hip.record(b, stream)
    ms = hip.ms(a, b)
    hip.sync()
    return ms


def time_chain_per_kernel(hip, stream, chains, steps):
    """Per-kernel HIP events around every launch of `steps` chain passes."""
    nops = len(chains[0])
    evs = [(hip.event(), hip.event()) for _ in range(steps * nops)]
    hip.sync()
    i = 0
    for k in range(steps):
        for _, _, fn in chains[k % len(chains)]:
            hip.record(evs[i][0], stream)
            fn()
            hip.record(evs[i][1], stream)
            i += 1
    hip.sync()
    per = [[] for _ in range(nops)]
    for j, (a, b) in enumerate(evs):
        per[j % nops].append(hip.ms(a, b))
    return [statistics.mean(p) for p in per]


def time_seq(hip, stream, seqs, steps, warmup=3):
    """Mean time (ms) of one pass of an op sequence, cycling over rotated sets."""
    for k in range(warmup):
        for fn in seqs[k % len(seqs)]:
            fn()
    hip.sync()
    a, b = hip.event(), hip.event()
    hip.record(a, stream)
    for k in range(steps):
        for fn in seqs[k % len(seqs)]:
            fn()
    hip.record(b, stream)
    ms = hip.ms(a, b)
    hip.sync()
    return ms / steps


def time_op(hip, stream, fns, launches, warmup=3):
    """Mean per-launch time (ms) of an op cycling over rotated inputs."""
    for k in range(warmup):
        fns[k % len(fns)]()
    hip.sync()
    evs = [(hip.event(), hip.event()) for _ in range(launches)]
    for k in range(launches):
        hip.record(evs[k][0], stream)
        fns[k % len(fns)]()
        hip.record(evs[k][1], stream)
    hip.sync()
    return statistics.mean(hip.ms(a, b) for a, b in evs)


def gbs(nbytes: int, ms: float) -> float:
    return nbytes / (ms * 1e-3) / 1e9


# ---------------------------------------------------------------------------
# per-op table over the five configs
# ---------------------------------------------------------------------------


# Traffic mode: a row's launches sit between two marker dispatches -- a fill
# of a misaligned buffer (no row fills one), which runs the one-lane-per-
# element fill kernel on exactly MARK_BASE + 2*row (+1 for the end)
# workgroups of 256, about 1 MB -- so that a profile (rocprofv3 --pmc
# FETCH_SIZE / WRITE_SIZE, or a kernel trace) can attribute every dispatch to
# its row from the dispatch order and grid sizes alone. Every rotation runs
# once, untimed, before the begin marker: the traced passes then find their
# pages mapped (as in a stream of such calls) but their data, at least
# 512 MB back, out of the 256 MB Infinity Cache.
MARK_BASE = 1000
TRAFFIC_PASSES = 3


def per_op_table(gpu, hip, stream, launches: int, traffic=None):
    """The per-op table; with `traffic` (a list), no timing: each row's first
    TRAFFIC_PASSES launches (or call sequences) run once between markers and
    the row is appended to `traffic`."""
    from darknet_zig_amd.activations import Activation

    rows = {}
    if traffic is not None:
        mark_buf = gpu.alloc((MARK_BASE + 256) * 256 + 1)

    def marker(grid):
        gpu.fill(mark_buf.offset(1), grid * 256, 0.0)

    def traced(cfg, name, nbytes, seqs):
        i = len(traffic)
        passes = min(TRAFFIC_PASSES, len(seqs))
        for seq in seqs:
            for fn in seq:
                fn()
        hip.sync()
        marker(MARK_BASE + 2 * i)
        for seq in seqs[:passes]:
            for fn in seq:
                fn()
        marker(MARK_BASE + 2 * i + 1)
        hip.sync()
        traffic.append({"row": f"{cfg}/{name}", "bytes": nbytes, "passes": passes, "begin_grid": MARK_BASE + 2 * i})
        print(f"traffic row {i}: {cfg}/{name}", file=sys.stderr, flush=True)

    def row(cfg, name, nbytes, ms, single_ms=None):
        g = gbs(nbytes, ms)
        rows[f"{cfg}/{name}"] = r = {"us": round(ms * 1e3, 3), "GB/s": round(g, 1), "frac": round(g / PEAK_GBS, 4),
                                     "bytes": nbytes}
        if single_ms is not None:
            r["single_launch_us"] = round(single_ms * 1e3, 3)
            r["single_launch_frac"] = round(gbs(nbytes, single_ms) / PEAK_GBS, 4)

    def add(cfg, name, nbytes, fns):
        """One op over rotated inputs: sustained (back-to-back launches, events
        around the run: the per-launch figure of a stream of such calls) and
        single-launch (an event pair around each launch, which also times
        ~2 us of dispatch and completion)."""
        if traffic is not None:
            return traced(cfg, name, nbytes, [[f] for f in fns])
        k = max(launches, len(fns))
        row(cfg, name, nbytes, time_seq(hip, stream, [[f] for f in fns], k), time_op(hip, stream, fns, k))

    def add_seq(cfg, name, nbytes, seqs):
        """A call sequence (or a multi-launch entry point), events only around
        the whole timed region, as a layer would issue it back to back."""
        if traffic is not None:
            return traced(cfg, name, nbytes, seqs)
        row(cfg, name, nbytes, time_seq(hip, stream, seqs, max(launches, len(seqs))))

    # -- config 1: BN forward + leaky, [128,32,32,32], x~N(0,1), gamma~U(0.5,1.5), beta~N(0,0.1)
    dev = Device(gpu)
    B, F, S = 128, 32, 1024
    n = B * F * S
    E = 4 * n
    r = gen(1)
    x = r.normal(0, 1, n).astype(np.float32)
    R = rotations(E)
    xs = dev.clone(dev.up(x), n, R)
    gam, bet = dev.up(r.uniform(0.5, 1.5, F).astype(np.float32)), dev.up(r.normal(0, 0.1, F).astype(np.float32))
    m, v = dev.zeros(F), dev.zeros(F)
    gpu.mean(xs[0], B, F, S, m)
    gpu.variance(xs[0], m, B, F, S, v)
    cfg = "cfg1_bn_fwd[128,32,32,32]"
    add(cfg, "mean", E, [lambda b=b: gpu.mean(b, B, F, S, m) for b in xs])
    add(cfg, "variance", E, [lambda b=b: gpu.variance(b, m, B, F, S, v) for b in xs])
    add(cfg, "normalize", 2 * E, [lambda b=b: gpu.normalize(b, m, v, B, F, S) for b in xs])
    add(cfg, "scale_bias", 2 * E, [lambda b=b: gpu.scaleBias(b, gam, B, F, S) for b in xs])
    add(cfg, "add_bias", 2 * E, [lambda b=b: gpu.addBias(b, bet, B, F, S) for b in xs])
    add(cfg, "activate(leaky)", 2 * E, [lambda b=b: gpu.activateArray(b, n, Activation.leaky) for b in xs])
    ys = [dev.zeros(n) for _ in range(R)]
    add(cfg, "copy (x, x_norm)", 2 * E, [lambda a=a, b=b: gpu.copy(n, a, b) for a, b in zip(xs, ys)])
    # the named ops in the layer's order on one tensor (batchnorm.zig:137-152 + activate)
    seqs = [[lambda b=b: gpu.mean(b, B, F, S, m), lambda b=b: gpu.variance(b, m, B, F, S, v),
             lambda b=b: gpu.normalize(b, m, v, B, F, S), lambda b=b: gpu.scaleBias(b, gam, B, F, S),
             lambda b=b: gpu.addBias(b, bet, B, F, S), lambda b=b: gpu.activateArray(b, n, Activation.leaky)]
            for b in xs]
    add_seq(cfg, "chain: mean,variance,normalize,scale_bias,add_bias,leaky", 10 * E, seqs)
    rm, rv = dev.zeros(F), dev.zeros(F)
    mom, alpha = 0.99, float(np.float32(1) - np.float32(0.99))  # batchnorm.zig:16, :141

    def ema():
        gpu.scal(F, mom, rm)
        gpu.axpy(F, alpha, m, rm)
        gpu.scal(F, mom, rv)
        gpu.axpy(F, alpha, v, rv)

    add(cfg, "ema scal+axpy (C floats)", 4 * 3 * F, [ema])
    # the whole layer forward as batchnorm.zig:129-153 issues it (copies and
    # EMA included) and then the activation, against the fused entry point
    xcs, xns = [dev.zeros(n) for _ in range(R)], [dev.zeros(n) for _ in range(R)]
    seqs = [[lambda b=b, c=c: gpu.copy(n, b, c), lambda b=b: gpu.mean(b, B, F, S, m),
             lambda b=b: gpu.variance(b, m, B, F, S, v), ema, lambda b=b: gpu.normalize(b, m, v, B, F, S),
             lambda b=b, c=c: gpu.copy(n, b, c), lambda b=b: gpu.scaleBias(b, gam, B, F, S),
             lambda b=b: gpu.addBias(b, bet, B, F, S), lambda b=b: gpu.activateArray(b, n, Activation.leaky)]
            for b, c in zip(xs, xcs)]
    add_seq(cfg, "layer sequence: copy,mean,variance,ema,normalize,copy,scale_bias,add_bias,leaky", 14 * E, seqs)
    add_seq("fused", "cfg1 batchnorm_forward(train, leaky): stats + apply", 5 * E,
            [[lambda b=b, c=c, xn=xn: gpu.batchnormForward(B, F, S, Activation.leaky, True, b, b, c, xn, m, v, rm, rv,
                                                           gam, bet)] for b, c, xn in zip(xs, xcs, xns)])
    dev.free()

    # -- config 2: BN backward ops on their own
    h = config2_host()
    dev = Device(gpu)
    sets = upload_config2(dev, h, 3)
    chains = [config2_chain_ops(gpu, d, h) for d in sets]
    for j, (name, nbytes, _) in enumerate(chains[0]):
        add("cfg2_bn_bwd[64,128,56,56]", name, nbytes, [c[j][2] for c in chains])
    add_seq("fused", "cfg2 batchnorm_backward(leaky): sums + apply", 8 * 4 * h["n"],
            [[lambda d=d: fused_backward(gpu, d, h)] for d in sets])
    # config 1's forward ops on the largest batch-norm tensor of the configs
    # (config 2's x): each op at its largest shape, as the north star asks
    B2, F2, S2, n2 = 64, 128, 56 * 56, h["n"]
    cfg = "cfg1_ops_at_cfg2_shape[64,128,56,56]"
    bias2 = dev.up(gen(7).normal(0, 0.1, F2).astype(np.float32))
    add(cfg, "mean", 4 * n2, [lambda d=d: gpu.mean(d["x"], B2, F2, S2, d["md"]) for d in sets])
    add(cfg, "variance", 4 * n2, [lambda d=d: gpu.variance(d["x"], d["mean"], B2, F2, S2, d["vd"]) for d in sets])
    add(cfg, "normalize", 8 * n2, [lambda d=d: gpu.normalize(d["x_norm"], d["mean"], d["var"], B2, F2, S2)
                                   for d in sets])
    add(cfg, "add_bias", 8 * n2, [lambda d=d: gpu.addBias(d["x_norm"], bias2, B2, F2, S2) for d in sets])
    add(cfg, "activate(leaky)", 8 * n2, [lambda d=d: gpu.activateArray(d["x_norm"], n2, Activation.leaky)
                                         for d in sets])
    dev.free()

    # -- config 3: softmax + cross-entropy delta, [256,1000], logits ~N(0,4)
    dev = Device(gpu)
    b3, c3 = 256, 1000
    n3 = b3 * c3
    r = gen(3)
    logits = r.normal(0, 4.0, n3).astype(np.float32)
    truth = np.zeros(n3, np.float32)
    truth[np.arange(b3) * c3 + r.integers(0, c3, b3)] = 1.0
    R = rotations(4 * 4 * n3)
    ls = dev.clone(dev.up(logits), n3, R)
    ps = [dev.zeros(n3) for _ in range(R)]
    ts = dev.clone(dev.up(truth), n3, R)
    ds_ = [dev.zeros(n3) for _ in range(R)]
    es = [dev.zeros(n3) for _ in range(R)]
    cfg = "cfg3_softmax[256,1000]"
    add(cfg, "softmax", 2 * 4 * n3, [lambda a=a, p=p: gpu.softmax(a, c3, b3, c3, 1, c3, 1, 1.0, p) for a, p in zip(ls, ps)])
    add(cfg, "softmax_x_ent", 4 * 4 * n3,
        [lambda p=p, t=t, d=d, e=e: gpu.softmaxCrossEntropy(n3, p, t, d, e) for p, t, d, e in zip(ps, ts, ds_, es)])
    add_seq(cfg, "chain: softmax, softmax_x_ent (the layer's two calls)", 6 * 4 * n3,
            [[lambda a=a, p=p: gpu.softmax(a, c3, b3, c3, 1, c3, 1, 1.0, p),
              lambda p=p, t=t, d=d, e=e: gpu.softmaxCrossEntropy(n3, p, t, d, e)]
             for a, p, t, d, e in zip(ls, ps, ts, ds_, es)])
    add("fused", "cfg3 softmax_layer_forward (softmax + loss in one pass)", 5 * 4 * n3,
        [lambda a=a, p=p, t=t, d=d, e=e: gpu.softmaxLayerForward(b3, c3, 1, 1.0, a, t, p, d, e)
         for a, p, t, d, e in zip(ls, ps, ts, ds_, es)])
    dev.free()
    # the same two ops at a larger batch (config 3 is a 2 MB tensor, which one
    # launch cannot stream at full rate): each op at a large shape
    dev = Device(gpu)
    b3l = 8192
    n3l = b3l * c3
    logits = r.normal(0, 4.0, n3l).astype(np.float32)
    truth = np.zeros(n3l, np.float32)
    truth[np.arange(b3l) * c3 + r.integers(0, c3, b3l)] = 1.0
    R = rotations(4 * 4 * n3l)
    ls = dev.clone(dev.up(logits), n3l, R)
    ps = [dev.zeros(n3l) for _ in range(R)]
    ts = dev.clone(dev.up(truth), n3l, R)
    ds_ = [dev.zeros(n3l) for _ in range(R)]
    es = [dev.zeros(n3l) for _ in range(R)]
    cfg = f"cfg3_ops_at[{b3l},1000]"
    add(cfg, "softmax", 2 * 4 * n3l,
        [lambda a=a, p=p: gpu.softmax(a, c3, b3l, c3, 1, c3, 1, 1.0, p) for a, p in zip(ls, ps)])
    add(cfg, "softmax_x_ent", 4 * 4 * n3l,
        [lambda p=p, t=t, d=d, e=e: gpu.softmaxCrossEntropy(n3l, p, t, d, e) for p, t, d, e in zip(ps, ts, ds_, es)])
    dev.free()

    # -- config 4: SGD over 25e6 floats ~N(0,0.05), and the stride-2 shortcut
    dev = Device(gpu)
    n4 = 25_000_000
    r = gen(4)
    R = rotations(2 * 4 * n4)
    ws = dev.clone(dev.up(r.normal(0, 0.05, n4).astype(np.float32)), n4, R)
    dws = dev.clone(dev.up(r.normal(0, 0.05, n4).astype(np.float32)), n4, R)
    batch, lr, decay, momentum = 64, 0.1, 0.0005, 0.9
    cfg = "cfg4_sgd[25e6]"
    add(cfg, "axpy(-decay*batch, w, dw)", 3 * 4 * n4,
        [lambda w=w, d=d: gpu.axpy(n4, -decay * batch, w, d) for w, d in zip(ws, dws)])
    add(cfg, "axpy(lr/batch, dw, w)", 3 * 4 * n4, [lambda w=w, d=d: gpu.axpy(n4, lr / batch, d, w) for w, d in zip(ws, dws)])
    add(cfg, "scal(momentum, dw)", 2 * 4 * n4, [lambda d=d: gpu.scal(n4, momentum, d) for d in dws])
    seqs = [[lambda w=w, d=d: gpu.axpy(n4, -decay * batch, w, d), lambda w=w, d=d: gpu.axpy(n4, lr / batch, d, w),
             lambda d=d: gpu.scal(n4, momentum, d)] for w, d in zip(ws, dws)]
    add_seq(cfg, "chain: axpy,axpy,scal (one SGD step)", 8 * 4 * n4, seqs)
    dev.free()
    dev = Device(gpu)
    sb, w1, c1, w2, c2 = 64, 28, 256, 14, 512
    na, no = sb * c1 * w1 * w1, sb * c2 * w2 * w2
    s4 = sb * c1 * w2 * w2
    R = rotations(4 * (na + no))
    adds = dev.clone(dev.up(r.normal(0, 0.05, na).astype(np.float32)), na, R)
    outs = dev.clone(dev.up(r.normal(0, 0.05, no).astype(np.float32)), no, R)
    add("cfg4_shortcut[64,256,28,28]->[64,512,14,14]", "shortcut", 3 * 4 * s4,
        [lambda a=a, o=o: gpu.shortcut(sb, w1, w1, c1, a, w2, w2, c2, 1.0, 1.0, o) for a, o in zip(adds, outs)])
    dev.free()

    # -- config 5: pooling at [256,512,28,28], inputs ~U(-1,1)
    dev = Device(gpu)
    pb, pc, ph = 256, 512, 28
    nin = pb * pc * ph * ph
    oh = (ph + 1 - 2) // 2 + 1
    nout = pb * pc * oh * oh
    r = gen(5)
    R = 2
    ins = dev.clone(dev.up(r.uniform(-1, 1, nin).astype(np.float32)), nin, R)
    outs = [dev.zeros(nout) for _ in range(R)]
    idxs = [dev.zeros(nout) for _ in range(R)]
    dls = dev.clone(dev.up(r.uniform(-1, 1, nout).astype(np.float32)), nout, R)
    cfg = "cfg5_pool[256,512,28,28]"
    add(cfg, "maxpool_fwd 2x2/s2", 4 * (nin + 2 * nout),
        [lambda i=i, o=o, x=x: gpu.forwardMaxpool(nout, ph, ph, pc, 2, 2, 1, i, o, x) for i, o, x in zip(ins, outs, idxs)])
    add(cfg, "maxpool_bwd", 4 * (2 * nout + 2 * nin),
        [lambda d=d, p=p, x=x: gpu.backwardMaxpool(nin, ph, ph, pc, 2, 2, 1, d, p, x) for d, p, x in zip(dls, ins, idxs)])
    rows_ = pb * pc
    avg = [dev.zeros(rows_) for _ in range(R)]
    add(cfg, "avgpool_fwd (global)", 4 * (nin + rows_),
        [lambda i=i, a=a: gpu.forwardAvgpool(rows_, ph, ph, pc, i, a) for i, a in zip(ins, avg)])
    add(cfg, "avgpool_bwd (global)", 4 * (2 * nin + rows_),
        [lambda i=i, a=a: gpu.backwardAvgpool(rows_, ph, ph, pc, i, a) for i, a in zip(ins, avg)])
    # the dropout layer (misc.zig:128-141) on a config-5-sized activation
    seeds = [1234567 + j for j in range(R)]
    add("dropout[256,512,28,28]", "rand_uniform", 4 * nin,
        [lambda i=i, s_=s_: gpu.randUniform(nin, i, s_) for i, s_ in zip(ins, seeds)])
    add("dropout[256,512,28,28]", "dropout", 3 * 4 * nin,
        [lambda i=i, o=o: gpu.dropout(i, nin, o, 0.5, 2.0) for i, o in zip(ins, ins[::-1])])
    dev.free()

    # -- shapes off the configs' fast paths: a 3x3/s2 max pool (the generic
    # kernels), a detection head's spatial softmax (groups of 85 classes, 169
    # positions apart) and a connected layer's bias gradient (spatial 1)
    dev = Device(gpu)
    r = gen(6)
    gb, gc, gh, gsz, gst, gpad = 64, 128, 56, 3, 2, 2
    gin = gb * gc * gh * gh
    goh = (gh + gpad - gsz) // gst + 1
    gout = gb * gc * goh * goh
    R = rotations(4 * (gin + 2 * gout))
    gins = [dev.up(r.uniform(-1, 1, gin).astype(np.float32)) for _ in range(R)]
    gouts = [dev.zeros(gout) for _ in range(R)]
    gidx = [dev.zeros(gout) for _ in range(R)]
    cfg = "pool[64,128,56,56]"
    add(cfg, "maxpool_fwd 3x3/s2 (generic)", 4 * (gin + 2 * gout),
        [lambda i=i, o=o, x=x: gpu.forwardMaxpool(gout, gh, gh, gc, gst, gsz, gpad, i, o, x)
         for i, o, x in zip(gins, gouts, gidx)])
    add(cfg, "maxpool_bwd 3x3/s2 (generic)", 4 * (2 * gout + 2 * gin),
        [lambda d=d, p=p, x=x: gpu.backwardMaxpool(gin, gh, gh, gc, gst, gsz, gpad, d, p, x)
         for d, p, x in zip(gouts, gins, gidx)])
    dev.free()
    dev = Device(gpu)
    sb, sc, ss = 64, 85, 169
    sn = sb * sc * ss
    R = rotations(8 * sn)
    sxs = [dev.up(r.normal(0, 2, sn).astype(np.float32)) for _ in range(R)]
    sys_ = [dev.zeros(sn) for _ in range(R)]
    add(f"softmax[{sb},{sc},13,13]", "spatial softmax (groups across positions)", 2 * 4 * sn,
        [lambda x=x, y=y: gpu.softmax(x, sc, sb, sc * ss, ss, 1, ss, 1.0, y) for x, y in zip(sxs, sys_)])
    dev.free()
    dev = Device(gpu)
    cb, cf = 256, 1000
    R = rotations(4 * cb * cf)
    cds = [dev.up(r.normal(0, 1, cb * cf).astype(np.float32)) for _ in range(R)]
    cu = dev.zeros(cf)
    add(f"connected[{cb},{cf}]", "backward_bias (spatial 1)", 4 * (cb * cf + 2 * cf),
        [lambda d=d: gpu.backwardBias(cu, d, cb, cf, 1) for d in cds])
    dev.free()

    # -- the Adam update (gpu.zig:804-830) over config 4's 25e6 weights, one pass
    dev = Device(gpu)
    r = gen(6)
    R = rotations(4 * 4 * n4)
    vecs = [[dev.up(r.normal(0, s_, n4).astype(np.float32)) for s_ in (0.05, 0.05, 0.01, 0.001)] for _ in range(R)]
    add("cfg4_adam[25e6]", "adam_update (one pass over w, d, m, v)", 8 * 4 * n4,
        [lambda v=v: gpu.adamUpdate(v[0], v[1], v[2], v[3], 0.9, 0.999, 1e-7, 0.0005, 0.001, n4, 64, 3)
         for v in vecs])
    dev.free()

    # -- im2col / col2im of config 2's layer, one image (the layers call them per image)
    dev = Device(gpu)
    C2, H2, K2 = 128, 56, 3
    ncol = C2 * K2 * K2 * H2 * H2
    nim = C2 * H2 * H2
    R = rotations(4 * (ncol + nim))
    ims = [dev.up(r.uniform(-1, 1, nim).astype(np.float32)) for _ in range(R)]
    cols = [dev.zeros(ncol) for _ in range(R)]
    cfg = "conv[128,56,56]k3s1p1"
    add(cfg, "im2col (one image)", 4 * (nim + ncol),
        [lambda i=i, c=c: gpu.im2col(i, C2, H2, H2, K2, 1, 1, c) for i, c in zip(ims, cols)])
    add(cfg, "col2im (one image)", 4 * (ncol + 2 * nim),
        [lambda i=i, c=c: gpu.col2im(c, C2, H2, H2, K2, 1, 1, i) for i, c in zip(ims, cols)])
    dev.free()
    if traffic is not None:
        gpu.free(mark_buf)
    return rows


GEMM_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix-core peak


def gemm_table(gpu, hip, stream):
    """dkz_gemm at the shapes a convolutional layer issues for config 2's layer
    (forward, backward data, weight gradient; one image each, as
    convolutional.zig issues them) and at a large square size: TFLOP/s
    against the fp32 matrix-core peak."""
    rows = {}
    shapes = [("conv fwd NN 128x3136x1152", False, False, 128, 3136, 1152),
              ("conv bwd-data TN 1152x3136x128", True, False, 1152, 3136, 128),
              ("conv weight-grad NT 128x1152x3136", False, True, 128, 1152, 3136),
              ("square NN 4096x4096x4096", False, False, 4096, 4096, 4096),
              ("square NN 8192x8192x4096", False, False, 8192, 8192, 4096)]
    r = gen(7)
    for name, ta, tb, m, n, k in shapes:
        dev = Device(gpu)
        a = dev.up(r.uniform(-1, 1, m * k).astype(np.float32))
        b = dev.up(r.uniform(-1, 1, k * n).astype(np.float32))
        c = dev.zeros(m * n)
        lda, ldb = (m if ta else k), (k if tb else n)
        flops = 2 * m * n * k
        reps = max(3, min(100, int(3e11 / flops)))
        ms = time_seq(hip, stream, [[lambda: gpu.gemm(ta, tb, m, n, k, 1.0, a, lda, b, ldb, 1.0, c, n)]], reps)
        tf = flops / (ms * 1e-3) / 1e12
        rows[name] = {"us": round(ms * 1e3, 2), "TFLOP/s": round(tf, 2), "frac": round(tf / GEMM_PEAK_TFLOPS, 4),
                      "flops": flops}
        dev.free()
    # config 2's convolutional layer forward, the whole batch: the per-image
    # im2col + gemm loop of convolutional.zig:249-260 against one
    # dkz_convolution_forward call (implicit im2col, no workspace)
    B, C, H, F, K = 64, 128, 56, 128, 3
    hw, kk = H * H, C * K * K
    dev = Device(gpu)
    x = dev.up(r.uniform(-1, 1, B * C * hw).astype(np.float32))
    w = dev.up(r.uniform(-1, 1, F * kk).astype(np.float32))
    y = dev.zeros(B * F * hw)
    ws = dev.zeros(kk * hw)
    flops = 2 * B * F * hw * kk

    def per_image():
        for i in range(B):
            gpu.im2col(x.offset(i * C * hw), C, H, H, K, 1, 1, ws)
            gpu.gemm(False, False, F, hw, kk, 1.0, w, kk, ws, hw, 1.0, y.offset(i * F * hw), hw)

    # ... and its weight gradient (convolutional.zig:288-297): the per-image
    # im2col + gemm(false, true, beta 1) loop against one
    # dkz_convolution_weight_gradient call (split-K, partial tiles in the
    # library's scratch); y stands in for delta
    wu = dev.zeros(F * kk)

    def per_image_wgrad():
        for i in range(B):
            gpu.im2col(x.offset(i * C * hw), C, H, H, K, 1, 1, ws)
            gpu.gemm(False, True, F, kk, hw, 1.0, y.offset(i * F * hw), hw, ws, hw, 1.0, wu, kk)

    # ... and its data gradient (convolutional.zig:299-305): per image
    # gemm(true, false, beta 0) into the workspace and col2im into the
    # previous layer's delta, against one dkz_convolution_data_gradient call
    # (y stands in for delta, x for the previous delta)
    def per_image_dgrad():
        for i in range(B):
            gpu.gemm(True, False, kk, hw, F, 1.0, w, kk, y.offset(i * F * hw), hw, 0.0, ws, hw)
            gpu.col2im(ws, C, H, H, K, 1, 1, x.offset(i * C * hw))

    for name, fn, reps in (("conv layer fwd [64,128,56,56]->128 3x3: per-image im2col+gemm", per_image, 3),
                           ("conv layer fwd [64,128,56,56]->128 3x3: convolution_forward",
                            lambda: gpu.convolutionForward(B, 1, C, H, H, F, K, 1, 1, w, x, y), 10),
                           ("conv layer wgrad [64,128,56,56]->128 3x3: per-image im2col+gemm", per_image_wgrad, 3),
                           ("conv layer wgrad [64,128,56,56]->128 3x3: convolution_weight_gradient",
                            lambda: gpu.convolutionWeightGradient(B, 1, C, H, H, F, K, 1, 1, y, x, wu), 10),
                           ("conv layer dgrad [64,128,56,56]->128 3x3: per-image gemm+col2im", per_image_dgrad, 3),
                           ("conv layer dgrad [64,128,56,56]->128 3x3: convolution_data_gradient",
                            lambda: gpu.convolutionDataGradient(B, 1, C, H, H, F, K, 1, 1, w, y, x), 10)):
        ms = time_seq(hip, stream, [[fn]], reps)
        tf = flops / (ms * 1e-3) / 1e12
        rows[name] = {"us": round(ms * 1e3, 2), "TFLOP/s": round(tf, 2), "frac": round(tf / GEMM_PEAK_TFLOPS, 4),
                      "flops": flops}
    dev.free()
    return rows


# ---------------------------------------------------------------------------
# CPU baseline: the CPU twins (C restatement) on the same config-2 inputs
# ---------------------------------------------------------------------------


def cpu_baseline(h, repeats=3):
    from darknet_zig_amd.activations import Activation
    from oracle import ref

    B, F, S = h["B"], h["F"], h["S"]
    chain_bytes = 14 * 4 * h["n"]
    times = []
    for _ in range(repeats):
        d = h["delta"].copy()
        bu, su = np.zeros(F, np.float32), np.zeros(F, np.float32)
        md, vd = np.empty(F, np.float32), np.empty(F, np.float32)
        t0 = time.perf_counter()
        ref.gradientArray(h["y"], Activation.leaky, d)
        ref.backwardBias(bu, d, B, F, S)
        ref.backwardScale(h["x_norm"], d, B, F, S, su)
        ref.scaleBias(d, h["scales"], B, F, S)
        ref.meanDelta(d, h["var"], B, F, S, md)
        ref.varianceDelta(h["x"], d, h["mean"], h["var"], B, F, S, vd)
        ref.normalizeDelta(h["x"], h["mean"], h["var"], md, vd, B, F, S, d)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(chain_bytes / t / 1e9, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"full config-2 chain (7 ops over [64,128,56,56]) on the same inputs, median of {repeats} runs, "
                   f"{t * 1e3:.1f} ms per chain, 1 thread of {os.cpu_count()} ({model}); C restatement of the Zig "
                   "CPU twins built -O3 -march=x86-64-v3 -ffp-contract=off"),
    }


# ---------------------------------------------------------------------------


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--op-launches", type=int, default=24, help="timed launches per op in the per-op table")
    ap.add_argument("--no-per-op", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--per-op-only", action="store_true",
                    help="only run the per-op table (for a kernel trace without the chain's launches)")
    ap.add_argument("--per-op-traffic", action="store_true",
                    help="only run each per-op row's first launches once, between marker dispatches "
                         "(for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE per row)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run dkz_copy over MIB MiB (x4 launches, rotated): the known-size kernel "
                         "that scales rocprofv3's FETCH_SIZE/WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(every op runs on one device's share); run with --gpus 1.", file=sys.stderr)
        return 2

    from darknet_zig_amd import gpu

    gpu.init(0)
    hip = Hip()
    stream = C.c_void_p(None)  # the library's stream: the null stream

    if args.copy_calibration:
        n = args.copy_calibration << 18  # floats
        dev = Device(gpu)
        src = [dev.zeros(n) for _ in range(2)]
        dst = [dev.zeros(n) for _ in range(2)]
        fns = [lambda a=a, b=b: gpu.copy(n, a, b) for a, b in zip(src, dst)]
        ms = time_op(hip, stream, fns, 4, warmup=0)
        dev.free()
        print(json.dumps({"copy_calibration": {"bytes_read": 4 * n, "bytes_written": 4 * n, "launches": 4,
                                               "us": round(ms * 1e3, 2)}}), flush=True)
        return 0

    if args.per_op_traffic:
        traffic = []
        per_op_table(gpu, hip, stream, 1, traffic)
        print(json.dumps({"per_op_traffic": traffic, "mark_base": MARK_BASE}), flush=True)
        return 0

    if args.per_op_only:
        print(json.dumps({"per_op": per_op_table(gpu, hip, stream, args.op_launches),
                          "gemm": gemm_table(gpu, hip, stream)}), flush=True)
        return 0

    h = config2_host()
    dev = Device(gpu)
    sets = upload_config2(dev, h, 3)
    chains = [config2_chain_ops(gpu, d, h) for d in sets]
    chain_bytes = sum(b for _, b, _ in chains[0])
    hip.sync()
    ms = time_chain(hip, stream, chains, args.steps, args.warmup)
    per_kernel_ms = time_chain_per_kernel(hip, stream, chains, args.steps)
    fused_ms = time_seq(hip, stream, [[lambda d=d: fused_backward(gpu, d, h)] for d in sets], args.steps,
                        args.warmup)
    dev.free()

    names = [nm for nm, _, _ in chains[0]]
    byts = [b for _, b, _ in chains[0]]
    # A HIP event pair around a launch also times the dispatch and completion
    # latency that back-to-back launches hide. The clean region runs the same
    # kernels without inner events, so the per-pair overhead is the difference
    # of the two per-step times spread over the pairs of a step.
    overhead_ms = max(0.0, (sum(per_kernel_ms) - ms / args.steps) / len(names))
    kernel_ms = [t - overhead_ms for t in per_kernel_ms]
    dom = max(range(len(names)), key=lambda j: kernel_ms[j])
    achieved = gbs(byts[dom], kernel_ms[dom])
    traffic = None
    tfile = ROOT / "profiles" / "traffic_bn_backward.txt"
    if tfile.exists():
        for line in tfile.read_text().splitlines():
            if line.startswith(f"{names[dom]}:"):
                try:
                    traffic = int(line.split(":", 1)[1].split()[0])
                except ValueError:
                    traffic = None

    chain_kernels = {names[j]: {"us": round(kernel_ms[j] * 1e3, 2), "GB/s": round(gbs(byts[j], kernel_ms[j]), 1),
                                "event_pair_us": round(per_kernel_ms[j] * 1e3, 2)} for j in range(len(names))}
    result = {
        "metric": METRIC,
        "value": round(gbs(chain_bytes * args.steps, ms), 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded numpy: y=leaky(N(0,1)), delta/x/x_norm ~N(0,1), gamma ~U(0.5,1.5))",
        "config": {
            "workload": "configs[1]: BN backward layer step (gradient leaky, backward_bias, backward_scale, "
                        "scale_bias, mean_delta, variance_delta, normalize_delta), fp32 NCHW",
            "batch": 64, "channels": 128, "height": 56, "width": 56,
            "bytes_per_step": chain_bytes, "buffer_sets_rotated": 3,
            "parallelism": "1 GPU",
        },
        "roofline": {
            "kernel": names[dom],
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_GBS, 4),
            "traffic": traffic,
            "duration_us": round(kernel_ms[dom] * 1e3, 2),
            "event_pair_overhead_us": round(overhead_ms * 1e3, 2),
        },
        "chain_kernels": chain_kernels,
        "fused_bwd": {
            "entry": "dkz_batchnorm_backward (same step, same buffers: one sums pass + one apply pass)",
            "us": round(fused_ms * 1e3, 2),
            "bytes": 8 * 4 * h["n"],
            "GB/s": round(gbs(8 * 4 * h["n"], fused_ms), 1),
            "GElem/s": round(h["n"] / (fused_ms * 1e-3) / 1e9, 2),
            "speedup_vs_per_op_chain": round((ms / args.steps) / fused_ms, 3),
        },
    }
    if not args.no_per_op:
        table = per_op_table(gpu, hip, stream, args.op_launches)
        result["per_op"] = table
        result["gemm"] = gemm_table(gpu, hip, stream)
        named = ("mean", "variance", "normalize", "scale_bias", "add_bias", "activate(leaky)")
        cfg1, cfg2 = "cfg1_bn_fwd[", "cfg2_bn_bwd["  # the config rows, not the same ops at other shapes
        fwd = sum(v["us"] for k, v in table.items() if k.startswith(cfg1) and k.split("/", 1)[1] in named)
        fwd_chain = next(v["us"] for k, v in table.items() if k.startswith(cfg1) and "/chain" in k)
        fwd_layer = next(v["us"] for k, v in table.items() if k.startswith(cfg1) and "/layer sequence" in k)
        fwd_fused = next(v["us"] for k, v in table.items() if k.startswith("fused/cfg1"))
        bwd_fused = next(v["us"] for k, v in table.items() if k.startswith("fused/cfg2"))
        bwd = sum(v["us"] for k, v in table.items() if k.startswith(cfg2))
        e1, e2 = 128 * 32 * 1024, 64 * 128 * 3136
        result["bn_act_gelem_s"] = {
            "fwd_cfg1_chained": round(e1 / (fwd_chain * 1e-6) / 1e9, 2),
            "bwd_cfg2_chained": round(e2 / (ms / args.steps * 1e-3) / 1e9, 2),
            "fwd_cfg1_per_op_sum": round(e1 / (fwd * 1e-6) / 1e9, 2),
            "bwd_cfg2_per_op_sum": round(e2 / (bwd * 1e-6) / 1e9, 2),
            "fwd_cfg1_layer_sequence": round(e1 / (fwd_layer * 1e-6) / 1e9, 2),
            "fwd_cfg1_fused": round(e1 / (fwd_fused * 1e-6) / 1e9, 2),
            "bwd_cfg2_fused": round(e2 / (bwd_fused * 1e-6) / 1e9, 2),
        }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(h)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
