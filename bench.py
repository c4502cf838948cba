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
               MI355X's 8 TB/s HBM peak; traffic: that kernel's HBM bytes per
               launch from the committed counter table
               profiles/traffic_per_op.md (see traffic_table())
  chain_kernels  each chain kernel's time; only the first starts cold, the
               later ones re-read operands the previous kernel touched, which
               the 256 MB Infinity Cache may hold ("MALL-assisted")
  per_op       every op of BASELINE.json's five configs timed on its own,
               cold (rotated buffers, >= 512 MB per rotation), in GB/s and as
               a fraction of 8 TB/s: `us` sustained (the launches captured in
               a HIP graph and replayed back to back), `issued_us` (issued one
               by one from Python: host-bound below ~4 us), single-launch (an
               event pair around each launch); rows marked [hot cache] replay
               one buffer set, whose data the Infinity Cache holds; plus
               rand_uniform/dropout, the one-pass Adam update, im2col/col2im,
               shapes off the configs' fast paths (a 3x3/s2 max pool, a
               spatial softmax, a connected layer's bias gradient), and the
               batch-norm layer's other direction at each config's shape
  gemm         dkz_gemm at config 2's convolution shapes and a large square,
               and config 2's convolutional layer forward, weight gradient
               and data gradient over the batch (the per-image loops against
               dkz_convolution_forward / _weight_gradient / _data_gradient),
               TFLOP/s
               against the 157.3 TFLOP/s fp32 matrix-core peak
  fused_bwd    the same step through dkz_batchnorm_backward (at this size one
               launch that holds every element's delta * gradient * scale
               in registers and LDS and x - mean for 11 of each lane's 49
               float4s, and reads x of the other 38 again: about 23 B/elem
               moved instead of the chain's 56; its algorithmic bytes, each
               tensor once, are 20 B/elem)
  bn_act_gelem_s  batch-norm + activation elements per second: config 1's
               forward and config 2's backward (per op, the whole per-op layer
               forward, fused), and each config's layer forward + backward
  cpu_baseline the CPU twins' C restatement (oracle/) on every config's ops
               and inputs, one host thread, median of 5 runs; `value` is
               config 2's (the headline workload), `per_config` all five

Algorithmic bytes count every logical fp32/int32 element read or written once
(4 B); per-channel vectors of C floats are not counted.

--per-op-traffic runs each per-op row's first three launches once between two
marker dispatches (after one untimed pass over all its rotations) and prints
the rows, for rocprofv3 counter runs (READ_COUNTERS, WRITE_COUNTERS) and a
kernel trace that attribute HBM traffic and kernel time to each row;
--copy-calibration runs a known-size copy that checks the counter formula;
--traffic-table DIR prints the table (profiles/traffic_per_op.md) from them;
--sq-table DIR prints the instruction mix per row from two SQ counter runs of
--per-op-traffic (SQ_COUNTERS; profiles/softmax_instruction_mix.md).
--gemm-counters runs the GEMM table's products between markers, and
--gemm-counter-table DIR prints their matrix-core use from two counter runs
of it (MFMA_COUNTERS; profiles/gemm_mfma_counters.md).
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
            "hipStreamCreate": [C.POINTER(C.c_void_p)],
            "hipStreamDestroy": [C.c_void_p],
            "hipStreamSynchronize": [C.c_void_p],
            "hipStreamBeginCapture": [C.c_void_p, C.c_int],
            "hipStreamEndCapture": [C.c_void_p, C.POINTER(C.c_void_p)],
            "hipGraphInstantiate": [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t],
            "hipGraphLaunch": [C.c_void_p, C.c_void_p],
            "hipGraphExecDestroy": [C.c_void_p],
            "hipGraphDestroy": [C.c_void_p],
        }.items():
            fn = getattr(self.lib, name)
            fn.argtypes = args
            fn.restype = C.c_int
        self._stream = None

    def event(self) -> C.c_void_p:
        e = C.c_void_p()
        assert self.lib.hipEventCreate(C.byref(e)) == 0
        return e

    def destroy(self, *events) -> None:
        for e in events:
            self.lib.hipEventDestroy(e)

    def record(self, e, stream) -> None:
        assert self.lib.hipEventRecord(e, stream) == 0

    def ms(self, a, b) -> float:
        assert self.lib.hipEventSynchronize(b) == 0
        out = C.c_float()
        assert self.lib.hipEventElapsedTime(C.byref(out), a, b) == 0
        return float(out.value)

    def sync(self) -> None:
        assert self.lib.hipDeviceSynchronize() == 0

    def capture_stream(self) -> C.c_void_p:
        """A stream (default priority) to capture graphs on, made once."""
        if self._stream is None:
            s = C.c_void_p()
            assert self.lib.hipStreamCreate(C.byref(s)) == 0
            self._stream = s
        return self._stream


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
    """Buffer sets to cycle through so that an op touching `bytes_per_set`
    of them cycles >= 512 MB, twice the Infinity Cache: pass the footprint
    of the block's smallest op, so every row of the block starts cold."""
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
    """The same layer step through the fused entry point (at config 2 one
    launch: every element's y, delta, x_norm and x read once, x of 38 of
    each lane's 49 float4s read again after the channel meeting, delta
    written: about 23 B/elem moved, 20 B/elem algorithmic)."""
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
    hip.destroy(a, b)
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
    hip.destroy(*(e for pair in evs for e in pair))
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
    hip.destroy(a, b)
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
    ms = statistics.mean(hip.ms(a, b) for a, b in evs)
    hip.destroy(*(e for pair in evs for e in pair))
    return ms


def time_graph(hip, seqs, launches, warmup=1, replays=5):
    """Time (ms) of one pass of an op sequence, cycling over rotated sets,
    with `launches` passes captured into one HIP graph: the median over
    `replays` timed replays of the graph's mean per pass. The kernels run
    back to back on the GPU as in a stream of such calls, and the host's
    per-call issue time (ctypes, ~3 us a call) is not in the figure. The
    library is pointed at the capture stream for the capture and back at the
    null stream afterwards."""
    from darknet_zig_amd import _lib

    lib = _lib.load()
    s = hip.capture_stream()
    hip.sync()
    assert lib.dkz_set_stream(s) == 0
    graph, exe = C.c_void_p(), C.c_void_p()
    try:
        assert hip.lib.hipStreamBeginCapture(s, 0) == 0  # hipStreamCaptureModeGlobal
        try:
            for k in range(launches):
                for fn in seqs[k % len(seqs)]:
                    fn()
        finally:
            rc = hip.lib.hipStreamEndCapture(s, C.byref(graph))
        assert rc == 0, rc
    finally:
        lib.dkz_set_stream(None)
    assert hip.lib.hipGraphInstantiate(C.byref(exe), graph, None, None, 0) == 0
    try:
        for _ in range(warmup):
            assert hip.lib.hipGraphLaunch(exe, s) == 0
        assert hip.lib.hipStreamSynchronize(s) == 0
        times = []
        a, b = hip.event(), hip.event()
        try:
            for _ in range(replays):
                hip.record(a, s)
                assert hip.lib.hipGraphLaunch(exe, s) == 0
                hip.record(b, s)
                times.append(hip.ms(a, b))
                assert hip.lib.hipStreamSynchronize(s) == 0
        finally:
            hip.destroy(a, b)
    finally:
        hip.lib.hipGraphExecDestroy(exe)
        hip.lib.hipGraphDestroy(graph)
    return statistics.median(times) / launches


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
# once, untimed, before the begin marker, so the traced passes find their
# pages mapped (as in a stream of such calls); then a cached read of a
# separate 512 MB buffer leaves the 256 MB Infinity Cache holding clean lines
# of unrelated data. Each row thus starts from the same cache state, whatever
# ran before it: its data out of the cache, and no dirty lines of another
# row's writes for its own reads to evict.
MARK_BASE = 1000
TRAFFIC_PASSES = 3
FLUSH_BYTES = 512 << 20


def per_op_table(gpu, hip, stream, launches: int, traffic=None, only=None, graphs=True, hot_traffic=False):
    """The per-op table; with `traffic` (a list), no timing: each row's first
    TRAFFIC_PASSES launches (or call sequences) run once between markers and
    the row is appended to `traffic`. `only`: run only rows whose full name
    (config/op) contains one of these '|'-separated strings. `graphs` False:
    no HIP graph is captured; `us` is then the issued-from-Python time (for
    a kernel-trace profile, which times each kernel itself). `hot_traffic`:
    in traffic mode, rows that have a [hot cache] timing also run hot
    between markers (the first rotation twice untimed, so the Infinity Cache
    holds its data, then its passes), for counters of cold against hot."""
    from darknet_zig_amd.activations import Activation

    rows = {}

    def wanted(cfg, name):
        return only is None or any(o in f"{cfg}/{name}" for o in only.split("|"))
    if traffic is not None:
        mark_buf = gpu.alloc((MARK_BASE + 256) * 256 + 1)
        flush_f = FLUSH_BYTES // 4 // 128
        flush_buf, flush_out = gpu.alloc(flush_f * 128), gpu.alloc(128)
        gpu.fill(flush_buf, flush_f * 128, 1.0)

    def marker(grid):
        gpu.fill(mark_buf.offset(1), grid * 256, 0.0)

    def flush():
        # a per-channel sum over 128 channels: cached loads, 512 B written
        gpu.backwardBias(flush_out, flush_buf, 1, 128, flush_f)

    def traced(cfg, name, nbytes, seqs, hot=False):
        i = len(traffic)
        passes = min(TRAFFIC_PASSES, len(seqs))
        for seq in seqs:
            for fn in seq:
                fn()
        flush()
        hip.sync()
        marker(MARK_BASE + 2 * i)
        for seq in seqs[:passes]:
            for fn in seq:
                fn()
        marker(MARK_BASE + 2 * i + 1)
        hip.sync()
        traffic.append({"row": f"{cfg}/{name}", "bytes": nbytes, "passes": passes, "begin_grid": MARK_BASE + 2 * i})
        print(f"traffic row {i}: {cfg}/{name}", file=sys.stderr, flush=True)
        if hot and hot_traffic:
            i = len(traffic)
            for _ in range(2):
                for fn in seqs[0]:
                    fn()
            hip.sync()
            marker(MARK_BASE + 2 * i)
            for _ in range(TRAFFIC_PASSES):
                for fn in seqs[0]:
                    fn()
            marker(MARK_BASE + 2 * i + 1)
            hip.sync()
            traffic.append({"row": f"{cfg}/{name} [hot cache]", "bytes": nbytes, "passes": TRAFFIC_PASSES,
                            "begin_grid": MARK_BASE + 2 * i})
            print(f"traffic row {i}: {cfg}/{name} [hot cache]", file=sys.stderr, flush=True)

    def row(cfg, name, nbytes, ms, single_ms=None, issued_ms=None):
        g = gbs(nbytes, ms)
        rows[f"{cfg}/{name}"] = r = {"us": round(ms * 1e3, 3), "GB/s": round(g, 1), "frac": round(g / PEAK_GBS, 4),
                                     "bytes": nbytes}
        if issued_ms is not None:
            r["issued_us"] = round(issued_ms * 1e3, 3)
        if single_ms is not None:
            r["single_launch_us"] = round(single_ms * 1e3, 3)
            r["single_launch_frac"] = round(gbs(nbytes, single_ms) / PEAK_GBS, 4)

    def add(cfg, name, nbytes, fns, hot=False):
        """One op over rotated inputs (cold: >= 512 MB between two uses of a
        buffer): sustained (`us`: the launches captured in a HIP graph and
        replayed back to back, the per-launch figure of a stream of such
        calls), `issued_us` (the same calls issued one by one from Python,
        which for launches under ~4 us measures the host's issue rate),
        single-launch (an event pair around each launch, which also times
        ~2 us of dispatch and completion). `hot`: also a row labelled
        [hot cache], the op replayed on one buffer set, whose data the 256 MB
        Infinity Cache then holds."""
        if not wanted(cfg, name):
            return
        if traffic is not None:
            return traced(cfg, name, nbytes, [[f] for f in fns], hot)
        k = max(launches, len(fns))
        seqs = [[f] for f in fns]
        issued = time_seq(hip, stream, seqs, k)
        row(cfg, name, nbytes, time_graph(hip, seqs, k) if graphs else issued, time_op(hip, stream, fns, k), issued)
        if hot:
            hk = max(launches, 64)
            row(cfg, name + " [hot cache]", nbytes,
                time_graph(hip, seqs[:1], hk) if graphs else time_seq(hip, stream, seqs[:1], hk))

    def add_seq(cfg, name, nbytes, seqs, hot=False):
        """A call sequence (or a multi-launch entry point) over rotated sets,
        graph-replayed back to back as a layer would issue it (`issued_us`:
        issued from Python); `hot` as in add()."""
        if not wanted(cfg, name):
            return
        if traffic is not None:
            return traced(cfg, name, nbytes, seqs, hot)
        k = max(launches, len(seqs))
        issued = time_seq(hip, stream, seqs, k)
        row(cfg, name, nbytes, time_graph(hip, seqs, k) if graphs else issued, issued_ms=issued)
        if hot:
            hk = max(launches, 64)
            row(cfg, name + " [hot cache]", nbytes,
                time_graph(hip, seqs[:1], hk) if graphs else time_seq(hip, stream, seqs[:1], hk))

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
    add(cfg, "mean", E, [lambda b=b: gpu.mean(b, B, F, S, m) for b in xs], hot=True)
    add(cfg, "variance", E, [lambda b=b: gpu.variance(b, m, B, F, S, v) for b in xs], hot=True)
    add(cfg, "normalize", 2 * E, [lambda b=b: gpu.normalize(b, m, v, B, F, S) for b in xs], hot=True)
    add(cfg, "scale_bias", 2 * E, [lambda b=b: gpu.scaleBias(b, gam, B, F, S) for b in xs], hot=True)
    add(cfg, "add_bias", 2 * E, [lambda b=b: gpu.addBias(b, bet, B, F, S) for b in xs], hot=True)
    add(cfg, "activate(leaky)", 2 * E, [lambda b=b: gpu.activateArray(b, n, Activation.leaky) for b in xs], hot=True)
    ys = [dev.zeros(n) for _ in range(R)]
    add(cfg, "copy (x, x_norm)", 2 * E, [lambda a=a, b=b: gpu.copy(n, a, b) for a, b in zip(xs, ys)])
    # the named ops in the layer's order on one tensor (batchnorm.zig:137-152 + activate)
    seqs = [[lambda b=b: gpu.mean(b, B, F, S, m), lambda b=b: gpu.variance(b, m, B, F, S, v),
             lambda b=b: gpu.normalize(b, m, v, B, F, S), lambda b=b: gpu.scaleBias(b, gam, B, F, S),
             lambda b=b: gpu.addBias(b, bet, B, F, S), lambda b=b: gpu.activateArray(b, n, Activation.leaky)]
            for b in xs]
    add_seq(cfg, "chain: mean,variance,normalize,scale_bias,add_bias,leaky", 10 * E, seqs, hot=True)
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
    add_seq("fused", "cfg1 batchnorm_forward(train, leaky)", 4 * E,
            [[lambda b=b, c=c, xn=xn: gpu.batchnormForward(B, F, S, Activation.leaky, True, b, b, c, xn, m, v, rm, rv,
                                                           gam, bet)] for b, c, xn in zip(xs, xcs, xns)], hot=True)
    # the backward step at config 1's shape, for the per-layer forward +
    # backward figure (buffers of the forward rows stand in for y, delta, x,
    # x_norm: the timing does not depend on the values)
    bu, su, md1, vd1 = dev.zeros(F), dev.zeros(F), dev.zeros(F), dev.zeros(F)
    add_seq("fused", "cfg1 shape batchnorm_backward(leaky)", 5 * E,
            [[lambda b=b, c=c, xx=xx, xn=xn: gpu.batchnormBackward(B, F, S, Activation.leaky, b, c, xx, xn, m, v, gam,
                                                                   bu, su, md1, vd1)]
             for b, c, xx, xn in zip(xs, xcs, ys, xns)])
    add_seq(cfg, "backward chain: gradient,backward_bias,backward_scale,scale_bias,mean_delta,variance_delta,"
                 "normalize_delta", 14 * E,
            [[lambda b=b, c=c: gpu.gradientArray(b, n, Activation.leaky, c),
              lambda c=c: gpu.backwardBias(bu, c, B, F, S),
              lambda c=c, xn=xn: gpu.backwardScale(xn, c, B, F, S, su),
              lambda c=c: gpu.scaleBias(c, gam, B, F, S),
              lambda c=c: gpu.meanDelta(c, v, B, F, S, md1),
              lambda c=c, xx=xx: gpu.varianceDelta(xx, c, m, v, B, F, S, vd1),
              lambda c=c, xx=xx: gpu.normalizeDelta(xx, m, v, md1, vd1, B, F, S, c)]
             for b, c, xx, xn in zip(xs, xcs, ys, xns)])
    dev.free()

    # -- config 2: BN backward ops on their own
    h = config2_host()
    dev = Device(gpu)
    sets = upload_config2(dev, h, 5)  # 5 x 102.8 MB of delta: backward_bias alone cycles 514 MB
    chains = [config2_chain_ops(gpu, d, h) for d in sets]
    for j, (name, nbytes, _) in enumerate(chains[0]):
        add("cfg2_bn_bwd[64,128,56,56]", name, nbytes, [c[j][2] for c in chains], hot=True)
    add_seq("fused", "cfg2 batchnorm_backward(leaky)", 5 * 4 * h["n"],
            [[lambda d=d: fused_backward(gpu, d, h)] for d in sets])
    # config 1's forward ops on the largest batch-norm tensor of the configs
    # (config 2's x): each op at its largest shape, as the north star asks
    B2, F2, S2, n2 = 64, 128, 56 * 56, h["n"]
    cfg = "cfg1_ops_at_cfg2_shape[64,128,56,56]"
    bias2 = dev.up(gen(7).normal(0, 0.1, F2).astype(np.float32))
    add_seq(cfg, "chain: mean,variance,normalize,scale_bias,add_bias,leaky", 40 * n2,
            [[lambda d=d: gpu.mean(d["x"], B2, F2, S2, d["md"]),
              lambda d=d: gpu.variance(d["x"], d["md"], B2, F2, S2, d["vd"]),
              lambda d=d: gpu.normalize(d["x"], d["mean"], d["var"], B2, F2, S2),
              lambda d=d: gpu.scaleBias(d["x"], d["scales"], B2, F2, S2),
              lambda d=d: gpu.addBias(d["x"], bias2, B2, F2, S2),
              lambda d=d: gpu.activateArray(d["x"], n2, Activation.leaky)] for d in sets])
    add(cfg, "mean", 4 * n2, [lambda d=d: gpu.mean(d["x"], B2, F2, S2, d["md"]) for d in sets])
    add(cfg, "variance", 4 * n2, [lambda d=d: gpu.variance(d["x"], d["mean"], B2, F2, S2, d["vd"]) for d in sets])
    add(cfg, "normalize", 8 * n2, [lambda d=d: gpu.normalize(d["x_norm"], d["mean"], d["var"], B2, F2, S2)
                                   for d in sets])
    add(cfg, "add_bias", 8 * n2, [lambda d=d: gpu.addBias(d["x_norm"], bias2, B2, F2, S2) for d in sets])
    add(cfg, "activate(leaky)", 8 * n2, [lambda d=d: gpu.activateArray(d["x_norm"], n2, Activation.leaky)
                                         for d in sets])
    # the fused forward at config 2's shape, for the per-layer forward +
    # backward figure (it overwrites y, delta and x_norm: these rows come last)
    m2, v2, rm2, rv2 = dev.zeros(F2), dev.zeros(F2), dev.zeros(F2), dev.zeros(F2)
    add_seq("fused", "cfg2 shape batchnorm_forward(train, leaky)", 16 * n2,
            [[lambda d=d: gpu.batchnormForward(B2, F2, S2, Activation.leaky, True, d["x"], d["y"], d["delta"],
                                               d["x_norm"], m2, v2, rm2, rv2, d["scales"], bias2)] for d in sets])
    dev.free()

    # -- config 3: softmax + cross-entropy delta, [256,1000], logits ~N(0,4)
    dev = Device(gpu)
    b3, c3 = 256, 1000
    n3 = b3 * c3
    r = gen(3)
    logits = r.normal(0, 4.0, n3).astype(np.float32)
    truth = np.zeros(n3, np.float32)
    truth[np.arange(b3) * c3 + r.integers(0, c3, b3)] = 1.0
    R = rotations(2 * 4 * n3)  # softmax alone touches x and p: 2 MB a set
    ls = dev.clone(dev.up(logits), n3, R)
    ps = [dev.zeros(n3) for _ in range(R)]
    ts = dev.clone(dev.up(truth), n3, R)
    ds_ = [dev.zeros(n3) for _ in range(R)]
    es = [dev.zeros(n3) for _ in range(R)]
    cfg = "cfg3_softmax[256,1000]"
    add(cfg, "softmax", 2 * 4 * n3, [lambda a=a, p=p: gpu.softmax(a, c3, b3, c3, 1, c3, 1, 1.0, p) for a, p in zip(ls, ps)],
        hot=True)
    add(cfg, "softmax_x_ent", 4 * 4 * n3,
        [lambda p=p, t=t, d=d, e=e: gpu.softmaxCrossEntropy(n3, p, t, d, e) for p, t, d, e in zip(ps, ts, ds_, es)],
        hot=True)
    add_seq(cfg, "chain: softmax, softmax_x_ent (the layer's two calls)", 6 * 4 * n3,
            [[lambda a=a, p=p: gpu.softmax(a, c3, b3, c3, 1, c3, 1, 1.0, p),
              lambda p=p, t=t, d=d, e=e: gpu.softmaxCrossEntropy(n3, p, t, d, e)]
             for a, p, t, d, e in zip(ls, ps, ts, ds_, es)])
    add("fused", "cfg3 softmax_layer_forward (softmax + loss in one pass)", 5 * 4 * n3,
        [lambda a=a, p=p, t=t, d=d, e=e: gpu.softmaxLayerForward(b3, c3, 1, 1.0, a, t, p, d, e)
         for a, p, t, d, e in zip(ls, ps, ts, ds_, es)], hot=True)
    dev.free()
    # the same two ops at a larger batch (config 3 is a 2 MB tensor, which one
    # launch cannot stream at full rate): each op at a large shape
    dev = Device(gpu)
    b3l = 8192
    n3l = b3l * c3
    logits = r.normal(0, 4.0, n3l).astype(np.float32)
    truth = np.zeros(n3l, np.float32)
    truth[np.arange(b3l) * c3 + r.integers(0, c3, b3l)] = 1.0
    R = rotations(2 * 4 * n3l)
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
    # the floor for softmax's traffic at this size: a copy of the same bytes
    add(cfg, "copy of the same bytes (reference)", 2 * 4 * n3l,
        [lambda a=a, p=p: gpu.copy(n3l, a, p) for a, p in zip(ls, ps)])
    dev.free()

    # -- config 4: SGD over 25e6 floats ~N(0,0.05), and the stride-2 shortcut
    dev = Device(gpu)
    n4 = 25_000_000
    r = gen(4)
    R = rotations(4 * n4)  # scal alone touches dw: 100 MB a set
    ws = dev.clone(dev.up(r.normal(0, 0.05, n4).astype(np.float32)), n4, R)
    dws = dev.clone(dev.up(r.normal(0, 0.05, n4).astype(np.float32)), n4, R)
    batch, lr, decay, momentum = 64, 0.1, 0.0005, 0.9
    cfg = "cfg4_sgd[25e6]"
    add(cfg, "axpy(-decay*batch, w, dw)", 3 * 4 * n4,
        [lambda w=w, d=d: gpu.axpy(n4, -decay * batch, w, d) for w, d in zip(ws, dws)], hot=True)
    add(cfg, "axpy(lr/batch, dw, w)", 3 * 4 * n4, [lambda w=w, d=d: gpu.axpy(n4, lr / batch, d, w) for w, d in zip(ws, dws)],
        hot=True)
    add(cfg, "scal(momentum, dw)", 2 * 4 * n4, [lambda d=d: gpu.scal(n4, momentum, d) for d in dws], hot=True)
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
        [lambda a=a, o=o: gpu.shortcut(sb, w1, w1, c1, a, w2, w2, c2, 1.0, 1.0, o) for a, o in zip(adds, outs)], hot=True)
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
    # spatial pyramid pooling's stride-1 windows (5 and 13, offset -(size-1)/2)
    dev = Device(gpu)
    qb, qc, qh = 64, 512, 19
    qn = qb * qc * qh * qh
    R = rotations(4 * 3 * qn)
    qins = [dev.up(r.uniform(-1, 1, qn).astype(np.float32)) for _ in range(R)]
    qouts = [dev.zeros(qn) for _ in range(R)]
    qidx = [dev.zeros(qn) for _ in range(R)]
    cfg = f"pool[{qb},{qc},{qh},{qh}]"
    for qs in (5, 13):
        add(cfg, f"maxpool_fwd {qs}x{qs}/s1", 4 * 3 * qn,
            [lambda i=i, o=o, x=x, qs=qs: gpu.forwardMaxpool(qn, qh, qh, qc, 1, qs, qs - 1, i, o, x)
             for i, o, x in zip(qins, qouts, qidx)])
        add(cfg, f"maxpool_bwd {qs}x{qs}/s1", 4 * 4 * qn,
            [lambda d=d, p=p, x=x, qs=qs: gpu.backwardMaxpool(qn, qh, qh, qc, 1, qs, qs - 1, d, p, x)
             for d, p, x in zip(qouts, qins, qidx)])
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
        for b in (mark_buf, flush_buf, flush_out):
            gpu.free(b)
    return rows


GEMM_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix-core peak


GEMM_SHAPES = [("conv fwd NN 128x3136x1152", False, False, 128, 3136, 1152),
               ("conv bwd-data TN 1152x3136x128", True, False, 1152, 3136, 128),
               ("conv weight-grad NT 128x1152x3136", False, True, 128, 1152, 3136),
               ("square NN 4096x4096x4096", False, False, 4096, 4096, 4096),
               ("square NN 8192x8192x4096", False, False, 8192, 8192, 4096)]


def gemm_table(gpu, hip, stream):
    """dkz_gemm at the shapes a convolutional layer issues for config 2's layer
    (forward, backward data, weight gradient; one image each, as
    convolutional.zig issues them) and at a large square size: TFLOP/s
    against the fp32 matrix-core peak."""
    rows = {}
    r = gen(7)
    for name, ta, tb, m, n, k in GEMM_SHAPES:
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
# CPU baseline: the CPU twins (the oracle's C restatement) on every config
# ---------------------------------------------------------------------------


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def _median_time(fn, repeats):
    """Median wall time (s) of `repeats` calls of fn(), each on fresh state
    made by fn's own setup (fn returns the timed seconds)."""
    return statistics.median(fn() for _ in range(repeats))


def cpu_baselines(h, repeats=5):
    """Each config's ops through the oracle's C restatement of the Zig CPU
    twins (blas.zig, activations.zig, pooling.zig), one host thread, median
    of `repeats` runs, as algorithmic GB/s (the GPU rows' byte counts). The
    ops and inputs are the GPU rows', every config at its stated size.
    About 15 s in all."""
    from darknet_zig_amd.activations import Activation
    from oracle import ref

    out = {}
    t0 = time.perf_counter

    # config 1: mean, variance, normalize, scale_bias, add_bias, leaky on [128,32,32,32]
    B, F, S = 128, 32, 1024
    n = B * F * S
    r = gen(1)
    x0 = r.normal(0, 1, n).astype(np.float32)
    gam, bet = r.uniform(0.5, 1.5, F).astype(np.float32), r.normal(0, 0.1, F).astype(np.float32)

    def cfg1():
        x = x0.copy()
        m, v = np.empty(F, np.float32), np.empty(F, np.float32)
        a = t0()
        ref.mean(x, B, F, S, m)
        ref.variance(x, m, B, F, S, v)
        ref.normalize(x, m, v, B, F, S)
        ref.scaleBias(x, gam, B, F, S)
        ref.addBias(x, bet, B, F, S)
        ref.activateArray(x, Activation.leaky)
        return t0() - a

    out["cfg1"] = (10 * 4 * n, _median_time(cfg1, repeats),
                   "config 1's six named ops (mean, variance, normalize, scale_bias, add_bias, leaky) on "
                   "[128,32,32,32]")

    # config 2: the backward chain on [64,128,56,56] (the headline workload)
    B, F, S = h["B"], h["F"], h["S"]

    def cfg2():
        d = h["delta"].copy()
        bu, su = np.zeros(F, np.float32), np.zeros(F, np.float32)
        md, vd = np.empty(F, np.float32), np.empty(F, np.float32)
        a = t0()
        ref.gradientArray(h["y"], Activation.leaky, d)
        ref.backwardBias(bu, d, B, F, S)
        ref.backwardScale(h["x_norm"], d, B, F, S, su)
        ref.scaleBias(d, h["scales"], B, F, S)
        ref.meanDelta(d, h["var"], B, F, S, md)
        ref.varianceDelta(h["x"], d, h["mean"], h["var"], B, F, S, vd)
        ref.normalizeDelta(h["x"], h["mean"], h["var"], md, vd, B, F, S, d)
        return t0() - a

    out["cfg2"] = (14 * 4 * h["n"], _median_time(cfg2, repeats),
                   "config 2's backward chain (7 ops) on [64,128,56,56], the headline workload's inputs")

    # config 3: softmax then softmax_x_ent on [256,1000], logits ~N(0,4)
    b3, c3 = 256, 1000
    n3 = b3 * c3
    r = gen(3)
    logits = r.normal(0, 4.0, n3).astype(np.float32)
    truth = np.zeros(n3, np.float32)
    truth[np.arange(b3) * c3 + r.integers(0, c3, b3)] = 1.0

    def cfg3():
        p, d, e = np.empty(n3, np.float32), np.empty(n3, np.float32), np.empty(n3, np.float32)
        a = t0()
        ref.softmax(logits, c3, b3, c3, 1, c3, 1, 1.0, p)
        ref.softmaxCrossEntropy(p, truth, d, e)
        return t0() - a

    out["cfg3"] = (6 * 4 * n3, _median_time(cfg3, repeats),
                   "config 3's softmax + softmax_x_ent on [256,1000]")

    # config 4: one SGD step over 25e6 floats, then the stride-2 shortcut
    n4 = 25_000_000
    r = gen(4)
    w0, dw0 = r.normal(0, 0.05, n4).astype(np.float32), r.normal(0, 0.05, n4).astype(np.float32)
    sb, w1, c1, w2, c2 = 64, 28, 256, 14, 512
    add0 = r.normal(0, 0.05, sb * c1 * w1 * w1).astype(np.float32)
    out0 = r.normal(0, 0.05, sb * c2 * w2 * w2).astype(np.float32)

    def cfg4():
        w, dw, o = w0.copy(), dw0.copy(), out0.copy()
        a = t0()
        ref.axpy(-0.0005 * 64, w, dw)
        ref.axpy(0.1 / 64, dw, w)
        ref.scal(0.9, dw)
        ref.shortcut(sb, w1, w1, c1, add0, w2, w2, c2, 1.0, 1.0, o)
        return t0() - a

    out["cfg4"] = (8 * 4 * n4 + 3 * 4 * sb * c1 * w2 * w2, _median_time(cfg4, repeats),
                   "config 4's SGD step (axpy, axpy, scal over 25e6 floats) and shortcut "
                   "[64,256,28,28] -> [64,512,14,14]")

    # config 5: max pool 2x2/s2 fwd + bwd, global avg pool fwd + bwd on [256,512,28,28]
    pb, pc, ph = 256, 512, 28
    nin = pb * pc * ph * ph
    oh = (ph + 1 - 2) // 2 + 1
    nout = pb * pc * oh * oh
    r = gen(5)
    xin = r.uniform(-1, 1, nin).astype(np.float32)
    dout = r.uniform(-1, 1, nout).astype(np.float32)

    def cfg5():
        o, idx = np.empty(nout, np.float32), np.empty(nout, np.int32)
        prev = np.zeros(nin, np.float32)
        avg = np.empty(pb * pc, np.float32)
        a = t0()
        ref.forwardMaxpool(pb, ph, ph, pc, 2, 2, 1, xin, o, idx)
        ref.backwardMaxpool(idx, dout, prev)
        ref.forwardAvgpool(pb, ph, ph, pc, xin, avg)
        ref.backwardAvgpool(pb, ph, ph, pc, avg, prev)
        return t0() - a

    out["cfg5"] = (4 * (nin + 2 * nout) + 4 * (2 * nout + 2 * nin) + 4 * (nin + pb * pc) + 4 * (2 * nin + pb * pc),
                   _median_time(cfg5, repeats),
                   "config 5's max pool 2x2/s2 forward + backward and global avg pool forward + backward, "
                   "[256,512,28,28]")

    cores = os.cpu_count()
    model = _cpu_model()
    per = {}
    for k, (nbytes, t, what) in out.items():
        per[k] = {"value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "ms": round(t * 1e3, 3),
                  "sample": f"{what}; median of {repeats} runs"}
    head = per["cfg2"]
    return {
        "value": head["value"],
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"{head['sample']}, {head['ms']} ms per chain; 1 thread of {cores} ({model}); the oracle's C "
                   "restatement of the Zig CPU twins built -O2 -march=x86-64-v3 -ffp-contract=off"),
        "per_config": per,
    }


# ---------------------------------------------------------------------------


def bn_gelem(table, bwd_chain_ms):
    """Batch-norm + activation throughput in GElem/s (elements of the layer's
    tensor per second): config 1's forward and config 2's backward, per op
    (chained, and the sum of the ops timed alone), the whole per-op layer
    forward (copies and EMA included) and the fused entry points; and the
    layer's forward + backward at each config's shape (E / (t_fwd + t_bwd)),
    per-op chains and fused."""
    def us(key):
        rows = [v["us"] for k, v in table.items() if k == key]
        return rows[0] if rows else None

    named = ("mean", "variance", "normalize", "scale_bias", "add_bias", "activate(leaky)")
    c1, c2, c12 = "cfg1_bn_fwd[128,32,32,32]", "cfg2_bn_bwd[64,128,56,56]", "cfg1_ops_at_cfg2_shape[64,128,56,56]"
    e1, e2 = 128 * 32 * 1024, 64 * 128 * 3136
    fwd_sum = sum(table[f"{c1}/{k}"]["us"] for k in named)
    bwd_sum = sum(v["us"] for k, v in table.items() if k.startswith(c2 + "/") and "[hot cache]" not in k)
    fwd1 = us(f"{c1}/chain: mean,variance,normalize,scale_bias,add_bias,leaky")
    bwd1 = us(f"{c1}/backward chain: gradient,backward_bias,backward_scale,scale_bias,mean_delta,variance_delta,"
              "normalize_delta")
    fwd2 = us(f"{c12}/chain: mean,variance,normalize,scale_bias,add_bias,leaky")
    bwd2 = bwd_chain_ms * 1e3
    ffwd1 = us("fused/cfg1 batchnorm_forward(train, leaky)")
    fbwd1 = us("fused/cfg1 shape batchnorm_backward(leaky)")
    ffwd2 = us("fused/cfg2 shape batchnorm_forward(train, leaky)")
    fbwd2 = us("fused/cfg2 batchnorm_backward(leaky)")
    layer1 = us(f"{c1}/layer sequence: copy,mean,variance,ema,normalize,copy,scale_bias,add_bias,leaky")

    def g(e, *t):
        return None if any(v is None for v in t) else round(e / (sum(t) * 1e-6) / 1e9, 2)

    return {
        "fwd_cfg1_chained": g(e1, fwd1),
        "bwd_cfg2_chained": g(e2, bwd2),
        "fwd_cfg1_per_op_sum": g(e1, fwd_sum),
        "bwd_cfg2_per_op_sum": g(e2, bwd_sum),
        "fwd_cfg1_layer_sequence": g(e1, layer1),
        "fwd_cfg1_fused": g(e1, ffwd1),
        "bwd_cfg2_fused": g(e2, fbwd2),
        "fwd_bwd_cfg1_shape_per_op": g(e1, fwd1, bwd1),
        "fwd_bwd_cfg1_shape_fused": g(e1, ffwd1, fbwd1),
        "fwd_bwd_cfg2_shape_per_op": g(e2, fwd2, bwd2),
        "fwd_bwd_cfg2_shape_fused": g(e2, ffwd2, fbwd2),
    }


# ---------------------------------------------------------------------------
# per-op traffic table from rocprofv3 runs of --per-op-traffic
# ---------------------------------------------------------------------------

# gfx950's L2 (TCC) counts its reads from HBM by request size -- 32, 64 and
# 128 bytes -- and its writes as 32- or 64-byte requests. FETCH_SIZE's
# gfx950 formula in rocprofiler-sdk's counter_defs.yaml weighs 128-byte
# requests through TCC_BUBBLE, which gfx950 does not define, so it undercounts
# them; these counters give the bytes directly.
READ_COUNTERS = ("TCC_EA0_RDREQ_32B_sum", "TCC_EA0_RDREQ_64B_sum", "TCC_EA0_RDREQ_128B_sum", "TCC_EA0_RDREQ_sum")
WRITE_COUNTERS = ("TCC_EA0_WRREQ_sum", "TCC_EA0_WRREQ_64B_sum")


def _csv(directory: Path, suffix: str):
    import csv
    import glob

    files = sorted(glob.glob(str(directory / f"*{suffix}")))
    if not files:
        raise FileNotFoundError(f"no *{suffix} under {directory}")
    with open(files[0]) as f:
        return list(csv.DictReader(f))


def _dispatch_counters(directory: Path):
    """[(kernel name, workgroups, {counter: value})] in dispatch order."""
    d = {}
    for r in _csv(directory, "counter_collection.csv"):
        k = int(r["Dispatch_Id"])
        e = d.setdefault(k, [r["Kernel_Name"], int(r["Grid_Size"]) // 256, {}])
        e[2][r["Counter_Name"]] = e[2].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    return [d[k] for k in sorted(d)]


def _is_marker(name: str, blocks: int, base: int) -> bool:
    return "FillOp" in name and "ew_scalar_kernel" in name and blocks >= base


def _segments(dispatches, base):
    """Row index -> the dispatches between its begin and end markers."""
    out, cur = {}, None
    for name, blocks, val in dispatches:
        if _is_marker(name, blocks, base):
            idx = blocks - base
            cur = idx // 2 if idx % 2 == 0 else None
            if cur is not None:
                out[cur] = []
            continue
        if cur is not None:
            out[cur].append((name, val))
    return out


def _read_bytes(c):
    return 32 * c["TCC_EA0_RDREQ_32B_sum"] + 64 * c["TCC_EA0_RDREQ_64B_sum"] + 128 * c["TCC_EA0_RDREQ_128B_sum"]


def _write_bytes(c):
    return 32 * (c["TCC_EA0_WRREQ_sum"] - c["TCC_EA0_WRREQ_64B_sum"]) + 64 * c["TCC_EA0_WRREQ_64B_sum"]


def traffic_table(d: Path) -> str:
    """The per-op traffic table (markdown) from the outputs under `d`:
    traffic_rows.json (stdout of `bench.py --per-op-traffic`), read/ and
    write/ (rocprofv3 --pmc READ_COUNTERS / WRITE_COUNTERS of that command),
    trace/ (rocprofv3 --kernel-trace of it), and copy.json, copy_read/,
    copy_write/ (the same for `bench.py --copy-calibration 1024`, whose known
    bytes check the counter formula)."""
    def last_json(path):
        return json.loads([ln for ln in open(path) if ln.startswith("{")][-1])

    meta = last_json(d / "traffic_rows.json")
    rows, base = meta["per_op_traffic"], meta["mark_base"]
    rd = _segments([(n, b, c) for n, b, c in _dispatch_counters(d / "read")], base)
    wr = _segments([(n, b, c) for n, b, c in _dispatch_counters(d / "write")], base)
    trace = []
    for r in sorted(_csv(d / "trace", "kernel_trace.csv"), key=lambda r: int(r["Dispatch_Id"])):
        trace.append((r["Kernel_Name"], int(r["Grid_Size_X"]) // 256,
                      (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3))
    tr = _segments(trace, base)
    check = ""
    if (d / "copy.json").exists():
        cal = last_json(d / "copy.json")["copy_calibration"]
        cr = [c for n, b, c in _dispatch_counters(d / "copy_read") if "CopyOp" in n][-4:]
        cw = [c for n, b, c in _dispatch_counters(d / "copy_write") if "CopyOp" in n][-4:]
        fr = statistics.mean(_read_bytes(c) for c in cr) / cal["bytes_read"]
        fw = statistics.mean(_write_bytes(c) for c in cw) / cal["bytes_written"]
        check = (f"Check of the formula: a copy of {cal['bytes_read'] / 2**30:.0f} GiB reads {fr:.4f}x and writes "
                 f"{fw:.4f}x its known bytes by these counters (no scale factor is applied).")
    lines = [
        "| row | algorithmic MB | counter MB (read + write) | ratio | 128-B share of reads | kernels | rocprof us "
        "| algorithmic GB/s | of 8 TB/s | counter GB/s | of 8 TB/s |",
        "|---|---|---|---|---|---|---|---|---|---|---|",
    ]
    for i, r in enumerate(rows):
        p = r["passes"]
        reads = sum(_read_bytes(c) for _, c in rd.get(i, [])) / p
        writes = sum(_write_bytes(c) for _, c in wr.get(i, [])) / p
        n128 = sum(c["TCC_EA0_RDREQ_128B_sum"] for _, c in rd.get(i, []))
        nall = sum(c["TCC_EA0_RDREQ_32B_sum"] + c["TCC_EA0_RDREQ_64B_sum"] + c["TCC_EA0_RDREQ_128B_sum"]
                   for _, c in rd.get(i, []))
        durs = [t for _, t in tr.get(i, [])]
        per = max(1, len(durs) // p)
        us = sorted(sum(durs[k * per:(k + 1) * per]) for k in range(p))[p // 2] if durs else float("nan")
        t = reads + writes
        b = r["bytes"]
        ratio = f"{t / b:.3f}" if b > 1e5 else "(C floats)"
        share = f"{128 * n128 / max(reads * p, 1):.2f}" if nall else "-"
        lines.append(f"| {r['row']} | {b / 1e6:.2f} | {t / 1e6:.2f} | {ratio} | {share} | {per} | {us:.2f} | "
                     f"{b / us / 1e3:.0f} | {b / us / 8e6:.3f} | {t / us / 1e3:.0f} | {t / us / 8e6:.3f} |")
    return "\n".join(([check, ""] if check else []) + lines)


def counter_traffic(row: str):
    """HBM bytes per launch of a per-op row, from the committed counter table
    (profiles/traffic_per_op.md, 'counter MB' column), or None."""
    path = ROOT / "profiles" / "traffic_per_op.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) > 3 and cells[0] == row:
            try:
                return int(round(float(cells[2]) * 1e6))
            except ValueError:
                return None
    return None


SQ_COUNTERS = ("SQ_WAVES SQ_INSTS_VALU SQ_INSTS_SALU SQ_INSTS_VMEM_RD SQ_INSTS_VMEM_WR SQ_INSTS_LDS "
               "SQ_WAIT_INST_ANY SQ_WAVE_CYCLES GRBM_GUI_ACTIVE",
               "SQ_INSTS_VALU_TRANS_F32 SQ_INSTS_VALU_FMA_F32 SQ_INSTS_VALU_ADD_F32 SQ_INSTS_VALU_MUL_F32 "
               "SQ_INSTS_VALU_FMA_F64 SQ_ACTIVE_INST_VALU SQ_BUSY_CYCLES SQ_WAIT_ANY")


def sq_table(d: Path) -> str:
    """Instruction mix per row (markdown) from the outputs under `d`:
    rows.json (stdout of `bench.py --per-op-traffic --rows ...`) and sq_a/,
    sq_b/ (rocprofv3 --pmc with the two SQ_COUNTERS groups over that
    command). Per pass: waves, instructions per wave, VALU lane-operations
    per element moved (instructions x 64 / (algorithmic bytes / 4)), and the
    shares of a wave's cycles spent issuing VALU work and waiting."""
    def last_json(path):
        return json.loads([ln for ln in open(path) if ln.startswith("{")][-1])

    meta = last_json(d / "rows.json")
    rows, base = meta["per_op_traffic"], meta["mark_base"]
    segs = [_segments([(n, b, c) for n, b, c in _dispatch_counters(d / sub)], base) for sub in ("sq_a", "sq_b")]
    lines = [
        "| row | waves | VALU / wave | SALU / wave | VMEM rd / wave | VMEM wr / wave | LDS / wave "
        "| VALU lane-ops / elem | of which exp2 (trans) | f32 fma+add+mul | f64 fma | VALU-issue share "
        "| wait share | GRBM_GUI_ACTIVE cycles |",
        "|---|---|---|---|---|---|---|---|---|---|---|---|---|---|",
    ]
    for i, r in enumerate(rows):
        p = r["passes"]
        c = {}
        for seg in segs:
            for _, vals in seg.get(i, []):
                for k, v in vals.items():
                    c[k] = c.get(k, 0.0) + v / p
        if not c.get("SQ_WAVES"):
            continue
        w, elems = c["SQ_WAVES"], r["bytes"] / 4

        def per_elem(k):
            return 64 * c.get(k, 0.0) / elems
        f32 = per_elem("SQ_INSTS_VALU_FMA_F32") + per_elem("SQ_INSTS_VALU_ADD_F32") + per_elem("SQ_INSTS_VALU_MUL_F32")
        lines.append(
            f"| {r['row']} | {w:.0f} | {c['SQ_INSTS_VALU'] / w:.1f} | {c['SQ_INSTS_SALU'] / w:.1f} | "
            f"{c['SQ_INSTS_VMEM_RD'] / w:.1f} | {c['SQ_INSTS_VMEM_WR'] / w:.1f} | {c['SQ_INSTS_LDS'] / w:.1f} | "
            f"{per_elem('SQ_INSTS_VALU'):.2f} | {per_elem('SQ_INSTS_VALU_TRANS_F32'):.2f} | {f32:.2f} | "
            f"{per_elem('SQ_INSTS_VALU_FMA_F64'):.2f} | "
            f"{c['SQ_ACTIVE_INST_VALU'] / c['SQ_WAVE_CYCLES']:.3f} | {c['SQ_WAIT_INST_ANY'] / c['SQ_WAVE_CYCLES']:.3f} | "
            f"{c['GRBM_GUI_ACTIVE']:.0f} |")
    return "\n".join(lines)


LATENCY_COUNTERS = "TCC_EA0_RDREQ_LEVEL_sum TCC_EA0_RDREQ_sum TCC_EA0_WRREQ_LEVEL_sum TCC_EA0_WRREQ_sum GRBM_GUI_ACTIVE"


def latency_table(d: Path) -> str:
    """Memory latency per row (markdown) from the outputs under `d`:
    rows.json (stdout of `bench.py --per-op-traffic --hot --rows ...`) and
    lat/ (rocprofv3 --pmc LATENCY_COUNTERS over that command). Per pass: the
    average number of L2 read and write requests in flight to the fabric
    (EA) and their average latency (in-flight sum / requests, in L2 clock
    cycles), for a row run cold (its data in HBM) and hot (in the Infinity
    Cache)."""
    def last_json(path):
        return json.loads([ln for ln in open(path) if ln.startswith("{")][-1])

    meta = last_json(d / "rows.json")
    rows, base = meta["per_op_traffic"], meta["mark_base"]
    seg = _segments([(n, b, c) for n, b, c in _dispatch_counters(d / "lat")], base)
    lines = [
        "| row | EA read requests | avg read latency (cycles) | EA write requests | avg write latency (cycles) "
        "| GRBM_GUI_ACTIVE cycles |",
        "|---|---|---|---|---|---|",
    ]
    for i, r in enumerate(rows):
        p = r["passes"]
        c = {}
        for _, vals in seg.get(i, []):
            for k, v in vals.items():
                c[k] = c.get(k, 0.0) + v / p
        if not c:
            continue
        rq, wq = c.get("TCC_EA0_RDREQ_sum", 0.0), c.get("TCC_EA0_WRREQ_sum", 0.0)
        rl = c.get("TCC_EA0_RDREQ_LEVEL_sum", 0.0) / rq if rq else float("nan")
        wl = c.get("TCC_EA0_WRREQ_LEVEL_sum", 0.0) / wq if wq else float("nan")
        lines.append(f"| {r['row']} | {rq:.0f} | {rl:.0f} | {wq:.0f} | {wl:.0f} | {c.get('GRBM_GUI_ACTIVE', 0):.0f} |")
    return "\n".join(lines)


MFMA_COUNTERS = ("SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU_MFMA_F32 SQ_WAVE_CYCLES SQ_WAIT_INST_ANY SQ_WAIT_INST_LDS "
                 "GRBM_GUI_ACTIVE",
                 "SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_INSTS_LDS")
GEMM_COUNTER_PASSES = 2


def gemm_counters(gpu, hip):
    """Counter mode of the GEMM table: each shape of GEMM_SHAPES runs once
    untimed, then GEMM_COUNTER_PASSES times between two marker fills (as in
    the traffic mode), so that rocprofv3 --pmc can attribute every dispatch
    -- the product and, for split K, its reduction -- to its shape."""
    mark_buf = gpu.alloc((MARK_BASE + 256) * 256 + 1)

    def marker(grid):
        gpu.fill(mark_buf.offset(1), grid * 256, 0.0)
    out = []
    r = gen(7)
    for i, (name, ta, tb, m, n, k) in enumerate(GEMM_SHAPES):
        dev = Device(gpu)
        a = dev.up(r.uniform(-1, 1, m * k).astype(np.float32))
        b = dev.up(r.uniform(-1, 1, k * n).astype(np.float32))
        c = dev.zeros(m * n)
        lda, ldb = (m if ta else k), (k if tb else n)
        gpu.gemm(ta, tb, m, n, k, 1.0, a, lda, b, ldb, 1.0, c, n)
        hip.sync()
        marker(MARK_BASE + 2 * i)
        for _ in range(GEMM_COUNTER_PASSES):
            gpu.gemm(ta, tb, m, n, k, 1.0, a, lda, b, ldb, 1.0, c, n)
        marker(MARK_BASE + 2 * i + 1)
        hip.sync()
        dev.free()
        out.append({"row": name, "flops": 2 * m * n * k, "passes": GEMM_COUNTER_PASSES,
                    "begin_grid": MARK_BASE + 2 * i})
        print(f"gemm counter row {i}: {name}", file=sys.stderr, flush=True)
    gpu.free(mark_buf)
    return {"gemm_counters": out, "mark_base": MARK_BASE}


def gemm_counter_table(d: Path) -> str:
    """Matrix-core use per GEMM shape (markdown) from the outputs under `d`:
    rows.json (stdout of `bench.py --gemm-counters`) and mfma_a/, mfma_b/
    (rocprofv3 --pmc with the two MFMA_COUNTERS groups over that command).
    Per product: fp32 MFMA instructions, the MFMA pipe's busy cycles per
    instruction, the busy share of all SIMD cycles (GRBM_GUI_ACTIVE is summed
    over the 8 XCDs, each of 32 CUs x 4 SIMDs), the share of the waves'
    cycles spent waiting (all causes, and on LDS), and LDS bank conflicts as
    a share of LDS-active cycles."""
    def last_json(path):
        return json.loads([ln for ln in open(path) if ln.startswith("{")][-1])

    meta = last_json(d / "rows.json")
    rows, base = meta["gemm_counters"], meta["mark_base"]
    segs = [_segments([(n, b, c) for n, b, c in _dispatch_counters(d / sub)], base) for sub in ("mfma_a", "mfma_b")]
    lines = [
        "| product | MFMA instructions | MFMA-busy cycles / MFMA | MFMA-busy share of SIMD cycles | wait share "
        "| LDS-wait share | LDS bank-conflict share | GPU-active cycles (per XCD) |",
        "|---|---|---|---|---|---|---|---|",
    ]
    for i, r in enumerate(rows):
        p = r["passes"]
        c = {}
        for seg in segs:
            for _, vals in seg.get(i, []):
                for k, v in vals.items():
                    c[k] = c.get(k, 0.0) + v / p
        if not c.get("SQ_INSTS_VALU_MFMA_F32"):
            continue
        mf, busy = c["SQ_INSTS_VALU_MFMA_F32"], c["SQ_VALU_MFMA_BUSY_CYCLES"]
        gui = c["GRBM_GUI_ACTIVE"] / 8
        lines.append(
            f"| {r['row']} | {mf:.0f} | {busy / mf:.1f} | {busy / (gui * 32 * 4 * 8):.3f} | "
            f"{c['SQ_WAIT_INST_ANY'] / c['SQ_WAVE_CYCLES']:.3f} | {c['SQ_WAIT_INST_LDS'] / c['SQ_WAVE_CYCLES']:.3f} | "
            f"{c['SQ_LDS_BANK_CONFLICT'] / max(c['SQ_LDS_IDX_ACTIVE'], 1.0):.3f} | {gui:.0f} |")
    return "\n".join(lines)


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
    ap.add_argument("--hot", action="store_true",
                    help="with --per-op-traffic: also run each row that has a [hot cache] timing hot, between "
                         "markers of its own")
    ap.add_argument("--no-graph", action="store_true",
                    help="with --per-op-only: capture no HIP graph (per-op `us` is then the issued time); for "
                         "rocprofv3 --kernel-trace, under which the graph-replay timing ended in a host "
                         "segmentation fault")
    ap.add_argument("--per-op-traffic", action="store_true",
                    help="only run each per-op row's first launches once, between marker dispatches "
                         "(for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE per row)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run dkz_copy over MIB MiB (x4 launches, rotated): a known-size kernel that "
                         "checks the counter formula of the traffic table")
    ap.add_argument("--rows", default=None, metavar="SUBSTR",
                    help="with --per-op-only or --per-op-traffic: only the per-op rows whose name "
                         "(config/op) contains SUBSTR ('|'-separated alternatives)")
    ap.add_argument("--latency-table", default=None, metavar="DIR",
                    help="print the memory-latency table (cold against hot rows) from DIR/rows.json and DIR/lat")
    ap.add_argument("--sq-table", default=None, metavar="DIR",
                    help="only print the instruction-mix table (markdown) from the rocprofv3 SQ counter outputs "
                         "in DIR (see sq_table())")
    ap.add_argument("--traffic-table", default=None, metavar="DIR",
                    help="only print the per-op traffic table (markdown) from the rocprofv3 outputs in DIR "
                         "(see traffic_table())")
    ap.add_argument("--gemm-counters", action="store_true",
                    help="only run the GEMM table's products a few times each, between marker dispatches "
                         "(for rocprofv3 --pmc with MFMA_COUNTERS)")
    ap.add_argument("--gemm-counter-table", default=None, metavar="DIR",
                    help="only print the matrix-core table (markdown) from the rocprofv3 outputs in DIR "
                         "(see gemm_counter_table())")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(every op runs on one device's share); run with --gpus 1.", file=sys.stderr)
        return 2

    if args.traffic_table:
        print(traffic_table(Path(args.traffic_table)))
        return 0
    if args.sq_table:
        print(sq_table(Path(args.sq_table)))
        return 0
    if args.latency_table:
        print(latency_table(Path(args.latency_table)))
        return 0
    if args.gemm_counter_table:
        print(gemm_counter_table(Path(args.gemm_counter_table)))
        return 0

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

    if args.gemm_counters:
        print(json.dumps(gemm_counters(gpu, hip)), flush=True)
        return 0

    if args.per_op_traffic:
        traffic = []
        per_op_table(gpu, hip, stream, 1, traffic, only=args.rows, hot_traffic=args.hot)
        print(json.dumps({"per_op_traffic": traffic, "mark_base": MARK_BASE}), flush=True)
        return 0

    if args.per_op_only:
        res = {"per_op": per_op_table(gpu, hip, stream, args.op_launches, only=args.rows,
                                      graphs=not args.no_graph)}
        if args.rows is None:
            res["gemm"] = gemm_table(gpu, hip, stream)
        print(json.dumps(res), flush=True)
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
    traffic = counter_traffic(f"cfg2_bn_bwd[64,128,56,56]/{names[dom]}")

    # Only the step's first kernel starts from data the previous step left
    # >= 512 MB behind; every later kernel re-reads delta (and x) that the
    # kernel before it read or wrote, which the 256 MB Infinity Cache may
    # still hold, so their rates are not pure HBM rates.
    chain_kernels = {names[j]: {"us": round(kernel_ms[j] * 1e3, 2), "GB/s": round(gbs(byts[j], kernel_ms[j]), 1),
                                "event_pair_us": round(per_kernel_ms[j] * 1e3, 2),
                                "cache": "cold (HBM)" if j == 0 else "MALL-assisted (re-reads the previous "
                                                                      "kernel's operands)"}
                     for j in range(len(names))}
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
            "entry": "dkz_batchnorm_backward (same step, same buffers; here one launch holding each element's "
                     "delta term in registers and LDS and reading x of most again, about 23 B/elem moved; bytes "
                     "below are algorithmic, 20 B/elem)",
            "us": round(fused_ms * 1e3, 2),
            "bytes": 5 * 4 * h["n"],
            "GB/s": round(gbs(5 * 4 * h["n"], fused_ms), 1),
            "GElem/s": round(h["n"] / (fused_ms * 1e-3) / 1e9, 2),
            "speedup_vs_per_op_chain": round((ms / args.steps) / fused_ms, 3),
        },
    }
    if not args.no_per_op:
        table = per_op_table(gpu, hip, stream, args.op_launches)
        result["per_op"] = table
        result["gemm"] = gemm_table(gpu, hip, stream)
        result["bn_act_gelem_s"] = bn_gelem(table, ms / args.steps)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baselines(h)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
