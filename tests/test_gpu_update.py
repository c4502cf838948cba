"""GPU parity of the rest of gpu.zig's elementwise surface: add_scalar,
rand_uniform, dropout (layers/misc.zig:125-141's forward and backward) and
the Adam update (gpu.zig:804-830), all bit-exact against the oracle.

rand_uniform and the Adam step have no CPU twin; the oracle restates their
device kernels (darknet_kernels.hip:168-183, 588-595) and is itself pinned in
tests/test_oracle_ext.py. The fused Adam pass is also checked against the
eight per-op launches gpu.zig issues, on the GPU.
"""

from __future__ import annotations

import numpy as np
import pytest

from darknet_zig_amd import gpu
from oracle import ref
from tests.helpers import assert_bitexact, down, normal, rng, uniform, up

pytestmark = pytest.mark.gpu

SIZES = [1, 3, 4, 5, 4099, 65536 + 7]


def _with_offset(host: np.ndarray, offset: int):
    whole = up(np.concatenate([np.zeros(offset, np.float32), host]))
    return whole, whole.offset(offset)


def _pull_view(whole: gpu.Buf, n: int, offset: int) -> np.ndarray:
    out = np.empty(n + offset, np.float32)
    gpu.pull(whole, out)
    return out[offset:]


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("offset", [0, 1])
def test_add_scalar(dev, n, offset):
    x = uniform(rng(100 + n), n, -3, 3)
    cpu = x.copy()
    ref.addScalar(0.0125, cpu)
    whole, view = _with_offset(x, offset)
    gpu.addScalar(n, 0.0125, view)
    assert_bitexact(_pull_view(whole, n, offset), cpu, f"add_scalar n={n} off={offset}")
    gpu.free(whole)


@pytest.mark.parametrize("n", SIZES + [(1 << 22) + 3])
@pytest.mark.parametrize("offset", [0, 1])
@pytest.mark.parametrize("seed", [0, 1, 0xDEADBEEF, 0xFFFFFFFF])
def test_rand_uniform(dev, n, offset, seed):
    cpu = np.empty(n, np.float32)
    ref.randUniform(cpu, seed)
    whole, view = _with_offset(np.full(n, np.nan, np.float32), offset)
    gpu.randUniform(n, view, seed)
    assert_bitexact(_pull_view(whole, n, offset), cpu, f"rand_uniform n={n} off={offset} seed={seed:#x}")
    gpu.free(whole)


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("prob", [0.0, 0.1, 0.5, 0.95])
def test_dropout_forward_backward(dev, n, prob):
    """misc.zig:128-141: randUniform then dropout on the input; backward:
    dropout on the delta with the same draws."""
    r = rng(200 + n)
    x, delta = normal(r, n), normal(r, n)
    scale = float(np.float32(1.0) / (np.float32(1.0) - np.float32(prob)))  # misc.zig:97
    seed = 0x1234567 + n
    rand_cpu = np.empty(n, np.float32)
    ref.randUniform(rand_cpu, seed)
    x_cpu, d_cpu = x.copy(), delta.copy()
    ref.dropout(x_cpu, rand_cpu, prob, scale)
    ref.dropout(d_cpu, rand_cpu, prob, scale)

    dx, dd, drand = up(x), up(delta), gpu.alloc(n)
    gpu.randUniform(n, drand, seed)
    gpu.dropout(dx, n, drand, prob, scale)
    gpu.dropout(dd, n, drand, prob, scale)
    assert_bitexact(down(drand, rand_cpu), rand_cpu, "rand")
    assert_bitexact(down(dx, x_cpu), x_cpu, f"dropout fwd n={n} p={prob}")
    assert_bitexact(down(dd, d_cpu), d_cpu, f"dropout bwd n={n} p={prob}")
    for b in (dx, dd, drand):
        gpu.free(b)


def test_dropout_large_array(dev):
    """Arrays of 128 MB and more take nontemporal loads and stores: the
    same results. 2^25 + 4099 floats (134 MB), a ragged float4 tail."""
    n = (1 << 25) + 4099
    r = rng(7)
    x = normal(r, n)
    prob = 0.3
    scale = float(np.float32(1.0) / (np.float32(1.0) - np.float32(prob)))
    rand_cpu = np.empty(n, np.float32)
    ref.randUniform(rand_cpu, 0x2468ACE)
    x_cpu = x.copy()
    ref.dropout(x_cpu, rand_cpu, prob, scale)
    dx, drand = up(x), gpu.alloc(n)
    gpu.randUniform(n, drand, 0x2468ACE)
    gpu.dropout(dx, n, drand, prob, scale)
    assert_bitexact(down(dx, x_cpu), x_cpu, f"dropout fwd n={n} p={prob}")
    for b in (dx, drand):
        gpu.free(b)


def test_dropout_misaligned_and_boundary(dev):
    n = 1031
    r = rng(5)
    x = normal(r, n)
    u = uniform(r, n, 0, 1)
    u[::7] = np.float32(0.25)  # draws equal to prob survive
    cpu = x.copy()
    ref.dropout(cpu, u, 0.25, 4.0 / 3.0)
    whole, view = _with_offset(x, 3)
    du_whole, du = _with_offset(u, 1)
    gpu.dropout(view, n, du, 0.25, 4.0 / 3.0)
    assert_bitexact(_pull_view(whole, n, 3), cpu, "dropout misaligned")
    gpu.free(whole)
    gpu.free(du_whole)


ADAM = dict(b1=0.9, b2=0.999, eps=1e-7, decay=0.0005, rate=0.001)


def _adam_sequence_gpu(w, d, m, v, b1, b2, eps, decay, rate, n, batch, t, c1, c2):
    """gpu.zig:819-829's launches through the per-op entry points, with the
    adam_kernel step done on the host from the pulled m and v (it has no
    per-op entry point of its own)."""
    gpu.scal(n, b1, m)
    gpu.scal(n, b2, v)
    gpu.axpy(n, float(np.float32(-decay) * np.float32(batch)), w, d)
    gpu.axpy(n, float(np.float32(1) - np.float32(b1)), d, m)
    gpu.mul(n, d, d)
    gpu.axpy(n, float(np.float32(1) - np.float32(b2)), d, v)


@pytest.mark.parametrize("n", SIZES + [1 << 20])
def test_adam_update_matches_oracle_over_steps(dev, n):
    r = rng(300 + n)
    batch = 32
    w = normal(r, n, 0, 0.1)
    m, v = np.zeros(n, np.float32), np.zeros(n, np.float32)
    dw, dm, dv = up(w), up(m), up(v)
    dd = gpu.alloc(n)
    for t in range(1, 5):
        d = normal(r, n, 0, 0.05)
        gpu.push(dd, d)
        ref.adamUpdate(w, d, m, v, ADAM["b1"], ADAM["b2"], ADAM["eps"], ADAM["decay"], ADAM["rate"], n, batch, t)
        gpu.adamUpdate(dw, dd, dm, dv, ADAM["b1"], ADAM["b2"], ADAM["eps"], ADAM["decay"], ADAM["rate"], n,
                       batch, t)
        assert_bitexact(down(dw, w), w, f"adam w n={n} t={t}")
        assert_bitexact(down(dm, m), m, f"adam m n={n} t={t}")
        assert_bitexact(down(dv, v), v, f"adam v n={n} t={t}")
        assert_bitexact(down(dd, d), d, f"adam d n={n} t={t}")
    for b in (dw, dd, dm, dv):
        gpu.free(b)


def test_adam_update_equals_per_op_launches(dev):
    """The fused pass against gpu.zig's own launch sequence on the device
    (the moment updates through dkz_scal/axpy/mul), t = 3."""
    n, batch, t = 50001, 8, 3
    r = rng(11)
    w, d = normal(r, n, 0, 0.1), normal(r, n, 0, 0.05)
    m, v = normal(r, n, 0, 0.01), np.abs(normal(r, n, 0, 0.001))
    a = ADAM
    # per-op moment updates on the device
    sw, sd, sm, sv = up(w), up(d), up(m), up(v)
    _adam_sequence_gpu(sw, sd, sm, sv, a["b1"], a["b2"], a["eps"], a["decay"], a["rate"], n, batch, t, 0, 0)
    m_seq, v_seq = down(sm, m), down(sv, v)
    # fused
    fw, fd, fm, fv = up(w), up(d), up(m), up(v)
    gpu.adamUpdate(fw, fd, fm, fv, a["b1"], a["b2"], a["eps"], a["decay"], a["rate"], n, batch, t)
    assert_bitexact(down(fm, m), m_seq, "adam m vs per-op")
    assert_bitexact(down(fv, v), v_seq, "adam v vs per-op")
    # and the weight step from the per-op moments equals the oracle's full update
    w_cpu, d_cpu, m_cpu, v_cpu = w.copy(), d.copy(), m.copy(), v.copy()
    ref.adamUpdate(w_cpu, d_cpu, m_cpu, v_cpu, a["b1"], a["b2"], a["eps"], a["decay"], a["rate"], n, batch, t)
    assert_bitexact(m_cpu, m_seq, "oracle m vs per-op")
    assert_bitexact(down(fw, w), w_cpu, "adam w")
    assert np.all(down(fd, d) == 0)
    for b in (sw, sd, sm, sv, fw, fd, fm, fv):
        gpu.free(b)


def test_adam_update_rejects_overlap_and_noops(dev):
    n = 64
    b = gpu.alloc(4 * n)
    w, d, m, v = b.offset(0), b.offset(n), b.offset(2 * n), b.offset(3 * n)
    with pytest.raises(gpu.GpuError):
        gpu.adamUpdate(w, w, m, v, 0.9, 0.999, 1e-7, 0.0, 0.1, n, 1, 1)
    with pytest.raises(gpu.GpuError):
        gpu.adamUpdate(w, b.offset(n - 1), m, v, 0.9, 0.999, 1e-7, 0.0, 0.1, n, 1, 1)
    gpu.adamUpdate(w, d, m, v, 0.9, 0.999, 1e-7, 0.0, 0.1, 0, 1, 1)  # n == 0: no-op
    gpu.randUniform(0, gpu.Buf(), 1)
    gpu.dropout(gpu.Buf(), 0, gpu.Buf(), 0.5, 2.0)
    gpu.addScalar(0, 1.0, gpu.Buf())
    gpu.free(b)
