"""GPU parity of dkz_gemm (gpu.zig:671-719) against the CPU twin gemm.zig.

The twin sums under @setFloatMode(.optimized), so its order (and the GPU's
matrix-core order) is one of many valid fp32 summation orders. Tolerance,
stated per element: |got - f64| <= gamma_(k+3) * (|alpha| * sum_p |a_ip b_pq|
+ |beta c_iq|), gamma_j = j*u/(1 - j*u), u = 2^-24 -- Higham's a-priori bound
for any fp32 summation order, which the CPU twin is checked to meet too.
Integer-valued inputs (the gemm.zig:265-315 known answer) are exact in any
order and must match bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest

from darknet_zig_amd import gpu
from oracle import ref
from tests.helpers import assert_bitexact, down, rng, up

pytestmark = pytest.mark.gpu

U = 2.0 ** -24
VARIANTS = [(False, False), (True, False), (False, True), (True, True)]


def layout(A, B, ta, tb, pad_a=0, pad_b=0):
    """Row-major storage of A (m x k) and B (k x n) as gemm takes them, with
    leading dimensions widened by pad."""
    m, k = A.shape
    n = B.shape[1]
    sa = A.T if ta else A
    sb = B.T if tb else B
    lda, ldb = sa.shape[1] + pad_a, sb.shape[1] + pad_b
    ga = np.zeros((sa.shape[0], lda), np.float32)
    ga[:, : sa.shape[1]] = sa
    gb = np.zeros((sb.shape[0], ldb), np.float32)
    gb[:, : sb.shape[1]] = sb
    return ga, lda, gb, ldb


def bound(A, B, C0, alpha, beta, k):
    g = (k + 3) * U / (1 - (k + 3) * U)
    return g * (abs(alpha) * (np.abs(A.astype(np.float64)) @ np.abs(B.astype(np.float64)))
                + abs(beta) * np.abs(C0.astype(np.float64)))


def run_gpu(ta, tb, m, n, k, alpha, ga, lda, gb, ldb, beta, gc, ldc):
    da, db, dc = up(ga.ravel()), up(gb.ravel()), up(gc.ravel())
    gpu.gemm(ta, tb, m, n, k, alpha, da, lda, db, ldb, beta, dc, ldc)
    out = down(dc, gc.ravel()).reshape(gc.shape)
    for b in (da, db, dc):
        gpu.free(b)
    return out


def check(ta, tb, m, n, k, alpha, beta, seed, pad=(0, 0, 0), scale=1.0):
    r = rng(seed)
    A = r.uniform(-scale, scale, (m, k)).astype(np.float32)
    B = r.uniform(-scale, scale, (k, n)).astype(np.float32)
    C0 = r.uniform(-1, 1, (m, n)).astype(np.float32)
    ga, lda, gb, ldb = layout(A, B, ta, tb, pad[0], pad[1])
    ldc = n + pad[2]
    gc = np.full((m, ldc), 3.0, np.float32)
    gc[:, :n] = C0
    if beta == 0.0:
        gc[:, :n][::7, ::5] = np.nan  # beta == 0 clears C, NaN included
    got = run_gpu(ta, tb, m, n, k, alpha, ga, lda, gb, ldb, beta, gc, ldc)
    want = alpha * (A.astype(np.float64) @ B.astype(np.float64))
    if beta != 0.0:
        want += beta * C0.astype(np.float64)
    bd = bound(A, B, C0, alpha, beta, k)
    err = np.abs(got[:, :n] - want)
    bad = ~(err <= bd)
    assert not bad.any(), (f"gemm {'T' if ta else 'N'}{'T' if tb else 'N'} {m}x{n}x{k}: {int(bad.sum())} beyond the "
                           f"fp32 bound; max err/bound {float(np.max(err / np.maximum(bd, 1e-300))):.3g}")
    assert np.all(got[:, n:] == 3.0), "columns past n were written"
    return got, ga, lda, gb, ldb, gc, ldc


def test_known_integer_gemm_bitexact(dev):
    """gemm.zig:265-315: a[i] = i%7, b[i] = i%5, alpha 2, beta 1 into zeros,
    all four variants; small integers make every order exact."""
    m, n, k = 5, 4, 3
    A = (np.arange(m * k) % 7).astype(np.float32).reshape(m, k)
    B = (np.arange(k * n) % 5).astype(np.float32).reshape(k, n)
    want = (2 * (A.astype(np.float64) @ B.astype(np.float64))).astype(np.float32)
    for ta, tb in VARIANTS:
        ga, lda, gb, ldb = layout(A, B, ta, tb)
        got = run_gpu(ta, tb, m, n, k, 2.0, ga, lda, gb, ldb, 1.0, np.zeros((m, n), np.float32), n)
        assert_bitexact(got, want, f"gemm {ta},{tb}")


@pytest.mark.parametrize("ta,tb", VARIANTS)
def test_gputest_shape(dev, ta, tb):
    """gputest.zig:347-387: m=37, n=29, k=53, alpha 1.5, beta 1, U(-1,1);
    and against the CPU twin (oracle) at the reference's own 1e-3."""
    got, ga, lda, gb, ldb, gc, ldc = check(ta, tb, 37, 29, 53, 1.5, 1.0, seed=20240921)
    cpu = gc.copy()
    ref.gemm(ta, tb, 37, 29, 53, 1.5, ga.ravel(), lda, gb.ravel(), ldb, 1.0, cpu.reshape(-1), ldc)
    d = np.abs(cpu - got)
    rel = d / np.maximum(np.maximum(np.abs(cpu), np.abs(got)), 1e-4)
    assert d.max() <= 1e-3 or rel.max() <= 1e-3  # gputest.zig:35-52


@pytest.mark.parametrize("ta,tb", VARIANTS)
@pytest.mark.parametrize("m,n,k,alpha,beta", [
    (1, 1, 1, 1.0, 1.0), (3, 70, 5, -2.0, 0.0), (65, 63, 17, 1.0, 0.5), (64, 64, 16, 1.0, 1.0),
    (129, 255, 33, 0.75, -1.0), (130, 7, 300, 1.0, 0.0), (9, 200, 1, 1.0, 2.0), (40, 40, 0, 1.0, 0.5),
])
def test_shapes_edges_and_strides(dev, ta, tb, m, n, k, alpha, beta):
    check(ta, tb, m, n, k, alpha, beta, seed=m * 7 + n + k, pad=(3, 1, 2))


@pytest.mark.parametrize("ta,tb,m,n,k", [
    (False, False, 128, 3136, 1152),  # convolutional forward, one image (config 2's layer)
    (True, False, 1152, 3136, 128),  # backward data: weights^T * delta into the column buffer
    (False, True, 128, 1152, 3136),  # weight gradient: delta * col^T
    (False, False, 2048, 2048, 1024),  # 128x128 tiles
])
def test_layer_shapes(dev, ta, tb, m, n, k):
    check(ta, tb, m, n, k, 1.0, 1.0 if not ta else 0.0, seed=k, scale=0.5)


@pytest.mark.parametrize("ta,tb", VARIANTS)
@pytest.mark.parametrize("m,n,k", [
    (256, 192, 96),  # 64x64 tiles, one K range
    (128, 256, 1024),  # 64x64 tiles, K split over several ranges (partials in the scratch)
    (4096, 2048, 64),  # 128x128 tiles (512 of them)
])
def test_interior_tiles_match_the_checked_loop(dev, ta, tb, m, n, k):
    """Tiles wholly inside aligned operands run a slab loop without edge
    checks; the same product with every leading dimension one wider (no
    operand aligned) runs the checked loop. Both feed the MFMAs the same
    slabs in the same order, so the results agree bit for bit (and meet the
    fp32 bound)."""
    got_fast = check(ta, tb, m, n, k, 1.25, 0.5, seed=m + n + k)[0]
    got_checked = check(ta, tb, m, n, k, 1.25, 0.5, seed=m + n + k, pad=(1, 1, 1))[0]
    assert_bitexact(got_checked[:, :n], got_fast[:, :n], f"gemm {ta},{tb} {m}x{n}x{k}")


def test_cpu_twin_meets_the_same_bound():
    """The oracle (the twin) satisfies the bound the GPU is held to."""
    m, n, k = 33, 17, 500
    r = rng(1)
    A = r.uniform(-1, 1, (m, k)).astype(np.float32)
    B = r.uniform(-1, 1, (k, n)).astype(np.float32)
    C0 = r.uniform(-1, 1, (m, n)).astype(np.float32)
    for ta, tb in VARIANTS:
        ga, lda, gb, ldb = layout(A, B, ta, tb)
        c = C0.copy()
        ref.gemm(ta, tb, m, n, k, 1.25, ga.ravel(), lda, gb.ravel(), ldb, 0.5, c.reshape(-1), n)
        want = 1.25 * (A.astype(np.float64) @ B.astype(np.float64)) + 0.5 * C0
        assert np.all(np.abs(c - want) <= bound(A, B, C0, 1.25, 0.5, k))
