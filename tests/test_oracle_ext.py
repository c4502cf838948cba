"""Pinning the oracle's restatement of the rest of gpu.zig's op surface:
add_scalar, rand_uniform (with its integer hash), dropout, the Adam update,
im2col/col2im and gemm.

add_scalar, rand_uniform and the last step of the Adam update have no CPU twin
in the reference: their only definition is the device kernel
(darknet_kernels.hip:150-153, 168-183, 588-595). Each is checked here against
something other than its own formula: a published inverse of the hash,
distribution properties, the textbook form of Adam (Kingma & Ba 2015,
Algorithm 1) in f64, numpy's independent arithmetic, the reference's own
im2col.zig and gemm.zig test blocks, the adjoint identity between im2col and
col2im, and Higham's a-priori error bound of an fp32 dot product against
numpy's f64 matrix product.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
from numpy.lib.stride_tricks import sliding_window_view

from oracle import ref

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())["cases"]
f32 = np.float32
M32 = 0xFFFFFFFF


def case(op):
    return next(c for c in GOLDEN if c["op"] == op)


def rng(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------------------
# add_scalar (darknet_kernels.hip:150-153)
# ---------------------------------------------------------------------------


def test_add_scalar_matches_numpy():
    x = rng(1).normal(0, 1, 4099).astype(f32)
    want = x + f32(0.37)
    ref.addScalar(0.37, x)
    np.testing.assert_array_equal(x, want)


# ---------------------------------------------------------------------------
# the hash behind rand_uniform: pinned by the inverse Wellons publishes with
# it ("lowbias32_r", the constants are the inverses mod 2^32 of the forward
# multipliers), written out independently here
# ---------------------------------------------------------------------------


def lowbias32_r(x: np.ndarray) -> np.ndarray:
    x = x.astype(np.uint64)
    x ^= x >> 16
    x = (x * 0x43021123) & M32
    x ^= (x >> 15) ^ (x >> 30)
    x = (x * 0x1D69E2A5) & M32
    x ^= x >> 16
    return x.astype(np.uint32)


def test_hash_inverts_with_the_published_inverse():
    xs = np.concatenate([np.arange(0, 4096, dtype=np.uint32),
                         rng(2).integers(0, 1 << 32, 20000, dtype=np.uint64).astype(np.uint32),
                         np.array([M32, 0x80000000, 0x7FFFFFFF], np.uint32)])
    hs = np.array([ref.hash_u32(int(v)) for v in xs], np.uint32)
    np.testing.assert_array_equal(lowbias32_r(hs), xs)
    assert ref.hash_u32(0) == 0  # every step maps 0 to 0
    assert len(set(hs.tolist())) == len(set(xs.tolist()))  # injective on the sample


def test_rand_uniform_structure():
    """Element i is hash(seed ^ hash(i)) >> 8, scaled by 2^-24 (.hip:177-183):
    undo the scale, then the outer hash with the published inverse, for each
    of the 256 possible low bytes; one of them must give seed ^ hash(i)."""
    seed = 0xC0FFEE11
    n = 64
    x = np.empty(n, f32)
    ref.randUniform(x, seed)
    q = (x.astype(np.float64) * 16777216.0)
    assert np.all(q == np.floor(q)) and np.all(q < 16777216)
    q = q.astype(np.uint64)
    for i in range(n):
        cand = lowbias32_r(((q[i] << 8) | np.arange(256, dtype=np.uint64)).astype(np.uint32))
        assert (seed ^ ref.hash_u32(i)) in set(cand.tolist()), i


def test_rand_uniform_distribution_and_prefix():
    n = 1 << 20
    x = np.empty(n, f32)
    ref.randUniform(x, 7)
    assert x.min() >= 0.0 and x.max() < 1.0
    # mean and variance of U(0,1): 1/2 and 1/12, within 6 standard errors
    assert abs(float(x.mean()) - 0.5) < 6 * np.sqrt(1 / 12 / n)
    assert abs(float(x.var()) - 1 / 12) < 6 * np.sqrt(1 / 180 / n)
    counts = np.bincount((x * 256).astype(np.int64), minlength=256)
    chi2 = float(((counts - n / 256) ** 2 / (n / 256)).sum())
    assert chi2 < 255 + 8 * np.sqrt(2 * 255)
    # counter based: element i depends on (seed, i) only
    y = np.empty(1000, f32)
    ref.randUniform(y, 7)
    np.testing.assert_array_equal(y, x[:1000])
    z = np.empty(1000, f32)
    ref.randUniform(z, 8)
    assert np.mean(z == y) < 0.01


def test_rand_uniform_window():
    """A window starting at element `first` (how the maximum-size GPU tests
    check the top of a 2^31-element buffer) is that slice of the whole
    sequence, including one that crosses 2^24 (where a float index would
    stop being exact)."""
    full = np.empty((1 << 24) + 4096, f32)
    ref.randUniform(full, 11)
    for first, n in ((0, 100), (1, 4096), (9000, 1007), (5003, 1), ((1 << 24) - 2048, 4096)):
        w = np.empty(n, f32)
        ref.randUniform(w, 11, first)
        np.testing.assert_array_equal(w, full[first:first + n])


# ---------------------------------------------------------------------------
# dropout (misc.zig:105-127)
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("prob", [0.0, 0.25, 0.5, 0.9])
def test_dropout_matches_numpy(prob):
    r = rng(3)
    x = r.normal(0, 1, 5000).astype(f32)
    u = r.uniform(0, 1, 5000).astype(f32)
    u[:3] = f32(prob)  # the boundary draw survives (strict <)
    scale = f32(1.0) / (f32(1.0) - f32(prob))
    want = np.where(u < f32(prob), f32(0), x * scale).astype(f32)
    ref.dropout(x, u, prob, float(scale))
    np.testing.assert_array_equal(x, want)


# ---------------------------------------------------------------------------
# Adam (gpu.zig:804-830 + darknet_kernels.hip:588-595) against the textbook
# algorithm in f64. darknet's update buffer holds the negative gradient, with
# weight decay folded in first: g = -(d - decay*batch*w).
# ---------------------------------------------------------------------------


def test_adam_matches_textbook_f64():
    r = rng(4)
    n, batch = 3000, 16
    b1, b2, eps, decay, rate = 0.9, 0.999, 1e-7, 0.0005, 0.001
    w = r.normal(0, 0.1, n).astype(f32)
    m = np.zeros(n, f32)
    v = np.zeros(n, f32)
    W, Mt, Vt = w.astype(np.float64), np.zeros(n), np.zeros(n)
    for t in range(1, 6):
        d = r.normal(0, 0.05, n).astype(f32)
        # textbook step on the same incoming update buffer
        g = -(d.astype(np.float64) - decay * batch * W)
        Mt = b1 * Mt + (1 - b1) * g
        Vt = b2 * Vt + (1 - b2) * g * g
        mhat = Mt / (1 - b1 ** t)
        vhat = Vt / (1 - b2 ** t)
        W = W - rate * mhat / (np.sqrt(vhat) + eps)
        ref.adamUpdate(w, d, m, v, b1, b2, eps, decay, rate, n, batch, t)
        assert np.all(d == 0)
        np.testing.assert_allclose(m, -Mt, rtol=2e-5, atol=1e-8)  # |terms| ~ 5e-3: f32 rounding ~1e-9 each
        np.testing.assert_allclose(v, Vt, rtol=2e-5, atol=1e-12)
        # the step moves w by about `rate`; its f32 rounding is ~1e-7 of w
        np.testing.assert_allclose(w, W, rtol=0, atol=2e-6)


def test_adam_first_step_is_rate_times_sign():
    """At t = 1 from zero moments, mhat = g and vhat = g^2 exactly in the
    reals, so the step is rate * g / (|g| + eps)."""
    n = 1000
    r = rng(5)
    w = r.normal(0, 0.1, n).astype(f32)
    d = r.normal(0, 0.05, n).astype(f32)
    w0, d0 = w.astype(np.float64), d.astype(np.float64)
    m, v = np.zeros(n, f32), np.zeros(n, f32)
    ref.adamUpdate(w, d, m, v, 0.9, 0.999, 1e-8, 0.0, 0.01, n, 1, 1)
    step = w.astype(np.float64) - w0
    np.testing.assert_allclose(step, 0.01 * d0 / (np.abs(d0) + 1e-8), rtol=1e-4, atol=1e-7)


# ---------------------------------------------------------------------------
# im2col / col2im (im2col.zig)
# ---------------------------------------------------------------------------


def test_known_im2col():  # im2col.zig:87-95
    c = case("im2col")
    a = c["args"]
    im = np.array(a["im"], f32)
    col = np.full(a["col_len"], np.nan, f32)
    ref.im2col(im, a["channels"], a["height"], a["width"], a["ksize"], a["stride"], a["pad"], col)
    np.testing.assert_array_equal(col[0:4], c["expect"]["col[0:4]"])
    np.testing.assert_array_equal(col[12:16], c["expect"]["col[12:16]"])


def test_known_col2im():  # im2col.zig:97-104
    c = case("col2im")
    a = c["args"]
    col = np.full(a["col_len"], a["col_fill"], f32)
    im = np.zeros(a["im_len"], f32)
    ref.col2im(col, a["channels"], a["height"], a["width"], a["ksize"], a["stride"], a["pad"], im)
    assert abs(im[4] - c["expect"]["im[4]"]) <= c["expect"]["abs_tol"]
    assert abs(im[0] - c["expect"]["im[0]"]) <= c["expect"]["abs_tol"]


def im2col_numpy(im, C, H, W, k, s, p):
    """Independent lowering: pad, take every k x k window with numpy's
    sliding windows, subsample by the stride, lay out as (c, kh, kw) rows."""
    x = np.pad(im.reshape(C, H, W), ((0, 0), (p, p), (p, p)))
    win = sliding_window_view(x, (k, k), axis=(1, 2))[:, ::s, ::s]  # C, Ho, Wo, k, k
    return np.ascontiguousarray(win.transpose(0, 3, 4, 1, 2)).reshape(-1)


CONV = [(1, 3, 3, 2, 1, 0), (3, 7, 5, 3, 1, 1), (4, 9, 9, 3, 2, 1), (2, 6, 6, 1, 1, 0), (5, 13, 11, 5, 3, 2),
        (16, 14, 14, 3, 1, 1), (3, 8, 8, 2, 2, 0), (2, 5, 5, 3, 1, 2)]


@pytest.mark.parametrize("C,H,W,k,s,p", CONV)
def test_im2col_matches_numpy_windows(C, H, W, k, s, p):
    im = rng(6).normal(0, 1, C * H * W).astype(f32)
    Ho, Wo = ref.conv_out_dim(H, k, s, p), ref.conv_out_dim(W, k, s, p)
    col = np.full(C * k * k * Ho * Wo, np.nan, f32)
    ref.im2col(im, C, H, W, k, s, p, col)
    np.testing.assert_array_equal(col, im2col_numpy(im, C, H, W, k, s, p))


@pytest.mark.parametrize("C,H,W,k,s,p", CONV)
def test_col2im_is_the_adjoint_and_matches_scatter(C, H, W, k, s, p):
    r = rng(7)
    Ho, Wo = ref.conv_out_dim(H, k, s, p), ref.conv_out_dim(W, k, s, p)
    ncol = C * k * k * Ho * Wo
    x = r.normal(0, 1, C * H * W).astype(f32)
    y = r.normal(0, 1, ncol).astype(f32)
    cx = np.empty(ncol, f32)
    ref.im2col(x, C, H, W, k, s, p, cx)
    ty = np.zeros(C * H * W, f32)
    ref.col2im(y, C, H, W, k, s, p, ty)
    lhs = float(np.dot(cx.astype(np.float64), y.astype(np.float64)))
    rhs = float(np.dot(x.astype(np.float64), ty.astype(np.float64)))
    assert abs(lhs - rhs) <= 1e-5 * (abs(lhs) + np.sqrt(ncol))
    # scatter-add of the padded windows, in column order, in f32
    pad = np.zeros((C, H + 2 * p, W + 2 * p), f32)
    yc = y.reshape(C, k, k, Ho, Wo)
    for c in range(C):
        for kh in range(k):
            for kw in range(k):
                for h in range(Ho):
                    for w in range(Wo):
                        pad[c, kh + h * s, kw + w * s] += yc[c, kh, kw, h, w]
    want = pad[:, p:p + H, p:p + W].reshape(-1)
    # the same contributions in the same (column) order on a zero start
    np.testing.assert_array_equal(ty, want)


# ---------------------------------------------------------------------------
# gemm (gemm.zig)
# ---------------------------------------------------------------------------


def test_known_gemm_variants():  # gemm.zig:265-315
    c = case("gemm")
    a_ = c["args"]
    m, n, k = a_["m"], a_["n"], a_["k"]
    a = (np.arange(m * k) % 7).astype(f32)
    b = (np.arange(k * n) % 5).astype(f32)
    at = np.ascontiguousarray(a.reshape(m, k).T).ravel()
    bt = np.ascontiguousarray(b.reshape(k, n).T).ravel()
    want = np.zeros(m * n, f32)
    for i in range(m):
        for q in range(n):
            s = f32(0)
            for p in range(k):
                s = f32(s + a[i * k + p] * b[p * n + q])
            want[i * n + q] = 2 * s
    for ta, tb in a_["variants"]:
        got = np.zeros(m * n, f32)
        ref.gemm(ta, tb, m, n, k, a_["alpha"], at if ta else a, m if ta else k, bt if tb else b, k if tb else n,
                 a_["beta"], got, n)
        assert np.max(np.abs(got - want)) <= c["expect"]["abs_tol"], (ta, tb)
        np.testing.assert_array_equal(got, want)  # small integers: exact in any order


def gemm_bound(a64, b64, c64, alpha, beta, k):
    """Higham's a-priori bound for an fp32 dot product of length k, any
    summation order: gamma_k * sum|alpha a b|, plus the rounding of beta*c and
    of the final add (3 more roundings)."""
    u = 2.0 ** -24
    g = (k + 3) * u / (1 - (k + 3) * u)
    return g * (abs(alpha) * (np.abs(a64) @ np.abs(b64)) + abs(beta) * np.abs(c64))


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
@pytest.mark.parametrize("m,n,k,alpha,beta", [(37, 29, 53, 1.5, 1.0), (8, 16, 300, -0.5, 0.0), (13, 7, 1, 1.0, 0.25),
                                              (4, 9, 0, 2.0, 3.0)])
def test_gemm_within_fp32_bound_of_f64(ta, tb, m, n, k, alpha, beta):
    """gputest.zig:347-387's shapes and flags, against numpy's f64 product;
    lda/ldb/ldc wider than the matrices (sub-matrix views)."""
    r = rng(8)
    A = r.uniform(-1, 1, (m, k)).astype(f32)
    B = r.uniform(-1, 1, (k, n)).astype(f32)
    C0 = r.uniform(-1, 1, (m, n)).astype(f32)
    lda = (m if ta else k) + 3
    ldb = (k if tb else n) + 2
    ldc = n + 5
    ga = np.zeros(((k if ta else m), lda), f32)
    ga[:, : (m if ta else k)] = A.T if ta else A
    gb = np.zeros(((n if tb else k), ldb), f32)
    gb[:, : (k if tb else n)] = B.T if tb else B
    gc = np.full((m, ldc), 7.0, f32)
    gc[:, :n] = C0
    if beta == 0.0:
        gc[0, 0] = np.nan  # beta = 0 clears C, NaN included (gemm.zig:125-126)
    ref.gemm(ta, tb, m, n, k, alpha, ga.ravel(), lda, gb.ravel(), ldb, beta, gc.reshape(-1), ldc)  # views
    A64, B64, C64 = A.astype(np.float64), B.astype(np.float64), C0.astype(np.float64)
    want = alpha * (A64 @ B64) + (beta * C64 if beta != 0 else 0.0)
    bound = gemm_bound(A64, B64, C64, alpha, beta, k)
    assert np.all(np.abs(gc[:, :n] - want) <= bound + 1e-30)
    assert np.all(gc[:, n:] == 7.0)  # columns past n untouched
