"""Shared helpers: seeded inputs, device round trips and the parity rules.

Parity rules (north star):
  * elementwise, broadcast and index results: bit-exact (NaNs compare equal
    to each other whatever their payload);
  * reductions, softmax and softmax-derived losses: an element passes when
    |gpu - cpu| <= 1e-5 * max(|cpu|, FLT_MIN), or when the GPU value is at
    least as close to an f64 evaluation of the same formula as the CPU twin's
    is. The second clause covers ill-conditioned sums (a channel mean of
    N(0,1) data is ~0), where the twin's own sequential f32 rounding error
    exceeds 1e-5 relative. The FLT_MIN floor covers subnormal results, which
    carry fewer than 24 significant bits, so that 1e-5 relative is finer than
    their spacing (a softmax probability below 2^-126).
"""

from __future__ import annotations

import numpy as np

from darknet_zig_amd import gpu

RTOL = 1e-5
FLT_MIN = float(np.finfo(np.float32).tiny)


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def uniform(r: np.random.Generator, shape, lo=-1.0, hi=1.0) -> np.ndarray:
    return r.uniform(lo, hi, size=shape).astype(np.float32)


def normal(r: np.random.Generator, shape, mu=0.0, sigma=1.0) -> np.ndarray:
    return r.normal(mu, sigma, size=shape).astype(np.float32)


def up(a: np.ndarray) -> gpu.Buf:
    return gpu.make(np.ascontiguousarray(a))


def down(b: gpu.Buf, like: np.ndarray) -> np.ndarray:
    out = np.empty_like(like)
    gpu.pull(b, out)
    return out


def bits(a: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(a).view(np.uint32).copy()
    nan = np.isnan(a.astype(np.float32, copy=False)) if a.dtype == np.float32 else np.zeros(a.shape, bool)
    u[nan] = 0x7FC00000
    return u


def chan_sum64(terms: np.ndarray, shape) -> np.ndarray:
    """Per-channel f64 sums of per-element terms that are already rounded to
    f32 exactly as the CPU twin rounds them (the product delta*x_norm,
    (x-m)^2 of the f32 difference, ...): the f64 evaluation the reduction
    rule compares against."""
    B, F, S = shape
    return terms.astype(np.float32).astype(np.float64).reshape(B, F, S).sum(axis=(0, 2))


def chan_f32(vec: np.ndarray, shape) -> np.ndarray:
    """A per-channel vector broadcast over an NCHW tensor, in f32."""
    B, F, S = shape
    return np.broadcast_to(vec.astype(np.float32)[None, :, None], (B, F, S)).ravel()


def assert_bitexact(got: np.ndarray, want: np.ndarray, name: str) -> None:
    assert got.shape == want.shape and got.dtype == want.dtype, (name, got.shape, want.shape)
    g, w = bits(got).ravel(), bits(want).ravel()
    bad = np.nonzero(g != w)[0]
    if bad.size:
        i = bad[:5]
        raise AssertionError(
            f"{name}: {bad.size} of {g.size} elements differ; first at {i.tolist()}: "
            f"gpu={got.ravel()[i].tolist()} cpu={want.ravel()[i].tolist()}"
        )


def assert_r5(got: np.ndarray, cpu: np.ndarray, ref64: np.ndarray, name: str) -> dict:
    """The reduction rule above; returns error statistics for reporting."""
    got64, cpu64, ref = got.astype(np.float64), cpu.astype(np.float64), ref64.astype(np.float64)
    d = np.abs(got64 - cpu64)
    ok = (d <= RTOL * np.maximum(np.abs(cpu64), FLT_MIN)) | (np.abs(got64 - ref) <= np.abs(cpu64 - ref))
    ok |= (np.isnan(got64) & np.isnan(cpu64)) | (got64 == cpu64)
    if not ok.all():
        i = np.nonzero(~ok)[0][:5]
        raise AssertionError(
            f"{name}: {int((~ok).sum())} of {ok.size} outside 1e-5 of the CPU twin and farther from f64; "
            f"first {i.tolist()}: gpu={got.ravel()[i].tolist()} cpu={cpu.ravel()[i].tolist()} "
            f"f64={ref.ravel()[i].tolist()}"
        )
    scale = np.maximum(np.abs(ref), 1e-30)
    return {
        "max_rel_gpu_vs_cpu": float(np.max(d / np.maximum(np.abs(cpu64), 1e-30))),
        "max_rel_gpu_vs_f64": float(np.max(np.abs(got64 - ref) / scale)),
        "max_rel_cpu_vs_f64": float(np.max(np.abs(cpu64 - ref) / scale)),
    }


def col2im64(col: np.ndarray, channels: int, height: int, width: int, ksize: int, stride: int,
             pad: int) -> np.ndarray:
    """col2im (im2col.zig:51-79) in f64 into a zero image: every column entry
    (c, kh, kw, h, w) added to image element (c, h*stride + kh - pad,
    w*stride + kw - pad) when that lies inside the image. For fixed (kh, kw)
    the targets are distinct, so each tap is one vectorised add."""
    ho = (height + 2 * pad - ksize) // stride + 1
    wo = (width + 2 * pad - ksize) // stride + 1
    colr = np.asarray(col, np.float64).reshape(channels, ksize, ksize, ho, wo)
    im = np.zeros((channels, height, width))
    for kh in range(ksize):
        ys = kh - pad + stride * np.arange(ho)
        vy = (ys >= 0) & (ys < height)
        for kw in range(ksize):
            xs = kw - pad + stride * np.arange(wo)
            vx = (xs >= 0) & (xs < width)
            im[:, ys[vy][:, None], xs[vx][None, :]] += colr[:, kh, kw][:, vy][:, :, vx]
    return im.ravel()


def softmax_groups(n, batch, batch_offset, groups, group_offset, stride) -> np.ndarray:
    """[batch*groups, n] flat indices of every group's elements
    (gpu.zig:614-629: group (b, g) starts at b*batch_offset + g*group_offset,
    its elements `stride` apart)."""
    b = np.arange(batch)[:, None] * batch_offset
    g = np.arange(groups)[None, :] * group_offset
    start = (b + g).reshape(-1, 1)
    return start + np.arange(n)[None, :] * stride


def softmax_f64(x: np.ndarray, n, batch, batch_offset, groups, group_offset, stride, temp) -> np.ndarray:
    """The twin's softmax (blas.zig:213-223) in f64 from the twin's own f32
    exp arguments: max, then a = f32(x/T) - f32(max/T) rounded to f32 exactly
    as the twin rounds it, then exp, sum and divide in f64. Returns an array
    shaped like x (NaN outside the groups)."""
    idx = softmax_groups(n, batch, batch_offset, groups, group_offset, stride)
    v = x[idx].astype(np.float32)
    mx = np.maximum(np.max(v, axis=1, keepdims=True), np.float32(-np.finfo(np.float32).max))
    t = np.float32(temp)
    with np.errstate(invalid="ignore"):  # inf - inf in rows holding infinities, as in the twin
        a = (v / t - mx / t).astype(np.float32)
    e = np.exp(a.astype(np.float64))
    out = np.full(x.shape, np.nan)
    out[idx] = e / e.sum(axis=1, keepdims=True)
    return out


def assert_softmax(got: np.ndarray, cpu: np.ndarray, p64: np.ndarray, name: str, rel: float = 1e-6) -> dict:
    """Softmax probabilities: the 1e-5 rule against the twin (assert_r5), and
    every probability within `rel` relative (FLT_MIN floor) of the f64
    evaluation -- the device sums in f64 and its exp is within one ulp, so a
    dropped term, a wrong max or a misplaced element fails this by orders of
    magnitude."""
    stats = assert_r5(got, cpu, p64, name)
    g = got.astype(np.float64)
    bad = np.abs(g - p64) > rel * np.maximum(np.abs(p64), FLT_MIN)
    if bad.any():
        i = np.nonzero(bad)[0][:5]
        raise AssertionError(f"{name}: {int(bad.sum())} probabilities farther than {rel} from f64; first "
                             f"{i.tolist()}: gpu={got[i].tolist()} f64={p64[i].tolist()}")
    return stats
