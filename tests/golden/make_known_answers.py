"""Writes reference_known_answers.json: the known answers held by the
reference's own tests for the tensor-op path, as data.

Each entry records the inputs, the call, the expected values and the tolerance
the reference test uses, with the file:line it comes from. The reference
stores no fixture files and its gputest pins nothing bit-level
(gputest.zig:27-52, 1e-3 either-abs-or-rel), so these test-block values are
all the golden data it has for this path. Values are transcribed; nothing
from the reference is executed.

Usage: python tests/golden/make_known_answers.py
"""

from __future__ import annotations

import json
from pathlib import Path

OUT = Path(__file__).resolve().parent / "reference_known_answers.json"

CASES = [
    {
        "source": "src/blas.zig:324-332",
        "name": "softmax sums to one and cross entropy matches",
        "op": "softmax",
        "args": {"input": [1.0, 2.0, 3.0, 4.0], "n": 4, "batch": 1, "batch_offset": 4, "groups": 1,
                 "group_offset": 4, "stride": 1, "temp": 1.0},
        "expect": {"sum": 1.0, "sum_abs_tol": 1e-6, "output3_gt_output0": True},
    },
    {
        "source": "src/blas.zig:334-346",
        "name": "normalize then denormalize round trips",
        "op": "mean_variance_normalize",
        "args": {"x": [1, 2, 3, 4, 5, 6, 7, 8], "batch": 1, "filters": 2, "spatial": 4},
        "expect": {"mean": [2.5, 6.5], "mean_abs_tol": 1e-6, "normalized_channel0_sum": 0.0,
                   "normalized_sum_abs_tol": 1e-5},
    },
    {
        "source": "src/activations.zig:145-150",
        "name": "leaky activation and its gradient agree with darknet",
        "op": "leaky",
        "args": {"activate": [2.0, -2.0], "gradient": [2.0, -0.2]},
        "expect": {"activate": [2.0, -0.2], "gradient": [1.0, 0.1], "abs_tol": 1e-6},
    },
    {
        "source": "src/smoke_test.zig:229-274",
        "name": "batch norm rolling statistics follow darknet's 0.99 EMA",
        "op": "bn_rolling_ema",
        "args": {"batch": 4, "w": 3, "h": 3, "c": 2, "input_uniform": [-2.0, 2.0], "steps": 200,
                 "momentum": 0.99},
        "expect": {"rolling_over_batch_stat": "1 - 0.99**steps", "rel_tol": 1e-3,
                   "fraction_range": [0.86, 0.88]},
    },
    {
        "source": "src/smoke_test.zig:276-308",
        "name": "flat-index decomposition covers every output element exactly once",
        "op": "nchw_bijection",
        "args": {"batch": 3, "n": 5, "size": 7},
        "expect": {"each_index_hit": 1},
    },
    {
        "source": "src/im2col.zig:87-95",
        "name": "im2col of a 3x3 image with a 2x2 kernel",
        "op": "im2col",
        "args": {"im": [1, 2, 3, 4, 5, 6, 7, 8, 9], "channels": 1, "height": 3, "width": 3, "ksize": 2,
                 "stride": 1, "pad": 0, "col_len": 16},
        "expect": {"col[0:4]": [1, 2, 4, 5], "col[12:16]": [5, 6, 8, 9], "exact": True},
    },
    {
        "source": "src/im2col.zig:97-104",
        "name": "col2im accumulates overlapping contributions",
        "op": "col2im",
        "args": {"col_fill": 1.0, "col_len": 16, "channels": 1, "height": 3, "width": 3, "ksize": 2,
                 "stride": 1, "pad": 0, "im_len": 9},
        "expect": {"im[4]": 4.0, "im[0]": 1.0, "abs_tol": 1e-6},
    },
    {
        "source": "src/gemm.zig:265-315",
        "name": "gemm variants agree with a naive reference",
        "op": "gemm",
        "args": {"m": 5, "n": 4, "k": 3, "a": "a[i] = i % 7 over m*k, row-major m x k",
                 "b": "b[i] = i % 5 over k*n, row-major k x n",
                 "transposed": "at[p*m + i] = a[i*k + p], bt[q*k + p] = b[p*n + q]",
                 "alpha": 2.0, "beta": 1.0, "c0": 0.0, "lda": "m if ta else k", "ldb": "k if tb else n",
                 "ldc": "n", "variants": [[False, False], [True, False], [False, True], [True, True]]},
        "expect": {"want": "want[i*n + q] = 2 * sum_p a[i*k + p] * b[p*n + q]", "abs_tol": 1e-4},
    },
]


def main() -> None:
    OUT.write_text(json.dumps({"reference": "Eightscer/darknet_zig", "cases": CASES}, indent=2) + "\n")
    print(OUT)


if __name__ == "__main__":
    main()
