"""The C ABI as a boundary: declared == exported == bound, and the host-side
argument handling that runs before any HIP call (no GPU needed).

gpu.zig's contract for these cases: n == 0 / filters == 0 launch nothing
(gpu.zig:468, 475); a bad size would panic in ci() (gpu.zig:416-418) and a bad
device index returns NoSuchDevice (gpu.zig:274-277). Here they are status
codes: 0, or hipErrorInvalidValue (1) / a HIP error.
"""

from __future__ import annotations

import ctypes as C
import re
import subprocess

import pytest

from darknet_zig_amd import _lib, gpu
from darknet_zig_amd.activations import Activation

ROOT = _lib.LIB_PATH.parents[1]
HEADER = ROOT / "include" / "dkz_ops.h"

# The public op wrappers of src/gpu.zig:483-800 on this path, and their
# mirror in darknet_zig_amd.gpu.
GPU_ZIG_OPS = [
    "fill", "copy", "axpy", "scal", "mul", "addScalar", "constrainArray", "randUniform", "activateArray",
    "gradientArray",
    "addBias", "scaleBias", "backwardBias", "backwardScale", "mean", "variance", "normalize",
    "meanDelta", "varianceDelta", "normalizeDelta", "softmax", "softmaxCrossEntropy", "l2", "l1",
    "smoothL1", "forwardMaxpool", "backwardMaxpool", "forwardAvgpool", "backwardAvgpool", "im2col", "col2im", "gemm",
    "dropout", "shortcut",
    "adamUpdate",
]


def header_symbols() -> list[str]:
    text = HEADER.read_text()
    return re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(dkz_\w+)\s*\(", text, flags=re.M)


def exported_symbols() -> set[str]:
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    return {ln.split()[-1] for ln in out.splitlines() if ln.split() and ln.split()[-1].startswith("dkz_")}


def test_header_exports_and_binding_agree():
    declared = header_symbols()
    assert len(declared) == len(set(declared)) == 58
    assert set(declared) == exported_symbols()
    assert list(_lib.SIGNATURES) == declared  # same set, same order as the header


def test_only_dkz_symbols_exported():
    """The library exports exactly the header's entry points: no kernel, no
    internal C++ function, no compiler-emitted host symbol (hidden
    visibility plus darknet_zig_amd/libdkz.map)."""
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    names = sorted(ln.split()[-1] for ln in out.splitlines() if len(ln.split()) >= 3)
    assert names == sorted(header_symbols()), sorted(set(names) ^ set(header_symbols()))


def test_library_loads_every_symbol():
    lib = _lib.load()
    for name in _lib.SIGNATURES:
        assert getattr(lib, name) is not None


def test_gpu_mirror_has_gpu_zig_ops():
    for name in GPU_ZIG_OPS:
        assert callable(getattr(gpu, name)), name


def test_activation_codes():
    # activations.zig:14-27
    assert [a.name for a in Activation] == ["logistic", "relu", "relie", "linear", "ramp", "tanh", "plse",
                                            "leaky", "elu", "loggy", "stair", "hardtan", "lhtan", "selu"]
    assert [int(a) for a in Activation] == list(range(14))
    assert Activation.fromString("leaky") is Activation.leaky
    assert Activation.fromString("nonsense") is Activation.relu  # activations.zig:49-50


INVALID = 1  # hipErrorInvalidValue

P = C.c_void_p(16)  # a non-null pointer value; never dereferenced in these calls


@pytest.mark.parametrize(
    "call, expect",
    [
        (lambda L: L.dkz_axpy(-1, 1.0, P, P), INVALID),
        (lambda L: L.dkz_axpy(0, 1.0, None, None), 0),
        (lambda L: L.dkz_axpy(5, 1.0, None, P), INVALID),
        (lambda L: L.dkz_fill(None, 0, 1.0), 0),
        (lambda L: L.dkz_scal(3, 2.0, None), INVALID),
        (lambda L: L.dkz_activate_array(P, 4, 14), INVALID),
        (lambda L: L.dkz_activate_array(P, 4, -1), INVALID),
        (lambda L: L.dkz_activate_array(P, 4, int(Activation.linear)), 0),  # linear: nothing to do
        (lambda L: L.dkz_gradient_array(P, 0, 99, P), INVALID),  # the code is checked before n == 0
        (lambda L: L.dkz_add_bias(P, P, 2, -1, 3), INVALID),
        (lambda L: L.dkz_add_bias(None, None, 0, 5, 3), 0),
        (lambda L: L.dkz_mean(P, 2, 0, 3, None), 0),  # filters == 0
        (lambda L: L.dkz_mean(P, 2, 3, 3, None), INVALID),
        (lambda L: L.dkz_backward_bias(None, None, 0, 4, 9), 0),  # batch 0 adds nothing
        (lambda L: L.dkz_normalize_delta(P, P, P, P, P, 2, 3, -4, P), INVALID),
        (lambda L: L.dkz_softmax(P, 10, 2, 10, 1, 10, 1, 1.0, None), INVALID),
        (lambda L: L.dkz_softmax(None, 10, 0, 10, 1, 10, 1, 1.0, None), 0),
        (lambda L: L.dkz_softmax(P, 10, 2, -10, 1, 10, 1, 1.0, P), INVALID),
        (lambda L: L.dkz_softmax_cross_entropy(4, P, None, P, P), INVALID),
        (lambda L: L.dkz_forward_maxpool(98, 14, 14, 2, 0, 2, 1, P, P, P), INVALID),  # stride 0
        (lambda L: L.dkz_forward_maxpool(98, 1, 1, 2, 1, 3, 0, P, P, P), INVALID),  # window > input
        (lambda L: L.dkz_forward_maxpool(97, 14, 14, 2, 2, 2, 1, P, P, P), INVALID),  # not whole planes
        (lambda L: L.dkz_backward_maxpool(0, 14, 14, 2, 2, 2, 1, None, None, None), 0),
        (lambda L: L.dkz_forward_avgpool(0, 7, 7, 3, None, None), 0),
        (lambda L: L.dkz_backward_avgpool(6, 7, 7, 3, None, P), INVALID),
        (lambda L: L.dkz_shortcut(2, 8, 8, 0, None, 8, 8, 4, 1.0, 1.0, None), 0),  # min channels 0
        (lambda L: L.dkz_shortcut(2, 8, 8, 4, None, 8, 8, 4, 1.0, 1.0, P), INVALID),
        (lambda L: L.dkz_batchnorm_forward(2, 3, 4, 14, 1, P, P, P, P, P, P, P, P, P, P), INVALID),
        (lambda L: L.dkz_batchnorm_forward(2, -3, 4, 7, 1, P, P, P, P, P, P, P, P, P, P), INVALID),
        (lambda L: L.dkz_batchnorm_forward(2, 0, 4, 7, 1, *[None] * 10), 0),  # filters 0: nothing to do
        (lambda L: L.dkz_batchnorm_forward(2, 3, 4, 7, 1, P, P, P, None, P, P, P, P, P, P), INVALID),  # x_norm
        (lambda L: L.dkz_batchnorm_forward(2, 3, 4, 7, 0, P, P, P, P, P, P, None, P, P, P), INVALID),  # rolling
        (lambda L: L.dkz_batchnorm_forward(65536, 65536, 4, 7, 1, P, P, P, P, P, P, P, P, P, P), INVALID),
        (lambda L: L.dkz_batchnorm_backward(2, 3, 4, -1, P, P, P, P, P, P, P, P, P, P, P), INVALID),
        (lambda L: L.dkz_batchnorm_backward(2, 3, 4, 7, None, P, P, P, P, P, P, P, P, P, P), INVALID),  # y
        (lambda L: L.dkz_batchnorm_backward(2, 3, 4, 7, P, P, P, P, P, P, P, P, P, None, P), INVALID),
        (lambda L: L.dkz_batchnorm_backward(0, 0, 4, 7, *[None] * 11), 0),
        (lambda L: L.dkz_add_scalar(-2, 1.0, P), INVALID),
        (lambda L: L.dkz_add_scalar(3, 1.0, None), INVALID),
        (lambda L: L.dkz_rand_uniform(0, None, 7), 0),
        (lambda L: L.dkz_rand_uniform(9, None, 7), INVALID),
        (lambda L: L.dkz_dropout(P, 5, None, 0.5, 2.0), INVALID),
        (lambda L: L.dkz_dropout(None, 0, None, 0.5, 2.0), 0),
        (lambda L: L.dkz_adam_update(None, None, None, None, 0.9, 0.999, 1e-7, 0.0, 0.1, 0, 1, 1), 0),
        (lambda L: L.dkz_adam_update(P, P, C.c_void_p(4096), C.c_void_p(8192), 0.9, 0.999, 1e-7, 0.0, 0.1, 4, 1,
                                     1), INVALID),  # w and d overlap
        (lambda L: L.dkz_adam_update(P, C.c_void_p(32), C.c_void_p(4096), C.c_void_p(8192), 0.9, 0.999, 1e-7, 0.0,
                                     0.1, 5, 1, 1), INVALID),  # [16, 36) and [32, 52) overlap
        (lambda L: L.dkz_adam_update(P, P, P, P, 0.9, 0.999, 1e-7, 0.0, 0.1, -1, 1, 1), INVALID),
        (lambda L: L.dkz_im2col(P, 3, 4, 4, 7, 1, 1, P), INVALID),  # window larger than the padded image
        (lambda L: L.dkz_im2col(P, 3, 4, 4, 3, 0, 1, P), INVALID),  # stride 0
        (lambda L: L.dkz_im2col(P, 3, 4, 4, 0, 1, 1, P), INVALID),  # ksize 0
        (lambda L: L.dkz_im2col(None, 0, 4, 4, 3, 1, 1, None), 0),  # no channels
        (lambda L: L.dkz_col2im(P, 3, 4, -4, 3, 1, 1, P), INVALID),
        (lambda L: L.dkz_col2im(P, 3, 4, 4, 3, 1, 1, None), INVALID),
        (lambda L: L.dkz_col2im(P, 65536, 256, 256, 3, 1, 1, P), INVALID),  # beyond 32-bit indexing
        # shapes whose element count passes 2^31 - 1 (each argument fits an int)
        (lambda L: L.dkz_mean(P, 65536, 65536, 1, P), INVALID),
        (lambda L: L.dkz_backward_bias(P, P, 46341, 46341, 1), INVALID),
        (lambda L: L.dkz_add_bias(P, P, 46341, 46341, 1), INVALID),
        (lambda L: L.dkz_softmax(P, 1000, 2147484, 1000, 1, 1000, 1, 1.0, P), INVALID),  # last row ends past 2^31
        (lambda L: L.dkz_forward_maxpool(1 << 29, 256, 256, 32768, 2, 2, 0, P, P, P), INVALID),  # 2^31 inputs
        (lambda L: L.dkz_forward_avgpool(32768, 256, 256, 1, P, P), INVALID),
        (lambda L: L.dkz_backward_avgpool(32768, 256, 256, 1, P, P), INVALID),
        (lambda L: L.dkz_gemm(0, 0, 0, 5, 5, 1.0, None, 5, None, 5, 0.0, None, 5), 0),  # m == 0
        (lambda L: L.dkz_gemm(0, 0, 4, 5, 3, 1.0, P, 2, P, 5, 0.0, P, 5), INVALID),  # lda < k
        (lambda L: L.dkz_gemm(1, 0, 4, 5, 3, 1.0, P, 3, P, 5, 0.0, P, 5), INVALID),  # lda < m (A transposed)
        (lambda L: L.dkz_gemm(0, 1, 4, 5, 3, 1.0, P, 3, P, 2, 0.0, P, 5), INVALID),  # ldb < k (B transposed)
        (lambda L: L.dkz_gemm(0, 0, 4, 5, 3, 1.0, P, 3, P, 5, 0.0, P, 4), INVALID),  # ldc < n
        (lambda L: L.dkz_gemm(0, 0, 4, 5, 3, 1.0, None, 3, P, 5, 0.0, P, 5), INVALID),
        (lambda L: L.dkz_gemm(0, 0, 65536, 65536, 3, 1.0, P, 3, P, 65536, 0.0, P, 65536), INVALID),  # > 2^31
        # the three convolution entry points share their shape checks
        *[(lambda L, f=f, a=a, ptrs=ptrs: getattr(L, f)(*a, *ptrs), want)
          for f in ("dkz_convolution_forward", "dkz_convolution_weight_gradient", "dkz_convolution_data_gradient")
          for a, ptrs, want in (
              ((2, 0, 4, 8, 8, 4, 3, 1, 1), (P, P, P), INVALID),  # groups 0
              ((2, 3, 4, 8, 8, 6, 3, 1, 1), (P, P, P), INVALID),  # channels % groups != 0
              ((2, 2, 4, 8, 8, 5, 3, 1, 1), (P, P, P), INVALID),  # filters % groups != 0
              ((2, 1, 4, 8, 8, 6, 0, 1, 1), (P, P, P), INVALID),  # ksize 0
              ((2, 1, 4, 8, 8, 6, 3, 0, 1), (P, P, P), INVALID),  # stride 0
              ((2, 1, 4, 8, 8, 6, 3, 1, -1), (P, P, P), INVALID),  # pad < 0
              ((2, 1, 4, 2, 2, 6, 7, 1, 1), (P, P, P), INVALID),  # window larger than the padded image
              ((2, 1, 4, 8, 8, 6, 1, 1, 1), (P, P, P), INVALID),  # ksize 1 reading past the image (n > h*w)
              ((2, 1, 4, 8, 8, 6, 3, 1, 1), (None, P, P), INVALID),
              ((2, 1, 4, 8, 8, 6, 3, 1, 1), (P, P, None), INVALID),
              ((65536, 1, 1, 256, 256, 1, 1, 1, 0), (P, P, P), INVALID),  # beyond 32-bit indexing
              ((0, 1, 4, 8, 8, 6, 3, 1, 1), (None, None, None), 0),  # no images: nothing to do
          )],
        (lambda L: L.dkz_softmax_layer_forward(2, 10, 3, 1.0, P, P, P, P, P), INVALID),  # 10 % 3 != 0
        (lambda L: L.dkz_softmax_layer_forward(0, 10, 2, 1.0, None, None, None, None, None), 0),
        (lambda L: L.dkz_softmax_layer_forward(2, 100, 1, 1.0, P, P, P, None, P), INVALID),  # truth without delta
        (lambda L: L.dkz_malloc(None, 4), INVALID),
        (lambda L: L.dkz_free(None), 0),
        (lambda L: L.dkz_copy_to_host(None, None, 0), 0),
    ],
)
def test_host_side_validation(call, expect):
    assert call(_lib.load()) == expect


def test_error_context_names_the_check():
    lib = _lib.load()
    assert lib.dkz_scal(-3, 1.0, P) == INVALID
    assert b"dkz_scal" in lib.dkz_last_error_context()
    assert lib.dkz_error_string(INVALID)


def test_sync_after_launch_toggle():
    lib = _lib.load()
    before = lib.dkz_get_sync_after_launch()
    lib.dkz_set_sync_after_launch(1)
    assert lib.dkz_get_sync_after_launch() == 1
    lib.dkz_set_sync_after_launch(0)
    assert lib.dkz_get_sync_after_launch() == 0
    lib.dkz_set_sync_after_launch(before)


def test_stream_selection_round_trips():
    lib = _lib.load()
    assert lib.dkz_set_stream(None) == 0
    assert lib.dkz_get_stream() is None


def test_init_without_a_device_fails_loudly():
    lib = _lib.load()
    n = C.c_int(0)
    if lib.dkz_device_count(C.byref(n)) == 0 and n.value > 0:
        pytest.skip("a GPU is present")
    assert lib.dkz_init(0) != 0
    with pytest.raises(gpu.GpuError):
        gpu.init(0)


def test_buf_offset():
    b = gpu.Buf(4096, 10)
    assert b.offset(3) == gpu.Buf(4096 + 12, 7)
    assert gpu.Buf().offset(2).is_null()


def test_gputest_program_links_and_fails_loudly_without_a_gpu():
    """The gputest harness resolves libdkz and the oracle, and without a
    device it stops with gpu.zig's must() message instead of running."""
    from tests.native import build as native_build

    lib = _lib.load()
    n = C.c_int(0)
    if lib.dkz_device_count(C.byref(n)) == 0 and n.value > 0:
        pytest.skip("a GPU is present")
    proc = subprocess.run([str(native_build.GPUTEST)], capture_output=True, text=True, timeout=60)
    assert proc.returncode == 2, proc.stdout + proc.stderr
    assert "selecting the device failed" in proc.stdout
