"""ctypes binding of libdkz.so, the C ABI declared in include/dkz_ops.h.

This is the Python-side equivalent of the extern declarations a Zig host would
write against the same header. Every exported symbol is listed in SIGNATURES;
tests check the table against the header and the built library.

There is deliberately no fallback: if libdkz.so has not been built (or cannot
be loaded), load() raises and nothing runs.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libdkz.so"

_p = C.c_void_p
_i = C.c_int
_f = C.c_float
_sz = C.c_size_t

# name -> (restype, argtypes), in the order of include/dkz_ops.h.
SIGNATURES: dict[str, tuple] = {
    "dkz_init": (_i, [_i]),
    "dkz_device_count": (_i, [C.POINTER(_i)]),
    "dkz_device_name": (_i, [_i, C.c_char_p, _i]),
    "dkz_mem_info": (_i, [C.POINTER(_sz), C.POINTER(_sz)]),
    "dkz_malloc": (_i, [C.POINTER(_p), _sz]),
    "dkz_free": (_i, [_p]),
    "dkz_memset_zero": (_i, [_p, _sz]),
    "dkz_copy_to_device": (_i, [_p, _p, _sz]),
    "dkz_copy_to_host": (_i, [_p, _p, _sz]),
    "dkz_synchronize": (_i, []),
    "dkz_error_string": (C.c_char_p, [_i]),
    "dkz_set_sync_after_launch": (None, [_i]),
    "dkz_get_sync_after_launch": (_i, []),
    "dkz_last_error_context": (C.c_char_p, []),
    "dkz_set_stream": (_i, [_p]),
    "dkz_get_stream": (_p, []),
    "dkz_fill": (_i, [_p, _i, _f]),
    "dkz_copy": (_i, [_i, _p, _p]),
    "dkz_axpy": (_i, [_i, _f, _p, _p]),
    "dkz_scal": (_i, [_i, _f, _p]),
    "dkz_mul": (_i, [_i, _p, _p]),
    "dkz_add_scalar": (_i, [_i, _f, _p]),
    "dkz_constrain": (_i, [_i, _f, _p]),
    "dkz_rand_uniform": (_i, [_i, _p, C.c_uint]),
    "dkz_activate_array": (_i, [_p, _i, _i]),
    "dkz_gradient_array": (_i, [_p, _i, _i, _p]),
    "dkz_add_bias": (_i, [_p, _p, _i, _i, _i]),
    "dkz_scale_bias": (_i, [_p, _p, _i, _i, _i]),
    "dkz_backward_bias": (_i, [_p, _p, _i, _i, _i]),
    "dkz_backward_scale": (_i, [_p, _p, _i, _i, _i, _p]),
    "dkz_mean": (_i, [_p, _i, _i, _i, _p]),
    "dkz_variance": (_i, [_p, _p, _i, _i, _i, _p]),
    "dkz_normalize": (_i, [_p, _p, _p, _i, _i, _i]),
    "dkz_mean_delta": (_i, [_p, _p, _i, _i, _i, _p]),
    "dkz_variance_delta": (_i, [_p, _p, _p, _p, _i, _i, _i, _p]),
    "dkz_normalize_delta": (_i, [_p, _p, _p, _p, _p, _i, _i, _i, _p]),
    "dkz_softmax": (_i, [_p, _i, _i, _i, _i, _i, _i, _f, _p]),
    "dkz_softmax_layer_forward": (_i, [_i, _i, _i, _f, _p, _p, _p, _p, _p]),
    "dkz_softmax_cross_entropy": (_i, [_i, _p, _p, _p, _p]),
    "dkz_l2": (_i, [_i, _p, _p, _p, _p]),
    "dkz_l1": (_i, [_i, _p, _p, _p, _p]),
    "dkz_smooth_l1": (_i, [_i, _p, _p, _p, _p]),
    "dkz_forward_maxpool": (_i, [_i, _i, _i, _i, _i, _i, _i, _p, _p, _p]),
    "dkz_backward_maxpool": (_i, [_i, _i, _i, _i, _i, _i, _i, _p, _p, _p]),
    "dkz_forward_avgpool": (_i, [_i, _i, _i, _i, _p, _p]),
    "dkz_backward_avgpool": (_i, [_i, _i, _i, _i, _p, _p]),
    "dkz_shortcut": (_i, [_i, _i, _i, _i, _p, _i, _i, _i, _f, _f, _p]),
    "dkz_im2col": (_i, [_p, _i, _i, _i, _i, _i, _i, _p]),
    "dkz_col2im": (_i, [_p, _i, _i, _i, _i, _i, _i, _p]),
    "dkz_gemm": (_i, [_i, _i, _i, _i, _i, _f, _p, _i, _p, _i, _f, _p, _i]),
    "dkz_convolution_forward": (_i, [_i] * 9 + [_p] * 3),
    "dkz_convolution_weight_gradient": (_i, [_i] * 9 + [_p] * 3),
    "dkz_convolution_data_gradient": (_i, [_i] * 9 + [_p] * 3),
    "dkz_dropout": (_i, [_p, _i, _p, _f, _f]),
    "dkz_adam_update": (_i, [_p, _p, _p, _p, _f, _f, _f, _f, _f, _i, _i, _i]),
    "dkz_batchnorm_forward": (_i, [_i, _i, _i, _i, _i] + [_p] * 10),
    "dkz_batchnorm_backward": (_i, [_i, _i, _i, _i] + [_p] * 11),
    "dkz_batchnorm_backward_noalloc": (_i, [_i, _i, _i, _i] + [_p] * 11),
}

_LIB: C.CDLL | None = None


def load(path: Path | str | None = None) -> C.CDLL:
    """Loads libdkz.so (once) and declares every signature. Raises if absent.

    $DKZ_LIBRARY names another build of the library, as $DARKNET_KERNELS names
    another code object in the reference (gpu.zig:240-244).
    """
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    env = os.environ.get("DKZ_LIBRARY")
    p = Path(path) if path is not None else Path(env) if env else LIB_PATH
    if not p.exists():
        raise ImportError(
            f"{p} is not built; the HIP tensor-op library is required "
            "(build it with `python -m darknet_zig_amd.build`)"
        )
    lib = C.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError names a missing export
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _LIB = lib
    return lib
