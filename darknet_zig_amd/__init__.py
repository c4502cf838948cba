"""MI355X-native (gfx950) implementation of darknet-zig's tensor-op layer.

The product is libdkz.so, a C-ABI library (include/dkz_ops.h) of hand-written
HIP kernels for the elementwise, broadcast, reduction, softmax, pooling and
shortcut ops that darknet-zig's src/gpu.zig dispatches. This package builds it
(`darknet_zig_amd.build`), binds it (`darknet_zig_amd._lib`) and mirrors
gpu.zig's op API on top of it (`darknet_zig_amd.gpu`).
"""

from .activations import Activation  # noqa: F401

__all__ = ["Activation", "gpu", "build"]
