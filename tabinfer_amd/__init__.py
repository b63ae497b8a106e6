"""tabinfer_amd — MI355X (gfx950) implementation of TabInfer's quantized decode path.

The product is libtabinfer.so (C ABI in include/ti.h, HIP kernels in csrc/)
and the Node.js host in js/. This package holds the build script and the
ctypes binding used by Python callers.
"""
__all__ = ["abi", "build"]
