"""tabinfer_amd — MI355X (gfx950) implementation of TabInfer's quantized decode path.

The product is libtabinfer.so (C ABI in include/ti.h, HIP kernels in csrc/)
and the Node.js host in host/ (the N-API addon ti_node.cc, the engine launchers
ti-engine.js, the Qwen3 host qwen3-host.js with conversation.js, tokenizer.js and
quant-cache.js). This package also holds the build script and the ctypes binding
used by Python callers.
"""
__all__ = ["abi", "build"]
