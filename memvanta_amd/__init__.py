"""MI355X (gfx950) backend for MemVanta's quantized-matmul + paged F16 attention hot path.

The product is the C ABI in include/memvanta_hip.h, implemented by
libmemvanta_hip.so (hand-written HIP kernels in csrc/).  ``capi`` binds it for
Python callers; ``synth`` writes the synthetic GGUF inputs the benchmarks use.
"""
from .capi import Context, KVCache, MvhError, Tensor, load_library  # noqa: F401

__all__ = ["Context", "KVCache", "MvhError", "Tensor", "load_library"]
