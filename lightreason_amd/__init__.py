"""MI355X-native MoE expert-layer hot path for the Qwen3.6-35B-A3B runner.

``lightreason_amd.moe`` is the torch-facing API over ``liblrmoe.so`` (HIP
kernels for gfx950, C ABI in ``include/lrmoe.h``); ``lightreason_amd.edge35b``
keeps the reference runner's module surface (fused_experts,
native_bf16_gather, packed_native, ...) on top of it.  Importing the package
does not load the library; the first kernel call does, and raises if it is
missing.
"""

__all__ = ["moe", "synthetic", "edge35b"]
