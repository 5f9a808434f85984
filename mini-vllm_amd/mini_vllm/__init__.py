"""Mini-vLLM's paged-attention hot path, MI355X-native.

The package keeps the reference's module names (``mini_vllm.kernels.ops``,
``mini_vllm.kernels.extension``, ...) so callers switch by import path alone. The
kernels live in ``libminivllm_hip.so`` (HIP for gfx950, C ABI in
``include/minivllm_hip.h``); the modules here are the host side around it.
"""

__all__ = ["__version__"]
__version__ = "0.1.0"
