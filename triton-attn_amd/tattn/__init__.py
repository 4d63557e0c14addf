"""FlashAttention-2 style fused attention for AMD Instinct MI355X (gfx950), HIP kernels.

Drop-in for amaanmithani/triton-attn's `tattn` package (src/tattn/__init__.py:3-5).
"""

from tattn.api import attention, autotune_cache, configs, hip_available, set_autotune, triton_available

__all__ = ["attention", "triton_available", "hip_available", "configs", "set_autotune", "autotune_cache"]
