"""MI355X (gfx950) attention backend for mini-sglang-mlx's attention hot path.

Host side in Python over a C ABI (include/msgl_attn.h); device side is
hand-written HIP in ``csrc/``. Public pieces mirror the reference's
``minisgl_mlx.attention`` and ``minisgl_mlx.kvcache`` interfaces.
"""

from .ops import paged_decode_attention, store_kv  # noqa: F401

__all__ = ["paged_decode_attention", "store_kv"]
