"""Attention-backend registry (counterpart of attention/__init__.py:15-26)."""

from __future__ import annotations

from typing import TYPE_CHECKING

from .base import BaseAttnBackend, PrefillMetadata
from .hip import HipAttnBackend, HipDecodeMetadata

if TYPE_CHECKING:
    import numpy as np

    from minisgl_hip.core import ModelConfig
    from minisgl_hip.kvcache import MHAKVCache

SUPPORTED_ATTENTION_BACKENDS = {
    "hip": HipAttnBackend,  # gfx950 paged decode + ragged prefill kernels
}


def create_attention_backend(
    name: str, config: "ModelConfig", kv_cache: "MHAKVCache", page_table: "np.ndarray"
) -> BaseAttnBackend:
    if name not in SUPPORTED_ATTENTION_BACKENDS:
        raise ValueError(f"Unknown attention backend {name!r}: {list(SUPPORTED_ATTENTION_BACKENDS)}")
    return SUPPORTED_ATTENTION_BACKENDS[name](config, kv_cache, page_table)


__all__ = [
    "BaseAttnBackend",
    "PrefillMetadata",
    "HipAttnBackend",
    "HipDecodeMetadata",
    "SUPPORTED_ATTENTION_BACKENDS",
    "create_attention_backend",
]
