"""Attention-backend interface (counterpart of attention/base.py:40-105).

q/k/v arrive packed as [T, H, D]; each token may only attend to tokens of its
own request at positions not after its own, and those tokens' K/V sit at
arbitrary slots of the shared pool, found through the token-granular page
table. Prefill and decode are prepared and run separately
(attention/base.py:49-60): ``prepare_metadata`` is called once per step on the
host, ``forward`` once per layer after ``kv_cache.store_kv`` has written the
step's rows (layers.py:109-110).
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from dataclasses import dataclass
from typing import TYPE_CHECKING, Any, List, Optional

import numpy as np

if TYPE_CHECKING:
    import torch

    from minisgl_hip.core import Batch, ModelConfig
    from minisgl_hip.kvcache import MHAKVCache


@dataclass
class PrefillMetadata:
    """attention/base.py:32-37 plus the device-side ragged description the kernel reads.

    ``last_indices`` [R]: packed index of each request's last token (read by
    models/transformer.py:112); ``q_offsets`` [R+1] (host list);
    ``kv_indices``: per request, slots of the full (prefix + extend) KV or None
    when nothing was cached (attention/base.py:70-83).
    """

    last_indices: "torch.Tensor"
    q_offsets: List[int]
    kv_indices: List[Optional[np.ndarray]]
    device: Any = None  # backend-specific device tensors


class BaseAttnBackend(ABC):
    def __init__(self, config: "ModelConfig", kv_cache: "MHAKVCache", page_table: np.ndarray) -> None:
        self.config = config
        self.kv_cache = kv_cache
        self.page_table = page_table
        self.scale = config.head_dim**-0.5  # attention/base.py:45

    # ------------------------------------------------------------------ interface

    def prepare_metadata(self, batch: "Batch") -> None:
        """attention/base.py:49-54: host-side index preparation before forward.
        A ``"mixed"`` batch (decode requests first, then prefill chunks; the
        reference never forms one) goes to ``prepare_mixed``."""
        if batch.phase == "mixed":
            batch.attn_metadata = self.prepare_mixed(batch)
        elif batch.is_prefill:
            batch.attn_metadata = self._prepare_prefill(batch)
        else:
            batch.attn_metadata = self.prepare_decode(batch)

    def forward(self, q, k, v, layer_id: int, batch: "Batch"):
        """attention/base.py:56-60. q [T, Hq, D], k/v [T, Hkv, D] (already stored) -> o [T, Hq, D]."""
        if batch.phase == "mixed":
            return self.forward_mixed(q, k, v, layer_id, batch.attn_metadata)
        if batch.is_prefill:
            return self._forward_prefill(q, k, v, layer_id, batch.attn_metadata)
        return self.forward_decode(q, layer_id, batch.attn_metadata)

    def prepare_mixed(self, batch: "Batch"):
        raise NotImplementedError(f"{type(self).__name__} runs one phase per batch (attention/base.py:49-60)")

    def forward_mixed(self, q, k, v, layer_id: int, metadata):
        raise NotImplementedError(f"{type(self).__name__} runs one phase per batch (attention/base.py:49-60)")

    @abstractmethod
    def prepare_decode(self, batch: "Batch"): ...

    @abstractmethod
    def forward_decode(self, q, layer_id: int, metadata): ...

    # prefill: shared in the reference (an MLX SDPA loop); each backend here
    # provides its own.
    @abstractmethod
    def _prepare_prefill(self, batch: "Batch") -> PrefillMetadata: ...

    @abstractmethod
    def _forward_prefill(self, q, k, v, layer_id: int, meta: PrefillMetadata): ...
