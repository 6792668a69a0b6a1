"""The data contract the attention path reads (counterpart of core.py:29-158).

Only the fields the backend touches are kept: a request's ``table_idx``,
``cached_len`` and ``device_len`` (core.py:42-96), a batch's ``reqs``,
``phase``, ``positions``, ``out_loc`` and ``attn_metadata`` (core.py:99-120),
and the process-wide context (core.py:123-158). Scheduling, sampling and the
prefix cache are the caller's business and are not restated.
"""

from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass, field
from typing import Any, List, Literal, Optional

import numpy as np


@dataclass(eq=False)
class Req:
    """core.py:42-96: token span [cached_len, device_len) is this step's extend part."""

    input_ids: np.ndarray
    table_idx: int
    cached_len: int
    output_len: int = 1
    uid: int = 0

    def __post_init__(self) -> None:
        self.device_len = len(self.input_ids)
        self.max_device_len = len(self.input_ids) + self.output_len
        assert 0 <= self.cached_len < self.device_len <= self.max_device_len

    @property
    def extend_len(self) -> int:
        return self.device_len - self.cached_len

    def complete_one(self) -> None:
        """core.py:81-83."""
        self.cached_len = self.device_len
        self.device_len += 1


@dataclass
class Batch:
    """core.py:99-120. ``positions``/``out_loc`` are filled by the caller, ``attn_metadata`` by the backend.

    ``phase`` ``"mixed"`` (not formed by the reference, whose batches hold one
    phase, core.py:102): decode requests (one new token each) first, then
    prefill chunks, run as one continuous-batching step."""

    reqs: List[Req]
    phase: Literal["prefill", "decode", "mixed"]
    input_ids: Any = field(default=None, init=False)
    positions: Any = field(default=None, init=False)
    out_loc: Any = field(default=None, init=False)
    attn_metadata: Any = field(default=None, init=False)

    @property
    def is_prefill(self) -> bool:
        return self.phase == "prefill"

    @property
    def is_decode(self) -> bool:
        return self.phase == "decode"

    @property
    def size(self) -> int:
        return len(self.reqs)


@dataclass
class Context:
    """core.py:123-145: page table (token-granular, CPU int32), KV pool, backend, active batch."""

    page_size: int
    page_table: np.ndarray = field(default=None, init=False)
    kv_cache: Any = field(default=None, init=False)
    attn_backend: Any = field(default=None, init=False)
    _batch: Optional[Batch] = field(default=None, init=False)

    @property
    def batch(self) -> Batch:
        assert self._batch is not None, "No active batch in context"
        return self._batch

    @contextmanager
    def forward_batch(self, batch: Batch):
        assert self._batch is None, "Nested forward_batch is not allowed"
        try:
            self._batch = batch
            yield
        finally:
            self._batch = None


_GLOBAL_CTX: Optional[Context] = None


def set_global_ctx(ctx: Optional[Context]) -> None:
    global _GLOBAL_CTX
    _GLOBAL_CTX = ctx


def get_global_ctx() -> Context:
    assert _GLOBAL_CTX is not None, "Global context is not set"
    return _GLOBAL_CTX


@dataclass(frozen=True)
class ModelConfig:
    """The attention-shape subset of models/config.py:18-35 the backend reads."""

    num_qo_heads: int
    num_kv_heads: int
    head_dim: int
    num_layers: int = 1


@dataclass(frozen=True)
class RotaryConfig:
    """models/config.py:9-15: rotary_dim = head_dim * partial_rotary_factor, rope_theta, rope_scaling."""

    head_dim: int
    rotary_dim: int
    base: float
    max_position: int = 4096
    scaling: Optional[dict] = None
