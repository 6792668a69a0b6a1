"""``hip`` attention backend: gfx950 kernels behind the reference's backend interface.

Decode metadata is the CSR form of attention/metal.py:145-152
(kv_indptr [B+1], kv_indices [sum L] token slots), built with numpy from the
host page table and copied to the device once per step; every layer then
runs one paged-decode launch (plus the split-K merge) over its own pool, with
the step's KV store performed inside the decode launch.
Prefill metadata mirrors attention/base.py:70-83 and additionally carries the
packed ragged description (q_indptr, kv_indptr, kv_indices, seq_lens) that
the ragged prefill kernel reads in one launch instead of a per-request loop.

Each step's index tensors are fresh device tensors, so a step that is still
running on the stream never sees the next step's indices (the overlap loop of
scheduler/scheduler.py:88-118 prepares step t+1 while step t runs).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import TYPE_CHECKING, Optional

import numpy as np
import torch

from .. import ops
from .base import BaseAttnBackend, PrefillMetadata

if TYPE_CHECKING:
    from minisgl_hip.core import Batch


def _to_device(x: np.ndarray, device: torch.device) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.int32))
    if device.type == "cuda":
        return t.pin_memory().to(device, non_blocking=True)
    return t.to(device)


@dataclass
class HipDecodeMetadata:
    kv_indptr: torch.Tensor  # [B+1] int32, device
    kv_indices: torch.Tensor  # [sum L] int32, device
    max_seq_len: int
    max_splits: int
    workspace: torch.Tensor  # this step's: the decode work list (planned once) and split-K partials


@dataclass
class HipPrefillDevice:
    q_indptr: torch.Tensor  # [R+1]
    kv_indptr: torch.Tensor  # [R+1]
    kv_indices: torch.Tensor  # [sum (P+E)] token slots
    seq_lens: torch.Tensor  # [R]
    max_extend_len: int
    num_tokens: int
    max_seq_len: int
    max_splits: int
    workspace: Optional[torch.Tensor] = None  # this step's work list (planned once) and split-K partials


class HipAttnBackend(BaseAttnBackend):
    """``fuse_decode_store``: during decode steps the pool defers ``store_kv`` and
    ``forward_decode`` performs it inside the decode launch (one kernel instead of
    two per layer); results and pool contents are identical to the eager order."""

    # every key and value is read from the pool (prefill included), never from the k/v arguments
    reads_kv_from_pool = True

    def __init__(self, config, kv_cache, page_table: np.ndarray, fuse_decode_store: bool = True) -> None:
        super().__init__(config, kv_cache, page_table)
        self.device = kv_cache.k[0].device
        # (an fp8 pool's deferred store quantises inside the fp8 decode launch)
        self.fuse_decode_store = fuse_decode_store and hasattr(kv_cache, "take_pending")

    def prepare_metadata(self, batch: "Batch") -> None:
        if self.fuse_decode_store:
            self.kv_cache.flush()
            self.kv_cache.defer_stores = batch.is_decode
        super().prepare_metadata(batch)

    def _kv_scale(self, layer_id: int) -> Optional[torch.Tensor]:
        """fp8 pools: the layer's (K, V) scales; None for unquantised pools."""
        return self.kv_cache.kv_scale[layer_id] if getattr(self.kv_cache, "quantized", False) else None

    # ------------------------------------------------------------------ decode

    def prepare_decode(self, batch: "Batch") -> HipDecodeMetadata:
        """attention/metal.py:145-152 (CSR over token slots), then one H2D copy."""
        lens = np.array([r.device_len for r in batch.reqs])
        rows = np.array([r.table_idx for r in batch.reqs])
        max_len = int(lens.max())
        valid = np.arange(max_len)[None, :] < lens[:, None]
        kv_indices = self.page_table[rows, :max_len][valid]
        kv_indptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        cfg = self.config
        b = len(lens)
        splits = ops.default_splits(b, cfg.num_kv_heads, max_len)
        indptr_dev = _to_device(kv_indptr, self.device)
        # a workspace per step, so a step prepared while the previous one still
        # runs (scheduler/scheduler.py:88-118) never touches the running step's plan
        ws = torch.empty(ops.decode_workspace_bytes(b, cfg.num_qo_heads, cfg.num_kv_heads, cfg.head_dim, splits),
                         dtype=torch.uint8, device=self.device)
        ops.paged_decode_plan(indptr_dev, None, b, cfg.num_qo_heads, cfg.num_kv_heads, cfg.head_dim, splits, ws)
        return HipDecodeMetadata(
            kv_indptr=indptr_dev,
            kv_indices=_to_device(kv_indices, self.device),
            max_seq_len=max_len,
            max_splits=splits,
            workspace=ws,
        )

    def forward_decode(self, q: torch.Tensor, layer_id: int, meta: HipDecodeMetadata) -> torch.Tensor:
        ws = meta.workspace
        pending = self.kv_cache.take_pending(layer_id) if self.fuse_decode_store else None
        if pending is not None and pending[0].shape[0] != q.shape[0]:
            self.kv_cache.store_now(*pending, layer_id)  # not one new token per request: store eagerly
            pending = None
        return ops.paged_decode_attention(
            q,
            self.kv_cache.k[layer_id] if pending is not None else self.kv_cache.k_cache(layer_id),
            self.kv_cache.v[layer_id] if pending is not None else self.kv_cache.v_cache(layer_id),
            meta.kv_indptr,
            meta.kv_indices,
            self.scale,
            max_splits=meta.max_splits,
            workspace=ws,
            new_kv=pending,
            planned=True,
            kv_scale=self._kv_scale(layer_id),
        )

    # ------------------------------------------------------------------ prefill

    def _prepare_prefill(self, batch: "Batch") -> PrefillMetadata:
        """attention/base.py:70-83, plus the packed ragged form for one kernel launch."""
        extend_lens = [r.extend_len for r in batch.reqs]
        q_offsets = np.concatenate([[0], np.cumsum(extend_lens)]).tolist()
        kv_indices = []
        flat = []
        for req in batch.reqs:
            row = self.page_table[req.table_idx, : req.device_len]
            kv_indices.append(None if req.cached_len == 0 else row.copy())
            flat.append(row)
        seq_lens = np.array([r.device_len for r in batch.reqs], dtype=np.int32)
        dev = HipPrefillDevice(
            q_indptr=_to_device(np.asarray(q_offsets, dtype=np.int32), self.device),
            kv_indptr=_to_device(np.concatenate([[0], np.cumsum(seq_lens)]).astype(np.int32), self.device),
            kv_indices=_to_device(np.concatenate(flat), self.device),
            seq_lens=_to_device(seq_lens, self.device),
            max_extend_len=int(max(extend_lens)),
            num_tokens=int(q_offsets[-1]),
            max_seq_len=int(seq_lens.max()),
            max_splits=1,
        )
        cfg = self.config
        if self.kv_cache.dtype != torch.float32:  # fp32 runs one pass per query block, with no work list
            r = len(batch.reqs)
            dev.max_splits = ops.prefill_default_splits(
                r, cfg.num_qo_heads, cfg.num_kv_heads, cfg.head_dim, dev.max_extend_len, dev.max_seq_len
            )
            # a workspace per step (see prepare_decode); the work list is built once for all layers
            dev.workspace = torch.empty(
                ops.prefill_workspace_bytes(r, dev.num_tokens, dev.max_extend_len, cfg.num_qo_heads,
                                            cfg.num_kv_heads, cfg.head_dim, dev.max_splits),
                dtype=torch.uint8, device=self.device)
            ops.prefill_plan(dev.q_indptr, dev.kv_indptr, dev.seq_lens, num_tokens=dev.num_tokens,
                             max_extend_len=dev.max_extend_len, max_seq_len=dev.max_seq_len,
                             num_qo_heads=cfg.num_qo_heads, num_kv_heads=cfg.num_kv_heads, head_dim=cfg.head_dim,
                             dtype=self.kv_cache.dtype, max_splits=dev.max_splits, workspace=dev.workspace)
        return PrefillMetadata(
            last_indices=_to_device(np.array(q_offsets[1:], dtype=np.int32) - 1, self.device),
            q_offsets=q_offsets,
            kv_indices=kv_indices,
            device=dev,
        )

    def _forward_prefill(self, q, k, v, layer_id: int, meta: PrefillMetadata) -> torch.Tensor:
        d = meta.device
        return ops.prefill_ragged_attention(
            q,
            self.kv_cache.k_cache(layer_id),
            self.kv_cache.v_cache(layer_id),
            d.q_indptr,
            d.kv_indptr,
            d.kv_indices,
            d.seq_lens,
            self.scale,
            max_extend_len=d.max_extend_len,
            max_seq_len=d.max_seq_len,
            max_splits=d.max_splits,
            workspace=d.workspace,
            planned=d.workspace is not None,
            kv_scale=self._kv_scale(layer_id),
        )
