"""``hip`` attention backend: gfx950 kernels behind the reference's backend interface.

Step metadata is built on the GPU. The backend keeps a device mirror of the
scheduler's token-granular page table (``page_table``, written on the host by
scheduler/cache.py:53-72) and brings it up to date once per step with one
small host-to-device copy of the entries written since the last step (a
prefill step sends its requests' rows in full, a decode step one slot per
request); ``msgl_build_step_indices`` then writes the step's CSR
(attention/metal.py:145-152: kv_indptr [B+1], kv_indices token slots) and the
prefill offsets (attention/base.py:70-83) from that table, so the per-step
index lists never cross PCIe. Every layer then runs one paged-decode launch
(plus the split-K merge) over its own pool, with the step's KV store
performed inside the decode launch, or one ragged-prefill launch.

A ``"mixed"`` batch (decode requests first, one new token each, then prefill
chunks) runs both phases of a continuous-batching step in one launch per
layer (``msgl_mixed_attention``), the HybridBackend the reference's
docs/04-attention.md:15 describes; per request the results are those of the
decode or prefill path.

Each step's index tensors and workspaces are fresh device tensors, so a step
that is still running on the stream never sees the next step's indices (the
overlap loop of scheduler/scheduler.py:88-118 prepares step t+1 while step t
runs).

``validate`` (default: environment ``MSGL_VALIDATE_METADATA=1``) checks every
step's indices on the device before use (``ops.validate_metadata``; one host
sync per step) and raises ``ValueError`` on metadata the kernels would read
outside the pool or the index arrays.
"""

from __future__ import annotations

import os
from dataclasses import dataclass
from typing import TYPE_CHECKING, List, Optional

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
    seq_lens: Optional[torch.Tensor]  # [R], or None: L_i = kv_indptr[i+1] - kv_indptr[i]
    max_extend_len: int
    num_tokens: int
    max_seq_len: int
    max_splits: int
    workspace: Optional[torch.Tensor] = None  # this step's work list (planned once) and split-K partials


@dataclass
class HipMixedMetadata:
    """A mixed batch: requests [0, num_decode) decode (one token each), the rest prefill."""

    num_decode: int
    decode: HipDecodeMetadata  # over kv_indptr[: num_decode + 1]
    prefill: HipPrefillDevice  # over q_indptr[num_decode:], kv_indptr[num_decode:]
    last_indices: torch.Tensor  # [R] packed index of each request's last token


class HipAttnBackend(BaseAttnBackend):
    """``fuse_decode_store``: during decode (and mixed) steps the pool defers
    ``store_kv`` and the decode launch performs the store of the decode rows
    (one kernel instead of two per layer); results and pool contents are
    identical to the eager order."""

    # every key and value is read from the pool (prefill included), never from the k/v arguments
    reads_kv_from_pool = True

    def __init__(self, config, kv_cache, page_table: np.ndarray, fuse_decode_store: bool = True,
                 validate: Optional[bool] = None) -> None:
        super().__init__(config, kv_cache, page_table)
        self.device = kv_cache.k[0].device
        # (an fp8 pool's deferred store quantises inside the fp8 decode launch)
        self.fuse_decode_store = fuse_decode_store and hasattr(kv_cache, "take_pending")
        self.validate = os.environ.get("MSGL_VALIDATE_METADATA", "0") == "1" if validate is None else validate
        # device mirror of page_table: row r holds valid entries [0, _mirrored[r])
        self.table_dev = torch.zeros(page_table.shape, dtype=torch.int32, device=self.device)
        self._mirrored = np.zeros(page_table.shape[0], dtype=np.int64)

    def prepare_metadata(self, batch: "Batch") -> None:
        if self.fuse_decode_store:
            self.kv_cache.flush()
            self.kv_cache.defer_stores = batch.is_decode or batch.phase == "mixed"
        super().prepare_metadata(batch)

    def _kv_scale(self, layer_id: int) -> Optional[torch.Tensor]:
        """fp8 pools: the layer's (K, V) scales; None for unquantised pools."""
        return self.kv_cache.kv_scale[layer_id] if getattr(self.kv_cache, "quantized", False) else None

    # ------------------------------------------------------------ step indices

    def _step_indices(self, reqs: List, full_rows: np.ndarray) -> dict:
        """Mirror the page-table entries the step reads, then build its indices on
        the GPU. full_rows[i]: request i's row is sent whole (its first step in this
        row); otherwise only the entries past what the device already holds."""
        rows = np.array([r.table_idx for r in reqs], dtype=np.int64)
        cached = np.array([r.cached_len for r in reqs], dtype=np.int64)
        lens = np.array([r.device_len for r in reqs], dtype=np.int64)
        lo = np.where(full_rows, 0, np.minimum(self._mirrored[rows], lens))
        cnt = lens - lo
        n = int(cnt.sum())
        r_idx = np.repeat(rows, cnt)
        c_idx = (np.arange(n) - np.repeat(np.cumsum(cnt) - cnt, cnt) + np.repeat(lo, cnt)).astype(np.int64)
        vals = self.page_table[r_idx, c_idx] if n else np.zeros(0, np.int32)
        b = len(reqs)
        # one host-to-device copy: [table_idx | cached_len | device_len | rows | cols | values]
        packed = _to_device(np.concatenate([rows, cached, lens, r_idx, c_idx, vals]), self.device)
        t_idx, t_cached, t_lens = packed[:b], packed[b: 2 * b], packed[2 * b: 3 * b]
        if n:
            ops.table_scatter(self.table_dev, packed[3 * b: 3 * b + n], packed[3 * b + n: 3 * b + 2 * n],
                              packed[3 * b + 2 * n:])
        self._mirrored[rows] = lens
        num_tokens = int((lens - cached).sum())
        idx = ops.build_step_indices(self.table_dev, t_idx, t_cached, t_lens, num_tokens=num_tokens,
                                     num_kv=int(lens.sum()), page_size=1)
        idx["num_tokens"] = num_tokens
        idx["max_len"] = int(lens.max())
        idx["seq_lens"] = t_lens
        return idx

    def _validate(self, kv_indptr, kv_indices, q_indptr=None, num_tokens=0) -> None:
        if self.validate:
            ops.validate_metadata(kv_indptr, kv_indices, None, num_slots=self.kv_cache.num_tokens,
                                  q_indptr=q_indptr, num_tokens=num_tokens)

    def _decode_meta(self, kv_indptr, kv_indices, lens: np.ndarray) -> HipDecodeMetadata:
        cfg = self.config
        b, max_len = len(lens), int(lens.max())
        if getattr(self.kv_cache, "quantized", False):
            splits = ops.default_splits(b, cfg.num_kv_heads, max_len)
        else:  # near-uniform batches that fill the device: one launch, no merge
            splits = ops.decode_splits_for(lens, cfg.num_kv_heads)
        # a workspace per step, so a step prepared while the previous one still
        # runs (scheduler/scheduler.py:88-118) never touches the running step's plan
        ws = torch.empty(ops.decode_workspace_bytes(b, cfg.num_qo_heads, cfg.num_kv_heads, cfg.head_dim, splits),
                         dtype=torch.uint8, device=self.device)
        ops.paged_decode_plan(kv_indptr, None, b, cfg.num_qo_heads, cfg.num_kv_heads, cfg.head_dim, splits, ws)
        return HipDecodeMetadata(kv_indptr=kv_indptr, kv_indices=kv_indices, max_seq_len=max_len,
                                 max_splits=splits, workspace=ws)

    def _prefill_device(self, q_indptr, kv_indptr, kv_indices, num_reqs: int, num_tokens: int, max_e: int,
                        max_len: int) -> HipPrefillDevice:
        """The ragged description plus, for 16-bit pools, this step's work list."""
        dev = HipPrefillDevice(q_indptr=q_indptr, kv_indptr=kv_indptr, kv_indices=kv_indices, seq_lens=None,
                               max_extend_len=max_e, num_tokens=num_tokens, max_seq_len=max_len, max_splits=1)
        cfg = self.config
        if self.kv_cache.dtype != torch.float32:  # fp32 runs one pass per query block, with no work list
            dev.max_splits = ops.prefill_default_splits(num_reqs, cfg.num_qo_heads, cfg.num_kv_heads, cfg.head_dim,
                                                        max_e, max_len)
            # a workspace per step (see _decode_meta); the work list is built once for all layers
            dev.workspace = torch.empty(
                ops.prefill_workspace_bytes(num_reqs, num_tokens, max_e, cfg.num_qo_heads, cfg.num_kv_heads,
                                            cfg.head_dim, dev.max_splits),
                dtype=torch.uint8, device=self.device)
            ops.prefill_plan(q_indptr, kv_indptr, None, num_tokens=num_tokens, max_extend_len=max_e,
                             max_seq_len=max_len, num_qo_heads=cfg.num_qo_heads, num_kv_heads=cfg.num_kv_heads,
                             head_dim=cfg.head_dim, dtype=self.kv_cache.dtype, max_splits=dev.max_splits,
                             workspace=dev.workspace)
        return dev

    # ------------------------------------------------------------------ decode

    def prepare_decode(self, batch: "Batch") -> HipDecodeMetadata:
        """attention/metal.py:145-152 (CSR over token slots), built on the GPU."""
        reqs = batch.reqs
        idx = self._step_indices(reqs, np.zeros(len(reqs), dtype=bool))
        self._validate(idx["kv_indptr"], idx["kv_indices"])
        return self._decode_meta(idx["kv_indptr"], idx["kv_indices"], np.array([r.device_len for r in reqs]))

    def _pending_store(self, layer_id: int, num_rows: int):
        """The layer's deferred store, or None (stored now if it is not one row per decode request)."""
        pending = self.kv_cache.take_pending(layer_id) if self.fuse_decode_store else None
        if pending is not None and pending[0].shape[0] != num_rows:
            self.kv_cache.store_now(*pending, layer_id)
            pending = None
        return pending

    def _decode(self, q, layer_id: int, meta: HipDecodeMetadata, pending, out=None) -> torch.Tensor:
        return ops.paged_decode_attention(
            q,
            self.kv_cache.k[layer_id] if pending is not None else self.kv_cache.k_cache(layer_id),
            self.kv_cache.v[layer_id] if pending is not None else self.kv_cache.v_cache(layer_id),
            meta.kv_indptr,
            meta.kv_indices,
            self.scale,
            max_splits=meta.max_splits,
            workspace=meta.workspace,
            new_kv=pending,
            planned=True,
            kv_scale=self._kv_scale(layer_id),
            out=out,
        )

    def forward_decode(self, q: torch.Tensor, layer_id: int, meta: HipDecodeMetadata) -> torch.Tensor:
        return self._decode(q, layer_id, meta, self._pending_store(layer_id, q.shape[0]))

    # ------------------------------------------------------------------ prefill

    def _prepare_prefill(self, batch: "Batch") -> PrefillMetadata:
        """attention/base.py:70-83, plus the packed ragged form for one kernel launch."""
        reqs = batch.reqs
        idx = self._step_indices(reqs, np.ones(len(reqs), dtype=bool))
        extend_lens = [r.extend_len for r in reqs]
        q_offsets = np.concatenate([[0], np.cumsum(extend_lens)]).tolist()
        kv_indices = [None if r.cached_len == 0 else self.page_table[r.table_idx, : r.device_len].copy() for r in reqs]
        self._validate(idx["kv_indptr"], idx["kv_indices"], idx["q_indptr"], idx["num_tokens"])
        dev = self._prefill_device(idx["q_indptr"], idx["kv_indptr"], idx["kv_indices"], len(reqs),
                                   idx["num_tokens"], int(max(extend_lens)), idx["max_len"])
        return PrefillMetadata(last_indices=idx["last_indices"], q_offsets=q_offsets, kv_indices=kv_indices,
                               device=dev)

    def _prefill(self, q, layer_id: int, d: HipPrefillDevice, out=None) -> torch.Tensor:
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
            out=out,
        )

    def _forward_prefill(self, q, k, v, layer_id: int, meta: PrefillMetadata) -> torch.Tensor:
        return self._prefill(q, layer_id, meta.device)

    # ------------------------------------------------------------------ mixed

    def prepare_mixed(self, batch: "Batch") -> HipMixedMetadata:
        """A continuous-batching step: the leading requests that extend by one token
        are decode requests, the rest prefill chunks (a one-token chunk after them
        is a prefill of one query, which attends exactly like a decode)."""
        reqs = batch.reqs
        ext = np.array([r.extend_len for r in reqs])
        nd = int(np.argmin(ext == 1)) if (ext != 1).any() else len(reqs)
        full = np.arange(len(reqs)) >= nd  # prefill chunks send their rows whole
        idx = self._step_indices(reqs, full)
        t = idx["num_tokens"]
        self._validate(idx["kv_indptr"], idx["kv_indices"], idx["q_indptr"], t)
        lens = np.array([r.device_len for r in reqs])
        dec = self._decode_meta(idx["kv_indptr"][: nd + 1], idx["kv_indices"], lens[:nd]) if nd else None
        pf = None
        if nd < len(reqs):
            pf = self._prefill_device(idx["q_indptr"][nd:], idx["kv_indptr"][nd:], idx["kv_indices"],
                                      len(reqs) - nd, t, int(ext[nd:].max()), int(lens[nd:].max()))
        return HipMixedMetadata(num_decode=nd, decode=dec, prefill=pf, last_indices=idx["last_indices"])

    def forward_mixed(self, q, k, v, layer_id: int, meta: HipMixedMetadata) -> torch.Tensor:
        nd = meta.num_decode
        pending = self.kv_cache.take_pending(layer_id) if self.fuse_decode_store else None
        new_kv = None
        if pending is not None:
            kn, vn, loc = pending
            if kn.shape[0] != q.shape[0]:
                self.kv_cache.store_now(kn, vn, loc, layer_id)
            else:
                if q.shape[0] > nd:  # the prefill rows are stored now; the decode rows inside the launch
                    self.kv_cache.store_now(kn[nd:], vn[nd:], loc[nd:], layer_id)
                if nd:
                    new_kv = (kn[:nd], vn[:nd], loc[:nd])
        if meta.prefill is None:
            return self._decode(q, layer_id, meta.decode, new_kv)
        if nd == 0:
            return self._prefill(q, layer_id, meta.prefill)
        out = torch.empty_like(q)
        single = q.dtype in (torch.bfloat16, torch.float16) and not getattr(self.kv_cache, "quantized", False)
        if not single:  # fp32 or fp8 pools: the two phases one after the other
            self._decode(q[:nd], layer_id, meta.decode, new_kv, out=out[:nd])
            return self._prefill(q, layer_id, meta.prefill, out=out)
        dm, pm = meta.decode, meta.prefill
        return ops.mixed_attention(
            q, self.kv_cache.k[layer_id], self.kv_cache.v[layer_id], self.scale, num_decode=nd,
            dec_kv_indptr=dm.kv_indptr, dec_kv_indices=dm.kv_indices, dec_seq_lens=None,
            dec_max_splits=dm.max_splits, dec_workspace=dm.workspace, new_kv=new_kv,
            q_indptr=pm.q_indptr, pf_kv_indptr=pm.kv_indptr, pf_kv_indices=pm.kv_indices, pf_seq_lens=None,
            max_extend_len=pm.max_extend_len, max_seq_len=pm.max_seq_len, pf_max_splits=pm.max_splits,
            pf_workspace=pm.workspace, out=out,
        )
