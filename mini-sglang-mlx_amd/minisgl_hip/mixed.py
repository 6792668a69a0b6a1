"""One continuous-batching step with decode and prefill requests in one packed batch.

The reference never mixes phases in a batch (core.py:102, attention/base.py:49-60
dispatch on batch.phase); this runner executes both on one stream so a
scheduler that does mix them pays one metadata build per step:

1. ``msgl_build_step_indices`` from the device page table (positions,
   out_loc, q offsets and the page-level CSR for every request), the GPU form
   of scheduler/scheduler.py:154-157 and attention/metal.py:145-152;
2. the prefill requests' KV store (kvcache/pool.py:47-50);
3. paged decode over the decode requests with their KV store fused in;
4. ragged prefill over the prefill chunks (attention/base.py:85-105).

Decode requests come first in the packed batch (one token each), prefill
requests after them; q and out are the packed [T, Hq, D] tensors. Per request
the results are those of the reference's decode or prefill path.

Steps 3 and 4 touch disjoint output rows and pool rows no other part writes.
With ``single_launch`` (the default) they are one launch (``msgl_mixed_attention``: one grid
whose workgroups take decode and prefill work items in proportion, after the
two work-list plans), plus one merge launch; with ``concurrent`` (and no single
launch) the prefill runs on a second stream of default priority, forked after
step 2 and joined before ``run`` returns. Either way the HBM-bound decode and
the matrix-core-bound prefill share the GPU instead of running one after the
other. The two-stream form runs the same launches as running the phases in
turn, so its results are bit-identical to them. The single launch is
bit-identical to them too while the decode phase splits requests into chunks.
With one split the separate decode call runs its shared-head form, and for
long-context batches it splits by equal key ranges; then the two agree to fp32
rounding.
"""

from __future__ import annotations

from typing import Optional

import numpy as np
import torch

from . import ops


class MixedStep:
    """Device copies of a step's per-request arrays plus reusable workspaces.

    ``table_idx``, ``cached_len`` and ``device_len`` are the scheduler's host
    arrays (one entry per request, decode requests first); the output sizes of
    the index build (tokens, index entries, longest chunk and sequence) are
    derived from them, so they always fit the indices the GPU builds."""

    def __init__(
        self,
        req_to_token: torch.Tensor,
        table_idx,
        cached_len,
        device_len,
        *,
        num_decode: int,
        num_qo_heads: int,
        num_kv_heads: int,
        head_dim: int,
        page_size: int,
        decode_splits: Optional[int] = None,
        prefill_splits: Optional[int] = None,
    ) -> None:
        dev = req_to_token.device
        table_idx = np.asarray(table_idx, dtype=np.int32)
        cached = np.asarray(cached_len, dtype=np.int32)
        lens = np.asarray(device_len, dtype=np.int32)
        if not (table_idx.shape == cached.shape == lens.shape) or table_idx.ndim != 1:
            raise ValueError("table_idx, cached_len and device_len must be [R] host arrays")
        ext = lens.astype(np.int64) - cached
        if (ext < 1).any() or (cached < 0).any():
            raise ValueError("every request must extend by at least one token")
        if not 0 <= num_decode <= len(lens) or (ext[:num_decode] != 1).any():
            raise ValueError("the first num_decode requests must extend by exactly one token")
        self.req_to_token = req_to_token
        self.table_idx = torch.from_numpy(table_idx).to(dev)
        self.cached_len = torch.from_numpy(cached).to(dev)
        self.device_len = torch.from_numpy(lens).to(dev)
        self.num_decode = num_decode
        self.num_tokens = int(ext.sum())
        self.num_pages = int(((lens.astype(np.int64) + page_size - 1) // page_size).sum())
        self.max_chunk = int(ext[num_decode:].max()) if num_decode < len(lens) else 0
        self.max_seq_len = int(lens.max())
        self.page_size = page_size
        self._host_lens = (cached, lens)
        num_reqs = len(lens)
        num_prefill = num_reqs - num_decode
        max_seq_len = self.max_seq_len
        max_chunk = self.max_chunk
        num_tokens = self.num_tokens
        if decode_splits is None:
            decode_splits = ops.default_splits(max(num_decode, 1), num_kv_heads, max_seq_len)
        if prefill_splits is None:
            prefill_splits = (
                ops.prefill_default_splits(num_prefill, num_qo_heads, num_kv_heads, head_dim, max_chunk, max_seq_len)
                if num_prefill
                else 1
            )
        self.decode_splits = decode_splits
        self.prefill_splits = prefill_splits
        self.decode_ws = ops.decode_workspace(max(num_decode, 1), num_qo_heads, num_kv_heads, head_dim,
                                              decode_splits, dev)
        self.prefill_ws = (
            ops.prefill_workspace(num_prefill, num_tokens, max_chunk, num_qo_heads, num_kv_heads, head_dim,
                                  prefill_splits, dev)
            if num_prefill
            else None
        )
        self.indices: Optional[dict] = None
        self._side: Optional[torch.cuda.Stream] = None

    def build_indices(self) -> dict:
        self.indices = ops.build_step_indices(
            self.req_to_token, self.table_idx, self.cached_len, self.device_len,
            num_tokens=self.num_tokens, num_kv=self.num_pages, page_size=self.page_size, host_lens=self._host_lens,
        )
        return self.indices

    def run(self, q, k_new, v_new, k_pool, v_pool, out, scale: float, concurrent: bool = True,
            single_launch: bool = True) -> torch.Tensor:
        """q, k_new, v_new, out: packed [T, H, D]; the pools are one layer's.

        ``single_launch`` (default): decode and prefill in one launch; otherwise
        two streams (``concurrent``) or one after the other."""
        idx = self.build_indices()
        nd = self.num_decode
        has_prefill = self.num_tokens > nd
        if has_prefill:
            ops.store_kv(k_new[nd:], v_new[nd:], idx["out_loc"][nd:], k_pool, v_pool)
        if single_launch and has_prefill and nd:
            return self._run_single(idx, q, k_new, v_new, k_pool, v_pool, out, scale)

        def prefill():
            ops.prefill_ragged_attention(
                q, k_pool, v_pool, idx["q_indptr"][nd:], idx["kv_indptr"][nd:], idx["kv_indices"],
                self.device_len[nd:], scale, max_extend_len=self.max_chunk, max_seq_len=self.max_seq_len,
                page_size=self.page_size, max_splits=self.prefill_splits, out=out, workspace=self.prefill_ws,
            )

        joined = None
        if has_prefill and nd and concurrent:
            main = torch.cuda.current_stream(q.device)
            if self._side is None:
                self._side = torch.cuda.Stream(device=q.device)  # default priority
            side = self._side
            side.wait_stream(main)  # indices and the prefill rows' store are done
            with torch.cuda.stream(side):
                prefill()
            for t in idx.values():  # this step's index tensors now also live on the side stream
                t.record_stream(side)
            joined = side
        elif has_prefill and not nd:
            prefill()
        if nd:
            ops.paged_decode_attention(
                q[:nd], k_pool, v_pool, idx["kv_indptr"][: nd + 1], idx["kv_indices"], scale,
                seq_lens=self.device_len[:nd], page_size=self.page_size, max_splits=self.decode_splits,
                out=out[:nd], workspace=self.decode_ws, new_kv=(k_new[:nd], v_new[:nd], idx["out_loc"][:nd]),
            )
        if joined is not None:
            torch.cuda.current_stream(q.device).wait_stream(joined)
        elif has_prefill and nd:
            prefill()
        return out

    def _run_single(self, idx, q, k_new, v_new, k_pool, v_pool, out, scale: float) -> torch.Tensor:
        """Both plans, then the decode and the prefill in one launch (``ops.mixed_attention``)."""
        nd = self.num_decode
        t, hq, d = q.shape
        hkv = k_pool.shape[1]
        ops.paged_decode_plan(idx["kv_indptr"][: nd + 1], self.device_len[:nd], nd, hq, hkv, d, self.decode_splits,
                              self.decode_ws)
        ops.prefill_plan(idx["q_indptr"][nd:], idx["kv_indptr"][nd:], self.device_len[nd:], num_tokens=t,
                         max_extend_len=self.max_chunk, max_seq_len=self.max_seq_len, num_qo_heads=hq,
                         num_kv_heads=hkv, head_dim=d, dtype=q.dtype, max_splits=self.prefill_splits,
                         workspace=self.prefill_ws)
        return ops.mixed_attention(
            q, k_pool, v_pool, scale, num_decode=nd, dec_kv_indptr=idx["kv_indptr"][: nd + 1],
            dec_kv_indices=idx["kv_indices"], dec_seq_lens=self.device_len[:nd], dec_max_splits=self.decode_splits,
            dec_workspace=self.decode_ws, new_kv=(k_new[:nd], v_new[:nd], idx["out_loc"][:nd]),
            q_indptr=idx["q_indptr"][nd:], pf_kv_indptr=idx["kv_indptr"][nd:], pf_kv_indices=idx["kv_indices"],
            pf_seq_lens=self.device_len[nd:], max_extend_len=self.max_chunk, max_seq_len=self.max_seq_len,
            pf_max_splits=self.prefill_splits, pf_workspace=self.prefill_ws, page_size=self.page_size, out=out,
        )
