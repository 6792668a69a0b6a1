"""Paged KV pool on the GPU (counterpart of kvcache/pool.py:24-54).

    k[layer] : [num_tokens, num_kv_heads, head_dim]
    v[layer] : [num_tokens, num_kv_heads, head_dim]

A slot is an index along dim 0. One K and one V buffer per layer, zero
initialised, in the model dtype (kvcache/pool.py:25-39). ``store_kv`` writes
this step's rows with the HIP scatter kernel, in place.

Deferred stores: with ``defer_stores`` set (the hip backend sets it for decode
steps), ``store_kv`` only records the rows; the backend then performs the
store inside its decode launch (``take_pending``). Any other read of that
layer's pool (``k_cache``/``v_cache``) first performs the recorded store, so
every reader still observes the pool exactly as after an eager store.

fp8 pools (``kv_dtype=torch.float8_e4m3fn``, the extension docs/09-exercises.md:81-82
describes): ``k``/``v`` hold e4m3 codes and ``kv_scale[layer]`` [num_tokens,
num_kv_heads, 2] the K and V scale of each slot and head; a store quantises
(a deferred one inside the fp8 decode launch, with the same arithmetic),
``dtype`` stays the model's (q/k/v) type.
"""

from __future__ import annotations

from typing import List, Optional, Tuple

import torch

from .. import ops

PendingStore = Tuple[torch.Tensor, torch.Tensor, torch.Tensor]  # (k, v, out_loc)


class MHAKVCache:
    def __init__(
        self,
        num_layers: int,
        num_tokens: int,
        num_kv_heads: int,
        head_dim: int,
        dtype: torch.dtype,
        device: torch.device | str = "cuda",
        kv_dtype: Optional[torch.dtype] = None,
    ) -> None:
        shape = (num_tokens, num_kv_heads, head_dim)
        kv_dtype = dtype if kv_dtype is None else kv_dtype
        if kv_dtype not in (dtype, torch.float8_e4m3fn):
            raise ValueError("kv_dtype must be the model dtype or torch.float8_e4m3fn")
        self.quantized = kv_dtype == torch.float8_e4m3fn
        self.k: List[torch.Tensor] = [torch.zeros(shape, dtype=kv_dtype, device=device) for _ in range(num_layers)]
        self.v: List[torch.Tensor] = [torch.zeros(shape, dtype=kv_dtype, device=device) for _ in range(num_layers)]
        self.kv_scale: List[Optional[torch.Tensor]] = [
            torch.zeros((num_tokens, num_kv_heads, 2), dtype=torch.float32, device=device) if self.quantized else None
            for _ in range(num_layers)
        ]
        self.num_layers = num_layers
        self.num_tokens = num_tokens
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.defer_stores = False
        self._pending: List[Optional[PendingStore]] = [None] * num_layers

    def k_cache(self, layer_id: int) -> torch.Tensor:
        self.flush(layer_id)
        return self.k[layer_id]

    def v_cache(self, layer_id: int) -> torch.Tensor:
        self.flush(layer_id)
        return self.v[layer_id]

    def store_kv(self, k: torch.Tensor, v: torch.Tensor, out_loc: torch.Tensor, layer_id: int) -> None:
        """kvcache/pool.py:47-50: write this step's k/v ([T, Hkv, D]) to slots out_loc ([T])."""
        if self.defer_stores:
            self.flush(layer_id)
            self._pending[layer_id] = (k, v, out_loc)
        else:
            self.store_now(k, v, out_loc, layer_id)

    def store_now(self, k: torch.Tensor, v: torch.Tensor, out_loc: torch.Tensor, layer_id: int) -> None:
        """The store itself (quantising for fp8 pools), whatever ``defer_stores`` says."""
        if self.quantized:
            ops.store_kv_fp8(k, v, out_loc, self.k[layer_id], self.v[layer_id], self.kv_scale[layer_id])
        else:
            ops.store_kv(k, v, out_loc, self.k[layer_id], self.v[layer_id])

    def rope_store_kv(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, positions: torch.Tensor,
                      out_loc: torch.Tensor, layer_id: int, rotary, k_out: Optional[torch.Tensor] = None,
                      q_out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """layers.py:107-109 fused: rotate q and k, store rotated k and raw v; returns rotated q.

        ``rotary`` carries ``inv_freq`` and ``dims`` (a ``layers.RotaryEmbedding``).
        Unquantised pools: the store happens now, whatever ``defer_stores`` says.
        fp8 pools: rotate, then the quantising store (deferred like ``store_kv``)."""
        self.flush(layer_id)
        if self.quantized:
            q_rot = ops.rope(q, positions, rotary.inv_freq, rotary.dims, out=q_out)
            k_rot = ops.rope(k, positions, rotary.inv_freq, rotary.dims, out=k_out)
            self.store_kv(k_rot, v, out_loc, layer_id)
            return q_rot
        return ops.rope_store_kv(q, k, v, positions, out_loc, self.k[layer_id], self.v[layer_id], rotary.inv_freq,
                                 rotary.dims, q_out=q_out, k_out=k_out)

    def take_pending(self, layer_id: int) -> Optional[PendingStore]:
        """Hand a recorded store to the caller, who becomes responsible for performing it."""
        pending, self._pending[layer_id] = self._pending[layer_id], None
        return pending

    def flush(self, layer_id: Optional[int] = None) -> None:
        """Perform recorded stores (of one layer, or of all layers)."""
        layers = range(self.num_layers) if layer_id is None else (layer_id,)
        for i in layers:
            pending = self.take_pending(i)
            if pending is not None:
                self.store_now(*pending, i)

    @property
    def nbytes(self) -> int:
        scales = self.kv_scale[0].numel() * 4 if self.quantized else 0
        return self.num_layers * (2 * self.k[0].numel() * self.k[0].element_size() + scales)
