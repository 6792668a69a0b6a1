"""Paged KV pool on the GPU (counterpart of kvcache/pool.py:24-54).

    k[layer] : [num_tokens, num_kv_heads, head_dim]
    v[layer] : [num_tokens, num_kv_heads, head_dim]

A slot is an index along dim 0. One K and one V buffer per layer, zero
initialised, in the model dtype (kvcache/pool.py:25-39). ``store_kv`` writes
this step's rows with the HIP scatter kernel, in place.
"""

from __future__ import annotations

from typing import List

import torch

from .. import ops


class MHAKVCache:
    def __init__(
        self,
        num_layers: int,
        num_tokens: int,
        num_kv_heads: int,
        head_dim: int,
        dtype: torch.dtype,
        device: torch.device | str = "cuda",
    ) -> None:
        shape = (num_tokens, num_kv_heads, head_dim)
        self.k: List[torch.Tensor] = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(num_layers)]
        self.v: List[torch.Tensor] = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(num_layers)]
        self.num_layers = num_layers
        self.num_tokens = num_tokens
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype

    def k_cache(self, layer_id: int) -> torch.Tensor:
        return self.k[layer_id]

    def v_cache(self, layer_id: int) -> torch.Tensor:
        return self.v[layer_id]

    def store_kv(self, k: torch.Tensor, v: torch.Tensor, out_loc: torch.Tensor, layer_id: int) -> None:
        """kvcache/pool.py:47-50: write this step's k/v ([T, Hkv, D]) to slots out_loc ([T])."""
        ops.store_kv(k, v, out_loc, self.k[layer_id], self.v[layer_id])

    @property
    def nbytes(self) -> int:
        return 2 * self.num_layers * self.k[0].numel() * self.k[0].element_size()
