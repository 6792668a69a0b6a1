"""RoPE and the attention layer's KV-cache side (counterpart of layers.py:19-111).

``RotaryEmbedding`` keeps the reference's constructor (a rotary config with
``rotary_dim``, ``base`` and optional ``scaling`` of type default / linear /
llama3, layers.py:30-44) and call signature ``(x [T, H, D], positions [T])``,
and runs the HIP rotate-half kernel. ``AttentionLayer.__call__`` performs the
reference's order -- rotate q and k, store rotated k and raw v at
``batch.out_loc``, run the backend -- with the first two steps in one launch
(``msgl_rope_store_kv``).
"""

from __future__ import annotations

import math
from typing import Any, Dict, Optional

import torch

from . import ops
from .core import RotaryConfig, get_global_ctx


def rope_inv_freq(rotary_dim: int, base: float, scaling: Optional[Dict[str, Any]] = None) -> torch.Tensor:
    """Angular frequency of each rotated pair as float32 [rotary_dim / 2], position scale folded in.

    default: base^(-2i/dims); linear: positions times 1/factor (layers.py:37-38);
    llama3: the reciprocal of the smoothed periods of layers.py:59-74."""
    rope_type = "default"
    if scaling:
        rope_type = scaling.get("rope_type", scaling.get("type", "default"))
    exponent = torch.arange(0, rotary_dim, 2, dtype=torch.float64) / rotary_dim
    period = torch.pow(torch.tensor(float(base), dtype=torch.float64), exponent)
    pos_scale = 1.0
    if rope_type == "linear":
        pos_scale = 1.0 / float(scaling["factor"])
    elif rope_type == "llama3":
        factor = float(scaling["factor"])
        low, high = float(scaling.get("low_freq_factor", 1.0)), float(scaling.get("high_freq_factor", 4.0))
        context = float(scaling.get("original_max_position_embeddings", 8192))
        wavelength = 2.0 * math.pi * period
        long_wave = wavelength > context / low
        band = (wavelength > context / high) & (wavelength < context / low)
        blend = (context / wavelength - low) / (high - low)
        period = torch.where(long_wave, period * factor, period)
        period = torch.where(band, period / ((1.0 - blend) / factor + blend), period)
    elif rope_type != "default":
        raise NotImplementedError(f"rope_scaling type {rope_type!r} is not supported yet")
    return (pos_scale / period).to(torch.float32)


class RotaryEmbedding:
    """layers.py:19-56: rotate-half RoPE with one position per packed token."""

    def __init__(self, config: RotaryConfig, device: torch.device | str = "cuda") -> None:
        self.dims = config.rotary_dim
        self.inv_freq = rope_inv_freq(config.rotary_dim, config.base, config.scaling).to(device)

    def __call__(self, x: torch.Tensor, positions: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        return ops.rope(x, positions, self.inv_freq, self.dims, out=out)


class AttentionLayer:
    """layers.py:77-111: the stateless part of one attention layer.

    q [T, Hq, D], k/v [T, Hkv, D] -> o [T, Hq * D]. Metadata (positions, out_loc,
    attn_metadata) comes from the global context, as in the reference."""

    def __init__(self, layer_id: int, num_qo_heads: int, num_kv_heads: int, head_dim: int,
                 rotary_config: RotaryConfig, device: torch.device | str = "cuda") -> None:
        assert num_qo_heads % num_kv_heads == 0
        self.layer_id = layer_id
        self.num_qo_heads = num_qo_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.rotary = RotaryEmbedding(rotary_config, device)

    def __call__(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        ctx = get_global_ctx()
        batch = ctx.batch
        backend = ctx.attn_backend
        # a backend that reads every key from the pool never sees the rotated k tensor
        k_rot = None if getattr(backend, "reads_kv_from_pool", False) else torch.empty_like(k)
        q = ctx.kv_cache.rope_store_kv(q, k, v, batch.positions, batch.out_loc, self.layer_id, self.rotary,
                                       k_out=k_rot)
        o = backend.forward(q, k if k_rot is None else k_rot, v, self.layer_id, batch)
        return o.reshape(o.shape[0], self.num_qo_heads * self.head_dim)
