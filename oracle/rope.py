"""numpy restatement of the reference's rotary embedding (oracle; test infrastructure only).

Follows ``layers.py:19-74`` of the reference's ``python/minisgl_mlx/``:
``RotaryEmbedding.__call__`` runs ``mx.fast.rope(x.reshape(T, H, 1, D), dims,
traditional=False, base, scale, offset=positions, freqs)``, i.e. every token
is its own length-1 sequence rotated at its own position, in the "rotate
half" layout: element i < dims/2 pairs with element i + dims/2, elements
>= dims pass through unchanged. ``layers.py:107-109`` then rotates q and k
(not v) and stores k, v into the pool.

Angles: theta[t, i] = positions[t] * inv_freq[i] is formed as one float32
product (the rotation kernels compute in float32, as mx.fast.rope does);
cos/sin of that float32 angle and the rotation are then evaluated in float64.
"""

from __future__ import annotations

from typing import Any, Dict, Optional

import numpy as np


def rope_periods(rotary_dim: int, base: float, scaling: Optional[Dict[str, Any]] = None) -> np.ndarray:
    """Per-pair periods (positions per radian) in float64, ``layers.py:30-44, 59-74``.

    default / linear: base ** (2i / dims); llama3: ``_llama3_freqs`` (periods
    multiplied by ``factor`` for long wavelengths, smoothly interpolated in
    the medium band)."""
    i2 = np.arange(0, rotary_dim, 2, dtype=np.float64)
    periods = float(base) ** (i2 / rotary_dim)
    rope_type = "default"
    if scaling:
        rope_type = scaling.get("rope_type", scaling.get("type", "default"))
    if rope_type == "llama3":
        factor = float(scaling["factor"])
        lo_ff = float(scaling.get("low_freq_factor", 1.0))
        hi_ff = float(scaling.get("high_freq_factor", 4.0))
        old_len = float(scaling.get("original_max_position_embeddings", 8192))
        lo_wl, hi_wl = old_len / lo_ff, old_len / hi_ff
        wavelens = 2.0 * np.pi * periods
        scaled = np.where(wavelens > lo_wl, periods * factor, periods)
        medium = (wavelens > hi_wl) & (wavelens < lo_wl)
        smooth = (old_len / wavelens - lo_ff) / (hi_ff - lo_ff)
        return np.where(medium, scaled / ((1.0 - smooth) / factor + smooth), scaled)
    if rope_type not in ("default", "linear"):
        raise NotImplementedError(f"rope_scaling type {rope_type!r} is not supported")
    return periods


def rope_position_scale(scaling: Optional[Dict[str, Any]] = None) -> float:
    """``layers.py:37-38``: linear scaling multiplies positions by 1/factor."""
    if scaling and scaling.get("rope_type", scaling.get("type", "default")) == "linear":
        return 1.0 / float(scaling["factor"])
    return 1.0


def rope_inv_freq(rotary_dim: int, base: float, scaling: Optional[Dict[str, Any]] = None) -> np.ndarray:
    """Angular frequency per pair, position scale folded in, rounded to float32."""
    return (rope_position_scale(scaling) / rope_periods(rotary_dim, base, scaling)).astype(np.float32)


def rope_angles(positions, inv_freq: np.ndarray) -> np.ndarray:
    """[T, dims/2] float32 angles: one float32 product per element."""
    pos = np.asarray(positions).astype(np.float32)
    return pos[:, None] * np.asarray(inv_freq, dtype=np.float32)[None, :]


def rope(x: np.ndarray, positions, rotary_dim: int, inv_freq: np.ndarray) -> np.ndarray:
    """x: [T, H, D] -> float64 [T, H, D], rotate-half RoPE over the first rotary_dim elements."""
    x = np.asarray(x, dtype=np.float64)
    half = rotary_dim // 2
    theta = rope_angles(positions, inv_freq).astype(np.float64)[:, None, :]  # [T, 1, half]
    c, s = np.cos(theta), np.sin(theta)
    out = x.copy()
    lo, hi = x[..., :half], x[..., half:rotary_dim]
    out[..., :half] = lo * c - hi * s
    out[..., half:rotary_dim] = lo * s + hi * c
    return out


def rope_store_kv(q, k, v, positions, out_loc, k_pool: np.ndarray, v_pool: np.ndarray, rotary_dim: int,
                  inv_freq: np.ndarray):
    """``layers.py:107-109``: rotate q and k, store rotated k and raw v at out_loc.

    The pools keep their dtype (rotated k is rounded to it on store, as the
    pool write does); returns (q_rot, k_rot) in float64."""
    q_rot = rope(q, positions, rotary_dim, inv_freq)
    k_rot = rope(k, positions, rotary_dim, inv_freq)
    loc = np.asarray(out_loc, dtype=np.int64)
    k_pool[loc] = k_rot.astype(k_pool.dtype)
    v_pool[loc] = np.asarray(v).astype(v_pool.dtype)
    return q_rot, k_rot
