"""Pins for the rotary-embedding oracle (no GPU).

The oracle's rotation is checked against ``transformers``' own rotate-half
RoPE (``LlamaRotaryEmbedding`` + ``apply_rotary_pos_emb``, the layout the
reference selects with ``traditional=False``, layers.py:47-55), its frequency
tables against transformers' default / linear / llama3 initialisers
(layers.py:30-44, 59-74), and against closed forms: position 0 is the
identity, each rotated pair keeps its norm, scores depend only on the
position difference, and a one-hot vector rotates onto (cos, sin). Mutation
tests plant the interleaved layout and a flipped sine in a copy and show the
pins reject them.
"""

import numpy as np
import pytest
import torch

import oracle

transformers = pytest.importorskip("transformers")
from transformers import LlamaConfig  # noqa: E402
from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS  # noqa: E402
from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding, apply_rotary_pos_emb  # noqa: E402


def _cfg(head_dim, rope_parameters):
    return LlamaConfig(hidden_size=4 * head_dim, num_attention_heads=4, head_dim=head_dim,
                       max_position_embeddings=65536, rope_parameters=rope_parameters)


def _hf_rope(x, positions, rotary_dim, base):
    """transformers' rotation of the first rotary_dim elements; the rest passes through."""
    t, h, d = x.shape
    rot = LlamaRotaryEmbedding(_cfg(rotary_dim, {"rope_type": "default", "rope_theta": base}))
    xt = torch.from_numpy(np.asarray(x, np.float32)).permute(1, 0, 2)[None]  # [1, H, T, D]
    cos, sin = rot(xt, torch.as_tensor(positions, dtype=torch.int64)[None])
    xr, _ = apply_rotary_pos_emb(xt[..., :rotary_dim], xt[..., :rotary_dim], cos, sin)
    out = torch.cat([xr, xt[..., rotary_dim:]], dim=-1)
    return out[0].permute(1, 0, 2).double().numpy(), rot.inv_freq.numpy()


@pytest.mark.parametrize("d,rotary_dim,base", [(128, 128, 1e6), (64, 64, 1e4), (128, 64, 1e4), (256, 256, 5e5)])
def test_rope_matches_transformers(d, rotary_dim, base):
    x = np.random.default_rng(1).standard_normal((9, 3, d)).astype(np.float32)
    pos = np.array([0, 1, 2, 17, 300, 4095, 8191, 32767, 40000])
    ref, hf_inv = _hf_rope(x, pos, rotary_dim, base)
    # the frequency tables agree to float32 rounding ...
    np.testing.assert_allclose(oracle.rope_inv_freq(rotary_dim, base), hf_inv, rtol=4e-7, atol=0)
    # ... and with the same table the rotations agree to float32 cos/sin rounding
    out = oracle.rope(x, pos, rotary_dim, hf_inv)
    np.testing.assert_allclose(out, ref, rtol=0, atol=3e-6)


def test_rope_scaled_frequencies_match_transformers():
    llama3 = {"rope_type": "llama3", "rope_theta": 500000.0, "factor": 8.0, "low_freq_factor": 1.0,
              "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}
    hf, _ = ROPE_INIT_FUNCTIONS["llama3"](_cfg(128, llama3), "cpu")
    np.testing.assert_allclose(oracle.rope_inv_freq(128, 500000.0, llama3), hf.numpy(), rtol=2e-6, atol=0)
    linear = {"rope_type": "linear", "rope_theta": 10000.0, "factor": 4.0}
    hf, _ = ROPE_INIT_FUNCTIONS["linear"](_cfg(128, linear), "cpu")
    np.testing.assert_allclose(oracle.rope_inv_freq(128, 10000.0, linear), hf.numpy(), rtol=4e-7, atol=0)
    # the three bands of llama3: short wavelengths unchanged, long ones divided by factor
    plain = oracle.rope_inv_freq(128, 500000.0)
    scaled = oracle.rope_inv_freq(128, 500000.0, llama3)
    assert scaled[0] == plain[0] and np.isclose(scaled[-1], plain[-1] / 8.0, rtol=1e-6)


def test_rope_closed_forms():
    inv = oracle.rope_inv_freq(16, 10000.0)
    x = np.random.default_rng(2).standard_normal((5, 2, 16))
    # position 0 is the identity
    np.testing.assert_array_equal(oracle.rope(x, np.zeros(5, np.int32), 16, inv), x)
    # a rotation keeps each (i, i + dims/2) pair's norm
    out = oracle.rope(x, np.arange(5) * 977, 16, inv)
    np.testing.assert_allclose(np.hypot(out[..., :8], out[..., 8:]), np.hypot(x[..., :8], x[..., 8:]), rtol=1e-12)
    # q.k after rotation depends only on the position difference
    q, k = x[:1, :1], x[1:2, :1]
    s1 = np.sum(oracle.rope(q, [40], 16, inv) * oracle.rope(k, [15], 16, inv))
    s2 = np.sum(oracle.rope(q, [1040], 16, inv) * oracle.rope(k, [1015], 16, inv))
    assert abs(s1 - s2) < 1e-4
    # a one-hot vector rotates onto (cos, sin) in the rotate-half layout
    e0 = np.zeros((1, 1, 4))
    e0[0, 0, 0] = 1.0
    out = oracle.rope(e0, [1], 4, np.array([1.0, 0.01], np.float32))
    np.testing.assert_allclose(out[0, 0], [np.cos(1.0), 0.0, np.sin(1.0), 0.0], atol=1e-15)


def test_rope_store_kv_oracle():
    inv = oracle.rope_inv_freq(8, 10000.0)
    q = np.random.default_rng(3).standard_normal((3, 4, 8))
    k = np.random.default_rng(4).standard_normal((3, 2, 8))
    v = np.random.default_rng(5).standard_normal((3, 2, 8))
    kp0 = np.random.default_rng(6).standard_normal((16, 2, 8)).astype(np.float32)
    vp0 = np.random.default_rng(7).standard_normal((16, 2, 8)).astype(np.float32)
    kp, vp = kp0.copy(), vp0.copy()
    pos, loc = np.array([5, 9, 200]), np.array([11, 2, 7])
    q_rot, k_rot = oracle.rope_store_kv(q, k, v, pos, loc, kp, vp, 8, inv)
    np.testing.assert_array_equal(q_rot, oracle.rope(q, pos, 8, inv))
    np.testing.assert_array_equal(kp[loc], k_rot.astype(np.float32))
    np.testing.assert_array_equal(vp[loc], v.astype(np.float32))  # v is stored unrotated
    rest = np.setdiff1d(np.arange(16), loc)
    np.testing.assert_array_equal(kp[rest], kp0[rest])
    np.testing.assert_array_equal(vp[rest], vp0[rest])


def _mutant_interleaved(x, positions, rotary_dim, inv_freq):
    """Planted mistake: pairs (2i, 2i+1) (traditional=True) instead of (i, i + dims/2)."""
    x = np.asarray(x, np.float64)
    th = oracle.rope_angles(positions, inv_freq).astype(np.float64)[:, None, :]
    out = x.copy()
    a, b = x[..., 0:rotary_dim:2], x[..., 1:rotary_dim:2]
    out[..., 0:rotary_dim:2] = a * np.cos(th) - b * np.sin(th)
    out[..., 1:rotary_dim:2] = a * np.sin(th) + b * np.cos(th)
    return out


def test_rope_mutants_are_caught():
    x = np.random.default_rng(8).standard_normal((4, 2, 64)).astype(np.float32)
    pos = np.array([3, 70, 900, 5000])
    ref, hf_inv = _hf_rope(x, pos, 64, 1e4)
    assert not np.allclose(_mutant_interleaved(x, pos, 64, hf_inv), ref, atol=1e-3)
    # a flipped sine (rotation by -theta) fails the same pin and the one-hot closed form
    assert not np.allclose(oracle.rope(x, -pos, 64, hf_inv), ref, atol=1e-3)
    e0 = np.zeros((1, 1, 4))
    e0[0, 0, 0] = 1.0
    assert not np.allclose(oracle.rope(e0, [-1], 4, np.array([1.0, 0.01], np.float32))[0, 0, 2], np.sin(1.0))
