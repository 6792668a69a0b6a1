"""Rotary embedding (layers.py:45-56) and the fused rotate-and-store
(layers.py:107-109) on the GPU vs the float64 oracle, plus the attention layer
driven through the global context in the reference's order."""

import numpy as np
import pytest
import torch

import oracle
from gpu_util import DTYPES, assert_close, i32, randn, to_np64
from minisgl_hip import ops
from minisgl_hip.attention import create_attention_backend
from minisgl_hip.core import Batch, Context, ModelConfig, Req, RotaryConfig, set_global_ctx
from minisgl_hip.kvcache import MHAKVCache
from minisgl_hip.layers import AttentionLayer, rope_inv_freq

pytestmark = pytest.mark.gpu

LLAMA3 = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_embeddings": 8192}

CASES = [  # (T, H, D, rotary_dim, base, scaling)
    (37, 16, 128, 128, 1e6, None),  # Qwen3
    (5, 4, 64, 64, 1e4, None),
    (19, 8, 128, 64, 1e4, None),  # partial rotary: the upper half passes through
    (11, 4, 256, 256, 5e5, LLAMA3),
    (9, 2, 128, 128, 1e4, {"rope_type": "linear", "factor": 4.0}),
    (13, 4, 32, 24, 1e4, None),  # half the rotary dim not a multiple of 8: 8-byte items for 16-bit types
    (7, 3, 36, 32, 1e4, None),  # a pass-through tail of 4 elements
]


def _positions(t, seed):
    pos = np.random.default_rng(seed).integers(0, 40000, t)
    pos[0] = 0
    return pos


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: f"T{c[0]}H{c[1]}D{c[2]}r{c[3]}")
def test_rope_matches_oracle(cuda_device, dt, case):
    t, h, d, rot, base, scaling = case
    dtype = DTYPES[dt]
    print(f"case rope {dt} {case[:4]}", flush=True)
    x = randn((t, h, d), 1, dtype).to(cuda_device)
    pos = _positions(t, 2)
    inv = rope_inv_freq(rot, base, scaling)
    out = ops.rope(x, i32(pos, cuda_device), inv.to(cuda_device), rot)
    torch.cuda.synchronize()
    ref = oracle.rope(to_np64(x), pos, rot, oracle.rope_inv_freq(rot, base, scaling))
    assert_close(out, ref, dtype, f"rope {dt} {case[:4]}")
    # pass-through elements are copied exactly; position 0 is the identity
    assert torch.equal(out[..., rot:], x[..., rot:])
    assert torch.equal(out[0], x[0])


def test_rope_in_place(cuda_device):
    x = randn((64, 16, 128), 3, torch.bfloat16).to(cuda_device)
    pos = i32(np.arange(64) * 311, cuda_device)
    inv = rope_inv_freq(128, 1e6).to(cuda_device)
    ref = ops.rope(x, pos, inv, 128)
    y = x.clone()
    ops.rope(y, pos, inv, 128, out=y)
    torch.cuda.synchronize()
    assert torch.equal(y, ref)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("d,rot", [(128, 128), (32, 24), (36, 32)])
def test_rope_store_kv_matches_oracle(cuda_device, dt, d, rot):
    """Qwen3's full rotation (16-byte items), and two shapes the 16-bit kernel
    moves in 8-byte items: half the rotary dim not a multiple of 8 (24), and a
    pass-through tail of 4 elements (36 / 32)."""
    dtype = DTYPES[dt]
    t, hq, hkv, n = 300, 32, 8, 4096
    q = randn((t, hq, d), 10, dtype).to(cuda_device)
    k = randn((t, hkv, d), 11, dtype).to(cuda_device)
    v = randn((t, hkv, d), 12, dtype).to(cuda_device)
    kp0 = randn((n, hkv, d), 13, dtype).to(cuda_device)
    vp0 = randn((n, hkv, d), 14, dtype).to(cuda_device)
    kp, vp = kp0.clone(), vp0.clone()
    loc = np.random.default_rng(15).permutation(n)[:t]
    pos = _positions(t, 16)
    inv = rope_inv_freq(rot, 1e6).to(cuda_device)
    print(f"case rope_store_kv {dt} d={d} rot={rot}", flush=True)
    k_out = torch.empty_like(k)
    q_out = ops.rope_store_kv(q, k, v, i32(pos, cuda_device), i32(loc, cuda_device), kp, vp, inv, rot, k_out=k_out)
    torch.cuda.synchronize()
    oinv = oracle.rope_inv_freq(rot, 1e6)
    assert_close(q_out, oracle.rope(to_np64(q), pos, rot, oinv), dtype, "rotated q")
    loc_t = torch.from_numpy(loc).to(cuda_device)
    assert_close(kp[loc_t], oracle.rope(to_np64(k), pos, rot, oinv), dtype, "stored rotated k")
    assert torch.equal(kp[loc_t], k_out)  # k_out is exactly what was stored
    assert torch.equal(vp[loc_t], v)  # v is stored unrotated, bit-exact
    # same arithmetic as the plain rotation kernel, bit for bit
    posd = i32(pos, cuda_device)
    assert torch.equal(q_out, ops.rope(q, posd, inv, rot))
    assert torch.equal(k_out, ops.rope(k, posd, inv, rot))
    rest = torch.ones(n, dtype=torch.bool, device=cuda_device)
    rest[loc_t] = False
    assert torch.equal(kp[rest], kp0[rest]) and torch.equal(vp[rest], vp0[rest])
    # in place on q and k
    q2, k2 = q.clone(), k.clone()
    ops.rope_store_kv(q2, k2, v, posd, i32(loc, cuda_device), kp, vp, inv, rot, q_out=q2, k_out=k2)
    torch.cuda.synchronize()
    assert torch.equal(q2, q_out) and torch.equal(k2, k_out)


def test_rope_store_kv_skips_slots_outside_pool(cuda_device):
    dtype = torch.bfloat16
    t, hkv, d, n = 4, 2, 64, 16
    q = randn((t, 4, d), 20, dtype).to(cuda_device)
    k = randn((t, hkv, d), 21, dtype).to(cuda_device)
    v = randn((t, hkv, d), 22, dtype).to(cuda_device)
    kp = torch.zeros((n, hkv, d), dtype=dtype, device=cuda_device)
    vp = torch.zeros_like(kp)
    loc = i32([3, -1, n, 7], cuda_device)
    inv = rope_inv_freq(d, 1e4).to(cuda_device)
    q_out = ops.rope_store_kv(q, k, v, i32([1, 2, 3, 4], cuda_device), loc, kp, vp, inv, d)
    torch.cuda.synchronize()
    assert torch.equal(q_out, ops.rope(q, i32([1, 2, 3, 4], cuda_device), inv, d))
    written = torch.zeros(n, dtype=torch.bool, device=cuda_device)
    written[[3, 7]] = True
    assert torch.equal(vp[3], v[0]) and torch.equal(vp[7], v[3])
    assert not kp[~written].any() and not vp[~written].any()


def _layer_setup(device, dtype):
    cfg = ModelConfig(num_qo_heads=16, num_kv_heads=8, head_dim=128, num_layers=2)
    kv = MHAKVCache(2, 8192, 8, 128, dtype, device)
    table = np.zeros((8, 1024), dtype=np.int32)
    backend = create_attention_backend("hip", cfg, kv, table)
    ctx = Context(page_size=1)
    ctx.page_table, ctx.kv_cache, ctx.attn_backend = table, kv, backend
    rotary = RotaryConfig(head_dim=128, rotary_dim=128, base=1e6)
    layers = [AttentionLayer(i, 16, 8, 128, rotary, device) for i in range(2)]
    return cfg, kv, table, backend, ctx, layers


def test_attention_layer_prefill_then_decode(cuda_device):
    """layers.py:103-111 through the global context: a chunked prefill (one request
    with a cached prefix) and a decode step, vs rotate -> store -> attention in fp64."""
    dt = torch.bfloat16
    cfg, kv, table, backend, ctx, layers = _layer_setup(cuda_device, dt)
    set_global_ctx(ctx)
    try:
        free = np.random.default_rng(30).permutation(8192).astype(np.int32)
        reqs = [Req(input_ids=np.zeros(50, np.int32), table_idx=0, cached_len=20),
                Req(input_ids=np.zeros(33, np.int32), table_idx=1, cached_len=0)]
        free = oracle.allocate_paged(table, free, [0, 1], [0, 0], [50, 33], 1)
        for layer in range(2):  # the cached prefix of request 0 holds rotated keys already
            kv.k[layer].copy_(randn(kv.k[layer].shape, 31 + layer, dt).to(cuda_device))
            kv.v[layer].copy_(randn(kv.v[layer].shape, 33 + layer, dt).to(cuda_device))
        inv = oracle.rope_inv_freq(128, 1e6)
        scale = 128**-0.5
        for phase in ("prefill", "decode"):
            batch = Batch(reqs=reqs, phase=phase)
            if phase == "decode":
                free = oracle.allocate_paged(table, free, [0, 1], [r.cached_len for r in reqs],
                                             [r.device_len for r in reqs], 1)
            rows = [r.table_idx for r in reqs]
            cached, dlen = [r.cached_len for r in reqs], [r.device_len for r in reqs]
            pos, out_loc = oracle.prepare_batch_indices(table, rows, cached, dlen)
            batch.positions, batch.out_loc = i32(pos, cuda_device), i32(out_loc, cuda_device)
            backend.prepare_metadata(batch)
            with ctx.forward_batch(batch):
                for layer in range(2):
                    t = len(pos)
                    q = randn((t, 16, 128), 40 + layer, dt).to(cuda_device)
                    k = randn((t, 8, 128), 50 + layer, dt).to(cuda_device)
                    v = randn((t, 8, 128), 60 + layer, dt).to(cuda_device)
                    print(f"case attention layer {phase} layer={layer}", flush=True)
                    o = layers[layer](q, k, v)
                    torch.cuda.synchronize()
                    assert o.shape == (t, 16 * 128)
                    kp, vp = to_np64(kv.k[layer]), to_np64(kv.v[layer])
                    np.testing.assert_allclose(kp[out_loc], oracle.rope(to_np64(k), pos, 128, inv), rtol=1e-2,
                                               atol=1e-2)
                    assert torch.equal(kv.v[layer][batch.out_loc.long()], v)
                    q_rot = oracle.rope(to_np64(q), pos, 128, inv)
                    if phase == "prefill":
                        offs = np.concatenate([[0], np.cumsum(np.array(dlen) - np.array(cached))])
                        idx = [table[r, :d] for r, d in zip(rows, dlen)]
                        ref = oracle.forward_prefill(q_rot, None, None, kp, vp, offs, idx, scale)
                    else:
                        kvi, mask = oracle.naive_decode_metadata(table, rows, dlen)
                        ref = oracle.naive_forward_decode(q_rot, kp, vp, kvi, mask, scale)
                    assert_close(o.view(t, 16, 128), ref, dt, f"attention layer {phase} {layer}")
            for r in reqs:
                r.complete_one()
    finally:
        set_global_ctx(None)
