"""Parity at the exact sizes the benchmark measures, run the way it runs them.

* The headline decode step (Qwen3-0.6B heads, batch 128, contexts U[200,2048],
  page 1, a 262144-slot bf16 pool per layer, 28 layers): one work-list plan,
  then per layer the fused KV store + decode launch without its merge and the
  merge launch -- the bench's exact sequence -- with every layer's pool
  checked bit for bit at out_loc and sampled requests of several layers
  checked against the float64 oracle (attention/naive.py:50-60).
* The Qwen3-8B-head decode (batch 256, contexts U[1024,8192], page 16, a
  4M-slot pool): sampled requests against the oracle, run-to-run determinism.
"""

import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_close, to_np64
from minisgl_hip import ops, workloads

pytestmark = pytest.mark.gpu


def _oracle_rows(q, kp, vp, slots, scale):
    st = torch.from_numpy(np.asarray(slots, np.int64)).to(kp.device)
    kb = to_np64(kp.index_select(0, st))
    vb = to_np64(vp.index_select(0, st))
    return oracle.sdpa(to_np64(q)[:, None, :], kb.transpose(1, 0, 2), vb.transpose(1, 0, 2), scale)[:, 0]


def test_headline_decode_step_28_layers(cuda_device):
    hq, hkv, d, batch, pool, layers = 16, 8, 128, 128, 262144, 28
    c = workloads.decode_case(batch, 200, 2048, pool, 1, seed=0)
    dev = cuda_device
    gen = torch.Generator(device=dev).manual_seed(0)
    dt = torch.bfloat16
    kps = [torch.randn((pool, hkv, d), generator=gen, device=dev, dtype=dt) for _ in range(layers)]
    vps = [torch.randn((pool, hkv, d), generator=gen, device=dev, dtype=dt) for _ in range(layers)]
    qs = [torch.randn((batch, hq, d), generator=gen, device=dev, dtype=dt) for _ in range(layers)]
    ks = [torch.randn((batch, hkv, d), generator=gen, device=dev, dtype=dt) for _ in range(layers)]
    vs = [torch.randn((batch, hkv, d), generator=gen, device=dev, dtype=dt) for _ in range(layers)]
    outs = [torch.empty_like(x) for x in qs]
    indptr = torch.from_numpy(c.kv_indptr).to(dev)
    indices = torch.from_numpy(c.kv_indices).to(dev)
    out_loc = torch.from_numpy(c.out_loc).to(dev)
    splits = ops.default_splits(batch, hkv, int(c.lens.max()))
    ws = ops.decode_workspace(batch, hq, hkv, d, splits, dev)
    scale = d**-0.5
    print(f"case headline step 28 layers splits={splits}", flush=True)
    ops.paged_decode_plan(indptr, None, batch, hq, hkv, d, splits, ws)
    for layer in range(layers):
        ops.paged_decode_attention(qs[layer], kps[layer], vps[layer], indptr, indices, scale, max_splits=splits,
                                   out=outs[layer], workspace=ws, new_kv=(ks[layer], vs[layer], out_loc),
                                   planned=True, merge=False)
        ops.paged_decode_merge(outs[layer], indptr, None, hkv, splits, ws)
    torch.cuda.synchronize()
    loc = out_loc.long()
    for layer in range(layers):
        assert torch.equal(kps[layer][loc], ks[layer]) and torch.equal(vps[layer][loc], vs[layer]), (
            f"layer {layer}: new rows not at out_loc")
    pick = [0, 1, 31, 64, 100, 127, int(np.argmax(c.lens)), int(np.argmin(c.lens))]
    for layer in (0, 13, 27):
        ref = np.stack([_oracle_rows(qs[layer][b], kps[layer], vps[layer],
                                     c.kv_indices[c.kv_indptr[b]: c.kv_indptr[b + 1]], scale) for b in pick])
        assert_close(outs[layer][pick], ref, dt, f"headline step layer {layer}")
    # the same step through the one-call form (store fused, merge inside): same bits
    again = torch.empty_like(outs[27])
    ops.paged_decode_attention(qs[27], kps[27], vps[27], indptr, indices, scale, max_splits=splits, out=again,
                               workspace=ws, new_kv=(ks[27], vs[27], out_loc), planned=True)
    torch.cuda.synchronize()
    assert torch.equal(again, outs[27])
    del kps, vps
    torch.cuda.empty_cache()


def test_8b_heads_batch256_page16_full_size(cuda_device):
    hq, hkv, d, batch, pool, ps = 32, 8, 128, 256, 4 << 20, 16
    c = workloads.decode_case(batch, 1024, 8192, pool, ps, seed=0)
    dev = cuda_device
    gen = torch.Generator(device=dev).manual_seed(1)
    dt = torch.bfloat16
    kp = torch.randn((pool, hkv, d), generator=gen, device=dev, dtype=dt)
    vp = torch.randn((pool, hkv, d), generator=gen, device=dev, dtype=dt)
    q = torch.randn((batch, hq, d), generator=gen, device=dev, dtype=dt)
    pi = torch.from_numpy(c.page_indptr).to(dev)
    pid = torch.from_numpy(c.page_ids).to(dev)
    sl = torch.from_numpy(c.lens).to(dev)
    splits = ops.default_splits(batch, hkv, int(c.lens.max()))
    print(f"case 8b b256 page16 full splits={splits}", flush=True)
    out = ops.paged_decode_attention(q, kp, vp, pi, pid, d**-0.5, seq_lens=sl, page_size=ps, max_splits=splits)
    out2 = ops.paged_decode_attention(q, kp, vp, pi, pid, d**-0.5, seq_lens=sl, page_size=ps, max_splits=splits)
    torch.cuda.synchronize()
    assert torch.equal(out, out2), "not deterministic"
    pick = [0, 1, 77, 128, 200, 255, int(np.argmax(c.lens)), int(np.argmin(c.lens))]
    ref = []
    for b in pick:
        slots = oracle.expand_page_indices(c.page_ids[c.page_indptr[b]: c.page_indptr[b + 1]], ps, int(c.lens[b]))
        ref.append(_oracle_rows(q[b], kp, vp, slots, d**-0.5))
    assert_close(out[pick], np.stack(ref), dt, "8b b256 page16 sampled")
    del kp, vp
    torch.cuda.empty_cache()


def test_fp8_decode_step_measured_config(cuda_device):
    """The fp8 decode workload as the benchmark runs it (batch 128, contexts
    U[200,2048] seed 0, page 1, 262144-slot fp8 pools with per-(slot, kv head)
    scales), over 4 distinct layer pools: one plan, then per layer the decode
    launch with the quantising store fused in and no merge, then the merge.
    Each layer's output equals store-then-decode (msgl_store_kv_fp8, then the
    unplanned decode) bit for bit, the codes and scales at out_loc equal the
    store's, and sampled requests match the oracle over the dequantised pool
    (kvcache/pool.py:47-50 + attention/naive.py:50-60)."""
    hq, hkv, d, batch, pool, layers = 16, 8, 128, 128, 262144, 4
    c = workloads.decode_case(batch, 200, 2048, pool, 1, seed=0)
    dev = cuda_device
    gen = torch.Generator(device=dev).manual_seed(5)
    dt, f8 = torch.bfloat16, torch.float8_e4m3fn
    indptr = torch.from_numpy(c.kv_indptr).to(dev)
    indices = torch.from_numpy(c.kv_indices).to(dev)
    out_loc = torch.from_numpy(c.out_loc).to(dev)
    splits = ops.default_splits(batch, hkv, int(c.lens.max()))
    ws = ops.decode_workspace(batch, hq, hkv, d, splits, dev)
    scale = d**-0.5
    pools = []
    for layer in range(layers):
        kp = torch.empty((pool, hkv, d), dtype=f8, device=dev)
        vp = torch.empty_like(kp)
        sc = torch.empty((pool, hkv, 2), dtype=torch.float32, device=dev)
        for s0 in range(0, pool, 65536):
            rows = torch.arange(s0, s0 + 65536, dtype=torch.int32, device=dev)
            ops.store_kv_fp8(torch.randn((65536, hkv, d), generator=gen, device=dev, dtype=dt),
                             torch.randn((65536, hkv, d), generator=gen, device=dev, dtype=dt), rows, kp, vp, sc)
        pools.append((kp, vp, sc))
    qs = [torch.randn((batch, hq, d), generator=gen, device=dev, dtype=dt) for _ in range(layers)]
    ks = [torch.randn((batch, hkv, d), generator=gen, device=dev, dtype=dt) for _ in range(layers)]
    vs = [torch.randn((batch, hkv, d), generator=gen, device=dev, dtype=dt) for _ in range(layers)]
    # the reference sequence first, on copies: store, then the one-call decode
    refs, ref_pools = [], []
    for layer in range(layers):
        kp, vp, sc = (x.clone() for x in pools[layer])
        ops.store_kv_fp8(ks[layer], vs[layer], out_loc, kp, vp, sc)
        refs.append(ops.paged_decode_attention(qs[layer], kp, vp, indptr, indices, scale, max_splits=splits,
                                               kv_scale=sc))
        ref_pools.append((kp, vp, sc))
    print(f"case fp8 decode step {layers} layers splits={splits}", flush=True)
    outs = [torch.empty_like(x) for x in qs]
    ops.paged_decode_plan(indptr, None, batch, hq, hkv, d, splits, ws)
    for layer in range(layers):
        kp, vp, sc = pools[layer]
        ops.paged_decode_attention(qs[layer], kp, vp, indptr, indices, scale, max_splits=splits, out=outs[layer],
                                   workspace=ws, new_kv=(ks[layer], vs[layer], out_loc), planned=True,
                                   kv_scale=sc, merge=False)
        ops.paged_decode_merge(outs[layer], indptr, None, hkv, splits, ws, kv_fp8=True)
    torch.cuda.synchronize()
    loc = out_loc.long()
    for layer in range(layers):
        kp, vp, sc = pools[layer]
        rk, rv, rs = ref_pools[layer]
        assert torch.equal(outs[layer], refs[layer]), f"layer {layer}: fused planned step differs from store + decode"
        assert torch.equal(kp[loc].view(torch.uint8), rk[loc].view(torch.uint8)), f"layer {layer}: K codes"
        assert torch.equal(vp[loc].view(torch.uint8), rv[loc].view(torch.uint8)), f"layer {layer}: V codes"
        assert torch.equal(sc[loc], rs[loc]), f"layer {layer}: scales"
    pick = [0, 5, 64, 127, int(np.argmax(c.lens)), int(np.argmin(c.lens))]
    for layer in (0, layers - 1):
        kp, vp, sc = pools[layer]
        ref = []
        for b in pick:
            slots = torch.from_numpy(c.kv_indices[c.kv_indptr[b]: c.kv_indptr[b + 1]].astype(np.int64)).to(dev)
            kb = oracle.dequantize_fp8(kp[slots].view(torch.uint8).cpu().numpy(), sc[slots][..., 0].cpu().numpy())
            vb = oracle.dequantize_fp8(vp[slots].view(torch.uint8).cpu().numpy(), sc[slots][..., 1].cpu().numpy())
            ref.append(oracle.sdpa(to_np64(qs[layer][b])[:, None, :], kb.transpose(1, 0, 2), vb.transpose(1, 0, 2),
                                   scale)[:, 0])
        assert_close(outs[layer][pick], np.stack(ref), dt, f"fp8 step layer {layer}")
    del pools, ref_pools
    torch.cuda.empty_cache()
