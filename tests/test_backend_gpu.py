"""The backend behind the reference's interface, driven in the caller's order
(layers.py:107-110: store_kv, then attn_backend.forward), over several layers
and decode steps, checked against the oracle."""

import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_close, i32, randn, to_np64
from minisgl_hip.attention import create_attention_backend
from minisgl_hip.core import Batch, ModelConfig, Req
from minisgl_hip.kvcache import MHAKVCache
from test_kvquant_gpu import FP8, _codes, _deq

pytestmark = pytest.mark.gpu


def _setup(device, dtype, num_layers=3, num_tokens=8192, max_req=8, max_len=1024, page_size=1, hq=16, hkv=8, d=128):
    cfg = ModelConfig(num_qo_heads=hq, num_kv_heads=hkv, head_dim=d, num_layers=num_layers)
    kv = MHAKVCache(num_layers, num_tokens, hkv, d, dtype, device)
    table = np.zeros((max_req, max_len), dtype=np.int32)
    backend = create_attention_backend("hip", cfg, kv, table)
    return cfg, kv, table, backend


def test_decode_steps_through_backend(cuda_device):
    dt = torch.bfloat16
    cfg, kv, table, backend = _setup(cuda_device, dt)
    rng = np.random.default_rng(0)
    free = rng.permutation(8192).astype(np.int32)
    # three requests with cached histories (prefill already done): fill pools with history
    reqs = []
    for i, n in enumerate([40, 300, 7]):
        reqs.append(Req(input_ids=np.zeros(n + 1, np.int32), table_idx=i + 2, cached_len=n))
    free = oracle.allocate_paged(table, free, [r.table_idx for r in reqs], [0] * 3, [r.cached_len for r in reqs], 1)
    for layer in range(cfg.num_layers):
        kv.k[layer].copy_(randn(kv.k[layer].shape, 10 + layer, dt).to(cuda_device))
        kv.v[layer].copy_(randn(kv.v[layer].shape, 20 + layer, dt).to(cuda_device))
    for step in range(2):
        batch = Batch(reqs=reqs, phase="decode")
        free = oracle.allocate_paged(table, free, [r.table_idx for r in reqs], [r.cached_len for r in reqs],
                                     [r.device_len for r in reqs], 1)
        pos, out_loc = oracle.prepare_batch_indices(table, [r.table_idx for r in reqs],
                                                    [r.cached_len for r in reqs], [r.device_len for r in reqs])
        batch.positions = i32(pos, cuda_device)
        batch.out_loc = i32(out_loc, cuda_device)
        backend.prepare_metadata(batch)
        # the device metadata is the CSR form of attention/metal.py:145-152, bit-exact
        lens = [r.device_len for r in reqs]
        indptr, indices = oracle.csr_decode_metadata(table, [r.table_idx for r in reqs], lens)
        assert np.array_equal(batch.attn_metadata.kv_indptr.cpu().numpy(), indptr)
        assert np.array_equal(batch.attn_metadata.kv_indices.cpu().numpy(), indices)
        for layer in range(cfg.num_layers):
            q = randn((3, 16, 128), 100 * step + layer, dt).to(cuda_device)
            k = randn((3, 8, 128), 200 * step + layer, dt).to(cuda_device)
            v = randn((3, 8, 128), 300 * step + layer, dt).to(cuda_device)
            print(f"case backend step={step} layer={layer}", flush=True)
            kv.store_kv(k, v, batch.out_loc, layer)
            o = backend.forward(q, k, v, layer, batch)
            torch.cuda.synchronize()
            kvi, mask = oracle.naive_decode_metadata(table, [r.table_idx for r in reqs], lens)
            ref = oracle.naive_forward_decode(to_np64(q), to_np64(kv.k[layer]), to_np64(kv.v[layer]), kvi, mask,
                                              cfg.head_dim**-0.5)
            assert_close(o, ref, dt, f"backend step {step} layer {layer}")
            # the new token's row landed at out_loc
            assert torch.equal(kv.k[layer][batch.out_loc.long()], k)
        for r in reqs:
            r.complete_one()


@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (40, 8, 128), (14, 2, 64)])
def test_prefill_then_decode_through_backend(cuda_device, hq, hkv, d):
    """Chunked prefill (one request with a cached prefix, one without) followed
    by a decode step, all through prepare_metadata / store_kv / forward; the
    Qwen3-0.6B head layout and two whose query-head groups are not powers of two
    (Qwen3-14B: 40/8, Qwen2.5-0.5B: 14/2 at head_dim 64)."""
    dt = torch.bfloat16
    cfg, kv, table, backend = _setup(cuda_device, dt, num_layers=2, hq=hq, hkv=hkv, d=d)
    rng = np.random.default_rng(1)
    free = rng.permutation(8192).astype(np.int32)
    # request A: 50-token prompt whose first 20 tokens are already cached
    # request B: 33-token prompt, nothing cached
    reqs = [Req(input_ids=np.zeros(50, np.int32), table_idx=0, cached_len=20),
            Req(input_ids=np.zeros(33, np.int32), table_idx=5, cached_len=0)]
    free = oracle.allocate_paged(table, free, [0], [0], [20], 1)  # the cached prefix's slots
    for layer in range(cfg.num_layers):
        kv.k[layer].copy_(randn(kv.k[layer].shape, 40 + layer, dt).to(cuda_device))
        kv.v[layer].copy_(randn(kv.v[layer].shape, 50 + layer, dt).to(cuda_device))
    for phase in ("prefill", "decode"):
        rows = [r.table_idx for r in reqs]
        cached = [r.cached_len for r in reqs]
        device = [r.device_len for r in reqs]
        free = oracle.allocate_paged(table, free, rows, cached, device, 1)
        pos, out_loc = oracle.prepare_batch_indices(table, rows, cached, device)
        batch = Batch(reqs=reqs, phase=phase)
        batch.positions = i32(pos, cuda_device)
        batch.out_loc = i32(out_loc, cuda_device)
        backend.prepare_metadata(batch)
        if phase == "prefill":
            q_off, last, kvi = oracle.prefill_metadata(table, rows, cached, device)
            assert batch.attn_metadata.q_offsets == q_off
            assert np.array_equal(batch.attn_metadata.last_indices.cpu().numpy(), last)
            assert batch.attn_metadata.kv_indices[1] is None
            assert np.array_equal(batch.attn_metadata.kv_indices[0], kvi[0])
        t = len(out_loc)
        for layer in range(cfg.num_layers):
            q = randn((t, hq, d), 60 + layer, dt).to(cuda_device)
            k = randn((t, hkv, d), 70 + layer, dt).to(cuda_device)
            v = randn((t, hkv, d), 80 + layer, dt).to(cuda_device)
            print(f"case backend {phase} {hq}/{hkv}/{d} layer={layer}", flush=True)
            kv.store_kv(k, v, batch.out_loc, layer)
            o = backend.forward(q, k, v, layer, batch)
            torch.cuda.synchronize()
            kp, vp = to_np64(kv.k[layer]), to_np64(kv.v[layer])
            if phase == "prefill":
                ref = oracle.forward_prefill(to_np64(q), to_np64(k), to_np64(v), kp, vp, q_off, kvi,
                                             cfg.head_dim**-0.5)
            else:
                kvi_d, mask = oracle.naive_decode_metadata(table, rows, device)
                ref = oracle.naive_forward_decode(to_np64(q), kp, vp, kvi_d, mask, cfg.head_dim**-0.5)
            assert_close(o, ref, dt, f"backend {phase} layer {layer}")
        for r in reqs:
            r.complete_one()


def test_fused_and_eager_store_agree(cuda_device):
    """The backend's fused decode store gives the same outputs and pool bits as
    the eager store_kv + forward order, and a pool read in between sees the store."""
    dt = torch.bfloat16
    outs, pools = [], []
    for fuse in (True, False):
        cfg = ModelConfig(num_qo_heads=16, num_kv_heads=8, head_dim=128, num_layers=2)
        kv = MHAKVCache(2, 4096, 8, 128, dt, cuda_device)
        table = np.zeros((4, 512), dtype=np.int32)
        backend = create_attention_backend("hip", cfg, kv, table)
        backend.fuse_decode_store = fuse
        free = np.random.default_rng(3).permutation(4096).astype(np.int32)
        reqs = [Req(input_ids=np.zeros(n + 1, np.int32), table_idx=i, cached_len=n) for i, n in enumerate([9, 200])]
        free = oracle.allocate_paged(table, free, [0, 1], [0, 0], [9, 200], 1)
        free = oracle.allocate_paged(table, free, [0, 1], [9, 200], [10, 201], 1)
        for layer in range(2):
            kv.k[layer].copy_(randn(kv.k[layer].shape, 5 + layer, dt).to(cuda_device))
            kv.v[layer].copy_(randn(kv.v[layer].shape, 7 + layer, dt).to(cuda_device))
        pos, out_loc = oracle.prepare_batch_indices(table, [0, 1], [9, 200], [10, 201])
        batch = Batch(reqs=reqs, phase="decode")
        batch.out_loc = i32(out_loc, cuda_device)
        backend.prepare_metadata(batch)
        res = []
        for layer in range(2):
            q = randn((2, 16, 128), 30 + layer, dt).to(cuda_device)
            k = randn((2, 8, 128), 40 + layer, dt).to(cuda_device)
            v = randn((2, 8, 128), 50 + layer, dt).to(cuda_device)
            kv.store_kv(k, v, batch.out_loc, layer)
            if layer == 1:  # a reader between store and forward must see the new rows
                assert torch.equal(kv.k_cache(1)[batch.out_loc.long()], k)
            res.append(backend.forward(q, k, v, layer, batch))
        torch.cuda.synchronize()
        outs.append(torch.stack(res))
        pools.append(torch.stack([kv.k_cache(0), kv.v_cache(0), kv.k_cache(1), kv.v_cache(1)]))
    assert torch.equal(outs[0], outs[1])
    assert torch.equal(pools[0].view(torch.int16), pools[1].view(torch.int16))


@pytest.mark.parametrize("cache", ["bf16", "fp8", "f32"])
def test_mixed_batch_through_backend(cuda_device, cache):
    """A continuous-batching step (4 decode requests, then a chunk over a cached
    prefix and a fresh prompt) as one batch of phase "mixed" through
    prepare_metadata / store_kv / forward, then a decode step of all six: every
    request vs the oracle, new rows at out_loc. A bf16 cache takes the single
    launch (msgl_mixed_attention). An fp8 cache runs the quantising fused decode,
    then fp8 prefill: codes and scales at out_loc are bit-exact to the
    quantiser, and the oracle reads the dequantised pool. An fp32 cache runs the
    two phases in turn."""
    fp8 = cache == "fp8"
    dt = torch.float32 if cache == "f32" else torch.bfloat16
    cfg = ModelConfig(num_qo_heads=32, num_kv_heads=8, head_dim=128, num_layers=2)
    kv = MHAKVCache(2, 16384, 8, 128, dt, cuda_device, kv_dtype=FP8 if fp8 else None)
    table = np.zeros((10, 2048), dtype=np.int32)
    backend = create_attention_backend("hip", cfg, kv, table)
    free = np.random.default_rng(4).permutation(16384).astype(np.int32)
    hist = [90, 700, 33, 1500]
    reqs = [Req(input_ids=np.zeros(n + 1, np.int32), table_idx=i, cached_len=n) for i, n in enumerate(hist)]
    free = oracle.allocate_paged(table, free, [0, 1, 2, 3], [0] * 4, hist, 1)
    reqs.append(Req(input_ids=np.zeros(300, np.int32), table_idx=7, cached_len=200))  # chunk over a cached prefix
    free = oracle.allocate_paged(table, free, [7], [0], [200], 1)
    reqs.append(Req(input_ids=np.zeros(77, np.int32), table_idx=9, cached_len=0))  # a fresh prompt
    all_slots = torch.arange(16384, dtype=torch.int32, device=cuda_device)
    for layer in range(2):
        k0 = randn(kv.k[layer].shape, 90 + layer, dt).to(cuda_device)
        v0 = randn(kv.v[layer].shape, 95 + layer, dt).to(cuda_device)
        if fp8:  # quantised rows in every slot
            kv.store_kv(k0, v0, all_slots, layer)
        else:
            kv.k[layer].copy_(k0)
            kv.v[layer].copy_(v0)
    for phase in ("mixed", "decode"):
        rows = [r.table_idx for r in reqs]
        cached = [r.cached_len for r in reqs]
        device = [r.device_len for r in reqs]
        free = oracle.allocate_paged(table, free, rows, cached, device, 1)
        pos, out_loc = oracle.prepare_batch_indices(table, rows, cached, device)
        batch = Batch(reqs=reqs, phase=phase)
        batch.positions = i32(pos, cuda_device)
        batch.out_loc = i32(out_loc, cuda_device)
        backend.prepare_metadata(batch)
        if phase == "mixed":
            assert batch.attn_metadata.num_decode == 4
            q_off, last, _ = oracle.prefill_metadata(table, rows, cached, device)
            assert np.array_equal(batch.attn_metadata.last_indices.cpu().numpy(), last)
        t = len(out_loc)
        for layer in range(2):
            q = randn((t, 32, 128), 300 + layer, dt).to(cuda_device)
            k = randn((t, 8, 128), 310 + layer, dt).to(cuda_device)
            v = randn((t, 8, 128), 320 + layer, dt).to(cuda_device)
            print(f"case backend {cache} {phase} layer={layer}", flush=True)
            kv.store_kv(k, v, batch.out_loc, layer)
            o = backend.forward(q, k, v, layer, batch)
            torch.cuda.synchronize()
            loc = batch.out_loc.long()
            if fp8:
                kc, ks = oracle.quantize_fp8(to_np64(k).astype(np.float32))
                vc, vs = oracle.quantize_fp8(to_np64(v).astype(np.float32))
                np.testing.assert_array_equal(_codes(kv.k_cache(layer))[out_loc], kc)
                np.testing.assert_array_equal(_codes(kv.v_cache(layer))[out_loc], vc)
                sc = kv.kv_scale[layer][loc].cpu().numpy()
                np.testing.assert_array_equal(sc[..., 0], ks)
                np.testing.assert_array_equal(sc[..., 1], vs)
                kp, vp = _deq(kv.k[layer], kv.kv_scale[layer], 0), _deq(kv.v[layer], kv.kv_scale[layer], 1)
            else:
                assert torch.equal(kv.k_cache(layer)[loc], k) and torch.equal(kv.v_cache(layer)[loc], v)
                kp, vp = to_np64(kv.k[layer]), to_np64(kv.v[layer])
            q_off, _, _ = oracle.prefill_metadata(table, rows, cached, device)
            # every request as a prefill of its extend rows over its whole context,
            # read from the pool (a one-row extend attends like decode:
            # attention/base.py:103, mask None)
            kvi = [table[r, :n] for r, n in zip(rows, device)]
            ref = oracle.forward_prefill(to_np64(q), None, None, kp, vp, q_off, kvi, 128**-0.5)
            assert_close(o, ref, dt, f"backend {cache} {phase} layer {layer}")
        for r in reqs:
            if r.extend_len == 1 or phase == "mixed":
                r.complete_one()


def test_backend_validation_rejects_slots_outside_the_pool(cuda_device):
    """validate=True: the step's device-built indices are checked before use; a
    page-table entry past the pool fails prepare_metadata with ValueError."""
    dt = torch.bfloat16
    cfg = ModelConfig(num_qo_heads=16, num_kv_heads=8, head_dim=128, num_layers=1)
    kv = MHAKVCache(1, 4096, 8, 128, dt, cuda_device)
    table = np.zeros((4, 512), dtype=np.int32)
    backend = create_attention_backend("hip", cfg, kv, table)
    backend.validate = True
    free = np.random.default_rng(6).permutation(4096).astype(np.int32)
    reqs = [Req(input_ids=np.zeros(n + 1, np.int32), table_idx=i, cached_len=n) for i, n in enumerate([30, 120])]
    free = oracle.allocate_paged(table, free, [0, 1], [0, 0], [31, 121], 1)
    batch = Batch(reqs=reqs, phase="decode")
    print("case backend validate ok", flush=True)
    backend.prepare_metadata(batch)  # valid
    table[1, 50] = 4096  # one slot past the pool
    backend._mirrored[:] = 0  # send the rows again
    with pytest.raises(ValueError, match="outside the pool"):
        backend.prepare_metadata(Batch(reqs=reqs, phase="decode"))


def test_uniform_decode_batch_runs_shared_head_form(cuda_device):
    """100 requests of near-uniform length (enough (request, kv head) pairs to fill
    the device): the backend picks max_splits = 1 (four wavefronts per
    (request, kv head), combined in LDS, no merge launch); sampled requests vs
    the oracle, and the fused store lands at out_loc."""
    dt = torch.bfloat16
    cfg = ModelConfig(num_qo_heads=16, num_kv_heads=8, head_dim=128, num_layers=2)
    kv = MHAKVCache(2, 65536, 8, 128, dt, cuda_device)
    table = np.zeros((100, 512), dtype=np.int32)
    backend = create_attention_backend("hip", cfg, kv, table)
    rng = np.random.default_rng(8)
    free = rng.permutation(65536).astype(np.int32)
    hist = rng.integers(400, 450, size=100)
    reqs = [Req(input_ids=np.zeros(n + 1, np.int32), table_idx=i, cached_len=int(n)) for i, n in enumerate(hist)]
    free = oracle.allocate_paged(table, free, list(range(100)), [0] * 100, [int(n) for n in hist], 1)
    free = oracle.allocate_paged(table, free, list(range(100)), [r.cached_len for r in reqs],
                                 [r.device_len for r in reqs], 1)
    for layer in range(2):
        kv.k[layer].copy_(randn(kv.k[layer].shape, 130 + layer, dt).to(cuda_device))
        kv.v[layer].copy_(randn(kv.v[layer].shape, 140 + layer, dt).to(cuda_device))
    rows = [r.table_idx for r in reqs]
    device = [r.device_len for r in reqs]
    pos, out_loc = oracle.prepare_batch_indices(table, rows, [r.cached_len for r in reqs], device)
    batch = Batch(reqs=reqs, phase="decode")
    batch.out_loc = i32(out_loc, cuda_device)
    backend.prepare_metadata(batch)
    assert batch.attn_metadata.max_splits == 1
    pick = [0, 1, 50, 98, 99]
    for layer in range(2):
        q = randn((100, 16, 128), 150 + layer, dt).to(cuda_device)
        k = randn((100, 8, 128), 160 + layer, dt).to(cuda_device)
        v = randn((100, 8, 128), 170 + layer, dt).to(cuda_device)
        print(f"case backend shared-head layer={layer}", flush=True)
        kv.store_kv(k, v, batch.out_loc, layer)
        o = backend.forward(q, k, v, layer, batch)
        torch.cuda.synchronize()
        loc = batch.out_loc.long()
        assert torch.equal(kv.k_cache(layer)[loc], k) and torch.equal(kv.v_cache(layer)[loc], v)
        kvi, mask = oracle.naive_decode_metadata(table, [rows[i] for i in pick], [device[i] for i in pick])
        ref = oracle.naive_forward_decode(to_np64(q[pick]), to_np64(kv.k[layer]), to_np64(kv.v[layer]), kvi, mask,
                                          128**-0.5)
        assert_close(o[pick], ref, dt, f"shared-head layer {layer}")
