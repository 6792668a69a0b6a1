"""fp8 KV cache on the GPU vs the oracle: the quantising store bit for bit
(codes and scales), and paged decode over fp8 pools against the float64 decode
of the dequantised pool (attention/naive.py:50-60 semantics), over the
reference test's shape grid, split settings, page ids and the headline batch."""

import numpy as np
import pytest
import torch

import oracle
from gpu_util import DTYPES, assert_close, i32, randn, to_np64
from minisgl_hip import ops, workloads

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn


def _codes(t):
    return t.view(torch.uint8).cpu().numpy()


def _fp8_pools(n, hkv, d, seed, device, src_dtype=torch.bfloat16, spread=2.0):
    """Quantise random rows into every slot with the HIP store; returns (kp, vp, kv_scale, k_src, v_src)."""
    g = torch.Generator(device=device).manual_seed(seed)
    k = torch.randn((n, hkv, d), generator=g, device=device, dtype=torch.float32)
    v = torch.randn((n, hkv, d), generator=g, device=device, dtype=torch.float32)
    if spread:  # rows of very different magnitudes (log-normal, sigma = spread), so the per-row scales matter
        k *= torch.exp(torch.randn((n, hkv, 1), generator=g, device=device) * spread)
        v *= torch.exp(torch.randn((n, hkv, 1), generator=g, device=device) * spread)
    k, v = k.to(src_dtype), v.to(src_dtype)
    kp = torch.empty((n, hkv, d), dtype=FP8, device=device)
    vp = torch.empty_like(kp)
    sc = torch.empty((n, hkv, 2), dtype=torch.float32, device=device)
    ops.store_kv_fp8(k, v, torch.arange(n, dtype=torch.int32, device=device), kp, vp, sc)
    return kp, vp, sc, k, v


def _deq(codes, sc, which):
    """Dequantised pool from the codes and column `which` (0 = K, 1 = V) of kv_scale."""
    return oracle.dequantize_fp8(_codes(codes), sc[..., which].cpu().numpy())


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("hkv,d", [(8, 128), (2, 64), (4, 256)])
def test_store_kv_fp8_bit_exact(cuda_device, dt, hkv, d):
    dtype = DTYPES[dt]
    t, n = 300, 4096
    g = torch.Generator().manual_seed(5)
    spread = 1.0 if dtype == torch.float16 else 3.0  # row magnitudes over many binades, finite in fp16
    k = (torch.randn((t, hkv, d), generator=g) * torch.exp(torch.randn((t, hkv, 1), generator=g) * spread)).to(dtype)
    v = (torch.randn((t, hkv, d), generator=g) * torch.exp(torch.randn((t, hkv, 1), generator=g) * spread)).to(dtype)
    k[7, 0] = 0.0  # zero rows: codes 0, scale 0
    v[9] = -0.0
    k, v = k.to(cuda_device), v.to(cuda_device)
    kp0 = torch.randint(0, 126, (n, hkv, d), dtype=torch.uint8, device=cuda_device)
    kp, vp = kp0.clone().view(FP8), kp0.clone().view(FP8)
    sc = torch.full((n, hkv, 2), 3.0, device=cuda_device)
    loc = np.random.default_rng(6).permutation(n)[:t].astype(np.int32)
    print(f"case store_kv_fp8 {dt} hkv={hkv} d={d}", flush=True)
    ops.store_kv_fp8(k, v, i32(loc, cuda_device), kp, vp, sc)
    torch.cuda.synchronize()
    ks, vs = sc[..., 0], sc[..., 1]
    kc, ksc = oracle.quantize_fp8(to_np64(k).astype(np.float32))
    vc, vsc = oracle.quantize_fp8(to_np64(v).astype(np.float32))
    np.testing.assert_array_equal(_codes(kp)[loc], kc)
    np.testing.assert_array_equal(_codes(vp)[loc], vc)
    np.testing.assert_array_equal(ks.cpu().numpy()[loc], ksc)
    np.testing.assert_array_equal(vs.cpu().numpy()[loc], vsc)
    rest = np.setdiff1d(np.arange(n), loc)
    np.testing.assert_array_equal(_codes(kp)[rest], kp0.cpu().numpy()[rest])
    assert (ks.cpu().numpy()[rest] == 3.0).all()


def test_store_kv_fp8_skips_slots_outside_pool(cuda_device):
    k = randn((3, 2, 64), 1, torch.bfloat16).to(cuda_device)
    kp = torch.zeros((8, 2, 64), dtype=torch.uint8, device=cuda_device).view(FP8)
    vp = torch.zeros_like(kp)
    sc = torch.zeros((8, 2, 2), device=cuda_device)
    ops.store_kv_fp8(k, k, i32([-1, 8, 5], cuda_device), kp, vp, sc)
    torch.cuda.synchronize()
    ks = sc[..., 0]
    written = np.zeros(8, bool)
    written[5] = True
    assert not _codes(kp)[~written].any() and not ks.cpu().numpy()[~written].any()
    assert _codes(kp)[5].any() and (ks.cpu().numpy()[5] > 0).all()


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (32, 8, 128), (8, 8, 64), (16, 2, 256), (64, 8, 128),
                                      (24, 12, 128), (32, 16, 64)])
@pytest.mark.parametrize("splits", [1, None, 8])
def test_fp8_decode_reference_grid(cuda_device, dt, hq, hkv, d, splits):
    """tests/test_attention.py:19-39's grid (B=7, lens [1,2,17,31,32,33,700], N=4096) over fp8 pools."""
    dtype = DTYPES[dt]
    c = workloads.reference_test_case()
    kp, vp, sc, _, _ = _fp8_pools(4096, hkv, d, 100, cuda_device)
    q = randn((7, hq, d), 102, dtype).to(cuda_device)
    print(f"case fp8 grid hq={hq} hkv={hkv} d={d} {dt} splits={splits}", flush=True)
    out = ops.paged_decode_attention(q, kp, vp, i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device),
                                     d**-0.5, max_splits=splits, kv_scale=sc)
    torch.cuda.synchronize()
    ref = oracle.paged_decode(to_np64(q), _deq(kp, sc, 0), _deq(vp, sc, 1), c.kv_indptr, c.kv_indices, d**-0.5)
    assert_close(out, ref, dtype, f"fp8 grid {hq}/{hkv}/{d} {dt} splits={splits}")


@pytest.mark.parametrize("splits", [1, 4, 64])
def test_fp8_decode_edge_lengths_and_pages(cuda_device, splits):
    lens = [1, 15, 16, 17, 63, 64, 65, 127, 128, 129, 1000, 4097]
    for page in (1, 16):
        c = workloads.decode_case_from_lens(lens, num_slots=16384, page_size=page, seed=7)
        kp, vp, sc, _, _ = _fp8_pools(16384, 8, 128, 200, cuda_device)
        q = randn((len(lens), 16, 128), 202, torch.bfloat16).to(cuda_device)
        print(f"case fp8 edge page={page} splits={splits}", flush=True)
        kwargs = dict(seq_lens=i32(c.lens, cuda_device), page_size=page) if page > 1 else {}
        indptr = c.page_indptr if page > 1 else c.kv_indptr
        indices = c.page_ids if page > 1 else c.kv_indices
        out = ops.paged_decode_attention(q, kp, vp, i32(indptr, cuda_device), i32(indices, cuda_device),
                                         128**-0.5, max_splits=splits, kv_scale=sc, **kwargs)
        torch.cuda.synchronize()
        ref = oracle.paged_decode(to_np64(q), _deq(kp, sc, 0), _deq(vp, sc, 1), c.kv_indptr, c.kv_indices, 128**-0.5)
        assert_close(out, ref, torch.bfloat16, f"fp8 edge page={page} splits={splits}")


def test_fp8_planned_matches_unplanned(cuda_device):
    c = workloads.decode_case(64, 10, 3000, 131072, 1, seed=3)
    kp, vp, sc, _, _ = _fp8_pools(131072, 8, 128, 300, cuda_device)
    q = randn((64, 32, 128), 301, torch.bfloat16).to(cuda_device)
    ip, ix = i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device)
    splits = ops.default_splits(64, 8, int(c.lens.max()))
    ws = ops.decode_workspace(64, 32, 8, 128, splits, cuda_device)
    a = ops.paged_decode_attention(q, kp, vp, ip, ix, 128**-0.5, max_splits=splits, kv_scale=sc)
    ops.paged_decode_plan(ip, None, 64, 32, 8, 128, splits, ws)
    b = ops.paged_decode_attention(q, kp, vp, ip, ix, 128**-0.5, max_splits=splits, kv_scale=sc,
                                   workspace=ws, planned=True)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("hq,hkv", [(16, 8), (24, 12)])
def test_fp8_key_ranges_long_contexts(cuda_device, hq, hkv):
    """~1M keys over fp8 pools (Qwen3-0.6B heads; and 12 kv heads, three kv-head
    groups): enough for the decode launch to split by equal key ranges. The
    fused quantising store gives the same bits as store + decode, and the
    result agrees with the unsplit decode (one workgroup per request and
    kv-head group)."""
    b, d = 160, 128
    c = workloads.decode_case(b, 4096, 8192, 1 << 21, 1, seed=13)
    cus = torch.cuda.get_device_properties(cuda_device).multi_processor_count
    assert int(c.lens.sum()) >= 2048 * 3 * cus // 2, "too few keys to select key ranges"
    n = 1 << 21
    kp, vp, sc, _, _ = _fp8_pools(n, hkv, d, 410, cuda_device, spread=1.0)
    kp2, vp2, sc2 = kp.clone(), vp.clone(), sc.clone()
    q = randn((b, hq, d), 411, torch.bfloat16).to(cuda_device)
    k_new = randn((b, hkv, d), 412, torch.bfloat16).to(cuda_device)
    v_new = randn((b, hkv, d), 413, torch.bfloat16).to(cuda_device)
    out_loc = i32(c.out_loc, cuda_device)
    ip, ix = i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device)
    print(f"case fp8 key ranges hkv={hkv}", flush=True)
    ops.store_kv_fp8(k_new, v_new, out_loc, kp, vp, sc)
    a = ops.paged_decode_attention(q, kp, vp, ip, ix, d**-0.5, kv_scale=sc, max_seq_len=int(c.lens.max()))
    f = ops.paged_decode_attention(q, kp2, vp2, ip, ix, d**-0.5, kv_scale=sc2, new_kv=(k_new, v_new, out_loc),
                                   max_seq_len=int(c.lens.max()))
    one = ops.paged_decode_attention(q, kp, vp, ip, ix, d**-0.5, kv_scale=sc, max_splits=1)
    torch.cuda.synchronize()
    assert torch.equal(a, f), "fused store != store + decode"
    assert torch.equal(kp.view(torch.uint8), kp2.view(torch.uint8)) and torch.equal(sc, sc2)
    assert_close(a, to_np64(one), torch.bfloat16, "key ranges vs unsplit")


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (32, 8, 128), (8, 8, 64), (16, 2, 256), (64, 8, 128),
                                      (24, 12, 128), (32, 16, 64)])
@pytest.mark.parametrize("planned", [False, True])
def test_fp8_fused_store_decode_bit_exact(cuda_device, dt, hq, hkv, d, planned):
    """msgl_paged_decode_store_fp8 (the new token quantised and stored inside the
    decode launch) against msgl_store_kv_fp8 followed by msgl_paged_decode_fp8:
    output, codes and scales bit for bit, for single- and multi-chunk requests
    and a request whose only token is the new one; a slot outside the pool is
    skipped by both."""
    dtype = DTYPES[dt]
    lens = [1, 2, 17, 64, 65, 700, 2500]
    n = 16384
    c = workloads.decode_case_from_lens(lens, num_slots=n, seed=11)
    b = len(lens)
    q = randn((b, hq, d), 400, dtype).to(cuda_device)
    g = torch.Generator(device=cuda_device).manual_seed(401)
    k_new = (torch.randn((b, hkv, d), generator=g, device=cuda_device) *
             torch.exp(torch.randn((b, hkv, 1), generator=g, device=cuda_device))).to(dtype)
    v_new = (torch.randn((b, hkv, d), generator=g, device=cuda_device) *
             torch.exp(torch.randn((b, hkv, 1), generator=g, device=cuda_device))).to(dtype)
    k_new[3, 0] = 0  # a row of zeros: +0 codes, scale 0
    out_loc = i32(c.out_loc, cuda_device)
    ip, ix = i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device)
    for splits in (1, None, 16):
        kp, vp, sc, _, _ = _fp8_pools(n, hkv, d, 402, cuda_device)
        kp2, vp2, sc2 = kp.clone(), vp.clone(), sc.clone()
        msplits = splits if splits is not None else ops.default_splits(b, hkv, max(lens))
        ws = ops.decode_workspace(b, hq, hkv, d, msplits, cuda_device)
        print(f"case fp8 fused store {hq}/{hkv}/{d} {dt} planned={planned} splits={splits}", flush=True)
        ops.store_kv_fp8(k_new, v_new, out_loc, kp, vp, sc)
        a = ops.paged_decode_attention(q, kp, vp, ip, ix, d**-0.5, max_splits=msplits, kv_scale=sc)
        if planned:
            ops.paged_decode_plan(ip, None, b, hq, hkv, d, msplits, ws)
        f = ops.paged_decode_attention(q, kp2, vp2, ip, ix, d**-0.5, max_splits=msplits, kv_scale=sc2,
                                       new_kv=(k_new, v_new, out_loc), workspace=ws, planned=planned)
        torch.cuda.synchronize()
        assert torch.equal(a, f), f"output splits={splits}"
        assert torch.equal(kp.view(torch.uint8), kp2.view(torch.uint8)), "K codes"
        assert torch.equal(vp.view(torch.uint8), vp2.view(torch.uint8)), "V codes"
        assert torch.equal(sc, sc2), "scales"
    # out_loc outside the pool: neither form writes anything
    bad = out_loc.clone()
    bad[2] = n + 5
    kp, vp, sc, _, _ = _fp8_pools(n, hkv, d, 403, cuda_device)
    before = (kp.view(torch.uint8).clone(), vp.view(torch.uint8).clone(), sc.clone())
    ops.paged_decode_attention(q, kp, vp, ip, ix, d**-0.5, kv_scale=sc, new_kv=(k_new, v_new, bad))
    torch.cuda.synchronize()
    changed = (kp.view(torch.uint8) != before[0]).any(dim=(1, 2)).nonzero().flatten().tolist()
    assert sorted(changed) == sorted(int(x) for i, x in enumerate(c.out_loc) if i != 2)
    assert torch.equal(sc[n - 1], before[2][n - 1])


def test_fp8_decode_headline_batch(cuda_device):
    """The headline decode shape (batch 128, L ~ U[200, 2048], 262144-slot pool) over an fp8 pool:
    sampled requests vs the oracle, and the quantisation error against the unquantised decode."""
    c = workloads.decode_case(128, 200, 2048, 262144, 1, seed=0)
    kp, vp, sc, k_src, v_src = _fp8_pools(262144, 8, 128, 400, cuda_device, spread=0)
    q = randn((128, 16, 128), 401, torch.bfloat16).to(cuda_device)
    ip, ix = i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device)
    print("case fp8 headline", flush=True)
    out = ops.paged_decode_attention(q, kp, vp, ip, ix, 128**-0.5, kv_scale=sc)
    exact = ops.paged_decode_attention(q, k_src, v_src, ip, ix, 128**-0.5)
    torch.cuda.synchronize()
    for b in (0, 17, 64, 127):
        s, e = int(c.kv_indptr[b]), int(c.kv_indptr[b + 1])
        slots = torch.from_numpy(c.kv_indices[s:e].astype(np.int64)).to(cuda_device)
        kb = oracle.dequantize_fp8(_codes(kp[slots]), sc[slots][..., 0].cpu().numpy())
        vb = oracle.dequantize_fp8(_codes(vp[slots]), sc[slots][..., 1].cpu().numpy())
        ref = oracle.paged_decode(to_np64(q[b:b + 1]), kb, vb, np.array([0, e - s]), np.arange(e - s), 128**-0.5)
        assert_close(out[b:b + 1], ref, torch.bfloat16, f"fp8 headline request {b}")
    # e4m3 keeps 3 mantissa bits: outputs stay within a few percent of the unquantised decode
    rel = ((out.float() - exact.float()).norm() / exact.float().norm()).item()
    print(f"fp8 vs bf16 decode relative error {rel:.4f}", flush=True)
    assert rel < 0.05


def _fp8_prefill(case, hq, hkv, d, dt, device, seed, splits=None, page_size=1, planned=False):
    """Quantise a random pool (prefix rows) and this step's rows into fp8, then run
    the ragged prefill over it; returns (q, kp, vp, kv_scale, out)."""
    n = case.num_slots
    # P enters the matrix core in 16 bits, so the output error scales with max |V|: moderate row spread
    kp, vp, sc, _, _ = _fp8_pools(n, hkv, d, seed, device, spread=0.5)
    q = randn((case.num_tokens, hq, d), seed + 2, dt).to(device)
    knew = randn((case.num_tokens, hkv, d), seed + 3, dt).to(device)
    vnew = randn((case.num_tokens, hkv, d), seed + 4, dt).to(device)
    ops.store_kv_fp8(knew, vnew, i32(case.out_loc, device), kp, vp, sc)
    if page_size == 1:
        kv_indptr, kv_indices, seq = case.kv_indptr, case.kv_indices, None
    else:
        pages = [case.page_table[i, : int(L)][::page_size] // page_size for i, L in enumerate(case.seq_lens)]
        kv_indptr = np.concatenate([[0], np.cumsum([len(x) for x in pages])]).astype(np.int32)
        kv_indices = np.concatenate(pages).astype(np.int32)
        seq = case.seq_lens
    args = (q, kp, vp, i32(case.q_indptr, device), i32(kv_indptr, device), i32(kv_indices, device),
            None if seq is None else i32(seq, device), d**-0.5)
    maxe, maxs = int(case.extend_lens.max()), int(case.seq_lens.max())
    if splits is None:
        splits = ops.prefill_default_splits(len(case.seq_lens), hq, hkv, d, maxe, maxs)
    ws = ops.prefill_workspace(len(case.seq_lens), case.num_tokens, maxe, hq, hkv, d, splits, device)
    if planned:
        ops.prefill_plan(args[3], args[4], args[6], num_tokens=case.num_tokens, max_extend_len=maxe,
                         max_seq_len=maxs, num_qo_heads=hq, num_kv_heads=hkv, head_dim=d, dtype=dt,
                         max_splits=splits, workspace=ws)
    out = ops.prefill_ragged_attention(*args, max_extend_len=maxe, max_seq_len=maxs, page_size=page_size,
                                       max_splits=splits, workspace=ws, planned=planned, kv_scale=sc)
    torch.cuda.synchronize()
    return q, kp, vp, sc, out


def _fp8_prefill_oracle(case, q, kp, vp, sc, d):
    kvi = [case.kv_indices[case.kv_indptr[i]: case.kv_indptr[i + 1]] for i in range(len(case.seq_lens))]
    return oracle.forward_prefill(to_np64(q), None, None, _deq(kp, sc, 0), _deq(vp, sc, 1),
                                  case.q_indptr.tolist(), kvi, d**-0.5)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (32, 8, 128), (8, 8, 64), (16, 2, 256)])
@pytest.mark.parametrize("splits", [1, 4])
def test_fp8_prefill_grid(cuda_device, dt, hq, hkv, d, splits):
    """Prefix P in {0,1,17,300,0}, extend E in {1,2,64,100,37} over fp8 pools (the
    step's rows quantised by the fp8 store first)."""
    dtype = DTYPES[dt]
    case = workloads.prefill_case_from_lens([0, 1, 17, 300, 0], [1, 2, 64, 100, 37], num_slots=2048, seed=3)
    print(f"case fp8 prefill grid {hq}/{hkv}/{d} {dt} splits={splits}", flush=True)
    q, kp, vp, sc, out = _fp8_prefill(case, hq, hkv, d, dtype, cuda_device, 10, splits=splits)
    assert_close(out, _fp8_prefill_oracle(case, q, kp, vp, sc, d), dtype, f"fp8 prefill {hq}/{hkv}/{d} {dt}")


def test_fp8_prefill_page16_and_planned(cuda_device):
    case = workloads.prefill_case_from_lens([0, 15, 16, 40, 333, 1500], [5, 1, 33, 100, 64, 300], num_slots=8192,
                                            page_size=16, seed=4)
    print("case fp8 prefill page16", flush=True)
    q, kp, vp, sc, out = _fp8_prefill(case, 32, 8, 128, torch.bfloat16, cuda_device, 20, page_size=16)
    assert_close(out, _fp8_prefill_oracle(case, q, kp, vp, sc, 128), torch.bfloat16, "fp8 prefill page16")
    _, _, _, _, out2 = _fp8_prefill(case, 32, 8, 128, torch.bfloat16, cuda_device, 20, page_size=16, planned=True)
    assert torch.equal(out, out2), "planned fp8 prefill differs"


def test_fp8_prefill_workload(cuda_device):
    """The 16-request prefill workload over an fp8 pool: sampled requests vs the oracle."""
    case = workloads.prefill_case(16, 4096, 64, 512, 2048, num_slots=1 << 17, seed=0)
    print("case fp8 prefill workload", flush=True)
    q, kp, vp, sc, out = _fp8_prefill(case, 16, 8, 128, torch.bfloat16, cuda_device, 30)
    for i in (0, 7, 15):
        s, e = int(case.q_indptr[i]), int(case.q_indptr[i + 1])
        slots = torch.from_numpy(case.kv_indices[case.kv_indptr[i]: case.kv_indptr[i + 1]].astype(np.int64))
        slots = slots.to(cuda_device)
        kb = oracle.dequantize_fp8(_codes(kp[slots]), sc[slots][..., 0].cpu().numpy())
        vb = oracle.dequantize_fp8(_codes(vp[slots]), sc[slots][..., 1].cpu().numpy())
        ref = oracle.forward_prefill(to_np64(q[s:e]), None, None, kb, vb, [0, e - s], [np.arange(len(slots))],
                                     128**-0.5)
        assert_close(out[s:e], ref, torch.bfloat16, f"fp8 prefill workload request {i}")


def test_backend_with_fp8_cache(cuda_device):
    """The attention layer and hip backend over an fp8 KV cache (layers.py:103-111 order:
    rotate, quantising store, attention): a chunked prefill with a cached prefix,
    then a decode step, vs the oracle over the dequantised pool."""
    from minisgl_hip.attention import create_attention_backend
    from minisgl_hip.core import Batch, Context, ModelConfig, Req, RotaryConfig, set_global_ctx
    from minisgl_hip.kvcache import MHAKVCache
    from minisgl_hip.layers import AttentionLayer

    dt = torch.bfloat16
    cfg = ModelConfig(num_qo_heads=16, num_kv_heads=8, head_dim=128, num_layers=2)
    kv = MHAKVCache(2, 8192, 8, 128, dt, cuda_device, kv_dtype=FP8)
    assert kv.quantized and kv.k[0].dtype == FP8 and kv.kv_scale[0].shape == (8192, 8, 2)
    table = np.zeros((8, 1024), dtype=np.int32)
    backend = create_attention_backend("hip", cfg, kv, table)
    ctx = Context(page_size=1)
    ctx.page_table, ctx.kv_cache, ctx.attn_backend = table, kv, backend
    layers = [AttentionLayer(i, 16, 8, 128, RotaryConfig(head_dim=128, rotary_dim=128, base=1e6), cuda_device)
              for i in range(2)]
    set_global_ctx(ctx)
    try:
        free = np.random.default_rng(30).permutation(8192).astype(np.int32)
        reqs = [Req(input_ids=np.zeros(50, np.int32), table_idx=0, cached_len=20),
                Req(input_ids=np.zeros(33, np.int32), table_idx=1, cached_len=0)]
        free = oracle.allocate_paged(table, free, [0, 1], [0, 0], [50, 33], 1)
        all_slots = torch.arange(8192, dtype=torch.int32, device=cuda_device)
        for layer in range(2):  # the cached prefix: quantised rows in every slot
            kv.store_kv(randn((8192, 8, 128), 31 + layer, dt).to(cuda_device),
                        randn((8192, 8, 128), 33 + layer, dt).to(cuda_device), all_slots, layer)
        inv = oracle.rope_inv_freq(128, 1e6)
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
                    print(f"case fp8 backend {phase} layer={layer}", flush=True)
                    o = layers[layer](q, k, v)
                    torch.cuda.synchronize()
                    kp, vp = _deq(kv.k[layer], kv.kv_scale[layer], 0), _deq(kv.v[layer], kv.kv_scale[layer], 1)
                    # the step's rows were quantised from the rotated k and the raw v
                    kc, _ = oracle.quantize_fp8(oracle.rope(to_np64(k), pos, 128, inv).astype(np.float32))
                    vc, _ = oracle.quantize_fp8(to_np64(v).astype(np.float32))
                    assert (np.abs(oracle.e4m3_decode(_codes(kv.k[layer])[out_loc]).astype(np.float64)
                                   - oracle.e4m3_decode(kc)) <= np.abs(oracle.e4m3_decode(kc)) / 8 + 1e-6).all()
                    np.testing.assert_array_equal(_codes(kv.v[layer])[out_loc], vc)
                    q_rot = oracle.rope(to_np64(q), pos, 128, inv)
                    if phase == "prefill":
                        offs = np.concatenate([[0], np.cumsum(np.array(dlen) - np.array(cached))])
                        ref = oracle.forward_prefill(q_rot, None, None, kp, vp, offs,
                                                     [table[r, :d] for r, d in zip(rows, dlen)], 128**-0.5)
                    else:
                        kvi, mask = oracle.naive_decode_metadata(table, rows, dlen)
                        ref = oracle.naive_forward_decode(q_rot, kp, vp, kvi, mask, 128**-0.5)
                    assert_close(o.view(t, 16, 128), ref, dt, f"fp8 backend {phase} {layer}")
            for r in reqs:
                r.complete_one()
    finally:
        set_global_ctx(None)


@pytest.mark.parametrize("splits", [1, 3])
def test_fp8_prefill_requests_without_extend(cuda_device, splits):
    """fp8 pools: requests with no extend tokens between real ones leave the
    other requests' outputs equal to the oracle's."""
    case = workloads.prefill_case_from_lens([100, 50, 0, 20, 2000], [37, 0, 5, 0, 130], num_slots=8192, seed=5)
    print(f"case fp8 prefill empty extends splits={splits}", flush=True)
    q, kp, vp, sc, out = _fp8_prefill(case, 16, 8, 128, torch.bfloat16, cuda_device, 70, splits=splits)
    assert_close(out, _fp8_prefill_oracle(case, q, kp, vp, sc, 128), torch.bfloat16, "fp8 prefill empty extends")
