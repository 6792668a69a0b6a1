"""Query-head groups beyond the powers of two up to 8, which the reference's
kernel takes as any integer ratio (attention/metal.py:122 asserts only
Hq % Hkv == 0; GQA maps q-head h to kv-head h // G, attention/naive.py:50-60):
- Hq / Hkv = 3, 5, 6, 7 through decode, fused store, planned decode, ragged
  prefill (one pass and key-range splits, 16-bit and fp32), fp8 pools and the
  single-launch mixed step. A prefill workgroup holds floor(128 / G) tokens of
  G heads; its remaining rows are padding that is computed and never stored.
- the layouts the decode runs over virtual kv heads (groups of 16, 32 and 64
  as groups of 8; a group of 8 over one or two kv heads as groups of 4): decode
  in every dtype, the fused store, a stored plan and the separate merge, a
  million keys in equal key ranges, fp8 pools.
Each case is checked against the float64 oracle or bit for bit against the
calls it replaces."""

import numpy as np
import pytest
import torch

import oracle
from gpu_util import DTYPES, assert_close, i32, randn, to_np64
from minisgl_hip import ops, workloads
from minisgl_hip.mixed import MixedStep
from test_kvquant_gpu import _deq, _fp8_pools, _fp8_prefill, _fp8_prefill_oracle
from test_mixed_gpu import _check_request
from test_prefill_gpu import _oracle as _prefill_oracle
from test_prefill_gpu import _run as _prefill_run

pytestmark = pytest.mark.gpu

# (Hq, Hkv, D): Llama-3.2-3B (G 3), Qwen3-14B (G 5), Qwen2.5-1.5B (G 6), Qwen2.5-7B (G 7), Qwen2.5-0.5B (G 7)
GROUPS = [(24, 8, 128), (40, 8, 128), (12, 2, 128), (28, 4, 128), (14, 2, 64)]


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("hq,hkv,d", GROUPS)
@pytest.mark.parametrize("splits", [1, None])
def test_decode_groups(cuda_device, hq, hkv, d, dtype, splits):
    """tests/test_attention.py:19-39's batch (lens [1,2,17,31,32,33,700], N=4096)."""
    dt = DTYPES[dtype]
    c = workloads.reference_test_case()
    kp = randn((4096, hkv, d), 300, dt).to(cuda_device)
    vp = randn((4096, hkv, d), 301, dt).to(cuda_device)
    q = randn((7, hq, d), 302, dt).to(cuda_device)
    print(f"case decode groups {hq}/{hkv}/{d} {dtype} splits={splits}", flush=True)
    out = ops.paged_decode_attention(q, kp, vp, i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device),
                                     d**-0.5, max_splits=splits)
    torch.cuda.synchronize()
    ref = oracle.paged_decode(to_np64(q), to_np64(kp), to_np64(vp), c.kv_indptr, c.kv_indices, d**-0.5)
    assert_close(out, ref, dt, f"decode groups {hq}/{hkv}/{d} {dtype} splits={splits}")


@pytest.mark.parametrize("hq,hkv,d", GROUPS)
def test_decode_groups_fused_store_and_planned(cuda_device, hq, hkv, d):
    """The fused store + decode equals the store then the decode, and a plan built
    once equals the self-planning call, bit for bit (bf16, lengths across tiles)."""
    dt = torch.bfloat16
    lens = [1, 2, 17, 64, 65, 300, 1000, 2500]
    c = workloads.decode_case_from_lens(lens, num_slots=8192, seed=23)
    kp = randn((8192, hkv, d), 310, dt).to(cuda_device)
    vp = randn((8192, hkv, d), 311, dt).to(cuda_device)
    q = randn((len(lens), hq, d), 312, dt).to(cuda_device)
    kn = randn((len(lens), hkv, d), 313, dt).to(cuda_device)
    vn = randn((len(lens), hkv, d), 314, dt).to(cuda_device)
    loc = i32(c.out_loc, cuda_device)
    indptr, indices = i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device)
    kp2, vp2 = kp.clone(), vp.clone()
    print(f"case decode groups fused/planned {hq}/{hkv}/{d}", flush=True)
    fused = ops.paged_decode_attention(q, kp, vp, indptr, indices, d**-0.5, max_splits=4, new_kv=(kn, vn, loc))
    ops.store_kv(kn, vn, loc, kp2, vp2)
    two = ops.paged_decode_attention(q, kp2, vp2, indptr, indices, d**-0.5, max_splits=4)
    ws = ops.decode_workspace(len(lens), hq, hkv, d, 4, cuda_device)
    ops.paged_decode_plan(indptr, None, len(lens), hq, hkv, d, 4, ws)
    planned = ops.paged_decode_attention(q, kp2, vp2, indptr, indices, d**-0.5, max_splits=4, workspace=ws,
                                         planned=True)
    torch.cuda.synchronize()
    assert torch.equal(kp.view(torch.int16), kp2.view(torch.int16))
    assert torch.equal(vp.view(torch.int16), vp2.view(torch.int16))
    assert torch.equal(fused, two)
    assert torch.equal(planned, two)
    ref = oracle.paged_decode(to_np64(q), to_np64(kp2), to_np64(vp2), c.kv_indptr, c.kv_indices, d**-0.5)
    assert_close(fused, ref, dt, f"fused decode groups {hq}/{hkv}/{d}")


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("hq,hkv,d", GROUPS)
def test_prefill_groups(cuda_device, hq, hkv, d, dtype):
    """Prefix P in {0,1,17,300,0}, extend E in {1,2,64,100,37} (E == 1, P == 0, causal edges)."""
    dt = DTYPES[dtype]
    case = workloads.prefill_case_from_lens([0, 1, 17, 300, 0], [1, 2, 64, 100, 37], num_slots=2048, seed=3)
    print(f"case prefill groups {hq}/{hkv}/{d} {dtype}", flush=True)
    q, kn, vn, kp, vp, out = _prefill_run(case, hq, hkv, d, dt, cuda_device, 40)
    assert_close(out, _prefill_oracle(case, q, kn, vn, kp, vp, d), dt, f"prefill groups {hq}/{hkv}/{d} {dtype}")


@pytest.mark.parametrize("hq,hkv,d", GROUPS)
@pytest.mark.parametrize("splits", [1, 3])
def test_prefill_groups_key_splits(cuda_device, hq, hkv, d, splits):
    """Extends that end inside, at and past the floor(128 / G)-token block edges,
    over prefixes long enough for key-range chunks (merged from fp32 partials)."""
    dt = torch.bfloat16
    g = hq // hkv
    bq = 128 // g
    extend = [bq - 1, bq, bq + 1, 3 * bq + 2, 130]
    case = workloads.prefill_case_from_lens([700, 1500, 0, 2100, 257], extend, num_slots=16384, seed=g)
    maxe, maxs = int(case.extend_lens.max()), int(case.seq_lens.max())
    kp = randn((case.num_slots, hkv, d), 320, dt).to(cuda_device)
    vp = randn((case.num_slots, hkv, d), 321, dt).to(cuda_device)
    q = randn((case.num_tokens, hq, d), 322, dt).to(cuda_device)
    print(f"case prefill groups splits {hq}/{hkv}/{d} splits={splits}", flush=True)
    out = ops.prefill_ragged_attention(q, kp, vp, i32(case.q_indptr, cuda_device), i32(case.kv_indptr, cuda_device),
                                       i32(case.kv_indices, cuda_device), None, d**-0.5, max_extend_len=maxe,
                                       max_seq_len=maxs, max_splits=splits)
    torch.cuda.synchronize()
    kvi = [case.kv_indices[case.kv_indptr[i]: case.kv_indptr[i + 1]] for i in range(len(case.seq_lens))]
    ref = oracle.forward_prefill(to_np64(q), None, None, to_np64(kp), to_np64(vp), case.q_indptr.tolist(), kvi,
                                 d**-0.5)
    assert_close(out, ref, dt, f"prefill groups {hq}/{hkv}/{d} splits={splits}")


@pytest.mark.parametrize("hq,hkv,d", GROUPS)
@pytest.mark.parametrize("splits", [1, 4])
def test_fp8_groups(cuda_device, hq, hkv, d, splits):
    """fp8 pools: decode over the reference batch and the ragged prefill grid."""
    dt = torch.bfloat16
    c = workloads.reference_test_case()
    kp, vp, sc, _, _ = _fp8_pools(4096, hkv, d, 330, cuda_device)
    q = randn((7, hq, d), 332, dt).to(cuda_device)
    print(f"case fp8 groups {hq}/{hkv}/{d} splits={splits}", flush=True)
    out = ops.paged_decode_attention(q, kp, vp, i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device),
                                     d**-0.5, max_splits=splits, kv_scale=sc)
    torch.cuda.synchronize()
    ref = oracle.paged_decode(to_np64(q), _deq(kp, sc, 0), _deq(vp, sc, 1), c.kv_indptr, c.kv_indices, d**-0.5)
    assert_close(out, ref, dt, f"fp8 decode groups {hq}/{hkv}/{d} splits={splits}")
    case = workloads.prefill_case_from_lens([0, 1, 17, 300, 0], [1, 2, 64, 100, 37], num_slots=2048, seed=3)
    q, kp, vp, sc, out = _fp8_prefill(case, hq, hkv, d, dt, cuda_device, 40, splits=splits)
    assert_close(out, _fp8_prefill_oracle(case, q, kp, vp, sc, d), dt, f"fp8 prefill groups {hq}/{hkv}/{d}")


@pytest.mark.parametrize("hq,hkv,d", [(24, 8, 128), (40, 8, 128), (28, 4, 128), (14, 2, 64), (32, 2, 128),
                                     (16, 2, 128)])
def test_mixed_groups(cuda_device, hq, hkv, d):
    """msgl_mixed_attention: bit-identical to the decode and prefill calls run in
    turn; every request against the oracle (head_dim 128)."""
    case = workloads.mixed_case(6, 20, 900, [0, 100, 1500], 96, num_slots=32768, page_size=16, seed=hq + d)
    dt = torch.bfloat16
    print(f"case mixed groups {hq}/{hkv}/{d}", flush=True)
    kp = randn((case.num_slots, hkv, d), 340, dt).to(cuda_device)
    vp = randn((case.num_slots, hkv, d), 341, dt).to(cuda_device)
    t = case.num_tokens
    q = randn((t, hq, d), 342, dt).to(cuda_device)
    kn = randn((t, hkv, d), 343, dt).to(cuda_device)
    vn = randn((t, hkv, d), 344, dt).to(cuda_device)
    step = MixedStep(
        i32(case.req_to_token, cuda_device), case.table_idx, case.cached_len, case.device_len,
        num_decode=case.num_decode, num_qo_heads=hq, num_kv_heads=hkv, head_dim=d, page_size=16,
    )
    kp1, vp1 = kp.clone(), vp.clone()
    a = torch.empty_like(q)
    step.run(q, kn, vn, kp, vp, a, d**-0.5, concurrent=False, single_launch=False)
    b = torch.empty_like(q)
    step.run(q, kn, vn, kp1, vp1, b, d**-0.5, single_launch=True)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(kp, kp1) and torch.equal(vp, vp1)
    if d == 128:
        for i in range(case.num_reqs):
            _check_request(case, i, q, kp, vp, b)


# Layouts the decode runs over virtual kv heads sharing their pool head's rows:
# groups above 8 that are multiples of 8 as groups of 8 (Qwen3-235B-A22B's 64 q
# / 4 kv, G 16 at head_dim 64, G 32 and 64), and groups of 8 over one or two
# pool heads as groups of 4 over twice the heads (Qwen2.5-3B's 16 / 2, 8 / 1).
LARGE = [(64, 4, 128), (32, 2, 64), (32, 1, 256), (64, 2, 128), (64, 1, 64), (16, 2, 128), (8, 1, 64)]


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("hq,hkv,d", LARGE)
@pytest.mark.parametrize("splits", [1, None])
def test_decode_large_groups(cuda_device, hq, hkv, d, dtype, splits):
    """tests/test_attention.py:19-39's batch (lens [1,2,17,31,32,33,700], N=4096)."""
    dt = DTYPES[dtype]
    c = workloads.reference_test_case()
    kp = randn((4096, hkv, d), 350, dt).to(cuda_device)
    vp = randn((4096, hkv, d), 351, dt).to(cuda_device)
    q = randn((7, hq, d), 352, dt).to(cuda_device)
    print(f"case decode large groups {hq}/{hkv}/{d} {dtype} splits={splits}", flush=True)
    out = ops.paged_decode_attention(q, kp, vp, i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device),
                                     d**-0.5, max_splits=splits)
    torch.cuda.synchronize()
    ref = oracle.paged_decode(to_np64(q), to_np64(kp), to_np64(vp), c.kv_indptr, c.kv_indices, d**-0.5)
    assert_close(out, ref, dt, f"decode large groups {hq}/{hkv}/{d} {dtype} splits={splits}")


@pytest.mark.parametrize("hq,hkv,d", LARGE)
def test_decode_large_groups_store_plan_merge(cuda_device, hq, hkv, d):
    """Bit for bit (bf16, lengths across tiles, page 16): the fused store + decode
    equals the store then the decode (the pools included), a plan built once
    equals the self-planning call, and the decode launch without its merge
    followed by the separate merge equals the call with it."""
    dt = torch.bfloat16
    lens = [1, 2, 17, 64, 65, 300, 1000, 2500]
    c = workloads.decode_case_from_lens(lens, num_slots=8192, page_size=16, seed=29)
    kp = randn((8192, hkv, d), 360, dt).to(cuda_device)
    vp = randn((8192, hkv, d), 361, dt).to(cuda_device)
    q = randn((len(lens), hq, d), 362, dt).to(cuda_device)
    kn = randn((len(lens), hkv, d), 363, dt).to(cuda_device)
    vn = randn((len(lens), hkv, d), 364, dt).to(cuda_device)
    loc = i32(c.out_loc, cuda_device)
    indptr, pages, sl = i32(c.page_indptr, cuda_device), i32(c.page_ids, cuda_device), i32(c.lens, cuda_device)
    kw = dict(seq_lens=sl, page_size=16, max_splits=4)
    kp2, vp2 = kp.clone(), vp.clone()
    print(f"case decode large groups store/plan/merge {hq}/{hkv}/{d}", flush=True)
    fused = ops.paged_decode_attention(q, kp, vp, indptr, pages, d**-0.5, new_kv=(kn, vn, loc), **kw)
    ops.store_kv(kn, vn, loc, kp2, vp2)
    two = ops.paged_decode_attention(q, kp2, vp2, indptr, pages, d**-0.5, **kw)
    ws = ops.decode_workspace(len(lens), hq, hkv, d, 4, cuda_device)
    ops.paged_decode_plan(indptr, sl, len(lens), hq, hkv, d, 4, ws)
    planned = ops.paged_decode_attention(q, kp2, vp2, indptr, pages, d**-0.5, workspace=ws, planned=True, **kw)
    apart = ops.paged_decode_attention(q, kp2, vp2, indptr, pages, d**-0.5, workspace=ws, planned=True, merge=False,
                                       **kw)
    ops.paged_decode_merge(apart, indptr, sl, hkv, 4, ws)
    torch.cuda.synchronize()
    assert torch.equal(kp.view(torch.int16), kp2.view(torch.int16))
    assert torch.equal(vp.view(torch.int16), vp2.view(torch.int16))
    assert torch.equal(fused, two) and torch.equal(planned, two) and torch.equal(apart, two)
    ref = oracle.paged_decode(to_np64(q), to_np64(kp2), to_np64(vp2), c.kv_indptr, c.kv_indices, d**-0.5)
    assert_close(fused, ref, dt, f"fused decode large groups {hq}/{hkv}/{d}")


def test_decode_large_group_long_contexts(cuda_device):
    """Qwen3-235B-A22B heads (64 q / 4 kv, head_dim 128, bf16) over about a
    million keys, long enough for equal key ranges: sampled requests vs the
    oracle, and the fused store bit for bit."""
    dt = torch.bfloat16
    hq, hkv, d = 64, 4, 128
    lens = np.random.default_rng(31).integers(6000, 14000, 96)
    n = int(lens.sum()) + 8192
    c = workloads.decode_case_from_lens(lens, num_slots=n, seed=31)
    g = torch.Generator(device=cuda_device).manual_seed(370)  # 1 GB pools: drawn on the device
    kp = torch.randn((n, hkv, d), generator=g, device=cuda_device).to(dt)
    vp = torch.randn((n, hkv, d), generator=g, device=cuda_device).to(dt)
    q = randn((len(lens), hq, d), 372, dt).to(cuda_device)
    kn = randn((len(lens), hkv, d), 373, dt).to(cuda_device)
    vn = randn((len(lens), hkv, d), 374, dt).to(cuda_device)
    loc = i32(c.out_loc, cuda_device)
    print(f"case decode large group long contexts keys={int(lens.sum())}", flush=True)
    out = ops.paged_decode_attention(q, kp, vp, i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device),
                                     d**-0.5, new_kv=(kn, vn, loc))
    torch.cuda.synchronize()
    lo = loc.long()
    assert torch.equal(kp[lo], kn) and torch.equal(vp[lo], vn)
    for b in (0, 17, 50, 95):
        idx = c.kv_indices[c.kv_indptr[b]: c.kv_indptr[b + 1]]
        sel = torch.from_numpy(idx.astype(np.int64)).to(cuda_device)
        ref = oracle.paged_decode(to_np64(q[b: b + 1]), to_np64(kp[sel]), to_np64(vp[sel]),
                                  np.array([0, len(idx)]), np.arange(len(idx)), d**-0.5)
        assert_close(out[b: b + 1], ref, dt, f"decode large group long contexts request {b}")


@pytest.mark.parametrize("hq,hkv,d", [(64, 4, 128), (32, 2, 64), (64, 1, 64), (16, 2, 128)])
@pytest.mark.parametrize("splits", [1, 4])
def test_fp8_decode_large_groups(cuda_device, hq, hkv, d, splits):
    """fp8 pools with groups of 16, 64 and 8 over two heads (virtual kv heads reading their pool
    head's codes and scales): decode over the reference batch against the
    oracle on the dequantised pool, and the fused quantising store + decode
    equal to msgl_store_kv_fp8 then the decode, codes, scales and output bit for
    bit (lengths across tiles, key-range chunks)."""
    dt = torch.bfloat16
    c = workloads.reference_test_case()
    kp, vp, sc, _, _ = _fp8_pools(4096, hkv, d, 380, cuda_device)
    q = randn((7, hq, d), 382, dt).to(cuda_device)
    print(f"case fp8 large groups {hq}/{hkv}/{d} splits={splits}", flush=True)
    out = ops.paged_decode_attention(q, kp, vp, i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device),
                                     d**-0.5, max_splits=splits, kv_scale=sc)
    torch.cuda.synchronize()
    ref = oracle.paged_decode(to_np64(q), _deq(kp, sc, 0), _deq(vp, sc, 1), c.kv_indptr, c.kv_indices, d**-0.5)
    assert_close(out, ref, dt, f"fp8 decode large groups {hq}/{hkv}/{d} splits={splits}")

    lens = [1, 2, 17, 64, 65, 300, 1000, 2500]
    c = workloads.decode_case_from_lens(lens, num_slots=8192, seed=37)
    kp, vp, sc, _, _ = _fp8_pools(8192, hkv, d, 390, cuda_device)
    q = randn((len(lens), hq, d), 392, dt).to(cuda_device)
    kn = randn((len(lens), hkv, d), 393, dt).to(cuda_device)
    vn = randn((len(lens), hkv, d), 394, dt).to(cuda_device)
    loc = i32(c.out_loc, cuda_device)
    indptr, indices = i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device)
    kp2, vp2, sc2 = kp.clone(), vp.clone(), sc.clone()
    fused = ops.paged_decode_attention(q, kp, vp, indptr, indices, d**-0.5, max_splits=splits, kv_scale=sc,
                                       new_kv=(kn, vn, loc))
    ops.store_kv_fp8(kn, vn, loc, kp2, vp2, sc2)
    two = ops.paged_decode_attention(q, kp2, vp2, indptr, indices, d**-0.5, max_splits=splits, kv_scale=sc2)
    torch.cuda.synchronize()
    assert torch.equal(kp.view(torch.uint8), kp2.view(torch.uint8))
    assert torch.equal(vp.view(torch.uint8), vp2.view(torch.uint8))
    assert torch.equal(sc, sc2)
    assert torch.equal(fused, two)
    ref = oracle.paged_decode(to_np64(q), _deq(kp2, sc2, 0), _deq(vp2, sc2, 1), c.kv_indptr, c.kv_indices, d**-0.5)
    assert_close(fused, ref, dt, f"fp8 fused decode large groups {hq}/{hkv}/{d} splits={splits}")
