"""Seeded random continuous-batching steps through the mixed-step runner
(decode requests first, then prefill chunks over cached prefixes; indices
built on the GPU from the page table): query-head groups 1 to 8 and 16,
head_dim 64/128/256, fp32/bf16/fp16, page 1 or 16, decode-only and
prefill-only batches, ragged chunk lengths (single-token chunks included) and
split settings. The single launch, or the phase launches msgl_mixed_attention
falls back to for shapes it is not built for, must equal the phases run one
after the other bit for bit: pools, prefill rows, and decode rows when the
decode splits (with one split the separate decode call runs its shared-head
form, which sums in another order). Both forms must match the float64 oracle
request by request: decode as attention/naive.py:50-60, prefill chunks as
attention/base.py:85-105, the step's KV rows as kvcache/pool.py:47-50."""

import numpy as np
import pytest
import torch

import oracle
from gpu_util import DTYPES, assert_close, i32, randn, to_np64
from minisgl_hip import workloads
from minisgl_hip.mixed import MixedStep

pytestmark = pytest.mark.gpu


def _case(seed):
    rng = np.random.default_rng(3000 + seed)
    g = int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 16]))
    hkv = int(rng.choice([1, 2, 4, 8] if g <= 4 else [1, 2, 4]))
    d = int(rng.choice([64, 128, 128, 256]))
    dtype = str(rng.choice(["f32", "bf16", "bf16", "f16"]))
    page = int(rng.choice([1, 16]))
    nd = int(rng.integers(0, 13))
    npf = int(rng.integers(0 if nd else 1, 5))
    prefixes = rng.integers(0, 1200, npf)
    prefixes[rng.random(npf) < 0.3] = 0
    chunks = rng.integers(1, 160, npf)
    chunks[rng.random(npf) < 0.2] = 1
    dec_splits = [None, 1, 4][int(rng.integers(3))]
    pf_splits = [None, 1, 3][int(rng.integers(3))]
    return g * hkv, hkv, d, dtype, page, nd, prefixes, chunks, dec_splits, pf_splits


def _rows(pool, slots):
    return to_np64(pool.index_select(0, torch.from_numpy(np.asarray(slots, np.int64)).to(pool.device)))


@pytest.mark.parametrize("seed", range(16))
def test_random_mixed_step(cuda_device, seed):
    hq, hkv, d, dtype, page, nd, prefixes, chunks, dec_splits, pf_splits = _case(seed)
    dt = DTYPES[dtype]
    print(f"case random mixed seed={seed} {hq}/{hkv}/{d} {dtype} page={page} decode={nd} "
          f"P={prefixes.tolist()} E={chunks.tolist()} splits={dec_splits}/{pf_splits}", flush=True)
    case = workloads.mixed_case(nd, 1, 1500, prefixes, chunks, num_slots=65536, page_size=page, seed=seed)
    kp = randn((case.num_slots, hkv, d), 900 + seed, dt).to(cuda_device)
    vp = randn((case.num_slots, hkv, d), 950 + seed, dt).to(cuda_device)
    t = case.num_tokens
    q = randn((t, hq, d), 1000 + seed, dt).to(cuda_device)
    kn = randn((t, hkv, d), 1050 + seed, dt).to(cuda_device)
    vn = randn((t, hkv, d), 1100 + seed, dt).to(cuda_device)
    step = MixedStep(
        i32(case.req_to_token, cuda_device), case.table_idx, case.cached_len, case.device_len,
        num_decode=nd, num_qo_heads=hq, num_kv_heads=hkv, head_dim=d, page_size=page,
        decode_splits=dec_splits, prefill_splits=pf_splits,
    )
    scale = d**-0.5
    kp1, vp1 = kp.clone(), vp.clone()
    a = torch.empty_like(q)
    step.run(q, kn, vn, kp, vp, a, scale, concurrent=False, single_launch=False)
    b = torch.empty_like(q)
    step.run(q, kn, vn, kp1, vp1, b, scale, single_launch=True)
    torch.cuda.synchronize()
    assert torch.equal(kp, kp1) and torch.equal(vp, vp1)
    t0 = 0
    for i in range(case.num_reqs):
        e = int(case.device_len[i] - case.cached_len[i])
        slots = case.slots(i)
        loc = torch.from_numpy(np.asarray(slots[-e:], np.int64)).to(cuda_device)
        assert torch.equal(kp.index_select(0, loc), kn[t0 : t0 + e]), f"request {i}: K rows not stored"
        assert torch.equal(vp.index_select(0, loc), vn[t0 : t0 + e]), f"request {i}: V rows not stored"
        kb, vb = _rows(kp, slots), _rows(vp, slots)
        if i < nd:
            ref = oracle.paged_decode(to_np64(q[t0 : t0 + 1]), kb, vb, np.array([0, len(slots)]),
                                      np.arange(len(slots)), scale)
        else:
            ref = oracle.forward_prefill(to_np64(q[t0 : t0 + e]), None, None, kb, vb, [0, e],
                                         [np.arange(len(slots))], scale)
        for form, out in (("single launch", b), ("phases", a)):
            assert_close(out[t0 : t0 + e], ref, dt, f"random mixed seed={seed} request {i} ({form})")
        if i >= nd or step.decode_splits > 1:
            assert torch.equal(a[t0 : t0 + e], b[t0 : t0 + e]), f"request {i}: the forms differ"
        t0 += e
