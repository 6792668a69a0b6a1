"""A continuous-batching step mixing decode and prefill requests (indices built
on the GPU from the page table) vs the float64 oracle, request by request:
decode requests as attention/naive.py:50-60, prefill chunks as
attention/base.py:85-105, the step's KV rows as kvcache/pool.py:47-50."""

import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_close, i32, randn, to_np64
from minisgl_hip import workloads
from minisgl_hip.mixed import MixedStep

pytestmark = pytest.mark.gpu

HQ, HKV, D = 32, 8, 128
SCALE = D**-0.5


def _step(case, device):
    return MixedStep(
        i32(case.req_to_token, device), case.table_idx, case.cached_len, case.device_len,
        num_decode=case.num_decode, num_qo_heads=HQ, num_kv_heads=HKV, head_dim=D, page_size=case.page_size,
    )


def _rows(pool, slots):
    return to_np64(pool.index_select(0, torch.from_numpy(np.asarray(slots, np.int64)).to(pool.device)))


def _check_request(case, i, q, kp, vp, out, rows=None):
    """Request i of the step vs the oracle (rows: extend rows to check, default all)."""
    slots = case.slots(i)
    kb, vb = _rows(kp, slots), _rows(vp, slots)
    t0 = int((case.device_len[:i] - case.cached_len[:i]).sum())
    e = int(case.device_len[i] - case.cached_len[i])
    if i < case.num_decode:
        ref = oracle.paged_decode(to_np64(q[t0 : t0 + 1]), kb, vb, np.array([0, len(slots)]),
                                  np.arange(len(slots)), SCALE)
        assert_close(out[t0 : t0 + 1], ref, torch.bfloat16, f"mixed decode request {i}")
        return
    n = e if rows is None else rows
    # bottom-right causal: query t sees keys <= P + t whatever E is, so the first
    # n rows of the chunk equal a request truncated to n extend tokens
    keep = int(case.cached_len[i]) + n
    ref = oracle.forward_prefill(to_np64(q[t0 : t0 + n]), None, None, kb[:keep], vb[:keep], [0, n],
                                 [np.arange(keep)], SCALE)
    assert_close(out[t0 : t0 + n], ref, torch.bfloat16, f"mixed prefill request {i} rows<{n}")
    # and the chunk's last row sees the whole context (a single query, no mask)
    ref_last = oracle.forward_prefill(to_np64(q[t0 + e - 1 : t0 + e]), None, None, kb, vb, [0, 1],
                                      [np.arange(len(slots))], SCALE)
    assert_close(out[t0 + e - 1 : t0 + e], ref_last, torch.bfloat16, f"mixed prefill request {i} last row")


def test_mixed_step_small(cuda_device):
    """8 decode requests (L in [20, 600]) + chunks of 64 over prefixes 0 and 300, page 16."""
    case = workloads.mixed_case(8, 20, 600, [0, 300], 64, num_slots=16384, page_size=16, seed=7)
    print("case mixed small", flush=True)
    dt = torch.bfloat16
    kp = randn((case.num_slots, HKV, D), 60, dt).to(cuda_device)
    vp = randn((case.num_slots, HKV, D), 61, dt).to(cuda_device)
    t = case.num_tokens
    q = randn((t, HQ, D), 62, dt).to(cuda_device)
    kn = randn((t, HKV, D), 63, dt).to(cuda_device)
    vn = randn((t, HKV, D), 64, dt).to(cuda_device)
    out = torch.empty_like(q)
    kp1, vp1 = kp.clone(), vp.clone()
    step = _step(case, cuda_device)
    step.run(q, kn, vn, kp, vp, out, SCALE, single_launch=False)  # two streams
    out1 = torch.empty_like(q)
    step.run(q, kn, vn, kp1, vp1, out1, SCALE, single_launch=True)
    torch.cuda.synchronize()
    assert torch.equal(out, out1), "the single-launch step differs from the two-stream step"
    assert torch.equal(kp, kp1) and torch.equal(vp, vp1), "the single-launch step stored different rows"
    # the step's rows are in the pool at the slots of positions [cached, device)
    positions, out_loc = oracle.prepare_batch_indices(case.req_to_token, case.table_idx, case.cached_len,
                                                      case.device_len)
    np.testing.assert_array_equal(step.indices["out_loc"].cpu().numpy(), out_loc)
    sl = torch.from_numpy(out_loc.astype(np.int64)).to(cuda_device)
    assert torch.equal(kp.index_select(0, sl), kn) and torch.equal(vp.index_select(0, sl), vn)
    for i in range(case.num_reqs):
        _check_request(case, i, q, kp, vp, out)


def test_mixed_step_full_size(cuda_device):
    """128 decode requests with contexts 512..32768, chunks of 1024 over prefixes 0 and
    8192, Qwen3-8B heads, page 16, a pool of 8M slots (32 GiB): sampled requests."""
    case = workloads.mixed_case(128, 512, 32768, [0, 8192], 1024, num_slots=8 << 20, page_size=16, seed=0)
    print("case mixed full", flush=True)
    dt = torch.bfloat16
    g = torch.Generator(device=cuda_device).manual_seed(70)
    kp = torch.randn((case.num_slots, HKV, D), generator=g, device=cuda_device, dtype=dt)
    vp = torch.randn((case.num_slots, HKV, D), generator=g, device=cuda_device, dtype=dt)
    t = case.num_tokens
    q = torch.randn((t, HQ, D), generator=g, device=cuda_device, dtype=dt)
    kn = torch.randn((t, HKV, D), generator=g, device=cuda_device, dtype=dt)
    vn = torch.randn((t, HKV, D), generator=g, device=cuda_device, dtype=dt)
    out = torch.empty_like(q)
    step = _step(case, cuda_device)
    step.run(q, kn, vn, kp, vp, out, SCALE, single_launch=False)  # two streams
    out2 = torch.empty_like(q)
    step.run(q, kn, vn, kp, vp, out2, SCALE, single_launch=False)
    out3 = torch.empty_like(q)
    step.run(q, kn, vn, kp, vp, out3, SCALE, concurrent=False, single_launch=False)  # decode, then prefill
    out4 = torch.empty_like(q)
    print("case mixed full single launch", flush=True)
    step.run(q, kn, vn, kp, vp, out4, SCALE, single_launch=True)  # one grid for both
    torch.cuda.synchronize()
    assert torch.equal(out, out2), "mixed step is not deterministic"
    assert torch.equal(out, out3), "the two-stream step differs from the one-stream order"
    # The decode call alone splits this batch (2.2M keys) by equal key ranges; the
    # single launch runs per-request chunks, so the two agree to rounding, not bits
    # (the prefill rows are the same bits).
    np_dec = case.num_decode  # decode rows come first in the packed batch
    assert torch.equal(out[np_dec:], out4[np_dec:]), "single-launch prefill rows differ"
    assert_close(out4[:np_dec], to_np64(out[:np_dec]), dt, "single launch vs decode call")
    longest = int(np.argmax(case.device_len[: case.num_decode]))
    for i in sorted({0, 5, longest, case.num_decode - 1}):
        _check_request(case, i, q, kp, vp, out)
    for i in (case.num_decode, case.num_decode + 1):
        _check_request(case, i, q, kp, vp, out, rows=64)
    del kp, vp
    torch.cuda.empty_cache()


@pytest.mark.parametrize("hq,hkv,d,page", [(16, 8, 128, 1), (32, 8, 128, 16), (8, 2, 64, 1), (16, 16, 128, 16)])
def test_mixed_single_launch_shapes(cuda_device, hq, hkv, d, page):
    """msgl_mixed_attention over head groups 1..4, head_dim 64/128, pages 1/16, fp16
    and bf16: bit-identical to the decode and prefill calls run in turn, and the
    oracle for every request."""
    case = workloads.mixed_case(6, 20, 900, [0, 100, 1500], 96, num_slots=32768, page_size=page, seed=hq + d)
    for dt in (torch.bfloat16, torch.float16):
        print(f"case mixed single {hq}/{hkv}/{d} page={page} {dt}", flush=True)
        kp = randn((case.num_slots, hkv, d), 80, dt).to(cuda_device)
        vp = randn((case.num_slots, hkv, d), 81, dt).to(cuda_device)
        t = case.num_tokens
        q = randn((t, hq, d), 82, dt).to(cuda_device)
        kn = randn((t, hkv, d), 83, dt).to(cuda_device)
        vn = randn((t, hkv, d), 84, dt).to(cuda_device)
        step = MixedStep(
            i32(case.req_to_token, cuda_device), case.table_idx, case.cached_len, case.device_len,
            num_decode=case.num_decode, num_qo_heads=hq, num_kv_heads=hkv, head_dim=d, page_size=page,
        )
        assert (step.num_tokens, step.num_pages, step.max_chunk) == (t, case.num_pages, case.max_chunk)
        kp1, vp1 = kp.clone(), vp.clone()
        a = torch.empty_like(q)
        step.run(q, kn, vn, kp, vp, a, d**-0.5, concurrent=False, single_launch=False)
        b = torch.empty_like(q)
        step.run(q, kn, vn, kp1, vp1, b, d**-0.5, single_launch=True)
        torch.cuda.synchronize()
        assert torch.equal(a, b) and torch.equal(kp, kp1) and torch.equal(vp, vp1)
        if dt == torch.bfloat16 and hq == HQ and hkv == HKV and d == D:
            for i in range(case.num_reqs):
                _check_request(case, i, q, kp, vp, b)
