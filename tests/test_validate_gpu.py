"""Metadata validation, the plan guards and the split decode launch on the GPU.

msgl_validate_metadata turns index metadata the attention kernels would read
outside the pool or the index arrays into an error (the reference asserts
its preconditions on the host, attention/metal.py:122); the planned launches
do nothing over a plan built for other sizes; msgl_paged_decode_planned_ex
without its merge plus msgl_paged_decode_merge equals the one-call decode bit
for bit. Malformed metadata is only ever given to the validation kernel, never
to an attention launch."""

import numpy as np
import pytest
import torch

from gpu_util import i32, randn
from minisgl_hip import _lib, ops, workloads

pytestmark = pytest.mark.gpu


def _decode_meta(device):
    c = workloads.reference_test_case()  # N = 4096, lens [1, 2, 17, 31, 32, 33, 700]
    return c, i32(c.kv_indptr, device), i32(c.kv_indices, device)


def test_valid_decode_and_prefill_metadata_pass(cuda_device):
    c, ip, ix = _decode_meta(cuda_device)
    print("case validate ok", flush=True)
    ops.validate_metadata(ip, ix, None, num_slots=4096)
    pc = workloads.prefill_case(5, 300, 1, 40, 1000, num_slots=8192, seed=3)
    ops.validate_metadata(i32(pc.kv_indptr, cuda_device), i32(pc.kv_indices, cuda_device), None, num_slots=8192,
                          q_indptr=i32(pc.q_indptr, cuda_device), num_tokens=pc.num_tokens)
    # page ids with per-request lengths
    d = workloads.decode_case(6, 30, 300, 1 << 14, 16, seed=2)
    ops.validate_metadata(i32(d.page_indptr, cuda_device), i32(d.page_ids, cuda_device), i32(d.lens, cuda_device),
                          num_slots=1 << 14, page_size=16)


@pytest.mark.parametrize("fault", ["decreasing", "negative", "beyond", "slot", "slot_negative", "seq_len", "page"])
def test_malformed_decode_metadata_is_reported(cuda_device, fault):
    c, ip, ix = _decode_meta(cuda_device)
    indptr = c.kv_indptr.copy()
    indices = c.kv_indices.copy()
    lens = None
    num_slots, page = 4096, 1
    if fault == "decreasing":
        indptr[3], indptr[4] = indptr[4], indptr[3]
    elif fault == "negative":
        indptr = indptr - 1
    elif fault == "beyond":
        indices = indices[:-5]  # kv_indptr[B] now names 5 entries kv_indices does not hold
    elif fault == "slot":
        indices[100] = 4096
    elif fault == "slot_negative":
        indices[0] = -3
    elif fault == "seq_len":
        lens = np.diff(c.kv_indptr).astype(np.int32)
        lens[6] += 1  # one key more than its row of indices
    elif fault == "page":
        d = workloads.decode_case(6, 30, 300, 1 << 14, 16, seed=2)
        indptr, indices, lens = d.page_indptr, d.page_ids.copy(), d.lens
        indices[7] = (1 << 14) // 16  # one page past the pool
        num_slots, page = 1 << 14, 16
    print(f"case validate fault={fault}", flush=True)
    with pytest.raises(ValueError, match="invalid attention metadata"):
        ops.validate_metadata(i32(indptr, cuda_device), i32(indices, cuda_device),
                              None if lens is None else i32(lens, cuda_device), num_slots=num_slots, page_size=page)


@pytest.mark.parametrize("fault", ["q_start", "q_total", "extend"])
def test_malformed_prefill_metadata_is_reported(cuda_device, fault):
    pc = workloads.prefill_case(5, 300, 1, 40, 1000, num_slots=8192, seed=3)
    q_indptr = pc.q_indptr.copy()
    num_tokens = pc.num_tokens
    if fault == "q_start":
        q_indptr = q_indptr + 1
    elif fault == "q_total":
        num_tokens -= 1
    elif fault == "extend":  # request 0 extends past its sequence
        q_indptr[1:] += int(pc.seq_lens[0])
        num_tokens = int(q_indptr[-1])
    print(f"case validate prefill fault={fault}", flush=True)
    with pytest.raises(ValueError, match="invalid attention metadata"):
        ops.validate_metadata(i32(pc.kv_indptr, cuda_device), i32(pc.kv_indices, cuda_device), None,
                              num_slots=8192, q_indptr=i32(q_indptr, cuda_device), num_tokens=num_tokens)


def test_split_decode_launch_equals_one_call(cuda_device):
    """planned_ex without the merge, then the merge: the same bits as
    msgl_paged_decode_store_planned, pools included (bf16 and an fp8 pool)."""
    b, hq, hkv, d = 40, 16, 8, 128
    c = workloads.decode_case(b, 10, 3000, 1 << 16, 1, seed=11)
    ip, ix, loc = i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device), i32(c.out_loc, cuda_device)
    dt = torch.bfloat16
    q = randn((b, hq, d), 1, dt).to(cuda_device)
    kn = randn((b, hkv, d), 2, dt).to(cuda_device)
    vn = randn((b, hkv, d), 3, dt).to(cuda_device)
    for splits in (1, 6):
        kp = randn((1 << 16, hkv, d), 4, dt).to(cuda_device)
        vp = randn((1 << 16, hkv, d), 5, dt).to(cuda_device)
        kp2, vp2 = kp.clone(), vp.clone()
        ws = ops.decode_workspace(b, hq, hkv, d, splits, cuda_device)
        print(f"case split decode splits={splits}", flush=True)
        ops.paged_decode_plan(ip, None, b, hq, hkv, d, splits, ws)
        a = ops.paged_decode_attention(q, kp, vp, ip, ix, d**-0.5, max_splits=splits, workspace=ws,
                                       new_kv=(kn, vn, loc), planned=True)
        o = torch.empty_like(q)
        ops.paged_decode_attention(q, kp2, vp2, ip, ix, d**-0.5, max_splits=splits, workspace=ws, out=o,
                                   new_kv=(kn, vn, loc), planned=True, merge=False)
        ops.paged_decode_merge(o, ip, None, hkv, splits, ws)
        torch.cuda.synchronize()
        assert torch.equal(a, o), f"split launch differs (splits={splits})"
        assert torch.equal(kp, kp2) and torch.equal(vp, vp2)
    # fp8 pools
    kq = torch.empty((1 << 16, hkv, d), dtype=torch.float8_e4m3fn, device=cuda_device)
    vq = torch.empty_like(kq)
    sc = torch.empty((1 << 16, hkv, 2), dtype=torch.float32, device=cuda_device)
    ops.store_kv_fp8(randn((1 << 16, hkv, d), 6, dt).to(cuda_device), randn((1 << 16, hkv, d), 7, dt).to(cuda_device),
                     torch.arange(1 << 16, dtype=torch.int32, device=cuda_device), kq, vq, sc)
    kq2, vq2, sc2 = kq.clone(), vq.clone(), sc.clone()
    ws = ops.decode_workspace(b, hq, hkv, d, 6, cuda_device)
    print("case split decode fp8", flush=True)
    ops.paged_decode_plan(ip, None, b, hq, hkv, d, 6, ws)
    a = ops.paged_decode_attention(q, kq, vq, ip, ix, d**-0.5, max_splits=6, workspace=ws, new_kv=(kn, vn, loc),
                                   planned=True, kv_scale=sc)
    o = torch.empty_like(q)
    ops.paged_decode_attention(q, kq2, vq2, ip, ix, d**-0.5, max_splits=6, workspace=ws, out=o,
                               new_kv=(kn, vn, loc), planned=True, kv_scale=sc2, merge=False)
    ops.paged_decode_merge(o, ip, None, hkv, 6, ws, kv_fp8=True)
    torch.cuda.synchronize()
    assert torch.equal(a, o), "split fp8 launch differs"
    assert torch.equal(sc, sc2) and torch.equal(kq.view(torch.uint8), kq2.view(torch.uint8))


def test_planned_launch_over_a_plan_for_other_sizes_does_nothing(cuda_device):
    """The C ABI called with a batch other than the plan's: the decode and merge
    launches read no work item and leave out untouched. Every buffer is sized
    for the plan's batch, so the call stays in bounds either way."""
    hq, hkv, d, splits = 16, 8, 128, 4
    n = 1 << 16
    c = workloads.decode_case(40, 10, 900, n, 1, seed=12)
    ip, ix = i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device)
    dt = torch.bfloat16
    kp = randn((n, hkv, d), 8, dt).to(cuda_device)
    vp = randn((n, hkv, d), 9, dt).to(cuda_device)
    q = randn((40, hq, d), 10, dt).to(cuda_device)
    ws = ops.decode_workspace(40, hq, hkv, d, splits, cuda_device)
    ops.paged_decode_plan(ip, None, 40, hq, hkv, d, splits, ws)
    out = torch.full_like(q, 7.0)
    lib = _lib.load()
    print("case plan guard", flush=True)
    st = lib.msgl_paged_decode_planned(
        _lib.ptr(q), _lib.ptr(kp), _lib.ptr(vp), _lib.ptr(ip), _lib.ptr(ix), None, 20, hq, hkv, d, 1, n,
        _lib.MSGL_BF16, d**-0.5, splits, _lib.ptr(out), _lib.ptr(ws), ws.numel(), _lib.current_stream(cuda_device))
    assert st == _lib.MSGL_OK
    torch.cuda.synchronize()
    assert torch.all(out == 7.0), "a launch over a plan for another batch wrote output"
    # the same workspace re-planned for batch 20 then works
    ops.paged_decode_plan(ip, None, 20, hq, hkv, d, splits, ws)
    st = lib.msgl_paged_decode_planned(
        _lib.ptr(q), _lib.ptr(kp), _lib.ptr(vp), _lib.ptr(ip), _lib.ptr(ix), None, 20, hq, hkv, d, 1, n,
        _lib.MSGL_BF16, d**-0.5, splits, _lib.ptr(out), _lib.ptr(ws), ws.numel(), _lib.current_stream(cuda_device))
    assert st == _lib.MSGL_OK
    torch.cuda.synchronize()
    ref = ops.paged_decode_attention(q[:20], kp, vp, ip[:21], ix, d**-0.5, max_splits=splits)
    torch.cuda.synchronize()
    assert torch.equal(out[:20], ref) and torch.all(out[20:] == 7.0)
