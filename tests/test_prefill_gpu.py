"""Ragged chunked prefill on the GPU vs the float64 oracle (attention/base.py:85-105,
bottom-right causal over a cached prefix)."""

import numpy as np
import pytest
import torch

import oracle
from gpu_util import DTYPES, assert_close, i32, randn, to_np64
from minisgl_hip import ops, workloads

pytestmark = pytest.mark.gpu


def _run(case, hq, hkv, d, dt, device, seed, page_size=1):
    n = case.num_slots
    kp = randn((n, hkv, d), seed, dt).to(device)
    vp = randn((n, hkv, d), seed + 1, dt).to(device)
    q = randn((case.num_tokens, hq, d), seed + 2, dt).to(device)
    knew = randn((case.num_tokens, hkv, d), seed + 3, dt).to(device)
    vnew = randn((case.num_tokens, hkv, d), seed + 4, dt).to(device)
    ops.store_kv(knew, vnew, i32(case.out_loc, device), kp, vp)
    if page_size == 1:
        kv_indptr, kv_indices, seq = case.kv_indptr, case.kv_indices, None
    else:
        pages = []
        for i, L in enumerate(case.seq_lens):
            row = case.page_table[i, : int(L)]
            pages.append(row[::page_size] // page_size)
        kv_indptr = np.concatenate([[0], np.cumsum([len(x) for x in pages])]).astype(np.int32)
        kv_indices = np.concatenate(pages).astype(np.int32)
        seq = case.seq_lens
    out = ops.prefill_ragged_attention(
        q, kp, vp, i32(case.q_indptr, device), i32(kv_indptr, device), i32(kv_indices, device),
        None if seq is None else i32(seq, device), d**-0.5,
        max_extend_len=int(case.extend_lens.max()), page_size=page_size,
    )
    torch.cuda.synchronize()
    return q, knew, vnew, kp, vp, out


def _oracle(case, q, knew, vnew, kp, vp, d, rows=None):
    kvi = [None if case.prefix_lens[i] == 0 else case.kv_indices[case.kv_indptr[i] : case.kv_indptr[i + 1]]
           for i in range(len(case.seq_lens))]
    if rows is None:
        return oracle.forward_prefill(to_np64(q), to_np64(knew), to_np64(vnew), to_np64(kp), to_np64(vp),
                                      case.q_indptr.tolist(), kvi, d**-0.5)
    outs = []
    for i in rows:
        s, e = int(case.q_indptr[i]), int(case.q_indptr[i + 1])
        slots = torch.from_numpy(case.kv_indices[case.kv_indptr[i] : case.kv_indptr[i + 1]].astype(np.int64))
        kb = to_np64(kp.index_select(0, slots.to(kp.device)))
        vb = to_np64(vp.index_select(0, slots.to(vp.device)))
        outs.append(oracle.forward_prefill(to_np64(q[s:e]), None, None, kb, vb, [0, e - s],
                                           [np.arange(len(slots))], d**-0.5))
    return np.concatenate(outs)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (32, 8, 128), (8, 8, 64), (16, 2, 256)])
def test_prefill_grid(cuda_device, hq, hkv, d, dtype):
    """Prefix P in {0,1,17,300,0}, extend E in {1,2,64,100,37}: causal edges, E == 1, P == 0."""
    dt = DTYPES[dtype]
    case = workloads.prefill_case_from_lens([0, 1, 17, 300, 0], [1, 2, 64, 100, 37], num_slots=2048, seed=3)
    print(f"case prefill grid {hq}/{hkv}/{d} {dtype}", flush=True)
    q, kn, vn, kp, vp, out = _run(case, hq, hkv, d, dt, cuda_device, 10)
    ref = _oracle(case, q, kn, vn, kp, vp, d)
    assert_close(out, ref, dt, f"prefill {hq}/{hkv}/{d} {dtype}")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_prefill_page_size_16(cuda_device, dtype):
    dt = DTYPES[dtype]
    case = workloads.prefill_case_from_lens([0, 15, 16, 40, 333], [5, 1, 33, 100, 64], num_slots=8192, page_size=16,
                                            seed=4)
    print(f"case prefill page16 {dtype}", flush=True)
    q, kn, vn, kp, vp, out = _run(case, 32, 8, 128, dt, cuda_device, 20, page_size=16)
    ref = _oracle(case, q, kn, vn, kp, vp, 128)
    assert_close(out, ref, dt, f"prefill page16 {dtype}")


def test_prefill_16req_sampled(cuda_device):
    """16 requests, P ~ U[0,4096], E ~ U[64,512] rescaled to <= 2048 packed tokens, bf16."""
    case = workloads.prefill_case(16, 4096, 64, 512, 2048, num_slots=1 << 17, seed=0)
    print("case prefill 16 requests", flush=True)
    q, kn, vn, kp, vp, out = _run(case, 16, 8, 128, torch.bfloat16, cuda_device, 30)
    rows = [0, 3, 7, 15]
    ref = _oracle(case, q, kn, vn, kp, vp, 128, rows=rows)
    sel = np.concatenate([np.arange(case.q_indptr[i], case.q_indptr[i + 1]) for i in rows])
    assert_close(out[torch.from_numpy(sel).to(cuda_device)], ref, torch.bfloat16, "prefill 16 requests sampled")
    out2 = ops.prefill_ragged_attention(
        q, kp, vp, i32(case.q_indptr, cuda_device), i32(case.kv_indptr, cuda_device),
        i32(case.kv_indices, cuda_device), None, 128**-0.5, max_extend_len=int(case.extend_lens.max()),
    )
    torch.cuda.synchronize()
    assert torch.equal(out, out2), "prefill is not deterministic"


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("hq,hkv", [(16, 8), (32, 8)])
@pytest.mark.parametrize("splits", [1, 2, 5, 16])
def test_prefill_key_splits(cuda_device, hq, hkv, dtype, splits):
    """Long prefixes cut into 1..16 key chunks (merged in fp32), one chunk longer
    than the 1024-key slot window (splits=1), rows that see no key of a chunk."""
    dt = DTYPES[dtype]
    case = workloads.prefill_case_from_lens([0, 1500, 2500, 700, 33], [300, 64, 129, 1, 200], num_slots=16384,
                                            seed=5)
    print(f"case prefill splits={splits} {hq}/{hkv} {dtype}", flush=True)
    n = case.num_slots
    kp = randn((n, hkv, 128), 40, dt).to(cuda_device)
    vp = randn((n, hkv, 128), 41, dt).to(cuda_device)
    q = randn((case.num_tokens, hq, 128), 42, dt).to(cuda_device)
    kn = randn((case.num_tokens, hkv, 128), 43, dt).to(cuda_device)
    vn = randn((case.num_tokens, hkv, 128), 44, dt).to(cuda_device)
    ops.store_kv(kn, vn, i32(case.out_loc, cuda_device), kp, vp)
    out = ops.prefill_ragged_attention(
        q, kp, vp, i32(case.q_indptr, cuda_device), i32(case.kv_indptr, cuda_device),
        i32(case.kv_indices, cuda_device), None, 128**-0.5, max_extend_len=int(case.extend_lens.max()),
        max_splits=splits,
    )
    torch.cuda.synchronize()
    ref = _oracle(case, q, kn, vn, kp, vp, 128)
    assert_close(out, ref, dt, f"prefill splits={splits} {hq}/{hkv} {dtype}")


def test_prefill_splits_page16(cuda_device):
    case = workloads.prefill_case_from_lens([0, 15, 1600, 40, 2333], [5, 1, 33, 100, 64], num_slots=16384,
                                            page_size=16, seed=6)
    print("case prefill splits page16", flush=True)
    q, kn, vn, kp, vp, out = _run(case, 32, 8, 128, torch.bfloat16, cuda_device, 50, page_size=16)
    ref = _oracle(case, q, kn, vn, kp, vp, 128)
    assert_close(out, ref, torch.bfloat16, "prefill splits page16")


def test_planned_matches_unplanned(cuda_device):
    """A work list built once (msgl_prefill_plan) and reused by the planned call
    gives the self-planning call's result bit for bit, over several layers' pools."""
    case = workloads.prefill_case(16, 4096, 64, 512, 2048, num_slots=1 << 17, seed=0)
    dt = torch.bfloat16
    t = case.num_tokens
    q = randn((t, 16, 128), 90, dt).to(cuda_device)
    qi, ki = i32(case.q_indptr, cuda_device), i32(case.kv_indptr, cuda_device)
    kx = i32(case.kv_indices, cuda_device)
    maxe, maxs = int(case.extend_lens.max()), int(case.seq_lens.max())
    splits = ops.prefill_default_splits(16, 16, 8, 128, maxe, maxs)
    ws = ops.prefill_workspace(16, t, maxe, 16, 8, 128, splits, cuda_device)
    ops.prefill_plan(qi, ki, None, num_tokens=t, max_extend_len=maxe, max_seq_len=maxs, num_qo_heads=16,
                     num_kv_heads=8, head_dim=128, dtype=dt, max_splits=splits, workspace=ws)
    for layer in range(3):
        kp = randn((1 << 17, 8, 128), 91 + layer, dt).to(cuda_device)
        vp = randn((1 << 17, 8, 128), 95 + layer, dt).to(cuda_device)
        print(f"case prefill planned layer={layer}", flush=True)
        a = ops.prefill_ragged_attention(q, kp, vp, qi, ki, kx, None, 128**-0.5, max_extend_len=maxe,
                                         max_seq_len=maxs, max_splits=splits)
        b = ops.prefill_ragged_attention(q, kp, vp, qi, ki, kx, None, 128**-0.5, max_extend_len=maxe,
                                         max_seq_len=maxs, max_splits=splits, workspace=ws, planned=True)
        torch.cuda.synchronize()
        assert torch.equal(a, b), f"layer {layer}"


@pytest.mark.parametrize("splits", [None, 3])
def test_prefill_many_short_requests(cuda_device, splits):
    """700 requests of 1..8 new tokens over prefixes of 0..300 (a batch of short
    prompts and chunk tails): a long work list of one-block items, most rows
    of each block dead. Sampled requests against the oracle; the plan reused
    by the planned call gives the same bits."""
    rng = np.random.default_rng(31)
    prefix = rng.integers(0, 301, size=700)
    extend = rng.integers(1, 9, size=700)
    case = workloads.prefill_case_from_lens(prefix, extend, num_slots=1 << 19, seed=32)
    hq, hkv, d = 16, 8, 128
    dt = torch.bfloat16
    n = case.num_slots
    kp = randn((n, hkv, d), 50, dt).to(cuda_device)
    vp = randn((n, hkv, d), 51, dt).to(cuda_device)
    q = randn((case.num_tokens, hq, d), 52, dt).to(cuda_device)
    kn = randn((case.num_tokens, hkv, d), 53, dt).to(cuda_device)
    vn = randn((case.num_tokens, hkv, d), 54, dt).to(cuda_device)
    ops.store_kv(kn, vn, i32(case.out_loc, cuda_device), kp, vp)
    qi, ki, kx = (i32(x, cuda_device) for x in (case.q_indptr, case.kv_indptr, case.kv_indices))
    max_e, max_l = int(case.extend_lens.max()), int(case.seq_lens.max())
    print(f"case prefill 700 short requests splits={splits}", flush=True)
    out = ops.prefill_ragged_attention(q, kp, vp, qi, ki, kx, None, d**-0.5, max_extend_len=max_e,
                                       max_seq_len=max_l, max_splits=splits)
    s = splits or ops.prefill_default_splits(len(extend), hq, hkv, d, max_e, max_l)
    ws = ops.prefill_workspace(len(extend), case.num_tokens, max_e, hq, hkv, d, s, cuda_device)
    ops.prefill_plan(qi, ki, None, num_tokens=case.num_tokens, max_extend_len=max_e, max_seq_len=max_l,
                     num_qo_heads=hq, num_kv_heads=hkv, head_dim=d, dtype=dt, max_splits=s, workspace=ws)
    again = ops.prefill_ragged_attention(q, kp, vp, qi, ki, kx, None, d**-0.5, max_extend_len=max_e,
                                         max_seq_len=max_l, max_splits=s, workspace=ws, planned=True)
    torch.cuda.synchronize()
    assert torch.equal(out, again), "planned != self-planning"
    rows = [0, 1, 350, 698, 699, int(np.argmax(prefix)), int(np.argmin(prefix))]
    got = torch.cat([out[int(case.q_indptr[i]): int(case.q_indptr[i + 1])] for i in rows])
    assert_close(got, _oracle(case, q, kn, vn, kp, vp, d, rows=rows), dt, "prefill 700 short requests")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("splits", [1, 3])
def test_prefill_requests_without_extend(cuda_device, dtype, splits):
    """Requests with no extend tokens (repeated q offsets) between real ones:
    none of their rows is computed or written and the others match the oracle.
    The scheduler never forms such a batch (scheduler/prefill.py:67-83: every
    chunk takes at least one token), but a caller's metadata may."""
    dt = DTYPES[dtype]
    case = workloads.prefill_case_from_lens([100, 50, 0, 20, 2000], [37, 0, 5, 0, 130], num_slots=8192, seed=5)
    hq, hkv, d = 16, 8, 128
    kp = randn((case.num_slots, hkv, d), 60, dt).to(cuda_device)
    vp = randn((case.num_slots, hkv, d), 61, dt).to(cuda_device)
    q = randn((case.num_tokens, hq, d), 62, dt).to(cuda_device)
    kn = randn((case.num_tokens, hkv, d), 63, dt).to(cuda_device)
    vn = randn((case.num_tokens, hkv, d), 64, dt).to(cuda_device)
    ops.store_kv(kn, vn, i32(case.out_loc, cuda_device), kp, vp)
    print(f"case prefill empty extends {dtype} splits={splits}", flush=True)
    out = ops.prefill_ragged_attention(q, kp, vp, i32(case.q_indptr, cuda_device), i32(case.kv_indptr, cuda_device),
                                       i32(case.kv_indices, cuda_device), None, d**-0.5,
                                       max_extend_len=int(case.extend_lens.max()),
                                       max_seq_len=int(case.seq_lens.max()), max_splits=splits)
    torch.cuda.synchronize()
    assert_close(out, _oracle(case, q, kn, vn, kp, vp, d), dt, f"prefill empty extends {dtype} splits={splits}")
