"""Seeded random configurations of paged decode (attention/naive.py:50-60
semantics) and ragged prefill (attention/base.py:85-105) against the float64
oracle: query-head groups 1 to 8 and 16, head_dim 64/128/256, fp32/bf16/fp16
queries over 16-bit or fp8 pools, token-slot or page-16 indices, ragged
lengths with short and single-key requests, and split settings -- the
combinations the grid tests do not enumerate one by one. Sizes are bounded so
the oracle finishes in about a second per case."""

import numpy as np
import pytest
import torch

import oracle
from gpu_util import DTYPES, assert_close, i32, randn, to_np64
from minisgl_hip import ops, workloads
from test_kvquant_gpu import _deq, _fp8_pools

pytestmark = pytest.mark.gpu

GROUPS = [1, 2, 3, 4, 5, 6, 7, 8, 16]


def _heads(rng, fp8):
    g = int(rng.choice([x for x in GROUPS if not fp8 or x <= 8]))
    hkv = int(rng.choice([1, 2, 4, 8] if g <= 4 else [1, 2, 4]))
    d = int(rng.choice([64, 128, 256]))
    return g * hkv, hkv, d


def _decode_case(seed, fp8=False):
    rng = np.random.default_rng(1000 + seed)
    hq, hkv, d = _heads(rng, fp8)
    dtype = str(rng.choice(["bf16", "f16"] if fp8 else ["f32", "bf16", "f16"]))
    page = int(rng.choice([1, 16]))
    splits = [1, None, 4, 16][int(rng.integers(4))]
    budget = 4_000_000 // (hkv * d)  # keys over the batch (the oracle's pool copy stays small)
    b = int(rng.integers(1, 20))
    lens = rng.integers(1, 2500, b)
    short = rng.random(b) < 0.25
    lens[short] = rng.integers(1, 40, int(short.sum()))
    if rng.random() < 0.3:
        lens[0] = 1
    lens = np.maximum(1, (lens * min(1.0, budget / max(1, lens.sum()))).astype(np.int64))
    n = int(-(-(int(lens.sum()) + 64 * b) // 16) * 16) + 256
    return hq, hkv, d, dtype, page, splits, lens, n


def _prefill_case(seed, fp8=False):
    rng = np.random.default_rng(2000 + seed)
    hq, hkv, d = _heads(rng, fp8)
    dtype = str(rng.choice(["bf16", "f16"] if fp8 else ["f32", "bf16", "f16"]))
    page = int(rng.choice([1, 16]))
    splits = [1, None, 3][int(rng.integers(3))]
    r = int(rng.integers(1, 7))
    prefix = rng.integers(0, 1500, r)
    prefix[rng.random(r) < 0.3] = 0
    extend = rng.integers(1, 200, r)
    extend[rng.random(r) < 0.2] = 1
    work = float((extend * (prefix + extend)).sum()) * hq * d
    if work > 2e9:  # keep the oracle to about a second
        f = (2e9 / work) ** 0.5
        prefix = (prefix * f).astype(np.int64)
        extend = np.maximum(1, (extend * f).astype(np.int64))
    n = int(-(-(int((prefix + extend).sum()) + 64 * r) // 16) * 16) + 256
    return hq, hkv, d, dtype, page, splits, prefix, extend, n


def _pools(n, hkv, d, dt, seed, device, fp8):
    if fp8:
        kp, vp, sc, _, _ = _fp8_pools(n, hkv, d, seed, device, spread=0.5)
        return kp, vp, sc, _deq(kp, sc, 0), _deq(vp, sc, 1)
    kp = randn((n, hkv, d), seed, dt).to(device)
    vp = randn((n, hkv, d), seed + 1, dt).to(device)
    return kp, vp, None, to_np64(kp), to_np64(vp)


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("seed", range(24))
def test_random_decode(cuda_device, seed, fp8):
    hq, hkv, d, dtype, page, splits, lens, n = _decode_case(seed, fp8)
    dt = DTYPES[dtype]
    print(f"case random decode seed={seed} fp8={fp8} {hq}/{hkv}/{d} {dtype} page={page} splits={splits} "
          f"B={len(lens)} sumL={int(lens.sum())}", flush=True)
    c = workloads.decode_case_from_lens(lens, num_slots=n, page_size=page, seed=seed)
    kp, vp, sc, k64, v64 = _pools(n, hkv, d, dt, 400 + seed, cuda_device, fp8)
    q = randn((len(lens), hq, d), 500 + seed, dt).to(cuda_device)
    if page == 1:
        out = ops.paged_decode_attention(q, kp, vp, i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device),
                                         d**-0.5, max_splits=splits, kv_scale=sc)
    else:
        out = ops.paged_decode_attention(q, kp, vp, i32(c.page_indptr, cuda_device), i32(c.page_ids, cuda_device),
                                         d**-0.5, seq_lens=i32(c.lens, cuda_device), page_size=16,
                                         max_splits=splits, kv_scale=sc)
    torch.cuda.synchronize()
    ref = oracle.paged_decode(to_np64(q), k64, v64, c.kv_indptr, c.kv_indices, d**-0.5)
    assert_close(out, ref, dt, f"random decode seed={seed} fp8={fp8}")


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("seed", range(24))
def test_random_prefill(cuda_device, seed, fp8):
    hq, hkv, d, dtype, page, splits, prefix, extend, n = _prefill_case(seed, fp8)
    dt = DTYPES[dtype]
    print(f"case random prefill seed={seed} fp8={fp8} {hq}/{hkv}/{d} {dtype} page={page} splits={splits} "
          f"P={prefix.tolist()} E={extend.tolist()}", flush=True)
    case = workloads.prefill_case_from_lens(prefix, extend, num_slots=n, page_size=page, seed=seed)
    kp, vp, sc, k64, v64 = _pools(n, hkv, d, dt, 600 + seed, cuda_device, fp8)
    q = randn((case.num_tokens, hq, d), 700 + seed, dt).to(cuda_device)
    if page == 1:
        kv_indptr, kv_indices, seq = case.kv_indptr, case.kv_indices, None
    else:
        pages = [case.page_table[i, : int(L)][::page] // page for i, L in enumerate(case.seq_lens)]
        kv_indptr = np.concatenate([[0], np.cumsum([len(x) for x in pages])]).astype(np.int32)
        kv_indices = np.concatenate(pages).astype(np.int32)
        seq = case.seq_lens
    out = ops.prefill_ragged_attention(
        q, kp, vp, i32(case.q_indptr, cuda_device), i32(kv_indptr, cuda_device), i32(kv_indices, cuda_device),
        None if seq is None else i32(seq, cuda_device), d**-0.5, max_extend_len=int(case.extend_lens.max()),
        max_seq_len=int(case.seq_lens.max()), page_size=page, max_splits=splits, kv_scale=sc)
    torch.cuda.synchronize()
    kvi = [case.kv_indices[case.kv_indptr[i]: case.kv_indptr[i + 1]] for i in range(len(case.seq_lens))]
    ref = oracle.forward_prefill(to_np64(q), None, None, k64, v64, case.q_indptr.tolist(), kvi, d**-0.5)
    assert_close(out, ref, dt, f"random prefill seed={seed} fp8={fp8}")
