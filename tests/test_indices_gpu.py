"""GPU step-metadata builder vs the oracle's restatements, bit-exact:
scheduler/scheduler.py:154-157 (positions, out_loc), attention/base.py:70-83
(q offsets, last_indices), attention/metal.py:145-152 (decode CSR), and the
page-level CSR for page_size > 1 (checked by expanding it back to the
token-granular table, scheduler/cache.py:138-143)."""

import numpy as np
import pytest
import torch

import oracle
from gpu_util import i32
from minisgl_hip import ops

pytestmark = pytest.mark.gpu


def _table(num_reqs, max_len, page_size, seed, num_rows=None, decode=False):
    """A page table filled as the scheduler does (allocate_paged over a shuffled free list)."""
    rng = np.random.default_rng(seed)
    num_rows = num_rows or num_reqs + 3
    device_len = rng.integers(1, max_len + 1, size=num_reqs)
    if decode:
        cached_len = device_len - 1
    else:
        cached_len = np.minimum(device_len, rng.integers(0, max_len + 1, size=num_reqs))
        cached_len[::7] = device_len[::7]  # zero extend
        cached_len[::5] = 0
    rows = rng.permutation(num_rows)[:num_reqs]
    stride = oracle.align_up(max_len, page_size) + page_size
    table = np.zeros((num_rows, stride), dtype=np.int32)
    pages = oracle.div_ceil(int(device_len.sum()), 1) + num_reqs * page_size
    free = (rng.permutation(pages + 16) * page_size).astype(np.int32)
    oracle.allocate_paged(table, free, rows, np.zeros(num_reqs, int), device_len, page_size)
    return table, rows.astype(np.int32), cached_len.astype(np.int32), device_len.astype(np.int32)


def _build(table, rows, cached, dlen, page_size, device, num_kv=None, num_tokens=None):
    extend = np.maximum(dlen - cached, 0)
    if num_kv is None:
        num_kv = int(dlen.sum()) if page_size == 1 else int(sum(oracle.div_ceil(int(L), page_size) for L in dlen))
    if num_tokens is None:
        num_tokens = int(extend.sum())
    out = ops.build_step_indices(i32(table, device), i32(rows, device), i32(cached, device), i32(dlen, device),
                                 num_tokens=num_tokens, num_kv=num_kv, page_size=page_size)
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in out.items()}


@pytest.mark.parametrize("page_size", [1, 16])
@pytest.mark.parametrize("num_reqs,max_len", [(1, 40), (7, 700), (130, 3000), (1500, 64), (5000, 20)])
def test_step_indices_match_oracle(cuda_device, num_reqs, max_len, page_size):
    print(f"case indices R={num_reqs} L<={max_len} page={page_size}", flush=True)
    table, rows, cached, dlen = _table(num_reqs, max_len, page_size, seed=num_reqs + page_size)
    got = _build(table, rows, cached, dlen, page_size, cuda_device)
    positions, out_loc = oracle.prepare_batch_indices(table, rows, cached, dlen)
    q_offsets, last_indices, _ = oracle.prefill_metadata(table, rows, cached, dlen)
    np.testing.assert_array_equal(got["q_indptr"], np.asarray(q_offsets, dtype=np.int32))
    np.testing.assert_array_equal(got["last_indices"], last_indices)
    np.testing.assert_array_equal(got["positions"], positions)
    np.testing.assert_array_equal(got["out_loc"], out_loc)
    if page_size == 1:
        kv_indptr, kv_indices = oracle.csr_decode_metadata(table, rows, dlen)
        np.testing.assert_array_equal(got["kv_indptr"], kv_indptr)
        np.testing.assert_array_equal(got["kv_indices"], kv_indices)
    else:
        npages = [oracle.div_ceil(int(L), page_size) for L in dlen]
        np.testing.assert_array_equal(got["kv_indptr"], np.concatenate([[0], np.cumsum(npages)]).astype(np.int32))
        for i, (row, L) in enumerate(zip(rows, dlen)):
            ids = got["kv_indices"][got["kv_indptr"][i] : got["kv_indptr"][i + 1]]
            np.testing.assert_array_equal(oracle.expand_page_indices(ids, page_size, int(L)), table[row, : int(L)])


def test_step_indices_decode_batch(cuda_device):
    """A decode step (extend 1 per request): out_loc is each request's last slot."""
    table, rows, cached, dlen = _table(128, 2048, 1, seed=11, decode=True)
    got = _build(table, rows, cached, dlen, 1, cuda_device)
    np.testing.assert_array_equal(got["q_indptr"], np.arange(129, dtype=np.int32))
    np.testing.assert_array_equal(got["out_loc"], table[rows, dlen - 1])
    kv_indptr, kv_indices = oracle.csr_decode_metadata(table, rows, dlen)
    np.testing.assert_array_equal(got["kv_indices"], kv_indices)


def test_step_indices_out_of_range_and_capacity(cuda_device):
    """Rows outside the table read as -1; outputs stop at the given capacities
    and the offsets are clamped to them (a launch reading them stays inside)."""
    table, rows, cached, dlen = _table(4, 50, 1, seed=3)
    rows = rows.copy()
    rows[2] = table.shape[0] + 5
    got = _build(table, rows, cached, dlen, 1, cuda_device)
    s, e = got["kv_indptr"][2], got["kv_indptr"][3]
    assert (got["kv_indices"][s:e] == -1).all()
    keep = np.ones(len(got["kv_indices"]), bool)
    keep[s:e] = False
    _, ref = oracle.csr_decode_metadata(table, np.where(np.arange(4) == 2, 0, rows), dlen)
    np.testing.assert_array_equal(got["kv_indices"][keep], ref[keep])
    short = _build(table, rows, cached, dlen, 1, cuda_device, num_kv=10)
    np.testing.assert_array_equal(short["kv_indices"], got["kv_indices"][:10])
    np.testing.assert_array_equal(short["kv_indptr"], np.minimum(got["kv_indptr"], 10))
    np.testing.assert_array_equal(short["q_indptr"], got["q_indptr"])
    t_short = int(got["q_indptr"][-1]) - 3
    shortq = _build(table, rows, cached, dlen, 1, cuda_device, num_tokens=t_short)
    np.testing.assert_array_equal(shortq["q_indptr"], np.minimum(got["q_indptr"], t_short))
    np.testing.assert_array_equal(shortq["last_indices"], np.minimum(got["q_indptr"][1:], t_short) - 1)
    np.testing.assert_array_equal(shortq["positions"], got["positions"][:t_short])
    np.testing.assert_array_equal(shortq["kv_indptr"], got["kv_indptr"])


def test_table_scatter(cuda_device):
    table = np.zeros((6, 40), dtype=np.int32)
    rows = np.array([0, 5, 3, 9, -1, 2], dtype=np.int32)
    cols = np.array([0, 39, 7, 1, 2, 40], dtype=np.int32)
    vals = np.array([11, 22, 33, 44, 55, 66], dtype=np.int32)
    t = i32(table, cuda_device)
    ops.table_scatter(t, i32(rows, cuda_device), i32(cols, cuda_device), i32(vals, cuda_device))
    torch.cuda.synchronize()
    ref = table.copy()
    ref[0, 0], ref[5, 39], ref[3, 7] = 11, 22, 33  # the out-of-range entries are skipped
    np.testing.assert_array_equal(t.cpu().numpy(), ref)
