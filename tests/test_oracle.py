"""Pins for the CPU oracle (no GPU).

Each oracle function is checked against something other than its own formula:
torch's CPU scaled_dot_product_attention (an independent library routine),
pure-Python loops on tiny inputs, closed forms, the reference test's fixture
construction (tests/test_attention.py:21-33) and page-layout assertion
(tests/test_cache_manager.py:66-75). Mutation tests plant a mistake in a copy
of the oracle and show that the pins reject it.
"""

import math

import numpy as np
import pytest
import torch

import oracle
from minisgl_hip import workloads


def _rand(shape, seed, dtype=np.float64):
    return np.random.default_rng(seed).standard_normal(shape).astype(dtype)


def torch_sdpa(q, k, v, scale, mask=None):
    """Independent check: torch CPU SDPA in float64, kv heads expanded by repeat_interleave."""
    hq, hkv = q.shape[0], k.shape[0]
    kt = torch.from_numpy(np.asarray(k, np.float64)).repeat_interleave(hq // hkv, dim=0)
    vt = torch.from_numpy(np.asarray(v, np.float64)).repeat_interleave(hq // hkv, dim=0)
    qt = torch.from_numpy(np.asarray(q, np.float64))
    m = None if mask is None else torch.from_numpy(mask)
    return torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=m, scale=scale).numpy()


def brute_decode(q, k_pool, v_pool, slots_per_req, scale):
    """Pure-Python loops: o[b,h,:] = sum_j softmax_j(scale q.k_j) v_j, kv head h // G."""
    b_count, hq, d = q.shape
    hkv = k_pool.shape[1]
    g = hq // hkv
    out = np.zeros((b_count, hq, d))
    for b in range(b_count):
        for h in range(hq):
            kh = h // g
            scores = []
            for s in slots_per_req[b]:
                scores.append(scale * sum(float(q[b, h, e]) * float(k_pool[s, kh, e]) for e in range(d)))
            mx = max(scores)
            w = [math.exp(x - mx) for x in scores]
            tot = sum(w)
            for e in range(d):
                out[b, h, e] = sum(wi * float(v_pool[s, kh, e]) for wi, s in zip(w, slots_per_req[b])) / tot
    return out


# --------------------------------------------------------------------------- sdpa


@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (32, 8, 128), (8, 8, 64), (16, 2, 256)])
def test_sdpa_matches_torch(hq, hkv, d):
    q = _rand((hq, 5, d), 1)
    k = _rand((hkv, 37, d), 2)
    v = _rand((hkv, 37, d), 3)
    mask = np.arange(37)[None, :] <= 32 + np.arange(5)[:, None]  # bottom-right causal
    for m in (None, mask):
        np.testing.assert_allclose(oracle.sdpa(q, k, v, d**-0.5, m), torch_sdpa(q, k, v, d**-0.5, m), atol=1e-12)


def test_sdpa_closed_forms():
    hq, hkv, d = 4, 2, 16
    q = _rand((hq, 1, d), 4)
    # one key: the output is that key's value row exactly
    k1, v1 = _rand((hkv, 1, d), 5), _rand((hkv, 1, d), 6)
    o = oracle.sdpa(q, k1, v1, 0.3)
    for h in range(hq):
        np.testing.assert_array_equal(o[h, 0], v1[h // 2, 0])
    # identical keys: uniform weights -> mean of the value rows
    k = np.repeat(_rand((hkv, 1, d), 7), 9, axis=1)
    v = _rand((hkv, 9, d), 8)
    o = oracle.sdpa(q, k, v, 0.3)
    for h in range(hq):
        np.testing.assert_allclose(o[h, 0], v[h // 2].mean(axis=0), atol=1e-14)
    # GQA map: kv head 0 values = +1, kv head 1 values = -1 -> heads 0,1 -> +1 and 2,3 -> -1
    vsign = np.stack([np.ones((9, d)), -np.ones((9, d))])
    o = oracle.sdpa(q, _rand((hkv, 9, d), 9), vsign, 0.3)
    np.testing.assert_allclose(o[:, 0, 0], [1, 1, -1, -1], atol=1e-14)


# --------------------------------------------------------------------------- decode


def test_reference_fixture_construction():
    """tests/test_attention.py:21-33: request slots are consecutive slices of rng(0).permutation(4096)."""
    c = workloads.reference_test_case()
    perm = np.random.default_rng(0).permutation(4096).astype(np.int32)
    lens = [1, 2, 17, 31, 32, 33, 700]
    assert c.lens.tolist() == lens
    np.testing.assert_array_equal(c.kv_indices, perm[: sum(lens)])
    np.testing.assert_array_equal(c.kv_indptr, np.concatenate([[0], np.cumsum(lens)]))


def test_decode_bruteforce_tiny():
    c = workloads.decode_case_from_lens([1, 2, 5, 9], num_slots=64, seed=3)
    q = _rand((4, 4, 8), 10)
    kp = _rand((64, 2, 8), 11)
    vp = _rand((64, 2, 8), 12)
    slots = [c.kv_indices[c.kv_indptr[b] : c.kv_indptr[b + 1]] for b in range(4)]
    ref = brute_decode(q, kp, vp, slots, 8**-0.5)
    np.testing.assert_allclose(oracle.paged_decode(q, kp, vp, c.kv_indptr, c.kv_indices, 8**-0.5), ref, atol=1e-12)
    kvi, mask = oracle.naive_decode_metadata(c.page_table, np.arange(4), c.lens)
    np.testing.assert_allclose(oracle.naive_forward_decode(q, kp, vp, kvi, mask, 8**-0.5), ref, atol=1e-12)


@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (8, 8, 64)])
def test_naive_equals_paged_on_reference_grid(hq, hkv, d):
    """The two restatements (naive.py gather+mask, metal.py CSR) agree on the reference test's case."""
    c = workloads.reference_test_case()
    q = _rand((7, hq, d), 20, np.float32)
    kp = _rand((4096, hkv, d), 21, np.float32)
    vp = _rand((4096, hkv, d), 22, np.float32)
    kvi, mask = oracle.naive_decode_metadata(c.page_table, np.arange(7), c.lens)
    a = oracle.naive_forward_decode(q, kp, vp, kvi, mask, d**-0.5)
    b = oracle.paged_decode(q, kp, vp, c.kv_indptr, c.kv_indices, d**-0.5)
    np.testing.assert_allclose(a, b, atol=1e-12)
    # and one request through torch's SDPA
    s = c.kv_indices[c.kv_indptr[6] : c.kv_indptr[7]]
    t = torch_sdpa(q[6][:, None], kp[s].transpose(1, 0, 2), vp[s].transpose(1, 0, 2), d**-0.5)[:, 0]
    np.testing.assert_allclose(b[6], t, atol=1e-10)


def test_paged_page_ids_equal_token_slots():
    """page_size 16 through page ids == the same request through token slots."""
    c = workloads.decode_case_from_lens([1, 15, 16, 17, 40], num_slots=2048, page_size=16, seed=5)
    q = _rand((5, 4, 32), 30)
    kp = _rand((2048, 2, 32), 31)
    vp = _rand((2048, 2, 32), 32)
    a = oracle.paged_decode(q, kp, vp, c.page_indptr, c.page_ids, 0.2, page_size=16, seq_lens=c.lens)
    b = oracle.paged_decode(q, kp, vp, c.kv_indptr, c.kv_indices, 0.2)
    np.testing.assert_array_equal(a, b)
    # page layout: page-aligned runs of consecutive slots (tests/test_cache_manager.py:66-75)
    for i, n in enumerate(c.lens):
        row = c.page_table[i, :n]
        assert np.all(row[::16] % 16 == 0)
        assert np.all(row - np.repeat(row[::16], 16)[:n] == np.arange(n) % 16)


# --------------------------------------------------------------------------- prefill


def test_prefill_bottom_right_causal_closed_form():
    """Equal keys + V[j] = j: query t of E over prefix P averages positions 0..P+t -> (P+t)/2."""
    p_len, e_len, hq, hkv, d = 7, 5, 2, 1, 4
    n = p_len + e_len
    kp = np.zeros((n, hkv, d))
    vp = np.repeat(np.arange(n, dtype=np.float64)[:, None, None], d, axis=2)
    q = _rand((e_len, hq, d), 40)
    o = oracle.forward_prefill(q, kp[p_len:], vp[p_len:], kp, vp, [0, e_len], [np.arange(n)], 0.5)
    expect = (p_len + np.arange(e_len)) / 2.0
    np.testing.assert_allclose(o[:, 0, 0], expect, atol=1e-12)


def test_prefill_reductions():
    hq, hkv, d = 4, 2, 16
    # P = 0: standard causal == torch is_causal (top-left == bottom-right when Lq == Lkv)
    e_len = 9
    q, k, v = _rand((e_len, hq, d), 41), _rand((e_len, hkv, d), 42), _rand((e_len, hkv, d), 43)
    o = oracle.forward_prefill(q, k, v, None, None, [0, e_len], [None], 0.25)
    qt = torch.from_numpy(q.transpose(1, 0, 2))
    kt = torch.from_numpy(k.transpose(1, 0, 2)).repeat_interleave(2, 0)
    vt = torch.from_numpy(v.transpose(1, 0, 2)).repeat_interleave(2, 0)
    t = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, is_causal=True, scale=0.25).numpy()
    np.testing.assert_allclose(o, t.transpose(1, 0, 2), atol=1e-12)
    # E = 1 over a prefix reduces to decode
    c = workloads.prefill_case_from_lens([6], [1], num_slots=64, seed=2)
    kp, vp = _rand((64, hkv, d), 44), _rand((64, hkv, d), 45)
    q1 = _rand((1, hq, d), 46)
    o = oracle.forward_prefill(q1, kp[c.out_loc], vp[c.out_loc], kp, vp, [0, 1], [c.kv_indices], 0.25)
    dd = oracle.paged_decode(q1, kp, vp, c.kv_indptr, c.kv_indices, 0.25)
    np.testing.assert_allclose(o, dd, atol=1e-14)


def test_prefill_bruteforce_ragged():
    c = workloads.prefill_case_from_lens([0, 3, 5], [4, 1, 3], num_slots=64, seed=9)
    hq, hkv, d = 2, 1, 4
    kp, vp = _rand((64, hkv, d), 50), _rand((64, hkv, d), 51)
    q = _rand((8, hq, d), 52)
    kvi = [None if c.prefix_lens[i] == 0 else c.kv_indices[c.kv_indptr[i] : c.kv_indptr[i + 1]] for i in range(3)]
    o = oracle.forward_prefill(q, kp[c.out_loc], vp[c.out_loc], kp, vp, c.q_indptr.tolist(), kvi, 0.7)
    for i in range(3):
        slots = c.kv_indices[c.kv_indptr[i] : c.kv_indptr[i + 1]]
        for t in range(int(c.extend_lens[i])):
            visible = slots[: int(c.prefix_lens[i]) + t + 1]
            row = int(c.q_indptr[i]) + t
            ref = brute_decode(q[row][None], kp, vp, [visible], 0.7)[0]
            np.testing.assert_allclose(o[row], ref, atol=1e-12)


# --------------------------------------------------------------------------- index work


def test_csr_and_padded_metadata():
    c = workloads.decode_case_from_lens([3, 130, 1, 64], num_slots=1024, seed=1)
    rows = np.array([2, 0, 3, 1])
    table = np.zeros((4, 300), dtype=np.int32)
    table[rows] = np.pad(c.page_table, ((0, 0), (0, 300 - c.page_table.shape[1])))
    indptr, indices = oracle.csr_decode_metadata(table, rows, c.lens)
    assert indptr.dtype == np.int32 and indices.dtype == np.int32
    assert indptr[0] == 0 and np.all(np.diff(indptr) == c.lens) and indptr[-1] == c.lens.sum()
    expect = np.concatenate([table[r, :n] for r, n in zip(rows, c.lens)])
    np.testing.assert_array_equal(indices, expect)
    kvi, mask = oracle.naive_decode_metadata(table, rows, c.lens)
    assert kvi.shape == (4, 256) and mask.sum(axis=1).tolist() == c.lens.tolist()  # align_up(130,128)=256
    kvi, _ = oracle.naive_decode_metadata(table[:, :200], rows, c.lens)
    assert kvi.shape[1] == 200  # capped by the table width


def test_prepare_batch_indices_and_prefill_metadata():
    table = np.arange(4 * 16, dtype=np.int32).reshape(4, 16) * 3
    rows, cached, device = [3, 1], [2, 0], [5, 4]
    pos, out_loc = oracle.prepare_batch_indices(table, rows, cached, device)
    assert pos.tolist() == [2, 3, 4, 0, 1, 2, 3]
    assert out_loc.tolist() == [table[3, p] for p in (2, 3, 4)] + [table[1, p] for p in range(4)]
    q_off, last, kvi = oracle.prefill_metadata(table, rows, cached, device)
    assert q_off == [0, 3, 7] and last.tolist() == [2, 6]
    assert kvi[1] is None and kvi[0].tolist() == table[3, :5].tolist()


def test_allocate_paged_page_layout():
    """The page layout assertion of tests/test_cache_manager.py:66-75 (page_size 4, 10 tokens -> 3 pages)."""
    table = np.zeros((4, 64), dtype=np.int32)
    free = np.arange(8, dtype=np.int32) * 4
    free = oracle.allocate_paged(table, free, [0], [0], [10], 4)
    pages = table[0, :12].reshape(3, 4)
    assert np.all(pages[:, 0] % 4 == 0) and np.all(pages - pages[:, :1] == np.arange(4))
    assert len(free) == 5
    # decode step on a partly filled page needs no new page
    free2 = oracle.allocate_paged(table, free, [0], [10], [11], 4)
    assert len(free2) == 5
    assert oracle.page_to_token(np.array([8, 0]), 4).tolist() == [8, 9, 10, 11, 0, 1, 2, 3]


def test_store_kv_oracle():
    kp = _rand((32, 2, 8), 60)
    vp = _rand((32, 2, 8), 61)
    k0, v0 = kp.copy(), vp.copy()
    k, v = _rand((3, 2, 8), 62), _rand((3, 2, 8), 63)
    loc = np.array([5, 30, 0])
    oracle.store_kv(kp, vp, k, v, loc)
    for t, s in enumerate(loc):
        np.testing.assert_array_equal(kp[s], k[t])
        np.testing.assert_array_equal(vp[s], v[t])
    untouched = np.setdiff1d(np.arange(32), loc)
    np.testing.assert_array_equal(kp[untouched], k0[untouched])
    np.testing.assert_array_equal(vp[untouched], v0[untouched])


# --------------------------------------------------------------------------- mutations


def _mutant_gqa_modulo(q, k, v, scale, mask=None):
    """Planted mistake: q head h reads kv head h % Hkv instead of h // G."""
    hq, hkv = q.shape[0], k.shape[0]
    g = hq // hkv
    perm = np.array([(h % g) * hkv + h // g for h in range(hq)])  # h -> slot so that grouping becomes modulo
    inv = np.argsort(perm)
    return oracle.sdpa(q[inv], k, v, scale, mask)[perm]


def _mutant_topleft_prefill(q, k, v, k_pool, v_pool, q_offsets, kv_indices, scale):
    """Planted mistake: top-left causal (query t sees j <= t) instead of bottom-right."""
    outs = []
    for i, idx in enumerate(kv_indices):
        s, e = q_offsets[i], q_offsets[i + 1]
        ki, vi = k_pool[idx], v_pool[idx]
        mask = np.arange(ki.shape[0])[None, :] <= np.arange(e - s)[:, None]
        outs.append(oracle.sdpa(q[s:e].transpose(1, 0, 2), ki.transpose(1, 0, 2), vi.transpose(1, 0, 2), scale, mask))
    return np.concatenate([o.transpose(1, 0, 2) for o in outs])


def test_mutants_are_caught():
    hq, hkv, d = 4, 2, 16
    q, k, v = _rand((hq, 3, d), 70), _rand((hkv, 11, d), 71), _rand((hkv, 11, d), 72)
    # wrong GQA grouping fails the torch pin and the +1/-1 closed form
    assert not np.allclose(_mutant_gqa_modulo(q, k, v, 0.25), torch_sdpa(q, k, v, 0.25), atol=1e-6)
    vsign = np.stack([np.ones((11, d)), -np.ones((11, d))])
    assert not np.allclose(_mutant_gqa_modulo(q, k, vsign, 0.25)[:, 0, 0], [1, 1, -1, -1])
    # dropped / doubled scale fails the torch pin
    assert not np.allclose(oracle.sdpa(q, k, v, 0.25**2), torch_sdpa(q, k, v, 0.25), atol=1e-6)
    # swapped K and V fails the torch pin
    assert not np.allclose(oracle.sdpa(q, v, k, 0.25), torch_sdpa(q, k, v, 0.25), atol=1e-6)
    # top-left causal fails the (P+t)/2 closed form
    p_len, e_len = 7, 5
    n = p_len + e_len
    kp = np.zeros((n, 1, 4))
    vp = np.repeat(np.arange(n, dtype=np.float64)[:, None, None], 4, axis=2)
    qq = _rand((e_len, 2, 4), 73)
    o = _mutant_topleft_prefill(qq, None, None, kp, vp, [0, e_len], [np.arange(n)], 0.5)
    assert not np.allclose(o[:, 0, 0], (p_len + np.arange(e_len)) / 2.0)
