"""numpy restatement of the reference attention path (oracle; test infrastructure only).

Each function names the reference lines it follows (relative to the
reference's ``python/minisgl_mlx/``). Integer work is int32 and bit-exact;
floating-point attention accumulates in float64 so that the HIP kernels'
fp32 and bf16 results can be held to absolute / relative tolerances.
"""

from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import numpy as np

# --------------------------------------------------------------------------
# small integer helpers  (utils.py:37-46)
# --------------------------------------------------------------------------


def div_ceil(a: int, b: int) -> int:
    """utils.py:37-38."""
    return (a + b - 1) // b


def align_up(a: int, b: int) -> int:
    """utils.py:45-46."""
    return div_ceil(a, b) * b


# --------------------------------------------------------------------------
# slot allocation and page-table layout  (scheduler/cache.py)
# --------------------------------------------------------------------------


def page_to_token(pages: np.ndarray, page_size: int) -> np.ndarray:
    """scheduler/cache.py:138-143: page base slots -> token slots, page by page."""
    pages = np.asarray(pages, dtype=np.int32)
    if page_size == 1:
        return pages
    offsets = np.arange(page_size, dtype=np.int32)
    return (pages[:, None] + offsets[None, :]).reshape(-1)


def allocate_paged(
    page_table: np.ndarray,
    free_slots: np.ndarray,
    table_idx: Sequence[int],
    cached_len: Sequence[int],
    device_len: Sequence[int],
    page_size: int,
) -> np.ndarray:
    """scheduler/cache.py:53-72 (without prefix-cache eviction).

    Writes slots for tokens [cached_len, device_len) of each request into
    ``page_table`` in place and returns the remaining free list. ``free_slots``
    holds page-aligned base slots, as built at scheduler/cache.py:31.
    """
    needed = 0
    info: List[Tuple[int, int, int]] = []
    for row, c, d in zip(table_idx, cached_len, device_len):
        first_page = div_ceil(int(c), page_size)
        last_page = div_ceil(int(d), page_size)
        if last_page > first_page:
            needed += last_page - first_page
            info.append((int(row), first_page, last_page))
    if needed == 0:
        return free_slots
    if needed > len(free_slots):
        raise RuntimeError("out of KV slots")
    allocated = page_to_token(free_slots[:needed], page_size)
    free_slots = free_slots[needed:]
    offset = 0
    for row, first_page, last_page in info:
        first_pos, last_pos = first_page * page_size, last_page * page_size
        n = last_pos - first_pos
        page_table[row, first_pos:last_pos] = allocated[offset : offset + n]
        offset += n
    assert offset == len(allocated)
    return free_slots


# --------------------------------------------------------------------------
# per-step index work  (bit-exact)
# --------------------------------------------------------------------------


def prepare_batch_indices(
    page_table: np.ndarray,
    table_idx: Sequence[int],
    cached_len: Sequence[int],
    device_len: Sequence[int],
) -> Tuple[np.ndarray, np.ndarray]:
    """scheduler/scheduler.py:154-157: packed positions and new-token slots (out_loc)."""
    positions = np.concatenate(
        [np.arange(c, d, dtype=np.int32) for c, d in zip(cached_len, device_len)]
    ).astype(np.int32)
    extend = [int(d) - int(c) for c, d in zip(cached_len, device_len)]
    rows = np.repeat(np.asarray(table_idx), extend)
    out_loc = page_table[rows, positions].astype(np.int32)
    return positions, out_loc


def naive_decode_metadata(
    page_table: np.ndarray, rows: Sequence[int], lens: Sequence[int]
) -> Tuple[np.ndarray, np.ndarray]:
    """attention/naive.py:36-48: padded kv_indices [B, L_max] and length mask [B, L_max].

    L_max = min(align_up(max(lens), 128), page_table.shape[1]); entries past a
    request's length are stale-but-valid table entries and are masked out.
    """
    lens = np.asarray(lens)
    rows = np.asarray(rows)
    max_len = min(align_up(int(lens.max()), 128), page_table.shape[1])
    kv_indices = page_table[rows, :max_len]
    mask = np.arange(max_len)[None, :] < lens[:, None]
    return kv_indices, mask


def csr_decode_metadata(
    page_table: np.ndarray, rows: Sequence[int], lens: Sequence[int]
) -> Tuple[np.ndarray, np.ndarray]:
    """attention/metal.py:145-152: CSR kv_indptr [B+1] and kv_indices [sum L] (int32)."""
    lens = np.asarray(lens)
    rows = np.asarray(rows)
    max_len = int(lens.max())
    valid = np.arange(max_len)[None, :] < lens[:, None]
    kv_indices = page_table[rows, :max_len][valid].astype(np.int32)
    kv_indptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    return kv_indptr, kv_indices


def prefill_metadata(
    page_table: np.ndarray,
    rows: Sequence[int],
    cached_len: Sequence[int],
    device_len: Sequence[int],
) -> Tuple[List[int], np.ndarray, List[Optional[np.ndarray]]]:
    """attention/base.py:70-83: (q_offsets, last_indices, per-request kv_indices or None)."""
    extend = [int(d) - int(c) for c, d in zip(cached_len, device_len)]
    q_offsets = np.concatenate([[0], np.cumsum(extend)]).astype(np.int64).tolist()
    kv_indices: List[Optional[np.ndarray]] = []
    for row, c, d in zip(rows, cached_len, device_len):
        kv_indices.append(None if int(c) == 0 else page_table[int(row), : int(d)].copy())
    last_indices = np.asarray(q_offsets[1:], dtype=np.int32) - 1
    return q_offsets, last_indices, kv_indices


def expand_page_indices(page_ids: np.ndarray, page_size: int, length: int) -> np.ndarray:
    """Token slots of a request whose KV lives in pages ``page_ids`` of ``page_size`` slots.

    Token t lives at slot page_ids[t // page_size] * page_size + t % page_size,
    the page layout fixed by scheduler/cache.py:138-143 (pages are page-aligned
    runs of consecutive slots; tests/test_cache_manager.py:66-75 asserts it).
    """
    t = np.arange(length)
    return (np.asarray(page_ids, dtype=np.int64)[t // page_size] * page_size + t % page_size).astype(
        np.int64
    )


# --------------------------------------------------------------------------
# KV store  (bit-exact copy)
# --------------------------------------------------------------------------


def store_kv(k_pool: np.ndarray, v_pool: np.ndarray, k: np.ndarray, v: np.ndarray, out_loc) -> None:
    """kvcache/pool.py:47-50: k_pool[out_loc] = k; v_pool[out_loc] = v (in place)."""
    out_loc = np.asarray(out_loc, dtype=np.int64)
    k_pool[out_loc] = k
    v_pool[out_loc] = v


# --------------------------------------------------------------------------
# attention (float64 accumulation)
# --------------------------------------------------------------------------


def sdpa(
    q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, mask: Optional[np.ndarray] = None
) -> np.ndarray:
    """Scaled dot-product attention with GQA, as the reference calls MLX's SDPA.

    q [Hq, Lq, D], k/v [Hkv, Lkv, D], boolean mask [Lq, Lkv] (True = attend) or
    None -> o [Hq, Lq, D] in float64. Query head h reads kv head h // (Hq / Hkv),
    the grouping MLX SDPA applies for Hq != Hkv (attention/base.py:97-103,
    attention/naive.py:53-59; consecutive q heads share a kv head,
    attention/metal.py:50). A fully masked row is 0/0 = NaN, as MLX would give.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    hq, lq, d = q.shape
    hkv = k.shape[0]
    assert hq % hkv == 0
    g = hq // hkv
    qg = q.reshape(hkv, g, lq, d)
    s = np.matmul(qg, k.transpose(0, 2, 1)[:, None]) * scale  # [Hkv, G, Lq, Lkv]
    if mask is not None:
        s = np.where(mask[None, None], s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    with np.errstate(invalid="ignore"):
        p = np.exp(s - m)
        o = np.matmul(p, v[:, None]) / p.sum(axis=-1, keepdims=True)
    return o.reshape(hq, lq, d)


def naive_forward_decode(
    q: np.ndarray,
    k_pool: np.ndarray,
    v_pool: np.ndarray,
    kv_indices: np.ndarray,
    mask: np.ndarray,
    scale: float,
    acc_dtype=np.float64,
) -> np.ndarray:
    """attention/naive.py:50-60: gather by padded indices, transpose, masked SDPA.

    q [B, Hq, D]; pools [N, Hkv, D]; kv_indices [B, L_max]; mask [B, L_max].
    Returns o [B, Hq, D] in ``acc_dtype`` (float64 for parity; float32 is the
    same algorithm at the reference's working precision, used for CPU timing).
    """
    k = k_pool[kv_indices].astype(acc_dtype, copy=False).transpose(0, 2, 1, 3)  # [B,Hkv,L,D]
    v = v_pool[kv_indices].astype(acc_dtype, copy=False).transpose(0, 2, 1, 3)
    b, hq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    qg = q.astype(acc_dtype, copy=False).reshape(b, hkv, g, d)
    s = np.matmul(qg, k.transpose(0, 1, 3, 2)) * acc_dtype(scale)  # [B,Hkv,G,L]
    s = np.where(mask[:, None, None, :], s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    p = np.exp(s - m)
    o = np.matmul(p, v) / p.sum(axis=-1, keepdims=True)  # [B,Hkv,G,D]
    return o.reshape(b, hq, d)


def paged_decode(
    q: np.ndarray,
    k_pool: np.ndarray,
    v_pool: np.ndarray,
    kv_indptr: np.ndarray,
    kv_indices: np.ndarray,
    scale: float,
    page_size: int = 1,
    seq_lens: Optional[np.ndarray] = None,
) -> np.ndarray:
    """Decode attention over CSR indices, one request at a time (float64).

    The semantics of ``paged_decode_attention`` (attention/metal.py:112-131):
    request b attends to pool rows kv_indices[kv_indptr[b]:kv_indptr[b+1]]
    (page_size 1). With page_size > 1 the entries are page ids and
    ``seq_lens`` gives token counts (token t at page[t//P]*P + t%P). It matches
    the reference test's per-request gather + SDPA (tests/test_attention.py:10-16).
    """
    b_count, hq, d = q.shape
    out = np.empty((b_count, hq, d), dtype=np.float64)
    for b in range(b_count):
        s, e = int(kv_indptr[b]), int(kv_indptr[b + 1])
        if page_size == 1 and seq_lens is None:
            slots = np.asarray(kv_indices[s:e], dtype=np.int64)
        else:
            length = int(seq_lens[b]) if seq_lens is not None else (e - s) * page_size
            slots = expand_page_indices(kv_indices[s:e], page_size, length)
        kb = k_pool[slots].transpose(1, 0, 2)  # [Hkv, L, D]
        vb = v_pool[slots].transpose(1, 0, 2)
        out[b] = sdpa(q[b][:, None, :], kb, vb, scale)[:, 0, :]
    return out


def forward_prefill(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    k_pool: np.ndarray,
    v_pool: np.ndarray,
    q_offsets: Sequence[int],
    kv_indices: Sequence[Optional[np.ndarray]],
    scale: float,
) -> np.ndarray:
    """attention/base.py:85-105: per-request SDPA over (cached prefix + extend).

    q [T, Hq, D]; k/v [T, Hkv, D] are this step's (already stored) rows. A
    request with no prefix (kv_indices None) attends to its own fresh k/v;
    otherwise to the pool rows kv_indices (length P + E). When E > 1 the mask is
    MLX's "causal", which is bottom-right aligned (docs/04-attention.md:35-36):
    query t of E sees keys j <= (Lkv - E) + t.
    """
    outs = []
    for i, kv_idx in enumerate(kv_indices):
        s, e = int(q_offsets[i]), int(q_offsets[i + 1])
        qi = q[s:e]
        if kv_idx is None:
            ki, vi = k[s:e], v[s:e]
        else:
            idx = np.asarray(kv_idx, dtype=np.int64)
            ki, vi = k_pool[idx], v_pool[idx]
        lq, lkv = e - s, ki.shape[0]
        mask = None
        if lq > 1:
            mask = np.arange(lkv)[None, :] <= (lkv - lq) + np.arange(lq)[:, None]
        oi = sdpa(qi.transpose(1, 0, 2), ki.transpose(1, 0, 2), vi.transpose(1, 0, 2), scale, mask)
        outs.append(oi.transpose(1, 0, 2))
    return np.concatenate(outs, axis=0)
