"""Seeded synthetic workloads for the attention path (host-side index data, numpy only).

Every generator returns plain numpy int32 index arrays; floating-point tensors
(q, K, V) are drawn by the caller with a seeded ``torch.Generator`` so the same
draw can be checked on the CPU and run on the GPU.

Constructions follow the reference's own test and tutorial:
- ``reference_test_case``: tests/test_attention.py:21-33 (pool N=4096, B=7,
  lens [1,2,17,31,32,33,700], request slots are consecutive slices of
  ``np.random.default_rng(0).permutation(N)``).
- ``decode_case``: lens ~ U_int[lo, hi] from ``default_rng(seed)``, then each
  request's pages are consecutive slices of a random permutation of the pool's
  pages (the token-granular page table of core.py:126-127 with the page layout
  of scheduler/cache.py:138-143).
- ``prefill_case``: cached prefix P ~ U_int[0, pmax], extend E ~ U_int[emin, emax],
  rescaled to a packed-token cap (E_i <- max(1, floor(E_i * cap / sum E))).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import List

import numpy as np

QWEN3_0_6B = dict(num_qo_heads=16, num_kv_heads=8, head_dim=128, num_layers=28)
QWEN3_8B = dict(num_qo_heads=32, num_kv_heads=8, head_dim=128, num_layers=36)


def _div_ceil(a: int, b: int) -> int:
    return (a + b - 1) // b


@dataclass
class DecodeCase:
    """One decode step's index data over a paged pool.

    ``page_table`` is token-granular ([B, max_len], row b = request b), exactly
    the layout of core.py:126-127. ``kv_indptr``/``kv_indices`` are the CSR
    form of attention/metal.py:145-152 (token slots). ``page_indptr``/
    ``page_ids`` are the page-granular form (page ids, Σ ceil(L/P) entries).
    """

    lens: np.ndarray  # [B] int32, includes the new token
    page_size: int
    num_slots: int
    page_table: np.ndarray  # [B, max_len] int32 token slots
    kv_indptr: np.ndarray  # [B+1] int32
    kv_indices: np.ndarray  # [sum L] int32 token slots
    page_indptr: np.ndarray  # [B+1] int32 (units: pages)
    page_ids: np.ndarray  # [sum ceil(L/P)] int32
    out_loc: np.ndarray = field(default=None)  # [B] slot of each request's newest token

    @property
    def batch_size(self) -> int:
        return int(self.lens.shape[0])


def _pages_to_case(lens: np.ndarray, page_size: int, num_slots: int, per_req_pages: List[np.ndarray]) -> DecodeCase:
    b = len(lens)
    max_len = int(lens.max()) if b else 0
    page_table = np.zeros((b, max(max_len, 1)), dtype=np.int32)
    token_lists = []
    for i, (n, pages) in enumerate(zip(lens, per_req_pages)):
        t = np.arange(int(n))
        slots = (pages[t // page_size].astype(np.int64) * page_size + t % page_size).astype(np.int32)
        page_table[i, : int(n)] = slots
        token_lists.append(slots)
    kv_indptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    kv_indices = np.concatenate(token_lists).astype(np.int32) if b else np.zeros(0, np.int32)
    npages = np.array([len(p) for p in per_req_pages], dtype=np.int64)
    page_indptr = np.concatenate([[0], np.cumsum(npages)]).astype(np.int32)
    page_ids = np.concatenate(per_req_pages).astype(np.int32) if b else np.zeros(0, np.int32)
    out_loc = np.array([page_table[i, int(n) - 1] for i, n in enumerate(lens)], dtype=np.int32)
    return DecodeCase(
        lens=lens.astype(np.int32),
        page_size=page_size,
        num_slots=num_slots,
        page_table=page_table,
        kv_indptr=kv_indptr,
        kv_indices=kv_indices,
        page_indptr=page_indptr,
        page_ids=page_ids,
        out_loc=out_loc,
    )


def reference_test_case(num_slots: int = 4096, lens=(1, 2, 17, 31, 32, 33, 700), seed: int = 0) -> DecodeCase:
    """tests/test_attention.py:21-33: consecutive slices of one slot permutation."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(num_slots).astype(np.int32)
    lens = np.asarray(lens, dtype=np.int32)
    per_req, off = [], 0
    for n in lens:
        per_req.append(perm[off : off + int(n)])
        off += int(n)
    return _pages_to_case(lens, 1, num_slots, per_req)


def decode_case(batch: int, lo: int, hi: int, num_slots: int, page_size: int = 1, seed: int = 0) -> DecodeCase:
    """Ragged decode batch: lens ~ U_int[lo, hi]; pages from one random permutation."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, size=batch).astype(np.int32)
    num_pages = num_slots // page_size
    perm = rng.permutation(num_pages).astype(np.int32)
    need = sum(_div_ceil(int(n), page_size) for n in lens)
    if need > num_pages:
        raise ValueError(f"pool of {num_slots} slots too small for {need} pages")
    per_req, off = [], 0
    for n in lens:
        p = _div_ceil(int(n), page_size)
        per_req.append(perm[off : off + p])
        off += p
    return _pages_to_case(lens, page_size, num_slots, per_req)


def decode_case_from_lens(lens, num_slots: int, page_size: int = 1, seed: int = 0) -> DecodeCase:
    """Like ``decode_case`` with explicit lengths (edge-case grids)."""
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, dtype=np.int32)
    num_pages = num_slots // page_size
    perm = rng.permutation(num_pages).astype(np.int32)
    per_req, off = [], 0
    for n in lens:
        p = _div_ceil(int(n), page_size)
        per_req.append(perm[off : off + p])
        off += p
    if off > num_pages:
        raise ValueError("pool too small")
    return _pages_to_case(lens, page_size, num_slots, per_req)


@dataclass
class PrefillCase:
    """One packed extend batch over cached prefixes in a paged pool."""

    prefix_lens: np.ndarray  # [R] cached tokens already in the pool
    extend_lens: np.ndarray  # [R] new tokens this step
    page_size: int
    num_slots: int
    page_table: np.ndarray  # [R, max(P+E)] token slots (prefix then extend)
    q_indptr: np.ndarray  # [R+1] int32 offsets into the packed q
    kv_indptr: np.ndarray  # [R+1] int32 offsets into kv_indices (token slots)
    kv_indices: np.ndarray  # [sum(P+E)] int32 token slots
    out_loc: np.ndarray  # [sum E] slots of the extend tokens
    seq_lens: np.ndarray  # [R] P + E

    @property
    def num_tokens(self) -> int:
        return int(self.extend_lens.sum())


def prefill_case_from_lens(prefix_lens, extend_lens, num_slots: int, page_size: int = 1, seed: int = 0) -> PrefillCase:
    rng = np.random.default_rng(seed)
    prefix_lens = np.asarray(prefix_lens, dtype=np.int32)
    extend_lens = np.asarray(extend_lens, dtype=np.int32)
    seq = prefix_lens + extend_lens
    num_pages = num_slots // page_size
    perm = rng.permutation(num_pages).astype(np.int32)
    max_len = int(seq.max())
    page_table = np.zeros((len(seq), max_len), dtype=np.int32)
    off = 0
    kv_lists, out_lists = [], []
    for i, n in enumerate(seq):
        p = _div_ceil(int(n), page_size)
        pages = perm[off : off + p]
        off += p
        if off > num_pages:
            raise ValueError("pool too small")
        t = np.arange(int(n))
        slots = (pages[t // page_size].astype(np.int64) * page_size + t % page_size).astype(np.int32)
        page_table[i, : int(n)] = slots
        kv_lists.append(slots)
        out_lists.append(slots[int(prefix_lens[i]) :])
    return PrefillCase(
        prefix_lens=prefix_lens,
        extend_lens=extend_lens,
        page_size=page_size,
        num_slots=num_slots,
        page_table=page_table,
        q_indptr=np.concatenate([[0], np.cumsum(extend_lens)]).astype(np.int32),
        kv_indptr=np.concatenate([[0], np.cumsum(seq)]).astype(np.int32),
        kv_indices=np.concatenate(kv_lists).astype(np.int32),
        out_loc=np.concatenate(out_lists).astype(np.int32),
        seq_lens=seq.astype(np.int32),
    )


def prefill_case(
    num_reqs: int, pmax: int, emin: int, emax: int, token_cap: int, num_slots: int, page_size: int = 1, seed: int = 0
) -> PrefillCase:
    """P ~ U_int[0, pmax], E ~ U_int[emin, emax]; if sum E > cap, E <- max(1, floor(E*cap/sum E))."""
    rng = np.random.default_rng(seed)
    prefix = rng.integers(0, pmax + 1, size=num_reqs)
    extend = rng.integers(emin, emax + 1, size=num_reqs)
    total = int(extend.sum())
    if total > token_cap:
        extend = np.maximum(1, (extend * token_cap) // total)
    return prefill_case_from_lens(prefix, extend, num_slots, page_size, seed=seed + 1)


def decode_bytes(lens: np.ndarray, hq: int, hkv: int, d: int, elem: int, page_size: int = 1) -> int:
    """Algorithmic HBM bytes of one decode layer: K+V rows, q in + o out, indices, indptr.

    bytes = ΣL·Hkv·D·e·2 + B·Hq·D·e·2 + (index entries)·4 + (B+1)·4.
    """
    lens = np.asarray(lens, dtype=np.int64)
    b = len(lens)
    kv = int(lens.sum()) * hkv * d * elem * 2
    qo = b * hq * d * elem * 2
    idx = int(sum(_div_ceil(int(n), page_size) for n in lens)) * 4
    return kv + qo + idx + (b + 1) * 4


def prefill_flops_bytes(prefix_lens, extend_lens, hq: int, hkv: int, d: int, elem: int):
    """Algorithmic flops (4·Hq·D·Σ(E·P + E(E+1)/2)) and bytes of one ragged prefill layer."""
    p = np.asarray(prefix_lens, dtype=np.int64)
    e = np.asarray(extend_lens, dtype=np.int64)
    flops = 4 * hq * d * int(np.sum(e * p + e * (e + 1) // 2))
    nbytes = int(np.sum(p + e)) * hkv * d * elem * 2 + int(e.sum()) * hq * d * elem * 2
    return flops, nbytes


@dataclass
class MixedCase:
    """A continuous-batching step over one token-granular page table.

    Requests 0..num_decode-1 decode one token (cached_len = L - 1, device_len =
    L); the others extend a chunk over a cached prefix. ``req_to_token`` is the
    scheduler's page table (core.py:126-127, engine/engine.py:74) with requests
    on shuffled rows ``table_idx``; each request's pages are consecutive slices
    of one random permutation of the pool's pages (scheduler/cache.py:138-143).
    Positions [cached_len, device_len) of every request are this step's tokens,
    their slots already allocated in the table (scheduler/cache.py:53-72).
    """

    req_to_token: np.ndarray  # [num_rows, max_len] int32
    table_idx: np.ndarray  # [R] int32
    cached_len: np.ndarray  # [R] int32
    device_len: np.ndarray  # [R] int32
    num_decode: int
    page_size: int
    num_slots: int

    @property
    def num_reqs(self) -> int:
        return int(self.device_len.shape[0])

    @property
    def num_tokens(self) -> int:
        return int((self.device_len - self.cached_len).sum())

    @property
    def num_pages(self) -> int:
        return int(sum(_div_ceil(int(n), self.page_size) for n in self.device_len))

    @property
    def max_chunk(self) -> int:
        e = self.device_len[self.num_decode :] - self.cached_len[self.num_decode :]
        return int(e.max()) if len(e) else 0

    def slots(self, i: int) -> np.ndarray:
        """Token slots of request i's full context (table row, first device_len entries)."""
        return self.req_to_token[self.table_idx[i], : int(self.device_len[i])]


def mixed_case(
    num_decode: int,
    dec_lo: int,
    dec_hi: int,
    prefill_prefixes,
    chunk,
    num_slots: int,
    page_size: int = 16,
    seed: int = 0,
) -> MixedCase:
    """num_decode decode requests with L ~ U_int[dec_lo, dec_hi], then one chunk of
    ``chunk`` tokens over each prefix in ``prefill_prefixes`` (``chunk``: one
    length for all, or one per prefix)."""
    rng = np.random.default_rng(seed)
    dec = rng.integers(dec_lo, dec_hi + 1, size=num_decode).astype(np.int64)
    pre = np.asarray(prefill_prefixes, dtype=np.int64)
    chunks = np.broadcast_to(np.asarray(chunk, dtype=np.int64), pre.shape)
    device_len = np.concatenate([dec, pre + chunks]).astype(np.int32)
    cached_len = np.concatenate([dec - 1, pre]).astype(np.int32)
    r = len(device_len)
    num_pages = num_slots // page_size
    need = sum(_div_ceil(int(n), page_size) for n in device_len)
    if need > num_pages:
        raise ValueError(f"pool of {num_slots} slots too small for {need} pages")
    perm = rng.permutation(num_pages).astype(np.int64)
    num_rows = r + 2
    max_len = _div_ceil(int(device_len.max()), page_size) * page_size
    table = np.zeros((num_rows, max_len), dtype=np.int32)
    table_idx = rng.permutation(num_rows)[:r].astype(np.int32)
    off = 0
    for i, n in enumerate(device_len):
        p = _div_ceil(int(n), page_size)
        pages = perm[off : off + p]
        off += p
        table[table_idx[i], : p * page_size] = (pages[:, None] * page_size + np.arange(page_size)).reshape(-1)
    return MixedCase(table, table_idx, cached_len, device_len, num_decode, page_size, num_slots)
