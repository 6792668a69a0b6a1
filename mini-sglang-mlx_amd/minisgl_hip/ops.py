"""torch-facing wrappers of the HIP kernels (argument checks + one C-ABI call each).

Tensors stay on the caller's device; work is enqueued on the current stream
and nothing synchronises. Preconditions raise ``ValueError`` like the
reference's asserts (attention/metal.py:122); kernel/runtime failures raise
``RuntimeError`` with the library's message.
"""

from __future__ import annotations

import weakref
from typing import Optional, Union

import torch

from . import _lib


def _check_device(name: str, t: torch.Tensor, device: torch.device) -> None:
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _check_index(name: str, t: Optional[torch.Tensor], device: torch.device) -> None:
    if t is None:
        return
    if t.dtype != torch.int32:
        raise ValueError(f"{name} must be int32 (got {t.dtype})")
    _check_device(name, t, device)


# id(tensor) -> (weak reference, tensor version, value) of device scales already read
_SCALE_CACHE: dict = {}


def scale_value(scale: Union[float, torch.Tensor]) -> float:
    """The softmax scale as a float. The reference passes it as a one-element
    array (attention/metal.py:143); a device tensor is read once (one host
    sync) and the value is reused for as long as that tensor is alive and
    unchanged (its version counter), so layers that share a scale tensor do not
    synchronise per call."""
    if not isinstance(scale, torch.Tensor):
        return float(scale)
    if scale.numel() != 1:
        raise ValueError(f"scale must have one element (got shape {tuple(scale.shape)})")
    if scale.device.type == "cpu":
        return float(scale.reshape(-1)[0])
    hit = _SCALE_CACHE.get(id(scale))
    if hit is not None and hit[0]() is scale and hit[1] == scale._version:
        return hit[2]
    value = float(scale.reshape(-1)[0].item())
    key = id(scale)
    _SCALE_CACHE[key] = (weakref.ref(scale, lambda _r, k=key: _SCALE_CACHE.pop(k, None)), scale._version, value)
    return value


def store_kv(
    k: torch.Tensor, v: torch.Tensor, out_loc: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor
) -> None:
    """k_pool[out_loc] = k; v_pool[out_loc] = v (kvcache/pool.py:47-50), in place."""
    if k.dim() != 3 or k.shape != v.shape:
        raise ValueError(f"k/v must both be [T, Hkv, D] (got {tuple(k.shape)}, {tuple(v.shape)})")
    if k_pool.dim() != 3 or k_pool.shape != v_pool.shape or k_pool.shape[1:] != k.shape[1:]:
        raise ValueError(f"pools must be [N, Hkv, D] matching k (got {tuple(k_pool.shape)})")
    if out_loc.dim() != 1 or out_loc.shape[0] != k.shape[0]:
        raise ValueError("out_loc must be [T]")
    if len({k.dtype, v.dtype, k_pool.dtype, v_pool.dtype}) != 1:
        raise ValueError("k, v and pools must share one dtype")
    dev = k_pool.device
    for name, t in (("k", k), ("v", v), ("k_pool", k_pool), ("v_pool", v_pool)):
        _check_device(name, t, dev)
    _check_index("out_loc", out_loc, dev)
    lib = _lib.load()
    status = lib.msgl_store_kv(
        _lib.ptr(k), _lib.ptr(v), _lib.ptr(out_loc), _lib.ptr(k_pool), _lib.ptr(v_pool),
        k.shape[0], k.shape[1], k.shape[2], k_pool.shape[0], _lib.dtype_code(k.dtype),
        _lib.current_stream(dev),
    )
    _lib.check(status, "msgl_store_kv")


def store_kv_fp8(
    k: torch.Tensor, v: torch.Tensor, out_loc: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
    kv_scale: torch.Tensor,
) -> None:
    """kvcache/pool.py:47-50 into an fp8 pool: per (token, kv head) row, codes
    e4m3(x * 448 / amax) in k_pool/v_pool (``torch.float8_e4m3fn`` [N, Hkv, D])
    and scale amax / 448 in kv_scale (float32 [N, Hkv, 2]: K scale, V scale), in place."""
    if k.dim() != 3 or k.shape != v.shape:
        raise ValueError(f"k/v must both be [T, Hkv, D] (got {tuple(k.shape)}, {tuple(v.shape)})")
    if k_pool.dtype != torch.float8_e4m3fn or v_pool.dtype != torch.float8_e4m3fn:
        raise ValueError("pools must be torch.float8_e4m3fn")
    if k_pool.dim() != 3 or k_pool.shape != v_pool.shape or k_pool.shape[1:] != k.shape[1:]:
        raise ValueError(f"pools must be [N, Hkv, D] matching k (got {tuple(k_pool.shape)})")
    n, hkv = k_pool.shape[:2]
    if kv_scale.dtype != torch.float32 or kv_scale.shape != (n, hkv, 2):
        raise ValueError("kv_scale must be float32 [N, Hkv, 2]")
    if out_loc.shape != (k.shape[0],):
        raise ValueError("out_loc must be [T]")
    if k.dtype != v.dtype:
        raise ValueError("k and v must share one dtype")
    dev = k_pool.device
    for name, t in (("k", k), ("v", v), ("k_pool", k_pool), ("v_pool", v_pool), ("kv_scale", kv_scale)):
        _check_device(name, t, dev)
    _check_index("out_loc", out_loc, dev)
    status = _lib.load().msgl_store_kv_fp8(
        _lib.ptr(k), _lib.ptr(v), _lib.ptr(out_loc), _lib.ptr(k_pool), _lib.ptr(v_pool), _lib.ptr(kv_scale),
        k.shape[0], k.shape[1], k.shape[2], n, _lib.dtype_code(k.dtype), _lib.current_stream(dev),
    )
    _lib.check(status, "msgl_store_kv_fp8")


def default_splits(batch: int, num_kv_heads: int, max_seq_len: int = 0) -> int:
    return int(_lib.load().msgl_paged_decode_default_splits(batch, num_kv_heads, max_seq_len))


# Resident 4-wavefront decode workgroups of MI355X (256 CUs x 3 at the decode
# kernel's register budget): a shared-head launch needs this many (request, kv
# head) pairs to fill the device.
SHARED_HEAD_MIN_UNITS = 768


def decode_splits_for(lens, num_kv_heads: int) -> int:
    """max_splits for a decode batch whose lengths the caller knows (host array).

    1 -- the shared-head form: the four wavefronts of a workgroup split one
    (request, kv head)'s keys and combine in LDS, one launch and no merge --
    when the pairs fill the device, no wavefront gets more than 512 keys and the
    lengths are near-uniform (longest <= 1.25 x mean: a ragged batch leaves
    wavefronts of short requests idle while long ones run, where the split form
    balances chunks of <= 512 keys). Otherwise the library default."""
    import numpy as np

    lens = np.asarray(lens, dtype=np.int64)
    b = len(lens)
    mx = int(lens.max()) if b else 0
    if (b * num_kv_heads >= SHARED_HEAD_MIN_UNITS and 0 < mx <= 2048 and mx <= 1.25 * float(lens.mean())):
        return 1
    return default_splits(b, num_kv_heads, mx)


def decode_workspace_bytes(batch: int, num_qo_heads: int, num_kv_heads: int, head_dim: int, max_splits: int) -> int:
    return int(
        _lib.load().msgl_paged_decode_workspace_size(batch, num_qo_heads, num_kv_heads, head_dim, max_splits)
    )


def decode_workspace(batch: int, num_qo_heads: int, num_kv_heads: int, head_dim: int, max_splits: int,
                     device) -> Optional[torch.Tensor]:
    """A workspace for ``paged_decode_attention`` (None when no split-K).

    Consecutive calls on one stream may reuse it; overlapping calls may not.
    """
    need = decode_workspace_bytes(batch, num_qo_heads, num_kv_heads, head_dim, max_splits)
    if need == 0:
        return None
    return torch.empty(need, dtype=torch.uint8, device=device)


def prefill_default_splits(num_reqs: int, num_qo_heads: int, num_kv_heads: int, head_dim: int,
                           max_extend_len: int, max_seq_len: int = 0) -> int:
    return int(_lib.load().msgl_prefill_default_splits(num_reqs, num_qo_heads, num_kv_heads, head_dim,
                                                       max_extend_len, max_seq_len))


def prefill_workspace_bytes(num_reqs: int, num_tokens: int, max_extend_len: int, num_qo_heads: int,
                            num_kv_heads: int, head_dim: int, max_splits: int) -> int:
    return int(_lib.load().msgl_prefill_workspace_size(num_reqs, num_tokens, max_extend_len, num_qo_heads,
                                                       num_kv_heads, head_dim, max_splits))


def prefill_workspace(num_reqs: int, num_tokens: int, max_extend_len: int, num_qo_heads: int, num_kv_heads: int,
                      head_dim: int, max_splits: int, device) -> Optional[torch.Tensor]:
    """A workspace for ``prefill_ragged_attention`` (bf16/fp16).

    Consecutive calls on one stream may reuse it; overlapping calls may not.
    """
    need = prefill_workspace_bytes(num_reqs, num_tokens, max_extend_len, num_qo_heads, num_kv_heads, head_dim,
                                   max_splits)
    if need == 0:
        return None
    return torch.empty(need, dtype=torch.uint8, device=device)


def paged_decode_plan(
    kv_indptr: torch.Tensor,
    seq_lens: Optional[torch.Tensor],
    batch: int,
    num_qo_heads: int,
    num_kv_heads: int,
    head_dim: int,
    max_splits: int,
    workspace: torch.Tensor,
) -> None:
    """Build the decode work list for these indices into ``workspace`` (reused by
    every ``paged_decode_attention(..., planned=True)`` call over them)."""
    dev = workspace.device
    _check_index("kv_indptr", kv_indptr, dev)
    _check_index("seq_lens", seq_lens, dev)
    if kv_indptr.dim() != 1 or kv_indptr.shape[0] < batch + 1:
        raise ValueError("kv_indptr must be [B+1]")
    status = _lib.load().msgl_paged_decode_plan(
        _lib.ptr(kv_indptr), _lib.ptr(seq_lens), batch, num_qo_heads, num_kv_heads, head_dim, max_splits,
        _lib.ptr(workspace), workspace.numel() * workspace.element_size(), _lib.current_stream(dev),
    )
    _lib.check(status, "msgl_paged_decode_plan")
    # the sizes this plan is for: a planned call with other sizes is rejected
    workspace._msgl_decode_plan = (batch, num_kv_heads, max_splits)


def paged_decode_attention(
    q: torch.Tensor,
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    kv_indptr: torch.Tensor,
    kv_indices: torch.Tensor,
    scale: Union[float, torch.Tensor],
    *,
    seq_lens: Optional[torch.Tensor] = None,
    page_size: int = 1,
    max_splits: Optional[int] = None,
    max_seq_len: int = 0,
    out: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
    new_kv: Optional[tuple] = None,
    planned: bool = False,
    kv_scale: Optional[torch.Tensor] = None,
    merge: bool = True,
) -> torch.Tensor:
    """Paged decode attention; counterpart of attention/metal.py:112-131.

    ``merge=False`` (with ``planned``) launches the decode kernel only; the
    rows of requests cut into several chunks are then completed by
    ``paged_decode_merge`` with the same arguments (msgl_paged_decode_planned_ex
    with MSGL_DECODE_NO_MERGE, then msgl_paged_decode_merge).

    fp8 pools (``torch.float8_e4m3fn``, written by ``store_kv_fp8``) take
    ``kv_scale`` (float32 [N, Hkv, 2]: K scale, V scale); q is bf16/fp16 and the
    result is the decode over the dequantised pool. With ``new_kv`` the launch
    quantises and stores the new rows exactly as ``store_kv_fp8`` would.

    q [B, Hq, D]; pools [N, Hkv, D]; kv_indptr [B+1] int32; kv_indices int32
    (token slots, or page ids when page_size > 1 with seq_lens [B] given).
    Returns o [B, Hq, D] in q's dtype. ``workspace`` (from ``decode_workspace``)
    is allocated per call when not given. With ``new_kv = (k_new, v_new,
    out_loc)`` the KV store of this step's rows (kvcache/pool.py:47-50) runs in
    the same launch: k_pool[out_loc] = k_new, v_pool[out_loc] = v_new, where
    out_loc[b] is the slot of request b's last position. With ``planned`` the
    workspace already holds the work list built by ``paged_decode_plan`` for
    these indices and sizes (one launch fewer per call).
    """
    if q.dim() != 3 or k_pool.dim() != 3 or k_pool.shape != v_pool.shape:
        raise ValueError("q must be [B, Hq, D] and pools [N, Hkv, D]")
    b, hq, d = q.shape
    n_slots, hkv, dk = k_pool.shape
    if dk != d or hq % hkv != 0:
        raise ValueError(f"head_dim mismatch or Hq ({hq}) not a multiple of Hkv ({hkv})")
    fp8 = k_pool.dtype == torch.float8_e4m3fn
    if fp8:
        if v_pool.dtype != k_pool.dtype or kv_scale is None:
            raise ValueError("fp8 pools need both pools fp8 and kv_scale")
        if q.dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("fp8 pools take bf16 or fp16 queries")
        if kv_scale.dtype != torch.float32 or kv_scale.shape != (n_slots, hkv, 2):
            raise ValueError("kv_scale must be float32 [N, Hkv, 2]")
        _check_device("kv_scale", kv_scale, q.device)
    elif len({q.dtype, k_pool.dtype, v_pool.dtype}) != 1:
        raise ValueError("q and pools must share one dtype")
    if page_size > 1 and seq_lens is None:
        raise ValueError("page_size > 1 needs seq_lens")
    if kv_indptr.dim() != 1 or kv_indptr.shape[0] < b + 1:
        raise ValueError("kv_indptr must be [B+1] (kv_indptr[B] = entries of kv_indices)")
    dev = q.device
    for name, t in (("q", q), ("k_pool", k_pool), ("v_pool", v_pool)):
        _check_device(name, t, dev)
    for name, t in (("kv_indptr", kv_indptr), ("kv_indices", kv_indices), ("seq_lens", seq_lens)):
        _check_index(name, t, dev)
    scale = scale_value(scale)
    if out is None:
        out = torch.empty_like(q)
    else:
        _check_device("out", out, dev)
        if out.shape != q.shape or out.dtype != q.dtype:
            raise ValueError("out must match q's shape and dtype")
    lib = _lib.load()
    if max_splits is None:
        max_splits = int(lib.msgl_paged_decode_default_splits(b, hkv, max_seq_len))
    need = int(lib.msgl_paged_decode_workspace_size(b, hq, hkv, d, max_splits))
    if need > 0 and (workspace is None or workspace.numel() * workspace.element_size() < need):
        if planned:
            raise ValueError("planned decode needs the workspace its plan was built in")
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    if planned and getattr(workspace, "_msgl_decode_plan", None) != (b, hkv, max_splits):
        raise ValueError(
            f"planned decode: the workspace holds no plan for batch {b}, {hkv} kv heads, max_splits {max_splits} "
            f"(plan: {getattr(workspace, '_msgl_decode_plan', None)})"
        )
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    common = (
        _lib.ptr(kv_indptr), _lib.ptr(kv_indices), _lib.ptr(seq_lens),
        b, hq, hkv, d, page_size, n_slots, _lib.dtype_code(q.dtype), float(scale),
        max_splits, _lib.ptr(out), _lib.ptr(workspace), ws_bytes, _lib.current_stream(dev),
    )
    if not merge:
        if not planned:
            raise ValueError("merge=False needs a planned call (the merge reads the plan)")
        k_new = v_new = out_loc = None
        if new_kv is not None:
            k_new, v_new, out_loc = new_kv
            if k_new.shape != (b, hkv, d) or v_new.shape != (b, hkv, d) or out_loc.shape != (b,):
                raise ValueError("k_new/v_new must be [B, Hkv, D] and out_loc [B]")
            if k_new.dtype != q.dtype or v_new.dtype != q.dtype:
                raise ValueError("k_new/v_new must share q's dtype")
            for name, t in (("k_new", k_new), ("v_new", v_new)):
                _check_device(name, t, dev)
            _check_index("out_loc", out_loc, dev)
        status = lib.msgl_paged_decode_planned_ex(
            _lib.ptr(q), _lib.ptr(k_new), _lib.ptr(v_new), _lib.ptr(out_loc), _lib.ptr(k_pool), _lib.ptr(v_pool),
            _lib.ptr(kv_scale), *common[:12], _lib.MSGL_DECODE_NO_MERGE, *common[12:],
        )
        _lib.check(status, "msgl_paged_decode_planned_ex")
        return out
    if fp8 and new_kv is None:
        fn = lib.msgl_paged_decode_fp8_planned if planned else lib.msgl_paged_decode_fp8
        status = fn(_lib.ptr(q), _lib.ptr(k_pool), _lib.ptr(v_pool), _lib.ptr(kv_scale), *common)
        _lib.check(status, "msgl_paged_decode_fp8")
    elif new_kv is None:
        fn = lib.msgl_paged_decode_planned if planned else lib.msgl_paged_decode
        status = fn(_lib.ptr(q), _lib.ptr(k_pool), _lib.ptr(v_pool), *common)
        _lib.check(status, "msgl_paged_decode")
    else:
        k_new, v_new, out_loc = new_kv
        if k_new.shape != (b, hkv, d) or v_new.shape != (b, hkv, d) or out_loc.shape != (b,):
            raise ValueError("k_new/v_new must be [B, Hkv, D] and out_loc [B]")
        if k_new.dtype != q.dtype or v_new.dtype != q.dtype:
            raise ValueError("k_new/v_new must share q's dtype")
        for name, t in (("k_new", k_new), ("v_new", v_new)):
            _check_device(name, t, dev)
        _check_index("out_loc", out_loc, dev)
        if fp8:
            fn = lib.msgl_paged_decode_store_fp8_planned if planned else lib.msgl_paged_decode_store_fp8
            status = fn(
                _lib.ptr(q), _lib.ptr(k_new), _lib.ptr(v_new), _lib.ptr(out_loc), _lib.ptr(k_pool), _lib.ptr(v_pool),
                _lib.ptr(kv_scale), *common,
            )
            _lib.check(status, "msgl_paged_decode_store_fp8")
        else:
            fn = lib.msgl_paged_decode_store_planned if planned else lib.msgl_paged_decode_store
            status = fn(
                _lib.ptr(q), _lib.ptr(k_new), _lib.ptr(v_new), _lib.ptr(out_loc), _lib.ptr(k_pool), _lib.ptr(v_pool),
                *common,
            )
            _lib.check(status, "msgl_paged_decode_store")
    return out


def paged_decode_merge(
    out: torch.Tensor,
    kv_indptr: torch.Tensor,
    seq_lens: Optional[torch.Tensor],
    num_kv_heads: int,
    max_splits: int,
    workspace: torch.Tensor,
    kv_fp8: bool = False,
) -> torch.Tensor:
    """The split-K merge of a ``paged_decode_attention(..., planned=True,
    merge=False)`` call with the same indices, sizes and workspace (``kv_fp8``:
    that call ran over fp8 pools): completes ``out`` [B, Hq, D] in place
    (msgl_paged_decode_merge)."""
    b, hq, d = out.shape
    dev = out.device
    _check_device("out", out, dev)
    _check_index("kv_indptr", kv_indptr, dev)
    _check_index("seq_lens", seq_lens, dev)
    if getattr(workspace, "_msgl_decode_plan", None) != (b, num_kv_heads, max_splits):
        raise ValueError("paged_decode_merge: the workspace holds no plan for these sizes")
    status = _lib.load().msgl_paged_decode_merge(
        _lib.ptr(kv_indptr), _lib.ptr(seq_lens), b, hq, num_kv_heads, d, _lib.dtype_code(out.dtype), int(kv_fp8),
        int(max_splits), _lib.ptr(out), _lib.ptr(workspace), workspace.numel() * workspace.element_size(),
        _lib.current_stream(dev),
    )
    _lib.check(status, "msgl_paged_decode_merge")
    return out


def prefill_ragged_attention(
    q: torch.Tensor,
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    q_indptr: torch.Tensor,
    kv_indptr: torch.Tensor,
    kv_indices: torch.Tensor,
    seq_lens: Optional[torch.Tensor],
    scale: Union[float, torch.Tensor],
    *,
    max_extend_len: int,
    max_seq_len: int = 0,
    page_size: int = 1,
    max_splits: Optional[int] = None,
    out: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
    planned: bool = False,
    kv_scale: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Ragged prefill over cached prefixes; counterpart of attention/base.py:85-105.

    q [T, Hq, D] packed; request i owns q rows q_indptr[i]:q_indptr[i+1] and
    attends (bottom-right causal) to the first seq_lens[i] tokens of its KV at
    kv_indices[kv_indptr[i]:] (token slots, or page ids when page_size > 1).
    ``max_extend_len`` must bound every request's extend length (host-known);
    ``max_seq_len`` (max total length, 0 = unknown) only tunes the key-range
    split (its default and the chunk length). ``workspace`` (from ``prefill_workspace``) is allocated per
    call when the split needs one and none large enough is given. With ``planned`` the workspace
    already holds the work list ``prefill_plan`` built for these indices and sizes.
    fp8 pools (``torch.float8_e4m3fn``, written by ``store_kv_fp8``) take ``kv_scale``
    (float32 [N, Hkv, 2]) and bf16/fp16 queries.
    """
    if q.dim() != 3 or k_pool.dim() != 3 or k_pool.shape != v_pool.shape:
        raise ValueError("q must be [T, Hq, D] and pools [N, Hkv, D]")
    t, hq, d = q.shape
    n_slots, hkv, dk = k_pool.shape
    if dk != d or hq % hkv != 0:
        raise ValueError(f"head_dim mismatch or Hq ({hq}) not a multiple of Hkv ({hkv})")
    fp8 = k_pool.dtype == torch.float8_e4m3fn
    if fp8:
        if v_pool.dtype != k_pool.dtype or kv_scale is None:
            raise ValueError("fp8 pools need both pools fp8 and kv_scale")
        if q.dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("fp8 pools take bf16 or fp16 queries")
        if kv_scale.dtype != torch.float32 or kv_scale.shape != (n_slots, hkv, 2):
            raise ValueError("kv_scale must be float32 [N, Hkv, 2]")
        _check_device("kv_scale", kv_scale, q.device)
    elif len({q.dtype, k_pool.dtype, v_pool.dtype}) != 1:
        raise ValueError("q and pools must share one dtype")
    if page_size > 1 and seq_lens is None:
        raise ValueError("page_size > 1 needs seq_lens")
    if q_indptr.dim() != 1 or q_indptr.shape[0] < 2:
        raise ValueError("q_indptr must be [R+1]")
    num_reqs = q_indptr.shape[0] - 1
    if kv_indptr.dim() != 1 or kv_indptr.shape[0] < num_reqs + 1:
        raise ValueError("kv_indptr must be [R+1] (kv_indptr[R] = entries of kv_indices)")
    dev = q.device
    for name, x in (("q", q), ("k_pool", k_pool), ("v_pool", v_pool)):
        _check_device(name, x, dev)
    for name, x in (("q_indptr", q_indptr), ("kv_indptr", kv_indptr), ("kv_indices", kv_indices),
                    ("seq_lens", seq_lens)):
        _check_index(name, x, dev)
    scale = scale_value(scale)
    if out is None:
        out = torch.empty_like(q)
    else:
        _check_device("out", out, dev)
        if out.shape != q.shape or out.dtype != q.dtype:
            raise ValueError("out must match q's shape and dtype")
    if t == 0:
        return out
    lib = _lib.load()
    if max_splits is None:
        max_splits = prefill_default_splits(num_reqs, hq, hkv, d, int(max_extend_len), int(max_seq_len))
    need = (prefill_workspace_bytes(num_reqs, t, int(max_extend_len), hq, hkv, d, max_splits)
            if q.dtype != torch.float32 else 0)
    if need > 0 and (workspace is None or workspace.numel() * workspace.element_size() < need):
        if planned:
            raise ValueError("planned prefill needs the workspace its plan was built in")
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    plan_key = (num_reqs, t, int(max_extend_len), int(max_seq_len), hq, hkv, d, int(max_splits))
    if planned and need > 0 and getattr(workspace, "_msgl_prefill_plan", None) != plan_key:
        raise ValueError(
            f"planned prefill: the workspace holds no plan for {plan_key} "
            f"(plan: {getattr(workspace, '_msgl_prefill_plan', None)})"
        )
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    if fp8:
        fn = lib.msgl_prefill_ragged_fp8_planned if planned else lib.msgl_prefill_ragged_fp8
        pools = (_lib.ptr(q), _lib.ptr(k_pool), _lib.ptr(v_pool), _lib.ptr(kv_scale))
    else:
        fn = lib.msgl_prefill_ragged_planned if planned else lib.msgl_prefill_ragged
        pools = (_lib.ptr(q), _lib.ptr(k_pool), _lib.ptr(v_pool))
    status = fn(
        *pools,
        _lib.ptr(q_indptr), _lib.ptr(kv_indptr), _lib.ptr(kv_indices), _lib.ptr(seq_lens),
        num_reqs, t, int(max_extend_len), int(max_seq_len), hq, hkv, d, page_size, n_slots, _lib.dtype_code(q.dtype), float(scale),
        int(max_splits), _lib.ptr(out), _lib.ptr(workspace), ws_bytes, _lib.current_stream(dev),
    )
    _lib.check(status, "msgl_prefill_ragged")
    return out


def prefill_plan(
    q_indptr: torch.Tensor,
    kv_indptr: torch.Tensor,
    seq_lens: Optional[torch.Tensor],
    *,
    num_tokens: int,
    max_extend_len: int,
    max_seq_len: int,
    num_qo_heads: int,
    num_kv_heads: int,
    head_dim: int,
    dtype: torch.dtype,
    max_splits: int,
    workspace: torch.Tensor,
) -> None:
    """Build the ragged prefill's work list into ``workspace`` once for a batch;
    every layer then calls ``prefill_ragged_attention(..., planned=True)`` with
    the same indices, sizes and workspace."""
    dev = workspace.device
    for name, x in (("q_indptr", q_indptr), ("kv_indptr", kv_indptr), ("seq_lens", seq_lens)):
        _check_index(name, x, dev)
    if kv_indptr.dim() != 1 or kv_indptr.shape[0] < q_indptr.shape[0]:
        raise ValueError("kv_indptr must be [R+1]")
    status = _lib.load().msgl_prefill_plan(
        _lib.ptr(q_indptr), _lib.ptr(kv_indptr), _lib.ptr(seq_lens), q_indptr.shape[0] - 1, int(num_tokens),
        int(max_extend_len), int(max_seq_len), num_qo_heads, num_kv_heads, head_dim, _lib.dtype_code(dtype),
        int(max_splits), _lib.ptr(workspace), workspace.numel() * workspace.element_size(), _lib.current_stream(dev),
    )
    _lib.check(status, "msgl_prefill_plan")
    workspace._msgl_prefill_plan = (q_indptr.shape[0] - 1, int(num_tokens), int(max_extend_len), int(max_seq_len),
                                    num_qo_heads, num_kv_heads, head_dim, int(max_splits))


def mixed_attention(
    q: torch.Tensor,
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    scale: float,
    *,
    num_decode: int,
    dec_kv_indptr: torch.Tensor,
    dec_kv_indices: torch.Tensor,
    dec_seq_lens: Optional[torch.Tensor],
    dec_max_splits: int,
    dec_workspace: torch.Tensor,
    new_kv: Optional[tuple],
    q_indptr: torch.Tensor,
    pf_kv_indptr: torch.Tensor,
    pf_kv_indices: torch.Tensor,
    pf_seq_lens: Optional[torch.Tensor],
    max_extend_len: int,
    max_seq_len: int,
    pf_max_splits: int,
    pf_workspace: torch.Tensor,
    page_size: int = 1,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """A mixed batch's decode and prefill attention in one launch (+ one merge launch).

    q/out: the packed [T, Hq, D] batch, decode requests first (rows [0, num_decode),
    one token each), the prefill chunks after them at the packed offsets of
    ``q_indptr``. ``new_kv = (k_new, v_new, out_loc)`` ([num_decode, Hkv, D] and
    [num_decode]) stores the decode requests' new rows in the same launch. The
    work lists must already be in the workspaces (``paged_decode_plan`` and
    ``prefill_plan`` over the same indices). Per request the result is that of
    ``paged_decode_attention`` / ``prefill_ragged_attention``."""
    if q.dim() != 3 or k_pool.dim() != 3 or k_pool.shape != v_pool.shape:
        raise ValueError("q must be [T, Hq, D] and pools [N, Hkv, D]")
    t, hq, d = q.shape
    n_slots, hkv, dk = k_pool.shape
    if dk != d or hq % hkv != 0 or len({q.dtype, k_pool.dtype, v_pool.dtype}) != 1:
        raise ValueError("q and pools must share head_dim and dtype, Hq a multiple of Hkv")
    if not 0 <= num_decode <= t:
        raise ValueError("num_decode must be in [0, T]")
    dev = q.device
    for name, x in (("q", q), ("k_pool", k_pool), ("v_pool", v_pool)):
        _check_device(name, x, dev)
    for name, x in (("dec_kv_indptr", dec_kv_indptr), ("dec_kv_indices", dec_kv_indices),
                    ("dec_seq_lens", dec_seq_lens), ("q_indptr", q_indptr), ("pf_kv_indptr", pf_kv_indptr),
                    ("pf_kv_indices", pf_kv_indices), ("pf_seq_lens", pf_seq_lens)):
        _check_index(name, x, dev)
    if out is None:
        out = torch.empty_like(q)
    elif out.shape != q.shape or out.dtype != q.dtype:
        raise ValueError("out must match q's shape and dtype")
    num_prefill = q_indptr.shape[0] - 1
    if num_decode and getattr(dec_workspace, "_msgl_decode_plan", None) != (num_decode, hkv, int(dec_max_splits)):
        raise ValueError("mixed attention: dec_workspace holds no decode plan for these sizes")
    pf_key = (num_prefill, t, int(max_extend_len), int(max_seq_len), hq, hkv, d, int(pf_max_splits))
    if num_prefill and getattr(pf_workspace, "_msgl_prefill_plan", None) != pf_key:
        raise ValueError("mixed attention: pf_workspace holds no prefill plan for these sizes")
    k_new = v_new = out_loc = None
    if new_kv is not None:
        k_new, v_new, out_loc = new_kv
        if k_new.shape != (num_decode, hkv, d) or v_new.shape != k_new.shape or out_loc.shape != (num_decode,):
            raise ValueError("k_new/v_new must be [num_decode, Hkv, D] and out_loc [num_decode]")
        if k_new.dtype != q.dtype or v_new.dtype != q.dtype:
            raise ValueError("k_new/v_new must share q's dtype")
        _check_device("k_new", k_new, dev)
        _check_device("v_new", v_new, dev)
        _check_index("out_loc", out_loc, dev)
    status = _lib.load().msgl_mixed_attention(
        _lib.ptr(q), _lib.ptr(k_new), _lib.ptr(v_new), _lib.ptr(out_loc), _lib.ptr(dec_kv_indptr),
        _lib.ptr(dec_kv_indices), _lib.ptr(dec_seq_lens), int(num_decode), int(dec_max_splits), _lib.ptr(out),
        _lib.ptr(dec_workspace), dec_workspace.numel() * dec_workspace.element_size(),
        _lib.ptr(q), _lib.ptr(q_indptr), _lib.ptr(pf_kv_indptr), _lib.ptr(pf_kv_indices), _lib.ptr(pf_seq_lens),
        q_indptr.shape[0] - 1, t, int(max_extend_len), int(max_seq_len), int(pf_max_splits), _lib.ptr(out),
        _lib.ptr(pf_workspace), pf_workspace.numel() * pf_workspace.element_size(),
        _lib.ptr(k_pool), _lib.ptr(v_pool), hq, hkv, d, int(page_size), n_slots, _lib.dtype_code(q.dtype),
        float(scale), _lib.current_stream(dev),
    )
    _lib.check(status, "msgl_mixed_attention")
    return out


def build_step_indices(
    req_to_token: torch.Tensor,
    table_idx: torch.Tensor,
    cached_len: torch.Tensor,
    device_len: torch.Tensor,
    *,
    num_tokens: int,
    num_kv: int,
    page_size: int = 1,
    host_lens: Optional[tuple] = None,
) -> dict:
    """Step metadata built on the GPU from a device page table.

    Counterpart of scheduler/scheduler.py:154-157 (positions, out_loc),
    attention/base.py:70-83 (q_indptr = q_offsets, last_indices) and
    attention/metal.py:145-152 (kv_indptr, kv_indices; page ids of
    ceil(L / page_size) pages when page_size > 1). ``num_tokens`` =
    sum(device_len - cached_len) and ``num_kv`` = sum of (page-)lengths are
    host-known sizes of the outputs; ``host_lens`` = (cached_len, device_len)
    host arrays checks them first (``check_step_sizes``). Returns device int32
    tensors.
    """
    if host_lens is not None:
        check_step_sizes(host_lens[0], host_lens[1], page_size, num_tokens, num_kv)
    if req_to_token.dim() != 2:
        raise ValueError("req_to_token must be [rows, max_seq_len]")
    r = table_idx.shape[0]
    if cached_len.shape != (r,) or device_len.shape != (r,):
        raise ValueError("table_idx, cached_len and device_len must all be [R]")
    dev = req_to_token.device
    for name, t in (("req_to_token", req_to_token), ("table_idx", table_idx), ("cached_len", cached_len),
                    ("device_len", device_len)):
        _check_index(name, t, dev)
    i32 = dict(dtype=torch.int32, device=dev)
    out = {
        "q_indptr": torch.empty(r + 1, **i32),
        "positions": torch.empty(num_tokens, **i32),
        "out_loc": torch.empty(num_tokens, **i32),
        "last_indices": torch.empty(r, **i32),
        "kv_indptr": torch.empty(r + 1, **i32),
        "kv_indices": torch.empty(num_kv, **i32),
    }
    if r == 0:
        out["q_indptr"].zero_()
        out["kv_indptr"].zero_()
        return out
    status = _lib.load().msgl_build_step_indices(
        _lib.ptr(req_to_token), req_to_token.shape[0], req_to_token.shape[1],
        _lib.ptr(table_idx), _lib.ptr(cached_len), _lib.ptr(device_len), r, page_size,
        _lib.ptr(out["q_indptr"]), _lib.ptr(out["positions"]), _lib.ptr(out["out_loc"]),
        _lib.ptr(out["last_indices"]), num_tokens,
        _lib.ptr(out["kv_indptr"]), _lib.ptr(out["kv_indices"]), num_kv, _lib.current_stream(dev),
    )
    _lib.check(status, "msgl_build_step_indices")
    return out


def profile_next_launch(start: Optional["torch.cuda.Event"], stop: Optional["torch.cuda.Event"]) -> None:
    """Arm this thread's next main-kernel launch (decode, decode merge, prefill
    or mixed kernel) to record ``start``/``stop`` (timing events) at its own
    dispatch start and end (msgl_profile_next_launch); ``stop`` then
    ``start.elapsed_time(stop)`` is that kernel's duration. None, None disarms."""
    handles = []
    for e in (start, stop):
        if e is None:
            handles.append(None)
            continue
        if not e.cuda_event:  # torch creates the event at its first record
            e.record()
        handles.append(e.cuda_event)
    _lib.check(_lib.load().msgl_profile_next_launch(*handles), "msgl_profile_next_launch")


def validate_metadata(
    kv_indptr: torch.Tensor,
    kv_indices: torch.Tensor,
    seq_lens: Optional[torch.Tensor],
    *,
    num_slots: int,
    page_size: int = 1,
    q_indptr: Optional[torch.Tensor] = None,
    num_tokens: int = 0,
) -> None:
    """Check a decode (``q_indptr`` None) or prefill call's index metadata on
    the device and raise ``ValueError`` naming the first violation found
    (``msgl_validate_metadata``); the counterpart of the reference's
    precondition asserts (attention/metal.py:122). Synchronises once to read the
    result, so it is opt-in."""
    dev = kv_indptr.device
    for name, t in (("kv_indptr", kv_indptr), ("kv_indices", kv_indices), ("seq_lens", seq_lens),
                    ("q_indptr", q_indptr)):
        _check_index(name, t, dev)
    if kv_indptr.dim() != 1 or kv_indptr.shape[0] < 1:
        raise ValueError("kv_indptr must be [R+1]")
    if page_size > 1 and seq_lens is None:
        raise ValueError("page_size > 1 needs seq_lens (as the attention calls do)")
    r = kv_indptr.shape[0] - 1
    if seq_lens is not None and seq_lens.shape[0] < r:
        raise ValueError("seq_lens must be [R]")
    if q_indptr is not None and q_indptr.shape[0] < r + 1:
        raise ValueError("q_indptr must be [R+1]")
    status = torch.empty(3, dtype=torch.int64, device=dev)
    st = _lib.load().msgl_validate_metadata(
        _lib.ptr(kv_indptr), _lib.ptr(kv_indices), _lib.ptr(seq_lens), _lib.ptr(q_indptr), r, int(page_size),
        kv_indices.numel(), int(num_slots), int(num_tokens), _lib.ptr(status), _lib.current_stream(dev),
    )
    _lib.check(st, "msgl_validate_metadata")
    code, where, value = status.tolist()
    if code != 0:
        what = _lib.META_ERRORS.get(code, f"error {code}")
        raise ValueError(f"invalid attention metadata: {what} (at {where}: {value})")


def check_step_sizes(cached_len, device_len, page_size: int, num_tokens: int, num_kv: int) -> None:
    """Host-side check of the output sizes given to ``build_step_indices``
    against the host copies of the step's lengths: the builder stops writing
    at its capacities, so a short capacity would leave the attention launches
    with fewer index entries than the offsets describe."""
    import numpy as np

    c = np.asarray(cached_len, dtype=np.int64)
    d = np.asarray(device_len, dtype=np.int64)
    if c.shape != d.shape:
        raise ValueError("cached_len and device_len must have one length")
    need_t = int(np.maximum(d - c, 0).sum())
    lens = np.maximum(d, 0)
    need_kv = int(lens.sum() if page_size == 1 else ((lens + page_size - 1) // page_size).sum())
    if num_tokens != need_t:
        raise ValueError(f"num_tokens is {num_tokens}, the step extends {need_t} tokens")
    if num_kv != need_kv:
        raise ValueError(f"num_kv is {num_kv}, the step's requests hold {need_kv} index entries")


def table_scatter(req_to_token: torch.Tensor, rows: torch.Tensor, cols: torch.Tensor, values: torch.Tensor) -> None:
    """req_to_token[rows, cols] = values on the device (entries outside the table skipped)."""
    n = rows.shape[0]
    if cols.shape != (n,) or values.shape != (n,) or req_to_token.dim() != 2:
        raise ValueError("rows, cols and values must be [n]; req_to_token [rows, max_seq_len]")
    dev = req_to_token.device
    for name, t in (("req_to_token", req_to_token), ("rows", rows), ("cols", cols), ("values", values)):
        _check_index(name, t, dev)
    if n == 0:
        return
    status = _lib.load().msgl_table_scatter(
        _lib.ptr(req_to_token), req_to_token.shape[0], req_to_token.shape[1], _lib.ptr(rows), _lib.ptr(cols),
        _lib.ptr(values), n, _lib.current_stream(dev),
    )
    _lib.check(status, "msgl_table_scatter")


def _check_rope(inv_freq: torch.Tensor, positions: torch.Tensor, rotary_dim: int, t: int, dev: torch.device) -> None:
    if inv_freq.dtype != torch.float32 or inv_freq.shape != (rotary_dim // 2,):
        raise ValueError(f"inv_freq must be float32 [rotary_dim / 2] = [{rotary_dim // 2}]")
    _check_device("inv_freq", inv_freq, dev)
    if positions.shape != (t,):
        raise ValueError("positions must be [T]")
    _check_index("positions", positions, dev)


def rope(
    x: torch.Tensor, positions: torch.Tensor, inv_freq: torch.Tensor, rotary_dim: int,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Rotate-half RoPE of x [T, H, D] at per-token positions (layers.py:45-56).

    ``out`` may be ``x`` (in place); inv_freq is [rotary_dim / 2] float32."""
    if x.dim() != 3:
        raise ValueError(f"x must be [T, H, D] (got {tuple(x.shape)})")
    dev = x.device
    _check_device("x", x, dev)
    _check_rope(inv_freq, positions, rotary_dim, x.shape[0], dev)
    if out is None:
        out = torch.empty_like(x)
    elif out.shape != x.shape or out.dtype != x.dtype:
        raise ValueError("out must match x")
    _check_device("out", out, dev)
    status = _lib.load().msgl_rope(
        _lib.ptr(x), _lib.ptr(out), _lib.ptr(positions), _lib.ptr(inv_freq), x.shape[0], x.shape[1], x.shape[2],
        rotary_dim, _lib.dtype_code(x.dtype), _lib.current_stream(dev),
    )
    _lib.check(status, "msgl_rope")
    return out


def rope_store_kv(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    positions: torch.Tensor,
    out_loc: torch.Tensor,
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    inv_freq: torch.Tensor,
    rotary_dim: int,
    q_out: Optional[torch.Tensor] = None,
    k_out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """layers.py:107-109 in one launch: rotate q and k, store rotated k and raw v
    at out_loc. Returns the rotated q (``q_out``, which may be ``q``); rotated k
    is also written to ``k_out`` when given (it may be ``k``)."""
    if q.dim() != 3 or k.dim() != 3 or k.shape != v.shape or q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2]:
        raise ValueError(f"q must be [T, Hq, D], k/v [T, Hkv, D] (got {tuple(q.shape)}, {tuple(k.shape)})")
    if k_pool.dim() != 3 or k_pool.shape != v_pool.shape or k_pool.shape[1:] != k.shape[1:]:
        raise ValueError(f"pools must be [N, Hkv, D] matching k (got {tuple(k_pool.shape)})")
    if out_loc.shape != (k.shape[0],):
        raise ValueError("out_loc must be [T]")
    if len({q.dtype, k.dtype, v.dtype, k_pool.dtype, v_pool.dtype}) != 1:
        raise ValueError("q, k, v and pools must share one dtype")
    dev = k_pool.device
    if q_out is None:
        q_out = torch.empty_like(q)
    for name, t in (("q", q), ("k", k), ("v", v), ("k_pool", k_pool), ("v_pool", v_pool), ("q_out", q_out)):
        _check_device(name, t, dev)
    if q_out.shape != q.shape or q_out.dtype != q.dtype:
        raise ValueError("q_out must match q")
    if k_out is not None:
        _check_device("k_out", k_out, dev)
        if k_out.shape != k.shape or k_out.dtype != k.dtype:
            raise ValueError("k_out must match k")
    _check_index("out_loc", out_loc, dev)
    _check_rope(inv_freq, positions, rotary_dim, q.shape[0], dev)
    status = _lib.load().msgl_rope_store_kv(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(positions), _lib.ptr(out_loc), _lib.ptr(inv_freq),
        _lib.ptr(q_out), _lib.ptr(k_out), _lib.ptr(k_pool), _lib.ptr(v_pool), q.shape[0], q.shape[1], k.shape[1],
        q.shape[2], rotary_dim, k_pool.shape[0], _lib.dtype_code(q.dtype), _lib.current_stream(dev),
    )
    _lib.check(status, "msgl_rope_store_kv")
    return q_out
