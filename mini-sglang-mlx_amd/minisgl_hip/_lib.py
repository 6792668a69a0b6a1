"""ctypes binding of ``libmsgl_attn.so`` (the C ABI declared in include/msgl_attn.h).

torch is imported before the library is opened: both torch and the library
depend on ``libamdhip64.so.7``, and loading torch first makes the dynamic linker
bind the library to torch's already-loaded HIP runtime, so device pointers and
streams from torch are valid in the library. There is no CPU fallback: if the
library is missing, every entry point raises.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (must precede the CDLL below)

LIB_PATH = Path(__file__).resolve().with_name("libmsgl_attn.so")

MSGL_OK = 0
MSGL_ERR_INVALID = 1
MSGL_ERR_UNSUPPORTED = 2
MSGL_ERR_WORKSPACE = 3
MSGL_ERR_HIP = 4

MSGL_F32 = 0
MSGL_BF16 = 1
MSGL_F16 = 2

_TORCH_TO_MSGL = {torch.float32: MSGL_F32, torch.bfloat16: MSGL_BF16, torch.float16: MSGL_F16}

_c_i32 = ctypes.c_int32
_c_i64 = ctypes.c_int64
_c_p = ctypes.c_void_p
_c_f = ctypes.c_float

# name -> (restype, argtypes); must match include/msgl_attn.h
SIGNATURES = {
    "msgl_abi_version": (ctypes.c_int, []),
    "msgl_last_error": (ctypes.c_char_p, []),
    "msgl_store_kv": (
        ctypes.c_int,
        [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i32, _c_i32, _c_i64, _c_i32, _c_p],
    ),
    "msgl_paged_decode_default_splits": (_c_i32, [_c_i32, _c_i32, _c_i32]),
    "msgl_paged_decode_workspace_size": (_c_i64, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32]),
    "msgl_paged_decode": (
        ctypes.c_int,
        [
            _c_p, _c_p, _c_p,  # q, k_pool, v_pool
            _c_p, _c_p, _c_p,  # kv_indptr, kv_indices, seq_lens
            _c_i32, _c_i32, _c_i32, _c_i32,  # batch, Hq, Hkv, D
            _c_i32, _c_i64, _c_i32, _c_f,  # page_size, num_slots, dtype, scale
            _c_i32, _c_p, _c_p, _c_i64, _c_p,  # max_splits, out, workspace, ws_bytes, stream
        ],
    ),
    "msgl_paged_decode_store": (
        ctypes.c_int,
        [
            _c_p, _c_p, _c_p, _c_p,  # q, k_new, v_new, out_loc
            _c_p, _c_p,  # k_pool, v_pool
            _c_p, _c_p, _c_p,  # kv_indptr, kv_indices, seq_lens
            _c_i32, _c_i32, _c_i32, _c_i32,  # batch, Hq, Hkv, D
            _c_i32, _c_i64, _c_i32, _c_f,  # page_size, num_slots, dtype, scale
            _c_i32, _c_p, _c_p, _c_i64, _c_p,  # max_splits, out, workspace, ws_bytes, stream
        ],
    ),
    "msgl_paged_decode_plan": (
        ctypes.c_int,
        [
            _c_p, _c_p, _c_i32,  # kv_indptr, seq_lens, batch
            _c_i32, _c_i32, _c_i32, _c_i32,  # Hq, Hkv, D, max_splits
            _c_p, _c_i64, _c_p,  # workspace, ws_bytes, stream
        ],
    ),
    "msgl_prefill_ragged": (
        ctypes.c_int,
        [
            _c_p, _c_p, _c_p,  # q, k_pool, v_pool
            _c_p, _c_p, _c_p, _c_p,  # q_indptr, kv_indptr, kv_indices, seq_lens
            _c_i32, _c_i32, _c_i32, _c_i32,  # num_reqs, num_tokens, max_extend_len, max_seq_len
            _c_i32, _c_i32, _c_i32,  # Hq, Hkv, D
            _c_i32, _c_i64, _c_i32, _c_f,  # page_size, num_slots, dtype, scale
            _c_i32, _c_p, _c_p, _c_i64, _c_p,  # max_splits, out, workspace, ws_bytes, stream
        ],
    ),
    "msgl_build_step_indices": (
        ctypes.c_int,
        [
            _c_p, _c_i64, _c_i64,  # req_to_token, num_rows, row_stride
            _c_p, _c_p, _c_p, _c_i32, _c_i32,  # table_idx, cached_len, device_len, num_reqs, page_size
            _c_p, _c_p, _c_p, _c_p, _c_i64,  # q_indptr, positions, out_loc, last_indices, token_capacity
            _c_p, _c_p, _c_i64, _c_p,  # kv_indptr, kv_indices, kv_capacity, stream
        ],
    ),
    "msgl_table_scatter": (ctypes.c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_p]),
    "msgl_rope": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_p]),
    "msgl_rope_store_kv": (
        ctypes.c_int,
        [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
         _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i64, _c_i32, _c_p],
    ),
    "msgl_prefill_default_splits": (_c_i32, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32]),
    "msgl_prefill_workspace_size": (_c_i64, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32]),
}

SIGNATURES["msgl_store_kv_fp8"] = (
    ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i32, _c_i32, _c_i64, _c_i32, _c_p]
)
SIGNATURES["msgl_paged_decode_fp8"] = (
    ctypes.c_int,
    [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i64, _c_i32,
     _c_f, _c_i32, _c_p, _c_p, _c_i64, _c_p],
)
SIGNATURES["msgl_paged_decode_fp8_planned"] = SIGNATURES["msgl_paged_decode_fp8"]
SIGNATURES["msgl_prefill_ragged_planned"] = SIGNATURES["msgl_prefill_ragged"]
SIGNATURES["msgl_prefill_ragged_fp8"] = (
    ctypes.c_int,
    [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
     _c_i64, _c_i32, _c_f, _c_i32, _c_p, _c_p, _c_i64, _c_p],
)
SIGNATURES["msgl_prefill_ragged_fp8_planned"] = SIGNATURES["msgl_prefill_ragged_fp8"]
SIGNATURES["msgl_prefill_plan"] = (
    ctypes.c_int,
    [_c_p, _c_p, _c_p, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_p, _c_i64, _c_p],
)
SIGNATURES["msgl_paged_decode_planned"] = SIGNATURES["msgl_paged_decode"]
SIGNATURES["msgl_paged_decode_store_planned"] = SIGNATURES["msgl_paged_decode_store"]
SIGNATURES["msgl_paged_decode_store_fp8"] = (
    ctypes.c_int,
    [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,  # q, k_new, v_new, out_loc, k_pool, v_pool, kv_scale
     _c_p, _c_p, _c_p, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i64, _c_i32,
     _c_f, _c_i32, _c_p, _c_p, _c_i64, _c_p],
)
SIGNATURES["msgl_paged_decode_store_fp8_planned"] = SIGNATURES["msgl_paged_decode_store_fp8"]
SIGNATURES["msgl_mixed_attention"] = (
    ctypes.c_int,
    [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i32, _c_i32, _c_p, _c_p, _c_i64,  # decode part
     _c_p, _c_p, _c_p, _c_p, _c_p, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_p, _c_p, _c_i64,  # prefill part
     _c_p, _c_p, _c_i32, _c_i32, _c_i32, _c_i32, _c_i64, _c_i32, _c_f, _c_p],
)

SIGNATURES["msgl_paged_decode_planned_ex"] = (
    ctypes.c_int,
    [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,  # q, k_new, v_new, out_loc, k_pool, v_pool, kv_scale
     _c_p, _c_p, _c_p, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i64, _c_i32,
     _c_f, _c_i32, ctypes.c_uint32, _c_p, _c_p, _c_i64, _c_p],
)
SIGNATURES["msgl_paged_decode_merge"] = (
    ctypes.c_int,
    [_c_p, _c_p, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_p, _c_p, _c_i64, _c_p],
)
MSGL_DECODE_NO_MERGE = 1

SIGNATURES["msgl_profile_next_launch"] = (ctypes.c_int, [_c_p, _c_p])
SIGNATURES["msgl_paged_decode_store_noalloc"] = (
    ctypes.c_int,
    [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p,  # q, k_new, v_new, out_loc, k_pool, v_pool
     _c_p, _c_p, _c_p, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i64, _c_i32,
     _c_f, _c_i32, _c_p, _c_p],  # scale, max_splits, out, stream
)
NOALLOC_WORKSPACE_BYTES = 32 << 20

SIGNATURES["msgl_validate_metadata"] = (
    ctypes.c_int,
    [_c_p, _c_p, _c_p, _c_p, _c_i32, _c_i32, _c_i64, _c_i64, _c_i32, _c_p, _c_p],
)

# msgl_meta_error codes of msgl_validate_metadata
META_ERRORS = {
    1: "kv_indptr is negative or decreasing",
    2: "kv_indptr[R] lies beyond the entries of kv_indices",
    3: "a sequence length is negative or needs more index entries than its kv_indptr row holds",
    4: "an index entry names a slot (page) outside the pool",
    5: "q_indptr does not run from 0 to num_tokens without decreasing",
    6: "an extend length exceeds its sequence length",
}

_lib = None


def load() -> ctypes.CDLL:
    """Open the library (once) and declare every entry point's signature."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built: run `python -m minisgl_hip._build` in mini-sglang-mlx_amd/"
            )
        lib = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
    return _lib


def last_error() -> str:
    msg = load().msgl_last_error()
    return msg.decode() if msg else ""


def check(status: int, what: str) -> None:
    if status == MSGL_OK:
        return
    msg = last_error()
    if status == MSGL_ERR_INVALID:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what} failed (status {status}): {msg}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _TORCH_TO_MSGL[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}; expected float32, bfloat16 or float16") from None


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


def current_stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
