"""C ABI checks that need no GPU: the library loads, exports every function
declared in include/*.h with the signature the binding declares, and rejects
bad arguments on the host before any device work."""

import ctypes
import re
from pathlib import Path

import pytest

from minisgl_hip import _lib

INCLUDE = Path(__file__).resolve().parent.parent / "include"


def declared_functions():
    names = set()
    for h in INCLUDE.glob("*.h"):
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(msgl_\w+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_every_declared_symbol_is_exported_and_bound():
    lib = _lib.load()
    names = declared_functions()
    assert names, "no declarations found"
    for name in sorted(names):
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_lib.SIGNATURES) == names


def test_build_compiles_every_source_to_its_own_object():
    """The build's source list is every csrc/*.hip, csrc/*.cpp and
    csrc/inst/*.hip, and no two sources share an object file (a shared name
    would leave one unit's kernels out of the link)."""
    from minisgl_hip import _build

    srcs = _build.sources()
    expected = (set(_build.CSRC.glob("*.hip")) | set(_build.CSRC.glob("*.cpp"))
                | set((_build.CSRC / "inst").glob("*.hip")))
    assert len(srcs) == len(expected) and set(srcs) == expected
    assert any(s.parent.name == "inst" for s in srcs)
    objs = [_build.object_path(s) for s in srcs]
    assert len(set(objs)) == len(objs)


def test_abi_version_and_sizes():
    lib = _lib.load()
    assert lib.msgl_abi_version() == 2
    up = lambda x: (x + 255) // 256 * 256  # noqa: E731
    # [meta | work list: B x splits x kv-head groups (8 heads / 4 per workgroup) int4 | key offsets (B + 1) i64 |
    #  partials]
    assert lib.msgl_paged_decode_workspace_size(128, 16, 8, 128, 1) == 256 + up(128 * 1 * 2 * 16) + up(129 * 8)
    ws = lib.msgl_paged_decode_workspace_size(128, 16, 8, 128, 16)
    units = 128 * 16 * 16
    assert ws == 256 + up(128 * 16 * 2 * 16) + up(129 * 8) + up(units * 8) + up(units * 128 * 4)
    assert lib.msgl_paged_decode_workspace_size(1, 16, 8, 128, 1000) == lib.msgl_paged_decode_workspace_size(
        1, 16, 8, 128, 64)
    # splits bound the key ranges one request may overlap: 2 + ceil(8192 / (B Hkv)) in [4, 64], and no more
    # than ranges of >= 64 keys can cut max_seq_len into (ceil(max_seq_len / 64) + 1); never below the
    # per-request chunk count (~4096 wavefronts, chunks of at most 2048 keys)
    assert lib.msgl_paged_decode_default_splits(128, 8, 32768) == 16
    assert lib.msgl_paged_decode_default_splits(128, 8, 2048) == 10
    assert lib.msgl_paged_decode_default_splits(128, 8, 0) == 10
    assert lib.msgl_paged_decode_default_splits(1, 8, 32768) == 64
    assert lib.msgl_paged_decode_default_splits(1, 8, 100) == 3
    assert lib.msgl_paged_decode_default_splits(1, 8, 64) == 2
    assert lib.msgl_paged_decode_default_splits(256, 8, 8192) == 6
    assert lib.msgl_paged_decode_default_splits(4096, 8, 8192) == 4
    assert lib.msgl_paged_decode_default_splits(0, 8, 8192) == 1
    # one or two kv heads over short contexts: 16 chunks at most; long contexts keep the bound
    assert lib.msgl_paged_decode_default_splits(64, 2, 3072) == 16
    assert lib.msgl_paged_decode_default_splits(16, 1, 4096) == 16
    assert lib.msgl_paged_decode_default_splits(256, 2, 3072) == 16
    assert lib.msgl_paged_decode_default_splits(16, 1, 16384) == 64
    assert lib.msgl_paged_decode_default_splits(64, 2, 0) > 16


def test_prefill_sizes():
    lib = _lib.load()
    up = lambda x: (x + 255) // 256 * 256  # noqa: E731
    # (R, T, maxE, Hq, Hkv, D, splits): 128 query rows per work item, so 64 tokens at Hq/Hkv = 2
    items = 16 * 8 * 8  # requests x query blocks (ceil(512 / 64)) x kv heads
    # work item = two int4 (item, request geometry); with splits > 1 a chunk count per token, then partials
    assert lib.msgl_prefill_workspace_size(16, 2048, 512, 16, 8, 128, 1) == 256 + up(items * 32)
    rows = 4 * 2048 * 16
    assert lib.msgl_prefill_workspace_size(16, 2048, 512, 16, 8, 128, 4) == (
        256 + up(4 * items * 32) + up(2048 * 4) + up(rows * 8) + up(rows * 128 * 4))
    assert lib.msgl_prefill_workspace_size(16, 2048, 512, 16, 6, 128, 4) == 0  # Hq not a multiple of Hkv
    # 16 requests x 8 kv heads x ceil(512 / 64) blocks = 1024 workgroups: two chunks reach 1536
    assert lib.msgl_prefill_default_splits(16, 16, 8, 128, 512, 4096) == 2
    assert lib.msgl_prefill_default_splits(16, 16, 8, 128, 199, 4160) == 3
    assert lib.msgl_prefill_default_splits(1, 32, 8, 128, 64, 100000) == 16  # capped at 16
    assert lib.msgl_prefill_default_splits(1, 32, 8, 128, 64, 300) == 2  # >= 256 keys per chunk
    assert lib.msgl_prefill_default_splits(0, 32, 8, 128, 64, 300) == 1


def test_host_side_argument_errors():
    lib = _lib.load()
    nul = None
    # Hq not a multiple of Hkv
    st = lib.msgl_paged_decode(1, 1, 1, 1, 1, nul, 1, 6, 4, 128, 1, 100, _lib.MSGL_BF16, 0.1, 1, 1, nul, 0, nul)
    assert st == _lib.MSGL_ERR_INVALID and "multiple" in _lib.last_error()
    # unknown dtype
    st = lib.msgl_paged_decode(16, 16, 16, 16, 16, nul, 1, 16, 8, 128, 1, 100, 9, 0.1, 1, 16, nul, 0, nul)
    assert st == _lib.MSGL_ERR_UNSUPPORTED
    # page_size > 1 without seq_lens
    st = lib.msgl_paged_decode(16, 16, 16, 16, 16, nul, 1, 16, 8, 128, 16, 100, 1, 0.1, 1, 16, nul, 0, nul)
    assert st == _lib.MSGL_ERR_INVALID and "seq_lens" in _lib.last_error()
    # workspace too small for split-K
    st = lib.msgl_paged_decode(16, 16, 16, 16, 16, nul, 4, 16, 8, 128, 1, 100, 1, 0.1, 8, 16, nul, 0, nul)
    assert st == _lib.MSGL_ERR_WORKSPACE
    # every decode needs the work-list workspace
    st = lib.msgl_paged_decode(16, 16, 16, 16, 16, nul, 4, 16, 8, 128, 1, 100, 1, 0.1, 1, 16, nul, 0, nul)
    assert st == _lib.MSGL_ERR_WORKSPACE
    # unsupported head_dim is reported (dispatch happens before any launch; the workspace is never touched)
    st = lib.msgl_paged_decode(16, 16, 16, 16, 16, nul, 1, 16, 8, 96, 1, 100, 1, 0.1, 1, 16, 256, 1 << 30, nul)
    assert st == _lib.MSGL_ERR_UNSUPPORTED and "head_dim" in _lib.last_error()
    # prefill: (q, kp, vp, q_indptr, kv_indptr, kv_indices, seq_lens, R, T, maxE, maxL, Hq, Hkv, D, page, slots,
    #           dtype, scale, splits, out, ws, ws_bytes, stream)
    pf = lambda splits, ws_bytes, dtype=1, d=128, scale=0.1: lib.msgl_prefill_ragged(  # noqa: E731
        16, 16, 16, 16, 16, 16, nul, 2, 64, 32, 0, 16, 8, d, 1, 100, dtype, scale, splits, 16, 256, ws_bytes, nul)
    assert pf(1, 0, scale=0.0) == _lib.MSGL_ERR_INVALID and "scale" in _lib.last_error()
    assert pf(1, 0, scale=-0.1) == _lib.MSGL_ERR_INVALID
    assert pf(0, 0) == _lib.MSGL_ERR_INVALID and "max_splits" in _lib.last_error()
    assert pf(17, 0) == _lib.MSGL_ERR_INVALID
    assert pf(4, 0) == _lib.MSGL_ERR_WORKSPACE
    assert pf(1, 0) == _lib.MSGL_ERR_WORKSPACE  # bf16 always needs the work-list workspace
    assert pf(4, 1 << 30, d=96) == _lib.MSGL_ERR_UNSUPPORTED and "head_dim" in _lib.last_error()
    assert pf(4, 0, dtype=0, d=96) == _lib.MSGL_ERR_UNSUPPORTED  # fp32 needs no workspace: reaches dispatch
    assert lib.msgl_prefill_ragged(nul, nul, nul, nul, nul, nul, nul, 0, 0, 0, 0, 16, 8, 128, 1, 100, 1, 0.1, 1,
                                   nul, nul, 0, nul) == _lib.MSGL_OK
    # prefill plan: (q_indptr, kv_indptr, seq_lens, R, T, maxE, maxL, Hq, Hkv, D, dtype, splits, ws, ws_bytes, stream)
    pp = lambda splits=2, ws_bytes=1 << 20, dtype=1: lib.msgl_prefill_plan(  # noqa: E731
        16, 16, nul, 2, 64, 32, 0, 16, 8, 128, dtype, splits, 256, ws_bytes, nul)
    assert pp(splits=0) == _lib.MSGL_ERR_INVALID and "max_splits" in _lib.last_error()
    assert pp(ws_bytes=0) == _lib.MSGL_ERR_WORKSPACE
    assert pp(dtype=0, ws_bytes=0) == _lib.MSGL_OK  # fp32 has no work list
    assert lib.msgl_prefill_plan(nul, nul, nul, 0, 0, 0, 0, 16, 8, 128, 1, 1, nul, 0, nul) == _lib.MSGL_OK
    # step indices: (table, rows, stride, table_idx, cached, device_len, R, page, q_indptr, positions, out_loc,
    #                last, token_cap, kv_indptr, kv_indices, kv_cap, stream)
    bi = lambda R, page=1, rows_=4, stride=64, tok_out=16, kv_out=16: lib.msgl_build_step_indices(  # noqa: E731
        16, rows_, stride, 16, 16, 16, R, page, 16, tok_out, nul, nul, 8, 16, kv_out, 8, nul)
    assert bi(0) == _lib.MSGL_OK
    assert bi(-1) == _lib.MSGL_ERR_INVALID
    assert bi(2, page=0) == _lib.MSGL_ERR_INVALID and "page_size" in _lib.last_error()
    assert bi(2, rows_=0) == _lib.MSGL_ERR_INVALID
    assert bi(2, tok_out=nul) == _lib.MSGL_ERR_INVALID and "null" in _lib.last_error()
    assert bi(2, kv_out=nul) == _lib.MSGL_ERR_INVALID
    assert lib.msgl_table_scatter(nul, 4, 64, nul, nul, nul, 0, nul) == _lib.MSGL_OK
    assert lib.msgl_table_scatter(16, 4, 64, nul, 16, 16, 3, nul) == _lib.MSGL_ERR_INVALID
    # rope: (x, out, positions, inv_freq, T, H, D, rotary_dim, dtype, stream)
    rp = lambda t=4, h=2, d=128, rot=128, dtype=1, x=16, pos=16: lib.msgl_rope(  # noqa: E731
        x, x, pos, 16, t, h, d, rot, dtype, nul)
    assert rp(t=0) == _lib.MSGL_OK
    assert rp(rot=12) == _lib.MSGL_ERR_INVALID and "rotary_dim" in _lib.last_error()
    assert rp(rot=136, d=128) == _lib.MSGL_ERR_INVALID
    assert rp(d=130, rot=64) == _lib.MSGL_ERR_INVALID and "head_dim" in _lib.last_error()
    assert rp(dtype=5) == _lib.MSGL_ERR_UNSUPPORTED
    assert rp(pos=nul) == _lib.MSGL_ERR_INVALID and "positions" in _lib.last_error()
    assert rp(x=8, dtype=0) == _lib.MSGL_ERR_INVALID and "aligned" in _lib.last_error()
    # rope_store_kv: (q, k, v, positions, out_loc, inv_freq, q_out, k_out, k_pool, v_pool, T, Hq, Hkv, D, rot,
    #                 slots, dtype, stream)
    rs = lambda loc=16, kp=16, slots=100, hkv=8: lib.msgl_rope_store_kv(  # noqa: E731
        16, 16, 16, 16, loc, 16, 16, nul, kp, 16, 4, 16, hkv, 128, 128, slots, 1, nul)
    assert rs(loc=nul) == _lib.MSGL_ERR_INVALID and "out_loc" in _lib.last_error()
    assert rs(kp=nul) == _lib.MSGL_ERR_INVALID and "pools" in _lib.last_error()
    assert rs(slots=0) == _lib.MSGL_ERR_INVALID
    assert rs(hkv=0) == _lib.MSGL_ERR_INVALID
    # fp8 store: (k, v, out_loc, k_pool, v_pool, kv_scale, T, Hkv, D, slots, dtype, stream)
    sf = lambda t=4, d=128, dtype=1, sc=16, slots=100: lib.msgl_store_kv_fp8(  # noqa: E731
        16, 16, 16, 16, 16, sc, t, 8, d, slots, dtype, nul)
    assert sf(t=0) == _lib.MSGL_OK
    assert sf(d=96) == _lib.MSGL_ERR_UNSUPPORTED and "head_dim" in _lib.last_error()
    assert sf(d=2048) == _lib.MSGL_ERR_UNSUPPORTED  # a row wider than one wavefront
    assert sf(dtype=7) == _lib.MSGL_ERR_UNSUPPORTED
    assert sf(sc=nul) == _lib.MSGL_ERR_INVALID
    assert sf(sc=12) == _lib.MSGL_ERR_INVALID and "aligned" in _lib.last_error()
    assert sf(slots=0) == _lib.MSGL_ERR_INVALID
    # fp8 decode: (q, kp, vp, kv_scale, indptr, indices, seq_lens, B, Hq, Hkv, D, page, slots, dtype, scale,
    #              splits, out, ws, ws_bytes, stream)
    df = lambda dtype=1, hq=16, sc=16, d=128: lib.msgl_paged_decode_fp8(  # noqa: E731
        16, 16, 16, sc, 16, 16, nul, 4, hq, 8, d, 1, 100, dtype, 0.1, 1, 16, 256, 1 << 30, nul)
    assert df(sc=nul) == _lib.MSGL_ERR_INVALID and "kv_scale" in _lib.last_error()
    assert df(dtype=0) == _lib.MSGL_ERR_UNSUPPORTED and "fp8" in _lib.last_error()  # fp32 q over fp8 pools
    assert df(hq=96) == _lib.MSGL_ERR_UNSUPPORTED and "fp8" in _lib.last_error()  # group 12: not built
    assert df(d=96) == _lib.MSGL_ERR_UNSUPPORTED and "head_dim" in _lib.last_error()
    assert df(sc=12) == _lib.MSGL_ERR_INVALID and "aligned" in _lib.last_error()
    # fp8 decode with the fused store: (q, k_new, v_new, out_loc, kp, vp, kv_scale, indptr, ...)
    dsf = lambda kn=16, loc=16, sc=16, dtype=1: lib.msgl_paged_decode_store_fp8(  # noqa: E731
        16, kn, 16, loc, 16, 16, sc, 16, 16, nul, 4, 16, 8, 128, 1, 100, dtype, 0.1, 1, 16, 256, 1 << 30, nul)
    assert dsf(sc=nul) == _lib.MSGL_ERR_INVALID and "kv_scale" in _lib.last_error()
    assert dsf(kn=nul) == _lib.MSGL_ERR_INVALID and "k_new" in _lib.last_error()
    assert dsf(loc=nul) == _lib.MSGL_ERR_INVALID and "out_loc" in _lib.last_error()
    assert dsf(kn=24) == _lib.MSGL_ERR_INVALID and "aligned" in _lib.last_error()
    assert dsf(dtype=0) == _lib.MSGL_ERR_UNSUPPORTED and "fp8" in _lib.last_error()
    # mixed step: (decode part ..., prefill part ..., pools, Hq, Hkv, D, page, slots, dtype, scale, stream)
    mx = lambda nd=4, npf=2, kn=16, loc=16, dtype=1: lib.msgl_mixed_attention(  # noqa: E731
        16, kn, kn, loc, 16, 16, nul, nd, 1, 16, 256, 1 << 30,
        16, 16, 16, 16, nul, npf, 64, 32, 0, 1, 16, 256, 1 << 30,
        16, 16, 16, 8, 128, 1, 100, dtype, 0.1, nul)
    assert mx(nd=-1) == _lib.MSGL_ERR_INVALID
    # an unknown dtype is rejected before any launch (fp32 now runs the phases apart, which would launch)
    assert mx(dtype=9) == _lib.MSGL_ERR_UNSUPPORTED and "dtype" in _lib.last_error()
    assert mx(loc=nul) == _lib.MSGL_ERR_INVALID and "out_loc" in _lib.last_error()
    assert mx(kn=24) == _lib.MSGL_ERR_INVALID and "aligned" in _lib.last_error()
    # fp8 prefill: (q, kp, vp, kv_scale, q_indptr, kv_indptr, kv_indices, seq_lens, R, T, maxE, maxL, Hq, Hkv, D,
    #               page, slots, dtype, scale, splits, out, ws, ws_bytes, stream)
    pf8 = lambda dtype=1, sc=16, d=128: lib.msgl_prefill_ragged_fp8(  # noqa: E731
        16, 16, 16, sc, 16, 16, 16, nul, 2, 64, 32, 0, 16, 8, d, 1, 100, dtype, 0.1, 1, 16, 256, 1 << 30, nul)
    assert pf8(sc=nul) == _lib.MSGL_ERR_INVALID and "kv_scale" in _lib.last_error()
    assert pf8(dtype=0) == _lib.MSGL_ERR_UNSUPPORTED and "fp8" in _lib.last_error()
    assert pf8(d=96) == _lib.MSGL_ERR_UNSUPPORTED and "head_dim" in _lib.last_error()
    # metadata validation: (kv_indptr, kv_indices, seq_lens, q_indptr, R, page, num_indices, slots, T, status,
    #                       stream)
    va = lambda st=16, r=2, page=1, nidx=8, slots=100, ip=16: lib.msgl_validate_metadata(  # noqa: E731
        ip, 16, nul, nul, r, page, nidx, slots, 0, st, nul)
    assert va(st=nul) == _lib.MSGL_ERR_INVALID and "status" in _lib.last_error()
    assert va(st=12) == _lib.MSGL_ERR_INVALID  # int64 words
    assert va(page=0) == _lib.MSGL_ERR_INVALID
    assert va(slots=0) == _lib.MSGL_ERR_INVALID
    assert va(ip=nul) == _lib.MSGL_ERR_INVALID and "null" in _lib.last_error()
    assert va(page=16) == _lib.MSGL_ERR_INVALID and "seq_lens" in _lib.last_error()  # page ids need lengths
    # store_kv: zero tokens is a no-op; bad row size is unsupported
    assert lib.msgl_store_kv(nul, nul, nul, nul, nul, 0, 8, 128, 10, 1, nul) == _lib.MSGL_OK
    assert lib.msgl_store_kv(16, 16, 16, 16, 16, 4, 1, 3, 10, 1, nul) == _lib.MSGL_ERR_UNSUPPORTED
    assert lib.msgl_store_kv(16, 16, 16, 16, 16, 4, 8, 128, 10, 7, nul) == _lib.MSGL_ERR_UNSUPPORTED
    assert lib.msgl_store_kv(16, 16, 16, 16, 16, -1, 8, 128, 10, 1, nul) == _lib.MSGL_ERR_INVALID


def test_python_wrapper_raises():
    import torch

    from minisgl_hip import ops

    q = torch.zeros(2, 6, 64)
    pool = torch.zeros(8, 4, 64)
    with pytest.raises(ValueError):
        ops.paged_decode_attention(q, pool, pool, torch.zeros(3, dtype=torch.int32), torch.zeros(2, dtype=torch.int32), 0.1)
    with pytest.raises(ValueError):
        ops.store_kv(torch.zeros(2, 4, 64), torch.zeros(2, 4, 64), torch.zeros(3, dtype=torch.int32), pool, pool)
    with pytest.raises(ValueError):
        _lib.dtype_code(torch.int8)
    fp8 = torch.zeros(8, 4, 64, dtype=torch.float8_e4m3fn)
    sc = torch.zeros(8, 4, 2)
    k = torch.zeros(2, 4, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError):  # pools must be fp8
        ops.store_kv_fp8(k, k, torch.zeros(2, dtype=torch.int32), pool, pool, sc)
    with pytest.raises(ValueError):  # kv_scale must be [N, Hkv, 2]
        ops.store_kv_fp8(k, k, torch.zeros(2, dtype=torch.int32), fp8, fp8, torch.zeros(8, 4))
    with pytest.raises(ValueError):  # fp8 pools need kv_scale
        ops.paged_decode_attention(torch.zeros(2, 8, 64, dtype=torch.bfloat16), fp8, fp8,
                                   torch.zeros(3, dtype=torch.int32), torch.zeros(2, dtype=torch.int32), 0.1)
    with pytest.raises(ValueError):  # and 16-bit queries
        ops.paged_decode_attention(torch.zeros(2, 8, 64), fp8, fp8, torch.zeros(3, dtype=torch.int32),
                                   torch.zeros(2, dtype=torch.int32), 0.1, kv_scale=sc)
    with pytest.raises(ValueError):  # rotary_dim / inv_freq mismatch
        ops.rope(k, torch.zeros(2, dtype=torch.int32), torch.zeros(16), 64)
    with pytest.raises(ValueError):  # kv_indptr must hold B + 1 offsets, also with seq_lens
        ops.paged_decode_attention(torch.zeros(2, 8, 64), pool, pool, torch.zeros(2, dtype=torch.int32),
                                   torch.zeros(2, dtype=torch.int32), 0.1, seq_lens=torch.ones(2, dtype=torch.int32))
    with pytest.raises(ValueError):  # the KV cache takes the model dtype or fp8 only
        from minisgl_hip.kvcache import MHAKVCache
        MHAKVCache(1, 8, 4, 64, torch.bfloat16, "cpu", kv_dtype=torch.float16)
