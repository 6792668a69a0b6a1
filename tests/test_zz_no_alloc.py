"""msgl_paged_decode_store_noalloc (no workspace argument: the library's own
device array) against msgl_paged_decode_store with a caller workspace, through
the C ABI: the same output and pool bits on two calls in a row, the second on a
smaller batch (the array keeps the first call's contents); sizes whose
workspace exceeds the array are rejected before any launch."""

import numpy as np
import pytest
import torch

from gpu_util import i32, randn
from minisgl_hip import _lib, ops, workloads

pytestmark = pytest.mark.gpu

HQ, HKV, D = 16, 8, 128


def _inputs(batch, lo, hi, num_slots, seed, device):
    c = workloads.decode_case(batch, lo, hi, num_slots, 1, seed=seed)
    dt = torch.bfloat16
    kp = randn((num_slots, HKV, D), seed + 1, dt).to(device)
    vp = randn((num_slots, HKV, D), seed + 2, dt).to(device)
    q = randn((batch, HQ, D), seed + 3, dt).to(device)
    kn = randn((batch, HKV, D), seed + 4, dt).to(device)
    vn = randn((batch, HKV, D), seed + 5, dt).to(device)
    return c, kp, vp, q, kn, vn


def _noalloc(lib, q, kn, vn, loc, kp, vp, ip, ix, batch, out, stream):
    return lib.msgl_paged_decode_store_noalloc(
        _lib.ptr(q), _lib.ptr(kn), _lib.ptr(vn), _lib.ptr(loc), _lib.ptr(kp), _lib.ptr(vp), _lib.ptr(ip),
        _lib.ptr(ix), None, batch, HQ, HKV, D, 1, kp.shape[0], _lib.MSGL_BF16, D**-0.5, 0, _lib.ptr(out), stream)


def _with_workspace(lib, q, kn, vn, loc, kp, vp, ip, ix, batch, out, stream, device):
    splits = int(lib.msgl_paged_decode_default_splits(batch, HKV, 0))
    ws = torch.empty(ops.decode_workspace_bytes(batch, HQ, HKV, D, splits), dtype=torch.uint8, device=device)
    st = lib.msgl_paged_decode_store(
        _lib.ptr(q), _lib.ptr(kn), _lib.ptr(vn), _lib.ptr(loc), _lib.ptr(kp), _lib.ptr(vp), _lib.ptr(ip),
        _lib.ptr(ix), None, batch, HQ, HKV, D, 1, kp.shape[0], _lib.MSGL_BF16, D**-0.5, splits, _lib.ptr(out),
        _lib.ptr(ws), ws.numel(), stream)
    return st, ws


def test_noalloc_decode_matches_workspace_decode(cuda_device):
    lib = _lib.load()
    stream = _lib.current_stream(cuda_device)
    # the headline batch, then a smaller one over the same device array
    for batch, lo, hi, n, seed in ((128, 200, 2048, 1 << 18, 0), (9, 1, 700, 1 << 14, 30)):
        c, kp, vp, q, kn, vn = _inputs(batch, lo, hi, n, seed, cuda_device)
        ip, ix, loc = i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device), i32(c.out_loc, cuda_device)
        kp2, vp2 = kp.clone(), vp.clone()
        out_a = torch.full_like(q, float("nan"))
        out_b = torch.full_like(q, float("nan"))
        print(f"case noalloc batch={batch}", flush=True)
        st = _noalloc(lib, q, kn, vn, loc, kp, vp, ip, ix, batch, out_a, stream)
        assert st == _lib.MSGL_OK, _lib.last_error()
        st, ws = _with_workspace(lib, q, kn, vn, loc, kp2, vp2, ip, ix, batch, out_b, stream, cuda_device)
        assert st == _lib.MSGL_OK, _lib.last_error()
        torch.cuda.synchronize()
        assert torch.equal(out_a, out_b), f"batch {batch}: outputs differ"
        assert torch.equal(kp.view(torch.int16), kp2.view(torch.int16)), f"batch {batch}: K pools differ"
        assert torch.equal(vp.view(torch.int16), vp2.view(torch.int16)), f"batch {batch}: V pools differ"
        sl = loc.long()
        assert torch.equal(kp[sl], kn) and torch.equal(vp[sl], vn)
        assert np.isfinite(out_a.float().cpu().numpy()).all()
        del kp, vp, kp2, vp2, ws
        torch.cuda.empty_cache()


def test_noalloc_rejects_sizes_past_its_array(cuda_device):
    lib = _lib.load()
    assert lib.msgl_paged_decode_workspace_size(4096, 64, 8, 256, 64) > _lib.NOALLOC_WORKSPACE_BYTES
    print("case noalloc oversize", flush=True)
    # rejected on the host before anything is launched (the pointers are never used)
    st = lib.msgl_paged_decode_store_noalloc(16, 16, 16, 16, 16, 16, 16, 16, None, 4096, 64, 8, 256, 1, 100,
                                             _lib.MSGL_BF16, 0.1, 64, 16, None)
    assert st == _lib.MSGL_ERR_WORKSPACE and "workspace" in _lib.last_error()


def test_noalloc_decode_captured_in_a_graph(cuda_device):
    """The callers this entry point is for: a decode step captured in a HIP
    graph (no allocation, no memset inside the library) and replayed three
    times, with an eager decode of another batch through the same device array
    between replays; every replay gives the eager call's bits."""
    lib = _lib.load()
    batch = 64
    c, kp, vp, q, kn, vn = _inputs(batch, 200, 2048, 1 << 17, 7, cuda_device)
    ip, ix, loc = i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device), i32(c.out_loc, cuda_device)
    out_e = torch.empty_like(q)
    print("case noalloc graph capture", flush=True)
    assert _noalloc(lib, q, kn, vn, loc, kp, vp, ip, ix, batch, out_e, _lib.current_stream(cuda_device)) == 0
    torch.cuda.synchronize()
    pools = (kp.clone(), vp.clone())
    out_g = torch.full_like(q, float("nan"))
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            st = _noalloc(lib, q, kn, vn, loc, kp, vp, ip, ix, batch, out_g, _lib.current_stream(cuda_device))
    assert st == _lib.MSGL_OK, _lib.last_error()
    torch.cuda.current_stream().wait_stream(side)
    for rep in range(3):
        out_g.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, out_e), f"replay {rep} differs from the eager call"
        assert torch.equal(kp, pools[0]) and torch.equal(vp, pools[1]), f"replay {rep}: pools changed"
        other = torch.empty_like(q[: batch // 2])
        st = _noalloc(lib, q, kn, vn, loc, kp, vp, ip, ix, batch // 2, other, _lib.current_stream(cuda_device))
        assert st == _lib.MSGL_OK
        torch.cuda.synchronize()
    del graph
    torch.cuda.empty_cache()
