"""Paged decode on the GPU vs the float64 oracle (attention/naive.py:50-60 semantics).

Shape grid and edge lengths follow tests/test_attention.py:19-39; the larger
cases are the benchmark's decode workloads (checked on sampled requests, plus
size-independent properties at full size).
"""

import types

import numpy as np
import pytest
import torch

import oracle
from gpu_util import DTYPES, assert_close, i32, randn, to_np64
from minisgl_hip import ops, workloads

pytestmark = pytest.mark.gpu


def _pools(n, hkv, d, dtype, seed, device):
    k = randn((n, hkv, d), seed, dtype).to(device)
    v = randn((n, hkv, d), seed + 1, dtype).to(device)
    return k, v


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (32, 8, 128), (8, 8, 64), (16, 2, 256)])
@pytest.mark.parametrize("splits", [1, None, 8])
def test_reference_grid(cuda_device, hq, hkv, d, dtype, splits):
    """tests/test_attention.py:19-39: N=4096, B=7, lens [1,2,17,31,32,33,700], rng(0) permuted slots."""
    dt = DTYPES[dtype]
    c = workloads.reference_test_case()
    kp, vp = _pools(4096, hkv, d, dt, 100, cuda_device)
    q = randn((7, hq, d), 102, dt).to(cuda_device)
    print(f"case grid hq={hq} hkv={hkv} d={d} {dtype} splits={splits}", flush=True)
    out = ops.paged_decode_attention(
        q, kp, vp, i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device), d**-0.5, max_splits=splits
    )
    torch.cuda.synchronize()
    ref = oracle.paged_decode(to_np64(q), to_np64(kp), to_np64(vp), c.kv_indptr, c.kv_indices, d**-0.5)
    assert_close(out, ref, dt, f"grid {hq}/{hkv}/{d} {dtype} splits={splits}")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("splits", [1, 4, 64])
def test_edge_lengths(cuda_device, dtype, splits):
    """Lengths around the 16-token tile, the 64-token index block and split boundaries."""
    dt = DTYPES[dtype]
    lens = [1, 15, 16, 17, 63, 64, 65, 127, 128, 129, 1000, 4097]
    c = workloads.decode_case_from_lens(lens, num_slots=8192, seed=7)
    kp, vp = _pools(8192, 8, 128, dt, 200, cuda_device)
    q = randn((len(lens), 16, 128), 202, dt).to(cuda_device)
    print(f"case edge {dtype} splits={splits}", flush=True)
    out = ops.paged_decode_attention(
        q, kp, vp, i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device), 128**-0.5, max_splits=splits
    )
    torch.cuda.synchronize()
    ref = oracle.paged_decode(to_np64(q), to_np64(kp), to_np64(vp), c.kv_indptr, c.kv_indices, 128**-0.5)
    assert_close(out, ref, dt, f"edge {dtype} splits={splits}")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_page_size_16_page_ids(cuda_device, dtype):
    """page ids + seq_lens (page_size 16) equal the token-slot CSR form."""
    dt = DTYPES[dtype]
    lens = [1, 15, 16, 17, 200, 1023, 3000]
    c = workloads.decode_case_from_lens(lens, num_slots=16384, page_size=16, seed=11)
    kp, vp = _pools(16384, 8, 128, dt, 300, cuda_device)
    q = randn((len(lens), 32, 128), 302, dt).to(cuda_device)
    print(f"case page16 {dtype}", flush=True)
    out = ops.paged_decode_attention(
        q, kp, vp, i32(c.page_indptr, cuda_device), i32(c.page_ids, cuda_device), 128**-0.5,
        seq_lens=i32(c.lens, cuda_device), page_size=16,
    )
    out_tok = ops.paged_decode_attention(
        q, kp, vp, i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device), 128**-0.5
    )
    torch.cuda.synchronize()
    ref = oracle.paged_decode(
        to_np64(q), to_np64(kp), to_np64(vp), c.page_indptr, c.page_ids, 128**-0.5, page_size=16, seq_lens=c.lens
    )
    assert_close(out, ref, dt, f"page16 {dtype}")
    assert torch.equal(out, out_tok), "page-id and token-slot forms differ"


def test_table_rows_with_seq_lens(cuda_device):
    """kv_indptr as row starts into a flattened token-granular page table (+ seq_lens)."""
    dt = torch.bfloat16
    c = workloads.decode_case_from_lens([5, 300, 77, 1], num_slots=4096, seed=12)
    stride = c.page_table.shape[1]
    assert c.page_table.shape[0] == 4
    # row starts, then the table's entry count (kv_indptr[B]: where index reads stop)
    starts = (np.arange(5) * stride).astype(np.int32)
    kp, vp = _pools(4096, 8, 128, dt, 400, cuda_device)
    q = randn((4, 16, 128), 402, dt).to(cuda_device)
    print("case table-rows", flush=True)
    out = ops.paged_decode_attention(
        q, kp, vp, i32(starts, cuda_device), i32(c.page_table.reshape(-1), cuda_device), 128**-0.5,
        seq_lens=i32(c.lens, cuda_device),
    )
    torch.cuda.synchronize()
    ref = oracle.paged_decode(to_np64(q), to_np64(kp), to_np64(vp), c.kv_indptr, c.kv_indices, 128**-0.5)
    assert_close(out, ref, dt, "table rows")


def test_zero_length_request_gives_zeros(cuda_device):
    dt = torch.bfloat16
    lens = np.array([3, 0, 70], dtype=np.int32)
    indptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    indices = np.arange(73, dtype=np.int32)
    kp, vp = _pools(128, 8, 128, dt, 500, cuda_device)
    q = randn((3, 16, 128), 502, dt).to(cuda_device)
    print("case zero-length", flush=True)
    for splits in (1, 8):
        out = ops.paged_decode_attention(q, kp, vp, i32(indptr, cuda_device), i32(indices, cuda_device), 0.1,
                                         max_splits=splits)
        torch.cuda.synchronize()
        assert torch.count_nonzero(out[1]) == 0
        ref = oracle.paged_decode(to_np64(q[[0, 2]]), to_np64(kp), to_np64(vp),
                                  np.array([0, 3, 73]), indices, 0.1)
        assert_close(out[[0, 2]], ref, dt, "zero-length neighbours")


def test_batch8_ctx1k_fp32_full(cuda_device):
    """B=8, L ~ U[100,1024], pool 16384, page 1, fp32: every request vs the oracle at 1e-5."""
    c = workloads.decode_case(8, 100, 1024, 16384, 1, seed=0)
    dt = torch.float32
    kp, vp = _pools(16384, 8, 128, dt, 600, cuda_device)
    q = randn((8, 16, 128), 602, dt).to(cuda_device)
    print("case batch8 ctx1k fp32", flush=True)
    out = ops.paged_decode_attention(q, kp, vp, i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device),
                                     128**-0.5)
    torch.cuda.synchronize()
    ref = oracle.paged_decode(to_np64(q), to_np64(kp), to_np64(vp), c.kv_indptr, c.kv_indices, 128**-0.5)
    assert_close(out, ref, dt, "batch8 ctx1k")


def _sampled_ref(q, kp, vp, c, pick, scale, page_size=1):
    """Oracle on a subset of requests (gathering only their slots)."""
    outs = []
    for b in pick:
        if page_size == 1:
            slots = c.kv_indices[c.kv_indptr[b] : c.kv_indptr[b + 1]].astype(np.int64)
        else:
            slots = oracle.expand_page_indices(c.page_ids[c.page_indptr[b] : c.page_indptr[b + 1]], page_size,
                                               int(c.lens[b]))
        st = torch.from_numpy(slots).to(kp.device)
        kb = to_np64(kp.index_select(0, st))
        vb = to_np64(vp.index_select(0, st))
        outs.append(oracle.sdpa(to_np64(q[b])[:, None, :], kb.transpose(1, 0, 2), vb.transpose(1, 0, 2), scale)[:, 0])
    return np.stack(outs)


def test_batch128_ctx2k_full_size(cuda_device):
    """Batch 128, L ~ U[200,2048], pool 262144, bf16: sampled requests vs oracle, plus
    bitwise invariance under relocation of the KV rows and run-to-run determinism."""
    c = workloads.decode_case(128, 200, 2048, 262144, 1, seed=0)
    dt = torch.bfloat16
    kp, vp = _pools(262144, 8, 128, dt, 700, cuda_device)
    q = randn((128, 16, 128), 702, dt).to(cuda_device)
    indptr, indices = i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device)
    print("case batch128 ctx2k", flush=True)
    out = ops.paged_decode_attention(q, kp, vp, indptr, indices, 128**-0.5)
    out2 = ops.paged_decode_attention(q, kp, vp, indptr, indices, 128**-0.5)
    torch.cuda.synchronize()
    assert torch.equal(out, out2), "decode is not deterministic"
    pick = [0, 1, 17, 63, 64, 100, 126, 127]
    ref = _sampled_ref(q, kp, vp, c, pick, 128**-0.5)
    assert_close(out[pick], ref, dt, "batch128 ctx2k sampled")
    # relocate every used row to a new slot (a fixed permutation of the pool): same bits out
    perm = torch.from_numpy(np.random.default_rng(5).permutation(262144).astype(np.int64)).to(cuda_device)
    kp2 = torch.empty_like(kp)
    vp2 = torch.empty_like(vp)
    kp2[perm] = kp
    vp2[perm] = vp
    out3 = ops.paged_decode_attention(q, kp2, vp2, indptr, perm[indices.long()].int(), 128**-0.5)
    torch.cuda.synchronize()
    assert torch.equal(out, out3), "result depends on where the rows live"


def test_8b_heads_long_contexts_page16(cuda_device):
    """Qwen3-8B heads (32/8/128), page 16, contexts 1024..8192 (reduced batch), split-K + merge."""
    c = workloads.decode_case(24, 1024, 8192, 1 << 20, 16, seed=0)
    dt = torch.bfloat16
    kp, vp = _pools(1 << 20, 8, 128, dt, 800, cuda_device)
    q = randn((24, 32, 128), 802, dt).to(cuda_device)
    print("case 8b heads ctx8k page16", flush=True)
    out = ops.paged_decode_attention(
        q, kp, vp, i32(c.page_indptr, cuda_device), i32(c.page_ids, cuda_device), 128**-0.5,
        seq_lens=i32(c.lens, cuda_device), page_size=16,
    )
    torch.cuda.synchronize()
    pick = list(range(0, 24, 3))
    ref = _sampled_ref(q, kp, vp, c, pick, 128**-0.5, page_size=16)
    assert_close(out[pick], ref, dt, "8b heads ctx8k sampled")


def test_key_ranges_long_contexts_page16(cuda_device):
    """~1.2M keys (Qwen3-8B heads, page 16, contexts 4096..8192): enough keys for the
    launch to split by equal key ranges of the batch's token stream (>= 2048 keys per
    range even at 4 resident workgroups per CU). Sampled requests vs the oracle; the
    fused store and a reused plan give the same bits as the separate calls."""
    batch = 200
    c = workloads.decode_case(batch, 4096, 8192, 1 << 21, 16, seed=3)
    cus = torch.cuda.get_device_properties(cuda_device).multi_processor_count
    assert int(c.lens.sum()) >= 2048 * 4 * cus // 2, "too few keys to select key ranges"
    dt = torch.bfloat16
    kp, vp = _pools(1 << 21, 8, 128, dt, 820, cuda_device)
    q = randn((batch, 32, 128), 822, dt).to(cuda_device)
    kn = randn((batch, 8, 128), 823, dt).to(cuda_device)
    vn = randn((batch, 8, 128), 824, dt).to(cuda_device)
    indptr, pages, lens = i32(c.page_indptr, cuda_device), i32(c.page_ids, cuda_device), i32(c.lens, cuda_device)
    loc = i32(c.out_loc, cuda_device)
    kp2, vp2 = kp.clone(), vp.clone()
    print("case key-ranges 8B page16", flush=True)
    kw = dict(seq_lens=lens, page_size=16)
    out = ops.paged_decode_attention(q, kp, vp, indptr, pages, 128**-0.5, new_kv=(kn, vn, loc), **kw)
    ops.store_kv(kn, vn, loc, kp2, vp2)
    ref_out = ops.paged_decode_attention(q, kp2, vp2, indptr, pages, 128**-0.5, **kw)
    splits = ops.default_splits(batch, 8, int(c.lens.max()))
    ws = ops.decode_workspace(batch, 32, 8, 128, splits, cuda_device)
    ops.paged_decode_plan(indptr, lens, batch, 32, 8, 128, splits, ws)
    planned = ops.paged_decode_attention(q, kp2, vp2, indptr, pages, 128**-0.5, max_splits=splits, workspace=ws,
                                         planned=True, **kw)
    torch.cuda.synchronize()
    assert torch.equal(kp.view(torch.int16), kp2.view(torch.int16))
    assert torch.equal(out, ref_out), "fused store != store + decode"
    assert torch.equal(planned, ref_out), "planned != unplanned"
    pick = [0, 1, 57, 99, 100, 150, 198, 199]
    ref = _sampled_ref(q, kp2, vp2, c, pick, 128**-0.5, page_size=16)
    assert_close(out[pick], ref, dt, "key ranges sampled")


@pytest.mark.parametrize("dtype,hq", [("bf16", 16), ("f16", 32), ("bf16", 64)])
def test_key_ranges_ragged_extremes(cuda_device, dtype, hq):
    """Key ranges over a batch with empty requests, one- and few-key requests between
    them and two requests of 400k / 350k keys (the range length is then set by the
    longest request, ceil(400000 / (S - 1))): zero rows for L = 0, the long requests
    agree with the unsplit decode (one workgroup per request), the short ones with
    the oracle."""
    rng = np.random.default_rng(11)
    lens = rng.integers(0, 4000, size=64).astype(np.int32)
    lens[[0, 5, 6, 40, 63]] = 0
    lens[[1, 7, 41]] = [1, 2, 17]
    lens[3], lens[50] = 400000, 350000
    n = int(lens.sum())
    cus = torch.cuda.get_device_properties(cuda_device).multi_processor_count
    assert n >= 2048 * 3 * cus // 2, "too few keys to select key ranges"
    indptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    indices = rng.permutation(1 << 21)[:n].astype(np.int32)
    dt = DTYPES[dtype]
    kp, vp = _pools(1 << 21, 8, 128, dt, 830, cuda_device)
    q = randn((64, hq, 128), 832, dt).to(cuda_device)
    ip, ix = i32(indptr, cuda_device), i32(indices, cuda_device)
    print(f"case key-ranges ragged extremes {dtype} hq={hq}", flush=True)
    out = ops.paged_decode_attention(q, kp, vp, ip, ix, 128**-0.5, max_seq_len=int(lens.max()))
    one = ops.paged_decode_attention(q, kp, vp, ip, ix, 128**-0.5, max_splits=1)
    torch.cuda.synchronize()
    zero = [i for i in range(64) if lens[i] == 0]
    assert torch.count_nonzero(out[zero]) == 0
    assert_close(out[[3, 50]], to_np64(one[[3, 50]]), dt, "long requests vs unsplit")
    short = [1, 2, 7, 41, 42, 62]
    case = types.SimpleNamespace(kv_indptr=indptr, kv_indices=indices)
    ref = _sampled_ref(q, kp, vp, case, short, 128**-0.5)
    assert_close(out[short], ref, dt, "short requests vs oracle")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("splits", [1, 4])
def test_fused_store_matches_two_calls(cuda_device, dtype, splits):
    """msgl_paged_decode_store == msgl_store_kv + msgl_paged_decode, bit for bit,
    even when the new tokens' slots hold NaN before the store."""
    dt = DTYPES[dtype]
    lens = [1, 2, 17, 64, 65, 300, 1000]
    c = workloads.decode_case_from_lens(lens, num_slots=4096, seed=21)
    kp, vp = _pools(4096, 8, 128, dt, 900, cuda_device)
    loc = i32(c.out_loc, cuda_device)
    kp[loc.long()] = float("nan")
    vp[loc.long()] = float("nan")
    q = randn((len(lens), 16, 128), 902, dt).to(cuda_device)
    kn = randn((len(lens), 8, 128), 903, dt).to(cuda_device)
    vn = randn((len(lens), 8, 128), 904, dt).to(cuda_device)
    indptr, indices = i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device)
    kp2, vp2 = kp.clone(), vp.clone()
    print(f"case fused-store {dtype} splits={splits}", flush=True)
    out = ops.paged_decode_attention(q, kp, vp, indptr, indices, 128**-0.5, max_splits=splits,
                                     new_kv=(kn, vn, loc))
    ops.store_kv(kn, vn, loc, kp2, vp2)
    ref_out = ops.paged_decode_attention(q, kp2, vp2, indptr, indices, 128**-0.5, max_splits=splits)
    torch.cuda.synchronize()
    assert torch.equal(kp.view(torch.int16 if dt != torch.float32 else torch.int32),
                       kp2.view(torch.int16 if dt != torch.float32 else torch.int32))
    assert torch.equal(vp.view(torch.int16 if dt != torch.float32 else torch.int32),
                       vp2.view(torch.int16 if dt != torch.float32 else torch.int32))
    assert torch.equal(out, ref_out)
    ref = oracle.paged_decode(to_np64(q), to_np64(kp2), to_np64(vp2), c.kv_indptr, c.kv_indices, 128**-0.5)
    assert_close(out, ref, dt, f"fused store {dtype}")


@pytest.mark.parametrize("splits", [1, 4, 16])
def test_planned_matches_unplanned(cuda_device, splits):
    """A plan built once and reused (msgl_paged_decode_plan + *_planned) gives the
    same bits as the self-planning calls, across layers with different pools."""
    c = workloads.decode_case(40, 1, 3000, 1 << 17, 1, seed=9)
    dt = torch.bfloat16
    q = randn((40, 16, 128), 901, dt).to(cuda_device)
    indptr, indices = i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device)
    ws = ops.decode_workspace(40, 16, 8, 128, splits, cuda_device)
    print(f"case planned decode splits={splits}", flush=True)
    ops.paged_decode_plan(indptr, None, 40, 16, 8, 128, splits, ws)
    for layer in range(3):
        kp, vp = _pools(1 << 17, 8, 128, dt, 910 + 2 * layer, cuda_device)
        a = ops.paged_decode_attention(q, kp, vp, indptr, indices, 128**-0.5, max_splits=splits, workspace=ws,
                                       planned=True)
        b = ops.paged_decode_attention(q, kp, vp, indptr, indices, 128**-0.5, max_splits=splits)
        torch.cuda.synchronize()
        assert torch.equal(a, b), f"planned != unplanned at layer {layer}"
    ref = _sampled_ref(q, kp, vp, c, [0, 13, 39], 128**-0.5)
    assert_close(b[[0, 13, 39]], ref, dt, "planned decode")


@pytest.mark.parametrize("splits", [None, 1])
def test_batch_past_plan_staging(cuda_device, splits):
    """20,000 requests of 0..64 keys: more than the plan kernel stages in LDS
    (8192 lengths), so it reads the rest from memory. Sampled requests against
    the oracle (an empty request gives zeros), and the reused plan gives the
    same bits as the self-planning call."""
    rng = np.random.default_rng(21)
    lens = rng.integers(0, 65, size=20000)
    lens[[5, 9000, 19999]] = 0
    n = 1 << 21
    c = workloads.decode_case_from_lens(list(lens), num_slots=n, seed=22)
    b, hq, hkv, d = len(lens), 16, 8, 128
    dt = torch.bfloat16
    kp, vp = _pools(n, hkv, d, dt, 930, cuda_device)
    q = randn((b, hq, d), 932, dt).to(cuda_device)
    ip, ix = i32(c.kv_indptr, cuda_device), i32(c.kv_indices, cuda_device)
    s = splits or ops.default_splits(b, hkv, int(lens.max()))
    ws = ops.decode_workspace(b, hq, hkv, d, s, cuda_device)
    print(f"case decode batch 20000 splits={s}", flush=True)
    a = ops.paged_decode_attention(q, kp, vp, ip, ix, d**-0.5, max_splits=s)
    ops.paged_decode_plan(ip, None, b, hq, hkv, d, s, ws)
    p = ops.paged_decode_attention(q, kp, vp, ip, ix, d**-0.5, max_splits=s, workspace=ws, planned=True)
    torch.cuda.synchronize()
    assert torch.equal(a, p), "planned != self-planning"
    pick = [0, 1, 8191, 8192, 8193, 12345, 19998] + [int(np.argmax(lens))]
    ref = _sampled_ref(q, kp, vp, c, pick, d**-0.5)
    assert_close(a[pick], ref, dt, "batch 20000")
    for z in (5, 9000, 19999):
        assert torch.all(a[z] == 0), f"empty request {z} not zero"
