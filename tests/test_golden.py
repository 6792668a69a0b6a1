"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
from the float64 oracle): the oracle must keep reproducing them (CPU), and the
HIP kernels must match them in fp32 to 1e-5 (GPU). Inputs are regenerated from
the recorded seeds with the seeded CPU generator of gpu_util.randn."""

from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from gpu_util import FP32_ATOL, i32, randn

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _decode_inputs(fx):
    n, b, hq, hkv, d, ps = (int(x) for x in fx["shape"])
    seed = int(fx["seed"])
    kp = randn((n, hkv, d), seed, torch.float32)
    vp = randn((n, hkv, d), seed + 1, torch.float32)
    q = randn((b, hq, d), seed + 2, torch.float32)
    return q, kp, vp, d, ps


def _prefill_inputs(fx):
    n, t, hq, hkv, d = (int(x) for x in fx["shape"])
    seed = int(fx["seed"])
    kp = randn((n, hkv, d), seed, torch.float32)
    vp = randn((n, hkv, d), seed + 1, torch.float32)
    q = randn((t, hq, d), seed + 2, torch.float32)
    return q, kp, vp, d


DECODE = ["decode_reference_grid", "decode_cpu_config", "decode_page16"]


@pytest.mark.parametrize("name", DECODE)
def test_oracle_reproduces_decode_fixture(name):
    fx = _load(name)
    q, kp, vp, d, ps = _decode_inputs(fx)
    out = oracle.paged_decode(q.double().numpy(), kp.double().numpy(), vp.double().numpy(), fx["kv_indptr"],
                              fx["kv_indices"], d**-0.5, page_size=ps, seq_lens=fx.get("seq_lens"))
    np.testing.assert_allclose(out, fx["expected"], rtol=1e-6, atol=1e-6)


def test_oracle_reproduces_prefill_fixture():
    fx = _load("prefill_edges")
    q, kp, vp, d = _prefill_inputs(fx)
    qi, ki, kx = fx["q_indptr"], fx["kv_indptr"], fx["kv_indices"]
    P = fx["seq_lens"] - np.diff(qi)
    kvi = [None if P[i] == 0 else kx[ki[i]:ki[i + 1]] for i in range(len(P))]
    # extend rows are the pool rows at the last E slots of each request
    out_loc = np.concatenate([kx[ki[i] + P[i]:ki[i + 1]] for i in range(len(P))])
    kn, vn = kp.double().numpy()[out_loc], vp.double().numpy()[out_loc]
    out = oracle.forward_prefill(q.double().numpy(), kn, vn, kp.double().numpy(), vp.double().numpy(), qi.tolist(),
                                 kvi, d**-0.5)
    np.testing.assert_allclose(out, fx["expected"], rtol=1e-6, atol=1e-6)


@pytest.mark.gpu
@pytest.mark.parametrize("name", DECODE)
def test_decode_kernel_matches_fixture(cuda_device, name):
    from minisgl_hip import ops

    fx = _load(name)
    q, kp, vp, d, ps = _decode_inputs(fx)
    print(f"case golden {name}", flush=True)
    seq = fx.get("seq_lens")
    out = ops.paged_decode_attention(
        q.to(cuda_device), kp.to(cuda_device), vp.to(cuda_device), i32(fx["kv_indptr"], cuda_device),
        i32(fx["kv_indices"], cuda_device), d**-0.5, page_size=ps,
        seq_lens=None if seq is None else i32(seq, cuda_device),
    )
    torch.cuda.synchronize()
    err = np.abs(out.cpu().double().numpy() - fx["expected"]).max()
    assert err <= FP32_ATOL, f"{name}: max abs err {err:.3e}"


@pytest.mark.gpu
def test_prefill_kernel_matches_fixture(cuda_device):
    from minisgl_hip import ops

    fx = _load("prefill_edges")
    q, kp, vp, d = _prefill_inputs(fx)
    print("case golden prefill_edges", flush=True)
    out = ops.prefill_ragged_attention(
        q.to(cuda_device), kp.to(cuda_device), vp.to(cuda_device), i32(fx["q_indptr"], cuda_device),
        i32(fx["kv_indptr"], cuda_device), i32(fx["kv_indices"], cuda_device), i32(fx["seq_lens"], cuda_device),
        d**-0.5, max_extend_len=int(np.diff(fx["q_indptr"]).max()),
    )
    torch.cuda.synchronize()
    err = np.abs(out.cpu().double().numpy() - fx["expected"]).max()
    assert err <= FP32_ATOL, f"prefill_edges: max abs err {err:.3e}"
