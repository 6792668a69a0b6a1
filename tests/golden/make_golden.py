"""Writes the golden fixtures of this directory from the float64 oracle.

Each fixture records the seeds and shapes of its inputs (q, K, V are drawn by
``gpu_util.randn``: N(0,1) in fp32 from a seeded CPU ``torch.Generator``, then
cast), the int32 index data, and the oracle's expected output (stored as
float32). Regenerate with ``python tests/golden/make_golden.py`` from the
repository root; ``tests/test_golden.py`` checks the oracle against them on the
CPU and the HIP kernels against them on the GPU.

Cases (the reference's own fixtures, tests/test_attention.py:19-39, and the
small cases listed for the path):
  decode_reference_grid  pool N=4096, B=7, lens [1,2,17,31,32,33,700], slots from
                         np.random.default_rng(0).permutation(4096) (as
                         tests/test_attention.py:21-33), 16 q / 8 kv / 128, fp32
  decode_cpu_config      B=8, L ~ U[100,1024] seed 0, pool 16384, 16 q / 8 kv / 128, fp32
  decode_page16          B=5 page ids of 16-slot pages, 32 q / 8 kv / 128, fp32
  prefill_edges          P in {0,1,17,300}, E in {1,2,64,3}, 16 q / 8 kv / 64, fp32
"""

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
for p in (str(ROOT), str(ROOT / "mini-sglang-mlx_amd"), str(HERE.parent)):
    if p not in sys.path:
        sys.path.insert(0, p)

import torch  # noqa: E402

import oracle  # noqa: E402
from gpu_util import randn  # noqa: E402
from minisgl_hip import workloads  # noqa: E402


def _np(t):
    return t.double().numpy()


def decode_fixture(case, hq, hkv, d, seed, page_size=1):
    n = case.num_slots
    kp = randn((n, hkv, d), seed, torch.float32)
    vp = randn((n, hkv, d), seed + 1, torch.float32)
    q = randn((case.batch_size, hq, d), seed + 2, torch.float32)
    if page_size == 1:
        indptr, indices, seq = case.kv_indptr, case.kv_indices, None
    else:
        indptr, indices, seq = case.page_indptr, case.page_ids, case.lens
    out = oracle.paged_decode(_np(q), _np(kp), _np(vp), indptr, indices, d**-0.5, page_size=page_size,
                              seq_lens=seq)
    fx = dict(seed=seed, shape=np.array([n, case.batch_size, hq, hkv, d, page_size]), kv_indptr=indptr,
              kv_indices=indices, expected=out.astype(np.float32))
    if seq is not None:
        fx["seq_lens"] = seq
    return fx


def prefill_fixture(case, hq, hkv, d, seed):
    n = case.num_slots
    kp = randn((n, hkv, d), seed, torch.float32)
    vp = randn((n, hkv, d), seed + 1, torch.float32)
    q = randn((case.num_tokens, hq, d), seed + 2, torch.float32)
    kvi = [None if case.prefix_lens[i] == 0 else case.kv_indices[case.kv_indptr[i]:case.kv_indptr[i + 1]]
           for i in range(len(case.seq_lens))]
    # the extend rows are already in the pool at out_loc (stored before attention)
    kn = _np(kp)[case.out_loc]
    vn = _np(vp)[case.out_loc]
    out = oracle.forward_prefill(_np(q), kn, vn, _np(kp), _np(vp), case.q_indptr.tolist(), kvi, d**-0.5)
    return dict(seed=seed, shape=np.array([n, case.num_tokens, hq, hkv, d]), q_indptr=case.q_indptr,
                kv_indptr=case.kv_indptr, kv_indices=case.kv_indices, seq_lens=case.seq_lens,
                expected=out.astype(np.float32))


def build():
    fixtures = {
        "decode_reference_grid": decode_fixture(workloads.reference_test_case(), 16, 8, 128, 1000),
        "decode_cpu_config": decode_fixture(workloads.decode_case(8, 100, 1024, 16384, 1, seed=0), 16, 8, 128, 1010),
        "decode_page16": decode_fixture(workloads.decode_case_from_lens([1, 15, 16, 17, 300], 4096, 16, seed=2),
                                        32, 8, 128, 1020, page_size=16),
        "prefill_edges": prefill_fixture(
            workloads.prefill_case_from_lens([0, 1, 17, 300], [1, 2, 64, 3], num_slots=1024, seed=3), 16, 8, 64,
            1030),
    }
    return fixtures


if __name__ == "__main__":
    for name, fx in build().items():
        np.savez_compressed(HERE / f"{name}.npz", **fx)
        print(name, {k: np.shape(v) for k, v in fx.items()})
