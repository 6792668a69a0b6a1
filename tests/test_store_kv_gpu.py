"""KV-store scatter on the GPU: bit-exact vs the oracle (kvcache/pool.py:47-50)."""

import numpy as np
import pytest
import torch

import oracle
from gpu_util import DTYPES, i32, randn
from minisgl_hip import ops

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("t,hkv,d", [(1, 8, 128), (128, 8, 128), (2048, 8, 128), (37, 2, 256), (5, 8, 64)])
def test_store_kv_bit_exact(cuda_device, dtype, t, hkv, d):
    dt = DTYPES[dtype]
    n = 4096
    kp = randn((n, hkv, d), 1, dt).to(cuda_device)
    vp = randn((n, hkv, d), 2, dt).to(cuda_device)
    k = randn((t, hkv, d), 3, dt).to(cuda_device)
    v = randn((t, hkv, d), 4, dt).to(cuda_device)
    loc = np.random.default_rng(t).permutation(n)[:t].astype(np.int32)
    exp_k = kp.cpu().clone()
    exp_v = vp.cpu().clone()
    # oracle on raw bits (int16/int32 views): a copy must be bit-exact
    bits = torch.int32 if dt == torch.float32 else torch.int16
    ek, ev = exp_k.view(bits).numpy(), exp_v.view(bits).numpy()
    oracle.store_kv(ek, ev, k.cpu().view(bits).numpy(), v.cpu().view(bits).numpy(), loc)
    print(f"case store t={t} hkv={hkv} d={d} {dtype}", flush=True)
    ops.store_kv(k, v, i32(loc, cuda_device), kp, vp)
    torch.cuda.synchronize()
    assert np.array_equal(kp.cpu().view(bits).numpy(), ek)
    assert np.array_equal(vp.cpu().view(bits).numpy(), ev)


def test_store_kv_skips_out_of_range_slots(cuda_device):
    """Slots outside [0, N) are never written; valid ones in the same call are."""
    dt = torch.bfloat16
    kp = torch.zeros((64, 8, 128), dtype=dt, device=cuda_device)
    vp = torch.zeros_like(kp)
    k = torch.ones((3, 8, 128), dtype=dt, device=cuda_device)
    loc = i32(np.array([5, 64, -1]), cuda_device)
    print("case store oob", flush=True)
    ops.store_kv(k, k, loc, kp, vp)
    torch.cuda.synchronize()
    assert torch.all(kp[5] == 1)
    assert torch.count_nonzero(kp) == 8 * 128 and torch.count_nonzero(vp) == 8 * 128
