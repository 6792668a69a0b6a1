"""Shared helpers for the GPU parity tests (inputs, tolerances)."""

import numpy as np
import torch

# Tolerances vs the float64 oracle: fp32 max-abs 1e-5; bf16/fp16 2e-2 relative
# (max |o - ref| / max |ref|) plus the reference test's allclose(atol=rtol=2e-2)
# (tests/test_attention.py:38-39).
FP32_ATOL = 1e-5
HALF_REL = 2e-2

DTYPES = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def randn(shape, seed, dtype):
    """N(0,1) drawn in fp32 from a seeded CPU generator, then cast (values exact in the oracle)."""
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype)


def to_np64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def assert_close(out: torch.Tensor, ref: np.ndarray, dtype: torch.dtype, what: str = ""):
    o = to_np64(out)
    assert np.all(np.isfinite(o)), f"{what}: non-finite output"
    err = np.abs(o - ref)
    if dtype == torch.float32:
        assert err.max() <= FP32_ATOL, f"{what}: max abs err {err.max():.3e} > {FP32_ATOL}"
    else:
        rel = err.max() / max(np.abs(ref).max(), 1e-30)
        assert rel <= HALF_REL, f"{what}: rel err {rel:.3e} > {HALF_REL}"
        assert np.allclose(o, ref, atol=HALF_REL, rtol=HALF_REL), f"{what}: allclose(2e-2) failed"
    return float(err.max())


def i32(x, device):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.int32)).to(device)
