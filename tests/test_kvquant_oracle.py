"""Pins for the fp8 KV-cache oracle (no GPU).

The e4m3 encoder/decoder is checked against torch's ``float8_e4m3fn`` casts (an
independent implementation of the OCP format) on every code, every midpoint
between neighbouring codes (ties to even) and random values over the whole
range; the quantiser against closed forms: the largest element of each
(token, head) maps to exactly +-448, a zero row has scale 0, and the
dequantised value is within half a code step of the input. Mutants (ties away
from zero, a scale of amax/240, a dropped scale on dequantisation) are rejected.
"""

import numpy as np
import pytest
import torch

import oracle


def _torch_encode(x):
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_decode_matches_torch_on_every_code():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    dec = oracle.e4m3_decode(codes)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(dec), nan) and nan.sum() == 2
    np.testing.assert_array_equal(dec[~nan], ref[~nan])
    assert oracle.e4m3_decode([0x7E])[0] == 448.0 and oracle.e4m3_decode([0x01])[0] == 2.0**-9


def test_e4m3_encode_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    vals = oracle.e4m3_decode(codes)
    finite = vals[~np.isnan(vals)].astype(np.float32)
    np.testing.assert_array_equal(oracle.e4m3_encode(finite), _torch_encode(finite))  # exact codes
    pos = np.unique(finite[finite >= 0])
    mids = ((pos[1:].astype(np.float64) + pos[:-1]) / 2).astype(np.float32)  # ties: round half to even
    mids = np.concatenate([mids, -mids])
    np.testing.assert_array_equal(oracle.e4m3_encode(mids), _torch_encode(mids))
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(100000) * np.exp(rng.uniform(-12, 6.1, 100000))).astype(np.float32)
    x = x[np.abs(x) <= 448]
    np.testing.assert_array_equal(oracle.e4m3_encode(x), _torch_encode(x))


def test_quantize_closed_forms():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((50, 8, 128)) * np.exp(rng.uniform(-6, 6, (50, 8, 1)))).astype(np.float32)
    x[3, 2] = 0.0  # a zero row
    codes, scale = oracle.quantize_fp8(x)
    assert codes.dtype == np.uint8 and scale.dtype == np.float32 and scale.shape == (50, 8)
    assert scale[3, 2] == 0 and not codes[3, 2].any()
    dec = oracle.e4m3_decode(codes)
    # the largest |element| of every non-zero row is encoded as +-448
    idx = np.argmax(np.abs(x), axis=-1)
    top = np.take_along_axis(dec, idx[..., None], axis=-1)[..., 0]
    nz = scale > 0
    np.testing.assert_array_equal(np.abs(top[nz]), 448.0)
    np.testing.assert_allclose(scale[nz], np.abs(x).max(-1)[nz] / 448.0, rtol=1e-7)
    # dequantised values are within half a code step (relative 2^-4, or 2^-10 x scale below the normal range)
    deq = oracle.dequantize_fp8(codes, scale)
    bound = np.maximum(np.abs(x) * 2.0**-4, scale[..., None] * 2.0**-10) * (1 + 1e-6)
    assert np.all(np.abs(deq - x) <= bound)


def test_store_kv_fp8_oracle():
    rng = np.random.default_rng(2)
    k = rng.standard_normal((5, 2, 16)).astype(np.float32)
    v = rng.standard_normal((5, 2, 16)).astype(np.float32)
    kc = np.full((32, 2, 16), 7, np.uint8)
    vc = kc.copy()
    ks = np.full((32, 2), 3.0, np.float32)
    vs = ks.copy()
    loc = np.array([9, 0, 31, 4, 17])
    oracle.store_kv_fp8(kc, vc, ks, vs, k, v, loc)
    c, s = oracle.quantize_fp8(k)
    np.testing.assert_array_equal(kc[loc], c)
    np.testing.assert_array_equal(ks[loc], s)
    rest = np.setdiff1d(np.arange(32), loc)
    assert (kc[rest] == 7).all() and (vs[rest] == 3.0).all()


def _mutant_ties_away(x):
    """Planted mistake: round half away from zero."""
    a = np.abs(np.asarray(x, np.float64))
    e = np.maximum(np.floor(np.log2(np.where(a > 0, a, 1.0))), -6)
    step = np.exp2(e - 3)
    q = np.floor(a / step + 0.5)
    return oracle.e4m3_decode(oracle.e4m3_encode(np.sign(x) * q * step))


def test_kvquant_mutants_are_caught():
    pos = np.unique(oracle.e4m3_decode(np.arange(127, dtype=np.uint8)))
    mids = ((pos[1:] + pos[:-1]) / 2).astype(np.float32)
    ref = torch.from_numpy(mids).to(torch.float8_e4m3fn).float().numpy()
    assert not np.array_equal(_mutant_ties_away(mids), ref)
    # a scale for the 240-max format fails the "largest element is 448" form
    x = np.random.default_rng(3).standard_normal((4, 64)).astype(np.float32)
    codes = oracle.e4m3_encode(x * (240.0 / np.abs(x).max(-1, keepdims=True)))
    assert not np.all(np.abs(oracle.e4m3_decode(codes)).max(-1) == 448.0)
    # dequantising without the scale fails the half-step bound
    c, s = oracle.quantize_fp8(x)
    assert not np.all(np.abs(oracle.e4m3_decode(c) - x) <= np.abs(x) * 2.0**-4 + 1e-3)
