"""numpy restatement of an fp8 KV cache (oracle; test infrastructure only).

The reference names this extension without code (docs/09-exercises.md:81-82:
store the KV pool as int8 / fp8 with one scale per token and head, and change
``store_kv`` (kvcache/pool.py:47-50) and the paged decode kernel accordingly).
The library fixes the format as follows, and the oracle restates it:

- element format: OCP fp8 e4m3 ("e4m3fn": bias 7, 3 mantissa bits, no
  infinities, largest finite 448, S.1111.111 is NaN), round to nearest even;
- one float32 scale per (slot, kv head): amax = max |x| over the head's D
  elements, scale = amax / 448, elements encoded as e4m3(x * (448 / amax)), each
  product and quotient a float32 operation; a row of zeros has scale 0 and
  codes 0;
- attention reads x = decode(code) * scale. Decode over a quantised pool is the
  decode of attention/naive.py:50-60 over the dequantised pool.
"""

from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0


def e4m3_decode(codes) -> np.ndarray:
    """uint8 codes -> float64 values (NaN for the two NaN codes)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    exp = (c >> 3) & 0xF
    man = c & 0x7
    val = np.where(exp == 0, man * 2.0**-9, (1.0 + man / 8.0) * np.exp2(exp.astype(np.float64) - 7.0))
    val = np.where((c & 0x7F) == 0x7F, np.nan, val)
    return sign * val


def e4m3_encode(x) -> np.ndarray:
    """float values -> uint8 codes, round to nearest even. |x| must not exceed 448
    after rounding (the quantiser guarantees it); larger values give NaN."""
    x = np.asarray(x, dtype=np.float64)
    sign = np.where(np.signbit(x), 0x80, 0).astype(np.int64)
    a = np.abs(x)
    # candidate exponent of the normal range, clamped below to the subnormal one
    e = np.floor(np.log2(np.where(a > 0, a, 1.0))).astype(np.int64)
    e = np.maximum(e, -6)
    step = np.exp2((e - 3).astype(np.float64))  # spacing of codes in the binade (2^-9 below 2^-6)
    q = np.rint(a / step).astype(np.int64)  # numpy rint rounds half to even
    # q counts steps from 0: normal binade e holds q in [8, 16); q == 16 rolls over
    e = np.where(q >= 16, e + 1, e)
    q = np.where(q >= 16, q // 2, q)
    normal = q >= 8
    exp_field = np.where(normal, e + 7, 0)
    man_field = np.where(normal, q - 8, q)
    code = sign | (exp_field << 3) | man_field
    overflow = (exp_field > 15) | ((exp_field == 15) & (man_field == 7))
    code = np.where(overflow, sign | 0x7F, code)
    return code.astype(np.uint8)


def quantize_fp8(x) -> "tuple[np.ndarray, np.ndarray]":
    """x [..., D] -> (codes uint8 [..., D], scale float32 [...]) per the format above."""
    x32 = np.asarray(x, dtype=np.float32)
    amax = np.max(np.abs(x32), axis=-1)
    nz = amax > 0
    safe = np.where(nz, amax, np.float32(1.0)).astype(np.float32)
    inv = (np.float32(E4M3_MAX) / safe).astype(np.float32)
    y = (x32 * inv[..., None]).astype(np.float32)
    codes = np.where(nz[..., None], e4m3_encode(y), np.uint8(0)).astype(np.uint8)
    scale = np.where(nz, (safe / np.float32(E4M3_MAX)).astype(np.float32), np.float32(0.0)).astype(np.float32)
    return codes, scale


def dequantize_fp8(codes, scale) -> np.ndarray:
    """(codes [..., D], scale [...]) -> float64 values."""
    return e4m3_decode(codes) * np.asarray(scale, dtype=np.float64)[..., None]


def store_kv_fp8(k_codes, v_codes, k_scale, v_scale, k, v, out_loc) -> None:
    """kvcache/pool.py:47-50 with quantisation: rows of k, v ([T, Hkv, D]) are
    encoded per (token, kv head) and written at slots out_loc, in place."""
    loc = np.asarray(out_loc, dtype=np.int64)
    kc, ks = quantize_fp8(k)
    vc, vs = quantize_fp8(v)
    k_codes[loc] = kc
    v_codes[loc] = vc
    k_scale[loc] = ks
    v_scale[loc] = vs
