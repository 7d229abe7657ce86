"""Oracle for the per-row e4m3 weight quantiser of the fp8 weight path (test infrastructure only).

The fp8 weight format the head takes: per row v, scale_v = max(max_k |W[v, k]| / 448, 1e-12) in fp32 (448 is the
largest OCP e4m3 value), and q[v, k] = e4m3(clamp(W[v, k] / scale_v, -448, 448)), the fp32 quotient rounded to the
nearest e4m3 value, ties to the even code. The reference itself ships no quantiser; this restates the format with
plain integer arithmetic on the fp32 bit patterns (no float8 library type), and tests/test_oracle.py pins it
against torch's float8_e4m3fn conversion over every fp32 bit pattern of the e4m3 range's codes, midpoints and their
neighbours.

OCP e4m3: 1 sign bit, 4 exponent bits (bias 7), 3 mantissa bits; codes 0x01..0x07 are the subnormals m * 2^-9;
0x7f / 0xff are NaN, so the largest finite magnitude is 0x7e = 448.
"""

from __future__ import annotations

import numpy as np


def e4m3_bits(x) -> np.ndarray:
    """uint8 OCP e4m3 codes of float32 values |x| <= 448, round to nearest, ties to even."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.int64)
    sign = ((u >> 31) & 1).astype(np.uint8) << 7
    mag = u & 0x7FFFFFFF
    exp = mag >> 23
    man = mag & 0x7FFFFF
    # value = (2^23 + man) * 2^(exp - 150) for normals; the e4m3 grid step at this magnitude is 2^(e - 3) for a
    # normal result of unbiased exponent e >= -6, and 2^-9 below that (subnormals)
    e_unb = exp - 127
    step_exp = np.maximum(e_unb, -6) - 3                     # log2 of the e4m3 grid step
    full = np.where(exp > 0, (1 << 23) + man, man)         # the fp32 significand as an integer
    shift = step_exp - (np.where(exp > 0, e_unb, -126) - 23)  # bits of `full` below the grid step
    shift = np.clip(shift, 0, 62)
    q = full >> shift                                       # grid units, truncated
    rem = full - (q << shift)
    half = np.where(shift > 0, 1 << np.maximum(shift - 1, 0), 0)
    up = (rem > half) | ((rem == half) & (shift > 0) & ((q & 1) == 1))
    q = q + up                                              # rounded count of 2^step_exp units
    # q units of 2^step_exp: subnormal range (step -9) holds q = 0..8 (8 is the smallest normal, 2^-6);
    # normal range: q in [8, 16] units of 2^(e-3); 16 carries into the next exponent
    e_res = np.where(step_exp == -9, -6, step_exp + 3)
    carry = q >= 16
    q = np.where(carry, q >> 1, q)
    e_res = np.where(carry, e_res + 1, e_res)
    normal = q >= 8
    code = np.where(normal, ((e_res + 7) << 3) | (q - 8), q)
    code = np.where(mag == 0, 0, code)
    return (code.astype(np.uint8) | sign).astype(np.uint8)


def e4m3_value(code) -> np.ndarray:
    """float64 values of uint8 OCP e4m3 codes (NaN for 0x7f / 0xff)."""
    c = np.asarray(code, dtype=np.int64)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 7
    v = np.where(e == 0, m * 2.0 ** -9, (1 + m / 8.0) * 2.0 ** (e - 7.0))
    return np.where((c & 0x7F) == 0x7F, np.nan, s * v)


def quantise_rows(W) -> tuple[np.ndarray, np.ndarray]:
    """(q [V, d] uint8 e4m3 codes, scale [V] float32) of W [V, d] (any float dtype, computed in fp32)."""
    W32 = np.asarray(W, dtype=np.float32)
    amax = np.abs(W32).max(axis=1) if W32.shape[1] else np.zeros(W32.shape[0], dtype=np.float32)
    scale = np.maximum(amax / np.float32(448.0), np.float32(1e-12)).astype(np.float32)
    x = np.clip(W32 / scale[:, None], np.float32(-448.0), np.float32(448.0)).astype(np.float32)
    return e4m3_bits(x), scale
