"""OCP float8 e4m3fn and bfloat16 codecs in numpy (test infrastructure only).

The reference harness quantises with ``(x / scale).to(torch.float8_e4m3fn)``
(tests/utils.py:68, tests/kernels/test_pa.py:346-351) and casts the attention
output with ``.to(torch.bfloat16)`` (tests/kernels/test_pa.py:273, :330).
This module restates both conversions from the format definitions:

* e4m3fn: 1 sign, 4 exponent bits (bias 7), 3 mantissa bits, no infinities,
  NaN = S.1111.111, largest finite 448, subnormals m * 2**-9.
  float -> e4m3fn rounds to nearest, ties to even; a value whose rounded
  magnitude exceeds 448 (and +-inf / NaN) becomes NaN (0x7F | sign).
* bfloat16: the upper 16 bits of an IEEE float32, rounded to nearest even.

Both are pinned against torch's own casts in tests/test_oracle_codecs.py.
"""

from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0


def _build_decode_table() -> np.ndarray:
    tab = np.zeros(256, dtype=np.float32)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        exp = (code >> 3) & 0xF
        man = code & 0x7
        if exp == 0xF and man == 0x7:
            tab[code] = np.nan
        elif exp == 0:
            tab[code] = sign * man * 2.0**-9
        else:
            tab[code] = sign * (1.0 + man / 8.0) * 2.0 ** (exp - 7)
    return tab


E4M3_DECODE = _build_decode_table()


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """uint8 e4m3fn codes -> float32 values (exact)."""
    return E4M3_DECODE[np.asarray(codes, dtype=np.uint8)]


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """float32 -> uint8 e4m3fn codes, round-to-nearest-even, overflow -> NaN."""
    with np.errstate(invalid="ignore", over="ignore"):
        return _e4m3_encode(x)


def _e4m3_encode(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32).astype(np.float64)
    sign = np.signbit(x).astype(np.uint8) << 7
    a = np.abs(x)
    out = np.zeros(x.shape, dtype=np.uint8)
    finite = np.isfinite(a)
    a_f = np.where(finite, a, 0.0)
    # subnormal range: a < 2**-6 -> code = rint(a / 2**-9) (a code of 8 is the
    # smallest normal, so rounding up across the boundary is already correct)
    sub = a_f < 2.0**-6
    q_sub = np.rint(a_f * 2.0**9)
    # normal range: a = m * 2**e with m in [1, 2)
    mant, e2 = np.frexp(np.where(sub, 1.0, a_f))  # mant in [0.5, 1)
    e = e2 - 1
    q = np.rint(mant * 16.0)  # 1.xxx scaled by 8 -> [8, 16]
    bump = q >= 16.0
    q = np.where(bump, 8.0, q)
    e = np.where(bump, e + 1, e)
    exp_field = e + 7
    normal_code = (exp_field.astype(np.int64) << 3) | (q.astype(np.int64) - 8)
    overflow = (exp_field > 15) | ((exp_field == 15) & (q - 8 >= 7))
    code = np.where(sub, np.where(finite, q_sub, 0).astype(np.int64), normal_code)
    code = np.where(overflow & ~sub, 0x7F, code)
    code = np.where(finite, code, 0x7F)
    out[...] = code.astype(np.uint8)
    return out | sign


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 (returned as float32 holding the bf16 value)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> uint16 bf16 bit patterns, round to nearest even (NaN -> 0x7FC0)."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    bits = x.view(np.uint32).astype(np.uint64)
    lsb = (bits >> 16) & 1
    rounded = ((bits + 0x7FFF + lsb) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        rounded = np.where(nan, np.uint16(0x7FC0), rounded)
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)
