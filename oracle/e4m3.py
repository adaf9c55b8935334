"""Independent float8_e4m3fn codec (numpy), from the OCP 8-bit FP spec.

E4M3 ("fn" variant): 1 sign, 4 exponent bits (bias 7), 3 mantissa bits, no
infinities, S.1111.111 is NaN, max finite 448, subnormals 2^-6 * m/8.

``encode`` reproduces what ``torch.Tensor.to(torch.float8_e4m3fn)`` is
documented to do on CPU: round to nearest, ties to even; magnitudes that
round past 448 (i.e. > 464, the midpoint to the next binade slot) and NaN /
inf become the NaN code 0x7F with the input's sign bit.  The test suite
checks this codec against torch over every bf16 bit pattern, so the oracle's
use of torch's conversion is pinned by an implementation that shares no code
with it.
"""

from __future__ import annotations

import numpy as np


def decode_table() -> np.ndarray:
    """float64 value of every code 0..255 (NaN for 0x7F / 0xFF)."""
    out = np.empty(256, dtype=np.float64)
    for code in range(256):
        s = -1.0 if code & 0x80 else 1.0
        e = (code >> 3) & 0xF
        m = code & 0x7
        if e == 0xF and m == 0x7:
            out[code] = np.nan
        elif e == 0:
            out[code] = s * (m / 8.0) * 2.0 ** -6
        else:
            out[code] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return out


_TABLE = decode_table()
# Positive magnitudes for codes 0x00..0x7E plus the virtual slot 0x7F = 480,
# which only serves as the upper neighbour of 448 for rounding.
_POS = np.concatenate([_TABLE[:0x7F], [480.0]])


def decode(codes: np.ndarray) -> np.ndarray:
    return _TABLE[np.asarray(codes, dtype=np.uint8)]


def encode(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even encode of float values (any float dtype) to uint8 codes."""
    x = np.asarray(x, dtype=np.float64)
    sign = np.signbit(x).astype(np.uint8) << 7
    a = np.abs(x)
    nan = ~np.isfinite(a)
    a = np.where(nan, 0.0, a)
    hi = np.searchsorted(_POS, a, side="left")  # first slot >= a
    hi = np.clip(hi, 0, 0x7F)
    lo = np.clip(hi - 1, 0, 0x7F)
    d_hi = _POS[hi] - a
    d_lo = a - _POS[lo]
    exact = d_hi == 0
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (hi % 2 == 0))
    code = np.where(exact, hi, np.where(pick_hi, hi, lo)).astype(np.int64)
    code = np.where(a > 480.0, 0x7F, code)
    code = np.where(nan, 0x7F, code)
    return (code.astype(np.uint8) | sign).astype(np.uint8)
