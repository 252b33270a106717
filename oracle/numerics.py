"""Number formats used by the FP8 hot path (oracle, test infrastructure only).

* OCP float8 e4m3fn: 1 sign bit, 4 exponent bits (bias 7), 3 mantissa bits, no
  infinities, NaN = 0x7F/0xFF, max finite 448 (0x7E).  The reference converts with
  Triton ``.to(tl.float8e4nv)`` (kernels/fp8_linear.py:22,
  kernels/fp8_attention.py:73,115,168) and reinterprets bytes with
  ``.to(tl.float8e4nv, bitcast=True)`` (kernels/fp8_attention.py:279); torch's
  ``float8_e4m3fn`` has the same bit patterns.  Rounding is round-to-nearest-even.
* bfloat16: the top 16 bits of an IEEE fp32 value, rounded to nearest even.

Both are implemented here from the format definitions (float64 / integer
arithmetic), independently of torch, so that the tests can pin them against torch.
"""
from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0
_MIN_NORMAL = 2.0 ** -6     # smallest normal e4m3 value (code 0x08)
_SUB_STEP = 2.0 ** -9       # spacing of e4m3 subnormals


def absmax_maxnum(x, axis) -> np.ndarray:
    """max |x| over `axis` with IEEE maxNum semantics: NaN elements are skipped (all-NaN
    gives NaN).  The reference's Triton `tl.max` / `tl.maximum` (default: no NaN
    propagation; `max.f32` on its GPUs) behave so (kernels/fp8_linear.py:20-21)."""
    return np.fmax.reduce(np.abs(np.asarray(x, np.float32)), axis=axis)


def clamp448_maxnum(q) -> np.ndarray:
    """`tl.minimum(tl.maximum(q, -448), 448)` (kernels/fp8_linear.py:22) with maxNum /
    minNum semantics: a NaN quotient becomes -448."""
    return np.fmin(np.fmax(q, np.float32(-E4M3_MAX)), np.float32(E4M3_MAX))


def e4m3_encode(x) -> np.ndarray:
    """Round fp32 values to e4m3fn codes (uint8), round-to-nearest-even.

    Magnitudes that round above 448 become NaN (0x7F | sign), like torch's cast;
    NaN inputs give 0x7F.  Callers on the hot path clamp to +-448 first.
    """
    x = np.asarray(x, dtype=np.float32)
    sign = np.where(np.signbit(x), 0x80, 0x00).astype(np.int64)
    a = np.abs(x).astype(np.float64)
    with np.errstate(invalid="ignore", divide="ignore"):
        mant, exp = np.frexp(a)               # a = mant * 2**exp, mant in [0.5, 1)
        e = exp.astype(np.int64) - 1           # a = (2*mant) * 2**e
        frac8 = np.rint((2.0 * mant - 1.0) * 8.0)   # exact in float64; RNE
        normal = (e + 7) * 8 + frac8.astype(np.int64)  # a mantissa carry bumps the exponent
        sub = np.rint(a / _SUB_STEP).astype(np.int64)  # 0..8 (8 == smallest normal)
    code = np.where(a < _MIN_NORMAL, sub, normal)
    code = np.where(np.isnan(a) | (code > 0x7F), 0x7F, code)  # overflow -> NaN (e4m3fn has no inf)
    code = np.where(np.isinf(a), 0x7F, code)
    return (code | sign).astype(np.uint8)


def e4m3_decode(codes) -> np.ndarray:
    """Exact fp32 value of e4m3fn codes (uint8 array)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    mag = np.where(e == 0, m * _SUB_STEP, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    mag = np.where((c & 0x7F) == 0x7F, np.nan, mag)
    return (s * mag).astype(np.float32)


def bf16_round(x) -> np.ndarray:
    """Round fp32 values to the nearest bfloat16 (ties to even); returns fp32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    r = np.where(np.isnan(x), u | 0x00400000, r)  # keep NaN a (quiet) NaN
    return r.astype(np.uint32).view(np.float32)


def bf16_bits(x) -> np.ndarray:
    """bfloat16 bit patterns (uint16) of fp32 values after RNE rounding."""
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(bits) -> np.ndarray:
    """fp32 values of bfloat16 bit patterns."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
