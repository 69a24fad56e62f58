"""Bit-level bf16 and OCP FP8 (e4m3fn) conversions in numpy.

Test infrastructure only (see ``oracle/__init__.py``).

The reference stores activations as bf16 and expert weights / quantised
activations as ``torch.float8_e4m3fn`` (OCP E4M3, no infinities, one NaN code
per sign, max finite 448).  Conversions to fp8 happen in Triton stores
(``moe_input.py:26-27``: ``q = clamp(x / scale, -448, 448)`` stored to an e4m3
buffer) which round to nearest, ties to even.  numpy has no fp8 type, so these
helpers work on the raw bit patterns; ``tests/test_oracle_numerics.py`` pins
them exhaustively against torch's own casts.
"""

from __future__ import annotations

import numpy as np

F32_464 = np.uint32(0x43E80000)  # 464.0: first magnitude torch maps to NaN
F32_MIN_NORMAL_E4M3 = np.uint32(0x3C800000)  # 2**-6


def f32_bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


def bits_f32(b: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(b, dtype=np.uint32).view(np.float32)


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float32 (exact)."""
    return bits_f32(np.asarray(h, dtype=np.uint32) << 16)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even; NaN stays NaN."""
    b = f32_bits(x).astype(np.uint64)
    rounded = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    out = np.where(nan, (b >> 16) | 0x40, rounded)
    return out.astype(np.uint16)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bf16 value, returned as float32."""
    return bf16_to_f32(f32_to_bf16(x))


def _e4m3_table() -> np.ndarray:
    table = np.empty(256, dtype=np.float32)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        exponent = (code >> 3) & 0xF
        mantissa = code & 7
        if exponent == 15 and mantissa == 7:
            table[code] = np.nan
        elif exponent == 0:
            table[code] = sign * mantissa * 2.0**-9
        else:
            table[code] = sign * (1.0 + mantissa / 8.0) * 2.0 ** (exponent - 7)
    return table


E4M3_TABLE = _e4m3_table()


def e4m3_to_f32(codes: np.ndarray) -> np.ndarray:
    """e4m3fn codes (uint8) -> float32 (exact)."""
    return E4M3_TABLE[np.asarray(codes, dtype=np.uint8)]


def f32_to_e4m3(x: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn codes, round to nearest even.

    Follows torch's ``float8_e4m3fn`` conversion: magnitudes >= 464 and NaN
    become the NaN code (0x7F | sign); smaller magnitudes round to nearest
    even, including into the subnormal range (step 2**-9).  The MoE path
    clamps to +-448 before converting, so the NaN branch is never taken there.
    """
    bits = f32_bits(x)
    sign = ((bits >> 24) & 0x80).astype(np.uint8)
    mag = bits & np.uint32(0x7FFFFFFF)
    out = np.zeros(bits.shape, dtype=np.uint8)

    nan = mag >= F32_464  # includes inf and NaN payloads (> 0x7F800000)
    sub = mag < F32_MIN_NORMAL_E4M3
    norm = ~nan & ~sub

    # Subnormal / zero range: value = m * 2**-9, m in [0, 8]; m == 8 is the
    # smallest normal code 0x08, which the integer encoding produces directly.
    if np.any(sub):
        v = bits_f32(mag[sub]) * np.float32(512.0)  # exact power-of-two scaling
        out[sub] = np.rint(v).astype(np.uint8)  # rint: ties to even

    if np.any(norm):
        m = mag[norm]
        # Re-bias the exponent (127 -> 7) and keep 3 mantissa bits, RNE.
        shifted = ((m >> 23).astype(np.int64) - 120) << 3 | ((m >> 20) & 7).astype(np.int64)
        rest = (m & np.uint32(0xFFFFF)).astype(np.int64)
        half = 0x80000
        round_up = (rest > half) | ((rest == half) & ((shifted & 1) == 1))
        out[norm] = (shifted + round_up).astype(np.uint8)

    out[nan] = 0x7F
    return out | sign


def f64_to_bf16(x: np.ndarray) -> np.ndarray:
    """float64 -> bf16 bit patterns with a single round-to-nearest-even.

    Used for the reference's single-rounding bf16 FMA (``kernels.py:467-474``):
    the exact f64 value of ``a*b + c`` for bf16 operands is rounded once.
    Finite, normal-range inputs only (the combine operands are activations).
    """
    b = np.ascontiguousarray(x, dtype=np.float64).view(np.uint64)
    sign = (b >> 63).astype(np.uint64)
    mag = b & np.uint64(0x7FFFFFFFFFFFFFFF)
    # bf16 keeps 7 of the 52 mantissa bits: drop 45 bits with RNE.
    drop = np.uint64(45)
    half = np.uint64(1) << np.uint64(44)
    rest = mag & ((np.uint64(1) << drop) - np.uint64(1))
    kept = mag >> drop
    round_up = (rest > half) | ((rest == half) & ((kept & np.uint64(1)) == 1))
    kept = kept + round_up.astype(np.uint64)
    # kept now holds (f64 exponent << 7 | mantissa7); re-bias 1023 -> 127.
    exponent = (kept >> np.uint64(7)).astype(np.int64) - 1023 + 127
    mantissa = (kept & np.uint64(0x7F)).astype(np.int64)
    zero = mag == 0
    if np.any(~zero & ((exponent <= 0) | (exponent >= 255))):
        raise ValueError("f64_to_bf16 handles normal-range values only")
    out = np.where(zero, 0, (exponent << 7) | mantissa).astype(np.uint64)
    return (out | (sign << np.uint64(15))).astype(np.uint16)
