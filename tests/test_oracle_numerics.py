"""Pin the oracle's bit-level conversions against torch's own casts and exact
rational arithmetic (CPU only)."""

from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle.numerics import (
    E4M3_TABLE,
    bf16_to_f32,
    e4m3_to_f32,
    f32_to_bf16,
    f32_to_e4m3,
    f64_to_bf16,
)


def torch_e4m3(values: np.ndarray) -> np.ndarray:
    return torch.from_numpy(values.astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_decode_table_matches_torch():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    expected = codes.view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(expected)
    assert np.array_equal(nan, np.isnan(E4M3_TABLE))
    assert np.array_equal(expected[~nan], E4M3_TABLE[~nan])
    assert E4M3_TABLE[0x7E] == 448.0 and E4M3_TABLE[0x01] == 2.0**-9


def test_e4m3_encode_exhaustive_over_bf16_values():
    """Every bf16 bit pattern (as fp32) in the finite range below the NaN
    threshold converts exactly as torch's float8_e4m3fn cast."""
    bits = np.arange(1 << 16, dtype=np.uint32)
    values = bf16_to_f32(bits.astype(np.uint16))
    finite = np.isfinite(values) & (np.abs(values) < 464.0)
    ours = f32_to_e4m3(values[finite])
    assert np.array_equal(ours, torch_e4m3(values[finite]))


def test_e4m3_encode_random_fp32_and_ties():
    rng = np.random.default_rng(0)
    values = (rng.standard_normal(200_000) * np.exp(rng.uniform(-12, 6, 200_000))).astype(np.float32)
    values = values[np.abs(values) < 464]
    assert np.array_equal(f32_to_e4m3(values), torch_e4m3(values))
    # exact midpoints between neighbouring codes round to the even code
    finite = E4M3_TABLE[:0x7F]
    mids = ((finite[:-1].astype(np.float64) + finite[1:]) / 2).astype(np.float32)
    assert np.array_equal(f32_to_e4m3(mids), torch_e4m3(mids))
    assert np.array_equal(f32_to_e4m3(-mids), torch_e4m3(-mids))


def test_e4m3_saturation_clamps_before_nan():
    # The MoE path clamps to +-448 first; 448 itself and values up to the
    # midpoint 464 map to the max code, beyond that torch produces NaN.
    values = np.array([448.0, 455.0, 463.9, -448.0, -463.9], np.float32)
    assert list(f32_to_e4m3(values)) == [0x7E, 0x7E, 0x7E, 0xFE, 0xFE]
    assert f32_to_e4m3(np.array([464.0, 1e6, np.inf, np.nan], np.float32)).tolist() == [0x7F] * 4


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(1)
    values = (rng.standard_normal(300_000) * np.exp(rng.uniform(-30, 30, 300_000))).astype(np.float32)
    # add exact ties: bf16 value + half ulp
    base = f32_to_bf16(values[:1000])
    ties = (base.astype(np.uint32) << 16 | 0x8000).view(np.float32)
    values = np.concatenate([values, ties, -ties])
    expected = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(f32_to_bf16(values), expected)


def _exact_bf16(x: Fraction) -> int:
    """Round an exact rational to bf16 bits (RNE) by brute force."""
    sign = 1 if x < 0 else 0
    x = abs(x)
    if x == 0:
        return sign << 15
    e = 0
    while x >= 2:
        x /= 2
        e += 1
    while x < 1:
        x *= 2
        e -= 1
    scaled = x * 128  # [128, 256)
    m = int(scaled)
    rest = scaled - m
    if rest > Fraction(1, 2) or (rest == Fraction(1, 2) and m % 2 == 1):
        m += 1
    if m == 256:
        m, e = 128, e + 1
    return (sign << 15) | ((e + 127) << 7) | (m - 128)


def test_fma_single_rounding_against_exact_rationals():
    rng = np.random.default_rng(2)
    a = f32_to_bf16(rng.standard_normal(3000).astype(np.float32))
    b = f32_to_bf16(rng.uniform(0, 1, 3000).astype(np.float32))
    c = f32_to_bf16((rng.standard_normal(3000) * np.exp(rng.uniform(-20, 5, 3000))).astype(np.float32))
    fa, fb, fc = bf16_to_f32(a), bf16_to_f32(b), bf16_to_f32(c)
    exact = fa.astype(np.float64) * fb.astype(np.float64) + fc.astype(np.float64)
    ours = f64_to_bf16(exact)
    for i in range(len(a)):
        want = _exact_bf16(Fraction(float(fa[i])) * Fraction(float(fb[i])) + Fraction(float(fc[i])))
        assert int(ours[i]) == want, i


def test_fma_single_rounding_differs_from_double_rounding():
    """A case where fp32 fma followed by bf16 rounding (two roundings) is
    wrong and the single rounding is right: a + tiny just above a tie."""
    a = np.float32(1.0 + 2.0**-8)  # exactly half-way between two bf16 values
    tiny = np.float32(2.0**-30)
    exact = np.float64(a) * 1.0 + np.float64(tiny)
    assert f64_to_bf16(np.array([exact]))[0] == f32_to_bf16(np.array([np.float32(1.0 + 2.0**-7)]))[0]
    double_rounded = f32_to_bf16(np.array([np.float32(exact)]))[0]
    assert double_rounded == f32_to_bf16(np.array([np.float32(1.0)]))[0]


@pytest.mark.parametrize("value", [0.0, -0.0, 1.0, -2.5, 3.0e38, 1.0e-38])
def test_bf16_roundtrip_exact(value):
    bits = f32_to_bf16(np.array([value], np.float32))
    assert bf16_to_f32(bits)[0] == np.float32(value) or abs(value) > 1e38 or abs(value) < 1e-37


def test_e4m3_roundtrip_all_codes():
    codes = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], np.uint8)
    assert np.array_equal(f32_to_e4m3(e4m3_to_f32(codes)), codes)
