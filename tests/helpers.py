"""Shared helpers of the parity tests: tensor <-> oracle conversions and the
stated tolerances."""

from __future__ import annotations

import numpy as np
import torch

from oracle import moe as om
from oracle.numerics import bf16_to_f32

# Tolerances of the bf16 expert outputs against the exact-arithmetic oracle.
#
# Every element is held to  |gpu - oracle| <= ulps * ulp(oracle) + floor * RMS(row)
# except a bounded fraction of outliers, which must still stay below
# GROSS * RMS(row).  The outliers are inherent to the reference's pipeline:
# the SwiGLU activation is requantised to e4m3 per 128 columns, so a one-ulp
# bf16 difference in an FC1 output can move a group's max (its scale) or an
# activation across an e4m3 rounding boundary; the activation then moves by
# one e4m3 step (6-12 %), and with a large W2 block scale that shows up as a
# visible error in that block's output columns.  The reference accepts this
# by comparing implementations with RRMS thresholds only.
#
# Exact path (work items with <= EXACT_ROUTES routes: every decode config):
# bf16 MFMAs on exactly widened FP8 operands, fp32-accurate sums; it differs
# from the oracle only by fp32 summation order.  RRMS < 1e-3.
#
# FP8 contraction path (larger items: prefill and mixed batches): FP8 MFMAs
# round the aligned products at ~1e-4 of sum|products| per instruction, as
# FP8 tensor-core GEMMs do.  RRMS < 0.003, the reference's own threshold for
# same-quantisation implementations (scripts/benchmark_native_moe.py:50,
# tune_prefill_moe.py:89).
RRMS_REFERENCE = 3e-3
RRMS_TIGHT = 1e-3
OUTLIER_FRACTION = 1e-4
GROSS = 0.5
EXACT = dict(ulps=2, row_floor=2.0 ** -6, rrms_max=RRMS_TIGHT)
CONTRACTION = dict(ulps=4, row_floor=2.0 ** -3, rrms_max=RRMS_REFERENCE)


def np_bf16(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def np_u8(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.uint8).cpu().numpy()


def np_f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def oracle_weights(experts) -> om.ExpertWeights:
    return om.ExpertWeights(np_u8(experts.w13_weight), np_f32(experts.w13_scale_inv),
                            np_u8(experts.w2_weight), np_f32(experts.w2_scale_inv))


def rrms(actual: np.ndarray, expected: np.ndarray) -> float:
    a = actual.astype(np.float64)
    e = expected.astype(np.float64)
    return float(np.sqrt(np.mean((a - e) ** 2) / max(np.mean(e ** 2), 1e-30)))


def bf16_ulp(values: np.ndarray) -> np.ndarray:
    """Spacing of bf16 numbers at each value (normal range)."""
    mag = np.maximum(np.abs(values.astype(np.float64)), 2.0 ** -126)
    return np.exp2(np.floor(np.log2(mag)) - 7)


def assert_bf16_close(actual_bits: np.ndarray, expected_bits: np.ndarray, ulps: int = 2,
                      row_floor: float = 2.0 ** -6, rrms_max: float = RRMS_TIGHT,
                      outlier_fraction: float = OUTLIER_FRACTION, gross: float = GROSS) -> dict:
    a = bf16_to_f32(actual_bits).astype(np.float64)
    e = bf16_to_f32(expected_bits).astype(np.float64)
    err = rrms(a, e)
    assert err < rrms_max, f"RRMS {err:.3g} >= {rrms_max}"
    row_rms = np.sqrt(np.mean(e ** 2, axis=-1, keepdims=True))
    diff = np.abs(a - e)
    ulp = bf16_ulp(e) * ulps
    bad = diff > ulp + row_floor * row_rms
    assert bad.mean() <= outlier_fraction, (
        f"{int(bad.sum())} of {bad.size} elements outside tolerance; worst {diff.max()}")
    worst = float((diff / (row_rms + 1e-30)).max())
    assert np.all(diff <= ulp + gross * row_rms), f"gross error {worst:.3g} x row RMS"
    return {"rrms": err, "max_abs": float(diff.max()), "max_over_row_rms": worst,
            "outliers": int(bad.sum()), "exact_fraction": float(np.mean(actual_bits == expected_bits))}
