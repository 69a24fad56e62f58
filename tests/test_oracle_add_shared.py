"""Pin ``om.add_shared`` (config 4's combine: ``bf16(routed + bf16(shared))``,
the reference's ``combine_experts`` with the gate at 1, ``kernels.py:433-439``)
by what the arithmetic fixes, not by a restatement of its formula:

* identities: a zero shared output returns the routed bytes, a zero routed
  output returns ``bf16(shared)``;
* exact sums: integer-valued operands whose sum bf16 holds exactly;
* rounding order: cases where skipping the shared output's own bf16 rounding
  (one rounding of the fp32 sum instead of two), rounding toward zero, or
  rounding ties away from zero would each give a different byte.
CPU only."""

import numpy as np

from oracle import moe as om
from oracle.numerics import bf16_to_f32, f32_to_bf16


def _bf16(values) -> np.ndarray:
    return f32_to_bf16(np.asarray(values, dtype=np.float32))


def test_zero_shared_returns_the_routed_bytes():
    rng = np.random.default_rng(3)
    routed = _bf16(rng.standard_normal(4096) * np.exp(rng.uniform(-20, 20, 4096)))
    got = om.add_shared(routed, np.zeros(4096, dtype=np.float32))
    # -0 + +0 is +0 in IEEE arithmetic; every other routed value comes back as it was
    negative_zero = routed == 0x8000
    assert np.array_equal(got[~negative_zero], routed[~negative_zero])
    assert np.all(got[negative_zero] == 0)


def test_zero_routed_returns_the_rounded_shared_output():
    rng = np.random.default_rng(4)
    shared = (rng.standard_normal(4096) * np.exp(rng.uniform(-20, 20, 4096))).astype(np.float32)
    got = om.add_shared(np.zeros(4096, dtype=np.uint16), shared)
    # bf16(shared) is shared with the low 16 bits rounded off (nearest, ties
    # to even): equal to it within half a bf16 ulp, and itself a bf16 value
    back = bf16_to_f32(got).astype(np.float64)
    ulp = np.exp2(np.floor(np.log2(np.abs(shared.astype(np.float64)))) - 7)
    assert np.all(np.abs(back - shared) <= ulp / 2)
    assert np.array_equal(f32_to_bf16(bf16_to_f32(got)), got)


def test_integer_sums_are_exact():
    rng = np.random.default_rng(5)
    a = rng.integers(-128, 128, 10000).astype(np.float32)
    b = rng.integers(-127, 128, 10000).astype(np.float32)
    got = bf16_to_f32(om.add_shared(_bf16(a), b))
    assert np.array_equal(got, a + b)  # |a + b| <= 255: every such integer is a bf16 value


def test_rounding_order_of_the_two_roundings():
    one = _bf16([1.0])
    # bf16 spacing at 1 is 2^-7.  shared = 2^-8 + 2^-20 rounds to 2^-8 on its
    # own; 1 + 2^-8 is then a tie that goes to the even neighbour 1.  One
    # rounding of the unrounded sum would give 1 + 2^-7.
    assert bf16_to_f32(om.add_shared(one, np.float32([2.0**-8 + 2.0**-20])))[0] == 1.0
    # 1 + 3 * 2^-8 lies halfway between 1 + 2^-7 (odd) and 1 + 2^-6 (even):
    # ties to even rounds up, truncation would round down.
    assert bf16_to_f32(om.add_shared(one, np.float32([3 * 2.0**-8])))[0] == 1.0 + 2.0**-6
    # 1 + 2^-8 + 2^-9 is above the halfway point: rounds up to 1 + 2^-7
    # (truncation would not).  shared = 2^-8 + 2^-9 is exactly a bf16 value.
    assert bf16_to_f32(om.add_shared(one, np.float32([2.0**-8 + 2.0**-9])))[0] == 1.0 + 2.0**-7
    # negative tie: -1 - 2^-8 goes to -1 (ties to even, not away from zero)
    assert bf16_to_f32(om.add_shared(_bf16([-1.0]), np.float32([-(2.0**-8)])))[0] == -1.0
