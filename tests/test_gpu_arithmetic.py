"""The arithmetic shortcuts of the quantisers and the SwiGLU requantisation
against their IEEE forms on the device (d3_check_epilogue_arithmetic):
hardware bf16 rounding over every non-NaN fp32 pattern, the Newton-corrected
hardware reciprocal over every d in [2^-43, 2^126), the division by 448 of
the group scale over every non-negative amax, the sigmoid over every
non-NaN g (within ulps of the float64 sigmoid), and the
residual-corrected division over every |v| up to the group maximum for
group scales max(amax, 1e-10) / 448 across the exponent range (the
all-ones significand, the 1e-10 floor and scale 1 included)."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

CHUNK = 1 << 28


def _run(device, kind, first, last, scale=1.0):
    from drama3_amd import _lib

    result = torch.tensor([0, -1], dtype=torch.int32, device=device)  # {count, first bad}
    for start in range(first, last, CHUNK):
        _lib.call("d3_check_epilogue_arithmetic", kind, start, min(CHUNK, last - start), scale,
                  result.data_ptr(), _lib.stream(device))
    torch.cuda.synchronize()
    count, first_bad = (int(v) & 0xffffffff for v in result.cpu().tolist())
    return count, first_bad


def test_hardware_bf16_rounding_every_pattern(device):
    count, first_bad = _run(device, 0, 0, 1 << 32)
    assert count == 0, f"{count} mismatches, first at {first_bad:#010x}"


def test_newton_reciprocal_every_input(device):
    """[2^-43, 2^126): the sigmoid's denominators 1 + exp(-g) from 1 on, and
    every finite group scale, from RN(1e-10 / 448) (about 2^-42) up to
    FLT_MAX / 448 (about 2^119)."""
    count, first_bad = _run(device, 1, 0x2A000000, 0x7E800000)
    assert count == 0, f"{count} mismatches, first at d = {first_bad:#010x}"


def test_group_scale_every_amax(device):
    """group_scale(m) = max(m, 1e-10) / 448 through a constant reciprocal and
    one residual correction, for every non-negative fp32 m up to +inf."""
    count, first_bad = _run(device, 4, 0, 0x7F800001)
    assert count == 0, f"{count} mismatches, first at m = {first_bad:#010x}"


def test_sigmoid_every_bf16_input_within_two_ulps(device):
    """Every sigmoid input of the SwiGLU is a bf16 value: over all 2^16 of
    them the fp32 sigmoid is within two ulps of the float64 one (the error
    distribution of the library expf with the same reciprocal), and below
    2^-125 where the true sigmoid is subnormal."""
    count, first_bad = _run(device, 5, 0, 1 << 16, scale=2.0)
    assert count == 0, f"{count} mismatches, first at g = {first_bad << 16:#010x}"
    # the bound is tight: about one bf16 input in a thousand is two ulps off
    count, _ = _run(device, 5, 0, 1 << 16, scale=1.0)
    assert 0 < count < 200


def test_sigmoid_every_fp32_input_within_three_ulps(device):
    count, first_bad = _run(device, 3, 0, 1 << 32, scale=3.0)
    assert count == 0, f"{count} mismatches, first at g = {first_bad:#010x}"


def _group_scales():
    rng = np.random.default_rng(41)
    amax = [448.0, 1.0, np.float32(1.0) - np.float32(2.0 ** -24), 1e-10, 3e-11, 65504.0]
    amax += list(rng.integers(0x2E000000, 0x47000000, 18, dtype=np.uint32).view(np.float32))
    out = []
    for a in amax:
        a = np.float32(a)
        scale = np.maximum(a, np.float32(1e-10)) / np.float32(448.0)  # IEEE float32
        out.append((float(a), float(scale)))
    return out


@pytest.mark.parametrize("amax,scale", _group_scales())
def test_residual_division_every_value_up_to_amax(device, amax, scale):
    last = int(np.float32(amax).view(np.uint32)) + 1
    count, first_bad = _run(device, 2, 0, last, scale)
    assert count == 0, f"{count} mismatches, first at v = {first_bad:#010x} (scale {scale!r})"
