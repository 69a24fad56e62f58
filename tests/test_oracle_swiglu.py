"""Pin the oracle's SwiGLU + e4m3 requantisation (``swiglu_f32``,
``silu_mul_quant``; the Fish ``silu_mul_quant_kernel`` step the reference
calls at ``kernels.py:344,748``) against library routines and the values the
mathematics fixes, and bound the one reading of the reference it cannot
decide: whether ``silu(gate)`` is rounded to bf16 before ``* up``
(``kernels.py:392-394`` rounds it in the in-repo bf16 SwiGLU).  CPU only."""

import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle.numerics import bf16_to_f32, e4m3_to_f32, f32_to_bf16

F32_EPS = 2.0 ** -23


def bf16_rows(rng, shape, scale=1.0):
    return f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


def wide_gate_up(rng, rows=64, inter=256):
    """[gate | up] bf16 rows with gates spread over +-40 (both saturated
    tails of the sigmoid) and ordinary up values."""
    gate = rng.standard_normal((rows, inter)) * np.exp(rng.uniform(-4, 3.7, (rows, inter)))
    up = rng.standard_normal((rows, inter)) * 3.0
    return f32_to_bf16(np.concatenate([gate, up], axis=1).astype(np.float32))


def torch_halves(gate_up_bits):
    t = torch.from_numpy(bf16_to_f32(gate_up_bits))
    width = t.shape[-1] // 2
    return t[:, :width], t[:, width:]


def torch_quant(a: torch.Tensor):
    """The per-128 rule evaluated with torch ops and torch's own e4m3 cast:
    scale = max(amax, 1e-10) / 448 (fp32), q = e4m3(clamp(a / scale))."""
    groups = a.reshape(a.shape[0], -1, 128)
    amax = groups.abs().amax(dim=-1, keepdim=True)
    scale = torch.clamp(amax, min=1e-10) / 448.0
    q = torch.clamp(groups / scale, -448.0, 448.0).to(torch.float8_e4m3fn)
    return q.view(torch.uint8).reshape(a.shape).numpy(), scale[..., 0].numpy()


def test_swiglu_matches_torch_silu():
    """swiglu_f32 against torch's silu: within 2 fp32 ulps of the float64
    value and within 3 of torch's float32 silu * up."""
    rng = np.random.default_rng(20)
    gu = wide_gate_up(rng)
    got = om.swiglu_f32(gu).astype(np.float64)
    g, u = torch_halves(gu)
    exact = (torch.nn.functional.silu(g.double()) * u.double()).numpy()
    f32 = (torch.nn.functional.silu(g) * u).double().numpy()
    tiny = 1e-36  # below it, fp32 subnormals (and torch's underflow to 0) set the error
    assert np.all(np.abs(got - exact) <= 2 * F32_EPS * np.abs(exact) + tiny)
    assert np.all(np.abs(got - f32) <= 3 * F32_EPS * np.abs(f32) + tiny)


def test_silu_mul_quant_matches_torch_float8_rule():
    """The requantisation of the oracle's activations equals torch's e4m3
    cast byte for byte; starting from torch's own float32 silu, codes agree
    except where an activation sits within an ulp of a rounding boundary."""
    rng = np.random.default_rng(21)
    gu = wide_gate_up(rng, rows=96, inter=512)
    codes, scales = om.silu_mul_quant(gu)
    want_codes, want_scales = torch_quant(torch.from_numpy(om.swiglu_f32(gu)))
    assert np.array_equal(codes, want_codes)
    assert np.array_equal(scales, want_scales)
    g, u = torch_halves(gu)
    t_codes, t_scales = torch_quant(torch.nn.functional.silu(g) * u)
    assert np.mean(codes != t_codes) < 1e-3
    steps = np.abs(codes.astype(np.int32) - t_codes.astype(np.int32))
    assert np.all((codes == t_codes) | (steps == 1))
    assert np.allclose(scales, t_scales, rtol=4 * F32_EPS, atol=0)


def test_swiglu_special_values():
    inter = 128
    rng = np.random.default_rng(22)
    up = rng.standard_normal((4, inter)).astype(np.float32)
    # g = 0: silu(0) = 0, so the whole group is zero: codes 0, scale 1e-10 / 448
    gu = f32_to_bf16(np.concatenate([np.zeros((4, inter), np.float32), up], axis=1))
    assert np.all(om.swiglu_f32(gu) == 0.0)
    codes, scales = om.silu_mul_quant(gu)
    assert np.all(codes & 0x7F == 0)
    assert np.all(scales == np.float32(1e-10) / np.float32(448.0))
    # u = 0: zero activations whatever the gate
    gate = rng.standard_normal((4, inter)).astype(np.float32) * 5
    gu = f32_to_bf16(np.concatenate([gate, np.zeros((4, inter), np.float32)], axis=1))
    codes, scales = om.silu_mul_quant(gu)
    assert np.all(codes & 0x7F == 0) and np.all(scales == np.float32(1e-10) / np.float32(448.0))
    # large positive gate: sigmoid rounds to 1 in fp32, so a = g * u exactly
    big = np.full((4, inter), 96.0, np.float32)
    gu = f32_to_bf16(np.concatenate([big, up], axis=1))
    u_b = bf16_to_f32(gu[:, inter:])
    assert np.array_equal(om.swiglu_f32(gu), (np.float32(96.0) * u_b).astype(np.float32))
    # large negative gate: silu(g) = g / (1 + e^-g) in (g e^g, 0): |a| <= |g| e^g |u|
    # and a has the sign of -u
    neg = np.full((4, inter), -30.0, np.float32)
    gu = f32_to_bf16(np.concatenate([neg, up], axis=1))
    a = om.swiglu_f32(gu).astype(np.float64)
    u_b = bf16_to_f32(gu[:, inter:]).astype(np.float64)
    bound = 30.0 * np.exp(-30.0) * np.abs(u_b) * (1 + 4 * F32_EPS)
    assert np.all(np.abs(a) <= bound + 1e-45)
    assert np.all(np.sign(a) == -np.sign(u_b))


def test_swiglu_sign_symmetry_in_up():
    """a(g, -u) = -a(g, u): the codes differ in the sign bit only and the
    scales are equal."""
    rng = np.random.default_rng(23)
    gu = wide_gate_up(rng, rows=16, inter=256)
    flipped = gu.copy()
    flipped[:, 256:] ^= 0x8000
    c1, s1 = om.silu_mul_quant(gu)
    c2, s2 = om.silu_mul_quant(flipped)
    assert np.array_equal(s1, s2)
    nonzero = (c1 & 0x7F) != 0
    assert np.array_equal(c1[nonzero] ^ 0x80, c2[nonzero])
    assert np.all((c2[~nonzero] & 0x7F) == 0)


def test_planted_swapped_halves_is_detected():
    """A plausible bug, gate and up swapped, must fail the torch pin."""
    rng = np.random.default_rng(24)
    gu = wide_gate_up(rng, rows=8, inter=128)
    swapped = np.concatenate([gu[:, 128:], gu[:, :128]], axis=1)
    g, u = torch_halves(gu)
    exact = (torch.nn.functional.silu(g.double()) * u.double()).numpy()
    bad = om.swiglu_f32(swapped).astype(np.float64)
    assert not np.all(np.abs(bad - exact) <= 2 * F32_EPS * np.abs(exact) + 1e-40)
    codes, _ = om.silu_mul_quant(swapped)
    want, _ = torch_quant(torch.nn.functional.silu(g) * u)
    assert np.mean(codes != want) > 0.5


def test_silu_bf16_reading_differs_by_at_most_one_code():
    """The bf16-rounded silu reading moves an activation by at most half a
    bf16 ulp relative, so a requantised code by at most one step."""
    rng = np.random.default_rng(25)
    gu = wide_gate_up(rng, rows=64, inter=512)
    c32, s32 = om.silu_mul_quant(gu)
    c16, s16 = om.silu_mul_quant(gu, silu_bf16=True)
    assert np.allclose(s32, s16, rtol=2.0 ** -8, atol=0)
    value32 = e4m3_to_f32(c32) * np.repeat(s32, 128, axis=1)
    value16 = e4m3_to_f32(c16) * np.repeat(s16, 128, axis=1)
    amax = np.repeat(np.abs(value32).reshape(64, -1, 128).max(-1), 128, axis=1)
    # one e4m3 step is at most 1/8 of the value (normal range) or 2^-9 * 448 scale units
    assert np.all(np.abs(value32 - value16) <= np.abs(value32) / 8 + amax * 2.0 ** -9 / 448 * 2)


# The bf16-silu reading against the fp32 reading on each measured
# configuration's own inputs and weights, on a bounded row sample.  Measured
# RRMS 0.9e-3 - 1.33e-3 (c1 highest) with 0.16 - 0.31 % of activation codes
# one step apart: above the 1e-3 bound that holds this build's exact path to
# its own oracle, so the bound that faces the reference is the reference's
# own same-quantisation threshold, RRMS < 3e-3 (benchmark_native_moe.py:50),
# which this reading must clear with a factor of two to spare.
SAMPLE_ROWS = {1: 4, 2: 12, 3: 16, 4: 12, 5: 24}


@pytest.mark.parametrize("config", [1, 2, 3, 4, 5])
def test_silu_bf16_reading_within_stated_tolerance(config):
    from drama3_amd import workloads as wl

    from helpers import RRMS_REFERENCE, np_bf16, oracle_weights, rrms

    work = wl.CONFIGS[config]()
    step = work.steps[0]
    x, logits = step.packed()
    rows = SAMPLE_ROWS[config]
    pick = np.linspace(0, x.shape[0] - 1, rows).round().astype(np.int64)
    x_b = np_bf16(x)[pick]
    weights, ids = om.route(bf16_to_f32(np_bf16(logits)[pick]))
    wt = oracle_weights(work.experts)
    fp32 = om.expert_ffn(x_b, ids, weights, wt)
    rounded = om.expert_ffn(x_b, ids, weights, wt, silu_bf16=True)
    err = rrms(bf16_to_f32(rounded), bf16_to_f32(fp32))
    print(f"config {config}: RRMS(bf16 silu vs fp32 silu) = {err:.3e} over {rows} rows")
    assert err < RRMS_REFERENCE / 2
