"""Pin the oracle's routing (kernels.py:360-383) and per-128 quantisation
(moe_input.py:24-27) against torch library routines, hand-built tie cases and
the reference validator's special inputs (CPU only)."""

import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle.numerics import bf16_to_f32, f32_to_bf16


def bf16_values(shape, rng, scale=1.0):
    return bf16_to_f32(f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32)))


def test_route_ids_match_topk_for_distinct_values():
    rng = np.random.default_rng(0)
    logits = bf16_values((512, 128), rng)
    distinct = np.array([len(np.unique(row)) == len(row) for row in logits])
    logits = logits[distinct]
    _, ids = om.route(logits)
    expected = torch.topk(torch.from_numpy(logits), 8, dim=-1).indices.numpy()
    assert np.array_equal(ids, expected)


def test_route_weights_match_torch_softmax():
    rng = np.random.default_rng(1)
    logits = bf16_values((256, 256), rng)
    weights, ids = om.route(logits)
    probs = torch.from_numpy(logits).double().softmax(-1)
    sel = torch.gather(probs, 1, torch.from_numpy(ids))
    expected = (sel / sel.sum(-1, keepdim=True)).float().to(torch.bfloat16)
    got = bf16_to_f32(weights)
    assert np.abs(got - expected.float().numpy()).max() <= 2.0**-9  # < one bf16 ulp at [0.0625,1)
    assert np.allclose(got.sum(-1), 1.0, atol=8 * 2.0**-8)


def test_route_tie_breaks_lower_expert_index():
    row = np.zeros((1, 16), np.float32)
    _, ids = om.route(row)
    assert ids[0].tolist() == list(range(8))
    row = np.full((1, 16), -1.0, np.float32)
    row[0, [3, 9, 12]] = 2.0
    row[0, [1, 4, 5, 10, 14, 15]] = 1.0  # 6 candidates for the last 5 places
    _, ids = om.route(row)
    assert ids[0].tolist() == [3, 9, 12, 1, 4, 5, 10, 14]


def test_route_positive_zero_outranks_negative_zero():
    # The ordered-bits key separates +0.0 and -0.0 (kernels.py:366-367).
    row = np.full((1, 16), -5.0, np.float32)
    row[0, 2] = -0.0
    row[0, 7] = 0.0
    _, ids = om.route(row)
    assert ids[0, 0] == 7 and ids[0, 1] == 2


def test_route_fp32_logits_rank_by_bf16_half_only():
    # Two fp32 values with the same upper 16 bits tie; the lower index wins
    # even though the other is larger in fp32.
    base = np.float32(1.5)
    bigger = (np.array([base]).view(np.uint32) | 0x7FFF).view(np.float32)[0]
    row = np.full((1, 16), -3.0, np.float32)
    row[0, 4] = bigger
    row[0, 2] = base
    weights, ids = om.route(row, out_dtype="f32")
    assert ids[0, 0] == 2 and ids[0, 1] == 4
    assert weights[0, 1] > weights[0, 0]  # weights still use the full fp32 values


def quant_torch(x: np.ndarray):
    """The same rule evaluated with torch ops (independent division and fp8 cast)."""
    t = torch.from_numpy(x.astype(np.float32)).view(len(x), -1, 128)
    scale = torch.maximum(t.abs().amax(-1), torch.tensor(1e-10, dtype=torch.float32)) / 448.0
    q = (t / scale[..., None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q.view(torch.uint8).reshape(len(x), -1).numpy(), scale.numpy()


@pytest.mark.parametrize("magnitude", [0.0, 1e-12, 1.0, 1000.0])
@pytest.mark.parametrize("rows", [12, 64])
def test_quantize_matches_torch_rule(magnitude, rows):
    """Mirrors validate_moe_input.py:27-36 (batches, magnitudes incl. zeros)."""
    rng = np.random.default_rng(rows)
    x = bf16_values((rows, 2048), rng, magnitude)
    q, scales = om.quantize_rows(x)
    tq, ts = quant_torch(x)
    assert np.array_equal(q, tq)
    assert np.array_equal(scales, ts)


def test_quantize_zero_rows_scale_floor():
    q, scales = om.quantize_rows(np.zeros((2, 256), np.float32))
    assert not q.any()
    assert np.all(scales == np.float32(np.float32(1e-10) / np.float32(448.0)))


def test_quantize_invariants():
    rng = np.random.default_rng(5)
    x = bf16_values((32, 1024), rng, 3.0)
    q, scales = om.quantize_rows(x)
    deq = om.dequantize_rows(q, scales)
    grouped = x.reshape(32, 8, 128)
    # the group maximum maps exactly onto +-448
    arg = np.abs(grouped).argmax(-1)
    codes = np.take_along_axis(q.reshape(32, 8, 128), arg[..., None], -1)[..., 0]
    assert np.all((codes & 0x7F) == 0x7E)
    # relative error bounded by half an e4m3 step (2^-4) plus subnormal floor
    err = np.abs(deq - x).reshape(32, 8, 128)
    bound = np.maximum(np.abs(grouped) * 2.0**-4, scales[..., None] * 2.0**-10)
    assert np.all(err <= bound * 1.0001)


def test_prepare_moe_input_layout_and_padding_router():
    rng = np.random.default_rng(6)
    x = bf16_values((6, 256), rng)
    router = bf16_values((6, 16), rng)
    slots = np.array([3, 40, 1, 33, 32, 0])
    q, scales_t, logits = om.prepare_moe_input(f32_to_bf16(x), router, slots, 32)
    q2, s2 = om.quantize_rows(x)
    assert np.array_equal(q, q2) and np.array_equal(scales_t, s2.T)
    padding = slots >= 32
    assert np.array_equal(logits[padding], np.repeat(router[:1], padding.sum(), 0))
    assert np.array_equal(logits[~padding], router[~padding])
