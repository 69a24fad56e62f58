"""Pin the oracle's combine / norm epilogues (kernels.py:386-556), ragged
packing (packed_prefill.py:51-78), slot compaction and the request-state
trace of scripts/validate_runtime_state.py:10-47 (CPU only)."""

import numpy as np
import torch

from oracle import moe as om
from oracle.numerics import bf16_to_f32, f32_to_bf16
from oracle.state import RequestState


def bf16(rng, shape, scale=1.0):
    return f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


def tb(bits):
    return torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16)


def bf16_neighbours(bits):
    """The bf16 values one ulp below and above each (finite, nonzero) value."""
    f = bf16_to_f32(bits).astype(np.float64)
    up = bf16_to_f32(np.where(f >= 0, bits + 1, bits - 1).astype(np.uint16)).astype(np.float64)
    down = bf16_to_f32(np.where(f > 0, bits - 1, bits + 1).astype(np.uint16)).astype(np.float64)
    return down, up


def test_combine_experts_is_the_nearest_bf16_of_the_exact_fma():
    """combine_experts (kernels.py:427-445 as compiled: one bf16 FMA,
    kernels.py:465-474) is the bf16 value nearest to shared * bf16(sigmoid(g))
    + routed, ties to even; the two-rounding reading of the source differs
    from it on some elements, so this test tells the two apart."""
    rng = np.random.default_rng(0)
    routed, shared, gate = bf16(rng, (64, 256)), bf16(rng, (64, 256)), bf16(rng, (64,))
    got = om.combine_experts(routed, shared, gate)
    g = torch.sigmoid(tb(gate).float()).to(torch.bfloat16).double()[:, None]
    exact = (tb(shared).double() * g + tb(routed).double()).numpy()  # exact in float64
    value = bf16_to_f32(got).astype(np.float64)
    down, up = bf16_neighbours(got)
    dist = np.abs(value - exact)
    assert np.all(dist <= np.abs(down - exact)) and np.all(dist <= np.abs(up - exact))
    tie = (dist == np.abs(down - exact)) | (dist == np.abs(up - exact))
    assert np.all((got[tie] & 1) == 0)
    weighted = (tb(shared).float() * g.float()).to(torch.bfloat16).float()
    twice = (tb(routed).float() + weighted).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    # (about a fifth of the elements differ by one ulp on N(0,1) data)
    assert np.mean(got == twice) > 0.5 and np.mean(got != twice) > 0.05


def test_combine_then_add_norm_equals_fused_combine_add_norm():
    rng = np.random.default_rng(5)
    routed, shared, gate = bf16(rng, (6, 512)), bf16(rng, (6, 512)), bf16(rng, (6,))
    residual, weight = bf16(rng, (6, 512)), bf16(rng, (512,), 0.1)
    combined = om.combine_experts(routed, shared, gate)
    out_a, res_a = om.add_norm(combined, residual, weight, 1e-6)
    out_b, res_b = om.combine_experts_add_norm(routed, shared, gate, residual, weight, 1e-6)
    assert np.array_equal(res_a, res_b) and np.array_equal(out_a, out_b)


def test_silu_mul_matches_torch():
    rng = np.random.default_rng(1)
    projected = bf16(rng, (5, 512), 3.0)
    got = om.silu_mul(projected)
    p = tb(projected).float()
    gate, up = p[:, :256].double(), p[:, 256:]
    act = (gate * torch.sigmoid(gate)).float().to(torch.bfloat16).float()
    want = (act * up).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


def test_combine_add_norm_residual_and_norm():
    rng = np.random.default_rng(2)
    rows, width = 4, 512
    routed, shared, gate = bf16(rng, (rows, width)), bf16(rng, (rows, width)), bf16(rng, (rows,))
    residual, weight = bf16(rng, (rows, width)), bf16(rng, (width,), 0.1)
    out, new_res = om.combine_experts_add_norm(routed, shared, gate, residual, weight, 1e-6)
    # residual: single-rounding FMA then a second bf16 rounding of the add
    g = om.sigmoid_bf16(bf16_to_f32(gate))[:, None].astype(np.float64)
    exact = bf16_to_f32(shared).astype(np.float64) * g + bf16_to_f32(routed)
    combined = bf16_to_f32(om.f64_to_bf16(exact))
    want_res = f32_to_bf16((combined + bf16_to_f32(residual)).astype(np.float32))
    assert np.array_equal(new_res, want_res)
    v = torch.from_numpy(bf16_to_f32(want_res)).double()
    ref = v * torch.rsqrt(v.square().mean(-1, keepdim=True) + 1e-6) * (1 + torch.from_numpy(bf16_to_f32(weight)).double())
    assert np.all(np.abs(bf16_to_f32(out) - ref.numpy()) <= np.abs(ref.numpy()) * 2.0**-8 + 1e-6)


def test_combine_add_norm_inverse_reads_source_rows():
    rng = np.random.default_rng(3)
    routed, shared, gate = bf16(rng, (3, 128)), bf16(rng, (3, 128)), bf16(rng, (3,))
    residual, weight = bf16(rng, (5, 128)), bf16(rng, (128,), 0.1)
    inverse = np.array([2, 0, 1, 1, 0])
    out, res = om.combine_experts_add_norm(routed, shared, gate, residual, weight, 1e-6, inverse)
    direct, dres = om.combine_experts_add_norm(routed[inverse], shared[inverse], gate[inverse],
                                               residual, weight, 1e-6)
    assert np.array_equal(out, direct) and np.array_equal(res, dres)


def test_add_norm_matches_torch():
    rng = np.random.default_rng(4)
    x, residual, weight = bf16(rng, (3, 256)), bf16(rng, (3, 256)), bf16(rng, (256,), 0.1)
    out, res = om.add_norm(x, residual, weight, 1e-6)
    want_res = (tb(x).float() + tb(residual).float()).to(torch.bfloat16)
    assert np.array_equal(res, want_res.view(torch.int16).numpy().view(np.uint16))


def test_row_metadata_matches_validator_expectations():
    """validate_packed_layers.py:116-136: positions restart per sequence,
    row slots are the sequence's slot and labels are the next prompt row."""
    lengths = [5, 3, 7]
    cu = np.concatenate([[0], np.cumsum(lengths)])
    slots = np.array([9, 4, 30])
    frames = np.arange(sum(lengths) * 11).reshape(-1, 11) + 1000
    pos, row_slots, labels = om.row_metadata(cu, slots, sum(lengths), frames, eos=7)
    assert pos.tolist() == [i for n in lengths for i in range(n)]
    assert row_slots.tolist() == [s for s, n in zip(slots, lengths) for _ in range(n)]
    offset = 0
    for n in lengths:
        assert np.array_equal(labels[offset:offset + n - 1], frames[offset + 1:offset + n])
        assert labels[offset + n - 1].tolist() == [7] + [0] * 10
        offset += n


def test_row_metadata_rows_beyond_last_boundary():
    # Rows past the last boundary belong to the last sequence (packed_prefill.py:63-66).
    cu = np.array([0, 2, 4])
    pos, row_slots, _ = om.row_metadata(cu, np.array([1, 2]), 6)
    assert pos.tolist() == [0, 1, 0, 1, 2, 3] and row_slots.tolist() == [1, 1, 2, 2, 2, 2]


def test_compact_slots_closed_form():
    rng = np.random.default_rng(5)
    occ = (rng.uniform(size=64) < 0.75).astype(np.uint8)
    active, n = om.compact_slots(occ)
    assert n == occ.sum() and np.all(np.diff(active) > 0) and np.all(occ[active] == 1)
    assert om.compact_slots(np.zeros(64, np.uint8))[1] == 0


def test_request_state_known_answer_trace():
    """Restates scripts/validate_runtime_state.py:10-47 on the CPU oracle."""
    state = RequestState(8, eos=999, max_length=512, max_frames=8)
    slots = np.array([5, 1, 3])
    histories = np.arange(48).reshape(3, 16)
    for row, slot in enumerate(slots):
        state.initialize(slot, np.arange(11), histories[row], 30 + row, row + 2)
    expected = [[], [], []]
    for step in range(6):
        output = np.arange(33).reshape(3, 11) + 100 * (step + 1)
        output[1, 0] = 999 if step >= 1 else 123
        state.save(slots, output)
        for row in range(3):
            if len(expected[row]) < row + 2 and not (row == 1 and step >= 1):
                expected[row].append(output[row].copy())
        last, history, positions = state.load(slots)
        for row, values in enumerate(expected):
            assert np.array_equal(last[row], values[-1])
            assert positions[row] == 30 + row + len(values)
            target = np.concatenate([histories[row], np.stack(values)[:, 0]])[-16:]
            assert np.array_equal(history[row], target)
    state.initialize(5, last[0], histories[0], 50, 1)
    fresh = np.arange(11)[None] + 500
    state.save(slots[:1], fresh)
    assert np.array_equal(state.codes[5, 0], fresh[0, 1:])
    assert state.metadata[5].tolist() == [51, 1, 1, 1]


def test_mixed_rows_order():
    kind, owner, cu = om.mixed_rows([3, 9], [2, 3])
    assert kind.tolist() == [0, 0, 1, 1, 1, 1, 1]
    assert owner.tolist() == [3, 9, 0, 0, 1, 1, 1]
    assert cu.tolist() == [0, 2, 5]
