"""Mixed decode + prefill steps on the device (d3_mixed_rows, MixedStep).

The row layout (active slots, decode slots with reserved padding, prefix
ownership, MoE rows and read-back map) is compared bit for bit with the
oracle's restatement of mixed_graph.py:139-179 / row_reuse.py:46-109; the
captured mixed step's routed rows are held to the FP8 contraction tolerance
of the oracle's expert FFN on the kept rows, and its residual + RMSNorm
combine back onto every row is held to one bf16 ulp of the oracle's given
those routed rows (the combine kernel's own bar: fp32 sum of squares and
rsqrt against the oracle's float64)."""

import numpy as np
import pytest
import torch

from helpers import CONTRACTION, assert_bf16_close, np_bf16, np_f32, oracle_weights
from oracle import moe as om

pytestmark = pytest.mark.gpu

CODES = 11


def prompts_with_prefixes(rng, lengths, share, codes=CODES):
    """Prompt frames where prompt i copies a leading run of an earlier prompt
    with probability ``share`` (then diverges at one random code)."""
    prompts = []
    for n in lengths:
        p = rng.integers(0, 4, (n, codes)).astype(np.int64)
        if prompts and rng.random() < share:
            src = prompts[int(rng.integers(0, len(prompts)))]
            run = int(rng.integers(0, min(n, len(src)) + 1))
            p[:run] = src[:run]
            if run < min(n, len(src)):
                p[run] = src[run]
                p[run, int(rng.integers(0, codes))] += 1 + int(rng.integers(0, 3))
        prompts.append(p)
    return prompts


def layout_inputs(rng, slots, live, lengths, capacity, share=0.8, codes=CODES):
    occupancy = np.zeros(slots, dtype=np.uint8)
    occupancy[rng.permutation(slots)[:live]] = 1
    prompts = prompts_with_prefixes(rng, lengths, share, codes)
    total = sum(lengths)
    frames = rng.integers(0, 4, (capacity, codes)).astype(np.int64)
    if total:
        frames[:total] = np.concatenate(prompts)
    boundaries = np.concatenate([[0], np.cumsum(lengths), [capacity]]).astype(np.int32)
    return occupancy, frames, boundaries


def run_layout(device, occupancy, decode_rows, padding_start, boundaries, prompts, capacity,
               frames):
    """The layout, and the suffix's row metadata from the same launch
    (checked against the oracle's row_metadata here)."""
    from drama3_amd.mixed import MixedRows

    rows = MixedRows(len(occupancy), decode_rows, capacity, padding_start, device)
    f = None if frames is None else torch.from_numpy(frames).to(device)
    sequences = len(boundaries) - 1
    seq_slots = np.arange(sequences, dtype=np.int64) + 7
    positions = torch.full((max(capacity, 1),), -5, dtype=torch.int64, device=device)
    row_slots = torch.full_like(positions, -5)
    rows(torch.from_numpy(occupancy).to(device), torch.from_numpy(boundaries).to(device),
         prompts, f, None, torch.from_numpy(seq_slots).to(device), positions, row_slots)
    torch.cuda.synchronize()
    want_pos, want_slots, _ = om.row_metadata(boundaries, seq_slots, capacity)
    assert np.array_equal(positions.cpu().numpy()[:capacity], want_pos)
    assert np.array_equal(row_slots.cpu().numpy()[:capacity], want_slots)
    return rows


def assert_layout(rows, expected, decode_rows):
    assert int(rows.count.item()) == expected.count
    assert np.array_equal(rows.active.cpu().numpy(), expected.active)
    if decode_rows:
        assert np.array_equal(rows.decode_slots.cpu().numpy()[:decode_rows], expected.decode_slots)
    assert int(rows.keep_count.item()) == expected.keep_count
    assert np.array_equal(rows.keep.cpu().numpy(), expected.keep)
    assert np.array_equal(rows.inverse.cpu().numpy(), expected.inverse)


@pytest.mark.parametrize("case", [
    # slots, live, decode_rows, prompt lengths, capacity, reuse
    (64, 48, 64, [256, 256], 640, True),
    (64, 48, 64, [256, 256], 640, False),
    (64, 64, 48, [100, 37, 100, 3], 300, True),       # more live slots than decode rows
    (64, 0, 16, [40, 40, 40], 128, True),             # no decode rows live
    (64, 10, 64, [], 256, True),                      # no prompts
    (3000, 1700, 1024, [500, 0, 500, 0, 480], 2048, True),  # multi-chunk compaction, empty prompts
    (256, 200, 256, [450] * 16, 7936, True),          # 16 prompts, 8192 rows
    (64, 33, 64, [300, 300, 300], 1024, False),
])
def test_layout_matches_oracle(device, case):
    slots, live, d, lengths, capacity, reuse = case
    rng = np.random.default_rng(slots + live + d + capacity)
    occupancy, frames, boundaries = layout_inputs(rng, slots, live, lengths, capacity)
    prompts = len(lengths)
    rows = run_layout(device, occupancy, d, slots // 2, boundaries, prompts, capacity,
                      frames if reuse else None)
    expected = om.mixed_layout(occupancy, d, slots // 2, boundaries, prompts, capacity,
                               frames if reuse and prompts >= 2 else None)
    assert_layout(rows, expected, d)


@pytest.mark.parametrize("codes", [1, 3, 16, 20])
def test_layout_frame_widths(device, codes):
    """Frame rows of 1 and 3 codes (fewer than the four threads of a
    comparison), 16 (the widest compared from registers) and 20 (compared
    by a loop over the codes)."""
    rng = np.random.default_rng(codes)
    lengths = [120, 60, 120, 90]
    occupancy, frames, boundaries = layout_inputs(rng, 64, 40, lengths, 400, share=1.0,
                                                  codes=codes)
    rows = run_layout(device, occupancy, 64, 32, boundaries, len(lengths), 400, frames)
    expected = om.mixed_layout(occupancy, 64, 32, boundaries, len(lengths), 400, frames,
                               codes=codes)
    assert_layout(rows, expected, 64)
    assert int(rows.keep_count.item()) < 40 + sum(lengths)  # some prefix was reused


def test_layout_clamps_bad_boundaries(device):
    """Decreasing or out-of-range boundaries read no frame outside the suffix;
    the layout equals the oracle's on the clamped boundaries."""
    rng = np.random.default_rng(7)
    occupancy = np.ones(64, dtype=np.uint8)
    frames = rng.integers(0, 2, (200, CODES)).astype(np.int64)
    frames[100:150] = frames[:50]
    boundaries = np.array([0, 100, 90, 150, 5000], dtype=np.int32)
    rows = run_layout(device, occupancy, 64, 32, boundaries, 3, 200, frames)
    clamped = np.array([0, 100, 100, 150, 200], dtype=np.int32)
    expected = om.mixed_layout(occupancy, 64, 32, clamped, 3, 200, frames)
    assert_layout(rows, expected, 64)


def stage_step(step, rng, experts_shape, occupancy, lengths, sequence_slots, share):
    """Write one step's inputs into the MixedStep staging buffers; returns
    the host copies the oracle needs."""
    e, h = experts_shape
    full, capacity = step.rows.full, step.rows.capacity
    prompts = prompts_with_prefixes(rng, lengths, share)
    frames = rng.integers(0, 4, (capacity, CODES)).astype(np.int64)
    frames[:sum(lengths)] = np.concatenate(prompts)
    boundaries = np.concatenate([[0], np.cumsum(lengths), [capacity]]).astype(np.int32)
    x = torch.randn((full, h), generator=rng_torch(rng)).to(torch.bfloat16)
    logits = torch.randn((full, e), generator=rng_torch(rng)).to(torch.bfloat16)
    residual = torch.randn((full, h), generator=rng_torch(rng)).to(torch.bfloat16)
    shared = (0.5 * torch.randn((full, h), generator=rng_torch(rng))).to(torch.bfloat16)
    gate = torch.randn(full, generator=rng_torch(rng)).to(torch.bfloat16)
    host = dict(occupancy=occupancy, frames=frames, boundaries=boundaries, x=x, logits=logits,
                residual=residual, shared=shared, gate=gate)
    load_step(step, host, sequence_slots)
    return host


def load_step(step, host, sequence_slots):
    step.occupancy.copy_(torch.from_numpy(host["occupancy"]))
    step.frames.copy_(torch.from_numpy(host["frames"]))
    step.boundaries.copy_(torch.from_numpy(host["boundaries"]))
    step.sequence_slots.copy_(torch.tensor(sequence_slots, dtype=torch.int64))
    for name in ("x", "logits", "residual", "shared", "gate"):
        getattr(step, name).copy_(host[name])


def rng_torch(rng):
    return torch.Generator("cpu").manual_seed(int(rng.integers(0, 2 ** 31)))


@pytest.mark.parametrize("reuse", [True, False])
def test_mixed_step_graph_replays(device, reuse):
    """Config-5 shape: 48 live decode slots of 64 (decode bucket 64, reserved
    padding from slot 32 on), two 256-row prompts with shared prefixes in a
    640-row suffix.  One capture; four replays with 4 slots retired and 4
    admitted between them and eager work in between; each replay equals an
    eager run bit for bit, its fused routed + residual combine equals the
    two-launch chain bit for bit, and it matches the oracle (layout exact,
    routed rows within the FP8 contraction tolerance, combine within one ulp
    on those rows)."""
    from drama3_amd import workloads
    from drama3_amd.kernels import combine_experts_add_norm_inverse
    from drama3_amd.mixed import MixedStep

    w = workloads.config5()
    experts = w.experts.to(device)
    wt = oracle_weights(w.experts)
    slots, d, capacity, padding_start = 64, 64, 640, 32
    sequence_slots = [40, 41, 63]
    step = MixedStep(slots, d, capacity, padding_start, 3, w.num_experts, w.hidden,
                     w.intermediate, device=device, reuse=reuse)
    rng = np.random.default_rng(11)
    norm = torch.randn(w.hidden, generator=rng_torch(rng)).to(torch.bfloat16)
    step.norm_weight.copy_(norm)
    first = w.steps[0].occupancy.numpy().astype(np.uint8)
    stage_step(step, rng, (w.num_experts, w.hidden), first, [256, 256], sequence_slots, 1.0)
    step.capture(experts)
    for index, ws in enumerate(w.steps):
        occupancy = ws.occupancy.numpy().astype(np.uint8)
        host = stage_step(step, rng, (w.num_experts, w.hidden), occupancy, [256, 256],
                          sequence_slots, 1.0 if index % 2 == 0 else 0.5)
        scratch = torch.randn(1000, 1000, device=device).sum()  # eager work between replays
        out = step.replay().clone()
        torch.cuda.synchronize()
        residual = step.residual.clone()
        keep = step.rows.keep.cpu().numpy()
        keep_count = int(step.rows.keep_count.item())
        inverse = step.rows.inverse.cpu().numpy()
        # the fused routed + residual combine equals the two-launch chain bit
        # for bit (d3_weighted_combine, then d3_combine_experts_add_norm)
        routed = step.workspace.combine(None, step.rows.keep_count, None, step.routed).clone()
        res2 = host["residual"].to(device)
        out2 = combine_experts_add_norm_inverse(routed, step.shared, step.gate, step.rows.inverse,
                                                res2, step.norm_weight, step.epsilon)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), out2.view(torch.int16))
        assert torch.equal(residual.view(torch.int16), res2.view(torch.int16))
        # the layout
        expected = om.mixed_layout(occupancy, d, padding_start, host["boundaries"], 2, capacity,
                                   host["frames"] if reuse else None)
        assert_layout(step.rows, expected, d)
        positions, row_slots, _ = om.row_metadata(host["boundaries"], sequence_slots, capacity)
        assert np.array_equal(step.positions.cpu().numpy(), positions)
        assert np.array_equal(step.row_slots.cpu().numpy(), row_slots)
        # the routed rows on the kept rows
        rows = keep[:keep_count]
        x_kept = np_bf16(host["x"])[rows]
        weights, ids = om.route(np_f32(host["logits"])[rows])
        want = om.expert_ffn(x_kept, ids, weights, wt)
        stats = assert_bf16_close(np_bf16(routed)[:keep_count], want, **CONTRACTION)
        # the combine back onto every row, given the routed rows
        want_out, want_res = om.combine_experts_add_norm(
            np_bf16(routed), np_bf16(host["shared"]), np_bf16(host["gate"]),
            np_bf16(host["residual"]), np_bf16(norm), step.epsilon, inverse)
        assert_bf16_close(np_bf16(residual), want_res, ulps=1, row_floor=0.0)
        assert_bf16_close(np_bf16(out), want_out, ulps=1, row_floor=0.0)
        # eager run on the same inputs
        load_step(step, host, sequence_slots)
        eager = step.forward(experts).clone()
        torch.cuda.synchronize()
        assert np.array_equal(np_bf16(eager), np_bf16(out))
        assert float(scratch) == float(scratch)
        print(f"mixed step {index}: kept {keep_count} of {expected.count + 512} live rows {stats}")
