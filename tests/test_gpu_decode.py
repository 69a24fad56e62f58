"""Sortless decode expert GEMMs (d3_decode_expert_gemm) and the three-launch
step that starts from the slots (d3_decode_route_fc1 + FC2 +
d3_decode_route_combine).  Every expert-GEMM workgroup finds its expert's
routes itself and rows are indexed by pair (the three-launch step's down
rows by slot pair, slot * top_k + rank).  All results are bit-identical to
the sorted chain's for the same pairs: ids, routing weights, the slot list,
gate_up (mapped through the sorted layout), down (mapped through the slot
list) and the combined output."""

import numpy as np
import pytest
import torch

from helpers import CONTRACTION, EXACT, assert_bf16_close, np_bf16, np_f32, oracle_weights
from oracle import moe as om

pytestmark = pytest.mark.gpu


def steps_for(w, device, experts, slots=64):
    """(frontless, sortless after the front, sorted chain) decode steps."""
    from drama3_amd.pipeline import DecodeStep

    args = (slots, w.num_experts, w.hidden, w.intermediate)
    frontless = DecodeStep(*args, device=device, sortless=True)
    front = DecodeStep(*args, device=device, sortless=True, frontless=False)
    sorted_chain = DecodeStep(*args, device=device, sortless=False)
    assert frontless.uses_sortless(experts) and front.uses_sortless(experts)
    assert not sorted_chain.uses_sortless(experts)
    return frontless, front, sorted_chain


def pair_rows(down, active, n, top_k):
    """Down rows stored by slot pair (the three-launch step), in pair order:
    row r's rank-k route is slot active[r]'s."""
    slots = active[:n].long()
    index = (slots[:, None] * top_k + torch.arange(top_k, device=down.device)).reshape(-1)
    return down[index]


def compare(sortless, chain, by_slot=False):
    n = int(chain.count.item())
    assert int(sortless.count.item()) == n
    assert torch.equal(sortless.active, chain.active)
    a, b = sortless.workspace, chain.workspace
    pairs = n * a.shape.top_k
    assert torch.equal(a.ids[:n], b.ids[:n])
    assert torch.equal(a.weights[:n].view(torch.int16 if a.weights.dtype == torch.bfloat16 else torch.int32),
                       b.weights[:n].view(torch.int16 if b.weights.dtype == torch.bfloat16 else torch.int32))
    down = pair_rows(a.down, sortless.active, n, a.shape.top_k) if by_slot else a.down[:pairs]
    assert torch.equal(down.view(torch.int32), b.down[:pairs].view(torch.int32))
    # chain gate_up row at sorted position p holds pair sorted_ids[p]
    total = int(b.total.item())
    order = b.sorted_ids[:total].cpu().numpy()
    positions = np.flatnonzero(order < pairs)
    chain_rows = np_bf16(b.gate_up)[positions]
    sortless_rows = np_bf16(a.gate_up)[order[positions]]
    assert np.array_equal(sortless_rows, chain_rows)
    assert torch.equal(a.out[:n].view(torch.int16), b.out[:n].view(torch.int16))
    return n


def run_all(steps, occ, xs, ls, experts):
    for ds in steps:
        ds(occ, xs, ls, experts)
    torch.cuda.synchronize()
    frontless, front, chain = steps
    assert frontless.uses_frontless(occ, xs, ls) and not front.uses_frontless(occ, xs, ls)
    n = compare(frontless, chain, by_slot=True)
    assert compare(front, chain) == n
    return n


@pytest.mark.parametrize("config", [1, 2, 3])
def test_sortless_matches_sorted_chain(device, config):
    from drama3_amd import workloads
    from drama3_amd.expert_weights import prepare_experts

    w = workloads.CONFIGS[config]()
    step = w.steps[0]
    experts = prepare_experts(w.experts.to(device))
    steps = steps_for(w, device, experts)
    occ = step.occupancy.to(device)
    xs, ls = step.x_slots.to(device), step.logits_slots.to(device)
    for launch in range(2):  # the second launch overwrites the first's buffers
        n = run_all(steps, occ, xs, ls, experts)
        print(f"config {config} launch {launch}: rows {n}", flush=True)


@pytest.mark.parametrize("pattern", ["none", "last", "all", "alternate"])
def test_sortless_occupancies(device, pattern):
    from drama3_amd import workloads
    from drama3_amd.expert_weights import prepare_experts

    w = workloads.config2()
    step = w.steps[0]
    experts = prepare_experts(w.experts.to(device))
    steps = steps_for(w, device, experts)
    occupancy = np.zeros(64, np.uint8)
    if pattern == "last":
        occupancy[63] = 1
    elif pattern == "all":
        occupancy[:] = 1
    elif pattern == "alternate":
        occupancy[1::2] = 1
    occ = torch.from_numpy(occupancy).to(device)
    xs, ls = step.x_slots.to(device), step.logits_slots.to(device)
    print(f"pattern {pattern}", flush=True)
    assert run_all(steps, occ, xs, ls, experts) == int(occupancy.sum())


@pytest.mark.parametrize("logits_dtype", [torch.bfloat16, torch.float32])
def test_frontless_ties_and_logit_dtypes(device, logits_dtype):
    """Logits on a coarse grid (many exact ties: the lower expert ranks
    first), in bf16 and f32, plus rows with +-inf and a zero x row."""
    from drama3_amd import workloads
    from drama3_amd.expert_weights import prepare_experts

    w = workloads.config1()
    experts = prepare_experts(w.experts.to(device))
    steps = steps_for(w, device, experts)
    gen = torch.Generator("cpu").manual_seed(11)
    logits = torch.randint(-2, 3, (64, w.num_experts), generator=gen).float() * 0.5
    logits[5, 3] = float("inf")
    logits[9, :] = 0.0
    logits[12, 7] = float("-inf")
    occupancy = (torch.rand(64, generator=gen) < 0.6).to(torch.uint8)
    occupancy[[5, 9, 12]] = 1
    xs = w.steps[0].x_slots.clone()
    xs[9] = 0.0
    ls = logits.to(logits_dtype).to(device)
    n = run_all(steps, occupancy.to(device), xs.to(device), ls, experts)
    print(f"{logits_dtype}: rows {n}", flush=True)
    frontless = steps[0]
    active, _ = om.compact_slots(occupancy.numpy())
    weights, ids = om.route(np_f32(ls)[active])
    assert np.array_equal(frontless.workspace.ids.cpu().numpy()[:n], ids)


def test_frontless_more_slots_and_odd_experts(device):
    """200 slots (four ranking passes, one weight tile per workgroup) and
    E = 20 (partial logit chunks)."""
    from drama3_amd.expert_weights import prepare_experts
    from drama3_amd.workloads import Workload, make_experts

    gen = torch.Generator("cpu").manual_seed(21)
    e, h, i, slots = 20, 1024, 256, 200
    experts_cpu = make_experts(gen, e, h, i)
    w = Workload("odd", 21, h, e, i, experts_cpu, [])
    experts = prepare_experts(experts_cpu.to(device))
    steps = steps_for(w, device, experts, slots=slots)
    occupancy = (torch.rand(slots, generator=gen) < 0.7).to(torch.uint8)
    occupancy[[0, 63, 64, 127, 128, 199]] = 1
    xs = torch.randn((slots, h), generator=gen).to(torch.bfloat16).to(device)
    ls = torch.randn((slots, e), generator=gen).to(torch.bfloat16)
    # rows 8 apart: 16-byte aligned rows of a wider buffer (a strided view)
    wide = torch.zeros((slots, 24), dtype=torch.bfloat16)
    wide[:, :e] = ls
    ls_dev = wide.to(device)[:, :e]
    n = run_all(steps, occupancy.to(device), xs, ls_dev, experts)
    assert n == int(occupancy.sum())
    active, _ = om.compact_slots(occupancy.numpy())
    weights, ids = om.route(np_f32(ls)[active])
    expected = om.expert_ffn(np_bf16(xs.cpu())[active], ids, weights, oracle_weights(experts_cpu))
    stats = assert_bf16_close(np_bf16(steps[0].workspace.out)[:n], expected, **EXACT)
    print(f"slots {slots}, E {e}: rows {n} {stats}", flush=True)


def test_sortless_matches_oracle_and_replays(device):
    """c3 shapes (16 experts, ~32 routes each: several route tiles per
    expert) captured once and replayed with changing occupancy."""
    from drama3_amd import workloads
    from drama3_amd.expert_weights import prepare_experts
    from drama3_amd.pipeline import DecodeStep

    w = workloads.config3()
    step = w.steps[0]
    experts = prepare_experts(w.experts.to(device))
    wt = oracle_weights(w.experts)
    ds = DecodeStep(64, w.num_experts, w.hidden, w.intermediate, device=device, sortless=True)
    occ = step.occupancy.to(device)
    xs, ls = step.x_slots.to(device), step.logits_slots.to(device)
    assert ds.uses_frontless(occ, xs, ls)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ds(occ, xs, ls, experts)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ds(occ, xs, ls, experts)
    rng = np.random.default_rng(7)
    for replay, p in enumerate([1.0, 0.3, 0.8, 0.0]):
        occupancy = (rng.uniform(size=64) < p).astype(np.uint8)
        occ.copy_(torch.from_numpy(occupancy))
        graph.replay()
        torch.cuda.synchronize()
        _ = torch.ones(1024, device=device).sum().item()  # eager work between replays
        active, n = om.compact_slots(occupancy)
        assert int(ds.count.item()) == n
        assert np.array_equal(ds.active.cpu().numpy()[:n], active)
        assert np.all(ds.active.cpu().numpy()[n:] == -1)
        if n == 0:
            continue
        weights, ids = om.route(np_f32(step.logits_slots)[active])
        assert np.array_equal(ds.workspace.ids.cpu().numpy()[:n], ids)
        expected = om.expert_ffn(np_bf16(step.x_slots)[active], ids, weights, wt)
        stats = assert_bf16_close(np_bf16(out)[:n], expected, **EXACT)
        print(f"replay {replay}: rows {n} {stats}", flush=True)


def test_real_drama3_shape_eight_tiles_per_workgroup(device):
    """The reference model's own MoE shape (H2048, 256 experts, I512; 64 live
    slots): 16 weight tiles per expert, eight per workgroup in both GEMMs;
    bit-identical to the sorted chain and within tolerance of the oracle."""
    from drama3_amd.expert_weights import prepare_experts
    from drama3_amd.workloads import Workload, make_experts

    gen = torch.Generator("cpu").manual_seed(41)
    e, h, i = 256, 2048, 512
    experts_cpu = make_experts(gen, e, h, i)
    w = Workload("real", 41, h, e, i, experts_cpu, [])
    experts = prepare_experts(experts_cpu.to(device))
    steps = steps_for(w, device, experts)
    occupancy = torch.ones(64, dtype=torch.uint8)
    occupancy[[5, 30]] = 0
    xs = torch.randn((64, h), generator=gen).to(torch.bfloat16).to(device)
    ls = torch.randn((64, e), generator=gen).to(torch.bfloat16)
    n = run_all(steps, occupancy.to(device), xs, ls.to(device), experts)
    active, _ = om.compact_slots(occupancy.numpy())
    weights, ids = om.route(np_f32(ls)[active])
    expected = om.expert_ffn(np_bf16(xs.cpu())[active], ids, weights, oracle_weights(experts_cpu))
    stats = assert_bf16_close(np_bf16(steps[0].workspace.out)[:n], expected, **EXACT)
    print(f"E 256 I 512: rows {n} {stats}", flush=True)


@pytest.mark.parametrize("slots,live", [(256, 256), (256, 200), (64, 17), (128, 33)])
def test_route_slices_of_hot_experts(device, slots, live):
    """Few experts (E16) and routing skewed so that the hottest experts take
    a route from nearly every live slot: the one-tile-per-workgroup GEMMs
    split each expert's route tiles over several workgroups (route slices;
    at 256 slots an expert's 16 route tiles are taken four per slice), and
    slices beyond the live rows exit early.  The frontless and front-started
    sortless steps agree bit for bit; with at most 64 routes per expert
    (the exact path everywhere) both equal the sorted chain bit for bit;
    all are within tolerance of the oracle (the FP8 contraction tolerance
    once an expert takes more than 64 routes)."""
    from drama3_amd.expert_weights import prepare_experts
    from drama3_amd.workloads import Workload, make_experts

    gen = torch.Generator("cpu").manual_seed(slots + live)
    e, h, i = 16, 1024, 256
    experts_cpu = make_experts(gen, e, h, i)
    w = Workload("hot", 0, h, e, i, experts_cpu, [])
    experts = prepare_experts(experts_cpu.to(device))
    steps = steps_for(w, device, experts, slots=slots)
    occupancy = torch.zeros(slots, dtype=torch.uint8)
    occupancy[torch.randperm(slots, generator=gen)[:live]] = 1
    xs = torch.randn((slots, h), generator=gen).to(torch.bfloat16)
    bias = torch.zeros(e)
    bias[[3, 7, 11, 12]] = 4.0  # four experts in (nearly) every row's top 8
    ls = (torch.randn((slots, e), generator=gen) + bias).to(torch.bfloat16)
    active, n = om.compact_slots(occupancy.numpy())
    weights, ids = om.route(np_f32(ls)[active])
    counts = np.bincount(ids.ravel(), minlength=e)
    assert counts.max() > 16  # a hot expert spans several route tiles
    occ_d, xs_d, ls_d = occupancy.to(device), xs.to(device), ls.to(device)
    for ds in steps:
        ds(occ_d, xs_d, ls_d, experts)
    torch.cuda.synchronize()
    frontless, front, chain = steps
    assert frontless.uses_frontless(occ_d, xs_d, ls_d)
    a, b = frontless.workspace, front.workspace
    assert int(frontless.count.item()) == n and torch.equal(frontless.active, chain.active)
    assert torch.equal(a.ids[:n], b.ids[:n]) and torch.equal(a.ids[:n], chain.workspace.ids[:n])
    assert torch.equal(pair_rows(a.down, frontless.active, n, 8).view(torch.int32),
                       b.down[:8 * n].view(torch.int32))
    assert torch.equal(a.out[:n].view(torch.int16), b.out[:n].view(torch.int16))
    if counts.max() <= 64:
        assert compare(frontless, chain, by_slot=True) == n
    expected = om.expert_ffn(np_bf16(xs)[active], ids, weights, oracle_weights(experts_cpu))
    tolerance = EXACT if counts.max() <= 64 else CONTRACTION
    stats = assert_bf16_close(np_bf16(a.out)[:n], expected, **tolerance)
    print(f"slots {slots} live {n}: routes per expert {counts.tolist()} {stats}", flush=True)


def test_standalone_entries_match_the_step(device):
    """d3_decode_route_fc1, d3_decode_expert_gemm mode 2 and
    d3_decode_route_combine called one by one: with row_slots = the slot
    list, FC2's down rows (by slot pair) and the combined rows equal
    d3_decode_step's byte for byte; without it, FC2 stores the same rows by
    pair (row * top_k + rank).  Config 2 with a quarter of the slots free."""
    from drama3_amd import workloads
    from drama3_amd.expert_weights import prepare_experts
    from drama3_amd.pipeline import DecodeStep

    w = workloads.config2()
    step = w.steps[0]
    experts = prepare_experts(w.experts.to(device))
    occ = step.occupancy.to(device)
    xs, ls = step.x_slots.to(device), step.logits_slots.to(device)
    whole = DecodeStep(64, w.num_experts, w.hidden, w.intermediate, device=device)
    parts = DecodeStep(64, w.num_experts, w.hidden, w.intermediate, device=device)
    assert whole.uses_frontless(occ, xs, ls)
    out_whole = whole(occ, xs, ls, experts).clone()
    ws = parts.workspace
    ws.decode_route_fc1(experts, occ, xs, ls, parts.active, parts.count)
    ws.decode_fc2(experts, parts.count, row_slots=parts.active)
    out_parts = ws.decode_route_combine(occ, ls).clone()
    torch.cuda.synchronize()
    n = int(whole.count.item())
    assert int(parts.count.item()) == n and torch.equal(parts.active, whole.active)
    slots = whole.active[:n].long()
    by_slot = (slots[:, None] * 8 + torch.arange(8, device=device)).reshape(-1)
    assert torch.equal(ws.down[by_slot].view(torch.int32), whole.workspace.down[by_slot].view(torch.int32))
    assert torch.equal(out_parts[:n].view(torch.int16), out_whole[:n].view(torch.int16))
    # the same FC2 without the slot list: rows by pair
    ws.decode_fc2(experts, parts.count)
    torch.cuda.synchronize()
    assert torch.equal(ws.down[:8 * n].view(torch.int32), whole.workspace.down[by_slot].view(torch.int32))
