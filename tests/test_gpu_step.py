"""The one-launch decode step (d3_moe_decode_step): every buffer it writes is
bit-identical to the multi-kernel chain's on the same inputs (front, sort,
FC1, SwiGLU requant, FC2, combine), its hand-off counters are back at zero
after each launch, and its output matches the oracle."""

import numpy as np
import pytest
import torch

from helpers import EXACT, assert_bf16_close, np_bf16, np_f32, np_u8, oracle_weights
from oracle import moe as om

pytestmark = pytest.mark.gpu


def make_steps(w, device):
    from drama3_amd.expert_weights import prepare_experts
    from drama3_amd.pipeline import DecodeStep

    experts = prepare_experts(w.experts.to(device))
    fused = DecodeStep(64, w.num_experts, w.hidden, w.intermediate, device=device, fused=True)
    chain = DecodeStep(64, w.num_experts, w.hidden, w.intermediate, device=device, fused=False,
                       sortless=False)
    chain.workspace.swiglu_in_fc2 = False  # the chain writes act / act_scales too
    return experts, fused, chain


def snapshot(ds):
    """Every buffer of the step, restricted to the entries a step defines."""
    ws = ds.workspace
    n = int(ds.count.item())
    pairs = n * ws.shape.top_k
    total = int(om.max_sorted_rows(pairs, ws.shape.num_experts, ws.tile))
    sorted_ids = ws.sorted_ids.cpu().numpy()
    valid = np.flatnonzero(sorted_ids[:total] < pairs)
    return {
        "count": n,
        "active": ds.active.cpu().numpy(),
        "ids": ws.ids.cpu().numpy()[:n],
        "weights": np_bf16(ws.weights)[:n],
        "q": np_u8(ws.q)[:n],
        "x_scales": np_f32(ws.x_scales)[:n],
        "sorted_ids": sorted_ids[valid],
        "positions": valid,
        "gate_up": np_bf16(ws.gate_up)[valid],
        "act": np_u8(ws.act)[valid],
        "act_scales": np_f32(ws.act_scales)[valid],
        "down": np_f32(ws.down)[:pairs].view(np.uint32),
        "out": np_bf16(ws.out)[:n],
    }


def assert_same(fused, chain):
    for key in chain:
        assert np.array_equal(np.asarray(fused[key]), np.asarray(chain[key])), key


def assert_sync_clear(ds):
    assert not ds.wait_failed()
    assert int(ds.sync.abs().sum()) == 0, "hand-off counters not reset"


@pytest.mark.parametrize("config", [1, 2, 3])
def test_fused_step_matches_chain_bit_for_bit(device, config):
    from drama3_amd import workloads

    w = workloads.CONFIGS[config]()
    step = w.steps[0]
    experts, fused, chain = make_steps(w, device)
    occ = step.occupancy.to(device)
    xs, ls = step.x_slots.to(device), step.logits_slots.to(device)
    assert fused.uses_fused(ls, experts) and not chain.uses_fused(ls, experts)
    for launch in range(2):  # the second launch runs on the counters the first left
        fused(occ, xs, ls, experts)
        chain(occ, xs, ls, experts)
        torch.cuda.synchronize()
        print(f"config {config} launch {launch}: rows {int(fused.count.item())}", flush=True)
        assert_same(snapshot(fused), snapshot(chain))
        assert_sync_clear(fused)


@pytest.mark.parametrize("pattern", ["none", "last", "all", "alternate", "first_half"])
def test_fused_step_occupancies(device, pattern):
    from drama3_amd import workloads

    w = workloads.config1()
    step = w.steps[0]
    experts, fused, chain = make_steps(w, device)
    occupancy = np.zeros(64, np.uint8)
    if pattern == "last":
        occupancy[63] = 1
    elif pattern == "all":
        occupancy[:] = 1
    elif pattern == "alternate":
        occupancy[::2] = 1
    elif pattern == "first_half":
        occupancy[:32] = 1
    occ = torch.from_numpy(occupancy).to(device)
    xs, ls = step.x_slots.to(device), step.logits_slots.to(device)
    fused(occ, xs, ls, experts)
    chain(occ, xs, ls, experts)
    torch.cuda.synchronize()
    got, want = snapshot(fused), snapshot(chain)
    assert got["count"] == int(occupancy.sum())
    assert_same(got, want)
    assert_sync_clear(fused)


def test_fused_step_matches_oracle_c2(device):
    from drama3_amd import workloads

    w = workloads.config2()
    step = w.steps[0]
    experts, fused, _ = make_steps(w, device)
    out = fused(step.occupancy.to(device), step.x_slots.to(device), step.logits_slots.to(device),
                experts)
    torch.cuda.synchronize()
    assert_sync_clear(fused)
    active, n = om.compact_slots(step.occupancy.numpy())
    assert int(fused.count.item()) == n
    assert np.array_equal(fused.active.cpu().numpy()[:n], active)
    weights, ids = om.route(np_f32(step.logits_slots)[active])
    assert np.array_equal(fused.workspace.ids.cpu().numpy()[:n], ids)
    expected = om.expert_ffn(np_bf16(step.x_slots)[active], ids, weights, oracle_weights(w.experts))
    stats = assert_bf16_close(np_bf16(out)[:n], expected, **EXACT)
    print(f"fused c2: rows {n} {stats}")


def test_fused_step_graph_replays(device):
    """One capture, replayed with a different occupancy each time and eager
    work in between: every replay equals a fresh eager chain run."""
    from drama3_amd import workloads
    from drama3_amd.pipeline import DecodeStep

    w = workloads.config2()
    step = w.steps[0]
    experts, fused, _ = make_steps(w, device)
    occ = step.occupancy.to(device)
    xs, ls = step.x_slots.to(device), step.logits_slots.to(device)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fused(occ, xs, ls, experts)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fused(occ, xs, ls, experts)
    chain = DecodeStep(64, w.num_experts, w.hidden, w.intermediate, device=device, fused=False,
                       sortless=False)
    rng = np.random.default_rng(1)
    for replay, p in enumerate([0.1, 0.5, 0.9, 1.0, 0.0]):
        occupancy = (rng.uniform(size=64) < p).astype(np.uint8)
        occ.copy_(torch.from_numpy(occupancy))
        graph.replay()
        torch.cuda.synchronize()
        got = np_bf16(out).copy()
        n = int(fused.count.item())
        _ = torch.ones(1024, device=device).sum().item()  # eager work between replays
        want = chain(occ, xs, ls, experts)
        torch.cuda.synchronize()
        print(f"replay {replay}: rows {n}", flush=True)
        assert n == int(occupancy.sum())
        assert np.array_equal(got[:n], np_bf16(want)[:n])
        assert_sync_clear(fused)


def test_fused_step_contract(device):
    from drama3_amd.pipeline import DecodeStep

    with pytest.raises(ValueError, match="one-launch step"):
        DecodeStep(64, 16, 1024, 384, device=device, fused=True)
    lib_ints = DecodeStep(64, 16, 1024, 256, device=device).sync.numel()
    assert lib_ints == 4 + 4 * 16 + 64 * 4
