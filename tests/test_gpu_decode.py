"""Sortless decode expert GEMMs (d3_decode_expert_gemm): every expert-GEMM
workgroup finds its expert's routes itself, rows are indexed by pair.  The
results are bit-identical to the sorted chain's for the same pairs: gate_up
(mapped through the sorted layout), down and the combined output."""

import numpy as np
import pytest
import torch

from helpers import EXACT, assert_bf16_close, np_bf16, np_f32, oracle_weights
from oracle import moe as om

pytestmark = pytest.mark.gpu


def steps_for(w, device, experts):
    from drama3_amd.pipeline import DecodeStep

    sortless = DecodeStep(64, w.num_experts, w.hidden, w.intermediate, device=device,
                          sortless=True)
    sorted_chain = DecodeStep(64, w.num_experts, w.hidden, w.intermediate, device=device,
                              sortless=False)
    assert sortless.uses_sortless(experts) and not sorted_chain.uses_sortless(experts)
    return sortless, sorted_chain


def compare(sortless, chain):
    n = int(chain.count.item())
    assert int(sortless.count.item()) == n
    assert torch.equal(sortless.active, chain.active)
    a, b = sortless.workspace, chain.workspace
    pairs = n * a.shape.top_k
    assert torch.equal(a.ids[:n], b.ids[:n])
    assert torch.equal(a.down[:pairs].view(torch.int32), b.down[:pairs].view(torch.int32))
    # chain gate_up row at sorted position p holds pair sorted_ids[p]
    total = int(b.total.item())
    order = b.sorted_ids[:total].cpu().numpy()
    positions = np.flatnonzero(order < pairs)
    chain_rows = np_bf16(b.gate_up)[positions]
    sortless_rows = np_bf16(a.gate_up)[order[positions]]
    assert np.array_equal(sortless_rows, chain_rows)
    assert torch.equal(a.out[:n], b.out[:n])
    return n


@pytest.mark.parametrize("config", [1, 2, 3])
def test_sortless_matches_sorted_chain(device, config):
    from drama3_amd import workloads
    from drama3_amd.expert_weights import prepare_experts

    w = workloads.CONFIGS[config]()
    step = w.steps[0]
    experts = prepare_experts(w.experts.to(device))
    sortless, chain = steps_for(w, device, experts)
    occ = step.occupancy.to(device)
    xs, ls = step.x_slots.to(device), step.logits_slots.to(device)
    for launch in range(2):
        sortless(occ, xs, ls, experts)
        chain(occ, xs, ls, experts)
        torch.cuda.synchronize()
        n = compare(sortless, chain)
        print(f"config {config} launch {launch}: rows {n}", flush=True)


@pytest.mark.parametrize("pattern", ["none", "last", "all", "alternate"])
def test_sortless_occupancies(device, pattern):
    from drama3_amd import workloads
    from drama3_amd.expert_weights import prepare_experts

    w = workloads.config2()
    step = w.steps[0]
    experts = prepare_experts(w.experts.to(device))
    sortless, chain = steps_for(w, device, experts)
    occupancy = np.zeros(64, np.uint8)
    if pattern == "last":
        occupancy[63] = 1
    elif pattern == "all":
        occupancy[:] = 1
    elif pattern == "alternate":
        occupancy[1::2] = 1
    occ = torch.from_numpy(occupancy).to(device)
    xs, ls = step.x_slots.to(device), step.logits_slots.to(device)
    sortless(occ, xs, ls, experts)
    chain(occ, xs, ls, experts)
    torch.cuda.synchronize()
    assert compare(sortless, chain) == int(occupancy.sum())


def test_sortless_matches_oracle_and_replays(device):
    """c1 shapes (16 experts, ~32 routes each: several route tiles per
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
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ds(occ, xs, ls, experts)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ds(occ, xs, ls, experts)
    rng = np.random.default_rng(7)
    for replay, p in enumerate([1.0, 0.3, 0.8]):
        occupancy = (rng.uniform(size=64) < p).astype(np.uint8)
        occ.copy_(torch.from_numpy(occupancy))
        graph.replay()
        torch.cuda.synchronize()
        active, n = om.compact_slots(occupancy)
        assert int(ds.count.item()) == n
        weights, ids = om.route(np_f32(step.logits_slots)[active])
        expected = om.expert_ffn(np_bf16(step.x_slots)[active], ids, weights, wt)
        stats = assert_bf16_close(np_bf16(out)[:n], expected, **EXACT)
        print(f"replay {replay}: rows {n} {stats}", flush=True)


def test_decode_gemm_contract(device):
    from drama3_amd import _lib

    with pytest.raises(ValueError, match="mode"):
        _lib.call("d3_decode_expert_gemm", 1, 16, 16, 4, 512, 1024, 16, None, 64, 8, 16, 16, 64,
                  16, None, None)
    with pytest.raises(ValueError, match="capacity"):
        _lib.call("d3_decode_expert_gemm", 0, 16, 16, 4, 512, 1024, 16, None, 300, 8, 16, 16, 64,
                  16, None, None)
    with pytest.raises(ValueError, match="K=768"):
        _lib.call("d3_decode_expert_gemm", 0, 16, 16, 4, 512, 768, 16, None, 64, 8, 16, 16, 64,
                  16, None, None)
