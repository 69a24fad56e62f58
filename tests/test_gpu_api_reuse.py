"""Eager reference-API calls reuse one workspace per (shape, options,
device, stream) and return fresh outputs; ``prepare_experts`` with
``keep_reference=False`` keeps only the fragment-major codes and gives the
same bytes as the two-layout object (decode, prefill-sized batch)."""

import torch
import pytest

pytestmark = pytest.mark.gpu


def test_native_moe_reuses_its_workspace_per_stream(device):
    from drama3_amd import kernels, workloads
    from drama3_amd.kernels import native_moe, route

    w = workloads.config1()
    x, logits = w.steps[0].packed()
    experts = w.experts.to(device)
    xd = x.to(device)
    weights, ids = route(logits.to(device))
    kernels._workspaces.clear()
    a = native_moe(xd, ids, weights, experts, block_m=64)
    b = native_moe(xd, ids, weights, experts, block_m=64)
    assert len(kernels._workspaces) == 1
    assert a.data_ptr() != b.data_ptr()
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        c = native_moe(xd, ids, weights, experts, block_m=64)
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize()
    assert len(kernels._workspaces) == 2  # another stream, another workspace
    assert torch.equal(a, b) and torch.equal(a, c)


@pytest.mark.parametrize("config", [2, 4])
def test_fragment_only_experts_match_two_layouts(device, config):
    from drama3_amd import workloads
    from drama3_amd.expert_weights import LAYOUT_FRAGMENT, fc1_operands, fc2_operands, prepare_experts
    from drama3_amd.kernels import routed_moe

    w = workloads.CONFIGS[config]()
    x, logits = w.steps[0].packed()
    rows = min(len(x), 1024)
    xd, ld = x[:rows].to(device), logits[:rows].to(device)
    both = prepare_experts(w.experts.to(device))
    single = prepare_experts(w.experts.to(device), keep_reference=False)
    w13 = single.w13_weight
    prepare_experts(single)  # a second call keeps the single copy as it is
    assert single.w13_weight is w13
    assert fc1_operands(single)[2] == LAYOUT_FRAGMENT and fc2_operands(single)[2] == LAYOUT_FRAGMENT
    assert torch.equal(single.w13_weight, both.d3_w13_packed)
    assert torch.equal(single.w2_weight, both.d3_w2_packed)
    got = routed_moe(xd, ld, single, True)
    want = routed_moe(xd, ld, both, True)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_routed_moe_small_batch_without_sort_matches_sorted(device):
    """routed_moe at 560 rows over 16 experts takes the grouped GEMMs that
    find their own routes (no sort); the output equals the sorted chain's."""
    from drama3_amd import kernels, workloads
    from drama3_amd.kernels import routed_moe
    from drama3_amd.pipeline import MoEWorkspace, Shape

    w = workloads.config5()
    x, logits = w.steps[0].packed()
    rows = 560
    xd, ld = x[:rows].to(device), logits[:rows].to(device)
    experts = w.experts.to(device)
    kernels._workspaces.clear()
    got = routed_moe(xd, ld, experts, True)
    ws = next(iter(kernels._workspaces.values()))
    assert ws.by_pair and ws.grouped
    sorted_ws = MoEWorkspace(Shape(rows, w.num_experts, w.hidden, w.intermediate), device,
                             item_rows=128)
    assert sorted_ws.grouped and not sorted_ws.by_pair
    want = sorted_ws.forward(xd, ld, experts, out=torch.empty_like(got))
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_routed_moe_graphs_of_one_shape_replay_in_any_order(device):
    """Two graphs that capture routed_moe at the same shape (a by-pair
    workspace, whose live row count is a device constant written when the
    workspace is built): under capture each gets a workspace of its own, none
    is cached, and the second graph replayed before the first gives the eager
    result."""
    from drama3_amd import kernels, workloads
    from drama3_amd.kernels import routed_moe

    w = workloads.config5()
    x, logits = w.steps[0].packed()
    rows = 560
    xd, ld = x[:rows].to(device), logits[:rows].to(device)
    experts = w.experts.to(device)
    kernels._workspaces.clear()
    want = routed_moe(xd, ld, experts, True).clone()
    kernels._workspaces.clear()
    torch.cuda.synchronize()
    graphs, outs = [], []
    for _ in range(2):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            outs.append(routed_moe(xd, ld, experts, True))
        graphs.append(g)
    assert len(kernels._workspaces) == 0  # nothing built under capture is cached
    for order in ((1, 0), (0, 1), (1, 1)):
        for k in order:
            outs[k].zero_()
            torch.cuda.synchronize()
            graphs[k].replay()
            torch.cuda.synchronize()
            assert torch.equal(outs[k].view(torch.int16), want.view(torch.int16)), f"graph {k}"
