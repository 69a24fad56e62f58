"""Tiled grouped FP8 GEMMs (d3_grouped_fc1_swiglu, d3_grouped_fc2) against
the chain they replace on contraction-sized work items: d3_expert_gemm on its
FP8 path (exact_routes 0) followed by d3_silu_mul_quant, and d3_expert_gemm
FC2.  Same MFMA per K block and the same rescale order, so the fp8 codes and
scales of the activations and the fp32 down rows must be identical, byte for
byte, for both weight layouts; end-to-end parity with the CPU oracle is in
test_gpu_moe (configs 4 and 5 run these kernels)."""

import numpy as np
import pytest
import torch

from helpers import CONTRACTION, assert_bf16_close, np_bf16, np_f32, oracle_weights
from oracle import moe as om

pytestmark = pytest.mark.gpu


def _workload(rows, experts, hidden, intermediate, seed):
    from drama3_amd import workloads

    gen = torch.Generator("cpu").manual_seed(seed)
    w = workloads.make_experts(gen, experts, hidden, intermediate)
    x = workloads._bf16(gen, (rows, hidden))
    logits = workloads._bf16(gen, (rows, experts))
    return w, x, logits


def _live_positions(ws):
    total = int(ws.total.item())
    pairs = int(ws.pairs_dev.item())
    sorted_ids = ws.sorted_ids[:total]
    return torch.nonzero(sorted_ids < pairs).flatten()


@pytest.mark.parametrize("item_rows", [64, 128])
@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("shape", [(3668, 128, 2048, 768), (560, 16, 1024, 256)],
                         ids=["c4_shapes", "c5_shapes"])
def test_grouped_matches_fp8_chain(device, shape, packed, item_rows):
    """Items of up to 64 routes leave half of every tile empty; 128 fill it."""
    from drama3_amd.expert_weights import prepare_experts
    from drama3_amd.pipeline import MoEWorkspace, Shape

    rows, e, h, i = shape
    w, x, logits = _workload(rows, e, h, i, seed=11)
    experts = w.to(device)
    if packed:
        prepare_experts(experts)
    ws = MoEWorkspace(Shape(rows, e, h, i), device, item_rows=item_rows, grouped=True)
    assert ws.grouped and ws.item_rows == item_rows
    ws.front(x.to(device), logits.to(device))
    live = _live_positions(ws)
    print(f"rows {rows} E {e} H {h} I {i} packed {packed} item_rows {item_rows}: "
          f"{live.numel()} routes, "
          f"{int(ws.num_items.item())} items", flush=True)

    ws.exact_routes = 0  # every item on the FP8 path of d3_expert_gemm
    ws.fc1(experts)
    ws.activation()
    ws.fc2(experts)
    torch.cuda.synchronize()
    act_ref = ws.act[live].clone()
    scales_ref = ws.act_scales[live].clone()
    down_ref = ws.down.clone()

    ws.act.zero_()
    ws.act_scales.zero_()
    ws.down.zero_()
    ws.grouped_fc1(experts)
    torch.cuda.synchronize()
    assert torch.equal(ws.act[live], act_ref), "activation codes differ"
    assert torch.equal(ws.act_scales[live].view(torch.int32), scales_ref.view(torch.int32))
    ws.grouped_fc2(experts)
    torch.cuda.synchronize()
    assert torch.equal(ws.down.view(torch.int32), down_ref.view(torch.int32)), "down rows differ"


@pytest.mark.parametrize("shape", [(300, 8, 512, 512), (260, 8, 1536, 256), (400, 16, 256, 1536)],
                         ids=["h512_i512", "h1536_i256", "h256_i1536"])
def test_grouped_other_contraction_lengths(device, shape):
    """K of 256 ... 2048 on both GEMMs (FC1 K = H, FC2 K = I), fragment-major
    weights, against the FP8 chain byte for byte."""
    from drama3_amd.expert_weights import prepare_experts
    from drama3_amd.pipeline import MoEWorkspace, Shape

    rows, e, h, i = shape
    w, x, logits = _workload(rows, e, h, i, seed=17)
    experts = prepare_experts(w.to(device))
    ws = MoEWorkspace(Shape(rows, e, h, i), device, item_rows=128, grouped=True)
    ws.front(x.to(device), logits.to(device))
    live = _live_positions(ws)
    ws.exact_routes = 0
    ws.fc1(experts)
    ws.activation()
    ws.fc2(experts)
    torch.cuda.synchronize()
    act_ref, scales_ref, down_ref = ws.act[live].clone(), ws.act_scales[live].clone(), ws.down.clone()
    ws.grouped_fc1(experts)
    ws.grouped_fc2(experts)
    torch.cuda.synchronize()
    assert torch.equal(ws.act[live], act_ref)
    assert torch.equal(ws.act_scales[live].view(torch.int32), scales_ref.view(torch.int32))
    pairs = ws.shape.pairs
    assert torch.equal(ws.down[:pairs].view(torch.int32), down_ref[:pairs].view(torch.int32))


def test_grouped_dense_expert_matches_fp8_chain(device):
    """The shared expert (identity routes, top_k 1) through both chains."""
    from drama3_amd.pipeline import DenseExpert, MoEWorkspace, Shape

    rows, h, i = 1000, 2048, 768
    w, x, logits = _workload(rows, 1, h, i, seed=12)
    shared = w.to(device)
    ws = MoEWorkspace(Shape(rows, 1, h, i), device)
    ws.quantize(x.to(device))
    old = DenseExpert(rows, h, i, device, exact_routes=0, grouped=False)
    new = DenseExpert(rows, h, i, device)
    assert new.grouped
    ref = old.forward(ws.q, ws.x_scales, shared).clone()
    got = new.forward(ws.q, ws.x_scales, shared)
    torch.cuda.synchronize()
    assert torch.equal(old.act, new.act) and torch.equal(old.act_scales, new.act_scales)
    assert torch.equal(got.view(torch.int32), ref.view(torch.int32))


def test_grouped_partial_items_and_oracle(device):
    """Ragged items (an expert with 1 route, items of 1..128 routes) end to
    end against the CPU oracle."""
    from drama3_amd.pipeline import MoEWorkspace, Shape

    rows, e, h, i = 300, 16, 1024, 256
    w, x, logits = _workload(rows, e, h, i, seed=13)
    # one dominant expert and one expert reached by a single route
    logits = logits.float()
    logits[:, 3] += 6.0
    logits[:, 9] -= 20.0
    logits[0, 9] = 40.0
    logits = logits.to(torch.bfloat16)
    experts = w.to(device)
    ws = MoEWorkspace(Shape(rows, e, h, i), device)
    assert ws.grouped
    out = ws.forward(x.to(device), logits.to(device), experts)
    torch.cuda.synchronize()
    counts = ws.counts.cpu().numpy()
    assert counts[9] == 1 and counts[3] == rows
    weights, ids = om.route(np_f32(logits))
    expected = om.expert_ffn(np_bf16(x), ids, weights, oracle_weights(w))
    stats = assert_bf16_close(np_bf16(out), expected, **CONTRACTION)
    print(f"ragged items: {stats}")


def test_shared_expert_on_side_stream_and_folded_graph_replays(device):
    """moe_with_shared with the shared expert on a side stream (the
    reference's moe_parts layout) and folded into the routed launches both
    equal the sequential chain bit for bit, eagerly and over repeated graph
    replays with eager work in between."""
    from drama3_amd import workloads
    from drama3_amd.pipeline import DenseExpert, MoEWorkspace, Shape, moe_with_shared

    rows, e, h, i = 1500, 64, 1024, 512
    gen = torch.Generator("cpu").manual_seed(31)
    w = workloads.make_experts(gen, e, h, i)
    sw = workloads.make_experts(gen, 1, h, i)
    x = workloads._bf16(gen, (rows, h)).to(device)
    logits = workloads._bf16(gen, (rows, e)).to(device)
    experts, shared = w.to(device), sw.to(device)
    ws = MoEWorkspace(Shape(rows, e, h, i), device)
    dense = DenseExpert(rows, h, i, device)
    assert ws.grouped and dense.grouped
    expected = moe_with_shared(ws, dense, x, logits, experts, shared).clone()
    side = torch.cuda.Stream(device)
    got = moe_with_shared(ws, dense, x, logits, experts, shared, side=side)
    torch.cuda.synchronize()
    assert torch.equal(got, expected)

    g = torch.cuda.CUDAGraph()
    warm = torch.cuda.Stream(device)
    warm.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(warm):
        moe_with_shared(ws, dense, x, logits, experts, shared, side=side)
    torch.cuda.current_stream().wait_stream(warm)
    with torch.cuda.graph(g):
        out = moe_with_shared(ws, dense, x, logits, experts, shared, side=side)
    for replay in range(3):
        ws.out.zero_()
        dense.down.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, expected), f"replay {replay}"
    # the shared expert folded into the routed launches: the same bytes
    folded = MoEWorkspace(Shape(rows, e, h, i), device, shared_rows=rows)
    got = moe_with_shared(folded, None, x, logits, experts, shared)
    torch.cuda.synchronize()
    assert torch.equal(got, expected)
    assert torch.equal(folded.shared_down, dense.down)
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2):
        out2 = moe_with_shared(folded, None, x, logits, experts, shared)
    for replay in range(3):
        folded.out.zero_()
        folded.down.zero_()
        torch.cuda.synchronize()
        g2.replay()
        torch.cuda.synchronize()
        assert torch.equal(out2, expected), f"folded replay {replay}"
    # against the oracle
    weights, ids = om.route(np_f32(logits))
    routed = om.expert_ffn(np_bf16(x), ids, weights, oracle_weights(w))
    so = oracle_weights(sw)
    shared_expected = om.dense_ffn(np_bf16(x), so.w13[0], so.s13[0], so.w2[0], so.s2[0])
    stats = assert_bf16_close(np_bf16(out), om.add_shared(routed, shared_expected), **CONTRACTION)
    print(f"side-stream shared expert: {stats}")


@pytest.mark.parametrize("shape", [(560, 16, 1024, 256), (300, 8, 512, 512), (1024, 128, 2048, 768),
                                   (37, 8, 256, 1536)],
                         ids=["c5_shapes", "h512_i512", "c4_model_1024_rows", "tiny"])
def test_grouped_by_pair_matches_sorted(device, shape):
    """FC1 finding its own routes (no sort) writes them as a route list of
    one 128-route item per (expert, part) - each expert's list equal to the
    sort's - with act codes and scales at the list's positions equal to the
    sorted launch's; FC2 over that list gives the sorted chain's fp32 down
    rows byte for byte; a live row count below the capacity leaves the rows
    past it untouched."""
    from drama3_amd.expert_weights import prepare_experts
    from drama3_amd.pipeline import MoEWorkspace, Shape

    rows, e, h, i = shape
    w, x, logits = _workload(rows, e, h, i, seed=23)
    experts = prepare_experts(w.to(device))
    sorted_ws = MoEWorkspace(Shape(rows, e, h, i), device, item_rows=128, grouped=True)
    pair_ws = MoEWorkspace(Shape(rows, e, h, i), device, item_rows=128, grouped=True, by_pair=True)
    live_rows = torch.tensor([rows - rows // 5], dtype=torch.int32, device=device)
    for ws in (sorted_ws, pair_ws):
        ws.front(x.to(device), logits.to(device), row_count=live_rows)
        ws.down.fill_(7.0)
        ws.routes_down(experts, live_rows)
    torch.cuda.synchronize()
    live = int(live_rows.item())
    live_pairs = live * 8
    assert torch.equal(pair_ws.ids[:live], sorted_ws.ids[:live])
    # the route list: item e * parts + j holds expert e's sorted routes [128 j, 128 j + 128)
    parts = -(-rows // 128)
    assert int(pair_ws.list_count.item()) == e * parts
    items = pair_ws.list_items.cpu()
    list_ids = pair_ws.list_ids.cpu()
    counts, starts = sorted_ws.counts.cpu(), sorted_ws.starts.cpu()
    sorted_ids = sorted_ws.sorted_ids.cpu()
    position = torch.full((live_pairs,), -1, dtype=torch.long)
    for ex in range(e):
        want = sorted_ids[starts[ex]:starts[ex] + counts[ex]]
        got = []
        for j in range(parts):
            item = ex * parts + j
            n = min(max(int(counts[ex]) - 128 * j, 0), 128)
            assert items[item].tolist() == [ex, 128 * item, n, 0]
            got.append(list_ids[128 * item:128 * item + n])
            position[list_ids[128 * item:128 * item + n].long()] = torch.arange(128 * item, 128 * item + n)
        assert torch.equal(torch.cat(got), want)
    assert bool((position >= 0).all())
    inverse = sorted_ws.inverse[:live_pairs].long()
    at = position.to(device)
    assert torch.equal(pair_ws.act[at], sorted_ws.act[inverse])
    assert torch.equal(pair_ws.act_scales[at].view(torch.int32), sorted_ws.act_scales[inverse].view(torch.int32))
    assert torch.equal(pair_ws.down[:live_pairs].view(torch.int32),
                       sorted_ws.down[:live_pairs].view(torch.int32))
    assert bool((pair_ws.down[live_pairs:] == 7.0).all())


def test_moe_with_shared_on_by_pair_workspace(device):
    """moe_with_shared on a by-pair workspace (its front skips the route
    sort): the routed experts run the by-pair FC1 and the FC2 over the route
    list it writes, so the result equals the sorted workspace's byte for
    byte, eagerly and after several replays of a captured graph."""
    from drama3_amd import workloads
    from drama3_amd.expert_weights import prepare_experts
    from drama3_amd.pipeline import DenseExpert, MoEWorkspace, Shape, moe_with_shared

    rows, e, h, i = 560, 16, 1024, 256
    gen = torch.Generator("cpu").manual_seed(41)
    w = workloads.make_experts(gen, e, h, i)
    sw = workloads.make_experts(gen, 1, h, i)
    x = workloads._bf16(gen, (rows, h)).to(device)
    logits = workloads._bf16(gen, (rows, e)).to(device)
    experts, shared = prepare_experts(w.to(device)), prepare_experts(sw.to(device))
    sorted_ws = MoEWorkspace(Shape(rows, e, h, i), device, item_rows=128, grouped=True)
    pair_ws = MoEWorkspace(Shape(rows, e, h, i), device, item_rows=128, grouped=True, by_pair=True)
    dense = DenseExpert(rows, h, i, device)
    expected = moe_with_shared(sorted_ws, dense, x, logits, experts, shared).clone()
    # stale sorted-route buffers must not matter on the by-pair workspace
    pair_ws.sorted_ids.fill_(-1)
    pair_ws.items.fill_(-1)
    pair_ws.num_items.fill_(1 << 20)
    got = moe_with_shared(pair_ws, dense, x, logits, experts, shared).clone()
    torch.cuda.synchronize()
    print(f"by-pair moe_with_shared rows {rows} E {e}: "
          f"{int(pair_ws.list_count.item())} listed items", flush=True)
    assert torch.equal(got, expected)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = moe_with_shared(pair_ws, dense, x, logits, experts, shared)
    for replay in range(3):
        pair_ws.out.zero_()
        pair_ws.down.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, expected), f"replay {replay}"
