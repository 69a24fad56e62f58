"""End-to-end parity of the MoE step on the five BASELINE configurations.

Integer outputs (active slots, routing ids, histogram, sorted route list,
inverse map) are compared bit for bit with the CPU oracle; the bf16 outputs
within the tolerances stated in helpers.py.  Everything runs through the C
ABI on cuda:0."""

import numpy as np
import pytest
import torch

from helpers import (CONTRACTION, EXACT, RRMS_REFERENCE, assert_bf16_close, np_bf16, np_f32,
                     oracle_weights, rrms)
from oracle import moe as om
from oracle.numerics import bf16_to_f32

pytestmark = pytest.mark.gpu


def check_integer_state(ws, ids_expected, experts, count):
    ids = ws.ids.cpu().numpy()[:count]
    assert np.array_equal(ids, ids_expected), "routing ids differ"
    o = om.sort_routes(ids_expected, experts, ws.tile)
    assert np.array_equal(ws.counts.cpu().numpy(), o.counts)
    assert int(ws.total.item()) == o.total
    assert np.array_equal(ws.sorted_ids.cpu().numpy()[:o.total], o.sorted_ids)
    assert np.array_equal(ws.inverse.cpu().numpy()[:ids_expected.size], o.inverse)


def run_decode(workload, device, step_index=0):
    from drama3_amd.pipeline import DecodeStep

    step = workload.steps[step_index]
    experts = workload.experts.to(device)
    ds = DecodeStep(64, workload.num_experts, workload.hidden, workload.intermediate,
                    device=device)
    out = ds(step.occupancy.to(device), step.x_slots.to(device), step.logits_slots.to(device),
             experts)
    torch.cuda.synchronize()
    return ds, out


@pytest.mark.parametrize("config", [1, 2, 3])
def test_decode_configs(device, config):
    from drama3_amd import workloads

    w = workloads.CONFIGS[config]()
    ds, out = run_decode(w, device)
    step = w.steps[0]
    active, n = om.compact_slots(step.occupancy.numpy())
    assert int(ds.count.item()) == n
    assert np.array_equal(ds.active.cpu().numpy()[:n], active)
    x, logits = np_bf16(step.x_slots)[active], np_f32(step.logits_slots)[active]
    weights, ids = om.route(logits)
    check_integer_state(ds.workspace, ids, w.num_experts, n)
    expected = om.expert_ffn(x, ids, weights, oracle_weights(w.experts))
    # decode items never exceed the exact-path route limit (rows <= 64)
    stats = assert_bf16_close(np_bf16(out)[:n], expected, **EXACT)
    print(f"config {config}: rows {n} {stats}")


@pytest.mark.parametrize("config", [1, 2, 3])
def test_decode_configs_benched_path(device, config):
    """The step bench.py times: fragment-major weights (prepare_experts), so
    DecodeStep runs its three launches (FC1 routing and quantising the slots,
    FC2 finding its routes, routed combine) with no front and no route sort;
    against the oracle directly."""
    from drama3_amd import workloads
    from drama3_amd.expert_weights import prepare_experts
    from drama3_amd.pipeline import DecodeStep

    w = workloads.CONFIGS[config]()
    step = w.steps[0]
    experts = prepare_experts(w.experts.to(device))
    ds = DecodeStep(64, w.num_experts, w.hidden, w.intermediate, device=device)
    occ, xs, ls = (step.occupancy.to(device), step.x_slots.to(device),
                   step.logits_slots.to(device))
    assert ds.uses_sortless(experts) and ds.uses_frontless(occ, xs, ls)
    out = ds(occ, xs, ls, experts)
    torch.cuda.synchronize()
    active, n = om.compact_slots(step.occupancy.numpy())
    assert int(ds.count.item()) == n
    assert np.array_equal(ds.active.cpu().numpy()[:n], active)
    weights, ids = om.route(np_f32(step.logits_slots)[active])
    assert np.array_equal(ds.workspace.ids.cpu().numpy()[:n], ids)
    # routing weights: fp32 exp / sums in another order, within one bf16 ulp
    got_w, want_w = np_f32(ds.workspace.weights)[:n], bf16_to_f32(weights)
    assert np.all(np.abs(got_w - want_w) <= np.abs(want_w) * 2.0**-8 + 1e-7)
    expected = om.expert_ffn(np_bf16(step.x_slots)[active], ids, weights, oracle_weights(w.experts))
    stats = assert_bf16_close(np_bf16(out)[:n], expected, **EXACT)
    print(f"config {config} (benched step): rows {n} {stats}")


def test_prefill_with_shared_expert(device):
    """Config 4: 16 packed prompts (cu_seqlens), routed + dense FP8 shared expert."""
    from drama3_amd import workloads
    from drama3_amd.pipeline import DenseExpert, MoEWorkspace, Shape

    w = workloads.config4()
    step = w.steps[0]
    x, logits = step.packed()
    rows = len(x)
    assert rows == int(step.cu_seqlens[-1])
    ws = MoEWorkspace(Shape(rows, w.num_experts, w.hidden, w.intermediate), device)
    dense = DenseExpert(rows, w.hidden, w.shared.intermediate, device)
    experts, shared = w.experts.to(device), w.shared.to(device)
    xd, ld = x.to(device), logits.to(device)
    ws.front(xd, ld)  # 29k pairs: fused route + quantise, then the sort kernel
    shared_y = dense.forward(ws.q, ws.x_scales, shared)
    out = ws.experts(experts, shared=shared_y)
    torch.cuda.synchronize()
    weights, ids = om.route(np_f32(logits))
    check_integer_state(ws, ids, w.num_experts, rows)
    routed = om.expert_ffn(np_bf16(x), ids, weights, oracle_weights(w.experts))
    sw = oracle_weights(w.shared)
    shared_expected = om.dense_ffn(np_bf16(x), sw.w13[0], sw.s13[0], sw.w2[0], sw.s2[0])
    expected = om.add_shared(routed, shared_expected)
    stats = assert_bf16_close(np_bf16(out), expected, **CONTRACTION)
    print(f"config 4: rows {rows} {stats}")


def test_mixed_batching_sequence(device):
    """Config 5: 4 steps of 48 decode slots + 2 x 256 prefill rows with 4
    slots retiring / admitted between steps; packing, routing permutation and
    unpermute indices bit-exact at every step, outputs within tolerance."""
    from drama3_amd import workloads
    from drama3_amd.packed_prefill import packed_row_metadata
    from drama3_amd.pipeline import MoEWorkspace, Shape, compact_slots

    w = workloads.config5()
    experts = w.experts.to(device)
    wt = oracle_weights(w.experts)
    slots = 64
    prefill = len(w.steps[0].prefill_x)
    capacity = 48 + prefill
    ws = MoEWorkspace(Shape(capacity, w.num_experts, w.hidden, w.intermediate), device)
    active = torch.empty(slots, dtype=torch.int32, device=device)
    count = torch.empty(1, dtype=torch.int32, device=device)
    previous = None
    for index, step in enumerate(w.steps):
        occ = step.occupancy
        if previous is not None:
            assert int((previous & ~occ.bool()).sum()) == 4 and int((occ.bool() & ~previous).sum()) == 4
        previous = occ.bool()
        compact_slots(occ.to(device), active, count)
        n = int(count.item())
        o_active, on = om.compact_slots(occ.numpy())
        assert n == on == 48 and np.array_equal(active.cpu().numpy()[:n], o_active)
        # one row source: [slot rows | prefill rows]; decode rows first
        source = torch.cat([step.x_slots, step.prefill_x]).to(device)
        source_logits = torch.cat([step.logits_slots, step.prefill_logits]).to(device)
        row_index = torch.cat([active[:n], slots + torch.arange(prefill, dtype=torch.int32,
                                                                device=device)])
        # packed prefill metadata of the suffix
        cu = step.cu_seqlens.to(device)
        seq_slots = torch.tensor([60, 61], dtype=torch.int64, device=device)
        positions = torch.empty(prefill, dtype=torch.int64, device=device)
        row_slots = torch.empty_like(positions)
        packed_row_metadata(cu, seq_slots, prefill, positions, row_slots)
        opos, oslots, _ = om.row_metadata(step.cu_seqlens.numpy(), [60, 61], prefill)
        assert np.array_equal(positions.cpu().numpy(), opos)
        assert np.array_equal(row_slots.cpu().numpy(), oslots)
        out = ws.forward(source, source_logits, experts, row_index=row_index)
        torch.cuda.synchronize()
        x, logits = step.packed()
        kind, owner, _ = om.mixed_rows(o_active, [256, 256])
        assert np.array_equal(kind[:48], np.zeros(48)) and np.array_equal(owner[:48], o_active)
        weights, ids = om.route(np_f32(logits))
        check_integer_state(ws, ids, w.num_experts, capacity)
        expected = om.expert_ffn(np_bf16(x), ids, weights, wt)
        stats = assert_bf16_close(np_bf16(out), expected, **CONTRACTION)
        print(f"config 5 step {index}: {stats}")


def test_decode_step_graph_replays(device):
    """Capture the decode step once; replay it with different occupancies
    (device-side row count) and eager work between replays; every replay
    matches both an eager run and the oracle."""
    from drama3_amd import workloads
    from drama3_amd.pipeline import DecodeStep

    w = workloads.config1()
    step = w.steps[0]
    experts = w.experts.to(device)
    wt = oracle_weights(w.experts)
    ds = DecodeStep(64, w.num_experts, w.hidden, w.intermediate, device=device)
    occ = step.occupancy.to(device)
    x_slots, logits_slots = step.x_slots.to(device), step.logits_slots.to(device)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ds(occ, x_slots, logits_slots, experts)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ds(occ, x_slots, logits_slots, experts)
    rng = np.random.default_rng(0)
    for replay in range(4):
        occupancy = (rng.uniform(size=64) < [0.1, 0.5, 0.9, 1.0][replay]).astype(np.uint8)
        occ.copy_(torch.from_numpy(occupancy))
        graph.replay()
        torch.cuda.synchronize()
        got = np_bf16(out).copy()
        _ = torch.ones(1024, device=device).sum().item()  # eager work between replays
        eager = DecodeStep(64, w.num_experts, w.hidden, w.intermediate, device=device)
        eager_out = eager(occ, x_slots, logits_slots, experts)
        torch.cuda.synchronize()
        active, n = om.compact_slots(occupancy)
        assert np.array_equal(got[:n], np_bf16(eager_out)[:n])
        if n:
            weights, ids = om.route(np_f32(step.logits_slots)[active])
            expected = om.expert_ffn(np_bf16(step.x_slots)[active], ids, weights, wt)
            assert_bf16_close(got[:n], expected, **EXACT)


def test_reference_api_small_and_native(device):
    """small_batch_moe / native_moe with reference-style inputs (int64 ids,
    bf16 weights from route) agree with the oracle and with each other."""
    from drama3_amd import workloads
    from drama3_amd.kernels import native_moe, route, small_batch_moe

    w = workloads.config1()
    x, logits = w.steps[0].packed()
    experts = w.experts.to(device)
    weights, ids = route(logits.to(device))
    a = small_batch_moe(x.to(device), ids, weights, experts)
    b = native_moe(x.to(device), ids, weights, experts, block_m=64)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    ow, oids = om.route(np_f32(logits))
    expected = om.expert_ffn(np_bf16(x), oids, ow, oracle_weights(w.experts))
    assert_bf16_close(np_bf16(a), expected, **EXACT)
    assert rrms(bf16_to_f32(np_bf16(a)), bf16_to_f32(expected)) < RRMS_REFERENCE


def test_routed_moe_dispatch_and_padding_router(device):
    """routed_moe (model.py:520-583): same result as the reference-API chain,
    and rows in reserved padding slots route exactly like row 0."""
    from drama3_amd import workloads
    from drama3_amd.kernels import routed_moe

    w = workloads.config1()
    x, logits = w.steps[0].packed()
    experts = w.experts.to(device)
    xd, ld = x.to(device), logits.to(device)
    out = routed_moe(xd, ld, experts, True)
    torch.cuda.synchronize()
    ow, oids = om.route(np_f32(logits))
    expected = om.expert_ffn(np_bf16(x), oids, ow, oracle_weights(w.experts))
    assert_bf16_close(np_bf16(out), expected, **EXACT)
    # slots >= 32 are reserved padding: rows 1 and 3 take row 0's routing
    slots = torch.tensor([3, 40, 17, 62], dtype=torch.int64, device=device)
    padded = routed_moe(xd, ld, experts, True, row_slots=slots, padding_start=32)
    forced = ld.clone()
    forced[1] = ld[0]
    forced[3] = ld[0]
    ref = routed_moe(xd, forced, experts, True)
    torch.cuda.synchronize()
    assert torch.equal(padded, ref)
    with pytest.raises(ValueError):
        routed_moe(xd, ld, experts, True, row_slots=slots)
