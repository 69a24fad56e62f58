"""The fused front end (d3_moe_front: compaction + routing + quantisation +
last-workgroup route sort) against the standalone kernels and the oracle,
bit for bit, including repeated launches (the ticket must return to 0)."""

import numpy as np
import pytest
import torch

from helpers import np_f32, np_u8
from oracle import moe as om
from oracle.numerics import bf16_to_f32

pytestmark = pytest.mark.gpu


def _inputs(device, slots, hidden, experts, seed):
    gen = torch.Generator("cpu").manual_seed(seed)
    x = torch.randn((slots, hidden), generator=gen).to(torch.bfloat16)
    logits = torch.randn((slots, experts), generator=gen).to(torch.bfloat16)
    return x, logits, x.to(device), logits.to(device)


def _state(ws, count):
    t = int(ws.total.item())
    return dict(ids=ws.ids.cpu().numpy()[:count], weights=ws.weights.cpu()[:count],
                q=np_u8(ws.q)[:count], scales=np_f32(ws.x_scales)[:count],
                counts=ws.counts.cpu().numpy(), starts=ws.starts.cpu().numpy(), total=t,
                sorted=ws.sorted_ids.cpu().numpy().copy(), experts=ws.expert_ids.cpu().numpy().copy(),
                inverse=ws.inverse.cpu().numpy()[:count * 8], items=ws.items.cpu().numpy().copy(),
                num_items=int(ws.num_items.item()), pairs=int(ws.pairs_dev.item()))


@pytest.mark.parametrize("hidden,experts,p", [(1024, 16, 0.07), (2048, 128, 0.75), (1024, 16, 1.0),
                                              (2048, 256, 0.5), (1024, 16, 0.0)])
def test_fused_front_matches_standalone_kernels(device, hidden, experts, p):
    from drama3_amd.pipeline import MoEWorkspace, Shape, compact_slots

    slots = 64
    x, logits, xd, ld = _inputs(device, slots, hidden, experts, int(p * 100) + experts)
    occ = (np.random.default_rng(experts).uniform(size=slots) < p).astype(np.uint8)
    occ_d = torch.from_numpy(occ).to(device)
    fused = MoEWorkspace(Shape(slots, experts, hidden, 256), device, fused_sort=True)
    active = torch.empty(slots, dtype=torch.int32, device=device)
    count = torch.empty(1, dtype=torch.int32, device=device)
    for launch in range(3):  # the ticket must be back to 0 after every launch
        fused.front(xd, ld, occupancy=occ_d, active=active, count=count)
        torch.cuda.synchronize()
        assert int(fused.ticket.item()) == 0
    n = int(count.item())
    o_active, on = om.compact_slots(occ)
    assert n == on and np.array_equal(active.cpu().numpy()[:n], o_active)
    assert np.all(active.cpu().numpy()[n:] == -1)

    ref = MoEWorkspace(Shape(slots, experts, hidden, 256), device)
    a2 = torch.empty_like(active)
    c2 = torch.empty_like(count)
    compact_slots(occ_d, a2, c2)
    ref.route(ld, a2, c2)
    ref.quantize(xd, a2, c2)
    ref.sort(None, c2)
    torch.cuda.synchronize()
    got, want = _state(fused, n), _state(ref, n)
    for key in got:
        if key == "weights":
            assert torch.equal(got[key], want[key])
        elif key == "items":
            assert np.array_equal(got[key][:got["num_items"]], want[key][:want["num_items"]])
        else:
            assert np.array_equal(np.asarray(got[key]), np.asarray(want[key])), key
    if n:
        weights, ids = om.route(np_f32(logits)[o_active])
        assert np.array_equal(got["ids"], ids)
        q, s = om.quantize_rows(bf16_to_f32(x.view(torch.int16).numpy().view(np.uint16))[o_active])
        assert np.array_equal(got["q"], q) and np.array_equal(got["scales"], s)


@pytest.mark.parametrize("rows,experts,live", [
    (560, 16, None),    # 4480 pairs: fused row-mask sort
    (1100, 16, None),   # 8800 pairs: the wide sort (aligned items)
    (1024, 128, None),  # 8192 pairs, 128 x 16 mask words: the row-mask sort at its limits
    (600, 256, None),   # 256 x 10 mask words: the fused ballot sort
    (1000, 128, 301),   # device row count below capacity
    (1, 16, None),
])
@pytest.mark.parametrize("fused", [True, False])
def test_fused_front_row_mode_with_index(device, rows, experts, live, fused):
    """Row mode (mixed batches): row_index gathers rows; the sort is fused
    (opt-in) while pairs <= 8192 (row masks while E x ceil(rows / 64) <= 2048,
    else the chunked ballot sort) and otherwise the sort kernel's (row masks
    while they fit, else the ballot sort; the wide sort above 8192 pairs);
    every variant gives the oracle's sort, inverse map and work items."""
    from drama3_amd.pipeline import MoEWorkspace, Shape

    x, logits, xd, ld = _inputs(device, rows + 7, 1024, experts, rows + experts)
    index = torch.from_numpy(np.random.default_rng(rows).permutation(rows + 7)[:rows]).to(torch.int32)
    ws = MoEWorkspace(Shape(rows, experts, 1024, 256), device, item_rows=128 if rows > 128 else None,
                      fused_sort=fused)
    count = None if live is None else torch.tensor([live], dtype=torch.int32, device=device)
    n = rows if live is None else live
    for _ in range(2):
        ws.front(xd, ld, row_index=index.to(device), row_count=count)
        torch.cuda.synchronize()
        idx = index.numpy()[:n]
        weights, ids = om.route(np_f32(logits)[idx])
        assert np.array_equal(ws.ids.cpu().numpy()[:n], ids)
        o = om.sort_routes(ids, experts, ws.tile)
        assert int(ws.total.item()) == o.total
        assert np.array_equal(ws.counts.cpu().numpy(), o.counts)
        assert np.array_equal(ws.starts.cpu().numpy(), o.starts)
        sorted_ids = ws.sorted_ids.cpu().numpy()
        assert np.array_equal(sorted_ids[:o.total], o.sorted_ids)
        assert np.all(sorted_ids[o.total:] == n * 8)
        assert np.array_equal(ws.expert_ids.cpu().numpy()[:o.total // ws.tile], o.expert_ids)
        assert np.array_equal(ws.inverse.cpu().numpy()[:n * 8], o.inverse)
        # work items: each expert's routes in chunks of item_rows, in expert
        # order; over the wide sort's aligned capacity, while the experts
        # with routes average at least 1.5 items, each expert's run is
        # padded to an even count with one empty item
        items = sum(-(-int(c) // ws.item_rows) for c in o.counts)
        padded = ws.aligned_items and 2 * items >= 3 * int(np.count_nonzero(o.counts))
        want = []
        for e in range(experts):
            run = [(e, int(o.starts[e]) + j, min(ws.item_rows, int(o.counts[e]) - j), 0)
                   for j in range(0, int(o.counts[e]), ws.item_rows)]
            want += run + ([(e, int(o.starts[e]), 0, 0)] if padded and len(run) % 2 else [])
        num_items = int(ws.num_items.item())
        assert num_items == len(want)
        assert np.array_equal(ws.items.cpu().numpy().reshape(-1, 4)[:num_items], np.array(want))
        assert int(ws.ticket.item()) == 0


@pytest.mark.parametrize("config", [1, 2, 3])
def test_swiglu_prologue_matches_chain(device, config):
    """FC2 with the SwiGLU requant in its prologue (three kernels) gives
    exactly the bytes of the four-kernel chain."""
    from drama3_amd import workloads
    from drama3_amd.pipeline import MoEWorkspace, Shape

    w = workloads.CONFIGS[config]()
    step = w.steps[0]
    experts = w.experts.to(device)
    occ = step.occupancy.to(device)
    xs, ls = step.x_slots.to(device), step.logits_slots.to(device)
    outs = {}
    for name in ("chain", "prologue"):
        ws = MoEWorkspace(Shape(64, w.num_experts, w.hidden, w.intermediate), device,
                          swiglu_in_fc2=name == "prologue")
        active = torch.empty(64, dtype=torch.int32, device=device)
        count = torch.empty(1, dtype=torch.int32, device=device)
        for _ in range(2):
            ws.front(xs, ls, occupancy=occ, active=active, count=count)
            out = ws.experts(experts, count)
        torch.cuda.synchronize()
        n = int(count.item())
        outs[name] = out[:n].cpu()
        assert ws.swiglu_in_fc2 == (name == "prologue")
    assert torch.equal(outs["prologue"], outs["chain"])
