"""The allocation-free decode step (d3_decode_step_static, intermediates in
the library's static device scratch) against d3_decode_step on a caller
workspace, through the C ABI: byte-identical outputs on two calls in a row,
the second with a smaller input, and sizes beyond the scratch rejected
before any launch."""

import numpy as np
import pytest
import torch

from helpers import np_bf16

pytestmark = pytest.mark.gpu


def _case(device, seed, slots, experts, hidden, inter, p):
    from drama3_amd import workloads as wl
    from drama3_amd.expert_weights import prepare_experts

    gen = torch.Generator("cpu").manual_seed(seed)
    ex = prepare_experts(wl.make_experts(gen, experts, hidden, inter).to(device))
    occ = (torch.rand(slots, generator=gen) < p).to(torch.uint8)
    x = torch.randn((slots, hidden), generator=gen).to(torch.bfloat16)
    logits = torch.randn((slots, experts), generator=gen).to(torch.bfloat16)
    return ex, occ.to(device), x.to(device), logits.to(device)


def _operands(ex):
    return (ex.d3_w13_packed.data_ptr(), ex.w13_scale_inv.data_ptr(), ex.d3_w2_packed.data_ptr(),
            ex.w2_scale_inv.data_ptr())


def _outputs(device, slots, hidden):
    active = torch.full((slots,), 12345, dtype=torch.int32, device=device)
    count = torch.full((1,), -7, dtype=torch.int32, device=device)
    out = torch.full((slots, hidden), 3.0, dtype=torch.bfloat16, device=device)
    return active, count, out


def _run_both(device, ex, occ, x, logits):
    from drama3_amd import _lib
    from drama3_amd.pipeline import DTYPE_BF16, EXACT_ROUTES

    slots, hidden = x.shape
    experts = logits.shape[1]
    inter = ex.w2_weight.shape[2]
    top_k = 8
    stream = _lib.stream(device)
    common = (*_operands(ex), experts, hidden, inter, occ.data_ptr(), slots, x.data_ptr(),
              x.stride(0), logits.data_ptr(), DTYPE_BF16, logits.stride(0), top_k, EXACT_ROUTES)
    # the existing entry point on a caller workspace
    ids = torch.empty((slots, top_k), dtype=torch.int32, device=device)
    weights = torch.empty((slots, top_k), dtype=torch.bfloat16, device=device)
    gate_up = torch.empty((slots * top_k, 2 * inter), dtype=torch.bfloat16, device=device)
    down = torch.empty((slots * top_k, hidden), dtype=torch.float32, device=device)
    active_a, count_a, out_a = _outputs(device, slots, hidden)
    _lib.call("d3_decode_step", *common, ids.data_ptr(), weights.data_ptr(), DTYPE_BF16,
              gate_up.data_ptr(), down.data_ptr(), active_a.data_ptr(), count_a.data_ptr(),
              out_a.data_ptr(), stream)
    # the allocation-free variant
    active_b, count_b, out_b = _outputs(device, slots, hidden)
    _lib.call("d3_decode_step_static", *common, active_b.data_ptr(), count_b.data_ptr(),
              out_b.data_ptr(), stream)
    torch.cuda.synchronize()
    n = int(count_a.item())
    assert n == int(occ.sum().item()) and int(count_b.item()) == n
    assert torch.equal(active_a, active_b)
    assert np.array_equal(np_bf16(out_a[:n]), np_bf16(out_b[:n]))
    assert np.all(np.isfinite(out_b[:n].float().cpu().numpy()))
    return n


def test_static_step_equals_workspace_step_twice_second_smaller(device):
    first = _case(device, 40, 64, 128, 2048, 768, 0.75)  # the headline decode shape
    n1 = _run_both(device, *first)
    second = _case(device, 41, 24, 16, 1024, 256, 0.5)  # fewer slots, smaller experts
    n2 = _run_both(device, *second)
    assert 0 < n2 < n1


def test_static_step_rejects_sizes_beyond_its_scratch(device):
    from drama3_amd import _lib
    from drama3_amd.pipeline import DTYPE_BF16, EXACT_ROUTES

    ex, occ, x, logits = _case(device, 42, 128, 16, 1024, 256, 0.5)
    active, count, out = _outputs(device, 128, 1024)
    with pytest.raises(ValueError, match="exceeds the static scratch"):
        _lib.call("d3_decode_step_static", *_operands(ex), 16, 1024, 256, occ.data_ptr(), 128,
                  x.data_ptr(), x.stride(0), logits.data_ptr(), DTYPE_BF16, logits.stride(0), 8,
                  EXACT_ROUTES, active.data_ptr(), count.data_ptr(), out.data_ptr(),
                  _lib.stream(device))
    torch.cuda.synchronize()
    assert int(count.item()) == -7  # nothing was launched


def test_static_step_captured_in_a_graph_replays_with_new_occupancy(device):
    """d3_decode_step_static captured in a graph (the callers it is for):
    the first call on the device, which looks up the scratch address, runs
    before the capture; the graph is then replayed twice with a different
    occupancy copied into the captured input each time, and every replay's
    outputs equal d3_decode_step's on a caller workspace byte for byte."""
    from drama3_amd import _lib
    from drama3_amd.pipeline import DTYPE_BF16, EXACT_ROUTES

    ex, occ, x, logits = _case(device, 43, 64, 128, 2048, 768, 0.75)
    slots, hidden = x.shape
    experts, inter, top_k = logits.shape[1], ex.w2_weight.shape[2], 8
    common = (*_operands(ex), experts, hidden, inter, occ.data_ptr(), slots, x.data_ptr(),
              x.stride(0), logits.data_ptr(), DTYPE_BF16, logits.stride(0), top_k, EXACT_ROUTES)
    active, count, out = _outputs(device, slots, hidden)
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):  # eager first call: the scratch lookup happens here
        _lib.call("d3_decode_step_static", *common, active.data_ptr(), count.data_ptr(),
                  out.data_ptr(), _lib.stream(device))
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _lib.call("d3_decode_step_static", *common, active.data_ptr(), count.data_ptr(),
                  out.data_ptr(), _lib.stream(device))
    gen = torch.Generator("cpu").manual_seed(44)
    for replay, p in enumerate((0.4, 0.9)):
        occ.copy_((torch.rand(slots, generator=gen) < p).to(torch.uint8))
        active.fill_(12345)
        count.fill_(-7)
        out.fill_(3.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        snapshot = (active.clone(), int(count.item()), out.clone())
        n = _run_both(device, ex, occ, x, logits)  # the workspace step, fresh buffers
        assert snapshot[1] == n, f"replay {replay}"
        ids = torch.empty((slots, top_k), dtype=torch.int32, device=device)
        weights = torch.empty((slots, top_k), dtype=torch.bfloat16, device=device)
        gate_up = torch.empty((slots * top_k, 2 * inter), dtype=torch.bfloat16, device=device)
        down = torch.empty((slots * top_k, hidden), dtype=torch.float32, device=device)
        active_a, count_a, out_a = _outputs(device, slots, hidden)
        _lib.call("d3_decode_step", *common, ids.data_ptr(), weights.data_ptr(), DTYPE_BF16,
                  gate_up.data_ptr(), down.data_ptr(), active_a.data_ptr(), count_a.data_ptr(),
                  out_a.data_ptr(), _lib.stream(device))
        torch.cuda.synchronize()
        assert torch.equal(snapshot[0], active_a), f"replay {replay}"
        assert np.array_equal(np_bf16(snapshot[2][:n]), np_bf16(out_a[:n])), f"replay {replay}"
