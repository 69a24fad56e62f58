"""One MoE layer around the routed experts (MoELayer: ``moe_parts`` /
``moe`` of model.py:485-518): the packed input projection, the bf16 shared
expert on a side stream and the routed FP8 experts.  Routing ids are
compared bit for bit with the oracle on the projected router columns, the
routed rows within the stated tolerances, the SwiGLU bytes exactly, the
shared expert's bf16 GEMM against an fp32 product, the combine within one
ulp; the side-stream and in-line schedules and graph replays agree bit for
bit."""

import numpy as np
import pytest
import torch

from helpers import CONTRACTION, EXACT, assert_bf16_close, np_bf16, np_f32, oracle_weights
from oracle import moe as om

pytestmark = pytest.mark.gpu


def _weights(gen, e, h, i, si, device):
    from drama3_amd.expert_weights import prepare_experts
    from drama3_amd.moe_layer import pack_input_projection
    from drama3_amd.workloads import make_experts

    experts_cpu = make_experts(gen, e, h, i)
    experts = prepare_experts(experts_cpu.to(device))
    scale = h ** -0.5

    def bf16(*shape, s=scale):
        return (torch.randn(shape, generator=gen) * s).to(torch.bfloat16).to(device)

    projection = pack_input_projection(bf16(si, h), bf16(si, h), bf16(e, h, s=1.0), bf16(1, h))
    down = bf16(h, si, s=si ** -0.5)
    return experts_cpu, experts, projection, down


@pytest.mark.parametrize("rows,e,h,i,si", [(48, 16, 1024, 256, 256), (300, 16, 1024, 256, 512),
                                           (64, 128, 2048, 768, 512)])
def test_moe_layer_parts_and_combine(device, rows, e, h, i, si):
    from drama3_amd.moe_layer import MoELayer

    gen = torch.Generator("cpu").manual_seed(rows + e)
    experts_cpu, experts, projection, down = _weights(gen, e, h, i, si, device)
    x = torch.randn((rows, h), generator=gen).to(torch.bfloat16).to(device)
    layers = {name: MoELayer(rows, e, h, i, si, device=device, overlap=name == "overlap")
              for name in ("overlap", "inline")}
    outs = {}
    for name, layer in layers.items():
        out = layer(x, projection, down, experts).clone()
        torch.cuda.synchronize()
        outs[name] = out
    assert torch.equal(outs["overlap"].view(torch.int16), outs["inline"].view(torch.int16))
    layer = layers["overlap"]
    projected = layer.projected.clone()
    assert torch.equal(projected.view(torch.int16),
                       torch.mm(x, projection.t()).view(torch.int16))
    gate_up = np_bf16(projected[:, :2 * si])
    router = np_f32(projected[:, 2 * si:2 * si + e])
    gate = np_bf16(projected[:, 2 * si + e])
    # shared expert: SwiGLU bytes exact, the bf16 GEMM within bf16 rounding of fp32
    assert np.array_equal(np_bf16(layer.act), om.silu_mul(gate_up))
    want_shared = layer.act.float() @ down.float().t()
    err = (layer.shared.float() - want_shared).abs()
    assert float((err / (want_shared.abs() + 1e-3)).max()) < 2 ** -6
    # routed experts on the projected router columns
    weights, ids = om.route(router)
    routed_expected = om.expert_ffn(np_bf16(x), ids, weights, oracle_weights(experts_cpu))
    routed = np_bf16(layer.routed)[:rows]
    tol = EXACT if layer.decode else CONTRACTION
    stats = assert_bf16_close(routed, routed_expected, **tol)
    want_out = om.combine_experts(routed, np_bf16(layer.shared), gate)
    assert_bf16_close(np_bf16(outs["overlap"]), want_out, ulps=1, row_floor=0.0)
    print(f"rows {rows} E {e}: routed {stats}")


def test_moe_layer_graph_replays(device):
    """Capture the layer (side stream forked and joined inside the graph);
    replay with new inputs and eager work in between; every replay equals an
    eager run."""
    from drama3_amd.moe_layer import MoELayer

    gen = torch.Generator("cpu").manual_seed(5)
    rows, e, h, i, si = 64, 16, 1024, 256, 256
    _, experts, projection, down = _weights(gen, e, h, i, si, device)
    layer = MoELayer(rows, e, h, i, si, device=device, overlap=True)
    x = torch.zeros((rows, h), dtype=torch.bfloat16, device=device)
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        layer(x, projection, down, experts)
    torch.cuda.current_stream(device).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        layer(x, projection, down, experts)
    for _ in range(3):
        fresh = torch.randn((rows, h), generator=gen).to(torch.bfloat16).to(device)
        x.copy_(fresh)
        torch.randn(500, 500, device=device).sum()
        graph.replay()
        replayed = layer.out.clone()
        eager = layer(x, projection, down, experts).clone()
        torch.cuda.synchronize()
        assert torch.equal(replayed.view(torch.int16), eager.view(torch.int16))
