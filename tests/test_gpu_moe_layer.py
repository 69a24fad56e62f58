"""One MoE layer around the routed experts (MoELayer: ``moe_parts`` /
``moe`` of model.py:485-518): the packed input projection and the shared
expert's down projection on the bf16 MFMA kernel (d3_dense_bf16, against an
fp32 product of the same bf16 operands), the SwiGLU formed inside the down
projection (the bytes of silu_mul), the routed FP8 experts (routing ids bit
for bit with the oracle on the projected router columns, routed rows within
the stated tolerances), the fused decode epilogue (d3_combine_route_logits)
byte-identical to the separate routed combine + combine_experts (+
add_norm), and the side-stream / in-line schedules and graph replays
agreeing bit for bit."""

import numpy as np
import pytest
import torch

from helpers import CONTRACTION, EXACT, assert_bf16_close, np_bf16, np_f32, oracle_weights
from oracle import moe as om
from oracle.numerics import bf16_to_f32

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


def _close_to_fp32_product(got: torch.Tensor, want: torch.Tensor) -> None:
    """bf16 result of an fp32-accumulated product: within one bf16 rounding
    (plus fp32 summation-order noise) of the fp32 product."""
    g, w = got.float().cpu(), want.float().cpu()
    bound = w.abs() * 2.0 ** -8 + w.abs().amax(dim=-1, keepdim=True) * 2.0 ** -16 + 1e-30
    assert bool(((g - w).abs() <= bound).all()), float(((g - w).abs() / bound).max())


@pytest.mark.parametrize("rows,n,k", [(64, 1408, 2048), (1, 16, 256), (37, 272, 768),
                                      (300, 1024, 512), (1024, 48, 1536), (129, 64, 1024),
                                      # the tiled kernel: above 768 rows, or K outside
                                      # the streaming kernel's set
                                      (1025, 1408, 2048), (2048, 1408, 2048), (4096, 2048, 512),
                                      (3001, 272, 64), (1500, 48, 1536), (100, 144, 320)])
def test_dense_bf16_against_fp32(device, rows, n, k):
    from drama3_amd.moe_layer import dense_bf16

    gen = torch.Generator("cpu").manual_seed(rows * 7 + n)
    x = torch.randn((rows, k), generator=gen).to(torch.bfloat16).to(device)
    w = (torch.randn((n, k), generator=gen) * k ** -0.5).to(torch.bfloat16).to(device)
    out = torch.full((rows, n), 7.0, dtype=torch.bfloat16, device=device)
    dense_bf16(x, w, out)
    torch.cuda.synchronize()
    _close_to_fp32_product(out, x.float() @ w.float().t())


@pytest.mark.parametrize("rows,pairs,n,k", [(64, 512, 1408, 2048), (5, 256, 656, 1024),
                                            (200, 128, 272, 768), (70, 64, 128, 512),
                                            (2048, 512, 1408, 2048), (1100, 64, 128, 512),
                                            (4096, 512, 1408, 2048), (1030, 192, 400, 1024)])
def test_dense_bf16_pairs_write_silu_mul(device, rows, pairs, n, k):
    """With gate / up pairs the projection's epilogue writes the shared
    expert's activation: the bytes of silu_mul on the projected rows."""
    from drama3_amd.kernels import silu_mul
    from drama3_amd.moe_layer import dense_bf16

    gen = torch.Generator("cpu").manual_seed(rows + k)
    x = torch.randn((rows, k), generator=gen).to(torch.bfloat16).to(device)
    w = (torch.randn((n, k), generator=gen) * k ** -0.5 * 2).to(torch.bfloat16).to(device)
    out = torch.empty((rows, n), dtype=torch.bfloat16, device=device)
    act = torch.empty((rows, pairs), dtype=torch.bfloat16, device=device)
    dense_bf16(x, w, out, pairs, act)
    want_act = silu_mul(out[:, :2 * pairs])
    torch.cuda.synchronize()
    _close_to_fp32_product(out, x.float() @ w.float().t())
    assert torch.equal(act.view(torch.int16), want_act.view(torch.int16))
    assert np.array_equal(np_bf16(act), om.silu_mul(np_bf16(out[:, :2 * pairs])))


@pytest.mark.parametrize("rows,e,h,i,si", [(48, 16, 1024, 256, 256), (300, 16, 1024, 256, 512),
                                           (64, 128, 2048, 768, 512),
                                           # the reference model's layer (E256, I512, shared I512)
                                           (64, 256, 2048, 512, 512),
                                           # prefill-sized layers: tiled projections
                                           (2048, 256, 2048, 512, 512), (4096, 64, 1024, 256, 512)],
                         ids=["r48_e16", "r300_e16", "r64_e128", "r64_reference_shape",
                              "r2048_reference_shape", "r4096_e64"])
def test_moe_layer_parts_and_combine(device, rows, e, h, i, si):
    from drama3_amd.kernels import combine_experts, combine_experts_add_norm
    from drama3_amd.moe_layer import MoELayer

    gen = torch.Generator("cpu").manual_seed(rows + e)
    experts_cpu, experts, projection, down = _weights(gen, e, h, i, si, device)
    x = torch.randn((rows, h), generator=gen).to(torch.bfloat16).to(device)
    layers = {name: MoELayer(rows, e, h, i, si, device=device, overlap=name == "overlap")
              for name in ("overlap", "inline")}
    outs = {}
    for name, layer in layers.items():
        outs[name] = layer(x, projection, down, experts).clone()
        torch.cuda.synchronize()
    assert torch.equal(outs["overlap"].view(torch.int16), outs["inline"].view(torch.int16))
    layer = layers["inline"]
    routed, shared, gate = (t.clone() for t in layer.parts(x, projection, down, experts))
    projected = layer.projected.clone()
    torch.cuda.synchronize()
    _close_to_fp32_product(projected, x.float() @ projection.float().t())
    gate_up = np_bf16(projected[:, :2 * si])
    router = np_f32(projected[:, 2 * si:2 * si + e])
    # shared expert: SwiGLU bytes of silu_mul, the down projection within one
    # bf16 rounding of the fp32 product
    act = torch.from_numpy(bf16_to_f32(om.silu_mul(gate_up)))
    assert np.array_equal(np_bf16(layer.act), om.silu_mul(gate_up))
    _close_to_fp32_product(shared, act @ down.float().cpu().t())
    # routed experts on the projected router columns
    weights, ids = om.route(router)
    routed_expected = om.expert_ffn(np_bf16(x), ids, weights, oracle_weights(experts_cpu))
    tol = EXACT if layer.decode else CONTRACTION
    stats = assert_bf16_close(np_bf16(routed)[:rows], routed_expected, **tol)
    # the layer's combine (fused into one launch for decode) is exactly
    # combine_experts of its parts, and both the oracle's single rounding
    want = combine_experts(routed, shared, gate)
    torch.cuda.synchronize()
    assert torch.equal(outs["inline"].view(torch.int16), want.view(torch.int16))
    assert np.array_equal(np_bf16(want), om.combine_experts(np_bf16(routed), np_bf16(shared),
                                                            np_bf16(gate)[:, 0]))
    # residual + RMSNorm form
    residual = torch.randn((rows, h), generator=gen).to(torch.bfloat16).to(device)
    norm_w = (torch.randn((h,), generator=gen) * 0.1).to(torch.bfloat16).to(device)
    res_a, res_b = residual.clone(), residual.clone()
    got = layer.add_norm(x, projection, down, experts, res_a, norm_w, 1e-6).clone()
    ref = combine_experts_add_norm(routed, shared, gate, res_b, norm_w, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(res_a.view(torch.int16), res_b.view(torch.int16))
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    print(f"rows {rows} E {e} H {h} I {i} shared {si}: routed {stats}, "
          f"fused epilogue {layer._fused(experts, x, layer._views()[1])}", flush=True)


@pytest.mark.parametrize("logits_dtype,weights_dtype", [(torch.float32, torch.float32),
                                                       (torch.bfloat16, torch.bfloat16)])
def test_combine_route_logits_equals_separate_launches(device, logits_dtype, weights_dtype):
    """d3_combine_route_logits after a frontless decode FC1 / FC2 equals
    d3_decode_route_combine + d3_combine_experts (and + d3_add_norm with a
    residual) byte for byte, stored weights included; live rows only."""
    from drama3_amd import _lib, workloads
    from drama3_amd.expert_weights import prepare_experts
    from drama3_amd.kernels import add_norm, combine_experts
    from drama3_amd.pipeline import DecodeStep, dtype_code

    gen = torch.Generator("cpu").manual_seed(17)
    rows, e, h, i = 40, 16, 1024, 256
    experts = prepare_experts(workloads.make_experts(gen, e, h, i).to(device))
    x = torch.randn((rows, h), generator=gen).to(torch.bfloat16).to(device)
    logits = torch.randn((rows, e), generator=gen).to(logits_dtype).to(device)
    shared = torch.randn((rows, h), generator=gen).to(torch.bfloat16).to(device)
    gate = torch.randn((rows, 3), generator=gen).to(torch.bfloat16).to(device)[:, 1:2]
    norm_w = (torch.randn((h,), generator=gen) * 0.1).to(torch.bfloat16).to(device)
    residual = torch.randn((rows, h), generator=gen).to(torch.bfloat16).to(device)
    step = DecodeStep(rows, e, h, i, device=device)
    step.workspace.weights = torch.empty((rows, 8), dtype=weights_dtype, device=device)
    occ = torch.ones(rows, dtype=torch.uint8, device=device)
    routed = step(occ, x, logits, experts).clone()  # routes ranked in FC1, separate combine
    want_weights = step.workspace.weights.clone()
    want = combine_experts(routed, shared, gate)
    res_b = residual.clone()
    want_norm = add_norm(want, res_b, norm_w, 1e-6)
    stream = _lib.stream(device)
    ws = step.workspace
    outs = []
    for res in (None, residual.clone()):
        weights = torch.full_like(want_weights, 9.0)
        out = torch.empty((rows, h), dtype=torch.bfloat16, device=device)
        _lib.call("d3_combine_route_logits", ws.down.data_ptr(), logits.data_ptr(),
                  dtype_code(logits_dtype), logits.stride(0), e, 8, weights.data_ptr(),
                  dtype_code(weights_dtype), shared.data_ptr(), gate.data_ptr(), gate.stride(0),
                  None if res is None else res.data_ptr(), norm_w.data_ptr(), 1e-6, rows, h,
                  out.data_ptr(), stream)
        outs.append((out, res, weights))
    torch.cuda.synchronize()
    (plain, _, w1), (normed, res_a, w2) = outs
    assert torch.equal(w1, want_weights) and torch.equal(w2, want_weights)
    assert torch.equal(plain.view(torch.int16), want.view(torch.int16))
    assert torch.equal(res_a.view(torch.int16), res_b.view(torch.int16))
    assert torch.equal(normed.view(torch.int16), want_norm.view(torch.int16))


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
