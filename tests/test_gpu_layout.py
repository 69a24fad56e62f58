"""Fragment-major expert weights (d3_pack_expert_weights): the packed bytes
are the documented permutation of the checkpoint layout, and every GEMM
result computed from them is bit-identical to the checkpoint-layout result
(the load addresses change, the arithmetic does not)."""

import numpy as np
import pytest
import torch

from helpers import EXACT, assert_bf16_close, np_bf16, np_f32, np_u8, oracle_weights
from oracle import moe as om

pytestmark = pytest.mark.gpu


def fragment_major(w: np.ndarray) -> np.ndarray:
    """[E, N, K] -> tile t, K block kb, half h, lane l = 16 g + r, 16 bytes:
    byte b of row 16 t + r at column 128 kb + 64 h + 16 g + b."""
    e, n, k = w.shape
    blocks = w.reshape(e, n // 16, 16, k // 128, 2, 4, 16)  # e t r kb h g b
    return blocks.transpose(0, 1, 3, 4, 5, 2, 6).reshape(e, n, k)


@pytest.mark.parametrize("e,n,k", [(1, 16, 128), (3, 48, 256), (4, 1536, 2048), (5, 2048, 768)])
def test_pack_matches_permutation(device, e, n, k):
    from drama3_amd.expert_weights import pack_expert_weights

    gen = torch.Generator("cpu").manual_seed(n + k)
    w = torch.randint(0, 256, (e, n, k), generator=gen, dtype=torch.uint8)
    packed = pack_expert_weights(w.to(device))
    torch.cuda.synchronize()
    assert np.array_equal(packed.cpu().numpy(), fragment_major(w.numpy()))


def test_pack_rejects_bad_shapes(device):
    from drama3_amd.expert_weights import pack_expert_weights

    with pytest.raises(ValueError, match="multiple of 16"):
        pack_expert_weights(torch.zeros((2, 24, 128), dtype=torch.uint8, device=device))
    with pytest.raises(ValueError, match="K=200"):
        pack_expert_weights(torch.zeros((2, 32, 200), dtype=torch.uint8, device=device))


EXACT_ALWAYS = 1 << 30
FP8_ALWAYS = -1


@pytest.mark.parametrize("path", ["exact", "fp8"])
@pytest.mark.parametrize("hidden,inter,experts,tokens", [(1024, 256, 16, 40), (2048, 768, 128, 48),
                                                         (512, 512, 8, 200)])
def test_packed_stages_bit_identical(device, hidden, inter, experts, tokens, path):
    from drama3_amd.expert_weights import prepare_experts
    from drama3_amd.pipeline import MoEWorkspace, Shape
    from drama3_amd.workloads import make_experts

    gen = torch.Generator("cpu").manual_seed(tokens)
    ex = make_experts(gen, experts, hidden, inter)
    x = torch.randn((tokens, hidden), generator=gen).to(torch.bfloat16).to(device)
    logits = torch.randn((tokens, experts), generator=gen).to(torch.bfloat16).to(device)
    plain = ex.to(device)
    packed = prepare_experts(ex.to(device))
    results = []
    for weights in (plain, packed):
        ws = MoEWorkspace(Shape(tokens, experts, hidden, inter), device,
                          exact_routes=EXACT_ALWAYS if path == "exact" else FP8_ALWAYS)
        ws.route(logits)
        ws.quantize(x)
        ws.sort()
        ws.fc1(weights)
        ws.activation()
        ws.fc2(weights)
        out = ws.combine()
        torch.cuda.synchronize()
        total = int(ws.total.item())
        valid = ws.sorted_ids.cpu().numpy()[:total] < ws.shape.pairs
        results.append((np_bf16(ws.gate_up)[:total][valid], np_u8(ws.act)[:total][valid],
                        np_f32(ws.down), np_bf16(out)))
    for a, b in zip(*results):
        assert np.array_equal(a, b)


def test_packed_decode_step_matches_oracle(device):
    """Config 2 decode step on packed weights: oracle parity (exact path) and
    the same bytes as the checkpoint layout."""
    from drama3_amd import workloads
    from drama3_amd.expert_weights import prepare_experts
    from drama3_amd.pipeline import DecodeStep

    w = workloads.config2()
    step = w.steps[0]
    occ = step.occupancy.to(device)
    xs, ls = step.x_slots.to(device), step.logits_slots.to(device)
    outs = []
    for experts in (w.experts.to(device), prepare_experts(w.experts.to(device))):
        ds = DecodeStep(64, w.num_experts, w.hidden, w.intermediate, device=device)
        outs.append(ds(occ, xs, ls, experts))
    torch.cuda.synchronize()
    n = int(ds.count.item())
    assert torch.equal(outs[0][:n], outs[1][:n])
    active, _ = om.compact_slots(step.occupancy.numpy())
    weights, ids = om.route(np_f32(step.logits_slots)[active])
    expected = om.expert_ffn(np_bf16(step.x_slots)[active], ids, weights, oracle_weights(w.experts))
    assert_bf16_close(np_bf16(outs[1])[:n], expected, **EXACT)


def test_stale_packed_copy_is_not_used(device):
    from drama3_amd.expert_weights import (LAYOUT_FRAGMENT, LAYOUT_REFERENCE, fc1_operands,
                                           fc2_operands, prepare_experts)
    from drama3_amd.workloads import make_experts

    ex = prepare_experts(make_experts(torch.Generator("cpu").manual_seed(0), 4, 256, 128).to(device))
    assert fc1_operands(ex)[2] == LAYOUT_FRAGMENT and fc2_operands(ex)[2] == LAYOUT_FRAGMENT
    ex.w13_weight.view(torch.uint8).add_(1)  # modified in place: packed copy is stale
    assert fc1_operands(ex)[2] == LAYOUT_REFERENCE
    assert fc1_operands(ex)[0] is ex.w13_weight
    assert fc2_operands(ex)[2] == LAYOUT_FRAGMENT
