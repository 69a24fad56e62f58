"""``moe_atomic.atomic_down`` (reference ``moe_atomic.py:60-78``) on the
reference's sorted-tile layout, against the oracle's FC2 + rank-order
combine, through the C ABI."""

import numpy as np
import pytest
import torch

from helpers import CONTRACTION, EXACT, assert_bf16_close, np_bf16, oracle_weights
from oracle import moe as om
from oracle.numerics import bf16_to_f32, f32_to_bf16

pytestmark = pytest.mark.gpu


def _experts(device, experts, hidden, inter, seed):
    from drama3_amd import workloads as wl

    gen = torch.Generator("cpu").manual_seed(seed)
    return wl.make_experts(gen, experts, hidden, inter).to(device)


@pytest.mark.parametrize("tokens,block_m,experts,hidden,inter", [
    (37, 16, 16, 1024, 256), (300, 64, 128, 2048, 768), (300, 128, 128, 2048, 768),
    (5, 32, 8, 512, 512)])
def test_atomic_down_matches_oracle(device, tokens, block_m, experts, hidden, inter):
    from drama3_amd.kernels import sort_routes
    from drama3_amd.moe_atomic import atomic_down

    rng = np.random.default_rng(tokens * 7 + block_m)
    dev_ex = _experts(device, experts, hidden, inter, seed=tokens)
    wt = oracle_weights(dev_ex)
    logits = rng.standard_normal((tokens, experts)).astype(np.float32)
    weights, ids = om.route(bf16_to_f32(f32_to_bf16(logits)))
    # SwiGLU activations by pair, as native_moe hands them to atomic_down
    gate_up = f32_to_bf16(rng.standard_normal((tokens * 8, 2 * inter)).astype(np.float32))
    act_q, act_s = om.silu_mul_quant(gate_up)
    ids_dev = torch.from_numpy(ids).to(device)
    _, _, total, sorted_ids, expert_ids, _ = sort_routes(ids_dev, experts, block_m)
    x = torch.from_numpy(act_q).to(device).view(torch.float8_e4m3fn)
    scales = torch.from_numpy(act_s).to(device)
    routing = torch.from_numpy(weights.view(np.int16)).view(torch.bfloat16).to(device).flatten()
    out = atomic_down(x, scales, dev_ex, routing, sorted_ids, expert_ids, total, tokens, block_m, 1)
    out2 = atomic_down(x, scales, dev_ex, routing, sorted_ids, expert_ids, total, tokens, block_m, 1)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))  # deterministic
    expected = om.weighted_combine(om.expert_fc2(act_q, act_s, ids, wt), bf16_to_f32(weights))
    tol = EXACT if block_m <= 64 else CONTRACTION
    assert_bf16_close(np_bf16(out), expected, **tol)


def test_atomic_down_rejects_bad_layouts(device):
    from drama3_amd.moe_atomic import atomic_down

    dev_ex = _experts(device, 4, 512, 256, seed=1)
    x = torch.zeros((16, 256), dtype=torch.float8_e4m3fn, device=device)
    s = torch.ones((16, 2), dtype=torch.float32, device=device)
    r = torch.zeros(16, dtype=torch.bfloat16, device=device)
    ids = torch.zeros(32, dtype=torch.int32, device=device)
    eids = torch.zeros(2, dtype=torch.int32, device=device)
    total = torch.zeros(1, dtype=torch.int32, device=device)
    with pytest.raises(ValueError):
        atomic_down(x, s, dev_ex, r, ids, eids, total, 2, 24, 1)  # block_m
    with pytest.raises(ValueError):
        atomic_down(x, s, dev_ex, r, ids, eids, total, 3, 16, 1)  # pairs != 8 T
    with pytest.raises(TypeError):
        atomic_down(x.view(torch.uint8), s, dev_ex, r, ids, eids, total, 2, 16, 1)
