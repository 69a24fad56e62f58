"""Pin the PyTorch-CPU restatement the bench times as its CPU baseline
(``oracle/cpu_step.py``) against the numpy oracle: routing ids and
quantised bytes identical, outputs within the exact-path tolerance (it sums
the expert GEMMs in float32 where the oracle uses float64).  CPU only."""

import numpy as np
import pytest
import torch

from helpers import EXACT, assert_bf16_close, np_bf16, np_u8, oracle_weights
from oracle import cpu_step
from oracle import moe as om
from oracle.numerics import bf16_to_f32


def test_route_and_quantisation_match_the_oracle():
    rng = np.random.default_rng(31)
    logits = torch.from_numpy(rng.standard_normal((40, 128)).astype(np.float32)).to(torch.bfloat16)
    logits[3, :] = 0.5  # all-equal row: lower expert index wins every tie
    weights, ids = cpu_step.route(logits.float())
    want_w, want_ids = om.route(logits.float().numpy())
    assert np.array_equal(ids.numpy(), want_ids)
    assert np.array_equal(np_bf16(weights.to(torch.bfloat16)), want_w)
    x = torch.from_numpy(rng.standard_normal((16, 1024)).astype(np.float32) * 4)
    x[2] = 0.0
    q, s = cpu_step.quantize_rows(x)
    want_q, want_s = om.quantize_rows(x.numpy())
    assert np.array_equal(np_u8(q.view(torch.uint8)), want_q) and np.array_equal(s.numpy(), want_s)


@pytest.mark.parametrize("config,rows", [(1, None), (3, 24), (2, 10), (4, 8)])
def test_step_matches_the_oracle(config, rows):
    from drama3_amd import workloads as wl

    work = wl.CONFIGS[config]()
    x, logits = work.steps[0].packed()
    if rows is not None:
        x, logits = x[:rows], logits[:rows]
    got = cpu_step.moe_step(x, logits, work.experts, work.shared)
    weights, ids = om.route(logits.float().numpy())
    want = om.expert_ffn(np_bf16(x), ids, weights, oracle_weights(work.experts))
    if work.shared is not None:
        sh = work.shared
        dense = om.dense_ffn(np_bf16(x), np_u8(sh.w13_weight[0]), sh.w13_scale_inv[0].numpy(),
                             np_u8(sh.w2_weight[0]), sh.w2_scale_inv[0].numpy())
        want = om.add_shared(want, dense)
    # float32 sums flip about 3e-4 of the bf16 FC1 outputs against the
    # oracle's float64 ones, each possibly moving one activation code
    assert_bf16_close(np_bf16(got), want, **EXACT)
    assert np.all(np.isfinite(bf16_to_f32(np_bf16(got))))
