"""PyTorch-CPU restatement of the MoE step, timed as the bench's CPU baseline.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): ``bench.py``'s
``cpu_baseline`` leg times it on the host cores and ``tests/`` pins it
against ``oracle.moe``.  It is the same algorithm as ``oracle.moe`` (the
reference's ``route`` ``kernels.py:360-383``, per-128 quantisation
``moe_input.py:24-27``, FC1 -> bf16 ``kernels.py:290-301,333``, SwiGLU +
requant ``kernels.py:344``, FC2 in fp32 and the rank-order weighted combine
``kernels.py:304-322``), written with torch CPU ops so that every stage runs
on ``torch.get_num_threads()`` threads: routing keys and softmax exactly as
the oracle, quantisation through torch's ``float8_e4m3fn`` cast, expert
GEMMs as float32 matmuls of the dequantised operands (the oracle sums in
float64; the two agree to fp32 rounding, which can move a bf16 FC1 output by
one ulp), SwiGLU with the sigmoid in float64 rounded once to fp32.
"""

from __future__ import annotations

import torch

GROUP = 128


def quantize_rows(x: torch.Tensor):
    """x float32 [T, W] -> (codes float8_e4m3fn [T, W], scales float32 [T, W/128])."""
    rows, width = x.shape
    g = x.reshape(rows, width // GROUP, GROUP)
    amax = g.abs().amax(dim=-1, keepdim=True)
    scale = torch.clamp(amax, min=1e-10) / 448.0
    q = torch.clamp(g / scale, -448.0, 448.0).to(torch.float8_e4m3fn)
    return q.reshape(rows, width), scale[..., 0]


def dequantize(q: torch.Tensor, scales: torch.Tensor, row_group: int = 1) -> torch.Tensor:
    """codes [N, K] * scales [N/row_group, K/128] (each scale repeated over
    its block) in float32."""
    full = scales.repeat_interleave(GROUP, dim=-1)
    if row_group > 1:
        full = full.repeat_interleave(row_group, dim=0)
    return q.to(torch.float32) * full


def route(logits: torch.Tensor, top_k: int = 8):
    """The routing-key rule of ``route_kernel`` (bf16 value first, lower
    column on ties) and the float64 softmax of the selected experts,
    renormalised -> (weights float32 [T, k] (bf16 values), ids int64 [T, k])."""
    bits = logits.to(torch.float32).view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    ordered = torch.where(bits >= 0x80000000, bits ^ 0xFFFFFFFF, bits ^ 0x80000000)
    columns = torch.arange(logits.shape[-1], dtype=torch.int64)
    keys = (ordered & 0xFFFF0000) | (65535 - columns)
    ids = torch.topk(keys, top_k, dim=-1).indices
    shifted = (logits - logits.amax(dim=-1, keepdim=True)).to(torch.float32)
    exps = torch.exp(shifted.to(torch.float64))
    selected = torch.gather(exps, -1, ids) / exps.sum(dim=-1, keepdim=True)
    weights = (selected / selected.sum(dim=-1, keepdim=True)).to(torch.float32)
    return weights.to(torch.bfloat16).to(torch.float32), ids


def expert_ffn(x: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor, experts) -> torch.Tensor:
    """Routed expert FFN of the rows x (bf16 [T, H]) -> bf16 [T, H].
    ``experts``: w13_weight [E, 2I, H] / w2_weight [E, H, I] float8_e4m3fn
    with their float32 block scales (the reference's layout)."""
    tokens, top_k = ids.shape
    w13, s13 = experts.w13_weight, experts.w13_scale_inv
    w2, s2 = experts.w2_weight, experts.w2_scale_inv
    inter = w13.shape[1] // 2
    hidden = w13.shape[2]
    q, xs = quantize_rows(x.to(torch.float32))
    x_dq = dequantize(q, xs)
    flat = ids.reshape(-1)
    order = torch.argsort(flat, stable=True)
    counts = torch.bincount(flat, minlength=w13.shape[0]).tolist()
    down = torch.empty((tokens * top_k, hidden), dtype=torch.float32)
    start = 0
    for e, count in enumerate(counts):
        if count == 0:
            continue
        pairs = order[start:start + count]
        start += count
        gate_up = x_dq[pairs // top_k] @ dequantize(w13[e], s13[e], GROUP).T
        gate_up = gate_up.to(torch.bfloat16).to(torch.float32)
        gate, up = gate_up[:, :inter], gate_up[:, inter:]
        sig = (1.0 / (1.0 + torch.exp(-gate.to(torch.float64)))).to(torch.float32)
        act = (gate * sig) * up
        aq, ascale = quantize_rows(act)
        down[pairs] = dequantize(aq, ascale) @ dequantize(w2[e], s2[e], GROUP).T
    y = down.reshape(tokens, top_k, hidden).to(torch.float64)
    out = (y * weights.to(torch.float64)[:, :, None]).sum(dim=1)
    return out.to(torch.float32).to(torch.bfloat16)


def moe_step(x: torch.Tensor, logits: torch.Tensor, experts, shared=None) -> torch.Tensor:
    """Route + experts for packed rows x (bf16 [T, H]) and their logits; a
    dense shared expert (config 4), when given, is added as
    ``bf16(routed + bf16(shared))``."""
    weights, ids = route(logits.to(torch.float32))
    out = expert_ffn(x, ids, weights, experts)
    if shared is not None:
        ones = torch.ones((len(x), 1), dtype=torch.float32)
        zero = torch.zeros((len(x), 1), dtype=torch.int64)
        dense = expert_ffn(x, zero, ones, shared)
        out = (out.to(torch.float32) + dense.to(torch.float32)).to(torch.bfloat16)
    return out
