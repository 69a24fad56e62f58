"""``atomic_down`` with the reference's signature (``src/drama3/moe_atomic.py:60-78``).

The reference's experimental down projection takes the SwiGLU activations by
pair, ``native_moe``'s sorted tiles and the routing weights, and atomically
adds each route's weighted FC2 row into its token's fp32 row.  Here the same
inputs run the library's FC2 over the caller's tiles and the rank-order
weighted combine: the sum is deterministic (the reference's atomic order is
not), so results equal ``native_moe``'s within the stated FP8 tolerance and
are identical from run to run.
"""

from __future__ import annotations

import torch

from . import _lib
from ._lib import call, ptr
from .expert_weights import fc2_operands
from .pipeline import EXACT_ROUTES, dtype_code, require_cuda

TOP_K = 8


def atomic_down(x, scales, experts, routing, ids, expert_ids, total, tokens, block_m, group_m):
    """Down projection of ``native_moe(..., atomic=True)``.

    x: e4m3 activations [pairs, I] by pair; scales: f32 [pairs, I/128];
    experts: ``w2_weight`` [E, H, I] e4m3 + ``w2_scale_inv``; routing: the
    flattened top-8 weights [pairs] (bf16 or f32); ids: the sorted pair list
    [max_rows] (sentinel ``pairs``); expert_ids: expert of each ``block_m``
    tile; total: int32 [1] sorted rows in use; tokens: T (pairs = 8 T).
    Returns bf16 [T, H].  ``group_m`` is a tile-order knob of the reference
    and is validated only.
    """
    require_cuda(x, scales, routing, ids, expert_ids, total)
    if x.dtype != torch.float8_e4m3fn:
        raise TypeError("x must be float8_e4m3fn activations")
    if scales.dtype != torch.float32:
        raise TypeError("scales must be float32")
    if routing.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("routing must be bfloat16 or float32")
    for name, t in (("ids", ids), ("expert_ids", expert_ids), ("total", total)):
        if t.dtype != torch.int32:
            raise TypeError(f"{name} must be int32")
    if not isinstance(block_m, int) or block_m not in (16, 32, 64, 128):
        raise ValueError("block_m must be 16, 32, 64 or 128")
    if not isinstance(group_m, int) or group_m < 1:
        raise ValueError("group_m must be a positive integer")
    w2, s2, layout = fc2_operands(experts)
    num_experts, hidden, inter = experts.w2_weight.shape
    pairs = int(tokens) * TOP_K
    if x.dim() != 2 or x.shape != (pairs, inter) or scales.shape != (pairs, inter // 128):
        raise ValueError(f"x / scales must be [{pairs}, {inter}] / [{pairs}, {inter // 128}] by pair")
    if routing.numel() != pairs or ids.dim() != 1 or ids.numel() % block_m:
        raise ValueError("routing must hold one weight per pair and ids whole block_m tiles")
    if expert_ids.numel() < ids.numel() // block_m or total.numel() != 1:
        raise ValueError("expert_ids must name every tile of ids; total is one int32")
    out = torch.empty((tokens, hidden), dtype=torch.bfloat16, device=x.device)
    if tokens == 0:
        return out
    x, scales = x.contiguous(), scales.contiguous()
    ids, expert_ids = ids.contiguous(), expert_ids.contiguous()
    routing = routing.contiguous().view(tokens, TOP_K)
    dev, stream = x.device, _lib.stream(x.device)
    max_rows = ids.numel()
    max_tiles = max_rows // block_m
    i32 = dict(dtype=torch.int32, device=dev)
    items = torch.empty((max(max_tiles, 1), 4), **i32)
    num_items = torch.empty(1, **i32)
    call("d3_items_from_tiles", ptr(ids), ptr(expert_ids), ptr(total), block_m, pairs, max_tiles,
         num_experts, ptr(items), ptr(num_items), stream)
    # activation rows and scales in sorted order (the permute the reference
    # does inside its GEMM's loads), then FC2 per tile, stored by pair
    act = torch.empty((max_rows, inter), dtype=torch.uint8, device=dev)
    act_scales = torch.empty((max_rows, inter // 128), dtype=torch.float32, device=dev)
    call("d3_gather_rows", ptr(x), inter, pairs, ptr(ids), ptr(total), max_rows, ptr(act), stream)
    call("d3_gather_rows", ptr(scales), 4 * (inter // 128), pairs, ptr(ids), ptr(total), max_rows,
         ptr(act_scales), stream)
    down = torch.empty((pairs, hidden), dtype=torch.float32, device=dev)
    call("d3_expert_gemm", 1, ptr(w2), ptr(s2), layout, num_experts, hidden, inter, ptr(act),
         ptr(act_scales), ptr(ids), 1, ptr(items), ptr(num_items), max_tiles, block_m,
         EXACT_ROUTES, None, ptr(down), stream)
    call("d3_weighted_combine", ptr(down), ptr(routing), dtype_code(routing.dtype), tokens, TOP_K,
         hidden, None, None, ptr(out), stream)
    return out
