"""MoE operators with the names and signatures of the reference's
``src/drama3/kernels.py``, running on the MI355X HIP kernels.

Shapes are generalised over (experts, hidden, intermediate); the reference
hard-codes 256 / 2048 / 512.  Tuning knobs of the reference (``up_rows``,
``block_m`` ...) are validated and otherwise have no effect: there is one
kernel family, tiled for CDNA4.  Errors follow the reference: ``ValueError``
for shape / device / contract violations, ``TypeError`` for dtypes.
"""

from __future__ import annotations

import torch

from . import _lib
from ._lib import call, ptr
from .pipeline import (WIDE_SORT_PAIRS, MoEWorkspace, Shape, by_pair_suited, dtype_code,
                       grouped_supported, require_cuda)

TOP_K = 8

# Workspaces of the eager entry points, reused across calls with the same
# shape, options, device and current stream (calls on one stream run in
# order, so they never share buffers concurrently); the oldest is dropped
# past _MAX_WORKSPACES.  Outputs are always fresh tensors.
#
# Under graph capture a workspace is built fresh and never cached: the
# constants a workspace fills when it is built (the live row count, the
# fused-sort ticket) would otherwise be written only inside the graph that
# built it, and every graph shares torch's capture stream, so a second graph
# of the same shape replayed before the first would read them unwritten.
_MAX_WORKSPACES = 16
_workspaces: dict = {}


def _workspace(shape: Shape, device: torch.device, **options) -> MoEWorkspace:
    if device.type == "cuda" and torch.cuda.is_current_stream_capturing():
        return MoEWorkspace(shape, device, **options)
    stream = torch.cuda.current_stream(device).cuda_stream if device.type == "cuda" else 0
    key = (str(device), stream, shape.rows, shape.num_experts, shape.hidden, shape.intermediate,
           shape.top_k, tuple(sorted(options.items())))
    ws = _workspaces.get(key)
    if ws is None:
        if len(_workspaces) >= _MAX_WORKSPACES:
            _workspaces.pop(next(iter(_workspaces)))
        ws = _workspaces[key] = MoEWorkspace(shape, device, **options)
    return ws


def check_experts(experts, hidden: int | None = None):
    """``experts`` exposes w13_weight [E,2I,H] e4m3, w13_scale_inv [E,2I/128,H/128],
    w2_weight [E,H,I] e4m3, w2_scale_inv [E,H/128,I/128] (``kernels.py:334-351``)."""
    w13, s13, w2, s2 = (experts.w13_weight, experts.w13_scale_inv, experts.w2_weight,
                        experts.w2_scale_inv)
    require_cuda(w13, s13, w2, s2)
    if w13.dtype != torch.float8_e4m3fn or w2.dtype != torch.float8_e4m3fn:
        raise TypeError("expert weights must be float8_e4m3fn")
    if s13.dtype != torch.float32 or s2.dtype != torch.float32:
        raise TypeError("expert block scales must be float32")
    e, two_i, h = w13.shape
    i = two_i // 2
    if hidden is not None and h != hidden:
        raise ValueError(f"expert hidden size {h} != activation width {hidden}")
    if (w2.shape != (e, h, i) or s13.shape != (e, two_i // 128, h // 128)
            or s2.shape != (e, h // 128, i // 128) or h % 128 or i % 128):
        raise ValueError("expert weights do not follow the [gate; up] / down 128x128 block layout")
    for t in (w13, s13, w2, s2):
        if not t.is_contiguous():
            raise ValueError("expert tensors must be contiguous")
    return e, h, i


def _check_rows(x: torch.Tensor, name: str = "x") -> None:
    require_cuda(x)
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError(f"{name} must be 2-D with unit column stride")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16")


def route(logits: torch.Tensor):
    """``route`` (``kernels.py:379-383``): ``(weights [T,8] logits.dtype,
    indices [T,8] int64)``; bf16 value ranks first, ties to the lower expert."""
    require_cuda(logits)
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be 2-D with unit column stride")
    if logits.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("logits must be bfloat16 or float32")
    rows, experts = logits.shape
    indices = torch.empty((rows, TOP_K), dtype=torch.int64, device=logits.device)
    weights = torch.empty((rows, TOP_K), dtype=logits.dtype, device=logits.device)
    call("d3_route", ptr(logits), dtype_code(logits.dtype), logits.stride(0), rows, experts,
         TOP_K, None, None, None, ptr(indices), ptr(weights), dtype_code(weights.dtype),
         _lib.stream(logits.device))
    return weights, indices


def _routed(x, topk_ids, topk_weights, experts, block_m: int = 16):
    _check_rows(x)
    require_cuda(topk_ids, topk_weights)
    e, h, i = check_experts(experts, x.shape[1])
    if topk_ids.dim() != 2 or topk_ids.shape != topk_weights.shape or len(topk_ids) != len(x):
        raise ValueError("topk_ids / topk_weights must be [T, k] for the T rows of x")
    if topk_ids.dtype not in (torch.int32, torch.int64):
        raise TypeError("topk_ids must be int32 or int64")
    if topk_weights.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("topk_weights must be bfloat16 or float32")
    if block_m not in (16, 32, 64, 128):
        raise ValueError("block_m must be 16, 32, 64 or 128")
    rows, top_k = topk_ids.shape
    out = torch.empty((rows, h), dtype=torch.bfloat16, device=x.device)
    if rows == 0:
        return out
    ws = _workspace(Shape(rows, e, h, i, top_k), x.device, tile=block_m,
                    item_rows=max(block_m, 128) if rows > 128 else None)
    ids, weights = topk_ids.contiguous(), topk_weights.contiguous()
    if x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    return ws.experts_forward(x, ids, weights, experts, out=out)


def small_batch_moe(x, topk_ids, topk_weights, experts, up_rows=4, down_rows=4, down_warps=8):
    """``small_batch_moe`` (``kernels.py:325-357``): quantise x per 128 group,
    FC1 -> bf16 gate|up, SwiGLU + FP8 requant, FC2 in fp32, routing-weighted
    sum over the top-k ranks -> bf16 [T, H]."""
    for value in (up_rows, down_rows, down_warps):
        if not isinstance(value, int) or value <= 0:
            raise ValueError("tile knobs must be positive integers")
    return _routed(x, topk_ids, topk_weights, experts)


def native_moe(x, topk_ids, topk_weights, experts, block_m=16, group_m=1, atomic=False):
    """``native_moe`` (``kernels.py:702-779``): device-only routing layout
    (histogram, padded offsets, stable scatter) then the grouped FP8 GEMMs.
    ``atomic`` selected the reference's fp32-atomic down projection
    (``moe_atomic.atomic_down``, also provided with its signature); here the
    reduction is always the deterministic rank-ordered one, which
    ``atomic_down`` computes as well."""
    if not isinstance(group_m, int) or group_m < 1:
        raise ValueError("group_m must be a positive integer")
    return _routed(x, topk_ids, topk_weights, experts, block_m)


def sort_routes(topk_ids: torch.Tensor, num_experts: int, block_m: int = 16):
    """``expert_counts_kernel`` + ``expert_offsets_kernel`` +
    ``expert_scatter_kernel`` as launched by ``native_moe`` (``kernels.py:710-731``).

    Returns ``(counts [E], starts [E], total [1], sorted_ids [max_rows],
    expert_ids [max_rows / block_m], inverse [pairs])`` int32; entries of
    ``sorted_ids`` from ``total`` on hold the sentinel ``pairs`` and those of
    ``expert_ids`` hold -1 (the reference leaves them uninitialised).
    """
    require_cuda(topk_ids)
    if topk_ids.dim() != 2:
        raise ValueError("topk_ids must be [T, k]")
    if topk_ids.dtype not in (torch.int32, torch.int64):
        raise TypeError("topk_ids must be int32 or int64")
    lib = _lib.load()
    ids = topk_ids.contiguous()
    rows, top_k = ids.shape
    pairs = rows * top_k
    max_rows = lib.d3_max_sorted_rows(pairs, num_experts, block_m)
    dev = ids.device
    i32 = dict(dtype=torch.int32, device=dev)
    counts, starts = torch.empty(num_experts, **i32), torch.empty(num_experts, **i32)
    total = torch.empty(1, **i32)
    sorted_ids = torch.empty(max_rows, **i32)
    expert_ids = torch.empty(max_rows // block_m, **i32)
    inverse = torch.empty(max(pairs, 1), **i32)
    args = (ptr(ids), dtype_code(ids.dtype), rows, None, top_k, num_experts, block_m, ptr(counts),
            ptr(starts), ptr(total), ptr(sorted_ids), ptr(expert_ids), max_rows, ptr(inverse),
            block_m, None, 0, None, None)
    if pairs > WIDE_SORT_PAIRS:  # prefill-sized: the ranking spread over many workgroups
        scratch = torch.empty(lib.d3_sort_wide_scratch_ints(rows, top_k, num_experts), **i32)
        call("d3_sort_routes_wide", *args, ptr(scratch), scratch.numel(), _lib.stream(dev))
    else:
        call("d3_sort_routes", *args, _lib.stream(dev))
    return counts, starts, total, sorted_ids, expert_ids, inverse[:pairs]


def silu_mul(projected: torch.Tensor) -> torch.Tensor:
    """``silu_mul`` (``kernels.py:386-402``): bf16 [T, 2W] -> bf16 [T, W]."""
    _check_rows(projected, "projected")
    width = projected.shape[-1] // 2
    out = torch.empty((len(projected), width), dtype=projected.dtype, device=projected.device)
    call("d3_silu_mul", ptr(projected), projected.stride(0), len(projected), width, ptr(out),
         _lib.stream(projected.device))
    return out


def _gate_args(gate: torch.Tensor, rows: int):
    require_cuda(gate)
    if gate.dtype != torch.bfloat16:
        raise TypeError("gate must be bfloat16")
    if gate.dim() == 2:
        if gate.shape[0] != rows:
            raise ValueError("one gate value per row is required")
        return gate.stride(0)
    if gate.dim() == 1 and gate.shape[0] == rows:
        return gate.stride(0)
    raise ValueError("gate must be [T] or [T, >=1]")


def combine_experts(routed, shared, gate):
    """``combine_experts`` (``kernels.py:427-445``) as the reference runs it:
    ``bf16(shared * bf16(sigmoid(gate)) + routed)`` in one single-rounding
    bf16 FMA (the contraction ``kernels.py:465-466`` describes), so
    ``add_norm(combine_experts(...))`` equals ``combine_experts_add_norm``.
    ``routed`` and ``shared`` are read as contiguous rows."""
    _check_rows(routed, "routed")
    _check_rows(shared, "shared")
    if routed.shape != shared.shape:
        raise ValueError("routed and shared must have the same shape")
    routed, shared = routed.contiguous(), shared.contiguous()
    stride = _gate_args(gate, len(routed))
    out = torch.empty_like(routed)
    call("d3_combine_experts", ptr(routed), ptr(shared), ptr(gate), stride, routed.shape[0],
         routed.shape[1], ptr(out), _lib.stream(routed.device))
    return out


def combine_experts_add_norm(routed, shared, gate, residual, weight, epsilon):
    """``combine_experts_add_norm`` (``kernels.py:483-499``); updates
    ``residual`` in place and returns the (1 + w) RMS-normalised rows."""
    return _combine_norm(routed, shared, gate, None, residual, weight, epsilon)


def combine_experts_add_norm_inverse(routed, shared, gate, inverse, residual, weight, epsilon):
    """``combine_experts_add_norm_inverse`` (``kernels.py:539-556``): row r
    reads MoE row ``inverse[r]``; output has the residual's rows."""
    require_cuda(inverse)
    if inverse.dtype != torch.int64 or inverse.dim() != 1 or len(inverse) != len(residual):
        raise ValueError("inverse must be int64 [len(residual)]")
    return _combine_norm(routed, shared, gate, inverse.contiguous(), residual, weight, epsilon)


def _combine_norm(routed, shared, gate, inverse, residual, weight, epsilon):
    for name, t in (("routed", routed), ("shared", shared), ("residual", residual)):
        _check_rows(t, name)
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    require_cuda(weight)
    if routed.shape != shared.shape or residual.shape[1] != routed.shape[1]:
        raise ValueError("routed, shared and residual widths must match")
    if inverse is None and residual.shape != routed.shape:
        raise ValueError("residual must match routed rows")
    if weight.shape != (routed.shape[1],) or weight.dtype != torch.bfloat16:
        raise ValueError("weight must be bf16 [width]")
    stride = _gate_args(gate, len(routed))
    weight = weight.contiguous()
    out = torch.empty_like(residual)
    call("d3_combine_experts_add_norm", ptr(routed), ptr(shared), ptr(gate), stride, ptr(inverse),
         ptr(residual), ptr(weight), float(epsilon), residual.shape[0],
         residual.shape[1], ptr(out), _lib.stream(routed.device))
    return out


def add_norm(x, residual, weight, epsilon):
    """``add_norm`` (``kernels.py:405-424``): residual <- bf16(x + residual);
    returns bf16 RMSNorm(residual) * (1 + w)."""
    _check_rows(x)
    _check_rows(residual, "residual")
    if x.shape != residual.shape or not x.is_contiguous() or not residual.is_contiguous():
        raise ValueError("x and residual must be contiguous and of the same shape")
    weight = weight.contiguous()
    out = torch.empty_like(x)
    call("d3_add_norm", ptr(x), ptr(residual), ptr(weight), float(epsilon),
         x.shape[0], x.shape[1], ptr(out), _lib.stream(x.device))
    return out


def routed_moe(x, router, experts, decode=True, *, row_slots=None, padding_start=None):
    """``DramaModel.routed_moe`` (``model.py:520-583``) as a function of the
    layer's inputs: top-8 routing of ``router`` [T, E], the routed FP8 SwiGLU
    experts and the weighted combine -> bf16 [T, H].

    The reference dispatches three numerically different backends (Triton
    GEMV for <= 8 rows, Fish's sorted GEMM for native prefill, FlashInfer for
    decode batches above 8 rows); here every batch runs the same MI355X path
    with ``route_kernel``'s ranking rule (``kernels.py:364-368``).  ``decode``
    is accepted for the signature.  With ``row_slots`` / ``padding_start``
    (both or neither), rows whose slot is >= ``padding_start`` take row 0's
    routing, the reserved-padding router of ``moe_input.py:31-37``.
    """
    _check_rows(x)
    require_cuda(router)
    if router.dim() != 2 or len(router) != len(x) or router.stride(1) != 1:
        raise ValueError("router must be [T, E] with unit column stride, one row per x row")
    if router.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("router must be bfloat16 or float32")
    if (row_slots is None) != (padding_start is None):
        raise ValueError("Reserved padding routing requires both row_slots and padding_start")
    e, h, i = check_experts(experts, x.shape[1])
    if router.shape[1] != e:
        raise ValueError(f"router has {router.shape[1]} experts, weights have {e}")
    rows = len(x)
    out = torch.empty((rows, h), dtype=torch.bfloat16, device=x.device)
    if rows == 0:
        return out
    logits = router
    if row_slots is not None:
        # The reference's decode path (model.py:543-552): prepare_moe_input
        # applies the padding rule to the fp32 logits in its fused launch.
        from .moe_input import prepare_moe_input

        _, _, logits = prepare_moe_input(x, router, row_slots=row_slots,
                                         padding_start=padding_start)
    if x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    by_pair = by_pair_suited(rows, e, TOP_K) and grouped_supported(h, i)
    ws = _workspace(Shape(rows, e, h, i, TOP_K), x.device,
                    item_rows=128 if rows > 128 else None, by_pair=by_pair)
    return ws.forward(x, logits, experts, out=out)
