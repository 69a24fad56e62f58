"""``prepare_moe_input`` with the reference's signature and contract
(``src/drama3/moe_input.py:40-79``), on the MI355X quantisation kernel."""

from __future__ import annotations

import torch

from . import _lib
from ._lib import DTYPE_I32, DTYPE_I64, call, ptr
from .pipeline import dtype_code, require_cuda


def prepare_moe_input(x, router, *, row_slots=None, padding_start=None):
    """Per-128 FP8 activation quantisation, transposed scales and fp32 router
    logits in one launch.  Rows whose slot is >= ``padding_start`` take row
    0's routing; quantisation stays per row (``moe_input.py:40-46``).

    Returns ``(q float8_e4m3fn [T, H], scales float32 [H/128, T],
    logits float32 [T, E])``.
    """
    require_cuda(x, router, row_slots)
    if x.dim() != 2 or router.dim() != 2 or x.shape[1] % 128 or router.shape[0] != len(x):
        raise ValueError("Expected x [T, H] with H % 128 == 0 and router [T, E]")
    if x.stride(1) != 1 or router.stride(1) != 1:
        raise ValueError("Channel strides must be contiguous")
    if x.dtype != torch.bfloat16:
        raise TypeError("x must be bfloat16")
    if router.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("router must be bfloat16 or float32")
    if (row_slots is None) != (padding_start is None):
        raise ValueError("Reserved padding routing requires both row_slots and padding_start")
    if row_slots is not None:
        if (
            row_slots.shape != (len(x),)
            or row_slots.stride(0) != 1
            or row_slots.device != x.device
            or row_slots.dtype not in (torch.int32, torch.int64)
        ):
            raise ValueError("Expected one contiguous integer slot per MoE row on the same device")
        if not isinstance(padding_start, int) or padding_start <= 0:
            raise ValueError("padding_start must be a positive reserved-slot boundary")
    if x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    rows, hidden = x.shape
    experts = router.shape[1]
    q = torch.empty(x.shape, device=x.device, dtype=torch.float8_e4m3fn)
    scales = torch.empty((hidden // 128, rows), device=x.device, dtype=torch.float32)
    logits = torch.empty((rows, experts), device=x.device, dtype=torch.float32)
    slots_dtype = 0
    if row_slots is not None:
        slots_dtype = DTYPE_I64 if row_slots.dtype == torch.int64 else DTYPE_I32
    call("d3_prepare_moe_input", ptr(x), x.stride(0), ptr(router), dtype_code(router.dtype),
         router.stride(0), rows, hidden, experts, ptr(row_slots), slots_dtype,
         int(padding_start or 0), ptr(q), ptr(scales), ptr(logits), _lib.stream(x.device))
    return q, scales, logits


def quantize_groups(x: torch.Tensor, width: int | None = None):
    """Per-row per-128 e4m3 quantisation in the native scale layout: the
    contract of Fish's ``quantize_groups(quant_kernel, x, H)`` as called at
    ``kernels.py:332,732`` -> ``(q [T, H] e4m3, scales [T, H/128] f32)``."""
    require_cuda(x)
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be 2-D with unit column stride")
    if x.dtype != torch.bfloat16:
        raise TypeError("x must be bfloat16")
    width = x.shape[1] if width is None else width
    if width != x.shape[1] or width % 128:
        raise ValueError("width must equal the row width and be a multiple of 128")
    if x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    rows = len(x)
    q = torch.empty((rows, width), device=x.device, dtype=torch.float8_e4m3fn)
    scales = torch.empty((rows, width // 128), device=x.device, dtype=torch.float32)
    call("d3_quantize_rows", ptr(x), x.stride(0), rows, width, None, None, ptr(q), ptr(scales), 0,
         _lib.stream(x.device))
    return q, scales
