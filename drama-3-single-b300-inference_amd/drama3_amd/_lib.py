"""ctypes binding of the C ABI in ``include/drama3_moe.h``.

The library is the in-tree ``_lib/libdrama3_moe.so`` built by ``_build.py``.
It must be loaded after ``import torch`` so that its ``libamdhip64.so.7``
dependency resolves to the HIP runtime torch already loaded (same SONAME):
the streams and device pointers torch hands over are then valid inside it.

There is no fallback: if the library is missing every operator raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime first, see module docstring)

LIBRARY = Path(__file__).resolve().parent / "_lib" / "libdrama3_moe.so"

D3_OK = 0
D3_ERR_INVALID_ARGUMENT = 1
D3_ERR_UNSUPPORTED = 2
D3_ERR_HIP = 3

DTYPE_BF16 = 0
DTYPE_F32 = 1
DTYPE_I32 = 2
DTYPE_I64 = 3

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float

# name -> (restype, argtypes); mirrors include/drama3_moe.h
SIGNATURES = {
    "d3_abi_version": (_i32, []),
    "d3_last_error": (ctypes.c_char_p, []),
    "d3_check_e4m3_conversion": (_i32, [ctypes.c_uint64, ctypes.c_uint64, _p, _p]),
    "d3_check_epilogue_arithmetic": (_i32, [_i32, ctypes.c_uint64, ctypes.c_uint64, _f32, _p, _p]),
    "d3_compact_slots": (_i32, [_p, _i32, _p, _p, _p]),
    "d3_route": (_i32, [_p, _i32, _i64, _i32, _i32, _i32, _p, _p, _p, _p, _p, _i32, _p]),
    "d3_quantize_rows": (_i32, [_p, _i64, _i32, _i32, _p, _p, _p, _p, _i32, _p]),
    "d3_prepare_moe_input": (
        _i32, [_p, _i64, _p, _i32, _i64, _i32, _i32, _i32, _p, _i32, _i64, _p, _p, _p, _p]),
    "d3_sort_routes": (
        _i32, [_p, _i32, _i32, _p, _i32, _i32, _i32, _p, _p, _p, _p, _p, _i32, _p, _i32, _p,
               _i32, _p, _p, _p]),
    "d3_moe_front": (
        _i32, [_p, _i32, _p, _p, _p, _i64, _p, _i32, _i64, _i32, _p, _p, _i32, _i32, _i32, _p, _p,
               _i32, _p, _p, _i32, _i32, _p, _p, _p, _p, _p, _i32, _p, _p, _i32, _p, _p, _p, _p]),
    "d3_sort_routes_wide": (
        _i32, [_p, _i32, _i32, _p, _i32, _i32, _i32, _p, _p, _p, _p, _p, _i32, _p, _i32, _p,
               _i32, _p, _p, _p, _i64, _p]),
    "d3_sort_wide_scratch_ints": (_i64, [_i32, _i32, _i32]),
    "d3_items_from_tiles": (_i32, [_p, _p, _p, _i32, _i32, _i32, _i32, _p, _p, _p]),
    "d3_gather_rows": (_i32, [_p, _i64, _i64, _p, _p, _i32, _p, _p]),
    "d3_max_sorted_rows": (_i32, [_i32, _i32, _i32]),
    "d3_max_items": (_i32, [_i32, _i32, _i32]),
    "d3_max_items_aligned": (_i32, [_i32, _i32, _i32]),
    "d3_expert_gemm": (
        _i32, [_i32, _p, _p, _i32, _i32, _i32, _i32, _p, _p, _p, _i32, _p, _p, _i32, _i32, _i32,
               _p, _p, _p]),
    "d3_expert_tile_rows": (_i32, [_i32]),
    "d3_grouped_fc1_swiglu": (
        _i32, [_p, _p, _i32, _i32, _i32, _i32, _p, _i64, _p, _p, _i32, _p, _p, _i32, _i32, _p, _p,
               _i32, _i32, _p, _p, _p]),
    "d3_grouped_fc2": (
        _i32, [_p, _p, _i32, _i32, _i32, _i32, _p, _i64, _p, _p, _i32, _p, _p, _i32, _i32, _p, _p,
               _i32, _i32, _i32, _p, _p]),
    "d3_grouped_fc1_swiglu_by_pair": (
        _i32, [_p, _p, _i32, _i32, _i32, _i32, _p, _i64, _p, _p, _i32, _p, _i32, _p, _p, _p, _p,
               _p, _p]),
    "d3_pack_expert_weights": (_i32, [_p, _i32, _i32, _i32, _p, _p]),
    "d3_expert_fc2_swiglu": (
        _i32, [_p, _p, _i32, _i32, _i32, _i32, _p, _p, _i32, _p, _p, _i32, _i32, _i32, _p, _p]),
    "d3_decode_expert_gemm": (
        _i32, [_i32, _p, _p, _i32, _i32, _i32, _p, _p, _p, _i32, _i32, _p, _p, _i32, _p, _p, _p]),
    "d3_decode_route_fc1": (
        _i32, [_p, _p, _i32, _i32, _i32, _p, _i32, _p, _i64, _p, _i32, _i64, _i32, _i32, _p, _p,
               _p, _p, _p]),
    "d3_decode_route_combine": (
        _i32, [_p, _i32, _p, _i32, _i64, _i32, _i32, _i32, _p, _p, _i32, _p, _p]),
    "d3_decode_step": (
        _i32, [_p, _p, _p, _p, _i32, _i32, _i32, _p, _i32, _p, _i64, _p, _i32, _i64, _i32, _i32,
               _p, _p, _i32, _p, _p, _p, _p, _p, _p]),
    "d3_decode_step_static": (
        _i32, [_p, _p, _p, _p, _i32, _i32, _i32, _p, _i32, _p, _i64, _p, _i32, _i64, _i32, _i32,
               _p, _p, _p, _p]),
    "d3_silu_mul_quant": (_i32, [_p, _i32, _i32, _p, _p, _p, _i32, _p, _p, _p]),
    "d3_weighted_combine": (_i32, [_p, _p, _i32, _i32, _i32, _i32, _p, _p, _p, _p]),
    "d3_combine_experts": (_i32, [_p, _p, _p, _i64, _i32, _i32, _p, _p]),
    "d3_combine_experts_add_norm": (
        _i32, [_p, _p, _p, _i64, _p, _p, _p, _f32, _i32, _i32, _p, _p]),
    "d3_combine_routes_add_norm": (_i32, [_p, _p, _i32, _i32, _p, _p, _i64, _p, _p, _p, _f32,
                                          _i32, _i32, _p, _p]),
    "d3_add_norm": (_i32, [_p, _p, _p, _f32, _i32, _i32, _p, _p]),
    "d3_silu_mul": (_i32, [_p, _i64, _i32, _i32, _p, _p]),
    "d3_dense_bf16": (_i32, [_p, _i64, _i32, _p, _i32, _i32, _i32, _p, _i64, _p, _i64, _p]),
    "d3_combine_route_logits": (_i32, [_p, _p, _i32, _i64, _i32, _i32, _p, _i32, _p, _p, _i64, _p,
                                       _p, _f32, _i32, _i32, _p, _p]),
    "d3_row_metadata": (_i32, [_p, _p, _i32, _i32, _p, _i32, _i64, _p, _p, _p, _p]),
    "d3_mixed_rows": (_i32, [_p, _i32, _i32, _i64, _p, _i32, _i32, _p, _i32, _p, _i32, _p, _p, _p,
                             _p, _p, _p, _p, _p, _p]),
    "d3_requests_load": (_i32, [_p, _p, _p, _p, _i32, _i64, _i64, _p, _p, _p, _p]),
    "d3_requests_save": (_i32, [_p, _p, _p, _p, _p, _i32, _p, _i64, _i64, _p]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raises if it was never built."""
    global _lib
    if _lib is None:
        path = Path(os.environ.get("DRAMA3_MOE_LIBRARY", LIBRARY))
        if not path.exists():
            raise RuntimeError(
                f"{path} is missing: build it with `python -m drama3_amd._build` "
                "(or __graft_entry__.build()); there is no CPU fallback")
        lib = ctypes.CDLL(str(path))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Call an entry point and map its status to the reference's exceptions:
    contract violations -> ValueError, HIP failures -> RuntimeError."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status == D3_OK:
        return
    message = lib.d3_last_error().decode(errors="replace")
    if status in (D3_ERR_INVALID_ARGUMENT, D3_ERR_UNSUPPORTED):
        raise ValueError(message)
    raise RuntimeError(message)


def ptr(tensor: torch.Tensor | None) -> int | None:
    return None if tensor is None else tensor.data_ptr()


def stream(device: torch.device | None = None) -> int:
    """Handle of torch's current stream on ``device`` (a hipStream_t)."""
    return torch.cuda.current_stream(device).cuda_stream


def exported_symbols() -> list[str]:
    return list(SIGNATURES)
