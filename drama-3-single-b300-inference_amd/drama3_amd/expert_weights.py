"""Expert weight layouts of the FP8 expert GEMM.

The checkpoint layout (``w13_weight [E, 2I, H]``, ``w2_weight [E, H, I]``,
``kernels.py:290-318``) is accepted as is.  ``prepare_experts`` additionally
attaches fragment-major copies of the fp8 codes (``d3_pack_expert_weights``):
each 16-row tile stored as [K block][half][lane][16 bytes], so that every
load instruction of an expert-GEMM wave reads 1 KiB of contiguous memory.
This is the counterpart of the reference's load-time re-layout for its
FlashInfer path (``model.py:195-205``: ``flashinfer_w13`` [up | gate] copies
and ``blocked_moe_weight``), done once when the model is loaded; the block
scales are shared by both layouts.
"""

from __future__ import annotations

import torch

from . import _lib
from ._lib import call, ptr

LAYOUT_REFERENCE = 0
LAYOUT_FRAGMENT = 1


def pack_expert_weights(weight: torch.Tensor, stream=None) -> torch.Tensor:
    """fp8 [E, N, K] (reference layout) -> fragment-major copy of the same shape."""
    if weight.dim() != 3 or weight.dtype.itemsize != 1:
        raise ValueError("weight must be a [E, N, K] tensor of 1-byte fp8 codes")
    if not weight.is_cuda:
        raise ValueError("weight must be on the GPU")
    e, n, k = weight.shape
    if n % 16 or k % 128:
        raise ValueError(f"N={n} must be a multiple of 16 and K={k} of 128")
    source = weight.contiguous()
    packed = torch.empty_like(source)
    stream = _lib.stream(weight.device) if stream is None else stream
    call("d3_pack_expert_weights", ptr(source), e, n, k, ptr(packed), stream)
    return packed


def prepare_experts(experts, stream=None, keep_reference: bool = True):
    """Attach ``d3_w13_packed`` / ``d3_w2_packed`` (fragment-major codes) to an
    experts object; the MoE ops use them from then on.  Returns ``experts``.

    The packed copies are tied to the tensors they were made from (pointer,
    shape and version counter); ``fc1_operands``/``fc2_operands`` fall back
    to the checkpoint layout if the source weights were replaced or modified.

    ``keep_reference=False`` keeps one copy of the codes: ``w13_weight`` /
    ``w2_weight`` are replaced by their fragment-major copies (same shape and
    dtype, half the expert bytes of keeping both).  The object then holds no
    checkpoint-layout codes: anything that reads those tensors as checkpoint
    rows (a CPU reference, a copy handed to other code) must not be given
    it.  Calling ``prepare_experts`` again on such an object does nothing.
    """
    for name in ("w13", "w2"):
        if getattr(experts, f"d3_{name}_fragment_only", False):
            continue  # already holds only the fragment-major codes
        weight = getattr(experts, f"{name}_weight")
        packed = pack_expert_weights(weight, stream)
        if not keep_reference:
            setattr(experts, f"{name}_weight", packed)
            setattr(experts, f"d3_{name}_fragment_only", True)
        setattr(experts, f"d3_{name}_packed", packed)
        setattr(experts, f"d3_{name}_source", _identity(packed if not keep_reference else weight))
    return experts


def _identity(weight: torch.Tensor):
    return (weight.data_ptr(), tuple(weight.shape), weight._version)


def _operands(experts, name: str):
    weight = getattr(experts, f"{name}_weight")
    scales = getattr(experts, f"{name}_scale_inv")
    packed = getattr(experts, f"d3_{name}_packed", None)
    if packed is not None and getattr(experts, f"d3_{name}_source", None) == _identity(weight):
        return packed, scales, LAYOUT_FRAGMENT
    return weight, scales, LAYOUT_REFERENCE


def fc1_operands(experts):
    """(w13 codes, w13 block scales, layout) for the FC1 GEMM."""
    return _operands(experts, "w13")


def fc2_operands(experts):
    """(w2 codes, w2 block scales, layout) for the FC2 GEMM."""
    return _operands(experts, "w2")
