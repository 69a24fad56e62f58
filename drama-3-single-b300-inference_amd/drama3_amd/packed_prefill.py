"""Ragged packed-row metadata with the reference's interface
(``src/drama3/packed_prefill.py:11-78``).

``row_metadata`` keeps the reference's launch form ``row_metadata[grid](...)``
(a Triton kernel there) so callers need no change; the grid and BLOCK are
accepted and the MI355X kernel picks its own launch shape.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from ._lib import call, ptr
from .pipeline import require_cuda


@dataclass
class PackedLayout:
    """``PackedLayout`` (``packed_prefill.py:11-17``): int32 cu_seqlens
    ``boundaries [n+1]``, int64 ``sequence_slots [n]``, ``max_length``."""

    boundaries: torch.Tensor
    sequence_slots: torch.Tensor
    max_length: int
    chunk_indices: torch.Tensor | None = None
    chunk_offsets: torch.Tensor | None = None


def packed_row_metadata(boundaries, sequence_slots, capacity, positions, row_slots,
                        labels=None, frames=None, eos=0):
    """Per packed row: sequence position and slot, plus next-frame labels.

    ``positions`` / ``row_slots`` int64 [capacity]; ``labels`` / ``frames``
    int64 [capacity, codes] (optional).
    """
    require_cuda(boundaries, sequence_slots, positions, row_slots, labels, frames)
    if boundaries.dtype != torch.int32 or sequence_slots.dtype != torch.int64:
        raise TypeError("boundaries must be int32 and sequence_slots int64")
    if positions.dtype != torch.int64 or row_slots.dtype != torch.int64:
        raise TypeError("positions and row_slots must be int64")
    sequences = len(boundaries) - 1
    if sequences < 1 or len(sequence_slots) < sequences:
        raise ValueError("need at least one sequence and one slot per sequence")
    codes = 0
    if labels is not None:
        if frames is None or frames.shape[1] != labels.shape[1]:
            raise ValueError("labels need frames with the same number of codes")
        codes = labels.shape[1]
        labels_ptr, frames_ptr = ptr(labels), ptr(frames)
    else:
        labels_ptr = frames_ptr = None
    call("d3_row_metadata", ptr(boundaries), ptr(sequence_slots), sequences, int(capacity),
         frames_ptr, codes, int(eos), ptr(positions), ptr(row_slots), labels_ptr,
         _lib.stream(boundaries.device))


class _RowMetadata:
    """``row_metadata[grid](CU, SLOTS, POS, ROW_SLOTS, LABELS, FRAMES, EOS,
    SEQUENCES, CAPACITY, BLOCK)`` with the reference's argument meaning."""

    def __getitem__(self, grid):
        def launch(cu, slots, pos, row_slots, labels, frames, eos, sequences, capacity, block=128):
            if sequences != len(cu) - 1:
                raise ValueError("SEQUENCES must equal len(CU) - 1")
            packed_row_metadata(cu, slots, capacity, pos, row_slots, labels, frames, eos)

        return launch


row_metadata = _RowMetadata()
