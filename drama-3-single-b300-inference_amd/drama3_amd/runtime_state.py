"""Per-slot request state of persistent decode slots
(``src/drama3/runtime_state.py:75-132``): ``load`` gathers each live slot's
last frame, token history and position into compact rows before a step and
``save`` appends the step's output afterwards (EOS / frame-limit
retirement).  Both run one MI355X kernel; layout and rules are the
reference's."""

from __future__ import annotations

import torch

from . import _lib
from ._lib import call, ptr
from .pipeline import require_cuda


class DeviceRequests:
    def __init__(self, slots: int, eos: int, max_length: int, max_frames: int = 500,
                 device="cuda", short_padding_context: bool = False):
        self.eos = eos
        self.max_frames = max_frames
        self.max_length = max_length
        self.short_padding_context = short_padding_context
        dev = torch.device(device)
        self.last = torch.zeros(slots, 11, device=dev, dtype=torch.int64)
        self.last[:, 0] = eos
        self.history = torch.full((slots, 16), -1, device=dev, dtype=torch.int64)
        self.metadata = torch.zeros(slots, 4, device=dev, dtype=torch.int64)
        self.metadata[:, 0] = max_length - 1
        self.metadata[:, 2] = max_frames
        self.codes = torch.zeros(slots, max_frames, 10, device=dev, dtype=torch.int64)

    def initialize(self, slot, frame, history, position, limit):
        self.last[slot].copy_(frame)
        self.history[slot].copy_(history)
        self.metadata[slot].copy_(torch.tensor([position, 0, limit, 0]))

    def load(self, slots, frames, history, positions, *, padding_start=None):
        """``DeviceRequests.load`` (``runtime_state.py:94-111``)."""
        if padding_start is not None and not 0 < padding_start <= self.metadata.shape[0]:
            raise ValueError("padding_start must identify a nonempty reserved slot range")
        require_cuda(slots, frames, history, positions)
        start = padding_start if self.short_padding_context and padding_start is not None else -1
        slots = slots.contiguous()
        call("d3_requests_load", ptr(self.last), ptr(self.history), ptr(self.metadata),
             ptr(slots), len(slots), self.max_length, start, ptr(frames),
             ptr(history), ptr(positions), _lib.stream(slots.device))

    def save(self, slots, frames):
        """``DeviceRequests.save`` (``runtime_state.py:113-124``)."""
        require_cuda(slots, frames)
        slots, frames = slots.contiguous(), frames.contiguous()
        call("d3_requests_save", ptr(self.last), ptr(self.history), ptr(self.metadata),
             ptr(self.codes), ptr(slots), len(slots), ptr(frames),
             self.eos, self.max_frames, _lib.stream(slots.device))
