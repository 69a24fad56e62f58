"""numpy restatement of the persistent-slot request state kernels.

Test infrastructure only (see ``oracle/__init__.py``).  Follows
``src/drama3/runtime_state.py``: ``_load`` (lines 10-32) and ``_save``
(lines 35-56) with the storage of ``DeviceRequests.__init__`` (lines 75-92).
"""

from __future__ import annotations

import numpy as np


class RequestState:
    def __init__(self, slots: int, eos: int, max_length: int, max_frames: int = 500):
        self.eos, self.max_length, self.max_frames = eos, max_length, max_frames
        self.last = np.zeros((slots, 11), np.int64)
        self.last[:, 0] = eos
        self.history = np.full((slots, 16), -1, np.int64)
        self.metadata = np.zeros((slots, 4), np.int64)
        self.metadata[:, 0] = max_length - 1
        self.metadata[:, 2] = max_frames
        self.codes = np.zeros((slots, max_frames, 10), np.int64)

    def initialize(self, slot, frame, history, position, limit):
        self.last[slot] = frame
        self.history[slot] = history
        self.metadata[slot] = [position, 0, limit, 0]

    def load(self, slots, padding_start: int = -1):
        """-> (frames [n, 11], history [n, 16], positions [n])."""
        slots = np.asarray(slots, np.int64)
        frames = self.last[slots].copy()
        history = self.history[slots].copy()
        positions = self.metadata[slots, 0].copy()
        if padding_start >= 0:
            positions[slots >= padding_start] = 0
        return frames, history, np.minimum(positions, self.max_length - 1)

    def save(self, slots, output):
        """Append one step's output frames [n, 11] (rows in ``slots`` order)."""
        for row, slot in enumerate(np.asarray(slots, np.int64)):
            main = output[row, 0]
            position, count, limit, done = self.metadata[slot]
            append = done == 0 and main != self.eos and count < limit
            if append:
                self.last[slot] = output[row]
                self.history[slot] = np.concatenate([self.history[slot, 1:], [main]])
                self.codes[slot, count] = output[row, 1:]
                count += 1
            self.metadata[slot, 0] = position + int(append)
            self.metadata[slot, 1] = count
            self.metadata[slot, 3] = int(done != 0 or main == self.eos or count >= limit)
