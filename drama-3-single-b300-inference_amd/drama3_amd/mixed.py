"""Mixed decode + prefill steps: the rows of the reference's ``MixedGraph``
(``src/drama3/mixed_graph.py:12-185``) and the MoE side of its
``mixed_backbone`` (``src/drama3/mixed_model.py:164-249``), on the device.

The reference prepares each mixed step on the host (``MixedGraph.prepare``:
decode slots padded with reserved slots, prompt boundaries, optionally a
prefix-reuse plan built by ``plan_row_reuse`` on CPU prompts and matched to
one of five pre-captured compact buckets) and then replays a graph.  Here
``d3_mixed_rows`` derives the same rows from device data inside the graph:
occupancy -> decode slots, boundaries + the prompt frames -> prefix
ownership -> the MoE rows (``keep``, a device count) and the read-back map
(``inverse``).  The MoE kernels are driven by that count, so one capture at
full capacity serves every occupancy, prompt set and amount of reuse, and
padding rows never reach the MoE.
"""

from __future__ import annotations

import torch

from . import _lib
from ._lib import call, ptr
from .pipeline import MoEWorkspace, Shape, by_pair_suited, grouped_supported, require_cuda

MAX_REUSE_PROMPTS = 16
MAX_REUSE_ROWS = 8192


class MixedRows:
    """Device buffers of one mixed row layout (``d3_mixed_rows``).

    Row space: ``decode_rows`` decode rows, then the prefill suffix's
    ``capacity`` rows.  After a call: ``active`` int32 [slots] (ascending,
    -1 padded) and ``count`` int32 [1]; ``decode_slots`` int64
    [decode_rows]; ``keep`` int32 [full] / ``keep_count`` int32 [1] (the
    MoE rows); ``inverse`` int64 [full] (MoE row read back by every row).
    """

    def __init__(self, slots: int, decode_rows: int, capacity: int, padding_start: int,
                 device="cuda"):
        if slots < 1 or decode_rows < 0 or capacity < 0 or decode_rows + capacity < 1:
            raise ValueError("need slots >= 1 and at least one row")
        if padding_start < 0:
            raise ValueError("padding_start must be a slot index")
        dev = torch.device(device)
        i32, i64 = dict(dtype=torch.int32, device=dev), dict(dtype=torch.int64, device=dev)
        self.slots, self.decode_rows, self.capacity = slots, decode_rows, capacity
        self.padding_start = padding_start
        self.full = decode_rows + capacity
        self.active = torch.empty(slots, **i32)
        self.count = torch.empty(1, **i32)
        self.decode_slots = torch.empty(max(decode_rows, 1), **i64)
        self.keep = torch.empty(self.full, **i32)
        self.keep_count = torch.empty(1, **i32)
        self.inverse = torch.empty(self.full, **i64)

    def __call__(self, occupancy: torch.Tensor, boundaries: torch.Tensor, prompts: int,
                 frames: torch.Tensor | None = None, stream=None,
                 sequence_slots: torch.Tensor | None = None, positions: torch.Tensor | None = None,
                 row_slots: torch.Tensor | None = None) -> None:
        """occupancy uint8 [slots]; boundaries int32 [>= prompts + 1] (prompt
        i = suffix rows [b[i], b[i+1]), rows from b[prompts] on are padding);
        frames int64 [capacity, codes] of the suffix (prefix reuse) or None.
        With ``positions`` / ``row_slots`` (int64 [capacity]) the same launch
        writes the suffix's row metadata (``row_metadata`` of
        ``packed_prefill.py:51-78``) over all ``len(boundaries) - 1``
        sequences, whose slots ``sequence_slots`` holds."""
        require_cuda(occupancy, boundaries, frames, sequence_slots, positions, row_slots)
        sequences = 0
        if positions is not None:
            sequences = boundaries.numel() - 1
            if (row_slots is None or sequence_slots is None or sequence_slots.numel() < sequences
                    or positions.dtype != torch.int64 or row_slots.dtype != torch.int64
                    or sequence_slots.dtype != torch.int64
                    or min(positions.numel(), row_slots.numel()) < self.capacity):
                raise ValueError("row metadata needs int64 positions / row_slots [capacity] and "
                                 "one int64 sequence slot per sequence")
        if occupancy.dtype != torch.uint8 or occupancy.numel() != self.slots:
            raise ValueError(f"occupancy must be uint8 [{self.slots}]")
        if boundaries.dtype != torch.int32 or not boundaries.is_contiguous() \
                or boundaries.numel() < prompts + 1 or prompts < 0:
            raise ValueError("boundaries must be contiguous int32 with prompts + 1 entries")
        codes = 0
        if frames is not None:
            if frames.dtype != torch.int64 or frames.dim() != 2 or len(frames) < self.capacity \
                    or not frames.is_contiguous():
                raise ValueError("frames must be contiguous int64 [capacity, codes]")
            codes = frames.shape[1]
        stream = _lib.stream(occupancy.device) if stream is None else stream
        call("d3_mixed_rows", ptr(occupancy), self.slots, self.decode_rows, self.padding_start,
             ptr(boundaries), prompts, self.capacity, ptr(frames), codes, ptr(sequence_slots),
             sequences, ptr(self.active), ptr(self.count), ptr(self.decode_slots), ptr(self.keep),
             ptr(self.keep_count), ptr(self.inverse), ptr(positions), ptr(row_slots), stream)


class MixedStep:
    """The MoE side of one mixed step, graph-capturable with fixed buffers.

    Per step (``forward``): the mixed rows and the prefill suffix's row
    metadata (``row_metadata`` of ``mixed_graph.py:96-107``) in one launch,
    the routed experts over
    the kept rows (``model.moe_parts(normalized.index_select(0, keep), ...)``,
    ``mixed_model.py:237-243``) and ``combine_experts_add_norm_inverse`` back
    onto every row (``mixed_model.py:198-201``), the routed rows' weighted
    combine folded into that last launch (``routed`` is then not written).

    Inputs written into the staging buffers before a replay: ``occupancy``,
    ``boundaries`` (int32 [sequences + 1], the reference layout's boundaries
    with the padding sequence last), ``sequence_slots``, ``frames`` (int64
    [capacity, codes], the prompt suffix), ``x`` / ``logits`` ([full] rows:
    the layer's normalised rows and router logits), ``residual`` [full, H],
    and the shared-expert output ``shared`` / ``gate`` on the kept rows
    (row k belongs to row ``keep[k]``, as the reference's ``moe_parts``
    outputs on its compact rows).
    """

    def __init__(self, slots: int, decode_rows: int, capacity: int, padding_start: int,
                 sequences: int, num_experts: int, hidden: int, intermediate: int,
                 top_k: int = 8, codes: int = 11, reuse: bool = True, device="cuda",
                 separate_combine: bool = False):
        dev = torch.device(device)
        self.device = dev
        self.rows = MixedRows(slots, decode_rows, capacity, padding_start, dev)
        full = self.rows.full
        if reuse and (sequences - 1 > MAX_REUSE_PROMPTS or full > MAX_REUSE_ROWS):
            raise ValueError(f"prefix reuse needs <= {MAX_REUSE_PROMPTS} prompts and "
                             f"<= {MAX_REUSE_ROWS} rows")
        self.sequences, self.reuse, self.hidden = sequences, reuse, hidden
        # separate_combine: the routed combine (into ``routed``) and the
        # residual + RMSNorm combine as two launches instead of one.
        self.separate_combine = separate_combine
        bf16 = dict(dtype=torch.bfloat16, device=dev)
        self.occupancy = torch.zeros(slots, dtype=torch.uint8, device=dev)
        self.boundaries = torch.zeros(sequences + 1, dtype=torch.int32, device=dev)
        self.sequence_slots = torch.zeros(sequences, dtype=torch.int64, device=dev)
        self.frames = torch.zeros((max(capacity, 1), codes), dtype=torch.int64, device=dev)
        self.positions = torch.empty(max(capacity, 1), dtype=torch.int64, device=dev)
        self.row_slots = torch.empty(max(capacity, 1), dtype=torch.int64, device=dev)
        self.x = torch.zeros((full, hidden), **bf16)
        self.logits = torch.zeros((full, num_experts), **bf16)
        self.residual = torch.zeros((full, hidden), **bf16)
        self.shared = torch.zeros((full, hidden), **bf16)
        self.gate = torch.zeros(full, **bf16)
        self.norm_weight = torch.zeros(hidden, **bf16)
        self.epsilon = 1e-6
        self.routed = torch.zeros((full, hidden), **bf16)
        self.out = torch.empty((full, hidden), **bf16)
        # The grouped GEMMs find their own routes (no per-layer sort launch)
        # whenever the step's rows allow it.
        by_pair = by_pair_suited(full, num_experts, top_k) and grouped_supported(hidden, intermediate)
        self.workspace = MoEWorkspace(Shape(full, num_experts, hidden, intermediate, top_k), dev,
                                      item_rows=128 if full > 128 else None, by_pair=by_pair)
        self.graph: torch.cuda.CUDAGraph | None = None

    def forward(self, experts) -> torch.Tensor:
        """One eager step on the current stream; returns ``out`` [full, H]
        (``residual`` is updated in place, as the reference's combine does)."""
        stream = _lib.stream(self.device)
        r = self.rows
        r(self.occupancy, self.boundaries, self.sequences - 1,
          self.frames if self.reuse else None, stream, self.sequence_slots, self.positions,
          self.row_slots)
        ws = self.workspace
        ws.front(self.x, self.logits, r.keep, r.keep_count, stream=stream)
        ws.routes_down(experts, r.keep_count, stream)
        if self.separate_combine:
            ws.combine(None, r.keep_count, None, self.routed, stream)
            call("d3_combine_experts_add_norm", ptr(self.routed), ptr(self.shared),
                 ptr(self.gate), 1, ptr(r.inverse), ptr(self.residual), ptr(self.norm_weight),
                 float(self.epsilon), r.full, self.hidden, ptr(self.out), stream)
        else:
            ws.combine_add_norm(self.shared, self.gate, self.residual, self.norm_weight,
                                self.epsilon, r.inverse, self.out, stream)
        return self.out

    def capture(self, experts, pool=None) -> None:
        """Capture ``forward`` once (after two warm-up runs on a side stream,
        as ``mixed_graph.py:73-80`` does); ``run`` replays it."""
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            for _ in range(2):
                self.forward(experts)
        torch.cuda.current_stream(self.device).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, pool=pool):
            self.forward(experts)

    def replay(self) -> torch.Tensor:
        if self.graph is None:
            raise RuntimeError("capture() first")
        self.graph.replay()
        return self.out
