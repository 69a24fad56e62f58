"""The packed FP8 top-k MoE step as a chain of C-ABI launches.

``MoEWorkspace`` owns every intermediate buffer for one capacity (rows,
experts, hidden, intermediate, top-k), so a step allocates nothing and can be
captured in a HIP graph.  Row counts may live on the device (``row_count``):
the kernels read them at run time, so one captured graph serves every
occupancy up to the capacity.

Step (one kernel each, all on the current stream):
    route            logits -> ids, weights            (kernels.py:360-383)
    quantize_rows    x -> e4m3 q + per-128 scales      (moe_input.py:24-27)
    sort_routes      ids -> histogram, padded offsets, stable sorted pair list,
                     inverse map, work items           (kernels.py:658-731)
    expert_gemm FC1  gather q rows by route, W13, bf16 gate|up at sorted rows
                                                       (kernels.py:290-301)
    silu_mul_quant   SwiGLU + e4m3 requant             (kernels.py:344,748)
    expert_gemm FC2  W2, fp32 per pair (unpermute)     (kernels.py:304-318)
    (decode-sized items: FC2 computes the SwiGLU requant in its prologue,
    d3_expert_fc2_swiglu, and silu_mul_quant is not launched)
    weighted_combine sum_r w[t,r] y[t*K+r] -> bf16     (kernels.py:319-322,779)

Decode step (``DecodeStep``, fragment-major weights, >= 1 route per expert): no
route sort and no front launch.  ``decode_route_fc1`` routes (expert ranks
from the logits), quantises and runs FC1 from the slots; ``decode_fc2``
finds each expert's routes from the ids FC1 wrote and stores its down rows
by slot pair (slot * top_k + rank); ``decode_route_combine`` recomputes the
routing weights and combines, loading each slot's down rows with its
logits.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from ._lib import DTYPE_BF16, DTYPE_F32, DTYPE_I32, DTYPE_I64, call, ptr
from .expert_weights import LAYOUT_FRAGMENT, fc1_operands, fc2_operands

SORT_TILE = 16  # MFMA route tile; also the padding granularity of the sorted layout
# Work items with at most this many routes take the exact (bf16-MFMA) path of
# the expert GEMM; larger items are real contractions and take FP8 MFMAs.
EXACT_ROUTES = 64
# Contraction lengths compiled for the tiled grouped GEMMs (d3_grouped_*).
GROUPED_K = (256, 512, 768, 1024, 1536, 2048)
GROUPED_ROUTES = 128  # most routes per work item of the tiled grouped GEMMs
GROUPED_ITEM_ROUTES = 128  # their default item size
BY_PAIR_MAX_PAIRS = 8192  # most (row, rank) pairs of the grouped GEMMs without a sort
# Up to this many (row, rank) pairs the route sort can run inside the fused
# front kernel (its last workgroup; opt-in, MoEWorkspace(fused_sort=True));
# otherwise the 1024-thread sort kernel follows the front, and from
# WIDE_SORT_PAIRS on the wide sort (one workgroup per 512 pairs).
FUSED_SORT_PAIRS = 8192
FUSED_SORT_EXPERTS = 256
WIDE_SORT_PAIRS = 8192


def grouped_supported(hidden: int, intermediate: int) -> bool:
    """Whether the tiled grouped FC1 (K = hidden) and FC2 (K = intermediate,
    N = hidden in 256-row tiles) cover these shapes."""
    return (hidden in GROUPED_K and intermediate in GROUPED_K and hidden % 256 == 0
            and intermediate % 128 == 0)


def dtype_code(dtype: torch.dtype) -> int:
    codes = {torch.bfloat16: DTYPE_BF16, torch.float32: DTYPE_F32, torch.int32: DTYPE_I32,
             torch.int64: DTYPE_I64}
    if dtype not in codes:
        raise TypeError(f"unsupported dtype {dtype}")
    return codes[dtype]


def require_cuda(*tensors: torch.Tensor | None) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("MI355X MoE operators need device tensors (no CPU fallback)")


def by_pair_suited(rows: int, num_experts: int, top_k: int = 8) -> bool:
    """Whether the grouped GEMMs without a route sort suit a batch: at most
    BY_PAIR_MAX_PAIRS (row, rank) pairs, and a grid of at most 128 (expert,
    128-route part) items, since every item's workgroups read all the ids
    before they know whether their part holds routes."""
    parts = -(-rows // 128)
    return rows > 128 and rows * top_k <= BY_PAIR_MAX_PAIRS and num_experts * parts <= 128


def default_item_rows(rows: int, tile: int = SORT_TILE, num_experts: int | None = None,
                      top_k: int = 8) -> int:
    """Routes per work item (a multiple of ``tile``).  Up to 128 rows an
    expert cannot receive more routes than rows, so one item covers all of an
    expert's routes (one weight read per expert); larger batches cap items at
    128 routes so busy experts spread over several workgroups.  When experts
    are sparse (at most 8 routes each on average at full capacity) items are
    one 16-route tile: the expert GEMM then pipelines two weight tiles per
    workgroup, and the rare expert with more routes is read once per item."""
    if num_experts is not None and rows <= 128 and rows * top_k <= 8 * num_experts:
        return tile
    rows = min(rows, 128) if rows > 128 else rows
    return max(tile, -(-rows // tile) * tile)


@dataclass
class Shape:
    rows: int
    num_experts: int
    hidden: int
    intermediate: int
    top_k: int = 8

    @property
    def pairs(self) -> int:
        return self.rows * self.top_k


class MoEWorkspace:
    """Buffers of one MoE step at a fixed capacity (see module docstring)."""

    def __init__(self, shape: Shape, device: torch.device | str = "cuda", tile: int = SORT_TILE,
                 item_rows: int | None = None, weights_dtype: torch.dtype = torch.bfloat16,
                 exact_routes: int = EXACT_ROUTES,
                 swiglu_in_fc2: bool | None = None, sortless: bool = False,
                 grouped: bool | None = None, shared_rows: int = 0, fused_sort: bool = False,
                 by_pair: bool = False):
        lib = _lib.load()
        self.shape = shape
        # front(): sort in the front launch's last workgroup (256 threads)
        # instead of the 1024-thread sort launch after it; the separate launch
        # is the faster of the two at every measured size (48-1024 rows).
        self.fused_sort = fused_sort
        self.device = torch.device(device)
        self.tile = tile
        self.exact_routes = exact_routes
        self.item_rows = item_rows or default_item_rows(shape.rows, tile, shape.num_experts,
                                                        shape.top_k)
        # Contraction-sized items go to the tiled grouped GEMMs, whose items
        # hold up to GROUPED_ROUTES routes.
        contraction = self.item_rows > EXACT_ROUTES
        h, i = shape.hidden, shape.intermediate
        if grouped is None:
            grouped = contraction and grouped_supported(h, i) and not sortless
        if grouped and item_rows is None and shape.rows > 128:
            self.item_rows = GROUPED_ITEM_ROUTES
        if self.item_rows % tile:
            raise ValueError("item_rows must be a multiple of the sort tile")
        pairs = shape.pairs
        self.max_rows = lib.d3_max_sorted_rows(pairs, shape.num_experts, tile)
        self.wide_sort = pairs > WIDE_SORT_PAIRS
        # The wide sort pads each expert's items to an even count when the
        # items array holds the padding: the tiled grouped GEMMs, which give
        # each XCD runs of two consecutive items, then never split a pair of
        # one expert's items over two XCDs' L2s.  The sort pads only while
        # the experts with routes average at least 1.5 items (config 4, 229
        # routes per expert: -5 us per step); at about one item per expert
        # most experts would take an empty item (4,096 rows x E256: +28 us
        # per layer when padded).  Other consumers keep the unpadded list.
        self.aligned_items = bool(self.wide_sort and grouped and not sortless)
        self.max_items = (lib.d3_max_items_aligned if self.aligned_items else lib.d3_max_items)(
            pairs, shape.num_experts, self.item_rows)
        dev = self.device
        i32 = dict(dtype=torch.int32, device=dev)
        h, e, i, t = shape.hidden, shape.num_experts, shape.intermediate, shape.rows
        self.ids = torch.empty((t, shape.top_k), **i32)
        self.weights = torch.empty((t, shape.top_k), dtype=weights_dtype, device=dev)
        self.q = torch.empty((t, h), dtype=torch.uint8, device=dev)
        self.x_scales = torch.empty((t, h // 128), dtype=torch.float32, device=dev)
        self.counts = torch.empty(e, **i32)
        self.starts = torch.empty(e, **i32)
        self.total = torch.empty(1, **i32)
        self.pairs_dev = torch.empty(1, **i32)
        self.sorted_ids = torch.empty(self.max_rows, **i32)
        self.expert_ids = torch.empty(self.max_rows // tile, **i32)
        self.inverse = torch.empty(pairs, **i32)
        self.items = torch.empty((max(self.max_items, 1), 4), **i32)
        self.num_items = torch.empty(1, **i32)
        self.ticket = torch.zeros(1, **i32)  # fused-sort ticket: 0 between launches
        # A dense shared expert folded into the tiled grouped launches takes
        # shared_rows extra activation rows (after the sorted ones) and fp32
        # output rows (after the pairs).
        self.shared_rows = shared_rows
        self.gate_up = torch.empty((self.max_rows, 2 * i), dtype=torch.bfloat16, device=dev)
        self.act = torch.empty((self.max_rows + shared_rows, i), dtype=torch.uint8, device=dev)
        self.act_scales = torch.empty((self.max_rows + shared_rows, i // 128), dtype=torch.float32,
                                      device=dev)
        self.down = torch.empty((pairs + shared_rows, h), dtype=torch.float32, device=dev)
        self.out = torch.empty((t, h), dtype=torch.bfloat16, device=dev)
        # SwiGLU requant in FC2's prologue: every FC2 workgroup of an item
        # recomputes the item's activations, which is free while its weights
        # stream in as long as items are a few route tiles (decode).
        if swiglu_in_fc2 is None:
            swiglu_in_fc2 = self.item_rows <= EXACT_ROUTES and i <= 1024
        self.swiglu_in_fc2 = bool(swiglu_in_fc2)
        # Sortless decode: the front skips the route sort and the expert GEMMs
        # (d3_decode_expert_gemm, fragment-major weights) find each expert's
        # routes themselves; gate_up / down rows are indexed by pair.
        self.sortless = sortless
        if sortless and (t > 256 or shape.top_k > 8):
            raise ValueError("sortless decode covers up to 256 rows and top_k <= 8")
        # Tiled grouped GEMMs (FP8 MFMA contraction, SwiGLU requant in FC1's
        # epilogue) for contraction-sized items: prefill and mixed batches.
        if grouped and not (self.item_rows <= GROUPED_ROUTES and grouped_supported(h, i)):
            raise ValueError(f"tiled grouped GEMMs need item_rows <= {GROUPED_ROUTES}, hidden and "
                             f"intermediate in {GROUPED_K}, hidden % 256 == 0")
        self.grouped = bool(grouped) and not sortless
        # Grouped GEMMs without the route sort (small batches): the front
        # launch skips the sort, FC1's workgroups find their routes in `ids`
        # and write them as a route list of one 128-route item per (expert,
        # part), act rows at the list's positions; FC2 reads that list as it
        # reads a sort's.
        if by_pair and not (self.grouped and shared_rows == 0 and pairs <= BY_PAIR_MAX_PAIRS):
            raise ValueError(f"by_pair needs the grouped GEMMs, no folded shared expert and "
                             f"<= {BY_PAIR_MAX_PAIRS} (row, rank) pairs")
        self.by_pair = bool(by_pair)
        if self.by_pair:
            self.list_items_max = e * -(-t // GROUPED_ROUTES)
            list_rows = self.list_items_max * GROUPED_ROUTES
            self.list_ids = torch.empty(list_rows, **i32)
            self.list_items = torch.empty((self.list_items_max, 4), **i32)
            self.list_count = torch.empty(1, **i32)
            if list_rows > len(self.act):
                self.act = torch.empty((list_rows, i), dtype=torch.uint8, device=dev)
                self.act_scales = torch.empty((list_rows, i // 128), dtype=torch.float32,
                                              device=dev)
        self.rows_dev = torch.full((1,), t, **i32)  # the live row count when none is given
        # Scratch of the wide route sort (prefill-sized batches).
        self.sort_scratch = torch.empty(
            lib.d3_sort_wide_scratch_ints(t, shape.top_k, e) if self.wide_sort else 1, **i32)

    # -- stages ---------------------------------------------------------------
    def _stream(self, stream):
        return _lib.stream(self.device) if stream is None else stream

    def route(self, logits: torch.Tensor, row_index=None, row_count=None, stream=None) -> None:
        s, stream = self.shape, self._stream(stream)
        call("d3_route", ptr(logits), dtype_code(logits.dtype), logits.stride(0), s.rows,
             s.num_experts, s.top_k, ptr(row_index), ptr(row_count), ptr(self.ids), None,
             ptr(self.weights), dtype_code(self.weights.dtype), stream)

    def quantize(self, x: torch.Tensor, row_index=None, row_count=None, stream=None) -> None:
        s, stream = self.shape, self._stream(stream)
        call("d3_quantize_rows", ptr(x), x.stride(0), s.rows, s.hidden, ptr(row_index),
             ptr(row_count), ptr(self.q), ptr(self.x_scales), 0, stream)

    def sort(self, ids: torch.Tensor | None = None, row_count=None, stream=None) -> None:
        s, stream = self.shape, self._stream(stream)
        ids = self.ids if ids is None else ids
        args = (ptr(ids), dtype_code(ids.dtype), s.rows, ptr(row_count), s.top_k,
                s.num_experts, self.tile, ptr(self.counts), ptr(self.starts), ptr(self.total),
                ptr(self.sorted_ids), ptr(self.expert_ids), self.max_rows, ptr(self.inverse),
                self.item_rows, ptr(self.items), self.max_items, ptr(self.num_items),
                ptr(self.pairs_dev))
        if self.wide_sort:
            call("d3_sort_routes_wide", *args, ptr(self.sort_scratch), self.sort_scratch.numel(),
                 stream)
        else:
            call("d3_sort_routes", *args, stream)

    def front(self, x, logits, row_index=None, row_count=None, occupancy=None, active=None,
              count=None, stream=None) -> None:
        """Route + quantise every live row, and sort the routes, in one launch
        (two when the batch exceeds the fused sort).  With ``occupancy`` the
        rows are the live slots (``active`` / ``count`` receive the list)."""
        s, stream = self.shape, self._stream(stream)
        fused = (self.fused_sort and s.pairs <= FUSED_SORT_PAIRS
                 and s.num_experts <= FUSED_SORT_EXPERTS and not self.sortless)
        slots = occupancy.numel() if occupancy is not None else 0
        if occupancy is not None and slots != s.rows:
            raise ValueError("slot mode needs a workspace with one row per slot")
        sort_args = ((ptr(self.counts), ptr(self.starts), ptr(self.total), ptr(self.sorted_ids),
                      ptr(self.expert_ids), self.max_rows, ptr(self.inverse), ptr(self.items),
                      self.max_items, ptr(self.num_items), ptr(self.pairs_dev), ptr(self.ticket))
                     if fused else (None, None, None, None, None, 0, None, None, 0, None, None,
                                    None))
        call("d3_moe_front", ptr(occupancy), slots, ptr(active), ptr(count), ptr(x), x.stride(0),
             ptr(logits), dtype_code(logits.dtype), logits.stride(0), s.rows, ptr(row_index),
             ptr(row_count), s.hidden, s.num_experts, s.top_k, ptr(self.ids), ptr(self.weights),
             dtype_code(self.weights.dtype), ptr(self.q), ptr(self.x_scales), self.tile,
             self.item_rows, *sort_args, stream)
        if not fused and not self.sortless and not self.by_pair:
            self.sort(None, count if occupancy is not None else row_count, stream)

    def fc1(self, experts, stream=None) -> None:
        s, stream = self.shape, self._stream(stream)
        w, ws, layout = fc1_operands(experts)
        call("d3_expert_gemm", 0, ptr(w), ptr(ws), layout,
             s.num_experts, 2 * s.intermediate, s.hidden, ptr(self.q), ptr(self.x_scales),
             ptr(self.sorted_ids), s.top_k, ptr(self.items), ptr(self.num_items), self.max_items,
             self.item_rows, self.exact_routes, ptr(self.gate_up), None, stream)

    def _shared_operands(self, shared, operands, layout):
        if shared is None:
            return None, None, 0
        if self.shared_rows < self.shape.rows:
            raise ValueError("fold a shared expert into a workspace built with shared_rows >= rows")
        w, ws, shared_layout = operands(shared)
        if shared_layout != layout:
            raise ValueError("the shared expert's weights must use the routed experts' layout")
        if w.shape[0] != 1:
            raise ValueError("a shared expert is one [1, N, K] expert")
        return w, ws, self.shape.rows

    def grouped_fc1(self, experts, shared=None, stream=None) -> None:
        """Tiled grouped FC1 + SwiGLU requant: act / act_scales at sorted rows
        (and, with ``shared``, the dense shared expert's rows after them)."""
        s, stream = self.shape, self._stream(stream)
        w, ws, layout = fc1_operands(experts)
        sw, sws, srows = self._shared_operands(shared, fc1_operands, layout)
        call("d3_grouped_fc1_swiglu", ptr(w), ptr(ws), layout, s.num_experts, s.intermediate,
             s.hidden, ptr(self.q), s.rows, ptr(self.x_scales), ptr(self.sorted_ids), s.top_k,
             ptr(self.items), ptr(self.num_items), self.max_items, self.item_rows, ptr(sw),
             ptr(sws), srows, self.max_rows, ptr(self.act), ptr(self.act_scales), stream)

    def grouped_fc2(self, experts, shared=None, stream=None) -> None:
        """Tiled grouped FC2: fp32 down rows by pair (and, with ``shared``, the
        shared expert's rows after the pairs: ``shared_down``)."""
        s, stream = self.shape, self._stream(stream)
        w, ws, layout = fc2_operands(experts)
        sw, sws, srows = self._shared_operands(shared, fc2_operands, layout)
        call("d3_grouped_fc2", ptr(w), ptr(ws), layout, s.num_experts, s.hidden, s.intermediate,
             ptr(self.act), self.max_rows + self.shared_rows, ptr(self.act_scales),
             ptr(self.sorted_ids), s.top_k, ptr(self.items), ptr(self.num_items), self.max_items,
             self.item_rows, ptr(sw), ptr(sws), srows, self.max_rows, s.pairs, ptr(self.down),
             stream)

    def grouped_fc1_by_pair(self, experts, row_count=None, stream=None) -> None:
        """Grouped FC1 + SwiGLU requant without a sorted route list: the
        routes found as ``list_ids`` / ``list_items`` / ``list_count``, act /
        act_scales at the list's positions."""
        s, stream = self.shape, self._stream(stream)
        w, ws, layout = fc1_operands(experts)
        count = self.rows_dev if row_count is None else row_count
        call("d3_grouped_fc1_swiglu_by_pair", ptr(w), ptr(ws), layout, s.num_experts,
             s.intermediate, s.hidden, ptr(self.q), s.rows, ptr(self.x_scales), ptr(self.ids),
             s.top_k, ptr(count), s.rows, ptr(self.act), ptr(self.act_scales),
             ptr(self.list_ids), ptr(self.list_items), ptr(self.list_count), stream)

    def grouped_fc2_listed(self, experts, stream=None) -> None:
        """Grouped FC2 over the route list grouped_fc1_by_pair wrote: fp32
        down rows by pair."""
        s, stream = self.shape, self._stream(stream)
        w, ws, layout = fc2_operands(experts)
        call("d3_grouped_fc2", ptr(w), ptr(ws), layout, s.num_experts, s.hidden, s.intermediate,
             ptr(self.act), len(self.act), ptr(self.act_scales), ptr(self.list_ids), s.top_k,
             ptr(self.list_items), ptr(self.list_count), self.list_items_max, GROUPED_ROUTES,
             None, None, 0, 0, 0, ptr(self.down), stream)

    @property
    def shared_down(self) -> torch.Tensor:
        """fp32 [rows, H] output of a folded shared expert."""
        return self.down[self.shape.pairs:self.shape.pairs + self.shape.rows]

    def activation(self, stream=None) -> None:
        s, stream = self.shape, self._stream(stream)
        call("d3_silu_mul_quant", ptr(self.gate_up), self.max_rows, s.intermediate,
             ptr(self.total), ptr(self.sorted_ids), ptr(self.pairs_dev), 0, ptr(self.act),
             ptr(self.act_scales), stream)

    def fc2(self, experts, stream=None) -> None:
        s, stream = self.shape, self._stream(stream)
        w, ws, layout = fc2_operands(experts)
        call("d3_expert_gemm", 1, ptr(w), ptr(ws), layout,
             s.num_experts, s.hidden, s.intermediate, ptr(self.act), ptr(self.act_scales),
             ptr(self.sorted_ids), s.top_k, ptr(self.items), ptr(self.num_items), self.max_items,
             self.item_rows, self.exact_routes, None, ptr(self.down), stream)

    def fc2_swiglu(self, experts, stream=None) -> None:
        """FC2 whose workgroups compute the SwiGLU requant of their routes
        from gate_up themselves (same bytes as activation() + fc2())."""
        s, stream = self.shape, self._stream(stream)
        w, ws, layout = fc2_operands(experts)
        call("d3_expert_fc2_swiglu", ptr(w), ptr(ws), layout, s.num_experts, s.hidden,
             s.intermediate, ptr(self.gate_up), ptr(self.sorted_ids), s.top_k, ptr(self.items),
             ptr(self.num_items), self.max_items, self.item_rows, self.exact_routes,
             ptr(self.down), stream)

    def combine(self, weights: torch.Tensor | None = None, row_count=None, shared=None,
                out=None, stream=None) -> torch.Tensor:
        s, stream = self.shape, self._stream(stream)
        weights = self.weights if weights is None else weights
        out = self.out if out is None else out
        call("d3_weighted_combine", ptr(self.down), ptr(weights), dtype_code(weights.dtype),
             s.rows, s.top_k, s.hidden, ptr(row_count), ptr(shared), ptr(out), stream)
        return out

    # -- whole step -------------------------------------------------------------
    def experts_forward(self, x, ids, weights, experts, row_index=None, row_count=None,
                        shared=None, out=None, stream=None) -> torch.Tensor:
        """Quantise, sort, FC1, SwiGLU requant, FC2, combine for given routes."""
        stream = _lib.stream(self.device) if stream is None else stream
        self.quantize(x, row_index, row_count, stream)
        self.sort(ids, row_count, stream)
        if self.grouped:
            self.grouped_fc1(experts, stream=stream)
            self.grouped_fc2(experts, stream=stream)
        else:
            self.fc1(experts, stream)
            self._fc2_stage(experts, stream)
        return self.combine(weights, row_count, shared, out, stream)

    def _fc2_stage(self, experts, stream) -> None:
        if self.swiglu_in_fc2:
            self.fc2_swiglu(experts, stream)
        else:
            self.activation(stream)
            self.fc2(experts, stream)

    def forward(self, x, logits, experts, row_index=None, row_count=None, shared=None,
                out=None, stream=None) -> torch.Tensor:
        """Route + experts.  ``row_index`` gathers x / logits rows (slot
        compaction), ``row_count`` is the live row count on the device."""
        stream = _lib.stream(self.device) if stream is None else stream
        self.front(x, logits, row_index, row_count, stream=stream)
        return self.experts(experts, row_count, shared, out, stream)

    def decode_fc1(self, experts, row_count=None, stream=None) -> None:
        """Sortless FC1: gate_up[pair] for every live route (fragment-major W13)."""
        s, stream = self.shape, self._stream(stream)
        w, ws, layout = fc1_operands(experts)
        if layout != LAYOUT_FRAGMENT:
            raise ValueError("sortless decode needs fragment-major weights (prepare_experts)")
        call("d3_decode_expert_gemm", 0, ptr(w), ptr(ws), s.num_experts, 2 * s.intermediate,
             s.hidden, ptr(self.ids), ptr(row_count), None, s.rows, s.top_k, ptr(self.q),
             ptr(self.x_scales), self.exact_routes, ptr(self.gate_up), None, stream)

    def decode_fc2(self, experts, row_count=None, stream=None, row_slots=None) -> None:
        """Sortless FC2 with the SwiGLU requant in its prologue: down[pair],
        or down[slot pair] with ``row_slots`` (decode_route_fc1's
        ``active``), the layout decode_route_combine reads."""
        s, stream = self.shape, self._stream(stream)
        w, ws, layout = fc2_operands(experts)
        if layout != LAYOUT_FRAGMENT:
            raise ValueError("sortless decode needs fragment-major weights (prepare_experts)")
        require_cuda(row_slots)
        call("d3_decode_expert_gemm", 2, ptr(w), ptr(ws), s.num_experts, s.hidden,
             s.intermediate, ptr(self.ids), ptr(row_count), ptr(row_slots), s.rows, s.top_k,
             ptr(self.gate_up), None, self.exact_routes, None, ptr(self.down), stream)

    def decode_route_fc1(self, experts, occupancy, x, logits, active, count,
                         stream=None) -> None:
        """Sortless FC1 straight from the slots (no front launch): every
        workgroup ranks its expert in each occupied slot, quantises its
        routes' x rows itself and writes gate_up[pair]; also writes ids,
        ``count`` and ``active`` as the front would (not q / x_scales)."""
        s, stream = self.shape, self._stream(stream)
        w, ws, layout = fc1_operands(experts)
        if layout != LAYOUT_FRAGMENT:
            raise ValueError("sortless decode needs fragment-major weights (prepare_experts)")
        call("d3_decode_route_fc1", ptr(w), ptr(ws), s.num_experts, 2 * s.intermediate, s.hidden,
             ptr(occupancy), s.rows, ptr(x), x.stride(0), ptr(logits), dtype_code(logits.dtype),
             logits.stride(0), s.top_k, self.exact_routes, ptr(self.ids), ptr(count),
             ptr(active), ptr(self.gate_up), stream)

    def decode_step(self, experts, occupancy, x, logits, active, count, out=None,
                    stream=None) -> torch.Tensor:
        """decode_route_fc1 + decode_fc2 + decode_route_combine as one C call
        (``d3_decode_step``: every stage checked before the first launch)."""
        s, stream = self.shape, self._stream(stream)
        out = self.out if out is None else out
        w13, s13, l13 = fc1_operands(experts)
        w2, s2, l2 = fc2_operands(experts)
        if l13 != LAYOUT_FRAGMENT or l2 != LAYOUT_FRAGMENT:
            raise ValueError("sortless decode needs fragment-major weights (prepare_experts)")
        call("d3_decode_step", ptr(w13), ptr(s13), ptr(w2), ptr(s2), s.num_experts, s.hidden,
             s.intermediate, ptr(occupancy), s.rows, ptr(x), x.stride(0), ptr(logits),
             dtype_code(logits.dtype), logits.stride(0), s.top_k, self.exact_routes,
             ptr(self.ids), ptr(self.weights), dtype_code(self.weights.dtype), ptr(self.gate_up),
             ptr(self.down), ptr(active), ptr(count), ptr(out), stream)
        return out

    def decode_route_combine(self, occupancy, logits, out=None, stream=None) -> torch.Tensor:
        """Combine of the step started by decode_route_fc1: the routing weights
        are recomputed from the logits (and stored in ``weights``)."""
        s, stream = self.shape, self._stream(stream)
        out = self.out if out is None else out
        call("d3_decode_route_combine", ptr(occupancy), s.rows, ptr(logits),
             dtype_code(logits.dtype), logits.stride(0), s.num_experts, s.top_k, s.hidden,
             ptr(self.down), ptr(self.weights), dtype_code(self.weights.dtype), ptr(out), stream)
        return out

    def experts(self, experts, row_count=None, shared=None, out=None, stream=None):
        """FC1, SwiGLU requant, FC2 and combine over the routes sorted by
        front(); a dense shared expert is added by the combine."""
        stream = _lib.stream(self.device) if stream is None else stream
        self.routes_down(experts, row_count, stream)
        return self.combine(None, row_count, shared, out, stream)

    def routes_down(self, experts, row_count=None, stream=None) -> torch.Tensor:
        """Everything experts() runs before the combine: the fp32 per-route
        rows in ``down`` (by pair)."""
        stream = _lib.stream(self.device) if stream is None else stream
        if self.sortless:
            self.decode_fc1(experts, row_count, stream)
            self.decode_fc2(experts, row_count, stream)
        elif self.by_pair:
            self.grouped_fc1_by_pair(experts, row_count, stream)
            self.grouped_fc2_listed(experts, stream)
        elif self.grouped:
            self.grouped_fc1(experts, stream=stream)
            self.grouped_fc2(experts, stream=stream)
        else:
            self.fc1(experts, stream)
            self._fc2_stage(experts, stream)
        return self.down

    def combine_add_norm(self, shared, gate, residual, norm_weight, epsilon, inverse=None,
                         out=None, stream=None) -> torch.Tensor:
        """The weighted combine of ``down`` fused with
        ``combine_experts_add_norm(_inverse)``: row r of ``residual`` / ``out``
        takes MoE row ``inverse[r]`` (int64; None = r) of the routed combine,
        gated ``shared`` and ``gate``; ``residual`` is updated in place.  The
        same bytes as combine() followed by that operator."""
        s, stream = self.shape, self._stream(stream)
        require_cuda(shared, gate, residual, norm_weight, inverse, out)
        rows, width = residual.shape
        if width != s.hidden or shared.shape[1] != s.hidden or len(shared) < 1:
            raise ValueError("shared and residual rows must be [*, hidden]")
        if inverse is not None and (inverse.dtype != torch.int64 or inverse.numel() != rows):
            raise ValueError("inverse must be int64 [rows]")
        if inverse is None and rows > s.rows:
            raise ValueError("without inverse, residual rows index MoE rows directly")
        gate_stride = gate.stride(0)
        out = torch.empty_like(residual) if out is None else out
        call("d3_combine_routes_add_norm", ptr(self.down), ptr(self.weights),
             dtype_code(self.weights.dtype), s.top_k, ptr(shared), ptr(gate), gate_stride,
             ptr(inverse), ptr(residual), ptr(norm_weight), float(epsilon), rows, width, ptr(out),
             stream)
        return out


class DenseExpert:
    """A dense FP8 SwiGLU expert applied to every row (config-4 shared expert),
    run through the same kernels with the identity route list."""

    def __init__(self, rows: int, hidden: int, intermediate: int, device="cuda",
                 item_rows: int | None = None, exact_routes: int = EXACT_ROUTES,
                 grouped: bool | None = None):
        self.rows, self.hidden, self.intermediate = rows, hidden, intermediate
        self.exact_routes = exact_routes
        if grouped is None:
            grouped = (item_rows or GROUPED_ROUTES) <= GROUPED_ROUTES and \
                grouped_supported(hidden, intermediate)
        self.grouped = bool(grouped)
        item_rows = item_rows or (GROUPED_ITEM_ROUTES if self.grouped else 128)
        dev = torch.device(device)
        self.item_rows = item_rows
        chunks = -(-rows // item_rows)
        self.max_items = chunks
        items = [[0, c * item_rows, min(item_rows, rows - c * item_rows), 0] for c in range(chunks)]
        self.items = torch.tensor(items or [[0, 0, 0, 0]], dtype=torch.int32, device=dev)
        self.num_items = torch.tensor([chunks], dtype=torch.int32, device=dev)
        self.sorted_ids = torch.arange(max(rows, 1), dtype=torch.int32, device=dev)
        self.gate_up = torch.empty((rows, 2 * intermediate), dtype=torch.bfloat16, device=dev)
        self.act = torch.empty((rows, intermediate), dtype=torch.uint8, device=dev)
        self.act_scales = torch.empty((rows, intermediate // 128), dtype=torch.float32, device=dev)
        self.down = torch.empty((rows, hidden), dtype=torch.float32, device=dev)

    def forward(self, q, x_scales, experts, stream=None) -> torch.Tensor:
        """q / x_scales: the already quantised rows [rows, H]; returns fp32 [rows, H]."""
        stream = _lib.stream(q.device) if stream is None else stream
        h, i = self.hidden, self.intermediate
        w13, s13, layout13 = fc1_operands(experts)
        w2, s2, layout2 = fc2_operands(experts)
        if self.grouped:  # identity routes: top_k 1, sorted_ids = row
            call("d3_grouped_fc1_swiglu", ptr(w13), ptr(s13), layout13, 1, i, h, ptr(q),
                 q.shape[0], ptr(x_scales), ptr(self.sorted_ids), 1, ptr(self.items),
                 ptr(self.num_items), self.max_items, self.item_rows, None, None, 0, 0,
                 ptr(self.act), ptr(self.act_scales), stream)
            call("d3_grouped_fc2", ptr(w2), ptr(s2), layout2, 1, h, i, ptr(self.act), self.rows,
                 ptr(self.act_scales), ptr(self.sorted_ids), 1, ptr(self.items),
                 ptr(self.num_items), self.max_items, self.item_rows, None, None, 0, 0, 0,
                 ptr(self.down), stream)
            return self.down
        call("d3_expert_gemm", 0, ptr(w13), ptr(s13), layout13, 1, 2 * i, h, ptr(q),
             ptr(x_scales), ptr(self.sorted_ids), 1, ptr(self.items), ptr(self.num_items),
             self.max_items, self.item_rows, self.exact_routes, ptr(self.gate_up), None, stream)
        call("d3_silu_mul_quant", ptr(self.gate_up), self.rows, i, None, None, None, 0,
             ptr(self.act), ptr(self.act_scales), stream)
        call("d3_expert_gemm", 1, ptr(w2), ptr(s2), layout2, 1, h, i, ptr(self.act),
             ptr(self.act_scales), ptr(self.sorted_ids), 1, ptr(self.items), ptr(self.num_items),
             self.max_items, self.item_rows, self.exact_routes, None, ptr(self.down), stream)
        return self.down


def moe_with_shared(ws: MoEWorkspace, dense: DenseExpert | None, x, logits, experts,
                    shared_experts, row_index=None, row_count=None, out=None,
                    side: torch.cuda.Stream | None = None):
    """Routed top-k experts plus an always-on dense shared expert, the shape of
    the reference's ``moe_parts`` (``model.py:503-518``).  Returns ``out``
    [rows, H] bf16: the combine of the routed rows plus the shared output.

    With a tiled-grouped workspace built with ``shared_rows >= rows`` the
    shared expert's rows are extra work items of the routed FC1 / FC2
    launches (they fill those launches' last rounds instead of under-filling
    launches of their own).  Otherwise ``dense`` runs it: on ``side`` (a
    default-priority stream, as the reference runs its shared expert on a
    side stream joined before the combine, ``model.py:506-517``) or in line.
    Graph-capturable either way.
    """
    main = torch.cuda.current_stream(ws.device)
    stream = main.cuda_stream
    if ws.sortless:
        raise ValueError("moe_with_shared needs a sorted-route workspace")
    ws.front(x, logits, row_index, row_count, stream=stream)
    if ws.grouped and ws.shared_rows >= ws.shape.rows:
        ws.grouped_fc1(experts, shared_experts, stream=stream)
        ws.grouped_fc2(experts, shared_experts, stream=stream)
        return ws.combine(None, row_count, ws.shared_down, out, stream)
    if dense is None:
        raise ValueError("without a shared-expert workspace, pass a DenseExpert")
    if side is None:
        shared_y = dense.forward(ws.q, ws.x_scales, shared_experts, stream=stream)
    else:
        side.wait_stream(main)  # q / x_scales are ready
        shared_y = dense.forward(ws.q, ws.x_scales, shared_experts, stream=side.cuda_stream)
    # The routed experts as the workspace's front left them: sorted items, or
    # (by-pair workspaces, whose front skips the sort) the by-pair FC1 and
    # the FC2 over the route list it writes.
    ws.routes_down(experts, row_count, stream)
    if side is not None:
        main.wait_stream(side)
    return ws.combine(None, row_count, shared_y, out, stream)


def compact_slots(occupancy: torch.Tensor, active: torch.Tensor, count: torch.Tensor,
                  stream=None) -> None:
    """occupancy uint8 [S] -> active int32 [S] (ascending, -1 padded), count int32 [1]."""
    require_cuda(occupancy, active, count)
    stream = _lib.stream(occupancy.device) if stream is None else stream
    call("d3_compact_slots", ptr(occupancy), occupancy.numel(), ptr(active), ptr(count), stream)


def _strided_rows_inside(t: torch.Tensor, rows: int) -> bool:
    """Whether ``rows`` full row strides from ``t``'s first element lie inside
    its storage (the range a kernel's buffer view of the rows covers)."""
    return (t.storage_offset() + rows * t.stride(0)) * t.element_size() <= t.untyped_storage().nbytes()


class DecodeStep:
    """The 64-slot decode MoE step: device-side slot compaction, then route +
    experts over the live rows, everything sized for the slot capacity and
    driven by the device count (graph-capturable, no host sync).

    Output row r belongs to slot ``active[r]`` for r < ``count``.

    The sortless chain (``sortless``) normally starts with the front launch;
    with ``frontless`` (default: whenever the sortless chain runs and the
    inputs fit ``d3_decode_route_fc1``) the FC1 routes and quantises the
    slots itself and the combine recomputes the routing weights, so the step
    is three launches.  Same outputs (``out``, ``active``, ``count``,
    workspace ``ids`` / ``weights`` / ``gate_up`` / ``down``); ``q`` and
    ``x_scales`` are not written.
    """

    def __init__(self, slots: int, num_experts: int, hidden: int, intermediate: int,
                 top_k: int = 8, device="cuda", item_rows: int | None = None,
                 sortless: bool | None = None,
                 frontless: bool | None = None):
        dev = torch.device(device)
        self.slots = slots
        self.active = torch.empty(slots, dtype=torch.int32, device=dev)
        self.count = torch.empty(1, dtype=torch.int32, device=dev)
        # Decode items take the exact path of the expert GEMMs (never the
        # FP8-only tiled grouped GEMMs of prefill-sized batches).
        self.workspace = MoEWorkspace(Shape(slots, num_experts, hidden, intermediate, top_k), dev,
                                      item_rows=item_rows, grouped=False)
        # Sortless expert GEMMs (default when the slots' routes could reach
        # every expert: at least one route per expert at full occupancy, and
        # the shapes are in the compiled set) on fragment-major weights.
        # Measured at 64 slots: E128 (8 routes per expert) and the reference
        # model's E256 / I512 (2 per expert: 127 us against 134 us for the
        # sorted chain).
        lib = _lib.load()
        decode_shapes = (hidden // 128 in (8, 16) and intermediate // 128 in (2, 4, 6, 8)
                         and hidden % 128 == 0 and intermediate % 128 == 0
                         and hidden % lib.d3_expert_tile_rows(intermediate) == 0)
        dense = slots * top_k >= num_experts
        if sortless is None:
            sortless = decode_shapes and dense and slots <= 256 and top_k <= 8
        self.sortless = bool(sortless)
        self.frontless = self.sortless if frontless is None else bool(frontless)
        if self.frontless and not self.sortless:
            raise ValueError("frontless runs the sortless chain (sortless=True)")

    def __call__(self, occupancy, x_slots, logits_slots, experts, stream=None) -> torch.Tensor:
        stream = _lib.stream(x_slots.device) if stream is None else stream
        ws = self.workspace
        ws.sortless = self.sortless and self.uses_sortless(experts)
        if ws.sortless and self.uses_frontless(occupancy, x_slots, logits_slots):
            return ws.decode_step(experts, occupancy, x_slots, logits_slots, self.active,
                                  self.count, stream=stream)
        ws.front(x_slots, logits_slots, occupancy=occupancy, active=self.active,
                 count=self.count, stream=stream)
        return ws.experts(experts, self.count, stream=stream)

    def uses_frontless(self, occupancy, x_slots, logits_slots) -> bool:
        """Whether a call with these inputs runs the three-launch step."""
        s = self.workspace.shape
        if not self.frontless or logits_slots.dtype not in (torch.bfloat16, torch.float32):
            return False
        f32 = logits_slots.dtype == torch.float32
        per_chunk = 4 if f32 else 8
        return (occupancy.dtype == torch.uint8 and occupancy.numel() == self.slots
                and x_slots.dtype == torch.bfloat16 and x_slots.dim() == 2
                and x_slots.shape[0] >= self.slots and x_slots.shape[1] == s.hidden
                and x_slots.stride(1) == 1 and x_slots.stride(0) % 8 == 0
                and x_slots.data_ptr() % 16 == 0
                and logits_slots.dim() == 2 and logits_slots.shape[0] >= self.slots
                and logits_slots.shape[1] == s.num_experts and logits_slots.stride(1) == 1
                and logits_slots.stride(0) % per_chunk == 0
                and logits_slots.data_ptr() % 16 == 0
                and s.num_experts <= 32 * per_chunk and s.top_k <= s.num_experts
                # the kernels' buffer ranges span slots * row stride elements
                and _strided_rows_inside(x_slots, self.slots)
                and _strided_rows_inside(logits_slots, self.slots))

    @staticmethod
    def uses_sortless_layout(experts) -> bool:
        return (fc1_operands(experts)[2] == LAYOUT_FRAGMENT
                and fc2_operands(experts)[2] == LAYOUT_FRAGMENT)

    def uses_sortless(self, experts) -> bool:
        return self.sortless and self.uses_sortless_layout(experts)
