"""One Drama-3 MoE layer around the routed experts: ``DramaModel.moe_parts``
and ``DramaModel.moe`` (``src/drama3/model.py:485-518``) with persistent
buffers, graph-capturable.

The reference projects the layer input once through a packed bf16 matrix
(``packed_input_projection``, ``model.py:230-245``: the shared expert's
gate and up rows, the router, the shared-expert gate, zero-padded by 127
rows), runs the bf16 shared expert (``silu_mul`` then ``down_proj``) on a
side stream while the routed top-8 FP8 experts run on the main stream, and
joins before the combine (``model.py:506-518``).  Here the two bf16 GEMMs
are plain library GEMMs (``torch.mm``, two-dimensional: hipBLASLt), the
SwiGLU, the routed experts and the combine are this package's kernels, and
the side stream is a default-priority stream forked after the projection
and joined before the routed rows are read.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _lib
from ._lib import call, ptr
from .pipeline import DecodeStep, MoEWorkspace, Shape, require_cuda

PROJECTION_PADDING = 127  # zero rows the reference appends (model.py:236-245)


def pack_input_projection(gate_proj: torch.Tensor, up_proj: torch.Tensor, router: torch.Tensor,
                          shared_gate: torch.Tensor) -> torch.Tensor:
    """``packed_input_projection`` (``model.py:230-245``): rows
    ``[shared gate_proj; shared up_proj; router; shared_expert_gate; 0 x 127]``
    of a bf16 [N, H] projection."""
    parts = (gate_proj, up_proj, router, shared_gate)
    hidden = gate_proj.shape[1]
    if any(p.dim() != 2 or p.shape[1] != hidden for p in parts) or shared_gate.shape[0] != 1:
        raise ValueError("projections must be [*, hidden] and the shared gate [1, hidden]")
    if gate_proj.shape != up_proj.shape:
        raise ValueError("shared gate_proj and up_proj must have the same shape")
    return F.pad(torch.cat(parts), (0, 0, 0, PROJECTION_PADDING))


class MoELayer:
    """``moe_parts`` / ``moe`` of one layer for up to ``rows`` rows.

    ``parts(x, ...)`` returns (routed, shared, shared_gate) views into the
    layer's buffers; ``__call__`` adds ``combine_experts``.  Routed experts:
    with ``rows <= 256`` the decode step (``DecodeStep`` with every row a
    live slot), otherwise the prefill path (``MoEWorkspace``: routes sorted,
    tiled grouped GEMMs when the shapes allow).  ``overlap`` runs the shared
    expert on a side stream; off by default: on MI355X the in-line order
    measured faster (one reference-shape layer, 64 rows: 147.4 us in line,
    158.7 us with the side stream), the routed GEMMs already filling the
    device while they stream their weights.
    """

    def __init__(self, rows: int, num_experts: int, hidden: int, intermediate: int,
                 shared_intermediate: int, top_k: int = 8, device="cuda", overlap: bool = False):
        dev = torch.device(device)
        self.device, self.rows, self.hidden = dev, rows, hidden
        self.num_experts, self.shared_intermediate = num_experts, shared_intermediate
        width = 2 * shared_intermediate + num_experts + 1 + PROJECTION_PADDING
        bf16 = dict(dtype=torch.bfloat16, device=dev)
        # One spare row: the router columns are a strided view starting past
        # the row start, and the decode kernels' buffer range spans rows full
        # row strides from that start.
        self.projected_storage = torch.zeros((rows + 1, width), **bf16)
        self.projected = self.projected_storage[:rows]
        self.act = torch.empty((rows, shared_intermediate), **bf16)
        self.shared = torch.empty((rows, hidden), **bf16)
        self.out = torch.empty((rows, hidden), **bf16)
        self.decode = rows <= 256
        if self.decode:
            self.step = DecodeStep(rows, num_experts, hidden, intermediate, top_k, device=dev)
            self.all_rows = torch.ones(rows, dtype=torch.uint8, device=dev)
        else:
            self.workspace = MoEWorkspace(Shape(rows, num_experts, hidden, intermediate, top_k),
                                          dev)
            self.routed = torch.empty((rows, hidden), **bf16)
        self.side = torch.cuda.Stream(dev) if overlap else None

    def _views(self):
        s = self.shared_intermediate
        gate_up = self.projected[:, :2 * s]
        router = self.projected[:, 2 * s:2 * s + self.num_experts]
        shared_gate = self.projected[:, 2 * s + self.num_experts:2 * s + self.num_experts + 1]
        return gate_up, router, shared_gate

    def _shared_expert(self, gate_up, down_proj) -> None:
        stream = _lib.stream(self.device)
        call("d3_silu_mul", ptr(gate_up), gate_up.stride(0), self.rows, self.shared_intermediate,
             ptr(self.act), stream)
        torch.mm(self.act, down_proj.t(), out=self.shared)

    def parts(self, x: torch.Tensor, projection: torch.Tensor, down_proj: torch.Tensor, experts):
        """x bf16 [rows, H]; projection = ``pack_input_projection(...)``;
        down_proj bf16 [H, shared_intermediate].  Returns (routed [rows, H],
        shared [rows, H], shared_gate [rows, 1])."""
        require_cuda(x, projection, down_proj)
        if x.shape != (self.rows, self.hidden) or x.dtype != torch.bfloat16:
            raise ValueError(f"x must be bf16 [{self.rows}, {self.hidden}]")
        if projection.shape != (self.projected.shape[1], self.hidden):
            raise ValueError("projection must be pack_input_projection's [N, H]")
        if down_proj.shape != (self.hidden, self.shared_intermediate):
            raise ValueError("down_proj must be [H, shared_intermediate]")
        main = torch.cuda.current_stream(self.device)
        torch.mm(x, projection.t(), out=self.projected)
        gate_up, router, shared_gate = self._views()
        if self.side is not None:
            # Fork after the projection; join before the outputs are read
            # (the reference's moe_shared_stream, model.py:506-517).
            self.side.wait_stream(main)
            with torch.cuda.stream(self.side):
                self._shared_expert(gate_up, down_proj)
        if self.decode:
            routed = self.step(self.all_rows, x, router, experts)
            self.routed = routed  # the decode step's output buffer
        else:
            routed = self.workspace.forward(x, router, experts, out=self.routed)
        if self.side is None:
            self._shared_expert(gate_up, down_proj)
        else:
            main.wait_stream(self.side)
        return routed, self.shared, shared_gate

    def __call__(self, x, projection, down_proj, experts) -> torch.Tensor:
        """``moe``: combine_experts(routed, shared, shared_gate) -> bf16 [rows, H]."""
        routed, shared, gate = self.parts(x, projection, down_proj, experts)
        call("d3_combine_experts", ptr(routed), ptr(shared), ptr(gate), gate.stride(0), self.rows,
             self.hidden, ptr(self.out), _lib.stream(self.device))
        return self.out
