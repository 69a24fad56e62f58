"""One Drama-3 MoE layer around the routed experts: ``DramaModel.moe_parts``
and ``DramaModel.moe`` (``src/drama3/model.py:485-518``) with persistent
buffers, graph-capturable.

The reference projects the layer input once through a packed bf16 matrix
(``packed_input_projection``, ``model.py:230-245``: the shared expert's
gate and up rows, the router, the shared-expert gate, zero-padded by 127
rows), runs the bf16 shared expert (``silu_mul`` then ``down_proj``) on a
side stream while the routed top-8 FP8 experts run on the main stream, and
joins before the combine (``model.py:506-518``).

Here both bf16 GEMMs are this package's MFMA kernels at every batch size
(``d3_dense_bf16``: the projection, whose epilogue also writes the shared
expert's ``silu_mul`` activation, and the shared down projection; a
streaming kernel up to 768 rows, a tiled one above).  With at most 256
rows the routed experts are the decode step, whose combine is folded into
the layer's (``d3_combine_route_logits``: routing weights, rank-order
routed sum, gated shared add and optionally the residual + RMSNorm of
``combine_experts_add_norm``, one launch); larger batches run the prefill
path, whose routed combine is folded into the layer's the same way
(``d3_combine_routes_add_norm`` over the fp32 per-route rows).  ``overlap``
puts the shared expert on a default-priority side stream
forked after the projection and joined before the combine.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _lib
from ._lib import call, ptr
from .pipeline import DTYPE_BF16, DecodeStep, MoEWorkspace, Shape, dtype_code, require_cuda

PROJECTION_PADDING = 127  # zero rows the reference appends (model.py:236-245)
DENSE_ROWS = 768  # most rows of d3_dense_bf16's streaming (small-batch) kernel
DENSE_K = (256, 512, 768, 1024, 1536, 2048)  # its contraction lengths
TILED_K = 64  # the tiled kernel (more rows): K a multiple of this
TILED_PAIRS = 64  # and gate / up pair rows a multiple of this


def dense_supported(rows: int, n: int, k: int, pair_rows: int = 0) -> bool:
    """Whether ``d3_dense_bf16`` covers an [rows, k] x [n, k]^T product with
    ``pair_rows`` gate / up pairs (the checks of its C entry point)."""
    if n % 16 or pair_rows % 16 or 2 * pair_rows > n or k <= 0:
        return False
    if rows <= DENSE_ROWS and k in DENSE_K:
        return True
    return k % TILED_K == 0 and pair_rows % TILED_PAIRS == 0


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


def dense_bf16(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor, pair_rows: int = 0,
               act: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """``out = x @ weight.T`` on the MFMA kernel (``d3_dense_bf16``).  With
    ``pair_rows`` P and ``act``, weight rows [0, P) / [P, 2P) are a gate /
    up pair and ``act`` receives ``silu_mul`` of the rounded outputs."""
    require_cuda(x, weight, out, act)
    if any(t is not None and t.dtype != torch.bfloat16 for t in (x, weight, out, act)):
        raise TypeError("dense_bf16 takes bf16 operands")
    n, k = weight.shape
    if weight.stride(1) != 1 or weight.stride(0) != k or x.stride(1) != 1 or out.stride(1) != 1:
        raise ValueError("weight must be contiguous, x and out rows unit-stride")
    if x.shape[1] != k or out.shape != (x.shape[0], n):
        raise ValueError("shapes do not match the projection")
    if act is not None and (act.shape != (x.shape[0], pair_rows) or act.stride(1) != 1):
        raise ValueError("act must be [rows, pair_rows] with unit column stride")
    stream = _lib.stream(x.device) if stream is None else stream
    call("d3_dense_bf16", ptr(x), x.stride(0), x.shape[0], ptr(weight), n, k, pair_rows, ptr(out),
         out.stride(0), ptr(act), act.stride(0) if act is not None else 0, stream)
    return out


class MoELayer:
    """``moe_parts`` / ``moe`` of one layer for up to ``rows`` rows.

    ``parts(x, ...)`` returns (routed, shared, shared_gate) views into the
    layer's buffers; ``__call__`` returns ``combine_experts`` of them and
    ``add_norm`` the residual + RMSNorm form (``combine_experts_add_norm``).
    Routed experts: with ``rows <= 256`` the decode step (``DecodeStep``
    with every row a live slot), otherwise the prefill path
    (``MoEWorkspace``: routes sorted, tiled grouped GEMMs when the shapes
    allow).  ``overlap`` runs the shared expert on a side stream; off by
    default: on MI355X the in-line order measured faster, the routed GEMMs
    already filling the device while they stream their weights.
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
        self.norm_out = torch.empty((rows, hidden), **bf16)
        # both bf16 GEMMs on d3_dense_bf16 (no library GEMM on the path)
        if not (dense_supported(rows, width, hidden, shared_intermediate)
                and dense_supported(rows, hidden, shared_intermediate)):
            raise ValueError(
                f"d3_dense_bf16 does not cover this layer: hidden {hidden} and shared "
                f"intermediate {shared_intermediate} must be in {DENSE_K} (up to {DENSE_ROWS} "
                f"rows) or multiples of {TILED_K}, the projection width {width} a multiple of 16")
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

    def _check(self, x, projection, down_proj) -> None:
        require_cuda(x, projection, down_proj)
        if x.shape != (self.rows, self.hidden) or x.dtype != torch.bfloat16:
            raise ValueError(f"x must be bf16 [{self.rows}, {self.hidden}]")
        if projection.shape != (self.projected.shape[1], self.hidden):
            raise ValueError("projection must be pack_input_projection's [N, H]")
        if down_proj.shape != (self.hidden, self.shared_intermediate):
            raise ValueError("down_proj must be [H, shared_intermediate]")

    def _project(self, x, projection) -> None:
        """The packed projection; its epilogue also writes the shared
        expert's activation ``silu_mul(gate | up)``."""
        dense_bf16(x, projection.contiguous(), self.projected, self.shared_intermediate, self.act)

    def _shared_expert(self, down_proj) -> None:
        """The shared expert's down projection of the activation the
        projection wrote."""
        dense_bf16(self.act, down_proj.contiguous(), self.shared)

    def _fused(self, experts, x, router) -> bool:
        """Whether the routed combine folds into the layer's combine: the
        decode step's three-launch path (routes ranked inside FC1)."""
        step = self.step if self.decode else None
        return (step is not None and step.sortless and step.uses_sortless(experts)
                and step.uses_frontless(self.all_rows, x, router) and self.hidden <= 2048
                and self.num_experts <= 256)

    def _routed_and_shared(self, x, projection, down_proj, experts, fuse: bool,
                           routes: bool = False):
        """Projection, routed experts (without their combine when ``fuse``,
        the decode step's; or when ``routes``, the prefill path's: the fp32
        per-route rows only) and shared expert; returns the router logits
        view."""
        self._check(x, projection, down_proj)
        main = torch.cuda.current_stream(self.device)
        self._project(x, projection)
        _, router, _ = self._views()
        if self.side is not None:
            # Fork after the projection; join before the outputs are read
            # (the reference's moe_shared_stream, model.py:506-517).
            self.side.wait_stream(main)
            with torch.cuda.stream(self.side):
                self._shared_expert(down_proj)
        if fuse:
            ws, stream = self.step.workspace, _lib.stream(self.device)
            ws.decode_route_fc1(experts, self.all_rows, x, router, self.step.active,
                                self.step.count, stream)
            ws.decode_fc2(experts, self.step.count, stream)
        elif self.decode:
            self.routed = self.step(self.all_rows, x, router, experts)
        elif routes:
            stream = _lib.stream(self.device)
            self.workspace.front(x, router, stream=stream)
            self.workspace.routes_down(experts, stream=stream)
        else:
            self.workspace.forward(x, router, experts, out=self.routed)
        if self.side is None:
            self._shared_expert(down_proj)
        else:
            main.wait_stream(self.side)
        return router

    def parts(self, x: torch.Tensor, projection: torch.Tensor, down_proj: torch.Tensor, experts):
        """x bf16 [rows, H]; projection = ``pack_input_projection(...)``;
        down_proj bf16 [H, shared_intermediate].  Returns (routed [rows, H],
        shared [rows, H], shared_gate [rows, 1])."""
        self._routed_and_shared(x, projection, down_proj, experts, fuse=False)
        _, _, shared_gate = self._views()
        return self.routed, self.shared, shared_gate

    def _combine(self, x, projection, down_proj, experts, residual=None, norm_weight=None,
                 eps=0.0, out=None) -> torch.Tensor:
        fuse = self._fused(experts, x, self._views()[1])
        # prefill-sized batches: the routed combine folds into the gated
        # shared add (and the norm), one launch over the per-route rows
        routes = not self.decode
        router = self._routed_and_shared(x, projection, down_proj, experts, fuse, routes)
        _, _, gate = self._views()
        stream = _lib.stream(self.device)
        if routes:
            ws = self.workspace
            call("d3_combine_routes_add_norm", ptr(ws.down), ptr(ws.weights),
                 dtype_code(ws.weights.dtype), ws.shape.top_k, ptr(self.shared), ptr(gate),
                 gate.stride(0), None, ptr(residual), ptr(norm_weight), float(eps), self.rows,
                 self.hidden, ptr(out), stream)
        elif fuse:
            ws = self.step.workspace
            call("d3_combine_route_logits", ptr(ws.down), ptr(router), DTYPE_BF16, router.stride(0),
                 self.num_experts, ws.shape.top_k, ptr(ws.weights), dtype_code(ws.weights.dtype),
                 ptr(self.shared), ptr(gate), gate.stride(0), ptr(residual), ptr(norm_weight),
                 float(eps), self.rows, self.hidden, ptr(out), stream)
        elif residual is None:
            call("d3_combine_experts", ptr(self.routed), ptr(self.shared), ptr(gate),
                 gate.stride(0), self.rows, self.hidden, ptr(out), stream)
        else:
            call("d3_combine_experts_add_norm", ptr(self.routed), ptr(self.shared), ptr(gate),
                 gate.stride(0), None, ptr(residual), ptr(norm_weight), float(eps), self.rows,
                 self.hidden, ptr(out), stream)
        return out

    def __call__(self, x, projection, down_proj, experts) -> torch.Tensor:
        """``moe``: combine_experts(routed, shared, shared_gate) -> bf16 [rows, H]."""
        return self._combine(x, projection, down_proj, experts, out=self.out)

    def add_norm(self, x, projection, down_proj, experts, residual: torch.Tensor,
                 norm_weight: torch.Tensor, eps: float) -> torch.Tensor:
        """``combine_experts_add_norm`` of the layer (``kernels.py:448-499``,
        as the backbone applies it, ``model.py:596-606``): residual is
        updated in place, the (1 + w) RMS-normalised rows are returned."""
        require_cuda(residual, norm_weight)
        if (residual.shape != (self.rows, self.hidden) or residual.dtype != torch.bfloat16
                or not residual.is_contiguous()):
            raise ValueError("residual must be contiguous bf16 [rows, hidden]")
        if norm_weight.shape != (self.hidden,) or norm_weight.dtype != torch.bfloat16:
            raise ValueError("norm weight must be bf16 [hidden]")
        return self._combine(x, projection, down_proj, experts, residual,
                             norm_weight.contiguous(), eps, out=self.norm_out)
