"""numpy restatement of the reference's packed FP8 top-8 MoE step.

Test infrastructure only (see ``oracle/__init__.py``).  Shapes are generalised
over (E experts, H hidden, I intermediate, K = top-k); the reference hard-codes
E=256, H=2048, I=512, K=8.

Array conventions: bf16 tensors are uint16 bit patterns, fp8 tensors are
uint8 e4m3fn codes, everything else is a numpy array of the stated dtype.
Weight layout (reference ``kernels.py:290-318``, ``model.py:196-199``):
    w13 [E, 2I, H] e4m3 rows [gate; up];  s13 [E, 2I/128, H/128] f32
    w2  [E, H, I]  e4m3;                  s2  [E, H/128, I/128] f32
Dequantised weight = e4m3 value x block scale.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .numerics import (
    bf16_to_f32,
    e4m3_to_f32,
    f32_bits,
    f32_to_bf16,
    f32_to_e4m3,
    f64_to_bf16,
    round_bf16,
)

GROUP = 128
FP8_MAX = np.float32(448.0)
SCALE_FLOOR = np.float32(1e-10)


# ---------------------------------------------------------------------------
# A1 active-slot compaction
# ---------------------------------------------------------------------------
def compact_slots(occupancy: np.ndarray) -> tuple[np.ndarray, int]:
    """Ascending list of occupied slots and its length.

    Reference: the engine filters live requests on the host
    (``engine.py:637-643``), builds the slot list (``engine.py:136-144``) and
    the device gathers per-slot state row by row (``runtime_state.py:10-32``).
    The device contract restated here is the one the MI355X build exposes:
    occupancy bytes [S] -> int32 slots in ascending order, no padding rows.
    """
    occ = np.asarray(occupancy).astype(bool)
    active = np.flatnonzero(occ).astype(np.int32)
    return active, int(active.size)


# ---------------------------------------------------------------------------
# A3 routing
# ---------------------------------------------------------------------------
def route_keys(logits: np.ndarray) -> np.ndarray:
    """32-bit ranking keys of ``route_kernel`` (``kernels.py:364-368``).

    ``ordered`` maps fp32 bits to an unsigned order; only its top 16 bits (the
    bf16 value) are kept and the low 16 bits hold ``65535 - column`` so equal
    values rank the lower expert index first.
    """
    bits = f32_bits(np.asarray(logits, dtype=np.float32)).astype(np.uint64)
    negative = (bits & 0x80000000) != 0
    ordered = np.where(negative, bits ^ 0xFFFFFFFF, bits ^ 0x80000000) & 0xFFFFFFFF
    columns = np.arange(logits.shape[-1], dtype=np.uint64)
    return ((ordered & 0xFFFF0000) | (65535 - columns)).astype(np.uint32)


def route(logits: np.ndarray, top_k: int = 8, out_dtype: str = "bf16"):
    """``route(logits) -> (weights, ids)`` of ``kernels.py:360-383``.

    Per row: fp32 softmax over all E logits, top-k by ``route_keys`` in
    descending key order, weights = p / sum(selected p), stored in the logits
    dtype.  The exponentials and sums are evaluated in float64 from the fp32
    differences ``l - max`` the reference forms, so this is the exactly
    rounded value of the reference formula; device results are compared
    within one bf16 ulp.

    logits: float32 values [T, E] (bf16 logits passed as their exact f32 value).
    Returns (weights [T,k] uint16 bf16 bits or float32, ids [T,k] int64).
    """
    logits = np.asarray(logits, dtype=np.float32)
    keys = route_keys(logits)
    ids = np.argsort(-keys.astype(np.int64), axis=-1, kind="stable")[:, :top_k]
    row_max = logits.max(axis=-1, keepdims=True)
    # fp32 subtraction, as the kernel; a row holding +inf gives inf - inf =
    # NaN there too (its weights are NaN; its ids still follow the keys)
    with np.errstate(invalid="ignore"):
        shifted = (logits - row_max).astype(np.float32)
    exps = np.exp(shifted.astype(np.float64))
    denominator = exps.sum(axis=-1, keepdims=True)
    selected = np.take_along_axis(exps, ids, axis=-1) / denominator
    weights = (selected / selected.sum(axis=-1, keepdims=True)).astype(np.float32)
    if out_dtype == "bf16":
        weights = f32_to_bf16(weights)
    return weights, ids.astype(np.int64)


def softmax_topk(logits: np.ndarray, top_k: int = 8):
    """Prefill routing of ``model.py:526-528``: softmax, ``topk``, renormalise.

    ``torch.topk`` breaks ties by an unspecified order, so the MI355X build
    uses ``route_keys`` everywhere; for logits with distinct bf16 values the
    two agree (pinned in ``tests/test_oracle_route.py``).
    """
    return route(logits, top_k)


# ---------------------------------------------------------------------------
# A4 per-128 FP8 activation quantisation
# ---------------------------------------------------------------------------
def quantize_rows(x: np.ndarray, group: int = GROUP):
    """Per-row, per-128-column e4m3 quantisation (``moe_input.py:24-27``).

    ``scale = max(max|x|, 1e-10) / 448`` in fp32 and
    ``q = e4m3(clamp(x / scale, -448, 448))``.  The reference validates this
    byte-for-byte against Fish's ``quant_kernel`` (``validate_moe_input.py:38-61``).

    x: float32 [T, W] (bf16 activations as exact f32).  W % group == 0.
    Returns (q uint8 [T, W], scales float32 [T, W/group]).
    """
    x = np.asarray(x, dtype=np.float32)
    rows, width = x.shape
    if width % group:
        raise ValueError("quantisation width must be a multiple of the group")
    grouped = x.reshape(rows, width // group, group)
    amax = np.abs(grouped).max(axis=-1)
    scales = (np.maximum(amax, SCALE_FLOOR) / FP8_MAX).astype(np.float32)
    scaled = (grouped / scales[..., None]).astype(np.float32)  # IEEE fp32 division
    clamped = np.clip(scaled, -FP8_MAX, FP8_MAX)
    q = f32_to_e4m3(clamped).reshape(rows, width)
    return q, scales


def dequantize_rows(q: np.ndarray, scales: np.ndarray, group: int = GROUP) -> np.ndarray:
    """fp32 ``q * scale`` per element, as the expert kernels form ``x * x_scale``."""
    values = e4m3_to_f32(q)
    return (values * np.repeat(scales, group, axis=-1)).astype(np.float32)


def prepare_moe_input(x_bf16, router, row_slots=None, padding_start=None, group: int = GROUP):
    """``prepare_moe_input`` of ``moe_input.py:40-79``.

    Returns (q [T,H] e4m3 codes, scales [H/128, T] f32 (transposed layout),
    logits [T,E] f32).  Rows whose slot is >= ``padding_start`` take row 0's
    router logits (``moe_input.py:31-37``); quantisation stays per row.
    """
    x = bf16_to_f32(x_bf16)
    q, scales = quantize_rows(x, group)
    logits = np.asarray(router, dtype=np.float32).copy()
    if row_slots is not None:
        padding = np.asarray(row_slots) >= padding_start
        logits[padding] = logits[0]
    return q, np.ascontiguousarray(scales.T), logits


# ---------------------------------------------------------------------------
# A5-A7 expert histogram, padded offsets, stable scatter (route sort)
# ---------------------------------------------------------------------------
def max_sorted_rows(pairs: int, num_experts: int, tile: int) -> int:
    """Sorted-buffer capacity of ``native_moe`` (``kernels.py:713``)."""
    raw = pairs + min(pairs, num_experts) * (tile - 1)
    return -(-raw // tile) * tile


@dataclass
class RouteSort:
    counts: np.ndarray  # int32 [E]
    starts: np.ndarray  # int32 [E]
    total: int
    sorted_ids: np.ndarray  # int32 [total]; padding slots hold the sentinel `pairs`
    expert_ids: np.ndarray  # int32 [total / tile]
    inverse: np.ndarray  # int32 [pairs]: sorted position of each pair (unpermute map)


def sort_routes(ids: np.ndarray, num_experts: int, tile: int) -> RouteSort:
    """Histogram + padded exclusive scan + stable scatter.

    ``expert_counts_kernel`` (``kernels.py:658-663``): counts[e] = #{p: ids[p]==e}.
    ``expert_offsets_kernel`` (``kernels.py:666-673``): padded = ceil(c/tile)*tile,
    starts = exclusive cumsum(padded), total = sum(padded).
    ``expert_scatter_kernel`` (``kernels.py:676-699``): pairs of expert e in
    ascending pair order at ``starts[e] + rank``; slots up to the padded end
    hold the sentinel ``pairs``; ``expert_ids[starts[e]/tile + b] = e``.
    ``inverse`` is the MI355X build's unpermute map (pair -> sorted position);
    the reference unpermutes by indexing with ``sorted_ids`` (``kernels.py:764-779``).
    """
    flat = np.asarray(ids).reshape(-1).astype(np.int64)
    pairs = flat.size
    counts = np.bincount(flat, minlength=num_experts).astype(np.int32)[:num_experts]
    padded = (-(-counts // tile) * tile).astype(np.int64)
    starts = (np.cumsum(padded) - padded).astype(np.int32)
    total = int(padded.sum())
    sorted_ids = np.full(total, pairs, dtype=np.int32)
    expert_ids = np.empty(total // tile, dtype=np.int32)
    order = np.argsort(flat, kind="stable")
    inverse = np.empty(pairs, dtype=np.int32)
    position = 0
    for e in range(num_experts):
        c = int(counts[e])
        members = order[position : position + c]
        position += c
        s = int(starts[e])
        sorted_ids[s : s + c] = members
        inverse[members] = np.arange(s, s + c, dtype=np.int32)
        expert_ids[s // tile : (s + int(padded[e])) // tile] = e
    return RouteSort(counts, starts, total, sorted_ids, expert_ids, inverse)


# ---------------------------------------------------------------------------
# A9-A11 expert FFN
# ---------------------------------------------------------------------------
def dequantize_weight(w: np.ndarray, s: np.ndarray) -> np.ndarray:
    """e4m3 weight [N, K] x block scales [N/128, K/128] -> fp32 ``w * scale``."""
    values = e4m3_to_f32(w)
    full = np.repeat(np.repeat(s, GROUP, axis=0), GROUP, axis=1)
    return (values * full).astype(np.float32)


def expert_matmul(activation_dq: np.ndarray, weight_dq: np.ndarray) -> np.ndarray:
    """sum_k (w * ws) * (x * xs) with fp32 operands, accumulated in float64.

    Reference FC1/FC2 arithmetic (``kernels.py:298-300,313-320``) is an fp32
    accumulation of these products; float64 accumulation gives the exactly
    rounded sum that every fp32 accumulation order approximates.
    """
    return (activation_dq.astype(np.float64) @ weight_dq.astype(np.float64).T).astype(np.float32)


def silu_mul(projected_bf16: np.ndarray) -> np.ndarray:
    """``silu_mul`` of ``kernels.py:386-402`` (bf16 in, bf16 out).

    ``activated = bf16(gate * sigmoid(gate))`` then ``out = bf16(activated * up)``.
    """
    width = projected_bf16.shape[-1] // 2
    gate = bf16_to_f32(projected_bf16[:, :width]).astype(np.float64)
    up = bf16_to_f32(projected_bf16[:, width:])
    sig = 1.0 / (1.0 + np.exp(-gate))
    activated = round_bf16((gate * sig).astype(np.float32))
    return f32_to_bf16((activated * up).astype(np.float32))


def swiglu_f32(gate_up_bf16: np.ndarray, silu_bf16: bool = False) -> np.ndarray:
    """fp32 SwiGLU of bf16 [gate | up] rows: ``silu(g) * u`` with
    ``silu(g) = g * sigmoid(g)``; sigmoid rounded once to fp32, then two fp32
    products.

    The reference applies Fish Speech's ``silu_mul_quant_kernel``
    (fish-speech @ 541566932abb, ``fp8_moe.py``, not vendored; called at
    ``kernels.py:344,748``), whose source is absent.  The build keeps fp32
    throughout, the arithmetic of the in-repo ``silu_mul``
    (``kernels.py:392-394``) without its bf16 roundings; ``silu_bf16=True``
    gives that kernel's other reading, ``silu(g)`` rounded to bf16 before the
    multiply, so its effect on the MoE output can be bounded.  Pinned against
    ``torch.nn.functional.silu`` (float32 and float64) and the mathematics'
    special values in ``tests/test_oracle_swiglu.py``.
    """
    width = gate_up_bf16.shape[-1] // 2
    gate = bf16_to_f32(gate_up_bf16[:, :width])
    up = bf16_to_f32(gate_up_bf16[:, width:])
    sig = (1.0 / (1.0 + np.exp(-gate.astype(np.float64)))).astype(np.float32)
    silu = (gate * sig).astype(np.float32)
    if silu_bf16:
        silu = round_bf16(silu)
    return (silu * up).astype(np.float32)


def silu_mul_quant(gate_up_bf16: np.ndarray, group: int = GROUP, silu_bf16: bool = False):
    """SwiGLU + per-128 e4m3 requantisation of the FC1 output (A10).

    Quantisation rule identical to ``quantize_rows``; the SwiGLU is
    ``swiglu_f32`` (``silu_bf16`` selects its bf16-rounded reading).
    """
    return quantize_rows(swiglu_f32(gate_up_bf16, silu_bf16), group)


@dataclass
class ExpertWeights:
    w13: np.ndarray  # uint8 [E, 2I, H]
    s13: np.ndarray  # f32 [E, 2I/128, H/128]
    w2: np.ndarray  # uint8 [E, H, I]
    s2: np.ndarray  # f32 [E, H/128, I/128]

    @property
    def shape(self):
        experts, two_i, hidden = self.w13.shape
        return experts, hidden, two_i // 2


@dataclass
class ExpertTrace:
    """Intermediate tensors of ``expert_ffn``, for stage-wise parity tests."""

    q: np.ndarray  # e4m3 [T, H]
    scales: np.ndarray  # f32 [T, H/128]
    gate_up: np.ndarray  # bf16 [R, 2I], indexed by pair p = t*K + rank
    act_q: np.ndarray  # e4m3 [R, I]
    act_scales: np.ndarray  # f32 [R, I/128]
    down: np.ndarray  # f32 [R, H]: unweighted FC2 output per pair
    out: np.ndarray  # bf16 [T, H]


def expert_fc1(q, scales, ids, weights_: ExpertWeights, experts=None):
    """FC1 gate|up per pair: ``gu[t*K+r] = bf16(sum_k W13[e]*S13 * q[t]*s[t])``.

    ``expert_up_kernel`` (``kernels.py:290-301``, bf16 output buffer ``:333``).
    Returns bf16 [R, 2I] indexed by pair.
    """
    tokens, top_k = ids.shape
    x_dq = dequantize_rows(q, scales)
    out = np.zeros((tokens * top_k, weights_.w13.shape[1]), dtype=np.uint16)
    flat = ids.reshape(-1)
    for e in np.unique(flat) if experts is None else experts:
        pairs = np.flatnonzero(flat == e)
        if pairs.size == 0:
            continue
        w = dequantize_weight(weights_.w13[e], weights_.s13[e])
        out[pairs] = f32_to_bf16(expert_matmul(x_dq[pairs // top_k], w))
    return out


def expert_fc2(act_q, act_scales, ids, weights_: ExpertWeights):
    """FC2 per pair, fp32, unweighted: ``y[p] = sum_k W2[e]*S2 * a[p]*as[p]``.

    ``expert_down_kernel`` (``kernels.py:304-322``) keeps this in fp32 before
    the routing-weighted sum.
    """
    flat = ids.reshape(-1)
    a_dq = dequantize_rows(act_q, act_scales)
    out = np.zeros((flat.size, weights_.w2.shape[1]), dtype=np.float32)
    for e in np.unique(flat):
        pairs = np.flatnonzero(flat == e)
        w = dequantize_weight(weights_.w2[e], weights_.s2[e])
        out[pairs] = expert_matmul(a_dq[pairs], w)
    return out


def weighted_combine(down: np.ndarray, topk_weights_f32: np.ndarray) -> np.ndarray:
    """``out[t] = bf16(sum_r w[t,r] * y[t*K+r])`` (``kernels.py:319-322``,
    ``:779``), evaluated in float64 then rounded once to bf16."""
    tokens, top_k = topk_weights_f32.shape
    y = down.reshape(tokens, top_k, -1).astype(np.float64)
    total = (y * topk_weights_f32.astype(np.float64)[:, :, None]).sum(axis=1)
    return f32_to_bf16(total.astype(np.float32))


def expert_ffn(x_bf16, ids, topk_weights_bf16, weights_: ExpertWeights, trace: bool = False,
               silu_bf16: bool = False):
    """Routed expert FFN of ``small_batch_moe`` / ``native_moe``.

    ``kernels.py:325-357`` and ``:702-779``: quantise x per 128 group, FC1
    (fp32 accumulate, bf16 out), SwiGLU + FP8 requant, FC2 (fp32), routing
    weighted sum over the K ranks in fp32, bf16 out.  ``silu_bf16``: see
    ``swiglu_f32``.
    """
    x = bf16_to_f32(x_bf16)
    q, scales = quantize_rows(x)
    gate_up = expert_fc1(q, scales, ids, weights_)
    act_q, act_scales = silu_mul_quant(gate_up, silu_bf16=silu_bf16)
    down = expert_fc2(act_q, act_scales, ids, weights_)
    out = weighted_combine(down, bf16_to_f32(topk_weights_bf16))
    if trace:
        return ExpertTrace(q, scales, gate_up, act_q, act_scales, down, out)
    return out


def dense_ffn(x_bf16, w13, s13, w2, s2):
    """Dense FP8 SwiGLU expert applied to every row (config-4 shared expert):
    the same quantisation boundaries as one routed expert with weight 1.
    Returns the fp32 FC2 output [T, H]."""
    x = bf16_to_f32(x_bf16)
    q, scales = quantize_rows(x)
    gate_up = f32_to_bf16(expert_matmul(dequantize_rows(q, scales), dequantize_weight(w13, s13)))
    act_q, act_scales = silu_mul_quant(gate_up)
    return expert_matmul(dequantize_rows(act_q, act_scales), dequantize_weight(w2, s2))


def add_shared(routed_bf16: np.ndarray, shared_f32: np.ndarray) -> np.ndarray:
    """Config-4 combine: ``bf16(routed + bf16(shared))`` -- the reference's
    ``combine_experts`` (``kernels.py:433-439``) with the gate fixed at 1."""
    routed = bf16_to_f32(routed_bf16)
    shared = round_bf16(shared_f32.astype(np.float32))
    return f32_to_bf16((routed + shared).astype(np.float32))


# ---------------------------------------------------------------------------
# A12 combine with the (gated) shared expert
# ---------------------------------------------------------------------------
def sigmoid_bf16(gate_f32: np.ndarray) -> np.ndarray:
    """``bf16(sigmoid(fp32 gate))`` as f32 (``kernels.py:434-438``)."""
    g = np.asarray(gate_f32, dtype=np.float64)
    return round_bf16((1.0 / (1.0 + np.exp(-g))).astype(np.float32))


def combine_experts(routed_bf16, shared_bf16, gate_bf16):
    """``combine_experts`` (``kernels.py:427-445``):
    ``out = fma_bf16(shared, bf16(sigmoid(gate)), routed)``, one rounding.

    The kernel source reads ``routed + bf16(shared * gate)``, but the
    reference states that its compiled form contracts the multiply-add into
    one single-rounding bf16 FMA and keeps that result in the fused residual
    variant (``kernels.py:465-474``), so the single rounding is the contract.
    gate: bf16 [T] (one gate column per row)."""
    routed = bf16_to_f32(routed_bf16).astype(np.float64)
    shared = bf16_to_f32(shared_bf16).astype(np.float64)
    gate = sigmoid_bf16(bf16_to_f32(gate_bf16)).astype(np.float64)[:, None]
    return f64_to_bf16(shared * gate + routed)


def _rms_norm(value: np.ndarray, weight_bf16, eps: float) -> np.ndarray:
    width = value.shape[-1]
    v = value.astype(np.float64)
    inv = 1.0 / np.sqrt((v * v).sum(axis=-1, keepdims=True) / width + eps)
    w = bf16_to_f32(weight_bf16).astype(np.float64)
    return f32_to_bf16((v * inv * (1.0 + w)).astype(np.float32))


def combine_experts_add_norm(routed_bf16, shared_bf16, gate_bf16, residual_bf16, weight_bf16, eps,
                             inverse=None):
    """``combine_experts_add_norm(_inverse)`` (``kernels.py:448-556``).

    combined = single-rounding bf16 FMA ``shared * bf16(sigmoid(gate)) + routed``
    (the ``fma.rn.bf16`` of ``kernels.py:467-474``); residual <- bf16(combined +
    residual); out = bf16(residual * rsqrt(mean(residual^2) + eps) * (1 + w)).
    With ``inverse``, row r reads MoE row ``inverse[r]`` (``kernels.py:512-518``).
    Returns (out bf16 [N, W], new residual bf16 [N, W]).
    """
    rows = np.arange(len(residual_bf16)) if inverse is None else np.asarray(inverse)
    routed = bf16_to_f32(routed_bf16[rows]).astype(np.float64)
    shared = bf16_to_f32(shared_bf16[rows]).astype(np.float64)
    gate = sigmoid_bf16(bf16_to_f32(gate_bf16[rows])).astype(np.float64)[:, None]
    combined = bf16_to_f32(f64_to_bf16(shared * gate + routed))
    value = round_bf16((combined + bf16_to_f32(residual_bf16)).astype(np.float32))
    return _rms_norm(value, weight_bf16, eps), f32_to_bf16(value)


def add_norm(x_bf16, residual_bf16, weight_bf16, eps):
    """``add_norm`` (``kernels.py:405-415``): residual <- bf16(x + residual),
    out = bf16(rmsnorm(residual) * (1 + w))."""
    value = round_bf16((bf16_to_f32(x_bf16) + bf16_to_f32(residual_bf16)).astype(np.float32))
    return _rms_norm(value, weight_bf16, eps), f32_to_bf16(value)


# ---------------------------------------------------------------------------
# A13 ragged packing
# ---------------------------------------------------------------------------
def row_metadata(boundaries, sequence_slots, capacity, frames=None, eos=0, codes=11):
    """``row_metadata`` of ``packed_prefill.py:51-78``.

    seq(row) = #{i in 1..n-1 : row >= cu[i]}; pos = row - cu[seq];
    row_slot = slots[seq]; labels[row, c] = frames[row+1, c] if row+1 < cu[seq+1]
    else (eos if c == 0 else 0).
    """
    cu = np.asarray(boundaries, dtype=np.int64)
    n = len(cu) - 1
    rows = np.arange(capacity, dtype=np.int64)
    seq = np.zeros(capacity, dtype=np.int64)
    for i in range(1, n):
        seq += rows >= cu[i]
    positions = rows - cu[seq]
    row_slots = np.asarray(sequence_slots, dtype=np.int64)[seq]
    labels = None
    if frames is not None:
        frames = np.asarray(frames, dtype=np.int64)
        labels = np.zeros((capacity, codes), dtype=np.int64)
        labels[:, 0] = eos
        nxt = rows + 1
        valid = nxt < cu[seq + 1]
        labels[valid] = frames[nxt[valid]]
    return positions, row_slots, labels


def mixed_rows(decode_slots, prompt_lengths):
    """Row order of a mixed step: decode rows first, then each prompt's rows
    contiguously (``mixed_model.py:1-7,174-181``; ``mixed_graph.py:139-179``).
    Returns (row_kind [N] 0=decode 1=prefill, row_owner [N] slot or prompt
    index, cu_seqlens of the prefill suffix)."""
    decode_slots = np.asarray(decode_slots, dtype=np.int64)
    lengths = np.asarray(prompt_lengths, dtype=np.int64)
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    kind = np.concatenate([np.zeros(decode_slots.size, np.int32), np.ones(int(cu[-1]), np.int32)])
    owner = np.concatenate([decode_slots, np.repeat(np.arange(lengths.size), lengths)])
    return kind, owner.astype(np.int64), cu


# ---------------------------------------------------------------------------
# A13 mixed decode + prefill rows and prefix row reuse
# ---------------------------------------------------------------------------
def prompt_row_owners(prompts, decode_rows, full_rows):
    """Owner row of every mixed row under prefix reuse (``row_reuse.py:74-92``).

    Rows are decode rows [0, decode_rows) then each prompt's rows in order.
    Prompt i's first ``longest`` rows alias the same positions of the earlier
    prompt j whose rows agree with prompt i's for the longest leading run
    (all columns compared; the first such j on ties); aliased rows take
    prompt j's owners, so owners are canonical (owner[owner[r]] == owner[r]).
    Every other row owns itself.
    """
    arrays = [np.asarray(p) for p in prompts]
    owners = np.arange(full_rows, dtype=np.int64)
    offsets = []
    offset = decode_rows
    for index, current in enumerate(arrays):
        longest, previous_owner = 0, None
        for previous, other in enumerate(arrays[:index]):
            limit = min(len(current), len(other))
            same = np.all(current[:limit] == other[:limit], axis=1)
            different = np.flatnonzero(~same)
            common = int(different[0]) if len(different) else limit
            if common > longest:
                longest, previous_owner = common, previous
        if longest:
            start = offsets[previous_owner]
            owners[offset:offset + longest] = owners[start:start + longest]
        offsets.append(offset)
        offset += len(current)
    return owners


def plan_row_reuse(prompts, decode_rows, prefill_capacity, compact_capacities):
    """``plan_row_reuse`` (``row_reuse.py:46-109``) without its argument
    checks: (compact_rows, unique_rows, packed int64 [compact + full]) or
    None when no compact capacity holds the unique rows rounded up to 64.
    packed = [kept rows ascending, zero padded to compact | for every row the
    kept-row index of its owner]."""
    full_rows = decode_rows + prefill_capacity
    capacities = sorted(set(compact_capacities))
    if not capacities:
        return None
    owners = prompt_row_owners(prompts, decode_rows, full_rows)
    keep = np.flatnonzero(owners == np.arange(full_rows))
    unique = len(keep)
    minimum = (unique + 63) // 64 * 64
    compact = next((k for k in capacities if k >= minimum), None)
    if compact is None:
        return None
    lookup = np.empty_like(owners)
    lookup[keep] = np.arange(unique, dtype=np.int64)
    packed = np.zeros(compact + full_rows, dtype=np.int64)
    packed[:unique] = keep
    packed[compact:] = lookup[owners]
    return compact, unique, packed


@dataclass
class MixedLayout:
    active: np.ndarray        # int32 [S]: occupied slots ascending, then -1
    count: int                # occupied slots
    decode_slots: np.ndarray  # int64 [decode_rows]
    keep: np.ndarray          # int32 [full]: MoE source rows, then 0
    keep_count: int
    inverse: np.ndarray       # int64 [full]: MoE row read back by every row


def mixed_layout(occupancy, decode_rows, padding_start, boundaries, prompts, capacity,
                 frames=None, codes=11):
    """The device contract of one mixed step's rows (``d3_mixed_rows``).

    Decode rows: the ascending occupied slots, then reserved padding slots
    ``padding_start + j`` for rows j >= count (``mixed_graph.py:147-152``).
    Prefill rows: the packed suffix of capacity rows whose first
    ``boundaries[prompts]`` rows are the prompts (``mixed_graph.py:161-179``:
    the remaining sequences are empty or padding).  Live rows are the
    occupied decode rows and the prompt rows; with ``frames`` (the suffix's
    int64 rows) prompt rows alias earlier prompts' rows by
    ``prompt_row_owners``.  The MoE runs on the live rows that own themselves
    (``keep`` ascending, ``keep_count`` of them, the reference's compact rows
    of ``mixed_model.py:193-198,239-242``); every live row reads back its
    owner's MoE row (``inverse``, the reference's lookup); rows that are not
    live (decode padding, prefill padding) read MoE row 0.
    """
    active, count = compact_slots(occupancy)
    slots_out = np.full(len(occupancy), -1, dtype=np.int32)
    slots_out[:count] = active
    used = min(count, decode_rows)
    decode_slots = padding_start + np.arange(decode_rows, dtype=np.int64)
    decode_slots[:used] = active[:used]
    full = decode_rows + capacity
    cu = np.asarray(boundaries, dtype=np.int64)
    lengths = [int(cu[i + 1] - cu[i]) for i in range(prompts)]
    live_prefill = int(cu[prompts])
    if frames is not None:
        rows = np.asarray(frames, dtype=np.int64).reshape(-1, codes)
        arrays = [rows[cu[i]:cu[i] + n] for i, n in enumerate(lengths)]
        owners = prompt_row_owners(arrays, decode_rows, full)
    else:
        owners = np.arange(full, dtype=np.int64)
    r = np.arange(full)
    live = np.where(r < decode_rows, r < used, (r - decode_rows) < live_prefill)
    kept = live & (owners == r)
    keep_rows = np.flatnonzero(kept)
    keep = np.zeros(full, dtype=np.int32)
    keep[:len(keep_rows)] = keep_rows
    rank = np.zeros(full, dtype=np.int64)
    rank[keep_rows] = np.arange(len(keep_rows))
    inverse = np.where(live, rank[owners], 0).astype(np.int64)
    return MixedLayout(slots_out, count, decode_slots, keep, len(keep_rows), inverse)
