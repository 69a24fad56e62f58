"""Stage-wise parity of the HIP kernels against the CPU oracle, called
through the C ABI (ctypes).  Integer / byte outputs are compared bit for
bit; floating-point outputs within the tolerances stated in helpers.py."""

import numpy as np
import pytest
import torch

from helpers import CONTRACTION, EXACT, assert_bf16_close, np_bf16, np_f32, np_u8, oracle_weights
from oracle import moe as om
from oracle.numerics import bf16_to_f32, f32_to_bf16

pytestmark = pytest.mark.gpu


def bf16_tensor(rng, shape, device, scale=1.0):
    bits = f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))
    return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).to(device)


# --------------------------------------------------------------------------- A1
@pytest.mark.parametrize("slots,p", [(64, 0.75), (64, 0.0), (64, 1.0), (4096, 0.3), (1, 1.0)])
def test_compact_slots(device, slots, p):
    from drama3_amd.pipeline import compact_slots

    rng = np.random.default_rng(slots)
    occ = (rng.uniform(size=slots) < p).astype(np.uint8)
    occ_t = torch.from_numpy(occ).to(device)
    active = torch.full((slots,), 123, dtype=torch.int32, device=device)
    count = torch.empty(1, dtype=torch.int32, device=device)
    compact_slots(occ_t, active, count)
    expected, n = om.compact_slots(occ)
    assert int(count.item()) == n
    got = active.cpu().numpy()
    assert np.array_equal(got[:n], expected)
    assert np.all(got[n:] == -1)


# --------------------------------------------------------------------------- A3
@pytest.mark.parametrize("rows,experts,dtype", [(4, 16, torch.bfloat16), (64, 128, torch.bfloat16),
                                                (300, 256, torch.bfloat16), (33, 128, torch.float32),
                                                (7, 512, torch.bfloat16)])
def test_route(device, rows, experts, dtype):
    from drama3_amd.kernels import route

    rng = np.random.default_rng(rows + experts)
    logits = bf16_tensor(rng, (rows, experts), device)
    if dtype == torch.float32:
        logits = (logits.float() + torch.from_numpy(rng.standard_normal((rows, experts)) * 1e-3)
                  .float().to(device))
    weights, ids = route(logits)
    ow, oids = om.route(np_f32(logits), out_dtype="bf16" if dtype == torch.bfloat16 else "f32")
    assert ids.dtype == torch.int64 and weights.dtype == dtype
    assert np.array_equal(ids.cpu().numpy(), oids)
    got = np_f32(weights)
    want = bf16_to_f32(ow) if dtype == torch.bfloat16 else ow
    assert np.all(np.abs(got - want) <= np.abs(want) * 2.0**-8 + 1e-7)


def test_route_ties_and_strided_rows(device):
    from drama3_amd.kernels import route

    base = torch.full((3, 32), -1.0)
    base[0] = 0.0  # all equal -> ids 0..7
    base[1, [3, 9, 12]] = 2.0
    base[1, [1, 4, 5, 10, 14, 15]] = 1.0
    base[2, 2] = -0.0
    base[2, 7] = 0.0
    storage = torch.zeros((3, 48), dtype=torch.bfloat16)
    storage[:, :32] = base.to(torch.bfloat16)
    logits = storage.to(device)[:, :32]  # row stride 48
    _, ids = route(logits)
    _, oids = om.route(base.numpy())
    assert np.array_equal(ids.cpu().numpy(), oids)
    assert ids[0].tolist() == list(range(8))
    assert ids[1].tolist() == [3, 9, 12, 1, 4, 5, 10, 14]
    assert ids[2, :2].tolist() == [7, 2]


# --------------------------------------------------------------------------- A4
@pytest.mark.parametrize("magnitude", [0.0, 1e-12, 1.0, 1000.0])
@pytest.mark.parametrize("strided", [False, True])
def test_prepare_moe_input_bytes(device, magnitude, strided):
    """validate_moe_input.py:27-61 cases: byte-exact q, scales and logits."""
    from drama3_amd.moe_input import prepare_moe_input, quantize_groups

    rng = np.random.default_rng(int(magnitude * 7) + strided)
    rows = 48
    storage = bf16_tensor(rng, (rows, 4096 if strided else 2048), device, magnitude)
    x = storage[:, :2048]
    router = bf16_tensor(rng, (rows, 1408 if strided else 256), device)[:, :256]
    q, scales, logits = prepare_moe_input(x, router)
    oq, os_, ol = om.prepare_moe_input(np_bf16(x), np_f32(router))
    assert np.array_equal(np_u8(q), oq)
    assert np.array_equal(np_f32(scales), os_)
    assert np.array_equal(np_f32(logits), ol)
    q2, s2 = quantize_groups(x)
    assert np.array_equal(np_u8(q2), oq) and np.array_equal(np_f32(s2), os_.T)


def test_prepare_moe_input_padding_router(device):
    from drama3_amd.moe_input import prepare_moe_input

    rng = np.random.default_rng(3)
    x = bf16_tensor(rng, (6, 256), device)
    router = bf16_tensor(rng, (6, 16), device)
    slots = torch.tensor([3, 40, 1, 33, 32, 0], device=device)
    q, scales, logits = prepare_moe_input(x, router, row_slots=slots, padding_start=32)
    oq, os_, ol = om.prepare_moe_input(np_bf16(x), np_f32(router), slots.cpu().numpy(), 32)
    assert np.array_equal(np_u8(q), oq) and np.array_equal(np_f32(logits), ol)


def test_prepare_moe_input_contract_errors(device):
    from drama3_amd.moe_input import prepare_moe_input

    x = torch.zeros((4, 256), dtype=torch.bfloat16, device=device)
    router = torch.zeros((4, 16), dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError):
        prepare_moe_input(x, router, row_slots=torch.zeros(4, dtype=torch.int64, device=device))
    with pytest.raises(ValueError):
        prepare_moe_input(x[:, :200], router)
    with pytest.raises(ValueError):
        prepare_moe_input(x, router.t())


# --------------------------------------------------------------------------- A5-A7
@pytest.mark.parametrize("tokens,experts,tile,dtype", [(4, 16, 16, torch.int64),
                                                       (48, 128, 16, torch.int32),
                                                       (64, 16, 64, torch.int64),
                                                       (4160, 128, 16, torch.int32),
                                                       (560, 16, 16, torch.int64),
                                                       (1, 256, 128, torch.int64)])
def test_sort_routes(device, tokens, experts, tile, dtype):
    from drama3_amd.kernels import sort_routes

    rng = np.random.default_rng(tokens * 3 + experts)
    ids = np.stack([rng.permutation(experts)[:8] for _ in range(tokens)])
    counts, starts, total, sorted_ids, expert_ids, inverse = sort_routes(
        torch.from_numpy(ids).to(dtype).to(device), experts, tile)
    o = om.sort_routes(ids, experts, tile)
    assert np.array_equal(counts.cpu().numpy(), o.counts)
    assert np.array_equal(starts.cpu().numpy(), o.starts)
    assert int(total.item()) == o.total
    got_sorted = sorted_ids.cpu().numpy()
    assert np.array_equal(got_sorted[:o.total], o.sorted_ids)
    assert np.all(got_sorted[o.total:] == ids.size)
    got_experts = expert_ids.cpu().numpy()
    assert np.array_equal(got_experts[:o.total // tile], o.expert_ids)
    assert np.all(got_experts[o.total // tile:] == -1)
    assert np.array_equal(inverse.cpu().numpy(), o.inverse)


@pytest.mark.parametrize("tokens,experts,where", [(300, 16, "last"), (40, 8, "every"),
                                                  (1000, 64, "first")])
def test_sort_routes_repeated_expert_in_a_row(device, tokens, experts, where):
    """Ids that repeat an expert inside a row (not router output, but the
    operator accepts them): the row-mask sort must hand over to the ballot
    sort and the result is still the oracle's stable sort."""
    from drama3_amd.kernels import sort_routes

    rng = np.random.default_rng(tokens + experts)
    ids = np.stack([rng.permutation(experts)[:8] for _ in range(tokens)])
    if where == "every":
        ids = rng.integers(0, experts, ids.shape)
    else:
        row = tokens - 1 if where == "last" else 0
        ids[row, 5] = ids[row, 2]
    counts, starts, total, sorted_ids, expert_ids, inverse = sort_routes(
        torch.from_numpy(ids).to(torch.int32).to(device), experts, 16)
    o = om.sort_routes(ids, experts, 16)
    assert np.array_equal(counts.cpu().numpy(), o.counts)
    assert int(total.item()) == o.total
    assert np.array_equal(sorted_ids.cpu().numpy()[:o.total], o.sorted_ids)
    assert np.array_equal(inverse.cpu().numpy(), o.inverse)


def test_sort_routes_skewed_single_expert(device):
    from drama3_amd.kernels import sort_routes

    ids = np.zeros((100, 1), np.int64)
    ids[::3] = 5
    out = sort_routes(torch.from_numpy(ids).to(device), 8, 16)
    o = om.sort_routes(ids, 8, 16)
    assert np.array_equal(out[3].cpu().numpy()[:o.total], o.sorted_ids)


# --------------------------------------------------------------------------- A8-A11
EXACT_ALWAYS = 1 << 30
FP8_ALWAYS = -1


def _stage_setup(device, tokens=40, experts=16, hidden=1024, inter=256, seed=0,
                 exact_routes=EXACT_ALWAYS):
    from drama3_amd.pipeline import MoEWorkspace, Shape
    from drama3_amd.workloads import make_experts

    gen = torch.Generator("cpu").manual_seed(seed)
    ex = make_experts(gen, experts, hidden, inter)
    x = torch.randn((tokens, hidden), generator=gen).to(torch.bfloat16)
    logits = torch.randn((tokens, experts), generator=gen).to(torch.bfloat16)
    dev_ex = ex.to(device)
    ws = MoEWorkspace(Shape(tokens, experts, hidden, inter), device, exact_routes=exact_routes)
    ws.route(logits.to(device))
    ws.quantize(x.to(device))
    ws.sort()
    return ws, dev_ex, oracle_weights(ex), np_bf16(x), np_f32(logits)


@pytest.mark.parametrize("path", ["exact", "fp8"])
@pytest.mark.parametrize("hidden,inter,experts,tokens", [(1024, 256, 16, 4), (1024, 256, 16, 64),
                                                         (2048, 768, 128, 48), (512, 512, 8, 200)])
def test_fc1_stage(device, hidden, inter, experts, tokens, path):
    ws, dev_ex, wt, x, logits = _stage_setup(
        device, tokens, experts, hidden, inter, seed=tokens,
        exact_routes=EXACT_ALWAYS if path == "exact" else FP8_ALWAYS)
    ws.fc1(dev_ex)
    torch.cuda.synchronize()
    _, ids = om.route(logits)
    assert np.array_equal(ws.ids.cpu().numpy(), ids)
    q, xs = om.quantize_rows(bf16_to_f32(x))
    assert np.array_equal(np_u8(ws.q), q)
    expected = om.expert_fc1(q, xs, ids, wt)  # [pairs, 2I] by pair
    total = int(ws.total.item())
    sorted_ids = ws.sorted_ids.cpu().numpy()[:total]
    valid = sorted_ids < ids.size
    got = np_bf16(ws.gate_up)[:total][valid]
    if path == "exact":  # fp32-accurate sums: at most one bf16 rounding apart
        stats = assert_bf16_close(got, expected[sorted_ids[valid]], ulps=1, row_floor=2.0**-14,
                                  outlier_fraction=0.0)
        assert stats["exact_fraction"] > 0.99
    else:
        stats = assert_bf16_close(got, expected[sorted_ids[valid]], ulps=2, row_floor=2.0**-8,
                                  rrms_max=4e-3, outlier_fraction=0.0)
    print(path, stats)


def test_fp8_mfma_exact_for_narrow_exponent_range(device):
    """FP8 MFMA rounding only appears when products span a wide exponent
    range: with weight codes in [1, 2) and unit scales both paths are exact."""
    from drama3_amd.pipeline import MoEWorkspace, Shape
    from drama3_amd.workloads import Experts

    gen = torch.Generator("cpu").manual_seed(1)
    e, h, i, t = 8, 1024, 256, 32
    codes = (torch.randint(0, 8, (e, 2 * i, h), generator=gen) + 0x38)
    codes |= torch.randint(0, 2, codes.shape, generator=gen) * 0x80
    w13 = codes.to(torch.uint8).view(torch.float8_e4m3fn)
    w2 = torch.zeros((e, h, i), dtype=torch.uint8).view(torch.float8_e4m3fn)
    ex = Experts(w13, torch.ones((e, 2 * i // 128, h // 128)), w2, torch.ones((e, h // 128, i // 128)))
    # activations 256 * (1 + k/8) <= 448, each 128-group holding 448: scale
    # 1, q = x exactly, and every product lies in [2^8, 2^10)
    x = (256.0 * (1.0 + torch.randint(0, 7, (t, h), generator=gen) / 8.0)).to(torch.bfloat16)
    x[:, ::128] = 448.0
    logits = torch.randn((t, e), generator=gen).to(torch.bfloat16)
    outs = {}
    for name, exact_routes in (("exact", EXACT_ALWAYS), ("fp8", FP8_ALWAYS)):
        ws = MoEWorkspace(Shape(t, e, h, i), device, exact_routes=exact_routes)
        ws.route(logits.to(device))
        ws.quantize(x.to(device))
        ws.sort()
        ws.fc1(ex.to(device))
        torch.cuda.synchronize()
        total = int(ws.total.item())
        outs[name] = np_bf16(ws.gate_up)[:total]
    sorted_ids = ws.sorted_ids.cpu().numpy()[:total]
    valid = sorted_ids < t * 8
    assert np.array_equal(outs["exact"][valid], outs["fp8"][valid])


@pytest.mark.parametrize("path", ["exact", "fp8"])
def test_activation_and_fc2_stages(device, path):
    """Feed each stage the device result of the previous one, so the check
    isolates the stage: SwiGLU requant bytes and FC2 fp32 outputs."""
    ws, dev_ex, wt, x, logits = _stage_setup(
        device, 48, 128, 2048, 768, seed=5,
        exact_routes=EXACT_ALWAYS if path == "exact" else FP8_ALWAYS)
    ws.fc1(dev_ex)
    ws.activation()
    ws.fc2(dev_ex)
    torch.cuda.synchronize()
    total = int(ws.total.item())
    pairs = ws.shape.pairs
    sorted_ids = ws.sorted_ids.cpu().numpy()[:total]
    valid = sorted_ids < pairs
    gu = np_bf16(ws.gate_up)[:total][valid]
    aq, as_ = om.silu_mul_quant(gu)
    got_q = np_u8(ws.act)[:total][valid]
    got_s = np_f32(ws.act_scales)[:total][valid]
    # exp() may differ by an ulp between libm and the device: allow rare
    # one-code flips and last-bit scale differences, nothing more.
    mismatch = got_q != aq
    assert mismatch.mean() < 1e-3
    assert np.all(np.abs(got_q[mismatch].astype(int) - aq[mismatch].astype(int)) <= 1)
    assert np.all(np.abs(got_s - as_) <= np.abs(as_) * 2.0**-20)
    # FC2 on the device activation, by pair
    flat_ids = ws.ids.cpu().numpy().reshape(-1)
    order = sorted_ids[valid]
    a_dq = om.dequantize_rows(got_q, got_s)
    expected = np.zeros((pairs, 2048), np.float32)
    for e in np.unique(flat_ids):
        rows = np.flatnonzero(flat_ids[order] == e)
        w = om.dequantize_weight(wt.w2[e], wt.s2[e])
        expected[order[rows]] = om.expert_matmul(a_dq[rows], w)
    got = np_f32(ws.down)
    scale = np.sqrt(np.mean(expected ** 2, axis=-1, keepdims=True))
    # exact path: fp32 summation-order noise; fp8 path: ~1e-4 of sum|products|
    # per MFMA, i.e. a few 1e-4 of the row RMS for I = 768
    rel = 1e-5 if path == "exact" else 3e-3
    assert np.all(np.abs(got - expected) <= rel * scale + 1e-6 * np.abs(expected))


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("path", ["exact", "fp8"])
@pytest.mark.parametrize("hidden,inter,experts,tokens", [(1024, 256, 16, 4), (2048, 768, 128, 52),
                                                         (512, 512, 8, 200), (1024, 1024, 16, 24)])
def test_fc2_swiglu_prologue_matches_separate_stages(device, hidden, inter, experts, tokens, path,
                                                     packed):
    """d3_expert_fc2_swiglu (SwiGLU requant inside FC2) gives the bytes of
    silu_mul_quant followed by FC2, for single- and multi-tile items (200
    tokens over 8 experts: items of 128 routes, eight route tiles)."""
    from drama3_amd.expert_weights import prepare_experts

    ws, dev_ex, _, _, _ = _stage_setup(
        device, tokens, experts, hidden, inter, seed=tokens + inter,
        exact_routes=EXACT_ALWAYS if path == "exact" else FP8_ALWAYS)
    if packed:
        prepare_experts(dev_ex)
    ws.fc1(dev_ex)
    ws.activation()
    ws.down.fill_(float("nan"))
    ws.fc2(dev_ex)
    separate = ws.down.clone()
    ws.down.fill_(float("nan"))
    ws.fc2_swiglu(dev_ex)
    torch.cuda.synchronize()
    assert torch.equal(ws.down.view(torch.int32), separate.view(torch.int32))


# --------------------------------------------------------------------------- A11 + A12
@pytest.mark.parametrize("top_k,wdtype,with_inverse", [(8, torch.bfloat16, True),
                                                       (8, torch.float32, False),
                                                       (6, torch.bfloat16, True),
                                                       (1, torch.float32, True)])
def test_combine_routes_add_norm_equals_two_launches(device, top_k, wdtype, with_inverse):
    """d3_combine_routes_add_norm = d3_weighted_combine followed by
    d3_combine_experts_add_norm, byte for byte (routed, residual and out);
    without a residual, d3_weighted_combine followed by d3_combine_experts."""
    from drama3_amd import _lib
    from drama3_amd._lib import call, ptr

    rng = np.random.default_rng(top_k + (7 if with_inverse else 0))
    moe_rows, rows, width = 37, 50, 1024
    down = torch.from_numpy(rng.standard_normal((moe_rows * top_k, width)).astype(np.float32)).to(device)
    w = torch.from_numpy(rng.random((moe_rows, top_k)).astype(np.float32)).to(wdtype).to(device)
    shared = bf16_tensor(rng, (moe_rows, width), device)
    gate = bf16_tensor(rng, (moe_rows,), device)
    norm = bf16_tensor(rng, (width,), device, 0.1)
    res0 = bf16_tensor(rng, (rows if with_inverse else moe_rows, width), device)
    inverse = (torch.from_numpy(rng.integers(0, moe_rows, rows)).to(device) if with_inverse
               else None)
    n = len(res0)
    wcode = 1 if wdtype == torch.float32 else 0
    stream = _lib.stream(device)
    routed = torch.empty((moe_rows, width), dtype=torch.bfloat16, device=device)
    call("d3_weighted_combine", ptr(down), ptr(w), wcode, moe_rows, top_k, width, None, None,
         ptr(routed), stream)
    res_a, out_a = res0.clone(), torch.empty_like(res0)
    call("d3_combine_experts_add_norm", ptr(routed), ptr(shared), ptr(gate), 1, ptr(inverse),
         ptr(res_a), ptr(norm), 1e-6, n, width, ptr(out_a), stream)
    res_b, out_b = res0.clone(), torch.empty_like(res0)
    call("d3_combine_routes_add_norm", ptr(down), ptr(w), wcode, top_k, ptr(shared), ptr(gate), 1,
         ptr(inverse), ptr(res_b), ptr(norm), 1e-6, n, width, ptr(out_b), stream)
    # residual == NULL: the combined row only, the bytes of d3_weighted_combine
    # followed by d3_combine_experts (gathered through inverse)
    combined = torch.empty((moe_rows, width), dtype=torch.bfloat16, device=device)
    call("d3_combine_experts", ptr(routed), ptr(shared), ptr(gate), 1, moe_rows, width,
         ptr(combined), stream)
    out_c = torch.full_like(res0, 5.0)
    call("d3_combine_routes_add_norm", ptr(down), ptr(w), wcode, top_k, ptr(shared), ptr(gate), 1,
         ptr(inverse), None, None, 0.0, n, width, ptr(out_c), stream)
    torch.cuda.synchronize()
    assert torch.equal(res_a.view(torch.int16), res_b.view(torch.int16))
    assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16))
    want_c = combined[inverse] if inverse is not None else combined
    assert torch.equal(out_c.view(torch.int16), want_c.view(torch.int16))


# --------------------------------------------------------------------------- A12
def test_combine_then_add_norm_equals_combine_add_norm(device):
    """d3_combine_experts followed by d3_add_norm gives the bytes of
    d3_combine_experts_add_norm (both combine with one bf16 FMA)."""
    from drama3_amd.kernels import add_norm, combine_experts, combine_experts_add_norm

    rng = np.random.default_rng(12)
    rows, width = 16, 2048
    routed, shared = bf16_tensor(rng, (rows, width), device), bf16_tensor(rng, (rows, width), device)
    gate = bf16_tensor(rng, (rows, 1), device)
    weight = bf16_tensor(rng, (width,), device, 0.1)
    res_a = bf16_tensor(rng, (rows, width), device)
    res_b = res_a.clone()
    out_a = add_norm(combine_experts(routed, shared, gate), res_a, weight, 1e-6)
    out_b = combine_experts_add_norm(routed, shared, gate, res_b, weight, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(res_a.view(torch.int16), res_b.view(torch.int16))
    assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16))


def test_combine_kernels(device):
    from drama3_amd.kernels import (add_norm, combine_experts, combine_experts_add_norm,
                                    combine_experts_add_norm_inverse, silu_mul)

    rng = np.random.default_rng(11)
    rows, width = 12, 2048
    routed, shared = bf16_tensor(rng, (rows, width), device), bf16_tensor(rng, (rows, width), device)
    gate_storage = bf16_tensor(rng, (rows, 3), device)
    gate = gate_storage[:, 1:2]
    out = combine_experts(routed, shared, gate)
    want = om.combine_experts(np_bf16(routed), np_bf16(shared), np_bf16(gate)[:, 0])
    assert np.array_equal(np_bf16(out), want)  # one bf16 FMA, single rounding

    residual = bf16_tensor(rng, (rows, width), device)
    weight = bf16_tensor(rng, (width,), device, 0.1)
    res0 = np_bf16(residual)
    out = combine_experts_add_norm(routed, shared, gate, residual, weight, 1e-6)
    want_out, want_res = om.combine_experts_add_norm(np_bf16(routed), np_bf16(shared),
                                                     np_bf16(gate)[:, 0], res0, np_bf16(weight), 1e-6)
    assert_bf16_close(np_bf16(residual), want_res, ulps=1, row_floor=0.0)
    assert_bf16_close(np_bf16(out), want_out, ulps=1, row_floor=0.0)

    big_res = bf16_tensor(rng, (20, width), device)
    inverse = torch.from_numpy(rng.integers(0, rows, 20)).to(device)
    r0 = np_bf16(big_res)
    out = combine_experts_add_norm_inverse(routed, shared, gate, inverse, big_res, weight, 1e-6)
    want_out, want_res = om.combine_experts_add_norm(np_bf16(routed), np_bf16(shared),
                                                     np_bf16(gate)[:, 0], r0, np_bf16(weight), 1e-6,
                                                     inverse.cpu().numpy())
    assert_bf16_close(np_bf16(big_res), want_res, ulps=1, row_floor=0.0)
    assert_bf16_close(np_bf16(out), want_out, ulps=1, row_floor=0.0)

    x = bf16_tensor(rng, (rows, width), device)
    res = bf16_tensor(rng, (rows, width), device)
    r0 = np_bf16(res)
    out = add_norm(x, res, weight, 1e-6)
    want_out, want_res = om.add_norm(np_bf16(x), r0, np_bf16(weight), 1e-6)
    assert np.array_equal(np_bf16(res), want_res)
    assert_bf16_close(np_bf16(out), want_out, ulps=1, row_floor=0.0)

    projected = bf16_tensor(rng, (rows, 1024), device, 3.0)
    out = silu_mul(projected)
    assert_bf16_close(np_bf16(out), om.silu_mul(np_bf16(projected)), ulps=1, row_floor=0.0)


# --------------------------------------------------------------------------- A13 / A1 state
def test_row_metadata(device):
    from drama3_amd.packed_prefill import row_metadata

    lengths = [5, 3, 7, 0, 9]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int32, device=device)
    slots = torch.tensor([9, 4, 30, 61, 62], dtype=torch.int64, device=device)
    capacity = 30
    frames = torch.arange(capacity * 11, dtype=torch.int64, device=device).view(capacity, 11) + 1000
    pos = torch.empty(capacity, dtype=torch.int64, device=device)
    row_slots = torch.empty_like(pos)
    labels = torch.empty((capacity, 11), dtype=torch.int64, device=device)
    row_metadata[(1,)](cu, slots, pos, row_slots, labels, frames, 7, len(lengths), capacity, 128)
    opos, oslots, olabels = om.row_metadata(cu.cpu().numpy(), slots.cpu().numpy(), capacity,
                                            frames.cpu().numpy(), eos=7)
    assert np.array_equal(pos.cpu().numpy(), opos)
    assert np.array_equal(row_slots.cpu().numpy(), oslots)
    assert np.array_equal(labels.cpu().numpy(), olabels)


def test_device_requests_known_answer(device):
    """scripts/validate_runtime_state.py:10-47 on the device kernels."""
    from drama3_amd.runtime_state import DeviceRequests

    state = DeviceRequests(8, eos=999, max_length=512, max_frames=8, device=device)
    slots = torch.tensor([5, 1, 3], device=device, dtype=torch.int64)
    histories = torch.arange(48, device=device).view(3, 16)
    for row, slot in enumerate(slots.tolist()):
        state.initialize(slot, torch.arange(11, device=device), histories[row], 30 + row, row + 2)
    expected = [[], [], []]
    last = torch.empty(3, 11, device=device, dtype=torch.int64)
    history = torch.empty(3, 16, device=device, dtype=torch.int64)
    positions = torch.empty(3, device=device, dtype=torch.int64)
    for step in range(6):
        output = torch.arange(33, device=device).view(3, 11) + 100 * (step + 1)
        output[1, 0] = 999 if step >= 1 else 123
        state.save(slots, output)
        for row in range(3):
            if len(expected[row]) < row + 2 and not (row == 1 and step >= 1):
                expected[row].append(output[row].clone())
        state.load(slots, last, history, positions)
        for row, values in enumerate(expected):
            assert torch.equal(last[row], values[-1])
            assert positions[row] == 30 + row + len(values)
            target = torch.cat((histories[row], torch.stack(values)[:, 0]))[-16:]
            assert torch.equal(history[row], target)
    state.initialize(5, last[0], histories[0], 50, 1)
    fresh = torch.arange(11, device=device)[None] + 500
    state.save(slots[:1], fresh)
    assert torch.equal(state.codes[5, 0], fresh[0, 1:])
    assert state.metadata[5].tolist() == [51, 1, 1, 1]


# --------------------------------------------------------------------------- empty batches
def test_empty_batches_launch_nothing_and_return_empty(device):
    """Zero rows through every reference-named operator and the layer's
    GEMM: empty outputs, no error (the reference's operators accept T = 0)."""
    from drama3_amd import workloads
    from drama3_amd.kernels import (add_norm, combine_experts, combine_experts_add_norm,
                                    native_moe, route, routed_moe, small_batch_moe)
    from drama3_amd.moe_layer import dense_bf16

    experts = workloads.config1().experts.to(device)
    x = torch.empty((0, 1024), dtype=torch.bfloat16, device=device)
    logits = torch.empty((0, 16), dtype=torch.bfloat16, device=device)
    weights, ids = route(logits)
    assert weights.shape == (0, 8) and ids.shape == (0, 8)
    for out in (routed_moe(x, logits, experts), small_batch_moe(x, ids, weights, experts),
                native_moe(x, ids, weights, experts)):
        assert out.shape == (0, 1024) and out.dtype == torch.bfloat16
    gate = torch.empty((0,), dtype=torch.bfloat16, device=device)
    norm = torch.zeros(1024, dtype=torch.bfloat16, device=device)
    assert combine_experts(x, x, gate).shape == (0, 1024)
    assert combine_experts_add_norm(x, x, gate, x.clone(), norm, 1e-6).shape == (0, 1024)
    assert add_norm(x, x.clone(), norm, 1e-6).shape == (0, 1024)
    w = torch.zeros((256, 1024), dtype=torch.bfloat16, device=device)
    assert dense_bf16(x, w, torch.empty((0, 256), dtype=torch.bfloat16, device=device)).shape == (0, 256)
    torch.cuda.synchronize()


def test_swiglu_sigmoid_tail(device):
    """Gates from -104 to -80 (the true sigmoid below 2^-126 from -87.3
    down, where the fp32 sigmoid returns 0 or a subnormal below 2^-125).
    The FP8 requantisation gives the float64 oracle's codes and scales byte
    for byte there: zeros of the right sign, next to groups whose other
    gates (20 to 30: sigmoid exactly 1) set normal scales.  The bf16
    silu_mul equals the oracle's bytes outside the tail and stays below
    2^-118 |u| inside it (where the oracle's value is a subnormal or a
    tiny normal)."""
    from drama3_amd import _lib
    from drama3_amd._lib import call, ptr
    from drama3_amd.kernels import silu_mul

    rng = np.random.default_rng(17)
    rows, width = 64, 256
    gate = np.linspace(-104.0, -80.0, rows * width).astype(np.float32).reshape(rows, width)
    up = (rng.standard_normal((rows, width)) * np.exp(rng.uniform(-4, 4, (rows, width)))).astype(np.float32)
    gate[::2, ::3] = rng.uniform(20.0, 30.0, gate[::2, ::3].shape).astype(np.float32)
    projected = np.concatenate([f32_to_bf16(gate), f32_to_bf16(up)], axis=1)
    x = torch.from_numpy(projected.view(np.int16)).view(torch.bfloat16).to(device)

    act = torch.empty((rows, width), dtype=torch.uint8, device=device)
    scales = torch.empty((rows, width // 128), dtype=torch.float32, device=device)
    call("d3_silu_mul_quant", ptr(x), rows, width, None, None, None, 0, ptr(act), ptr(scales),
         _lib.stream(device))
    got_bf16 = np_bf16(silu_mul(x))
    torch.cuda.synchronize()
    want_q, want_s = om.silu_mul_quant(projected)
    assert np.array_equal(np_u8(act), want_q)
    assert np.array_equal(np_f32(scales), want_s)

    g, u = bf16_to_f32(projected[:, :width]), bf16_to_f32(projected[:, width:])
    want = om.silu_mul(projected)
    tail = g < -87.3
    assert np.array_equal(got_bf16[~tail], want[~tail])
    assert np.all(np.abs(bf16_to_f32(got_bf16[tail])) <= 2.0**-118 * np.abs(u[tail]))
