"""Pin the oracle's route sort (kernels.py:658-731) and expert FFN
(kernels.py:290-357, 702-779) against brute force and closed forms (CPU)."""

import numpy as np
import pytest

from oracle import moe as om
from oracle.numerics import bf16_to_f32, e4m3_to_f32, f32_to_bf16, f32_to_e4m3


def random_ids(rng, tokens, experts, top_k=8):
    return np.stack([rng.permutation(experts)[:top_k] for _ in range(tokens)]).astype(np.int64)


@pytest.mark.parametrize("tokens,experts,tile", [(4, 16, 16), (48, 128, 16), (64, 16, 64),
                                                 (300, 128, 16), (1, 8, 16)])
def test_sort_against_brute_force(tokens, experts, tile):
    rng = np.random.default_rng(tokens)
    ids = random_ids(rng, tokens, experts)
    s = om.sort_routes(ids, experts, tile)
    flat = ids.reshape(-1)
    pairs = flat.size
    assert np.array_equal(s.counts, np.bincount(flat, minlength=experts))
    assert np.all(s.starts % tile == 0)
    assert s.total <= om.max_sorted_rows(pairs, experts, tile)
    for e in range(experts):
        members = [p for p in range(pairs) if flat[p] == e]  # ascending pair order
        start, c = s.starts[e], s.counts[e]
        assert s.sorted_ids[start:start + c].tolist() == members
        padded = -(-c // tile) * tile
        assert np.all(s.sorted_ids[start + c:start + padded] == pairs)
        assert np.all(s.expert_ids[start // tile:(start + padded) // tile] == e)
    valid = s.sorted_ids < pairs
    assert sorted(s.sorted_ids[valid].tolist()) == list(range(pairs))
    assert np.array_equal(s.sorted_ids[s.inverse], np.arange(pairs))


def test_sort_capacity_worst_cases():
    # every route to one expert, and every route to a distinct expert
    for ids, experts in ((np.zeros((37, 1), np.int64), 16),
                         (np.arange(128).reshape(16, 8), 128)):
        for tile in (16, 64):
            s = om.sort_routes(ids, experts, tile)
            assert s.total <= om.max_sorted_rows(ids.size, experts, tile)


def tiny_weights(rng, experts, hidden, inter):
    w13 = f32_to_e4m3(rng.standard_normal((experts, 2 * inter, hidden)).astype(np.float32))
    w2 = f32_to_e4m3(rng.standard_normal((experts, hidden, inter)).astype(np.float32))
    s13 = np.exp(0.5 * rng.standard_normal((experts, 2 * inter // 128, hidden // 128))).astype(np.float32)
    s2 = np.exp(0.5 * rng.standard_normal((experts, hidden // 128, inter // 128))).astype(np.float32)
    return om.ExpertWeights(w13, s13, w2, s2)


def brute_force_ffn(x_bf16, ids, w_bf16, wt: om.ExpertWeights):
    """Element-by-element evaluation straight from the reference formulas in
    Python floats, with non-square block-scale grids so a transposed scale
    index would not cancel out."""
    tokens, top_k = ids.shape
    experts, two_i, hidden = wt.w13.shape
    inter = two_i // 2
    x = bf16_to_f32(x_bf16)
    q, xs = om.quantize_rows(x)
    xq = e4m3_to_f32(q)
    out = np.zeros((tokens, hidden), np.float64)
    w = bf16_to_f32(w_bf16)
    for t in range(tokens):
        for r in range(top_k):
            e = int(ids[t, r])
            gu = np.zeros(two_i, np.float32)
            for n in range(two_i):
                acc = 0.0
                for k in range(hidden):
                    wv = float(np.float32(e4m3_to_f32(wt.w13[e, n, k]) * wt.s13[e, n // 128, k // 128]))
                    xv = float(np.float32(xq[t, k] * xs[t, k // 128]))
                    acc += wv * xv
                gu[n] = np.float32(acc)
            gu_b = f32_to_bf16(gu)[None]
            aq, as_ = om.silu_mul_quant(gu_b)
            a = e4m3_to_f32(aq[0])
            for n in range(hidden):
                acc = 0.0
                for k in range(inter):
                    wv = float(np.float32(e4m3_to_f32(wt.w2[e, n, k]) * wt.s2[e, n // 128, k // 128]))
                    av = float(np.float32(a[k] * as_[0, k // 128]))
                    acc += wv * av
                out[t, n] += float(w[t, r]) * float(np.float32(acc))
    return f32_to_bf16(out.astype(np.float32))


def test_expert_ffn_against_brute_force():
    rng = np.random.default_rng(7)
    experts, hidden, inter, tokens, top_k = 3, 256, 128, 2, 2
    wt = tiny_weights(rng, experts, hidden, inter)
    x = f32_to_bf16(rng.standard_normal((tokens, hidden)).astype(np.float32))
    ids = random_ids(rng, tokens, experts, top_k)
    weights, _ = om.route(rng.standard_normal((tokens, experts)).astype(np.float32), top_k)
    ours = bf16_to_f32(om.expert_ffn(x, ids, weights, wt))
    brute = bf16_to_f32(brute_force_ffn(x, ids, weights, wt))
    ulp = np.abs(brute) * 2.0**-7 + 1e-30
    assert np.all(np.abs(ours - brute) <= ulp)


def test_expert_ffn_integer_exact_case():
    """Unit scales and small integer weights/activations: every product and
    sum is exact in fp32, so FC1 equals the integer matmul exactly."""
    experts, hidden, inter = 2, 128, 128
    rng = np.random.default_rng(8)
    w13v = rng.integers(-3, 4, (experts, 2 * inter, hidden)).astype(np.float32)
    w13 = f32_to_e4m3(w13v)
    x = np.zeros((1, hidden), np.float32)
    x[0, :4] = [448.0, -224.0, 112.0, 56.0]  # amax 448 -> scale exactly 1.0
    q, xs = om.quantize_rows(x)
    assert xs[0, 0] == 1.0
    ids = np.array([[1]])
    wt = om.ExpertWeights(w13, np.ones((experts, 2, 1), np.float32),
                          np.zeros((experts, hidden, inter), np.uint8), np.ones((experts, 1, 1), np.float32))
    gu = bf16_to_f32(om.expert_fc1(q, xs, ids, wt))
    exact = w13v[1] @ x[0]
    assert np.array_equal(gu[0], bf16_to_f32(f32_to_bf16(exact.astype(np.float32))))


def test_expert_ffn_permutation_invariance():
    """Renaming experts (permuting weights and ids together) and permuting
    tokens leaves the per-token outputs unchanged."""
    rng = np.random.default_rng(9)
    experts, hidden, inter, tokens = 4, 128, 128, 5
    wt = tiny_weights(rng, experts, hidden, inter)
    x = f32_to_bf16(rng.standard_normal((tokens, hidden)).astype(np.float32))
    ids = random_ids(rng, tokens, experts, 2)
    w, _ = om.route(rng.standard_normal((tokens, experts)).astype(np.float32), 2)
    base = om.expert_ffn(x, ids, w, wt)
    perm = rng.permutation(experts)
    inv = np.argsort(perm)
    wt2 = om.ExpertWeights(wt.w13[perm], wt.s13[perm], wt.w2[perm], wt.s2[perm])
    assert np.array_equal(om.expert_ffn(x, inv[ids], w, wt2), base)
    tp = rng.permutation(tokens)
    assert np.array_equal(om.expert_ffn(x[tp], ids[tp], w[tp], wt), base[tp])


def test_planted_scale_transpose_is_detected():
    """A plausible bug (block scales indexed [k/128, n/128]) must change the
    FC1 output, so the brute-force comparison above can catch it."""
    rng = np.random.default_rng(10)
    wt = tiny_weights(rng, 2, 256, 256)  # square grid would hide nothing: use 4x2 vs 2x2
    x = f32_to_bf16(rng.standard_normal((1, 256)).astype(np.float32))
    q, xs = om.quantize_rows(bf16_to_f32(x))
    ids = np.array([[0]])
    good = om.expert_fc1(q, xs, ids, wt)
    bad_wt = om.ExpertWeights(wt.w13, np.ascontiguousarray(np.swapaxes(wt.s13, 1, 2)[:, :, :]).reshape(wt.s13.shape),
                              wt.w2, wt.s2)
    assert not np.array_equal(om.expert_fc1(q, xs, ids, bad_wt), good)


def test_weighted_combine_rank_order_sum():
    rng = np.random.default_rng(11)
    down = rng.standard_normal((3 * 8, 64)).astype(np.float32)
    w = rng.uniform(0, 1, (3, 8)).astype(np.float32)
    out = bf16_to_f32(om.weighted_combine(down, w))
    expected = np.einsum("tr,trh->th", w.astype(np.float64), down.reshape(3, 8, 64).astype(np.float64))
    assert np.all(np.abs(out - expected) <= np.abs(expected) * 2.0**-8 + 1e-6)
