"""Pin the oracle's prefix row reuse (row_reuse.py:46-109) and the mixed
decode + prefill row layout (mixed_graph.py:139-179) on the CPU.

The reuse cases are the ones the reference's own tests assert
(tests/test_row_reuse.py:19-117): ownership invariants on capture-shaped,
reordered, partial and cancelled prompt sets, the per-column causal rule,
and the capacity fallbacks; plus a pure-Python restatement of the ownership
rule (row tuples compared one by one) on random prompt sets."""

import numpy as np
import pytest

from oracle import moe as om

BUCKETS = ((64, 768, 256, 576), (64, 1024, 256, 832), (64, 1280, 256, 1088),
           (64, 1536, 256, 1088), (64, 1536, 256, 1344))


def prompt(length, value=0):
    rows = np.zeros((length, 11), dtype=np.int64)
    rows[:, 0] = value
    return rows


def owners_of(plan, d, full):
    compact, _, packed = plan
    keep, inverse = packed[:compact], packed[compact:]
    assert len(inverse) == full and inverse.min() >= 0 and inverse.max() < compact
    return keep, inverse, keep[inverse]


def check_plan(plan, prompts, d, capacity):
    full = d + capacity
    compact, unique, _ = plan
    keep, inverse, owner = owners_of(plan, d, full)
    assert np.array_equal(owner[:d], np.arange(d))
    starts = np.concatenate([[d], d + np.cumsum([len(p) for p in prompts])])
    assert np.array_equal(owner[starts[-1]:], np.arange(starts[-1], full))
    for i, p in enumerate(prompts):
        for pos in range(len(p)):
            src = int(owner[starts[i] + pos])
            assert d <= src <= starts[i] + pos
            j = int(np.searchsorted(starts, src, side="right") - 1)
            assert src - starts[j] == pos
            assert np.array_equal(p[:pos + 1], prompts[j][:pos + 1])
    assert len(np.unique(owner)) == unique
    assert np.array_equal(keep[:unique], np.flatnonzero(owner == np.arange(full)))
    assert np.all(keep[unique:] == 0)
    assert (unique + 63) // 64 * 64 <= compact


@pytest.mark.parametrize("d,capacity,span,compact", BUCKETS)
def test_capture_shaped_prompts(d, capacity, span, compact):
    sizes = [capacity // 9] * 8
    prompts = [prompt(n, 3) for n in sizes]
    plan = om.plan_row_reuse(prompts, d, capacity, (compact,))
    assert plan is not None and plan[0] == compact
    check_plan(plan, prompts, d, capacity)


@pytest.mark.parametrize("column", range(11))
def test_every_column_breaks_the_alias(column):
    a, b = prompt(128), prompt(128)
    b[17, column] = 7
    prompts = [a, b, a.copy(), b.copy()]
    plan = om.plan_row_reuse(prompts, 64, 768, (576,))
    assert plan is not None
    check_plan(plan, prompts, 64, 768)
    inverse = plan[2][plan[0]:]
    assert np.array_equal(inverse[64:81], inverse[192:209])
    assert np.all(inverse[81:192] != inverse[209:320])


def test_partial_reordered_and_cancelled():
    a, b = prompt(128), prompt(128)
    b[12, 10] = 1
    prompts = [a, b, a[:80], b[:100], a.copy()]
    plan = om.plan_row_reuse(prompts, 64, 768, (576,))
    assert plan is not None
    check_plan(plan, prompts, 64, 768)
    backwards = list(reversed(prompts))
    reverse = om.plan_row_reuse(backwards, 64, 768, (576,))
    assert reverse is not None
    check_plan(reverse, backwards, 64, 768)
    assert not np.array_equal(plan[2], reverse[2])
    survivors = [a, a.copy(), a.copy()]
    remaining = om.plan_row_reuse(survivors, 64, 768, (576,))
    assert remaining is not None
    check_plan(remaining, survivors, 64, 768)
    assert om.plan_row_reuse(survivors[:2], 64, 768, (576,)) is None


def test_capacity_fallbacks():
    distinct = [prompt(128, i) for i in range(6)]
    assert om.plan_row_reuse(distinct, 64, 768, (576,)) is None
    assert om.plan_row_reuse(distinct, 64, 768, ()) is None
    assert om.plan_row_reuse([prompt(3)] * 8, 64, 768, (576,)) is None
    prompts = [prompt(180), prompt(180), prompt(170, 1), prompt(170, 1)]
    plan = om.plan_row_reuse(prompts, 64, 1536, (1344, 1088))
    assert plan is not None and plan[0] == 1344
    check_plan(plan, prompts, 64, 1536)


def owners_by_tuples(prompts, d, full):
    """The ownership rule with rows compared as tuples, one row at a time."""
    owners = list(range(full))
    starts = []
    offset = d
    for i, p in enumerate(prompts):
        best, best_j = 0, -1
        for j in range(i):
            q = prompts[j]
            n = 0
            while n < min(len(p), len(q)) and tuple(p[n]) == tuple(q[n]):
                n += 1
            if n > best:
                best, best_j = n, j
        for pos in range(best):
            owners[offset + pos] = owners[starts[best_j] + pos]
        starts.append(offset)
        offset += len(p)
    return np.array(owners)


@pytest.mark.parametrize("seed", range(6))
def test_owners_match_row_by_row_rule(seed):
    rng = np.random.default_rng(seed)
    base = rng.integers(0, 3, (40, 11))
    prompts = []
    for _ in range(int(rng.integers(2, 9))):
        n = int(rng.integers(3, 41))
        p = base[:n].copy()
        if rng.random() < 0.7:
            p[int(rng.integers(0, n)), int(rng.integers(0, 11))] += 1
        prompts.append(p)
    d, capacity = 5, 400
    full = d + capacity
    got = om.prompt_row_owners(prompts, d, full)
    assert np.array_equal(got, owners_by_tuples(prompts, d, full))
    assert np.array_equal(got[got], got)  # canonical


def test_mixed_layout_small_case():
    occupancy = np.array([0, 1, 0, 1, 1, 0], dtype=np.uint8)
    a = prompt(4, 5)
    b = a.copy()
    b[2, 3] = 9
    frames = np.concatenate([a, b, prompt(2, 7)])  # last two rows: padding sequence
    boundaries = np.array([0, 4, 8, 8, 10], dtype=np.int32)
    lay = om.mixed_layout(occupancy, 4, 100, boundaries, 3, 10, frames)
    assert lay.count == 3 and lay.active.tolist() == [1, 3, 4, -1, -1, -1]
    assert lay.decode_slots.tolist() == [1, 3, 4, 103]
    # rows: decode 0-2 live, 3 padding; prompt a 4-7; b 8-11 (8, 9 alias 4, 5); padding 12, 13
    assert lay.keep_count == 9
    assert lay.keep[:9].tolist() == [0, 1, 2, 4, 5, 6, 7, 10, 11]
    assert np.all(lay.keep[9:] == 0)
    assert lay.inverse.tolist() == [0, 1, 2, 0, 3, 4, 5, 6, 3, 4, 7, 8, 0, 0]


def test_mixed_layout_without_reuse_and_overfull_decode():
    occupancy = np.ones(6, dtype=np.uint8)
    lay = om.mixed_layout(occupancy, 4, 50, np.array([0, 3, 5], dtype=np.int32), 1, 5)
    assert lay.count == 6 and lay.decode_slots.tolist() == [0, 1, 2, 3]
    assert lay.keep_count == 7 and lay.keep[:7].tolist() == [0, 1, 2, 3, 4, 5, 6]
    assert lay.inverse.tolist() == [0, 1, 2, 3, 4, 5, 6, 0, 0]
