"""The wide route sort (d3_sort_routes_wide: one workgroup per 512 pairs)
against the CPU oracle, bit for bit: histogram, padded offsets, stable
sorted pair list with sentinel padding, expert ids, inverse map and work
items, at prefill sizes, under skew, for int64 ids, with a device row count
below the capacity, and at the 512-expert limit.  With an items array of
d3_max_items_aligned's capacity, and experts with routes averaging at least
1.5 items, each expert's items are padded to an even count by one empty
item (rows 0).  The reference-named
sort_routes() takes this path above 8192 pairs."""

import numpy as np
import pytest
import torch

from oracle import moe as om

pytestmark = pytest.mark.gpu


def run_wide(device, ids_np, experts, tile, item_rows, live_rows=None, dtype=torch.int32,
             aligned=False):
    from drama3_amd import _lib
    from drama3_amd._lib import call, ptr
    from drama3_amd.pipeline import dtype_code

    lib = _lib.load()
    rows, top_k = ids_np.shape
    pairs = rows * top_k
    i32 = dict(dtype=torch.int32, device=device)
    max_rows = lib.d3_max_sorted_rows(pairs, experts, tile)
    max_items = (lib.d3_max_items_aligned if aligned else lib.d3_max_items)(pairs, experts, item_rows)
    out = dict(counts=torch.empty(experts, **i32), starts=torch.empty(experts, **i32),
               total=torch.empty(1, **i32), sorted_ids=torch.empty(max_rows, **i32),
               expert_ids=torch.empty(max_rows // tile, **i32), inverse=torch.empty(pairs, **i32),
               items=torch.empty((max_items, 4), **i32), num_items=torch.empty(1, **i32),
               pairs=torch.empty(1, **i32))
    scratch = torch.empty(lib.d3_sort_wide_scratch_ints(rows, top_k, experts), **i32)
    ids = torch.from_numpy(ids_np).to(dtype).to(device)
    count = None if live_rows is None else torch.tensor([live_rows], **i32)
    call("d3_sort_routes_wide", ptr(ids), dtype_code(ids.dtype), rows, ptr(count), top_k, experts,
         tile, ptr(out["counts"]), ptr(out["starts"]), ptr(out["total"]), ptr(out["sorted_ids"]),
         ptr(out["expert_ids"]), max_rows, ptr(out["inverse"]), item_rows, ptr(out["items"]),
         max_items, ptr(out["num_items"]), ptr(out["pairs"]), ptr(scratch), scratch.numel(),
         _lib.stream(device))
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in out.items()}


def padded_items(counts, item_rows) -> bool:
    """The wide sort's rule: pad while the experts with routes average at
    least 1.5 items."""
    items = sum(-(-int(c) // item_rows) for c in counts)
    used = int(np.count_nonzero(counts))
    return 2 * items >= 3 * used


def check(got, ids_np, experts, tile, item_rows, aligned=False):
    """Returns whether the items were padded."""
    o = om.sort_routes(ids_np, experts, tile)
    aligned = aligned and padded_items(o.counts, item_rows)
    pairs = ids_np.size
    assert np.array_equal(got["counts"], o.counts)
    assert np.array_equal(got["starts"], o.starts)
    assert int(got["total"][0]) == o.total and int(got["pairs"][0]) == pairs
    assert np.array_equal(got["sorted_ids"][:o.total], o.sorted_ids)
    assert np.all(got["sorted_ids"][o.total:] == pairs)
    assert np.array_equal(got["expert_ids"][:o.total // tile], o.expert_ids)
    assert np.all(got["expert_ids"][o.total // tile:] == -1)
    assert np.array_equal(got["inverse"][:pairs], o.inverse)
    items = []
    for e in range(experts):
        n_e = -(-int(o.counts[e]) // item_rows)
        items += [(e, int(o.starts[e]) + j * item_rows,
                   min(item_rows, int(o.counts[e]) - j * item_rows), 0) for j in range(n_e)]
        if aligned and n_e % 2:
            items.append((e, int(o.starts[e]), 0, 0))
    n = int(got["num_items"][0])
    assert n == len(items)
    assert np.array_equal(got["items"][:n], np.array(items, np.int32).reshape(-1, 4))
    assert np.all(got["items"][n:, 0] == -1)
    return aligned


@pytest.mark.parametrize("rows,experts,dtype", [(3668, 128, torch.int32), (4200, 16, torch.int64),
                                                 (1100, 512, torch.int32)])
def test_wide_sort_matches_oracle(device, rows, experts, dtype):
    rng = np.random.default_rng(rows + experts)
    ids = np.stack([rng.permutation(experts)[:8] for _ in range(rows)]).astype(np.int64)
    got = run_wide(device, ids, experts, 16, 128, dtype=dtype)
    check(got, ids, experts, 16, 128)


def test_wide_sort_skewed_and_live_rows(device):
    """Three quarters of the routes on one expert; only the first 2500 of
    3000 capacity rows live (device row count)."""
    rng = np.random.default_rng(7)
    rows, experts, live = 3000, 64, 2500
    ids = np.stack([np.concatenate([[5], rng.permutation(np.delete(np.arange(experts), 5))[:7]])
                    for _ in range(rows)]).astype(np.int64)
    ids[:, [0, 3]] = ids[:, [3, 0]]  # the hot expert at rank 3
    got = run_wide(device, ids, experts, 16, 128, live_rows=live)
    check({k: v for k, v in got.items()}, ids[:live], experts, 16, 128)


@pytest.mark.parametrize("rows,experts,item_rows,live,padded", [
    (4096, 256, 128, None, False),  # 128 routes per expert: about one item each, no padding
    (3001, 64, 256, None, True), (1100, 512, 16, None, True), (3668, 128, 128, 2900, True)])
def test_wide_sort_aligned_items(device, rows, experts, item_rows, live, padded):
    """Aligned capacity: when padded, every expert's first item sits at an
    even index and the list is the plain one with one empty item after each
    odd run (also with a device row count below the capacity)."""
    rng = np.random.default_rng(rows * 3 + experts)
    ids = np.stack([rng.permutation(experts)[:8] for _ in range(rows)]).astype(np.int64)
    got = run_wide(device, ids, experts, 16, item_rows, live_rows=live, aligned=True)
    assert check(got, ids if live is None else ids[:live], experts, 16, item_rows,
                 aligned=True) == padded
    if padded:
        items = got["items"][:int(got["num_items"][0])]
        first = np.flatnonzero(np.r_[True, items[1:, 0] != items[:-1, 0]])
        assert np.all(first % 2 == 0)


def test_reference_sort_routes_takes_wide_path(device):
    from drama3_amd.kernels import sort_routes

    rng = np.random.default_rng(3)
    ids = np.stack([rng.permutation(128)[:8] for _ in range(2000)])
    counts, starts, total, sorted_ids, expert_ids, inverse = sort_routes(
        torch.from_numpy(ids).to(device), 128, 16)
    o = om.sort_routes(ids, 128, 16)
    assert np.array_equal(sorted_ids.cpu().numpy()[:o.total], o.sorted_ids)
    assert np.array_equal(inverse.cpu().numpy(), o.inverse)


def test_workspace_allows_padded_items_over_the_wide_sort(device):
    """MoEWorkspace gives the wide sort the aligned capacity whenever it runs
    the tiled grouped GEMMs over it (the sort then pads or not from the
    live histogram), not below the wide sort."""
    from drama3_amd import _lib
    from drama3_amd.pipeline import MoEWorkspace, Shape

    lib = _lib.load()
    cases = [((3668, 128, 2048, 768), True), ((4096, 256, 2048, 512), True),
             ((1000, 128, 1024, 256), False)]
    for dims, aligned in cases:
        ws = MoEWorkspace(Shape(*dims), device)
        assert ws.aligned_items == aligned
        want = (lib.d3_max_items_aligned if aligned else lib.d3_max_items)(
            ws.shape.pairs, ws.shape.num_experts, ws.item_rows)
        assert ws.max_items == want
