"""The C-ABI library loads, exports every entry point declared in
include/drama3_moe.h with the declared arity, and rejects contract
violations before launching anything (CPU only: no kernel is run)."""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "drama3_moe.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for match in re.finditer(r"\b(?:int|int32_t|int64_t|const char \*)\s*(d3_\w+)\s*\(([^)]*)\)\s*;", text):
        params = match.group(2).strip()
        out[match.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


@pytest.fixture(scope="module")
def lib():
    from drama3_amd import _lib

    if not _lib.LIBRARY.exists():
        pytest.skip("library not built")
    return _lib.load()


def _params(signature: str):
    names = []
    for param in signature.split(","):
        param = param.strip()
        if param in ("", "void"):
            continue
        names.append(re.findall(r"(\w+)\s*$", param)[0])
    return names


def test_definitions_match_header_parameter_order():
    """Same-typed parameters in a different order compile silently; compare
    the names of every extern "C" definition with its declaration."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    declared = {m.group(1): _params(m.group(2)) for m in re.finditer(
        r"\b(?:int|int32_t|int64_t|const char \*)\s*(d3_\w+)\s*\(([^)]*)\)\s*;", text)}
    defined = {}
    for src in (ROOT / "drama-3-single-b300-inference_amd" / "csrc").glob("*.*"):
        for m in re.finditer(r'extern "C" (?:int|int32_t|int64_t|const char\*) (d3_\w+)\(([^)]*)\)\s*\{',
                             src.read_text()):
            defined[m.group(1)] = _params(m.group(2))
    assert set(defined) == set(declared)
    for name, params in declared.items():
        assert defined[name] == params, name


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ("d3_compact_slots", "d3_route", "d3_quantize_rows", "d3_prepare_moe_input",
                     "d3_sort_routes", "d3_expert_gemm", "d3_silu_mul_quant",
                     "d3_weighted_combine", "d3_combine_experts", "d3_combine_experts_add_norm",
                     "d3_row_metadata", "d3_requests_load", "d3_requests_save"):
        assert required in names


def test_every_declared_symbol_is_exported_with_its_arity(lib):
    from drama3_amd import _lib

    declared = declared_functions()
    assert set(declared) == set(_lib.SIGNATURES), "header and ctypes table disagree"
    for name, arity in declared.items():
        assert hasattr(lib, name), name
        assert len(_lib.SIGNATURES[name][1]) == arity, name


def test_capacity_helpers(lib):
    from oracle import moe as om

    for pairs, experts, tile in ((32, 16, 16), (384, 128, 16), (33280, 128, 64), (0, 8, 16)):
        assert lib.d3_max_sorted_rows(pairs, experts, tile) == om.max_sorted_rows(pairs, experts, tile)
    assert lib.d3_max_items(384, 128, 64) == (384 + 128 * 63) // 64
    assert lib.d3_abi_version() == 12
    # wide sort scratch: chunk histograms [ceil(pairs / 512)][E] + ranks [pairs]
    assert lib.d3_sort_wide_scratch_ints(3668, 8, 128) == (-(-3668 * 8 // 512)) * 128 + 3668 * 8
    assert lib.d3_sort_wide_scratch_ints(-1, 8, 128) == -1


def _histograms(pairs: int, experts: int):
    """Every expert histogram of `pairs` routes over `experts` experts."""
    if experts == 1:
        yield (pairs,)
        return
    for first in range(pairs + 1):
        for rest in _histograms(pairs - first, experts - 1):
            yield (first,) + rest


def test_capacities_bound_every_histogram(lib):
    """The sorted-row and work-item capacities against brute force over
    every histogram of small batches: d3_max_sorted_rows and d3_max_items
    are the largest padded row count and item count any histogram needs
    (tight), d3_max_items_aligned bounds the items with each odd run padded
    by one empty item (the wide sort's aligned layout)."""
    for experts in (1, 2, 3, 4):
        for pairs in range(0, 11):
            hists = list(_histograms(pairs, experts))
            for tile in (1, 2, 3, 4, 16):
                need = max(sum(-(-c // tile) * tile for c in h) for h in hists)
                assert lib.d3_max_sorted_rows(pairs, experts, tile) >= need
            for item_rows in (1, 2, 3, 4, 16):
                items = [[-(-c // item_rows) for c in h] for h in hists]
                plain = max(sum(n) for n in items)
                aligned = max(sum(k + (k & 1) for k in n) for n in items)
                assert lib.d3_max_items(pairs, experts, item_rows) == plain
                assert lib.d3_max_items_aligned(pairs, experts, item_rows) >= aligned
    assert lib.d3_max_items(-1, 4, 16) == -1 and lib.d3_max_items_aligned(4, 0, 16) == -1


def test_contract_violations_raise_value_error(lib):
    from drama3_amd import _lib

    with pytest.raises(ValueError, match="null"):
        _lib.call("d3_route", None, 0, 16, 4, 16, 8, None, None, None, None, None, 0, None)
    with pytest.raises(ValueError, match="num_experts"):
        _lib.call("d3_route", 16, 0, 1024, 4, 1024, 8, None, None, 16, None, 16, 0, None)
    with pytest.raises(ValueError, match="multiple of 128"):
        _lib.call("d3_quantize_rows", 16, 200, 4, 200, None, None, 16, 16, 0, None)
    with pytest.raises(ValueError, match="max_rows"):
        _lib.call("d3_sort_routes", 16, 3, 4, None, 8, 16, 16, 16, 16, 16, 16, 16, 8, None, 16,
                  None, 0, None, None, None)
    with pytest.raises(ValueError, match="K="):
        _lib.call("d3_expert_gemm", 0, 16, 16, 0, 4, 512, 384, 16, 16, 16, 8, 16, 16, 4, 16, 64,
                  16, None, None)
    with pytest.raises(ValueError, match="weight_layout"):
        _lib.call("d3_expert_gemm", 0, 16, 16, 7, 4, 512, 512, 16, 16, 16, 8, 16, 16, 4, 16, 64,
                  16, None, None)
    with pytest.raises(ValueError, match="intermediate 2048"):
        _lib.call("d3_expert_fc2_swiglu", 16, 16, 0, 4, 1024, 2048, 16, 16, 8, 16, 16, 4, 16, 64,
                  16, None)
    with pytest.raises(ValueError, match="multiple of 16"):
        _lib.call("d3_pack_expert_weights", 16, 4, 24, 128, 32, None)
    # tiled grouped GEMMs: item size, K, shared-expert operands, N tiling
    with pytest.raises(ValueError, match="item_rows 256"):
        _lib.call("d3_grouped_fc1_swiglu", 16, 16, 0, 4, 256, 1024, 16, 100, 16, 16, 8, 16, 16, 4,
                  256, None, None, 0, 0, 16, 16, None)
    with pytest.raises(ValueError, match="K=384"):
        _lib.call("d3_grouped_fc1_swiglu", 16, 16, 0, 4, 256, 384, 16, 100, 16, 16, 8, 16, 16, 4,
                  128, None, None, 0, 0, 16, 16, None)
    with pytest.raises(ValueError, match="shared expert"):
        _lib.call("d3_grouped_fc1_swiglu", 16, 16, 0, 4, 256, 1024, 16, 100, 16, 16, 8, 16, 16, 4,
                  128, 16, None, 100, 0, 16, 16, None)
    with pytest.raises(ValueError, match="shared expert"):
        _lib.call("d3_grouped_fc2", 16, 16, 0, 4, 1024, 256, 16, 100, 16, 16, 8, 16, 16, 4, 128,
                  16, 16, 60, 50, 0, 16, None)
    with pytest.raises(ValueError, match="multiple of 256"):
        _lib.call("d3_grouped_fc2", 16, 16, 0, 4, 640, 256, 16, 100, 16, 16, 8, 16, 16, 4, 128,
                  None, None, 0, 0, 0, 16, None)
    with pytest.raises(ValueError, match="scratch"):
        _lib.call("d3_sort_routes_wide", 16, 2, 1100, None, 8, 128, 16, 16, 16, 16, 16, 16,
                  lib.d3_max_sorted_rows(8800, 128, 16), 16, 16, None, 0, None, None, 16, 10, None)
    assert "scratch of 10 ints" in lib.d3_last_error().decode()
    # mixed rows: null outputs, prefix reuse limits (prompts, row space)
    with pytest.raises(ValueError, match="null pointer"):
        _lib.call("d3_mixed_rows", 16, 64, 48, 32, 16, 2, 512, None, 11, None, 0, 16, 16, 16, None,
                  16, 16, None, None, None)
    with pytest.raises(ValueError, match="17 prompts"):
        _lib.call("d3_mixed_rows", 16, 64, 48, 32, 16, 17, 512, 16, 11, None, 0, 16, 16, 16, 16,
                  16, 16, None, None, None)
    with pytest.raises(ValueError, match="9048 rows"):
        _lib.call("d3_mixed_rows", 16, 64, 48, 32, 16, 2, 9000, 16, 11, None, 0, 16, 16, 16, 16,
                  16, 16, None, None, None)
    with pytest.raises(ValueError, match="row metadata needs"):
        _lib.call("d3_mixed_rows", 16, 64, 48, 32, 16, 2, 512, None, 11, 16, 1, 16, 16, 16, 16,
                  16, 16, 16, 16, None)


def test_decode_step_entry_points_check_before_launching(lib):
    """Both decode-step entry points reject bad shapes with no GPU call: the
    static variant its scratch limits first, the workspace one every stage."""
    from drama3_amd import _lib

    args = (16, 16, 16, 16, 16, 1024, 256, 16, 128, 16, 1024, 16, 0, 16, 8, 64)
    with pytest.raises(ValueError, match="exceeds the static scratch"):
        _lib.call("d3_decode_step_static", *args, 16, 16, 16, None)
    with pytest.raises(ValueError, match="exceed the static scratch"):
        _lib.call("d3_decode_step_static", 16, 16, 16, 16, 16, 4096, 256, 16, 64, 16, 4096, 16,
                  0, 16, 8, 64, 16, 16, 16, None)
    with pytest.raises(ValueError, match="K=1536 not in the compiled set"):
        _lib.call("d3_decode_step", 16, 16, 16, 16, 16, 1536, 256, 16, 64, 16, 1536, 16, 0, 16,
                  8, 64, 16, 16, 0, 16, 16, 16, 16, 16, None)
    with pytest.raises(ValueError, match="null pointer"):
        _lib.call("d3_decode_step", 16, 16, 16, 16, 16, 1024, 256, 16, 64, 16, 1024, 16, 0, 16,
                  8, 64, None, 16, 0, 16, 16, 16, 16, 16, None)


def test_decode_gemm_contract(lib):
    """Every call is rejected by the host checks before a launch (the
    pointers are aligned dummies, never dereferenced)."""
    from drama3_amd import _lib

    with pytest.raises(ValueError, match="mode"):
        _lib.call("d3_decode_expert_gemm", 1, 16, 16, 4, 512, 1024, 16, None, None, 64, 8, 16, 16,
                  64, 16, None, None)
    with pytest.raises(ValueError, match="capacity"):
        _lib.call("d3_decode_expert_gemm", 0, 16, 16, 4, 512, 1024, 16, None, None, 300, 8, 16, 16,
                  64, 16, None, None)
    with pytest.raises(ValueError, match="K=768"):
        _lib.call("d3_decode_expert_gemm", 0, 16, 16, 4, 512, 768, 16, None, None, 64, 8, 16, 16,
                  64, 16, None, None)
    with pytest.raises(ValueError, match="row_slots"):  # the slot layout is FC2's only
        _lib.call("d3_decode_expert_gemm", 0, 16, 16, 4, 512, 1024, 16, None, 16, 64, 8, 16, 16,
                  64, 16, None, None)


def test_route_fc1_and_combine_contract(lib):
    from drama3_amd import _lib

    p = 256  # any aligned non-null address: every call below is rejected before a launch
    fc1 = [p, p, 128, 1536, 2048, p, 64, p, 2048, p, _lib.DTYPE_BF16, 128, 8, 16, p, p, p, p, None]
    bad = list(fc1)
    bad[3 - 1] = 300  # E above what a workgroup ranks
    with pytest.raises(ValueError, match="E=300"):
        _lib.call("d3_decode_route_fc1", *bad)
    bad = list(fc1)
    bad[11] = 130  # logits rows not 16-byte aligned
    with pytest.raises(ValueError, match="aligned"):
        _lib.call("d3_decode_route_fc1", *bad)
    bad = list(fc1)
    bad[6] = 300  # capacity
    with pytest.raises(ValueError, match="capacity"):
        _lib.call("d3_decode_route_fc1", *bad)
    bad = list(fc1)
    bad[10] = _lib.DTYPE_I32
    with pytest.raises(ValueError, match="logits"):
        _lib.call("d3_decode_route_fc1", *bad)
    combine = [p, 64, p, _lib.DTYPE_BF16, 128, 128, 8, 2048, p, p, _lib.DTYPE_BF16, p, None]
    bad = list(combine)
    bad[6] = 9  # top_k above 8
    with pytest.raises(ValueError, match="top_k"):
        _lib.call("d3_decode_route_combine", *bad)
    bad = list(combine)
    bad[0] = None
    with pytest.raises(ValueError, match="null"):
        _lib.call("d3_decode_route_combine", *bad)


def test_empty_batches_accept_null_buffers(lib):
    """Zero rows: NULL row buffers are accepted and nothing is launched (the
    calls below return before any HIP call); one row with the same NULLs is
    still a contract violation, and shape checks still apply at zero rows."""
    from drama3_amd import _lib

    bf16 = _lib.DTYPE_BF16
    for rows, ok in ((0, True), (1, False)):
        calls = [
            ("d3_route", (None, bf16, 16, rows, 16, 8, None, None, None, None, None, bf16, None)),
            ("d3_quantize_rows", (None, 1024, rows, 1024, None, None, None, None, 0, None)),
            ("d3_combine_experts", (None, None, None, 1, rows, 1024, None, None)),
            ("d3_add_norm", (None, None, None, 1e-6, rows, 1024, None, None)),
            ("d3_silu_mul", (None, 2048, rows, 1024, None, None)),
            ("d3_dense_bf16", (None, 1024, rows, None, 256, 1024, 0, None, 256, None, 0, None)),
        ]
        for name, args in calls:
            if ok:
                _lib.call(name, *args)
            else:
                with pytest.raises(ValueError, match="null"):
                    _lib.call(name, *args)
    with pytest.raises(ValueError, match="width"):
        _lib.call("d3_add_norm", None, None, None, 1e-6, 0, 1022, None, None)


def test_product_code_does_not_import_the_oracle():
    package = ROOT / "drama-3-single-b300-inference_amd"
    for path in package.rglob("*.py"):
        text = path.read_text()
        assert "oracle" not in re.findall(r"^\s*(?:from|import)\s+(\w+)", text, flags=re.M), path


def test_no_cpu_fallback_when_library_missing(monkeypatch, tmp_path):
    from drama3_amd import _lib

    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setenv("DRAMA3_MOE_LIBRARY", str(tmp_path / "missing.so"))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        _lib.load()


def test_ctypes_types_are_plain():
    from drama3_amd import _lib

    allowed = {ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float,
               ctypes.c_char_p}
    for restype, argtypes in _lib.SIGNATURES.values():
        assert restype in allowed and all(a in allowed for a in argtypes)


def test_packed_operands_follow_their_source_tensor():
    """prepare_experts' packed copies are used only while the checkpoint-layout
    tensor they were made from is unchanged (host logic; no kernel runs)."""
    import torch

    from drama3_amd import expert_weights as ew
    from drama3_amd.workloads import make_experts

    ex = make_experts(torch.Generator("cpu").manual_seed(0), 2, 256, 128)
    assert ew.fc1_operands(ex)[2] == ew.LAYOUT_REFERENCE
    for name in ("w13", "w2"):
        weight = getattr(ex, f"{name}_weight")
        setattr(ex, f"d3_{name}_packed", torch.empty_like(weight))
        setattr(ex, f"d3_{name}_source", ew._identity(weight))
    w, scales, layout = ew.fc1_operands(ex)
    assert layout == ew.LAYOUT_FRAGMENT and w is ex.d3_w13_packed and scales is ex.w13_scale_inv
    ex.w2_weight.view(torch.uint8).add_(1)
    assert ew.fc2_operands(ex)[2] == ew.LAYOUT_REFERENCE
    ex.w13_weight = ex.w13_weight.clone()
    assert ew.fc1_operands(ex)[2] == ew.LAYOUT_REFERENCE
