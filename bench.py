"""Benchmark of the 64-slot FP8 top-8 MoE decode step on
one MI355X.

One step = device-side slot compaction + routing + FP8 quantisation (one
launch), FC1 and FC2 (SwiGLU requant in FC2's prologue) as expert GEMMs that
find their own routes (no route sort), and the weighted combine, over the
live rows of 64 persistent slots (H=2048, 128 experts, I=768, top-8),
captured in a HIP graph.
Inputs are resident in HBM before timing.  ``value`` is the cold-cache rate:
the timed replays rotate over several copies of the expert weights whose
total far exceeds the 256 MB MALL, so every step streams its weights from HBM.

Prints one JSON line (see the ``--help`` text for options).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _path in (ROOT, ROOT / "drama-3-single-b300-inference_amd"):
    if str(_path) not in sys.path:
        sys.path.insert(0, str(_path))

HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E bandwidth
FP8_PEAK_TFLOPS = 5000.0  # MI355X dense FP8 MFMA
# HBM bytes per FC1 launch on this workload, from two rocprofv3 --pmc runs of
# this script (FETCH_SIZE x 2.000 + WRITE_SIZE x 1.000, the factors read off
# the 1 GiB device copy in the same runs); profiles/expert_gemm_c2_hbm_traffic.md.
# Re-measure whenever the FC1 kernel or its tiling changes.
FC1_TRAFFIC_BYTES = {"kernel": "decode_gemm_kernel<16,1,1,6,1,true>", "bytes": 401749606,
                     "measured_on": "bb4fea4, again on 294a999 and 218139f (profiles/expert_gemm_c2_hbm_traffic.md)"}


def parse():
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--copies", type=int, default=6, help="rotated weight copies (cold cache)")
    p.add_argument("--kernel-reps", type=int, default=8, help="FC1/FC2 graph repetitions per copy")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-runs", type=int, default=10,
                   help="timed runs per configuration of the CPU baseline (after 2 warm-ups)")
    p.add_argument("--replays", type=int, default=100,
                   help="individually timed graph replays for the per-replay statistics")
    p.add_argument("--no-parity", action="store_true",
                   help="skip the config-2 output check against the numpy oracle")
    p.add_argument("--no-decode-configs", action="store_true",
                   help="skip the config-1 and config-3 decode lines")
    p.add_argument("--no-prefill", action="store_true",
                   help="skip the config-4 packed-prefill measurement")
    p.add_argument("--prefill-only", action="store_true",
                   help="measure only the config-4 packed prefill (one JSON line)")
    p.add_argument("--prefill-steps", type=int, default=20)
    p.add_argument("--no-reference-shape", action="store_true",
                   help="skip the decode step and the whole MoE layer at the reference model's "
                        "shape (E256, I512)")
    p.add_argument("--no-mixed", action="store_true",
                   help="skip the config-5 mixed decode + prefill step")
    p.add_argument("--mixed-only", action="store_true",
                   help="measure only the config-5 mixed step (one JSON line)")
    p.add_argument("--mixed-steps", type=int, default=50)
    p.add_argument("--decode-config-only", type=int, choices=(1, 2, 3), default=None,
                   help="measure only this decode configuration's step (one JSON line)")
    p.add_argument("--reference-shape-only", action="store_true",
                   help="measure only the decode step at the reference model's shape (one JSON line)")
    p.add_argument("--layer-only", action="store_true",
                   help="measure only the whole MoE layer lines (64 and 4096 rows; one JSON line)")
    return p.parse_args()


def baseline_metric():
    return json.loads((ROOT / "BASELINE.json").read_text())["metric"]


def time_graphs(torch, graphs, count):
    """Mean time per replay (us) of `count` back-to-back replays."""
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for k in range(count):
        graphs[k % len(graphs)].replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1000.0 / count  # us


def replay_stats(torch, graph, replays, per_replay=1, warmup=10):
    """Per-replay timing: `warmup` untimed replays, then `replays` replays,
    each bracketed by its own events on the replay stream.  Returns the
    median and mean per step (us; a replay holds `per_replay` steps) and the
    mean of the whole back-to-back run."""
    import statistics

    for _ in range(warmup):
        graph.replay()
    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in range(replays)]
    first, last = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    first.record()
    for start, end in pairs:
        start.record()
        graph.replay()
        end.record()
    last.record()
    torch.cuda.synchronize()
    each = [s.elapsed_time(e) * 1000.0 / per_replay for s, e in pairs]
    return {"median_us": statistics.median(each), "mean_us": statistics.fmean(each),
            "min_us": min(each), "max_us": max(each),
            "run_mean_us": first.elapsed_time(last) * 1000.0 / (replays * per_replay),
            "replays": replays, "steps_per_replay": per_replay, "warmup_replays": warmup}


def host_cpu():
    """CPU model, usable cores and torch's intra-op thread setting of this host."""
    import torch

    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    info = [line.strip() for line in torch.__config__.parallel_info().splitlines()
            if line.strip().startswith(("ATen", "at::get_num_threads", "OpenMP", "MKL", "Intra-op"))]
    return {"cpu_model": model, "cores": cores, "threads": torch.get_num_threads(),
            "parallel_info": info}


def cpu_baseline(configs, runs: int = 10, warmup: int = 2) -> dict:
    """The PyTorch-CPU restatement of the step (``oracle/cpu_step.py``,
    pinned against the numpy oracle) on this host's cores: median of `runs`
    after `warmup`, per configuration, on each configuration's full first
    step (config 5: its first mixed step's 560 packed rows)."""
    import statistics

    import torch

    from oracle import cpu_step

    host = host_cpu()
    out = {}
    for name, (workload, step) in configs.items():
        x, logits = step.packed()
        times = []
        for k in range(warmup + runs):
            t0 = time.perf_counter()
            cpu_step.moe_step(x, logits, workload.experts, workload.shared)
            if k >= warmup:
                times.append(time.perf_counter() - t0)
        us = statistics.median(times) * 1e6
        out[name] = {"us_per_step": round(us, 1), "rows": len(x),
                     "tokens_per_s": round(len(x) / (us * 1e-6), 1), "runs": runs,
                     "warmup": warmup}
    return {**host, "configs": out}


def decode_parity(workload, step, out) -> dict:
    """The decode step's live output rows against the numpy oracle."""
    import numpy as np
    import torch

    from oracle import moe as om
    from oracle.numerics import bf16_to_f32

    active, _ = om.compact_slots(step.occupancy.numpy())
    x = step.x_slots.view(torch.int16).numpy().view(np.uint16)[active]
    weights, ids = om.route(step.logits_slots.float().numpy()[active])
    wt = om.ExpertWeights(*(t.view(torch.uint8).numpy() if t.dtype.itemsize == 1 else t.numpy()
                            for t in workload.experts.tensors()))
    expected = om.expert_ffn(x, ids, weights, wt)
    got = out.view(torch.int16).cpu().numpy().view(np.uint16)
    a, b = bf16_to_f32(got).astype(np.float64), bf16_to_f32(expected).astype(np.float64)
    err = float(np.sqrt(np.mean((a - b) ** 2) / np.mean(b ** 2)))
    return {"rrms_vs_oracle": err, "max_abs": float(np.abs(a - b).max()),
            "exact_fraction": float(np.mean(got == expected)), "tolerance_rrms": 1e-3,
            "ok": err < 1e-3}


def parity_stats(got_bits, expected_bits, tolerance_rrms: float) -> dict:
    """RRMS, max-abs and exact fraction of bf16 outputs (uint16 bits) against
    the oracle's."""
    import numpy as np

    from oracle.numerics import bf16_to_f32

    a = bf16_to_f32(got_bits).astype(np.float64)
    b = bf16_to_f32(expected_bits).astype(np.float64)
    err = float(np.sqrt(np.mean((a - b) ** 2) / np.mean(b ** 2)))
    return {"rrms_vs_oracle": err, "max_abs": float(np.abs(a - b).max()),
            "exact_fraction": float(np.mean(got_bits == expected_bits)),
            "tolerance_rrms": tolerance_rrms, "ok": err < tolerance_rrms}


def prefill_parity(workload, x, logits, out) -> dict:
    """Config 4's output (routed top-8 + the dense shared expert) against the
    numpy oracle: the FP8-MFMA contraction path, held to the reference's
    same-quantisation threshold (RRMS < 3e-3)."""
    import torch

    from oracle import moe as om

    def np_u8(t):
        return t.view(torch.uint8).numpy()

    ex, sh = workload.experts, workload.shared
    weights, ids = om.route(logits.float().numpy())
    xb = x.view(torch.int16).numpy().view("uint16")
    routed = om.expert_ffn(xb, ids, weights, om.ExpertWeights(
        np_u8(ex.w13_weight), ex.w13_scale_inv.numpy(), np_u8(ex.w2_weight), ex.w2_scale_inv.numpy()))
    shared = om.dense_ffn(xb, np_u8(sh.w13_weight[0]), sh.w13_scale_inv[0].numpy(),
                          np_u8(sh.w2_weight[0]), sh.w2_scale_inv[0].numpy())
    expected = om.add_shared(routed, shared)
    got = out.view(torch.int16).cpu().numpy().view("uint16")
    return parity_stats(got, expected, 3e-3)


def bench_decode_config(torch, config: int, replays: int, working_set: float = 6e8) -> dict:
    """A decode configuration's step (config 1: 4 of 64 slots; config 3: all
    64 slots under Zipf-skewed routing; E16 H1024 I256) through DecodeStep:
    one graph holds one step per weight copy, enough copies that their bytes
    exceed the 256 MB MALL (cold), timed per replay; hot = the same graph on
    one copy.  Parity of the live rows against the numpy oracle.  Reported,
    not a roofline claim: at 12.6 MB of weights the step is launch-bound."""
    from drama3_amd import workloads
    from drama3_amd.expert_weights import prepare_experts
    from drama3_amd.pipeline import DecodeStep

    device = torch.device("cuda:0")
    w = workloads.CONFIGS[config]()
    step = w.steps[0]
    rows = int(step.occupancy.sum())
    first = w.experts.to(device)
    n_copies = max(4, int(working_set // sum(t.numel() * t.element_size() for t in first.tensors())))
    copies = [first] + [workloads.Experts(*(t.clone() for t in first.tensors()))
                        for _ in range(n_copies - 1)]
    for c in copies:
        prepare_experts(c)
    occ = step.occupancy.to(device)
    x, logits = step.x_slots.to(device), step.logits_slots.to(device)
    ds = DecodeStep(workloads.SLOTS, w.num_experts, w.hidden, w.intermediate, device=device)
    for c in copies:
        out = ds(occ, x, logits, c)
    torch.cuda.synchronize()
    parity = decode_parity(w, step, out[:rows])

    def graph_of(sequence):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for c in sequence:
                ds(occ, x, logits, c)
        return g

    cold = replay_stats(torch, graph_of(copies), replays, len(copies))
    hot = replay_stats(torch, graph_of([copies[0]] * len(copies)), replays, len(copies))
    used = int(torch.unique(ds.workspace.ids[:rows]).numel())
    nbytes = workloads.algorithmic_bytes(w, step, used)
    return {"workload": w.name, "active_rows": rows, "used_experts": used,
            "algorithmic_bytes_per_step": nbytes,
            "us_per_step": round(cold["median_us"], 2), "mean_us": round(cold["mean_us"], 2),
            "GB_s": round(nbytes / cold["median_us"] / 1e3, 1),
            "hot_us_per_step": round(hot["median_us"], 2),
            "tokens_per_s": round(rows / (cold["median_us"] * 1e-6), 1),
            "parity": parity,
            "timing": f"median of {replays} replays (after 10) of a graph of {len(copies)} steps, "
                      f"one per weight copy ({len(copies)} copies, more bytes than the 256 MB "
                      "MALL: cold); hot: the same graph on one copy"}


def bench_prefill(torch, steps: int, copies: int = 2, replays: int = 100,
                  check_parity: bool = True) -> dict:
    """Config 4: 16 packed prompts (~3.7k rows), routed top-8 FP8 MoE (H2048,
    E128, I768) plus a dense FP8 shared expert: route + quantise, wide route
    sort, tiled grouped FC1 (SwiGLU requant in its epilogue) and FC2 with the
    shared expert's rows as extra items of the same launches, weighted combine
    with the shared output added.  Graph-captured steps rotate over `copies`
    weight copies (1.2 GB > the 256 MB MALL)."""
    from drama3_amd import workloads
    from drama3_amd.expert_weights import prepare_experts
    from drama3_amd.pipeline import MoEWorkspace, Shape, moe_with_shared

    device = torch.device("cuda:0")
    w = workloads.config4()
    step = w.steps[0]
    x, logits = step.packed()
    rows = len(x)
    # the shared expert's rows ride in the routed launches (shared_rows)
    ws = MoEWorkspace(Shape(rows, w.num_experts, w.hidden, w.intermediate), device,
                      shared_rows=rows)
    sets = []
    for c in range(copies):
        routed, shared = w.experts.to(device), w.shared.to(device)
        sets.append((prepare_experts(routed), prepare_experts(shared)))
    xd, ld = x.to(device), logits.to(device)

    def full(routed, shared):
        return moe_with_shared(ws, None, xd, ld, routed, shared)

    def graph_us(fns, reps):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(reps):
                for fn in fns:
                    fn()
        g.replay()
        torch.cuda.synchronize()
        return time_graphs(torch, [g], max(1, steps // reps)) / (reps * len(fns))

    for routed, shared in sets:
        out = full(routed, shared)
    torch.cuda.synchronize()
    parity = prefill_parity(w, x, logits, out) if check_parity else None
    step_us = graph_us([lambda r=r, s=s: full(r, s) for r, s in sets], 2)

    def graph_of(pairs):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for routed, shared in pairs:
                full(routed, shared)
        return g

    cold = replay_stats(torch, graph_of(sets), replays, len(sets))
    hot = replay_stats(torch, graph_of([sets[0]] * len(sets)), replays, len(sets))
    stage_us = {
        "route_quantize": graph_us([lambda: ws.front(xd, ld)], 4),
        "sort": graph_us([ws.sort], 4),
        "fc1_swiglu": graph_us([lambda r=r, s=s: ws.grouped_fc1(r, s) for r, s in sets], 2),
        "fc2": graph_us([lambda r=r, s=s: ws.grouped_fc2(r, s) for r, s in sets], 2),
        "combine": graph_us([lambda: ws.combine(None, None, ws.shared_down)], 4),
    }
    stage_us["route_quantize"] -= stage_us["sort"]  # front() = route + quantise, then the sort
    used = int(torch.unique(ws.ids).numel())
    flop = workloads.flops(w, rows)
    nbytes = workloads.algorithmic_bytes(w, step, used)
    h, i = w.hidden, w.intermediate
    routes = rows * workloads.TOP_K + rows  # routed pairs + the shared expert's rows
    fc1_flop, fc2_flop = 2 * routes * 2 * i * h, 2 * routes * i * h
    tflops = flop / step_us / 1e6
    return {
        "workload": w.name, "rows": rows, "sequences": len(step.cu_seqlens) - 1,
        "us_per_step": round(step_us, 2), "tokens_per_s": round(rows / (step_us * 1e-6), 1),
        "median_us_per_step": round(cold["median_us"], 2),
        "hot_median_us_per_step": round(hot["median_us"], 2),
        "TFLOP_s": round(tflops, 1), "mfma_frac": round(tflops / FP8_PEAK_TFLOPS, 4),
        "GB_s": round(nbytes / step_us / 1e3, 1), "hbm_frac": round(nbytes / step_us / 1e3 / HBM_PEAK_GBS, 4),
        "flop_per_step": flop, "algorithmic_bytes_per_step": nbytes, "used_experts": used,
        "stage_us": {k: round(v, 2) for k, v in stage_us.items()},
        "fc1_TFLOP_s": round(fc1_flop / stage_us["fc1_swiglu"] / 1e6, 1),
        "fc2_TFLOP_s": round(fc2_flop / stage_us["fc2"] / 1e6, 1),
        "peak_TFLOP_s": FP8_PEAK_TFLOPS, "dtype": "fp8_e4m3 MFMA (fp32 accumulate)",
        "parity": parity,
        "timing": f"hipGraph, {copies} rotated weight copies (routed + shared, fragment-major)",
    }


def bench_reference_shape(torch, steps: int = 30, copies: int = 3) -> dict:
    """The decode step at the reference model's own MoE shape (H2048, 256
    experts, I512, top-8; `model.py:565-571`), all 64 slots live, seeded
    uniform synthetic routing, three rotated weight copies (cold)."""
    from drama3_amd import workloads
    from drama3_amd.expert_weights import prepare_experts
    from drama3_amd.pipeline import DecodeStep

    device = torch.device("cuda:0")
    e, h, i, slots = 256, 2048, 512, workloads.SLOTS
    gen = torch.Generator("cpu").manual_seed(7)
    first = workloads.make_experts(gen, e, h, i).to(device)
    sets = [first] + [workloads.Experts(*(t.clone() for t in first.tensors()))
                      for _ in range(copies - 1)]
    for c in sets:
        prepare_experts(c)
    occ = torch.ones(slots, dtype=torch.uint8, device=device)
    x = workloads._bf16(gen, (slots, h)).to(device)
    logits = workloads._bf16(gen, (slots, e)).to(device)
    ds = DecodeStep(slots, e, h, i, device=device)
    for c in sets:
        ds(occ, x, logits, c)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for c in sets:
            ds(occ, x, logits, c)
    g.replay()
    us = time_graphs(torch, [g], max(1, steps // copies)) / copies
    used = int(torch.unique(ds.workspace.ids[:slots]).numel())
    per_expert = 3 * h * i + 4 * ((2 * i // 128) * (h // 128) + (h // 128) * (i // 128))
    nbytes = used * per_expert + 4 * slots * h + 2 * slots * e + 6 * slots * workloads.TOP_K
    return {"workload": "decode, 64 live slots, H2048 E256 I512 top-8 (the reference model's MoE)",
            "us_per_step": round(us, 2), "used_experts": used, "algorithmic_bytes_per_step": nbytes,
            "GB_s": round(nbytes / us / 1e3, 1), "hbm_frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
            "step": ("FC1 from the slots + sortless FC2 + routed combine"
                     if ds.workspace.sortless and ds.uses_frontless(occ, x, logits)
                     else "front + route sort + expert GEMMs + combine"),
            "timing": f"hipGraph, {copies} rotated weight copies"}


def bench_moe_layer(torch, steps: int = 30, copies: int = 3) -> dict:
    """One whole MoE layer (``MoELayer``: packed bf16 input projection, routed
    top-8 FP8 experts, bf16 shared expert, combine) at the reference model's
    shape (64 rows, H2048, E256, I512, shared I512), shared expert on a side
    stream and in line; three rotated weight copies per graph (cold)."""
    from drama3_amd import workloads
    from drama3_amd.expert_weights import prepare_experts
    from drama3_amd.moe_layer import MoELayer, pack_input_projection

    device = torch.device("cuda:0")
    rows, e, h, i, si = 64, 256, 2048, 512, 512
    gen = torch.Generator("cpu").manual_seed(9)

    def bf16(*shape, scale):
        return (torch.randn(shape, generator=gen) * scale).to(torch.bfloat16).to(device)

    sets = []
    for _ in range(copies):
        experts = prepare_experts(workloads.make_experts(gen, e, h, i).to(device))
        projection = pack_input_projection(bf16(si, h, scale=h ** -0.5), bf16(si, h, scale=h ** -0.5),
                                           bf16(e, h, scale=h ** -0.5), bf16(1, h, scale=h ** -0.5))
        sets.append((experts, projection, bf16(h, si, scale=si ** -0.5)))
    x = workloads._bf16(gen, (rows, h)).to(device)
    out = {}
    for name, overlap in (("side_stream", True), ("in_line", False)):
        layer = MoELayer(rows, e, h, i, si, device=device, overlap=overlap)
        for experts, projection, down in sets:
            layer(x, projection, down, experts)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for experts, projection, down in sets:
                layer(x, projection, down, experts)
        g.replay()
        out[name] = round(time_graphs(torch, [g], max(1, steps // copies)) / copies, 2)
    return {"workload": "one MoE layer, 64 rows, H2048 E256 I512 top-8 + bf16 shared expert "
                        "(I512), packed input projection (the reference model's layer)",
            "us_per_layer": out,
            "step": "d3_dense_bf16 projection (SwiGLU activation in its epilogue) -> routed "
                    "FC1 / FC2 (decode step) || d3_dense_bf16 shared down projection -> "
                    "d3_combine_route_logits (routing weights, routed sum, gated shared add)",
            "timing": f"hipGraph, {copies} rotated weight copies"}


def mixed_parity(step, workload, kept: int) -> dict:
    """The MoE rows of a replayed config-5 mixed step (the kept rows, after
    prefix reuse) against the numpy oracle: the routed combine of the
    step's own per-route rows, FP8-MFMA contraction path (RRMS < 3e-3)."""
    import torch

    from oracle import moe as om

    routed = step.workspace.combine(None, step.rows.keep_count, None, step.routed)
    torch.cuda.synchronize()
    rows = step.rows.keep.cpu().numpy()[:kept]
    x = step.x.view(torch.int16).cpu().numpy().view("uint16")[rows]
    weights, ids = om.route(step.logits.float().cpu().numpy()[rows])
    ex = workload.experts
    expected = om.expert_ffn(x, ids, weights, om.ExpertWeights(
        ex.w13_weight.view(torch.uint8).numpy(), ex.w13_scale_inv.numpy(),
        ex.w2_weight.view(torch.uint8).numpy(), ex.w2_scale_inv.numpy()))
    got = routed[:kept].view(torch.int16).cpu().numpy().view("uint16")
    return {**parity_stats(got, expected, 3e-3), "rows": kept}


def bench_moe_layer_prefill(torch, rows: int = 4096, steps: int = 20, copies: int = 2) -> dict:
    """``MoELayer`` at a prefill-sized batch (4096 packed rows) of the
    reference model's shape (H2048, E256, I512, shared I512): the tiled bf16
    projection (SwiGLU in its epilogue) and shared down projection on
    d3_dense_bf16, the routed experts on the prefill path (wide route sort,
    tiled grouped FP8 GEMMs), the combine; two rotated weight copies.  The
    two bf16 GEMMs are also timed alone, and next to them the same products
    through torch.mm (hipBLASLt) for context."""
    from drama3_amd import workloads
    from drama3_amd.expert_weights import prepare_experts
    from drama3_amd.moe_layer import MoELayer, dense_bf16, pack_input_projection

    device = torch.device("cuda:0")
    e, h, i, si = 256, 2048, 512, 512
    gen = torch.Generator("cpu").manual_seed(13)

    def bf16(*shape, scale):
        return (torch.randn(shape, generator=gen) * scale).to(torch.bfloat16).to(device)

    sets = []
    for _ in range(copies):
        experts = prepare_experts(workloads.make_experts(gen, e, h, i).to(device))
        projection = pack_input_projection(bf16(si, h, scale=h ** -0.5), bf16(si, h, scale=h ** -0.5),
                                           bf16(e, h, scale=1.0), bf16(1, h, scale=h ** -0.5))
        sets.append((experts, projection, bf16(h, si, scale=si ** -0.5)))
    x = workloads._bf16(gen, (rows, h)).to(device)
    layer = MoELayer(rows, e, h, i, si, device=device)
    for experts, projection, down in sets:
        layer(x, projection, down, experts)
    torch.cuda.synchronize()

    def graph_us(fn, reps):
        for experts, projection, down in sets:  # eager first (library set-up outside capture)
            fn(experts, projection, down)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(reps):
                for experts, projection, down in sets:
                    fn(experts, projection, down)
        g.replay()
        torch.cuda.synchronize()
        return time_graphs(torch, [g], max(1, steps // reps)) / (reps * len(sets))

    layer_us = graph_us(lambda ex, pr, dn: layer(x, pr, dn, ex), 1)
    out = torch.empty_like(layer.projected)
    act = torch.empty_like(layer.act)
    shared = torch.empty_like(layer.shared)
    proj_us = graph_us(lambda ex, pr, dn: dense_bf16(x, pr, out, si, act), 4)
    down_us = graph_us(lambda ex, pr, dn: dense_bf16(act, dn, shared), 4)
    lib_proj_us = graph_us(lambda ex, pr, dn: torch.mm(x, pr.t(), out=out), 4)
    lib_down_us = graph_us(lambda ex, pr, dn: torch.mm(act, dn.t(), out=shared), 4)
    n_proj = layer.projected.shape[1]
    proj_flop, down_flop = 2 * rows * n_proj * h, 2 * rows * h * si
    return {"workload": f"one MoE layer, {rows} packed rows, H2048 E256 I512 top-8 + bf16 shared "
                        "expert (I512), packed input projection (the reference model's layer)",
            "rows": rows, "us_per_layer": round(layer_us, 2),
            "tokens_per_s": round(rows / (layer_us * 1e-6), 1),
            "projection_us": round(proj_us, 2),
            "projection_TFLOP_s": round(proj_flop / proj_us / 1e6, 1),
            "shared_down_us": round(down_us, 2),
            "shared_down_TFLOP_s": round(down_flop / down_us / 1e6, 1),
            "hipblaslt_projection_us": round(lib_proj_us, 2),
            "hipblaslt_shared_down_us": round(lib_down_us, 2),
            "peak_bf16_TFLOP_s": 2500.0,
            "step": "d3_dense_bf16 tiled projection (SwiGLU in its epilogue) -> front + wide route "
                    "sort + tiled grouped FP8 FC1 / FC2 -> d3_dense_bf16 shared down projection "
                    "-> routed combine + combine_experts",
            "timing": f"hipGraph, {copies} rotated weight copies; the GEMMs alone: graphs of 4 "
                      "launches per copy; hipblaslt_*: torch.mm of the same operands, context only"}


def bench_mixed(torch, steps: int = 50, check_parity: bool = True) -> dict:
    """Config 5's mixed step as one captured graph (``MixedStep``): 48 live
    decode slots of 64 (decode bucket 64), two 256-row prompts in a 640-row
    prefill suffix (128 padding rows), E16 H1024 I256 top-8.  Timed twice:
    distinct prompts, and the second prompt sharing its first 128 rows with
    the first (prefix reuse folds them)."""
    from drama3_amd import workloads
    from drama3_amd.mixed import MixedStep

    device = torch.device("cuda:0")
    w = workloads.config5()
    experts = w.experts.to(device)
    slots, d, capacity = workloads.SLOTS, 64, 640
    step = MixedStep(slots, d, capacity, slots // 2, 3, w.num_experts, w.hidden, w.intermediate,
                     device=device)
    gen = torch.Generator("cpu").manual_seed(5)
    full = step.rows.full
    step.occupancy.copy_(w.steps[0].occupancy)
    step.boundaries.copy_(torch.tensor([0, 256, 512, capacity], dtype=torch.int32))
    step.sequence_slots.copy_(torch.tensor([40, 41, slots - 1]))
    step.x.copy_(workloads._bf16(gen, (full, w.hidden)))
    step.logits.copy_(workloads._bf16(gen, (full, w.num_experts)))
    step.shared.copy_(workloads._bf16(gen, (full, w.hidden)))
    step.gate.copy_(workloads._bf16(gen, (full,)))
    step.norm_weight.copy_(workloads._bf16(gen, (w.hidden,)))
    residual = workloads._bf16(gen, (full, w.hidden)).to(device)
    frames = torch.randint(0, 1024, (capacity, 11), generator=gen)
    step.frames.copy_(frames)
    step.residual.copy_(residual)
    step.capture(experts)
    out = {}
    parity = None
    for name, shared_rows in (("distinct_prompts", 0), ("shared_prefix_128", 128)):
        f = frames.clone()
        f[256:256 + shared_rows] = f[:shared_rows]
        step.frames.copy_(f)
        step.replay()
        torch.cuda.synchronize()
        kept = int(step.rows.keep_count.item())
        if name == "distinct_prompts" and check_parity:
            parity = mixed_parity(step, w, kept)
        us = time_graphs(torch, [step.graph], steps)
        stats = replay_stats(torch, step.graph, max(steps, 100))
        out[name] = {"us_per_step": round(us, 2), "median_us_per_step": round(stats["median_us"], 2),
                     "moe_rows": kept, "tokens_per_s": round((48 + 512) / (us * 1e-6), 1)}
    return {"workload": "config 5 mixed step: 48 of 64 decode slots + 2 x 256 prompt rows "
                        "(640-row suffix), E16 H1024 I256 top-8",
            "rows": full, "live_rows": 48 + 512, **out, "parity": parity,
            "step": "d3_mixed_rows (with the suffix's row metadata) + MoE on the kept rows, "
                    "then the routed combine + residual + RMSNorm onto all rows in one launch; "
                    "one hipGraph",
            "timing": "graph replays; the residual is updated in place on every replay"}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU; multi-GPU (expert "
                          "parallel) is a design note only", "n_gpus": args.gpus}))
        sys.exit(2)
    import numpy as np
    import torch

    from drama3_amd import workloads
    from drama3_amd.expert_weights import prepare_experts
    from drama3_amd.pipeline import DecodeStep

    if args.prefill_only:
        print(json.dumps({"prefill": bench_prefill(torch, args.prefill_steps, replays=args.replays,
                                                   check_parity=not args.no_parity)}),
              flush=True)
        return
    if args.decode_config_only is not None:
        print(json.dumps({"decode_config": bench_decode_config(torch, args.decode_config_only,
                                                               args.replays)}), flush=True)
        return
    if args.reference_shape_only:
        print(json.dumps({"reference_shape": bench_reference_shape(torch)}), flush=True)
        return
    if args.layer_only:
        layer = bench_moe_layer(torch)
        layer["prefill_4096_rows"] = bench_moe_layer_prefill(torch)
        print(json.dumps({"moe_layer": layer}), flush=True)
        return
    if args.mixed_only:
        print(json.dumps({"mixed": bench_mixed(torch, args.mixed_steps,
                                               check_parity=not args.no_parity)}), flush=True)
        return

    device = torch.device("cuda:0")
    w = workloads.config2()
    step = w.steps[0]
    rows = int(step.occupancy.sum())
    experts0 = w.experts.to(device)
    copies = [experts0] + [workloads.Experts(*(t.clone() for t in experts0.tensors()))
                           for _ in range(max(0, args.copies - 1))]
    # Load-time re-layout of the fp8 codes (fragment-major), as a deployment
    # would do once per layer; the step then streams only the packed copy.
    for c in copies:
        prepare_experts(c)
    occ = step.occupancy.to(device)
    x_slots, logits_slots = step.x_slots.to(device), step.logits_slots.to(device)
    ds = DecodeStep(workloads.SLOTS, w.num_experts, w.hidden, w.intermediate, device=device)

    # eager warm-up run, then one graph per weight copy
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for c in copies:
            ds(occ, x_slots, logits_slots, c)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    # One graph holds one step per weight copy, back to back: the copies play
    # the layers of a model whose decode step is captured whole, so the MoE
    # steps of consecutive layers follow each other inside one graph (no
    # per-step graph launch).  A second graph with the first K mod copies
    # steps makes the timed region exactly K steps.  `hot` runs the same
    # graphs on a single copy (weights resident in the 256 MB MALL).
    def step_graph(sequence):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for c in sequence:
                result = ds(occ, x_slots, logits_slots, c)
        return g, result

    def time_steps(sequence, steps):
        if steps <= 0:
            return 0.0, None
        full, result = step_graph(sequence)
        rest = step_graph(sequence[:steps % len(sequence)])[0] if steps % len(sequence) else None
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for _ in range(steps // len(sequence)):
            full.replay()
        if rest is not None:
            rest.replay()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) * 1000.0 / steps, result

    ws = ds.workspace
    time_steps(copies, args.warmup)
    step_us, out = time_steps(copies, args.steps)
    hot_us, _ = time_steps([copies[0]] * len(copies), args.steps)
    # BASELINE protocol next to the exact-K mean: >= 100 replays of the
    # one-step-per-copy graph after >= 10 warm-up replays, each timed alone.
    cold_replays = replay_stats(torch, step_graph(copies)[0], args.replays, len(copies))
    hot_replays = replay_stats(torch, step_graph([copies[0]] * len(copies))[0], args.replays,
                               len(copies))
    used = int(torch.unique(ws.ids[:rows]).numel())  # experts with at least one route
    step_bytes = workloads.algorithmic_bytes(w, step, used)

    # Dominant kernel (FC1, 2/3 of the weight bytes) and FC2, timed alone:
    # graphs of back-to-back launches over the rotated weight copies.
    def kernel_graph(fn):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(args.kernel_reps):
                for c in copies:
                    fn(c)
        return g

    frontless = ws.sortless and ds.uses_frontless(occ, x_slots, logits_slots)
    if frontless:  # the step's own expert kernels: FC1 from the slots, sortless FC2
        fc1_graph = kernel_graph(lambda c: ws.decode_route_fc1(c, occ, x_slots, logits_slots,
                                                               ds.active, ds.count))
        fc2_graph = kernel_graph(lambda c: ws.decode_fc2(c, ds.count, row_slots=ds.active))
    elif ws.sortless:  # sortless decode GEMMs after the front
        fc1_graph = kernel_graph(lambda c: ws.decode_fc1(c, ds.count))
        fc2_graph = kernel_graph(lambda c: ws.decode_fc2(c, ds.count))
    else:
        fc1_graph = kernel_graph(ws.fc1)
        fc2_graph = kernel_graph(ws.fc2_swiglu if ws.swiglu_in_fc2 else ws.fc2)
    launches = args.kernel_reps * len(copies)
    time_graphs(torch, [fc1_graph, fc2_graph], 2)  # warm-up
    fc1_us = time_graphs(torch, [fc1_graph], 5) / launches
    fc2_us = time_graphs(torch, [fc2_graph], 5) / launches
    h, i, e = w.hidden, w.intermediate, w.num_experts
    routes = rows * workloads.TOP_K
    fc1_weights = used * (2 * i * h + 4 * (2 * i // 128) * (h // 128))
    if frontless:  # bf16 x rows, the slots' logits and occupancy in; gate_up, ids, slot list out
        slots = workloads.SLOTS
        fc1_bytes = fc1_weights + rows * h * 2 + slots * e * 2 + slots + routes * 2 * i * 2 \
            + routes * 4 + slots * 4
    else:  # fp8 q rows + scales in, gate_up out
        fc1_bytes = fc1_weights + rows * h + rows * (h // 128) * 4 + routes * 2 * i * 2
    # FC2 reads its activations as fp8 codes + scales, or (SwiGLU in its
    # prologue) as FC1's bf16 gate|up rows.
    prologue = ws.sortless or ws.swiglu_in_fc2
    act_bytes = routes * 2 * i * 2 if prologue else routes * i + routes * (i // 128) * 4
    fc2_bytes = used * (h * i + 4 * (h // 128) * (i // 128)) + act_bytes + routes * h * 4
    # Practical streaming rate of this GPU for context: a large device copy
    # (torch), counting bytes read plus bytes written.
    src = torch.empty(1 << 30, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    copy_graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(copy_graph):
        dst.copy_(src)
    time_graphs(torch, [copy_graph], 2)
    copy_gbs = 2 * src.numel() / time_graphs(torch, [copy_graph], 5) / 1e3
    del src, dst
    fc1_gbs = fc1_bytes / fc1_us / 1e3
    fc2_gbs = fc2_bytes / fc2_us / 1e3
    step_gbs = step_bytes / step_us / 1e3

    parity = None if args.no_parity else decode_parity(w, step, out[:rows])
    decode_configs = None if args.no_decode_configs else {
        name: bench_decode_config(torch, c, args.replays) for name, c in (("c1", 1), ("c3", 3))}
    cpu = None
    if not args.no_cpu_baseline:
        sample = {f"c{c}": (lambda wl_: (wl_, wl_.steps[0]))(w if c == 2 else workloads.CONFIGS[c]())
                  for c in (1, 2, 3, 4, 5)}
        base = cpu_baseline(sample, args.cpu_runs)
        c2 = base["configs"]["c2"]
        cpu = {"value": round(step_bytes / c2["us_per_step"] / 1e3, 3), "unit": "GB/s",
               "cores": base["threads"], "kind": "port", "us_per_step": c2["us_per_step"],
               "sample": (f"config 2's full decode step ({rows} live rows) through the PyTorch-CPU "
                          f"restatement of the step (oracle/cpu_step.py: routing, quantisation, "
                          f"per-expert dequantise + FP32 FC1 / SwiGLU / FC2, combine) on "
                          f"{base['threads']} torch threads; median of {args.cpu_runs} runs after "
                          f"2 warm-ups; `configs` holds every configuration timed the same way"),
               **base}

    prefill = None if args.no_prefill else bench_prefill(torch, args.prefill_steps,
                                                         replays=args.replays,
                                                         check_parity=not args.no_parity)
    reference_shape = None if args.no_reference_shape else bench_reference_shape(torch)
    mixed = None if args.no_mixed else bench_mixed(torch, args.mixed_steps,
                                                   check_parity=not args.no_parity)
    moe_layer = None if args.no_reference_shape else bench_moe_layer(torch)
    if moe_layer is not None and not args.no_prefill:
        moe_layer["prefill_4096_rows"] = bench_moe_layer_prefill(torch)

    result = {
        "metric": baseline_metric(),
        "value": round(step_gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_us / 1000.0, 5),
        "us_per_step": round(step_us, 2),
        "pct_of_hbm_peak": round(100.0 * step_gbs / HBM_PEAK_GBS, 1),
        "tokens_per_s": round(rows / (step_us * 1e-6), 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3 (fp32 accumulate, bf16 activations)",
        "data": "synthetic",
        "config": {"workload": w.name, "slots": workloads.SLOTS, "active_rows": rows,
                   "experts": e, "hidden": h, "intermediate": i, "top_k": workloads.TOP_K,
                   "used_experts": used, "algorithmic_bytes_per_step": step_bytes,
                   "weight_copies": len(copies),
                   "step": ("FC1 routing + quantising the slots itself, sortless FC2, routed "
                            "combine (3 launches)" if frontless else
                            "front + sortless decode GEMMs + combine" if ws.sortless else
                            "front + sorted expert GEMMs + combine"),
                   "timing": "hipGraph of one step per weight copy (the copies act as consecutive "
                             "layers), replayed; cold: every step streams its copy from HBM"},
        "hot": {"us_per_step": round(hot_us, 2),
                "GB_s": round(step_bytes / hot_us / 1e3, 1)},
        "per_replay": {"cold": {k: round(v, 2) if isinstance(v, float) else v
                                for k, v in cold_replays.items()},
                       "hot": {k: round(v, 2) if isinstance(v, float) else v
                               for k, v in hot_replays.items()},
                       "cold_median_GB_s": round(step_bytes / cold_replays["median_us"] / 1e3, 1),
                       "cold_median_pct_of_hbm_peak": round(
                           100.0 * step_bytes / cold_replays["median_us"] / 1e3 / HBM_PEAK_GBS, 1)},
        "roofline": {"bound": "hbm",
                     "kernel": ("decode_route_fc1" if frontless else
                                "decode_expert_gemm FC1" if ws.sortless else "expert_gemm FC1"),
                     "achieved": round(fc1_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(fc1_gbs / HBM_PEAK_GBS, 4),
                     "traffic": FC1_TRAFFIC_BYTES["bytes"],
                     "traffic_kernel": FC1_TRAFFIC_BYTES["kernel"],
                     "traffic_measured_on": FC1_TRAFFIC_BYTES["measured_on"],
                     "us_per_launch": round(fc1_us, 2),
                     "algorithmic_bytes_per_launch": fc1_bytes},
        "fc2": {"kernel": ("decode_expert_gemm FC2 (SwiGLU prologue)" if ws.sortless else
                           "expert_fc2_swiglu" if ws.swiglu_in_fc2 else "expert_gemm FC2"),
                "us_per_launch": round(fc2_us, 2), "GB_s": round(fc2_gbs, 1),
                "algorithmic_bytes_per_launch": fc2_bytes},
        "device_copy_GB_s": round(copy_gbs, 1),
        "cpu_baseline": cpu,
        "parity": parity,
        "decode_configs": decode_configs,
        "prefill": prefill,
        "reference_shape": reference_shape,
        "mixed": mixed,
        "moe_layer": moe_layer,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
