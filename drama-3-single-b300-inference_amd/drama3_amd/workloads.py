"""Seeded synthetic inputs for the five measured configurations.

Everything is drawn from ``torch.Generator('cpu').manual_seed(seed)`` in a
fixed order, so the same seed gives the same bytes on every machine:

1. occupancy / sequence lengths,
2. expert weights: per expert ``w13`` then ``w2`` as e4m3 from N(0,1) (round to
   nearest even through torch's ``float8_e4m3fn`` cast), block scales
   ``exp(0.5 * N(0,1))`` (lognormal(0, 0.5)),
3. the optional shared expert (config 4), same recipe,
4. activations N(0,1) -> bf16, router logits N(0,1) (+ bias) -> bf16.

Weight layout follows the reference (``kernels.py:290-318``):
``w13 [E, 2I, H]`` rows [gate; up], ``w13_scale_inv [E, 2I/128, H/128]``,
``w2 [E, H, I]``, ``w2_scale_inv [E, H/128, I/128]``.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

SLOTS = 64
TOP_K = 8


@dataclass
class Experts:
    """Any object exposing these four attributes is accepted by the MoE ops
    (the reference's ``layer.experts`` contract, ``kernels.py:334-351``)."""

    w13_weight: torch.Tensor
    w13_scale_inv: torch.Tensor
    w2_weight: torch.Tensor
    w2_scale_inv: torch.Tensor

    def to(self, device) -> "Experts":
        return Experts(*(t.to(device) for t in self.tensors()))

    def tensors(self):
        return (self.w13_weight, self.w13_scale_inv, self.w2_weight, self.w2_scale_inv)

    @property
    def num_experts(self) -> int:
        return self.w13_weight.shape[0]

    @property
    def hidden(self) -> int:
        return self.w13_weight.shape[2]

    @property
    def intermediate(self) -> int:
        return self.w13_weight.shape[1] // 2

    def nbytes_per_expert(self) -> int:
        return sum(t[0].numel() * t.element_size() for t in self.tensors())


@dataclass
class Step:
    """One step of a ragged batch: MoE rows plus where they came from."""

    occupancy: torch.Tensor | None  # uint8 [SLOTS] (decode part) or None
    x_slots: torch.Tensor | None  # bf16 [SLOTS, H]: per-slot hidden rows
    logits_slots: torch.Tensor | None  # bf16 [SLOTS, E]
    prefill_x: torch.Tensor | None  # bf16 [P, H]: packed prefill rows
    prefill_logits: torch.Tensor | None  # bf16 [P, E]
    cu_seqlens: torch.Tensor | None  # int32 [n+1] of the prefill suffix

    def active_slots(self) -> torch.Tensor:
        return torch.nonzero(self.occupancy, as_tuple=False).flatten().to(torch.int32)

    def packed(self):
        """(x [T,H], logits [T,E]) in packing order: decode rows (ascending
        slot) first, then the packed prefill suffix."""
        xs, ls = [], []
        if self.occupancy is not None:
            active = self.active_slots().long()
            xs.append(self.x_slots[active])
            ls.append(self.logits_slots[active])
        if self.prefill_x is not None:
            xs.append(self.prefill_x)
            ls.append(self.prefill_logits)
        return torch.cat(xs), torch.cat(ls)


@dataclass
class Workload:
    name: str
    seed: int
    hidden: int
    num_experts: int
    intermediate: int
    experts: Experts
    steps: list[Step]
    shared: Experts | None = None  # config 4: dense FP8 SwiGLU added to the routed output
    description: str = ""
    extra: dict = field(default_factory=dict)


def _fp8(gen: torch.Generator, shape) -> torch.Tensor:
    return torch.randn(shape, generator=gen, dtype=torch.float32).to(torch.float8_e4m3fn)


def _scales(gen: torch.Generator, shape) -> torch.Tensor:
    return torch.exp(0.5 * torch.randn(shape, generator=gen, dtype=torch.float32))


def make_experts(gen: torch.Generator, experts: int, hidden: int, intermediate: int) -> Experts:
    if hidden % 128 or intermediate % 128:
        raise ValueError("hidden and intermediate sizes must be multiples of 128")
    w13 = torch.empty((experts, 2 * intermediate, hidden), dtype=torch.float8_e4m3fn)
    w2 = torch.empty((experts, hidden, intermediate), dtype=torch.float8_e4m3fn)
    for e in range(experts):  # per expert keeps the fp32 temporary small
        w13[e] = _fp8(gen, (2 * intermediate, hidden))
        w2[e] = _fp8(gen, (hidden, intermediate))
    s13 = _scales(gen, (experts, 2 * intermediate // 128, hidden // 128))
    s2 = _scales(gen, (experts, hidden // 128, intermediate // 128))
    return Experts(w13, s13, w2, s2)


def _bf16(gen, shape) -> torch.Tensor:
    return torch.randn(shape, generator=gen, dtype=torch.float32).to(torch.bfloat16)


def zipf_bias(gen: torch.Generator, experts: int, s: float = 1.2) -> torch.Tensor:
    """Per-expert logit bias ``3 * log(p_e)``, ``p_e`` the Zipf(s) pmf of the
    expert's rank under a seeded permutation (rank 1 = most popular)."""
    ranks = torch.randperm(experts, generator=gen).to(torch.float64) + 1.0
    pmf = ranks.pow(-s)
    pmf = pmf / pmf.sum()
    return (3.0 * pmf.log()).to(torch.float32)


def config1(seed: int = 0) -> Workload:
    """CPU-sized decode: 64 slots, active {3,17,40,62}; H=1024, E=16, I=256."""
    gen = torch.Generator("cpu").manual_seed(seed)
    occupancy = torch.zeros(SLOTS, dtype=torch.uint8)
    occupancy[[3, 17, 40, 62]] = 1
    experts = make_experts(gen, 16, 1024, 256)
    x = _bf16(gen, (SLOTS, 1024))
    logits = _bf16(gen, (SLOTS, 16))
    step = Step(occupancy, x, logits, None, None, None)
    return Workload("c1_tiny_decode", seed, 1024, 16, 256, experts, [step],
                    description="64 slots, 4 active at {3,17,40,62}, H1024 E16 I256 top-8")


def config2(seed: int = 2) -> Workload:
    """Drama-3-scale decode: Bernoulli(0.75) occupancy; H=2048, E=128, I=768."""
    gen = torch.Generator("cpu").manual_seed(seed)
    occupancy = (torch.rand(SLOTS, generator=gen) < 0.75).to(torch.uint8)
    experts = make_experts(gen, 128, 2048, 768)
    x = _bf16(gen, (SLOTS, 2048))
    logits = _bf16(gen, (SLOTS, 128))
    step = Step(occupancy, x, logits, None, None, None)
    return Workload("c2_decode_h2048_e128", seed, 2048, 128, 768, experts, [step],
                    description="64 slots, Bernoulli(0.75) occupancy, H2048 E128 I768 top-8")


def config3(seed: int = 3) -> Workload:
    """Skewed decode: all 64 slots active, Zipf(1.2) expert bias; c1 shapes."""
    gen = torch.Generator("cpu").manual_seed(seed)
    occupancy = torch.ones(SLOTS, dtype=torch.uint8)
    experts = make_experts(gen, 16, 1024, 256)
    bias = zipf_bias(gen, 16)
    x = _bf16(gen, (SLOTS, 1024))
    logits = (torch.randn((SLOTS, 16), generator=gen) + bias).to(torch.bfloat16)
    step = Step(occupancy, x, logits, None, None, None)
    return Workload("c3_skewed_decode", seed, 1024, 16, 256, experts, [step],
                    description="64 active slots, logits N(0,1) + 3 log Zipf(1.2) pmf",
                    extra={"bias": bias})


def config4(seed: int = 4, sequences: int = 16) -> Workload:
    """Packed ragged prefill: 16 lengths U{8..512}; c2 MoE plus a shared FP8 expert."""
    gen = torch.Generator("cpu").manual_seed(seed)
    lengths = torch.randint(8, 513, (sequences,), generator=gen)
    cu = torch.cat([torch.zeros(1, dtype=torch.int64), lengths.cumsum(0)]).to(torch.int32)
    experts = make_experts(gen, 128, 2048, 768)
    shared = make_experts(gen, 1, 2048, 768)
    rows = int(cu[-1])
    x = _bf16(gen, (rows, 2048))
    logits = _bf16(gen, (rows, 128))
    step = Step(None, None, None, x, logits, cu)
    return Workload("c4_packed_prefill", seed, 2048, 128, 768, experts, [step], shared=shared,
                    description=f"{sequences} packed prompts, {rows} rows, + shared FP8 expert")


def config5(seed: int = 5, steps: int = 4, decode: int = 48, chunk: int = 256, chunks: int = 2,
            churn: int = 4) -> Workload:
    """Mixed continuous batching: per step 48 decode slots + 2 x 256 prefill
    rows; between steps 4 slots retire and 4 are admitted (seeded)."""
    gen = torch.Generator("cpu").manual_seed(seed)
    experts = make_experts(gen, 16, 1024, 256)
    perm = torch.randperm(SLOTS, generator=gen)
    occupancy = torch.zeros(SLOTS, dtype=torch.uint8)
    occupancy[perm[:decode]] = 1
    cu = torch.arange(chunks + 1, dtype=torch.int32) * chunk
    out = []
    for _ in range(steps):
        x = _bf16(gen, (SLOTS, 1024))
        logits = _bf16(gen, (SLOTS, 16))
        px = _bf16(gen, (chunk * chunks, 1024))
        pl = _bf16(gen, (chunk * chunks, 16))
        out.append(Step(occupancy.clone(), x, logits, px, pl, cu.clone()))
        active = torch.nonzero(occupancy).flatten()
        free = torch.nonzero(occupancy == 0).flatten()
        retire = active[torch.randperm(active.numel(), generator=gen)[:churn]]
        admit = free[torch.randperm(free.numel(), generator=gen)[:churn]]
        occupancy[retire] = 0
        occupancy[admit] = 1
    return Workload("c5_mixed_batching", seed, 1024, 16, 256, experts, out,
                    description=f"{steps} steps x ({decode} decode + {chunks}x{chunk} prefill)")


CONFIGS = {1: config1, 2: config2, 3: config3, 4: config4, 5: config5}


def algorithmic_bytes(workload: Workload, step: Step, used_experts: int) -> int:
    """HBM bytes one MoE step must move at minimum.

    U = experts with at least one route in the realised routing; per expert
    FP8 weights 3*H*I plus f32 block scales; x in and out (bf16), bf16
    logits, and K ids (i32) + weights (bf16) per row.  Intermediates are
    excluded.  The shared expert (config 4) adds its weights once.
    """
    h, e, i = workload.hidden, workload.num_experts, workload.intermediate
    per_expert = 3 * h * i + 4 * ((2 * i // 128) * (h // 128) + (h // 128) * (i // 128))
    x, _ = step.packed()
    t = x.shape[0]
    total = used_experts * per_expert + 4 * t * h + 2 * t * e + 6 * t * TOP_K
    if workload.shared is not None:
        total += per_expert
    return total


def flops(workload: Workload, rows: int) -> int:
    """Dense-equivalent FLOPs of the routed (and shared) expert GEMMs."""
    h, i = workload.hidden, workload.intermediate
    total = 2 * rows * TOP_K * 3 * h * i
    if workload.shared is not None:
        total += 2 * rows * 3 * h * i
    return total

