"""Expert weights of one MoE layer from a Drama-3 safetensors checkpoint.

The reference loads its checkpoint through Fish Speech's ``FishOmniModel``
(``src/drama3/model.py:182-187``), whose experts expose ``w13_weight``
``[E, 2I, H]`` with rows ``[gate; up]`` ("the checkpoint stores
[gate | up]", ``model.py:196``), ``w13_scale_inv`` ``[E, 2I/128, H/128]``,
``w2_weight`` ``[E, H, I]`` and ``w2_scale_inv`` ``[E, H/128, I/128]``.  The
checkpoint itself stores one tensor per expert and projection under
``model.language_model.layers.{layer}.mlp.experts.{e}.{gate,up,down}_proj.
{weight,weight_scale_inv}``, sharded through ``model.safetensors.index.json``
(the key scheme the reference's own validation scripts read,
``evidence/20261016-ceiling/results/expert-resident-chain-v2/validation_contract.py.gz:83-99``).
This module reads those tensors with safetensors (no pickle, nothing
executed from the files) and stacks them into the layout above, the layout
every MoE operator of this package takes.
"""

from __future__ import annotations

import json
import re
from contextlib import ExitStack
from pathlib import Path

import torch

from .workloads import Experts

LAYER_PREFIX = "model.language_model.layers.{layer}.mlp"


def _weight_map(checkpoint: Path) -> dict[str, str]:
    """key -> shard file name (single-file checkpoints map every key to it)."""
    index = checkpoint / "model.safetensors.index.json"
    if index.exists():
        return json.loads(index.read_text())["weight_map"]
    single = checkpoint / "model.safetensors"
    if not single.exists():
        raise FileNotFoundError(f"{checkpoint} has neither model.safetensors.index.json nor "
                                "model.safetensors")
    from safetensors import safe_open

    with safe_open(str(single), framework="pt", device="cpu") as reader:
        return {key: single.name for key in reader.keys()}


class _Reader:
    def __init__(self, checkpoint: Path, weight_map: dict[str, str], stack: ExitStack):
        from safetensors import safe_open

        self._map = weight_map
        self._open = {}
        self._root = checkpoint
        self._stack = stack
        self._safe_open = safe_open

    def get(self, key: str) -> torch.Tensor:
        if key not in self._map:
            raise KeyError(f"checkpoint has no tensor {key}")
        name = self._map[key]
        if name not in self._open:
            self._open[name] = self._stack.enter_context(
                self._safe_open(str(self._root / name), framework="pt", device="cpu"))
        return self._open[name].get_tensor(key)


def expert_count(weight_map: dict[str, str], layer: int) -> int:
    prefix = re.escape(LAYER_PREFIX.format(layer=layer) + ".experts.")
    ids = {int(m.group(1)) for key in weight_map
           if (m := re.match(prefix + r"(\d+)\.", key))}
    if not ids:
        raise KeyError(f"no routed experts for layer {layer}")
    if ids != set(range(len(ids))):
        raise ValueError(f"layer {layer} experts are not numbered 0..{len(ids) - 1}")
    return len(ids)


def load_layer_experts(checkpoint: str | Path, layer: int, device="cpu") -> Experts:
    """Routed experts of ``layer`` as ``Experts`` (``w13`` rows [gate; up])."""
    checkpoint = Path(checkpoint)
    weight_map = _weight_map(checkpoint)
    count = expert_count(weight_map, layer)
    prefix = LAYER_PREFIX.format(layer=layer) + ".experts"
    w13, s13, w2, s2 = [], [], [], []
    with ExitStack() as stack:
        reader = _Reader(checkpoint, weight_map, stack)
        for e in range(count):
            def tensor(proj, suffix, e=e):
                return reader.get(f"{prefix}.{e}.{proj}.{suffix}")
            gate, up = tensor("gate_proj", "weight"), tensor("up_proj", "weight")
            gate_s, up_s = tensor("gate_proj", "weight_scale_inv"), tensor("up_proj", "weight_scale_inv")
            down, down_s = tensor("down_proj", "weight"), tensor("down_proj", "weight_scale_inv")
            _check_expert(e, gate, up, down, gate_s, up_s, down_s)
            w13.append(torch.cat((gate, up), dim=0))
            s13.append(torch.cat((gate_s, up_s), dim=0).float())
            w2.append(down)
            s2.append(down_s.float())
    experts = Experts(torch.stack(w13), torch.stack(s13), torch.stack(w2), torch.stack(s2))
    return experts.to(device) if str(device) != "cpu" else experts


def load_shared_expert(checkpoint: str | Path, layer: int) -> dict[str, torch.Tensor]:
    """The layer's shared expert projections (``mlp.shared_expert.{gate,up,
    down}_proj.weight``, bf16 in the reference, ``model.py:232-233,512``) and,
    when present, its gate (``mlp.shared_expert_gate.weight``)."""
    checkpoint = Path(checkpoint)
    weight_map = _weight_map(checkpoint)
    prefix = LAYER_PREFIX.format(layer=layer)
    out = {}
    with ExitStack() as stack:
        reader = _Reader(checkpoint, weight_map, stack)
        for proj in ("gate_proj", "up_proj", "down_proj"):
            out[proj] = reader.get(f"{prefix}.shared_expert.{proj}.weight")
        gate_key = f"{prefix}.shared_expert_gate.weight"
        if gate_key in weight_map:
            out["gate"] = reader.get(gate_key)
    return out


def _check_expert(e, gate, up, down, gate_s, up_s, down_s) -> None:
    fp8 = torch.float8_e4m3fn
    if gate.dtype != fp8 or up.dtype != fp8 or down.dtype != fp8:
        raise TypeError(f"expert {e}: projections must be float8_e4m3fn")
    i, h = gate.shape
    if up.shape != (i, h) or down.shape != (h, i) or h % 128 or i % 128:
        raise ValueError(f"expert {e}: gate/up [I, H], down [H, I] with H, I multiples of 128")
    blocks = (i // 128, h // 128)
    if gate_s.shape != blocks or up_s.shape != blocks or down_s.shape != blocks[::-1]:
        raise ValueError(f"expert {e}: weight_scale_inv must be one scale per 128 x 128 block")
