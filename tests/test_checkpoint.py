"""Expert weights from a sharded safetensors checkpoint (host logic, CPU):
per-expert gate/up/down tensors under the Drama-3 key scheme are stacked into
w13 [E, 2I, H] with rows [gate; up], w13_scale_inv, w2, w2_scale_inv."""

import json

import pytest
import torch

from drama3_amd.checkpoint import expert_count, load_layer_experts, load_shared_expert


def _fp8(gen, shape):
    return torch.randn(shape, generator=gen).mul(8).clamp(-448, 448).to(torch.float8_e4m3fn)


def write_checkpoint(path, layers=2, experts=4, hidden=256, inter=128, seed=0):
    from safetensors.torch import save_file

    gen = torch.Generator().manual_seed(seed)
    shards = [{}, {}]
    truth = {}
    for layer in range(layers):
        prefix = f"model.language_model.layers.{layer}.mlp"
        for e in range(experts):
            t = {"gate_proj.weight": _fp8(gen, (inter, hidden)),
                 "up_proj.weight": _fp8(gen, (inter, hidden)),
                 "down_proj.weight": _fp8(gen, (hidden, inter)),
                 "gate_proj.weight_scale_inv": torch.rand((inter // 128, hidden // 128), generator=gen),
                 "up_proj.weight_scale_inv": torch.rand((inter // 128, hidden // 128), generator=gen),
                 "down_proj.weight_scale_inv": torch.rand((hidden // 128, inter // 128), generator=gen)}
            for name, value in t.items():
                shards[(layer + e) % 2][f"{prefix}.experts.{e}.{name}"] = value
            truth[(layer, e)] = t
        for proj in ("gate_proj", "up_proj", "down_proj"):
            shape = (hidden, inter) if proj == "down_proj" else (inter, hidden)
            shards[layer % 2][f"{prefix}.shared_expert.{proj}.weight"] = torch.randn(
                shape, generator=gen).to(torch.bfloat16)
    weight_map = {}
    for k, shard in enumerate(shards):
        name = f"model-0000{k + 1}-of-00002.safetensors"
        save_file(shard, str(path / name))
        weight_map.update({key: name for key in shard})
    (path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))
    return truth


def test_layer_experts_stack_gate_then_up(tmp_path):
    truth = write_checkpoint(tmp_path)
    ex = load_layer_experts(tmp_path, 1)
    assert ex.w13_weight.shape == (4, 256, 256) and ex.w2_weight.shape == (4, 256, 128)
    assert ex.w13_scale_inv.shape == (4, 2, 2) and ex.w2_scale_inv.shape == (4, 2, 1)
    for e in range(4):
        t = truth[(1, e)]
        as_u8 = lambda x: x.view(torch.uint8)  # noqa: E731
        assert torch.equal(as_u8(ex.w13_weight[e, :128]), as_u8(t["gate_proj.weight"]))
        assert torch.equal(as_u8(ex.w13_weight[e, 128:]), as_u8(t["up_proj.weight"]))
        assert torch.equal(as_u8(ex.w2_weight[e]), as_u8(t["down_proj.weight"]))
        assert torch.equal(ex.w13_scale_inv[e, :1], t["gate_proj.weight_scale_inv"])
        assert torch.equal(ex.w13_scale_inv[e, 1:], t["up_proj.weight_scale_inv"])
        assert torch.equal(ex.w2_scale_inv[e], t["down_proj.weight_scale_inv"])
    shared = load_shared_expert(tmp_path, 0)
    assert shared["down_proj"].shape == (256, 128) and "gate" not in shared


def test_checkpoint_errors(tmp_path):
    write_checkpoint(tmp_path)
    weight_map = json.loads((tmp_path / "model.safetensors.index.json").read_text())["weight_map"]
    assert expert_count(weight_map, 0) == 4
    with pytest.raises(KeyError):
        load_layer_experts(tmp_path, 7)
    with pytest.raises(FileNotFoundError):
        load_layer_experts(tmp_path / "missing", 0)
