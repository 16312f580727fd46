"""Checkpoint packer: safetensors files -> the fused layer's [E,2I,H] / [E,H,I] layout."""
import json

import pytest
import torch

from easyinfra_amd.moe.pack import checkpoint, pack_layer

H, I, IS, E = 64, 32, 48, 4


def _tensors(scheme, layers=2, seed=0):
    g = torch.Generator().manual_seed(seed)
    t = {}
    for L in range(layers):
        for e in range(E):
            if scheme == "mlp":
                p = f"model.layers.{L}.mlp.experts.{e}."
                names = ("gate_proj", "up_proj", "down_proj")
            else:
                p = f"model.layers.{L}.block_sparse_moe.experts.{e}."
                names = ("w1", "w3", "w2")
            t[p + names[0] + ".weight"] = torch.randn(I, H, generator=g)
            t[p + names[1] + ".weight"] = torch.randn(I, H, generator=g)
            t[p + names[2] + ".weight"] = torch.randn(H, I, generator=g)
        sp = f"model.layers.{L}.mlp.shared_experts."
        t[sp + "gate_proj.weight"] = torch.randn(IS, H, generator=g)
        t[sp + "up_proj.weight"] = torch.randn(IS, H, generator=g)
        t[sp + "down_proj.weight"] = torch.randn(H, IS, generator=g)
    return t


def _sharded(tmp_path, t):
    from safetensors.torch import save_file
    keys = sorted(t)
    half = len(keys) // 2
    shards = {"model-00001-of-00002.safetensors": keys[:half], "model-00002-of-00002.safetensors": keys[half:]}
    wm = {}
    for name, ks in shards.items():
        save_file({k: t[k].contiguous() for k in ks}, str(tmp_path / name))
        wm.update({k: name for k in ks})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": wm}))
    return tmp_path


def _expect(t, L, experts, pre="model.layers.{L}.mlp.experts.{e}.", names=("gate_proj", "up_proj", "down_proj")):
    gu = torch.stack([torch.cat([t[pre.format(L=L, e=e) + names[0] + ".weight"],
                                 t[pre.format(L=L, e=e) + names[1] + ".weight"]]) for e in experts])
    dn = torch.stack([t[pre.format(L=L, e=e) + names[2] + ".weight"] for e in experts])
    return gu, dn


@pytest.mark.parametrize("experts", [range(E), range(2, 4), [0, 1, 2, 3, 0, 2]])   # whole, EP share, EPLB replicas
def test_pack_sharded_checkpoint(tmp_path, experts):
    t = _tensors("mlp")
    d = _sharded(tmp_path, t)
    gu, dn = pack_layer(d, 1, experts, dtype=torch.float32)
    egu, edn = _expect(t, 1, list(experts))
    assert torch.equal(gu, egu) and torch.equal(dn, edn)
    assert gu.shape == (len(list(experts)), 2 * I, H) and dn.shape == (len(list(experts)), H, I)
    # gate rows [0, I), up rows [I, 2I) of each expert, as FusedMoE.weight_loader stacks them
    assert torch.equal(gu[0, :I], t[f"model.layers.1.mlp.experts.{list(experts)[0]}.gate_proj.weight"])


def test_pack_shared_experts_and_bf16(tmp_path):
    t = _tensors("mlp")
    d = _sharded(tmp_path, t)
    ck = checkpoint(d)
    gu, dn, sgu, sdn = pack_layer(ck, 0, range(E), shared=True)
    assert gu.dtype == torch.bfloat16
    sp = "model.layers.0.mlp.shared_experts."
    assert torch.equal(sgu, torch.cat([t[sp + "gate_proj.weight"], t[sp + "up_proj.weight"]]).to(torch.bfloat16))
    assert torch.equal(sdn, t[sp + "down_proj.weight"].to(torch.bfloat16))
    assert sgu.shape == (2 * IS, H) and sdn.shape == (H, IS)


def test_pack_mixtral_names_single_file(tmp_path):
    from safetensors.torch import save_file
    t = _tensors("mixtral")
    save_file(t, str(tmp_path / "model.safetensors"))
    gu, dn = pack_layer(tmp_path / "model.safetensors", 1, range(E), scheme="mixtral", dtype=torch.float32)
    egu, edn = _expect(t, 1, range(E), "model.layers.{L}.block_sparse_moe.experts.{e}.", ("w1", "w3", "w2"))
    assert torch.equal(gu, egu) and torch.equal(dn, edn)


def test_pack_errors(tmp_path):
    t = _tensors("mlp")
    d = _sharded(tmp_path, t)
    with pytest.raises(KeyError):
        pack_layer(d, 5, range(E))
    with pytest.raises(ValueError):
        pack_layer(d, 0, [], dtype=torch.float32)
    with pytest.raises(ValueError):
        pack_layer(d, 0, range(E), scheme="other")
