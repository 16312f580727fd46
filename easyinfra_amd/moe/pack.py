"""Checkpoint -> fused-layer weight layout.

A Hugging Face checkpoint stores one tensor per expert projection:
``model.layers.{L}.mlp.experts.{e}.{gate,up,down}_proj.weight`` (Qwen3-MoE, DeepSeek-V2/V3;
Mixtral: ``block_sparse_moe.experts.{e}.{w1,w3,w2}.weight``), gate/up ``[I, H]`` and down
``[H, I]`` in ``nn.Linear`` layout.  The fused layer takes them stacked per layer:
``w_gate_up [E, 2I, H]`` (gate rows [0, I), up rows [I, 2I)) and ``w_down [E, H, I]``, the
layout ``FusedMoE.weight_loader`` builds one tensor at a time
(easyinfra/generation/modules/moe/fused_moe.py:77-104, with the checkpoint names mapped by
``Qwen3MoeForCausalLM.param_name_to_module_with_kwargs``, models/qwen3_moe/
modeling_qwen3_moe.py:576-600).  ``pack_layer`` reads a layer's experts straight from the
checkpoint into that layout: for an expert-parallel share (``experts=range(lo, hi)``) or an
EPLB physical layout (``experts`` = the physical->logical map, replicas repeated), plus the
shared experts (``shared_gate_up [2*Is, H]``, ``shared_down [H, Is]``).

Files are opened with ``safetensors.safe_open`` (no code runs from the file); a sharded
checkpoint is found through its ``model.safetensors.index.json``.
"""
from __future__ import annotations

import json
import os
from typing import Dict, Iterable, List, Tuple

import torch

NAME_SCHEMES: Dict[str, Tuple[str, str, str, str]] = {
    # scheme: (expert prefix, gate, up, down); {layer} and {e} are filled in
    "mlp": ("model.layers.{layer}.mlp.experts.{e}.", "gate_proj", "up_proj", "down_proj"),
    "mixtral": ("model.layers.{layer}.block_sparse_moe.experts.{e}.", "w1", "w3", "w2"),
}
SHARED_PREFIX = "model.layers.{layer}.mlp.shared_experts."


class _Checkpoint:
    """Tensor name -> file for a checkpoint directory, an index json, or a list of files."""

    def __init__(self, source):
        from safetensors import safe_open
        self._open = safe_open
        files: List[str]
        if isinstance(source, (str, os.PathLike)) and os.path.isdir(source):
            index = os.path.join(source, "model.safetensors.index.json")
            if os.path.exists(index):
                with open(index) as f:
                    wm = json.load(f)["weight_map"]
                self.where = {k: os.path.join(source, v) for k, v in wm.items()}
                return
            files = sorted(os.path.join(source, n) for n in os.listdir(source) if n.endswith(".safetensors"))
        elif isinstance(source, (str, os.PathLike)):
            files = [str(source)]
        else:
            files = [str(f) for f in source]
        self.where = {}
        for path in files:
            with safe_open(path, framework="pt") as f:
                for k in f.keys():
                    self.where[k] = path

    def get(self, name: str) -> torch.Tensor:
        path = self.where.get(name)
        if path is None:
            raise KeyError(f"{name} is not in the checkpoint")
        with self._open(path, framework="pt") as f:
            return f.get_tensor(name)

    def has(self, name: str) -> bool:
        return name in self.where


def pack_layer(source, layer: int, experts: Iterable[int], *, scheme: str = "mlp", dtype=torch.bfloat16,
               device="cpu", shared: bool = False):
    """Stack one layer's experts into the fused layout.

    ``experts``: the logical expert of each packed slot, in order (``range(lo, hi)`` for an
    expert-parallel share, ``phy2log.reshape(-1)`` for an EPLB physical layout).
    Returns ``(w_gate_up [len(experts), 2I, H], w_down [len(experts), H, I])``, plus
    ``(shared_gate_up [2*Is, H], shared_down [H, Is])`` when ``shared``.
    """
    if scheme not in NAME_SCHEMES:
        raise ValueError(f"scheme {scheme!r}: one of {sorted(NAME_SCHEMES)}")
    ck = source if isinstance(source, _Checkpoint) else _Checkpoint(source)
    prefix, g_name, u_name, d_name = NAME_SCHEMES[scheme]
    experts = [int(e) for e in experts]
    if not experts:
        raise ValueError("no experts to pack")
    gu, dn = [], []
    cache: Dict[int, Tuple[torch.Tensor, torch.Tensor]] = {}
    for e in experts:
        if e not in cache:
            p = prefix.format(layer=layer, e=e)
            gate = ck.get(p + g_name + ".weight")
            up = ck.get(p + u_name + ".weight")
            down = ck.get(p + d_name + ".weight")
            if gate.shape != up.shape or down.shape != (gate.shape[1], gate.shape[0]):
                raise ValueError(f"layer {layer} expert {e}: gate {tuple(gate.shape)}, up {tuple(up.shape)}, "
                                 f"down {tuple(down.shape)} are not [I,H], [I,H], [H,I]")
            cache[e] = (torch.cat([gate, up], dim=0).to(dtype), down.to(dtype))
        gu.append(cache[e][0])
        dn.append(cache[e][1])
    w_gate_up = torch.stack(gu).contiguous().to(device)
    w_down = torch.stack(dn).contiguous().to(device)
    if not shared:
        return w_gate_up, w_down
    sp = SHARED_PREFIX.format(layer=layer)
    sg, su, sd = (ck.get(sp + n + ".weight") for n in ("gate_proj", "up_proj", "down_proj"))
    shared_gate_up = torch.cat([sg, su], dim=0).to(dtype).contiguous().to(device)
    return w_gate_up, w_down, shared_gate_up, sd.to(dtype).contiguous().to(device)


def checkpoint(source) -> _Checkpoint:
    """Open a checkpoint once for several ``pack_layer`` calls."""
    return _Checkpoint(source)
