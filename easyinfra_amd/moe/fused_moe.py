"""HipFusedMoE: the MI355X expert module behind EasyInfra's MoE plugin point.

Mirrors ``FusedMoE`` (easyinfra/generation/modules/moe/fused_moe.py:15-156) and
its base ``_MoENoExperts`` (modules/moe/base.py:44-88): same constructor
arguments, the same parameters (``experts_gate_up_weight[E,2I,H]`` with gate rows
[0,I) and up rows [I,2I), ``experts_down_weight[E,H,I]``), the same
``weight_loader`` naming ("{physical_id}.{gate|up|down}_proj.weight"), and the same
``forward_ep(hidden_states, expert_count) -> [M,H]`` contract: rows grouped by
(source rank, local expert), output unweighted (the block applies routing weights
at combine, moe_all2all.py:84, 291-307), empty input returned as is.

The expert compute is two C-ABI grouped GEMMs (gate/up with SiLU*mul fused, then
down); segment offsets come from the counts on the device, so no host sync.  For
the whole layer (routing included) see ``forward_layer`` / ``easyinfra_amd.fused_moe``.
"""
from __future__ import annotations

from typing import List, Optional, Sequence, Union

import torch
from torch import nn
from torch.nn.parameter import Parameter

from .. import ops
from .groups import SingleRankGroup


class HipFusedMoE(nn.Module):
    def __init__(self, layer_idx: int, hidden_size: int, moe_intermediate_size: int, activation_key: str,
                 gate_up_bias: bool, down_bias: bool, num_logical_experts: int, ep_group=None, moe_tp_group=None,
                 phy2log_expert_map: Optional[torch.Tensor] = None, **kwargs):
        super().__init__()
        ep_group = ep_group if ep_group is not None else SingleRankGroup()
        moe_tp_group = moe_tp_group if moe_tp_group is not None else SingleRankGroup()
        if phy2log_expert_map is None:
            phy2log_expert_map = torch.arange(num_logical_experts).view(1, -1)
        # modules/moe/base.py:54-74
        self.layer_idx = layer_idx
        self.num_logical_experts = num_logical_experts
        self.ep_group = ep_group
        self.moe_tp_group = moe_tp_group
        self.ep_size = ep_group.group_size
        self.ep_rank = ep_group.local_rank
        self.moe_tp_size = moe_tp_group.group_size
        self.moe_tp_rank = moe_tp_group.local_rank
        self.moe_tp_intermediate_size = moe_intermediate_size // self.moe_tp_size
        if self.moe_tp_intermediate_size * self.moe_tp_size != moe_intermediate_size:
            raise ValueError(f"MoE intermediate size {moe_intermediate_size} cannot divide moe_tp size "
                             f"{self.moe_tp_size}")
        self.num_physical_experts = phy2log_expert_map.shape[-1]
        self.num_global_experts = self.num_physical_experts * self.ep_size
        if self.ep_size * (self.num_logical_experts // self.ep_size) != self.num_logical_experts:
            raise ValueError(f"Num logical experts cannot be devided by EP size: ep size is {self.ep_size}, but the "
                             f"number of experts is {self.num_logical_experts}.")
        if activation_key != "silu":
            raise NotImplementedError(f"activation {activation_key!r}: the fused epilogue implements SiLU*mul only")
        if gate_up_bias or down_bias:
            # The reference's fused path cannot run with a bias either: its launcher evaluates
            # `bias.stride(0) if bias else 0` (fused_moe.py:362), the truth value of an [E, N]
            # tensor, which torch refuses with a RuntimeError, and fused_moe_kernel takes the bias
            # pointer without reading it (fused_moe.py:213-296).  Refuse at construction instead.
            raise NotImplementedError("expert biases are not supported by the fused expert path")
        self.activation_key = activation_key
        self.hidden_size = hidden_size
        E, I, H = self.num_physical_experts, self.moe_tp_intermediate_size, hidden_size
        self.experts_gate_up_weight = Parameter(torch.empty((E, 2 * I, H)), requires_grad=False)
        self.experts_down_weight = Parameter(torch.empty((E, H, I)), requires_grad=False)
        self.experts_gate_up_bias = None
        self.experts_down_bias = None
        self.w_scales = None          # (s_gate_up [E,2I], s_down [E,H]) once quantised to fp8
        self.loaded_values = {"gate_up": [None] * E * 2, "down": [None] * E}
        self.proj_names_and_offsets = {"gate": ("gate_up", 0), "up": ("gate_up", 1), "down": ("down", 0)}
        self.proj_names_and_block_size = {"gate_up": 2, "down": 1}
        self.forward = self.forward_ep if self.ep_size > 1 else self.forward_noep

    # ------------------------------------------------------------------ weights
    def _device(self):
        return torch.device("cuda", torch.cuda.current_device()) if torch.cuda.is_available() else torch.device("cpu")

    def weight_loader(self, module_name: str, value: torch.Tensor, dtype: torch.dtype, param_name: str, **kwargs):
        """fused_moe.py:77-104: param_name "{physical_id}.{gate|up|down}_proj.weight"; the memory
        layout is [gate0, up0, gate1, up1, ...] stacked into [E, 2I, H] once every piece arrived."""
        parts = param_name.split(".")
        physical_expert_id = int(parts[0])
        short = parts[1][:-5]                       # drop "_proj"
        if short not in self.proj_names_and_offsets:
            raise ValueError(f"unknown projection {parts[1]!r} in {param_name!r}")
        proj_name, offset = self.proj_names_and_offsets[short]
        if not hasattr(self, "loaded_values") or proj_name not in self.loaded_values:
            raise ValueError(f"project name {proj_name} (from {short}) already loaded or unknown")
        block = self.proj_names_and_block_size[proj_name]
        self.loaded_values[proj_name][block * physical_expert_id + offset] = value.to(self._device())
        if not any(v is None for v in self.loaded_values[proj_name]):
            attr = "experts_" + proj_name + "_" + parts[2]
            old: torch.Tensor = getattr(self, attr)
            stacked = torch.stack(self.loaded_values[proj_name], dim=0).view(old.shape)
            if tuple(stacked.shape) != tuple(old.shape):
                raise ValueError(f"{attr}: loaded shape {tuple(stacked.shape)} != {tuple(old.shape)}")
            new = stacked.to(dtype if dtype is not None else old.dtype).contiguous()
            del self.loaded_values[proj_name]
            setattr(self, attr, Parameter(new, requires_grad=False))
        if hasattr(self, "loaded_values") and len(self.loaded_values) == 0:
            del self.loaded_values

    def quantize_weights_fp8(self):
        """Switch the expert weights to OCP e4m3 with per-output-channel scales (W8A16)."""
        qgu, sgu = ops.quantize_weights_fp8(self.experts_gate_up_weight.data.contiguous())
        qd, sd = ops.quantize_weights_fp8(self.experts_down_weight.data.contiguous())
        self.experts_gate_up_weight = Parameter(qgu, requires_grad=False)
        self.experts_down_weight = Parameter(qd, requires_grad=False)
        self.w_scales = (sgu, sd)

    # ------------------------------------------------------------------ compute
    def _counts_tensor(self, expert_count, device) -> torch.Tensor:
        if isinstance(expert_count, torch.Tensor):
            c = expert_count.reshape(-1)
        else:
            c = torch.tensor(list(expert_count), dtype=torch.int32)
        n_seg = c.numel()
        if n_seg % self.num_physical_experts != 0:
            raise ValueError(f"expert_count has {n_seg} entries while there are {self.num_physical_experts} "
                             "physical experts per rank")
        return c.to(device=device, dtype=torch.int32).contiguous()

    def forward_ep(self, hidden_states: torch.Tensor, expert_count: Union[torch.Tensor, Sequence[int]]):
        """fused_moe.py:106-156 with do_permute_unpermute=False: rows grouped by
        (src_rank, local_expert); segment s uses expert s % E_local.  Returns [M,H] unweighted."""
        if hidden_states.shape[0] == 0:
            return hidden_states
        x = hidden_states if hidden_states.is_contiguous() else hidden_states.contiguous()
        counts = self._counts_tensor(expert_count, x.device)
        offsets = ops.counts_to_offsets(counts)
        M = x.shape[0]
        E = self.num_physical_experts
        s_gu, s_d = self.w_scales if self.w_scales is not None else (None, None)
        h = ops.gemm_gate_up_silu(x, self.experts_gate_up_weight, offsets, M, w_scale=s_gu, e_mod=E)
        y = ops.gemm_down(h, self.experts_down_weight, offsets, M, out_dtype=x.dtype, w_scale=s_d, e_mod=E)
        return y[0]

    def forward_noep(self, hidden_states: torch.Tensor, expert_count: Union[torch.Tensor, Sequence[int]]):
        """ep=1: the same grouped expert compute (rows grouped by local expert)."""
        return self.forward_ep(hidden_states, expert_count)

    def forward_layer(self, hidden_states: torch.Tensor, router_logits: torch.Tensor, top_k: int,
                      renormalize: bool = True, expert_range=None, out_dtype=None):
        """The whole MoE layer on this GPU's experts: route, align, experts, combine."""
        return ops.fused_moe(hidden_states, router_logits, top_k, self.experts_gate_up_weight,
                             self.experts_down_weight, renormalize=renormalize, expert_range=expert_range,
                             w_scales=self.w_scales, out_dtype=out_dtype)
