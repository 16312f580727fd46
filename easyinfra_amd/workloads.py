"""Seeded synthetic MoE-layer workloads (inputs only; no reference math here).

Each workload is one MoE layer call: hidden states ``x[T,H]``, router logits
``logits[T,E]`` (fp32), top-k, and the expert weights in the reference's fused
layout (``experts_gate_up_weight[E,2I,H]`` with gate rows ``[0,I)`` and up rows
``[I,2I)``, ``experts_down_weight[E,H,I]``; easyinfra/generation/modules/moe/
fused_moe.py:46-47, 91-101).

Draw order per workload (one generator, seeded per workload):
x, gate_w, W_gate[E,I,H], W_up[E,I,H], W_down[E,H,I], shared weights, routing
draws.  Everything is drawn in fp32 and cast to the workload dtype; the logits
are computed once from the *cast* hidden states and handed to both the GPU
path and the CPU oracle, so routing inputs are identical.

The generator lives on ``device``: the same seed on the same device type gives
the same tensors.  Mixtral-size weights (1.4 G normals) take ~40 s to draw on a
CPU, so the large workloads are drawn on the GPU.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional

import torch


@dataclass(frozen=True)
class MoEShape:
    name: str
    seed: int
    hidden: int
    inter: int
    n_experts: int            # global expert count E (router width)
    top_k: int
    dtype: torch.dtype
    tokens: tuple             # token counts exercised
    renormalize: bool = True
    n_local: Optional[int] = None      # experts resident on this GPU (ids [0, n_local))
    shared_inter: int = 0              # concatenated shared-expert intermediate size
    routing: str = "softmax"           # softmax | zipf | hotcold

    @property
    def e_loc(self) -> int:
        return self.n_local if self.n_local is not None else self.n_experts


# The five layer shapes; the parity tests and the benchmark use these.
TINY_MIXTRAL_FP32 = MoEShape("tiny-mixtral-fp32", 0, 1024, 2816, 8, 2, torch.float32, (512,))
MIXTRAL_8X7B = MoEShape("mixtral-8x7b", 1, 4096, 14336, 8, 2, torch.bfloat16, (8192, 64))
DEEPSEEK_V2_LITE = MoEShape("deepseek-v2-lite", 2, 2048, 1408, 64, 6, torch.bfloat16, (4096,),
                            renormalize=False, shared_inter=2 * 1408, routing="zipf")
QWEN3_30B_A3B_LOCAL = MoEShape("qwen3-30b-a3b-local32", 3, 2048, 768, 128, 8, torch.bfloat16,
                               (1, 32, 256, 2048), n_local=32, routing="hotcold")
MIXTRAL_8X7B_FP8 = MoEShape("mixtral-8x7b-fp8", 1, 4096, 14336, 8, 2, torch.bfloat16, (8192, 64))

SHAPES = {s.name: s for s in (TINY_MIXTRAL_FP32, MIXTRAL_8X7B, DEEPSEEK_V2_LITE,
                              QWEN3_30B_A3B_LOCAL, MIXTRAL_8X7B_FP8)}


@dataclass
class MoEInputs:
    shape: MoEShape
    x: torch.Tensor                  # [T,H] workload dtype
    logits: torch.Tensor             # [T,E] fp32
    w_gate_up: torch.Tensor          # [E_loc,2I,H]
    w_down: torch.Tensor             # [E_loc,H,I]
    shared_gate_up: Optional[torch.Tensor] = None   # [2Is,H]
    shared_down: Optional[torch.Tensor] = None      # [H,Is]
    extra: dict = field(default_factory=dict)

    @property
    def expert_range(self):
        s = self.shape
        return (0, s.e_loc) if s.n_local is not None else None

    def to(self, device) -> "MoEInputs":
        mv = lambda t: None if t is None else t.to(device)
        return MoEInputs(self.shape, mv(self.x), mv(self.logits), mv(self.w_gate_up), mv(self.w_down),
                         mv(self.shared_gate_up), mv(self.shared_down), dict(self.extra))


def _normal(shape, std, gen, device):
    t = torch.empty(shape, dtype=torch.float32, device=device)
    t.normal_(0.0, std, generator=gen)
    return t


def make_inputs(shape: MoEShape, tokens: int, device="cpu", uniform_twin: bool = False,
                hidden: Optional[int] = None, inter: Optional[int] = None) -> MoEInputs:
    """Draw one workload.  ``hidden``/``inter`` override the sizes (small test variants)."""
    H = hidden or shape.hidden
    I = inter or shape.inter
    E, k, dt = shape.n_experts, shape.top_k, shape.dtype
    e_loc = shape.e_loc
    gen = torch.Generator(device=device)
    gen.manual_seed(shape.seed * 1000 + tokens)
    T = tokens
    x32 = _normal((T, H), 1.0, gen, device)
    x = x32.to(dt)
    gate_w = _normal((H, E), 0.02, gen, device)
    w_gate = _normal((e_loc, I, H), 0.02, gen, device).to(dt)
    w_up = _normal((e_loc, I, H), 0.02, gen, device).to(dt)
    w_gate_up = torch.cat([w_gate, w_up], dim=1).contiguous()
    del w_gate, w_up
    w_down = _normal((e_loc, H, I), 0.02, gen, device).to(dt).contiguous()
    sh_gu = sh_d = None
    if shape.shared_inter:
        Is = shape.shared_inter if inter is None else 2 * I
        sh_gu = _normal((2 * Is, H), 0.02, gen, device).to(dt).contiguous()
        sh_d = _normal((H, Is), 0.02, gen, device).to(dt).contiguous()
    extra = {}
    if shape.routing == "hotcold":
        logits, extra = _hotcold_logits(T, E, k, e_loc, gen, device, uniform_twin)
    else:
        logits = x.float() @ gate_w
        if shape.routing == "zipf":
            perm = torch.randperm(E, generator=gen, device=device).to(torch.float32) + 1.0
            bias = -1.2 * torch.log(perm)
            if not uniform_twin:
                logits = logits + bias
            extra["bias"] = bias
    return MoEInputs(shape, x.contiguous(), logits.contiguous(), w_gate_up, w_down, sh_gu, sh_d, extra)


def _hotcold_logits(T, E, k, e_loc, gen, device, uniform_twin):
    """Top-k sets drawn without replacement with known popularity, then written as logits.

    Local experts are ids [0, e_loc).  Ids [0, 4) are hot with 8x the weight of a
    cold local expert; remote experts get the weight that makes the local share of
    assignments about a quarter.  The uniform twin gives every expert the same weight
    (local share e_loc/E, also a quarter at 32/128).  Chosen experts get logits
    8 + clip(N(0,.5),±2) and the rest clip(N(0,.5),±2), so the chosen set is the
    top-k with a margin of at least 4.
    """
    wts = torch.ones(E, dtype=torch.float32, device=device)
    if not uniform_twin:
        n_hot = max(1, e_loc // 8)
        wts[:n_hot] = 8.0
        local_w = float(wts[:e_loc].sum())
        wts[e_loc:] = 3.0 * local_w / (E - e_loc)
    chosen = torch.multinomial(wts.expand(T, E), k, replacement=False, generator=gen)
    noise = _normal((T, E), 0.5, gen, device).clamp_(-2.0, 2.0)
    logits = noise.clone()
    logits.scatter_(1, chosen, noise.gather(1, chosen) + 8.0)
    return logits, {"popularity": wts}


def layer_flops(n_assign: int, T: int, H: int, I: int, shared_inter: int = 0) -> float:
    """Algorithmic FLOPs: 6*A*H*I routed + 6*T*H*Is shared (padding, router, SiLU, combine excluded)."""
    return 6.0 * n_assign * H * I + 6.0 * T * H * shared_inter


def layer_bytes(touched_experts: int, T: int, E: int, H: int, I: int, b_w: float, b_x: int, b_y: int,
                shared_inter: int = 0, fp8_scales: bool = False) -> float:
    """Algorithmic HBM bytes: touched expert weights + scales + x in + y out + logits."""
    b = touched_experts * 3.0 * H * I * b_w
    if fp8_scales:
        b += touched_experts * (2 * I + H) * 4.0
    b += 3.0 * H * shared_inter * b_w
    b += T * H * b_x + T * H * b_y + T * E * 4.0
    return b
