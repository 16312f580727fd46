"""MI355X (gfx950) fused-MoE expert path: hand-written HIP kernels behind a C ABI
(include/eimoe.h), with a PyTorch-facing layer API and a drop-in expert module for
EasyInfra's MoE plugin point.

    from easyinfra_amd import fused_moe
    out = fused_moe(hidden_states, router_logits, top_k, w_gate_up, w_down)
"""
from .ops import fused_moe  # noqa: F401

__all__ = ["fused_moe"]
