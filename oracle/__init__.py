"""CPU oracle (test infrastructure only): a restatement of EasyInfra's MoE-layer math.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
"""
from .moe_ref import (  # noqa: F401
    route_topk, route_grouped_topk, sigmoid_rn, eplb_map, moe_prologue, align, gather, silu, expert_mlp, shared_mlp, moe_forward,
    moe_forward_dense,
    quantize_rows_fp8, quantize_weights_fp8, gate_up_fp8, expert_mlp_fp8, moe_forward_fp8, grouped_gemm, rel_l2,
)
