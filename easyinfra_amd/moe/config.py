"""MoE implementation registry, mirroring get_moe_impl()
(easyinfra/generation/modules/moe/config.py:4-15) and the lazily read MOE_IMPL
flag (easyinfra/envs.py:9, 26-28).

This package provides the MI355X path only: MOE_IMPL "hip" (and "fused", the
reference's default name for its fused expert path) map to HipFusedMoE; the
reference's other backends ("native", "cutlass", "aten") are not part of it.
"""
from __future__ import annotations

import os


def moe_impl_name() -> str:
    return os.getenv("MOE_IMPL", "fused").lower()


def get_moe_impl():
    name = moe_impl_name()
    if name in ("hip", "fused"):
        from .fused_moe import HipFusedMoE
        return HipFusedMoE
    if name in ("native", "cutlass", "aten"):
        raise ValueError(f"MoE implementation {name!r} is not provided by easyinfra_amd (use MOE_IMPL=hip)")
    raise ValueError(f"Unrecognized MoE Implementation {name}")
