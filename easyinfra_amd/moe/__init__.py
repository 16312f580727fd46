from .config import get_moe_impl  # noqa: F401
from .fused_moe import HipFusedMoE  # noqa: F401
from .groups import SingleRankGroup  # noqa: F401
