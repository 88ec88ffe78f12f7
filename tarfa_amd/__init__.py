"""tarfa_amd: an MI355X-native (gfx950) per-layer MoE hot path behind Tarfa's experts.forward boundary.

Compute runs in hand-written HIP kernels in ``libtmoe.so`` (built by
``python -m tarfa_amd.build``), reached through a C ABI (``include/tmoe.h``).
There is no CPU or PyTorch fallback: without the library every entry point raises.
"""
from .moe import MoEShape, Workspace, dispatch, expert_table, experts_forward, moe_block, router_topk  # noqa: F401
from .experts import ExpertStore, TmoeSparseMoeBlock, install_experts, make_experts_forward  # noqa: F401

__all__ = ["MoEShape", "Workspace", "dispatch", "expert_table", "experts_forward", "moe_block", "router_topk",
           "ExpertStore", "TmoeSparseMoeBlock", "install_experts", "make_experts_forward"]
