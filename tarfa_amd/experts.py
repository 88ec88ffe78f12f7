"""Drop-in boundary: the reference's experts.forward and the whole MoE block.

The reference replaces the routed-compute step of each decoder layer by binding
a closure to the experts *instance*:

    experts.forward = types.MethodType(forward, experts)      tarfa/engine/fused_int4.py:262
    def forward(self, hidden_states, top_k_index, top_k_weights) -> Tensor[T, H]   :155

after popping the ``gate_up_proj`` / ``down_proj`` parameters (tarfa/engine/channel.py:27-30).
``install_experts`` does the same with libtmoe as the compute: the weights live
in HBM slabs (or anywhere the residency ledger places them), the expert ids
stay on the device, and no host synchronisation happens per layer (the
reference's ``top_k_index[0].tolist()``, fused_int4.py:166).

``TmoeSparseMoeBlock`` mirrors ``Qwen3_5MoeSparseMoeBlock.forward``
(transformers/.../modeling_qwen3_5_moe.py:787-798) with fp32 router logits.
"""
import types

import torch

from .moe import MoEShape, Workspace, expert_table, expert_table_q4, experts_forward, moe_block


class ExpertStore:
    """Where one layer's routed experts live: a device pointer table plus the shape."""

    def __init__(self, shape: MoEShape, table: torch.Tensor, device, keepalive=()):
        self.shape, self.table = shape, table
        self.workspace = Workspace(shape, device)
        self._keepalive = tuple(keepalive)   # tensors the table points into

    @classmethod
    def from_slabs(cls, shape, gate_up, down):
        return cls(shape, expert_table(gate_up, down), gate_up.device, keepalive=(gate_up, down))

    @classmethod
    def from_int4(cls, shape, gate_up_q, gate_up_s, down_q, down_s):
        """Int4 experts (labelled fast mode): packed [E,2I,H/2] / [E,H,I/2] u8, group scales bf16."""
        ts = (gate_up_q, gate_up_s, down_q, down_s)
        return cls(shape, expert_table_q4(*ts), gate_up_q.device, keepalive=ts)

    @property
    def int4(self):
        return self.table.shape[1] == 4


def make_experts_forward(store: ExpertStore):
    """The forward(self, hidden_states, top_k_index, top_k_weights) to bind on an experts module."""

    def forward(self, hidden_states, top_k_index, top_k_weights):
        # Returns a new tensor and mutates no input (fused_int4.py:161).  T == 1 accumulates
        # in router order, T > 1 in ascending expert id, as the reference does.
        x = hidden_states.contiguous()
        ids = top_k_index.contiguous()
        w = top_k_weights.to(torch.bfloat16).contiguous()
        return experts_forward(store.shape, x, ids, w, store.table, store.workspace)

    return forward


def _check_silu(experts):
    act = getattr(experts, "act_fn", None)
    if act is not None and not isinstance(act, torch.nn.SiLU) and type(act).__name__ not in ("SiLU", "SiLUActivation"):
        raise ValueError(f"libtmoe computes SwiGLU with SiLU; this module uses {type(act).__name__}")


def install_experts(experts, store: ExpertStore):
    """Bind the libtmoe routed-compute step on an experts module instance (fused_int4.py:262)."""
    _check_silu(experts)
    for name in ("gate_up_proj", "down_proj"):
        experts._parameters.pop(name, None)
    experts.forward = types.MethodType(make_experts_forward(store), experts)
    experts._tmoe_store = store
    return experts


class TmoeSparseMoeBlock(torch.nn.Module):
    """Router (fp32 logits) + routed experts + shared expert + combine on libtmoe."""

    def __init__(self, shape: MoEShape, router_w, store: ExpertStore, shared=None, heat=None):
        super().__init__()
        self.shape, self.router_w, self.store, self.shared, self.heat = shape, router_w, store, shared, heat
        self.last_ids = self.last_weights = None

    def forward(self, hidden_states, logits=None):
        B, S, H = hidden_states.shape
        x = hidden_states.reshape(-1, H).contiguous()
        out, ids, w = moe_block(self.shape, x, self.store.table, self.store.workspace, router_w=self.router_w,
                                logits=logits, shared=self.shared, heat=self.heat)
        self.last_ids, self.last_weights = ids, w
        return out.reshape(B, S, H)


def from_transformers_block(block, device=None):
    """Build a TmoeSparseMoeBlock from a transformers Qwen3_5MoeSparseMoeBlock (weights copied, bf16)."""
    dev = torch.device(device or "cuda")
    ex = block.experts
    _check_silu(ex)
    gu = ex.gate_up_proj.detach().to(dev, torch.bfloat16).contiguous()
    dn = ex.down_proj.detach().to(dev, torch.bfloat16).contiguous()
    E, I2, H = gu.shape
    sh = block.shared_expert
    Is = sh.gate_proj.weight.shape[0]
    shape = MoEShape(H, E, I2 // 2, block.gate.top_k, Is)
    shared = tuple(t.detach().to(dev, torch.bfloat16).contiguous()
                   for t in (sh.gate_proj.weight, sh.up_proj.weight, sh.down_proj.weight,
                             block.shared_expert_gate.weight.reshape(-1)))
    rw = block.gate.weight.detach().to(dev, torch.bfloat16).contiguous()
    return TmoeSparseMoeBlock(shape, rw, ExpertStore.from_slabs(shape, gu, dn), shared)
