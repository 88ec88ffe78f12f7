"""Seeded synthetic MoE layers generated on the device.

Every tensor element is a pure function of (seed, stream, index) computed by the
``tmoe_fill_*`` kernels (splitmix64 output function over ``key + (i+1) * golden``,
Irwin-Hall n=12 normal), so a full-size model (48 x 256 experts) is written
straight into HBM and any single expert can be regenerated on the host.

A stream id is ``(layer << 40) | (kind << 32) | expert``.
"""
import dataclasses
import math

import torch

GOLDEN = 0x9E3779B97F4A7C15
M64 = (1 << 64) - 1
STD16 = math.sqrt(65536.0 ** 2 - 1.0)   # std of a sum of twelve U{0..65535}
STD32 = math.sqrt(2.0 ** 64 - 1.0)      # std of a sum of twelve U{0..2^32-1}

KIND_GATE_UP, KIND_DOWN, KIND_ROUTER, KIND_SH_GATE, KIND_SH_UP, KIND_SH_DOWN, \
    KIND_SH_GATEW, KIND_X, KIND_LOGITS = range(9)

W_STD = 0.02   # expert / router / shared weights ~N(0, 0.02)
X_STD = 1.0    # activations and synthetic logits ~N(0, 1)


def _mix(z):
    z &= M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def stream_id(kind, layer=0, expert=0):
    return (int(layer) << 40) | (int(kind) << 32) | int(expert)


def key(seed, kind, layer=0, expert=0):
    return _mix((int(seed) & M64) ^ _mix(stream_id(kind, layer, expert) + GOLDEN))


def scale16(std):
    """Multiplier of the centred 16-bit sum (passed to the kernel as fp32)."""
    return std / STD16


def scale32(std):
    return std / STD32


@dataclasses.dataclass
class SeededLayer:
    """Device tensors of one seeded MoE layer (bf16 unless noted)."""
    gate_up: torch.Tensor     # [E, 2I, H]
    down: torch.Tensor        # [E, H, I]
    router_w: torch.Tensor    # [E, H]
    shared: tuple             # (gate [Is,H], up [Is,H], down [H,Is], gate_w [H]) or None


def fill_expert_slabs(gate_up, down, seed, layer, first_expert=0):
    """Fill [n, 2I, H] / [n, H, I] slabs with experts first_expert .. first_expert + n - 1."""
    from .moe import fill_bf16
    for j in range(gate_up.shape[0]):
        e = first_expert + j
        fill_bf16(gate_up[j], key(seed, KIND_GATE_UP, layer, e), W_STD)
        fill_bf16(down[j], key(seed, KIND_DOWN, layer, e), W_STD)


def make_layer(shape, seed, layer=0, device="cuda", gate_up=None, down=None):
    """Allocate (unless slabs are given) and fill one layer's weights on ``device``."""
    from .moe import fill_bf16
    H, E, I, Is = shape.hidden, shape.num_experts, shape.intermediate, shape.shared_intermediate
    bf = dict(dtype=torch.bfloat16, device=device)
    gate_up = torch.empty(E, 2 * I, H, **bf) if gate_up is None else gate_up
    down = torch.empty(E, H, I, **bf) if down is None else down
    fill_expert_slabs(gate_up, down, seed, layer)
    router_w, shared = make_block_weights(shape, seed, layer, device)
    return SeededLayer(gate_up, down, router_w, shared)


def make_block_weights(shape, seed, layer=0, device="cuda"):
    """The router and shared-expert weights of one layer (same streams as make_layer)."""
    from .moe import fill_bf16
    H, E, Is = shape.hidden, shape.num_experts, shape.shared_intermediate
    bf = dict(dtype=torch.bfloat16, device=device)
    router_w = fill_bf16(torch.empty(E, H, **bf), key(seed, KIND_ROUTER, layer), W_STD)
    shared = None
    if Is:
        shared = (fill_bf16(torch.empty(Is, H, **bf), key(seed, KIND_SH_GATE, layer), W_STD),
                  fill_bf16(torch.empty(Is, H, **bf), key(seed, KIND_SH_UP, layer), W_STD),
                  fill_bf16(torch.empty(H, Is, **bf), key(seed, KIND_SH_DOWN, layer), W_STD),
                  fill_bf16(torch.empty(H, **bf), key(seed, KIND_SH_GATEW, layer), W_STD))
    return router_w, shared


def make_tokens(shape, seed, tokens, layer=0, device="cuda"):
    from .moe import fill_bf16
    return fill_bf16(torch.empty(tokens, shape.hidden, dtype=torch.bfloat16, device=device),
                     key(seed, KIND_X, layer), X_STD)


def make_logits(shape, seed, tokens, layer=0, device="cuda"):
    from .moe import fill_f32
    return fill_f32(torch.empty(tokens, shape.num_experts, dtype=torch.float32, device=device),
                    key(seed, KIND_LOGITS, layer), X_STD)
