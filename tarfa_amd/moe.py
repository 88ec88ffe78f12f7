"""Host-side wrappers over the tmoe C ABI: validation, workspaces, launches.

Tensors are torch tensors used as device memory; every computation runs in
libtmoe's HIP kernels on the current torch stream.  Shapes follow the
reference's expert layout (transformers/.../modeling_qwen3_5_moe.py:729-730):
gate_up [E, 2I, H] with rows [0, I) = gate and [I, 2I) = up, down [E, H, I].
"""
import dataclasses

import torch

from ._lib import check, lib


@dataclasses.dataclass(frozen=True)
class MoEShape:
    hidden: int                  # H
    num_experts: int             # E
    intermediate: int            # I (per routed expert)
    top_k: int = 8               # k
    shared_intermediate: int = 0  # Is (0 = no shared expert)
    group_size: int = 128        # int4 quantisation group along K

    def ws_bytes(self, tokens):
        n = lib().tmoe_workspace_bytes(tokens, self.hidden, self.num_experts, self.intermediate, self.top_k,
                                       self.shared_intermediate)
        if n == 0:
            raise ValueError(f"unsupported MoE shape {self} at T={tokens}")
        return n


def _p(t):
    return None if t is None else t.data_ptr()


def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


def _need(t, name, dtype, shape=None, device=None):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if t.device.type != "cuda" or (device is not None and t.device != device):
        raise ValueError(f"{name} must be on {device or 'a cuda device'}, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")


class Workspace:
    """Zero-filled device scratch sized by tmoe_workspace_bytes; grows on demand.

    Calls sharing one workspace must be ordered on one stream.
    """

    def __init__(self, shape: MoEShape, device, tokens=1):
        self.shape, self.device = shape, torch.device(device)
        self.buf = None
        self.ensure(tokens)

    def ensure(self, tokens):
        need = self.shape.ws_bytes(tokens)
        if self.buf is None or self.buf.numel() < need:
            self.buf = torch.zeros(need, dtype=torch.uint8, device=self.device)
        return self.buf

    def status(self):
        """Synchronise and raise if a kernel flagged an out-of-range expert id."""
        check(lib().tmoe_workspace_status(_p(self.buf), _stream(self.device)), "device status")


def expert_table(gate_up, down):
    """[E, 2] uint64 device table of per-expert base pointers for contiguous slabs."""
    E = gate_up.shape[0]
    gs = gate_up.stride(0) * gate_up.element_size()
    ds = down.stride(0) * down.element_size()
    host = torch.tensor([[gate_up.data_ptr() + e * gs, down.data_ptr() + e * ds] for e in range(E)],
                        dtype=torch.int64)
    return host.to(gate_up.device)


def expert_table_q4(gate_up_q, gate_up_s, down_q, down_s):
    """[E, 4] uint64 device table for int4 experts: packed gate_up [E,2I,H/2] u8, its scales
    [E,2I,H/128] bf16, packed down [E,H,I/2] u8, its scales [E,H,I/128] bf16."""
    ts = (gate_up_q, gate_up_s, down_q, down_s)
    E = gate_up_q.shape[0]
    for t in ts:
        if t.shape[0] != E or not t.is_contiguous():
            raise ValueError("int4 expert tensors must be contiguous with a leading expert dimension")
    strides = [t.stride(0) * t.element_size() for t in ts]
    host = torch.tensor([[t.data_ptr() + e * st for t, st in zip(ts, strides)] for e in range(E)],
                        dtype=torch.int64)
    if (host % 16).any():
        raise ValueError("int4 expert slabs must start 16-byte aligned")
    return host.to(gate_up_q.device)


class Int4RowTable:
    """[E, 4] device table of int4 experts in the reference's own layout: packed rows with
    ONE fp16 scale per row (tarfa/engine/channel_q4.py:10-14, 18, 28-38)."""

    def __init__(self, table):
        self.table = table

    @property
    def shape(self):
        return self.table.shape

    def data_ptr(self):
        return self.table.data_ptr()


def expert_table_q4_rows(gate_up_q, gate_up_s, down_q, down_s):
    """Int4RowTable for packed gate_up [E,2I,H/2] u8, its scales [E,2I] fp16, packed down
    [E,H,I/2] u8, its scales [E,H] fp16."""
    for name, t, dt in (("gate_up_q", gate_up_q, torch.uint8), ("gate_up_s", gate_up_s, torch.float16),
                        ("down_q", down_q, torch.uint8), ("down_s", down_s, torch.float16)):
        if t.dtype != dt:
            raise TypeError(f"{name} must be {dt}, got {t.dtype}")
    if gate_up_s.dim() != 2 or down_s.dim() != 2:
        raise ValueError("per-row scales are [E, rows]")
    return Int4RowTable(expert_table_q4(gate_up_q, gate_up_s, down_q, down_s))


def dequant_int4_f16(packed, scales, group=None):
    """The reference's dequant_int4 (channel_q4.py:10-14) on the device: packed [..., K/2]
    uint8 and fp16 scales [..., K/group] (group = K, the default: one scale per row) ->
    fp16 [..., K] = fp16((nibble - 8) * scale), bit for bit."""
    _need(packed, "packed", torch.uint8)
    _need(scales, "scales", torch.float16, None, packed.device)
    K = packed.shape[-1] * 2
    N = packed.numel() * 2 // K
    group = K if group is None else group
    if scales.numel() != N * (K // group):
        raise ValueError("scales do not match packed and group")
    out = torch.empty(*packed.shape[:-1], K, dtype=torch.float16, device=packed.device)
    check(lib().tmoe_dequant_int4_f16(_p(packed), _p(scales), N, K, group, _p(out), _stream(packed.device)),
          "tmoe_dequant_int4_f16")
    return out


def quantize_int4(w, group=128):
    """bf16 [..., K] -> (packed [..., K/2] uint8, scales [..., K/group] bf16) on the device."""
    _need(w, "w", torch.bfloat16)
    K = w.shape[-1]
    N = w.numel() // K
    packed = torch.empty(*w.shape[:-1], K // 2, dtype=torch.uint8, device=w.device)
    scales = torch.empty(*w.shape[:-1], K // group, dtype=torch.bfloat16, device=w.device)
    check(lib().tmoe_quantize_int4(_p(w), N, K, group, _p(packed), _p(scales), _stream(w.device)),
          "tmoe_quantize_int4")
    return packed, scales


def dequant_int4(packed, scales, group=128):
    """(packed [..., K/2] uint8, scales [..., K/group] bf16) -> bf16 [..., K] (materialised)."""
    _need(packed, "packed", torch.uint8)
    _need(scales, "scales", torch.bfloat16, None, packed.device)
    K = packed.shape[-1] * 2
    N = packed.numel() * 2 // K
    if scales.numel() != N * (K // group):
        raise ValueError("scales do not match packed and group")
    out = torch.empty(*packed.shape[:-1], K, dtype=torch.bfloat16, device=packed.device)
    check(lib().tmoe_dequant_int4_bf16(_p(packed), _p(scales), N, K, group, _p(out), _stream(packed.device)),
          "tmoe_dequant_int4_bf16")
    return out


def _table_kind(table, E, dev):
    """0: bf16 experts ([E, 2]); 1: int4 with group scales ([E, 4]); 2: int4 in the
    reference's per-row fp16 layout (Int4RowTable)."""
    rows = isinstance(table, Int4RowTable)
    t = table.table if rows else table
    _need(t, "expert_table", torch.int64, None, dev)
    if t.dim() != 2 or t.shape[0] != E or t.shape[1] not in (2, 4) or (rows and t.shape[1] != 4):
        raise ValueError(f"expert_table must be [E, 2] (bf16) or [E, 4] (int4), got {tuple(t.shape)}")
    return 2 if rows else (1 if t.shape[1] == 4 else 0)


_INT4_SUFFIX = {0: "bf16", 1: "int4", 2: "int4_f16rows"}


def router_topk(shape: MoEShape, x=None, router_w=None, logits=None, heat=None):
    """fp32-logit router: returns (ids [T,k] int64, weights [T,k] bf16, logits [T,E] fp32)."""
    H, E, k = shape.hidden, shape.num_experts, shape.top_k
    if logits is None:
        _need(x, "x", torch.bfloat16)
        T = x.shape[0]
        dev = x.device
        _need(router_w, "router_w", torch.bfloat16, (E, H), dev)
        logits_out = torch.empty(T, E, dtype=torch.float32, device=dev)
    else:
        _need(logits, "logits", torch.float32)
        T, dev = logits.shape[0], logits.device
        logits_out = logits
    ids = torch.empty(T, k, dtype=torch.int64, device=dev)
    w = torch.empty(T, k, dtype=torch.bfloat16, device=dev)
    if heat is not None:
        _need(heat, "heat", torch.int32, (E,), dev)
    st = lib().tmoe_router_topk(_p(x) if logits is None else None, _p(router_w) if logits is None else None,
                                _p(logits), T, H, E, k, _p(ids), _p(w), _p(logits_out), _p(heat), _stream(dev))
    check(st, "tmoe_router_topk")
    return ids, w, logits_out


def dispatch(ids, num_experts, workspace: Workspace):
    """(offsets [E+1] int32, perm [T*k] int32, inv [T*k] int32) of the prefill permutation."""
    _need(ids, "ids", torch.int64)
    T, k = ids.shape
    dev = ids.device
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    perm = torch.empty(T * k, dtype=torch.int32, device=dev)
    inv = torch.empty(T * k, dtype=torch.int32, device=dev)
    buf = workspace.ensure(T)
    st = lib().tmoe_dispatch(_p(ids), T, k, num_experts, _p(offsets), _p(perm), _p(inv), _p(buf), buf.numel(),
                             _stream(dev))
    check(st, "tmoe_dispatch")
    return offsets, perm, inv


def topk_renorm(ids, weights, j):
    """The reference's re-truncation of a routing to j experts (tarfa/engine/fused_int4.py:157-160):
    per token the j largest bf16 weights (equal weights keep the lower slot first), their ids,
    and the weights renormalised in bf16; returns (ids [T,j] int64, weights [T,j] bf16)."""
    dev = ids.device
    T, k = ids.shape
    _need(ids, "top_k_index", torch.int64, (T, k), dev)
    _need(weights, "top_k_weights", torch.bfloat16, (T, k), dev)
    ids_out = torch.empty(T, j, dtype=torch.int64, device=dev)
    w_out = torch.empty(T, j, dtype=torch.bfloat16, device=dev)
    check(lib().tmoe_topk_renorm_bf16(_p(ids), _p(weights), T, k, j, _p(ids_out), _p(w_out), _stream(dev)),
          "tmoe_topk_renorm_bf16")
    return ids_out, w_out


def experts_forward(shape: MoEShape, x, ids, weights, table, workspace: Workspace, out=None):
    """Routed experts only (the reference's experts.forward); returns out [T,H] bf16.

    ``table`` [E, 2] selects exact bf16 experts, [E, 4] (expert_table_q4) the int4 fast mode,
    an Int4RowTable (expert_table_q4_rows) the reference's own per-row fp16 int4 layout.
    """
    H, E, I, k = shape.hidden, shape.num_experts, shape.intermediate, shape.top_k
    _need(x, "hidden_states", torch.bfloat16)
    T, dev = x.shape[0], x.device
    _need(x, "hidden_states", torch.bfloat16, (T, H), dev)
    _need(ids, "top_k_index", torch.int64, (T, k), dev)
    _need(weights, "top_k_weights", torch.bfloat16, (T, k), dev)
    q4 = _table_kind(table, E, dev)
    if out is None:
        out = torch.empty_like(x)
    buf = workspace.ensure(T)
    fn = "tmoe_experts_forward_" + _INT4_SUFFIX[q4]
    st = getattr(lib(), fn)(_p(x), T, _p(ids), _p(weights), _p(table), H, E, I, k, _p(out), _p(buf), buf.numel(),
                            _stream(dev))
    check(st, fn)
    return out


def moe_layer(shape: MoEShape, h, ln_w, eps, table, workspace: Workspace, **kw):
    """The MoE sublayer of a decoder layer: bf16(h + moe_block(rmsnorm(h)))
    (transformers modeling_qwen3_5_moe.py:870-875); ``ln_w`` is post_attention_layernorm's
    [H] bf16 weight (scale 1 + ln_w).  Other arguments and the result as moe_block."""
    _need(ln_w, "ln_w", torch.bfloat16, (shape.hidden,), h.device)
    return moe_block(shape, h, table, workspace, _ln=(ln_w, float(eps)), **kw)


def moe_block(shape: MoEShape, x, table, workspace: Workspace, router_w=None, logits=None, shared=None,
              heat=None, out=None, ids=None, weights=None, _ln=None):
    """Router + routed experts + shared expert + combine; returns (out, ids, weights).

    ``shared`` = (gate_proj [Is,H], up_proj [Is,H], down_proj [H,Is], shared_expert_gate [1,H] or [H]).
    """
    H, E, I, k, Is = shape.hidden, shape.num_experts, shape.intermediate, shape.top_k, shape.shared_intermediate
    _need(x, "hidden_states", torch.bfloat16)
    T, dev = x.shape[0], x.device
    _need(x, "hidden_states", torch.bfloat16, (T, H), dev)
    q4 = _table_kind(table, E, dev)
    if logits is not None:
        _need(logits, "logits", torch.float32, (T, E), dev)
    else:
        _need(router_w, "router_w", torch.bfloat16, (E, H), dev)
    sh = [None] * 4
    if shared is not None:
        g, u, d, sg = shared
        _need(g, "shared gate_proj", torch.bfloat16, (Is, H), dev)
        _need(u, "shared up_proj", torch.bfloat16, (Is, H), dev)
        _need(d, "shared down_proj", torch.bfloat16, (H, Is), dev)
        _need(sg, "shared_expert_gate", torch.bfloat16, None, dev)
        if sg.numel() != H:
            raise ValueError("shared_expert_gate must hold H values")
        sh = [g, u, d, sg]
    elif Is:
        raise ValueError("shape has a shared expert but no shared weights were given")
    if heat is not None:
        _need(heat, "heat", torch.int32, (E,), dev)
    out = torch.empty_like(x) if out is None else out
    ids = torch.empty(T, k, dtype=torch.int64, device=dev) if ids is None else ids
    weights = torch.empty(T, k, dtype=torch.bfloat16, device=dev) if weights is None else weights
    buf = workspace.ensure(T)
    ln = [] if _ln is None else [_p(_ln[0]), _ln[1]]
    if _ln is not None and q4 == 2:
        raise ValueError("the sublayer entry points take bf16 or group-scaled int4 experts")
    fn = ("tmoe_moe_layer_" if _ln is not None else "tmoe_moe_block_") + _INT4_SUFFIX[q4]
    st = getattr(lib(), fn)(_p(x), T, *ln, _p(router_w) if logits is None else None, _p(logits), _p(table),
                            *[_p(t) for t in sh], H, E, I, k, Is if shared is not None else 0, _p(out),
                            _p(ids), _p(weights), _p(heat), _p(buf), buf.numel(), _stream(dev))
    check(st, fn)
    return out, ids, weights


def fill_bf16(t, key, std, start=0):
    """Seeded Irwin-Hall normals into a bf16 device tensor (see tarfa_amd.seeded)."""
    from .seeded import scale16
    _need(t, "t", torch.bfloat16)
    check(lib().tmoe_fill_bf16(_p(t), t.numel(), key, scale16(std), start, _stream(t.device)), "tmoe_fill_bf16")
    return t


def fill_f32(t, key, std, start=0):
    from .seeded import scale32
    _need(t, "t", torch.float32)
    check(lib().tmoe_fill_f32(_p(t), t.numel(), key, scale32(std), start, _stream(t.device)), "tmoe_fill_f32")
    return t
