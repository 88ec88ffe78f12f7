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

Around each call the boundary keeps what the reference's closure keeps
(fused_int4.py:67-109): per-call MoE counters split decode / prefill
(``telemetry()``; seconds come from HIP events, not from a forced synchronisation),
and for decode calls the route-reuse counters (``routing_telemetry()``, recorded on
the device).  Device-detected errors (an expert id outside [0, E], an expired
bounded wait) are polled without stalling the compute stream: after every call (every
``status_poll`` calls, default 1) the workspace status word is copied to pinned host
memory on a side stream, and the next call that finds the copy landed raises
``RuntimeError`` if it is set -- at the latest the first call after the engine's next
synchronisation point (the reference synchronises after every call,
tarfa/engine/fused_int4.py:203-204).  ``check_status()`` is the synchronous check.

``TmoeSparseMoeBlock`` mirrors ``Qwen3_5MoeSparseMoeBlock.forward``
(transformers/.../modeling_qwen3_5_moe.py:787-798) with fp32 router logits.
"""
import dataclasses
import os
import threading
import types
import weakref

import torch

from ._lib import check
from .int4_files import Int4LayerFile
from .moe import (MoEShape, Workspace, expert_table, expert_table_q4, expert_table_q4_rows, experts_forward, moe_block,
                  topk_renorm)
from .residency import RouteTelemetry

ENGINE_DTYPE = torch.bfloat16
_KINDS = ("decode", "prefill")
_LOCK = threading.Lock()
_BOOKS = weakref.WeakSet()      # every live call book, for the module-level telemetry views


class _CallBook:
    """Counters, event timing, route telemetry and the asynchronous status poll of one layer's calls."""

    def __init__(self, shape: MoEShape, workspace: Workspace, device, route_telemetry=True, timing=True,
                 status_poll=1):
        self.shape, self.workspace, self.device = shape, workspace, torch.device(device)
        self.counts = {k: 0 for k in _KINDS}
        self.seconds = {k: 0.0 for k in _KINDS}
        self.timing = bool(timing)
        self._pending = []                      # (kind, start event, end event), oldest first
        self._free_events = []
        self.route = (RouteTelemetry(1, shape.top_k, shape.num_experts, self.device) if route_telemetry else None)
        self.status_poll = int(status_poll)
        self._status_host = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        self._status_event = None
        self._side = None
        _BOOKS.add(self)

    # ------------------------------------------------------------------ status
    def _raise_if_flagged(self, flags):
        if flags:
            code = -7 if flags & 2 else -6      # TMOE_ERR_TIMEOUT / TMOE_ERR_EXPERT_ID
            check(code, "libtmoe device status (asynchronous poll)")

    def _poll(self, stream):
        ev = self._status_event
        if ev is not None and ev.query():
            self._status_event = None
            self._raise_if_flagged(int(self._status_host[0]))
        total = self.counts["decode"] + self.counts["prefill"]
        if self.status_poll > 0 and self._status_event is None and total % self.status_poll == 0:
            if self._side is None:
                self._side = torch.cuda.Stream(self.device)
            buf = self.workspace.buf
            self._side.wait_stream(stream)
            with torch.cuda.stream(self._side):
                self._status_host.copy_(buf[:4].view(torch.int32), non_blocking=True)
                ev = torch.cuda.Event()
                ev.record(self._side)
            buf.record_stream(self._side)
            self._status_event = ev

    def check_status(self):
        """Synchronise and raise on a device-detected error (clears the status)."""
        self._status_event = None
        self.workspace.status()

    # ------------------------------------------------------------------ timing
    def _event(self):
        return self._free_events.pop() if self._free_events else torch.cuda.Event(enable_timing=True)

    def _harvest(self, block=False):
        while self._pending:
            kind, e0, e1 = self._pending[0]
            if not block and not e1.query():
                break
            e1.synchronize()
            self.seconds[kind] += e0.elapsed_time(e1) * 1e-3
            self._free_events += [e0, e1]
            self._pending.pop(0)

    def call(self, kind, fn, record_ids=None):
        """Run fn() (one libtmoe launch sequence on the current stream) as a ``kind`` call."""
        stream = torch.cuda.current_stream(self.device)
        self._poll(stream)
        if self.timing:
            e0 = self._event()
            e0.record(stream)
        out = fn()
        if self.timing:
            e1 = self._event()
            e1.record(stream)
            self._pending.append((kind, e0, e1))
            if len(self._pending) > 256:
                self._harvest()
        if record_ids is not None and self.route is not None:
            self.route.record(record_ids)
        with _LOCK:
            self.counts[kind] += 1
        return out


def telemetry(reset=False):
    """The reference's telemetry() fields (fused_int4.py:97-103) over every live store and block:
    calls and seconds, in total and split decode / prefill.  Synchronises on pending timing events.
    The reference's bf16 cache hit / miss counters count experts that were (not) already on the GPU;
    with every expert resident here, every routed expert use is a hit."""
    out = {"moe_calls": 0, "moe_seconds": 0.0, "prefill_moe_calls": 0, "prefill_moe_seconds": 0.0,
           "decode_moe_calls": 0, "decode_moe_seconds": 0.0, "bf16_cache_hits": 0, "bf16_cache_misses": 0}
    for b in list(_BOOKS):
        b._harvest(block=True)
        for k in _KINDS:
            out[f"{k}_moe_calls"] += b.counts[k]
            out[f"{k}_moe_seconds"] += b.seconds[k]
        if b.route is not None:
            out["bf16_cache_hits"] += int(b.route.counters()[0, 1])
        if reset:
            b.counts = {k: 0 for k in _KINDS}
            b.seconds = {k: 0.0 for k in _KINDS}
    out["moe_calls"] = out["prefill_moe_calls"] + out["decode_moe_calls"]
    out["moe_seconds"] = out["prefill_moe_seconds"] + out["decode_moe_seconds"]
    return out


def routing_telemetry(reset=False):
    """The reference's routing_telemetry() (fused_int4.py:86-95) summed over every live store's
    decode calls (each store is one layer)."""
    c = [0] * 8
    for b in list(_BOOKS):
        if b.route is None:
            continue
        cs = b.route.counters()[0].tolist()
        c = [a + v for a, v in zip(c, cs)]
        if reset:
            b.route.state.zero_()
    uses = c[1]
    out = {"decode_steps": c[0], "expert_uses": uses, "unique_layer_experts": c[7]}
    for i, w in enumerate((1, 2, 4, 8, 16)):
        out[f"reuse_{w}"] = c[2 + i]
    out["reuse_rates"] = {str(w): round(out[f"reuse_{w}"] / max(uses, 1), 4) for w in (1, 2, 4, 8, 16)}
    return out


class ExpertStore:
    """Where one layer's routed experts live: a device pointer table plus the shape, and the
    layer's call book (counters, route telemetry, status poll)."""

    def __init__(self, shape: MoEShape, table: torch.Tensor, device, keepalive=(), **book):
        self.shape, self.table = shape, table
        self.workspace = Workspace(shape, device)
        self._keepalive = tuple(keepalive)   # tensors the table points into
        self.book = _CallBook(shape, self.workspace, device, **book)

    @classmethod
    def from_slabs(cls, shape, gate_up, down, **book):
        for name, t in (("gate_up", gate_up), ("down", down)):
            if t.dtype != ENGINE_DTYPE:
                raise TypeError(f"{name} experts must be {ENGINE_DTYPE}, got {t.dtype}")
        return cls(shape, expert_table(gate_up, down), gate_up.device, keepalive=(gate_up, down), **book)

    @classmethod
    def from_int4(cls, shape, gate_up_q, gate_up_s, down_q, down_s, **book):
        """Int4 experts (labelled fast mode): packed [E,2I,H/2] / [E,H,I/2] u8, group scales bf16."""
        ts = (gate_up_q, gate_up_s, down_q, down_s)
        return cls(shape, expert_table_q4(*ts), gate_up_q.device, keepalive=ts, **book)

    @classmethod
    def from_int4_rows(cls, shape, gate_up_q, gate_up_s, down_q, down_s, **book):
        """Int4 experts in the reference's own layout: packed as above, ONE fp16 scale per
        row (gate_up_s [E,2I], down_s [E,H]; tarfa/engine/channel_q4.py:10-14)."""
        ts = (gate_up_q, gate_up_s, down_q, down_s)
        return cls(shape, expert_table_q4_rows(*ts), gate_up_q.device, keepalive=ts, **book)

    @classmethod
    def from_int4_file(cls, shape, path, device, **book):
        """One layer file of the reference's int4 experts (channel_q4.py:18, 28-38), all of
        its experts loaded into HBM."""
        f = Int4LayerFile(path)
        if (f.hidden, f.intermediate, f.num_experts) != (shape.hidden, shape.intermediate, shape.num_experts):
            raise ValueError(f"{path}: H={f.hidden} I={f.intermediate} E={f.num_experts} does not match {shape}")
        return cls.from_int4_rows(shape, *f.load(device), **book)

    @property
    def int4(self):
        return self.table.shape[1] == 4

    def check_status(self):
        self.book.check_status()


def engine_jtopk():
    """The reference engine's JTOPK: experts run per token (environment, default 8;
    tarfa/engine/fused_int4.py:17)."""
    return int(os.environ.get("JTOPK", "8"))


def make_experts_forward(store: ExpertStore, jtopk=None):
    """The forward(self, hidden_states, top_k_index, top_k_weights) to bind on an experts module.
    A routing with more than ``jtopk`` experts per token (default: engine_jtopk()) is first cut
    to its jtopk largest weights and renormalised, as the reference does (fused_int4.py:157-160)."""
    jtopk = engine_jtopk() if jtopk is None else int(jtopk)
    if jtopk < 1:
        raise ValueError(f"JTOPK must be at least 1, got {jtopk}")

    def forward(self, hidden_states, top_k_index, top_k_weights):
        # Returns a new tensor and mutates no input (fused_int4.py:161).  T == 1 accumulates
        # in router order, T > 1 in ascending expert id, as the reference does.
        if hidden_states.dtype != ENGINE_DTYPE:
            raise TypeError(f"libtmoe experts compute in {ENGINE_DTYPE}; hidden_states is {hidden_states.dtype} "
                            "(build the engine with dtype=torch.bfloat16)")
        x = hidden_states.contiguous()
        ids = top_k_index.contiguous()
        w = top_k_weights.to(ENGINE_DTYPE).contiguous()
        shape = store.shape
        if w.shape[-1] > jtopk:
            ids, w = topk_renorm(ids, w, jtopk)
        if ids.shape[-1] != shape.top_k:
            shape = dataclasses.replace(shape, top_k=ids.shape[-1])
        decode = x.shape[0] == 1
        return store.book.call("decode" if decode else "prefill",
                               lambda: experts_forward(shape, x, ids, w, store.table, store.workspace),
                               record_ids=ids if decode else None)

    return forward


def _check_silu(experts):
    act = getattr(experts, "act_fn", None)
    if act is not None and not isinstance(act, torch.nn.SiLU) and type(act).__name__ not in ("SiLU", "SiLUActivation"):
        raise ValueError(f"libtmoe computes SwiGLU with SiLU; this module uses {type(act).__name__}")


def _check_dtype(module, what):
    for name, p in list(module.named_parameters(recurse=False)) + list(module.named_buffers(recurse=False)):
        if p.is_floating_point() and p.dtype != ENGINE_DTYPE:
            raise TypeError(f"{what} parameter {name} is {p.dtype}; libtmoe computes in {ENGINE_DTYPE}, so the "
                            "engine must be built with dtype=torch.bfloat16")


def install_experts(experts, store: ExpertStore, jtopk=None):
    """Bind the libtmoe routed-compute step on an experts module instance (fused_int4.py:262);
    ``jtopk`` as in make_experts_forward."""
    _check_silu(experts)
    _check_dtype(experts, "experts")
    for name in ("gate_up_proj", "down_proj"):
        experts._parameters.pop(name, None)
    experts.forward = types.MethodType(make_experts_forward(store, jtopk), experts)
    experts._tmoe_store = store
    return experts


class TmoeSparseMoeBlock(torch.nn.Module):
    """Router (fp32 logits) + routed experts + shared expert + combine on libtmoe."""

    def __init__(self, shape: MoEShape, router_w, store: ExpertStore, shared=None, heat=None):
        super().__init__()
        self.shape, self.router_w, self.store, self.shared, self.heat = shape, router_w, store, shared, heat
        self.last_ids = self.last_weights = None

    def forward(self, hidden_states, logits=None):
        if hidden_states.dtype != ENGINE_DTYPE:
            raise TypeError(f"libtmoe computes in {ENGINE_DTYPE}; hidden_states is {hidden_states.dtype}")
        B, S, H = hidden_states.shape
        x = hidden_states.reshape(-1, H).contiguous()
        decode = x.shape[0] == 1
        res = {}

        def run():
            res["v"] = moe_block(self.shape, x, self.store.table, self.store.workspace, router_w=self.router_w,
                                 logits=logits, shared=self.shared, heat=self.heat)

        # The routing exists only after the launch, so the route is recorded right after it.
        self.store.book.call("decode" if decode else "prefill", run)
        out, ids, w = res["v"]
        if decode and self.store.book.route is not None:
            self.store.book.route.record(ids)
        self.last_ids, self.last_weights = ids, w
        return out.reshape(B, S, H)


def from_transformers_block(block, device=None, **book):
    """Build a TmoeSparseMoeBlock from a bf16 transformers Qwen3_5MoeSparseMoeBlock (weights copied)."""
    dev = torch.device(device or "cuda")
    ex = block.experts
    _check_silu(ex)
    for mod, what in ((ex, "experts"), (block.gate, "router"), (block.shared_expert.gate_proj, "shared gate_proj"),
                      (block.shared_expert.up_proj, "shared up_proj"), (block.shared_expert.down_proj,
                                                                        "shared down_proj"),
                      (block.shared_expert_gate, "shared_expert_gate")):
        _check_dtype(mod, what)
    gu = ex.gate_up_proj.detach().to(dev).contiguous()
    dn = ex.down_proj.detach().to(dev).contiguous()
    E, I2, H = gu.shape
    sh = block.shared_expert
    Is = sh.gate_proj.weight.shape[0]
    shape = MoEShape(H, E, I2 // 2, block.gate.top_k, Is)
    shared = tuple(t.detach().to(dev).contiguous()
                   for t in (sh.gate_proj.weight, sh.up_proj.weight, sh.down_proj.weight,
                             block.shared_expert_gate.weight.reshape(-1)))
    rw = block.gate.weight.detach().to(dev).contiguous()
    return TmoeSparseMoeBlock(shape, rw, ExpertStore.from_slabs(shape, gu, dn, **book), shared)
