"""Batch-1 decode through a stack of MoE layers (MoE blocks only) on one GPU.

Each token runs the L layers' MoE blocks back to back on one stream: router
(fp32 logits, or supplied logits), routed experts through the residency
ledger's tables, shared expert, combine -- one fused kernel launch per layer,
with the expert ids never leaving the device.  The block output of layer l is
the block input of layer l + 1 (the attention and norm steps between MoE
blocks are outside this path).  After the L layers, one launch records the
token's routing into the device-side route telemetry.

The per-layer arguments are built once (device pointers are stable), so a
token costs L + 1 C calls on the host and no synchronisation.
"""
import torch

from ._lib import check, lib
from .moe import MoEShape, Workspace, _need
from .residency import LayerWeights, ResidencyLedger, RouteTelemetry


class MoEStack:
    def __init__(self, ledger: ResidencyLedger, layers, telemetry=True, count_heat=True):
        """``layers``: one LayerWeights per ledger layer (router and shared expert weights)."""
        if len(layers) != ledger.L:
            raise ValueError("one LayerWeights per ledger layer")
        self.ledger, self.layers = ledger, list(layers)
        self.shape: MoEShape = ledger.shape
        s, dev = self.shape, ledger.device
        self.device = dev
        self.ws = Workspace(s, dev)
        self.buf = [torch.empty(1, s.hidden, dtype=torch.bfloat16, device=dev) for _ in range(2)]
        self.weights = torch.empty(ledger.L, s.top_k, dtype=torch.bfloat16, device=dev)
        self.telemetry = RouteTelemetry(ledger.L, s.top_k, s.num_experts, dev) if telemetry else None
        self.ids = (self.telemetry.ids if telemetry else
                    torch.empty(ledger.L, s.top_k, dtype=torch.int64, device=dev))
        self.count_heat = count_heat
        self._fn = lib().tmoe_moe_block_int4 if ledger.int4 else lib().tmoe_moe_block_bf16
        for lw in self.layers:
            _need(lw.router_w, "router_w", torch.bfloat16, (s.num_experts, s.hidden), dev)
            if (lw.shared is None) != (s.shared_intermediate == 0):
                raise ValueError("shared weights must match shape.shared_intermediate")

    def _args(self, l, x, out, logits, stream):
        s, lw = self.shape, self.layers[l]
        sh = [t.data_ptr() for t in lw.shared] if lw.shared is not None else [None] * 4
        table = self.ledger.table(l)
        heat = self.ledger.heat[l].data_ptr() if self.count_heat else None
        return (x.data_ptr(), 1, None if logits is not None else lw.router_w.data_ptr(),
                None if logits is None else logits.data_ptr(), table.data_ptr(), *sh, s.hidden, s.num_experts,
                s.intermediate, s.top_k, s.shared_intermediate, out.data_ptr(), self.ids[l].data_ptr(),
                self.weights[l].data_ptr(), heat, self.ws.buf.data_ptr(), self.ws.buf.numel(), stream)

    def decode(self, x, logits=None, per_layer_out=None):
        """One token through every layer.  x [1, H] bf16; logits None (computed by each
        layer's router) or [L, E] fp32 (one row per layer).  Returns the last block output
        (a view of an internal buffer, valid until the next call)."""
        s = self.shape
        _need(x, "x", torch.bfloat16, (1, s.hidden), self.device)
        if logits is not None:
            _need(logits, "logits", torch.float32, (self.ledger.L, s.num_experts), self.device)
        stream = torch.cuda.current_stream(self.device).cuda_stream
        cur = x
        for l in range(self.ledger.L):
            out = self.buf[l % 2]
            st = self._fn(*self._args(l, cur, out, None if logits is None else logits[l], stream))
            check(st, "moe block")
            if per_layer_out is not None:
                per_layer_out.append(out.clone())
            cur = out
        if self.telemetry is not None:
            self.telemetry.record()
        return cur

    def status(self):
        """Synchronise and raise on a device-detected error."""
        self.ws.status()
