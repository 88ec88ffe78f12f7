"""Expert residency ledger: where every (layer, expert) lives on one GPU, and the
device pointer tables the decode and prefill kernels read.

The reference decides *where* expert bytes come from (GPU cache -> RAM -> NVMe),
never *which* bytes: tarfa/engine/exact_bf16.py:118-193 (read_bf16: pinned
staging buffers, host-to-device copies on the current stream), :15-61
(ExpertArena, a RAM cache it rejected), fused_int4.py:171-178, 195-200 (per-layer
GPU LRU of bf16 experts), channel_q4.py:8, 100-129 (int4 LRU with a ``_pinned``
protection hook), fused_int4.py:110-144 (side-stream prefetch), and the hotlist
of format/JNF_V1.md:40-45 (per-layer expert counts and predicted coverage).

On MI355X the whole BF16 expert set of a 48-layer H=2560 model (194 GB) fits in
one GPU's 288 GB of HBM, so the ledger's main mode keeps every expert resident:
one slab pair per layer, tables [L, E, parts] of device pointers that never
change, and no per-layer host work at all.  For models larger than HBM the
tiered mode keeps ``hbm_slots`` experts per layer in HBM and every expert in
pinned host memory; a table entry points at the HBM slot or at the pinned host
copy, which the kernels read directly over the host link (slower, same bytes),
so routing never waits for a copy.  ``promote`` moves experts into HBM slots with
asynchronous copies on a side stream (after the work already queued on the
compute stream, so no queued kernel reads a slot being overwritten), then
switches their table rows; ``table(layer)`` makes the compute stream wait on that
stream's event before the layer's next call.

``load_jnf`` fills either mode from the reference's on-disk format (JNF v1, verified by
SHA-256 as it is read; tarfa_amd.jnf).

Heat: the fused router kernel adds 1 to heat[l, e] for every selection (device
atomics, no host sync).  ``hotlist`` turns a heat snapshot into the reference's
hotlist fields (per-layer counts and predicted coverage for 1, 2, 4, 8 slots).
"""
import dataclasses
import math

import torch

from . import seeded
from ._lib import check, lib
from .moe import MoEShape, quantize_int4


def part_shapes(shape: MoEShape, int4: bool):
    """Per-expert (shape, dtype) of each part, in table column order."""
    H, I, G = shape.hidden, shape.intermediate, shape.group_size
    if not int4:
        return [((2 * I, H), torch.bfloat16), ((H, I), torch.bfloat16)]
    return [((2 * I, H // 2), torch.uint8), ((2 * I, H // G), torch.bfloat16),
            ((H, I // 2), torch.uint8), ((H, I // G), torch.bfloat16)]


def expert_bytes(shape: MoEShape, int4=False):
    return sum(math.prod(s) * torch.empty(0, dtype=d).element_size() for s, d in part_shapes(shape, int4))


@dataclasses.dataclass
class LayerWeights:
    """The non-expert weights of one MoE layer the block kernels read."""
    router_w: torch.Tensor            # [E, H] bf16
    shared: tuple = None              # (gate [Is,H], up [Is,H], down [H,Is], gate_w [H]) or None


def _ptr_rows(parts, n):
    """Host int64 [n, len(parts)] of per-expert base pointers of [n, ...] tensors."""
    cols = []
    for t in parts:
        stride = t.stride(0) * t.element_size()
        cols.append(torch.arange(n, dtype=torch.int64) * stride + t.data_ptr())
    return torch.stack(cols, dim=1)


class ResidencyLedger:
    """Placement of the routed experts of ``n_layers`` layers on one device.

    ``hbm_slots`` = None keeps every expert in HBM.  Otherwise each layer keeps
    ``hbm_slots`` experts in HBM slots and all E in pinned host memory.
    """

    def __init__(self, shape: MoEShape, n_layers, device="cuda", int4=False, hbm_slots=None):
        self.shape, self.L, self.int4 = shape, int(n_layers), bool(int4)
        self.device = torch.device(device)
        E = shape.num_experts
        self.specs = part_shapes(shape, self.int4)
        self.tiered = hbm_slots is not None and hbm_slots < E
        self.S = E if not self.tiered else int(hbm_slots)
        if self.tiered and self.S < 1:
            raise ValueError("hbm_slots must be at least 1")
        dev = self.device
        # HBM storage: one [S, ...] tensor per part per layer.
        self.hbm = [[torch.empty(self.S, *s, dtype=d, device=dev) for s, d in self.specs] for _ in range(self.L)]
        self.host = None
        if self.tiered:
            self.host = [[torch.empty(E, *s, dtype=d, pin_memory=True) for s, d in self.specs]
                         for _ in range(self.L)]
        self.heat = torch.zeros(self.L, E, dtype=torch.int32, device=dev)
        self.tables = torch.empty(self.L, E, len(self.specs), dtype=torch.int64, device=dev)
        # slot bookkeeping (host): expert -> slot and slot -> expert per layer
        self.slot_of = [dict() for _ in range(self.L)]
        self.in_slot = [[-1] * self.S for _ in range(self.L)]
        self._side = None
        self._pending = [None] * self.L
        self.stats = {"promotions": 0, "evictions": 0, "bytes_promoted": 0}
        self._keep_rows = [None] * self.L
        # Initial placement: experts 0 .. S-1 in the HBM slots of every layer.
        for l in range(self.L):
            self.slot_of[l] = {e: e for e in range(self.S)}
            self.in_slot[l] = list(range(self.S))
        self._write_all_tables()

    # ------------------------------------------------------------------ tables
    def _row_host(self, l):
        """Host table of layer l from the bookkeeping: HBM slot or pinned host copy."""
        E = self.shape.num_experts
        hbm = _ptr_rows(self.hbm[l], self.S)
        if not self.tiered:
            return hbm
        rows = _ptr_rows(self.host[l], E)
        for e, s in self.slot_of[l].items():
            rows[e] = hbm[s]
        return rows

    def _write_all_tables(self):
        host = torch.stack([self._row_host(l) for l in range(self.L)])
        self.tables.copy_(host)

    def table(self, layer, stream=None):
        """[E, parts] device table of ``layer``; the stream waits for pending promotions of it."""
        ev = self._pending[layer]
        if ev is not None:
            (stream or torch.cuda.current_stream(self.device)).wait_event(ev)
        return self.tables[layer]

    def location(self, layer, expert):
        """'hbm' or 'host' (bookkeeping view)."""
        return "hbm" if expert in self.slot_of[layer] else "host"

    # ------------------------------------------------------------------ filling
    def fill_seeded(self, seed):
        """Write the seeded experts of every layer (tarfa_amd.seeded streams), quantised for int4."""
        E, dev = self.shape.num_experts, self.device
        H, I = self.shape.hidden, self.shape.intermediate
        chunk = 16
        for l in range(self.L):
            if not self.tiered and not self.int4:
                seeded.fill_expert_slabs(self.hbm[l][0], self.hbm[l][1], seed, l)   # straight into the slabs
                continue
            for e0 in range(0, E, chunk):
                n = min(chunk, E - e0)
                gu = torch.empty(n, 2 * I, H, dtype=torch.bfloat16, device=dev)
                dn = torch.empty(n, H, I, dtype=torch.bfloat16, device=dev)
                seeded.fill_expert_slabs(gu, dn, seed, l, first_expert=e0)
                parts = [gu, dn] if not self.int4 else [*quantize_int4(gu, self.shape.group_size),
                                                        *quantize_int4(dn, self.shape.group_size)]
                self._store(l, e0, parts)
        torch.cuda.synchronize(dev)

    @classmethod
    def quantized_from(cls, src: "ResidencyLedger"):
        """A fully resident int4 ledger holding the group-quantised experts of a resident bf16 ledger."""
        if src.int4 or src.tiered:
            raise ValueError("quantise from a fully resident bf16 ledger")
        q = cls(src.shape, src.L, src.device, int4=True)
        g = src.shape.group_size
        for l in range(src.L):
            for dst, part in zip(q.hbm[l], (*quantize_int4(src.hbm[l][0], g), *quantize_int4(src.hbm[l][1], g))):
                dst.copy_(part)
        torch.cuda.synchronize(src.device)
        return q

    def load_layer(self, layer, parts):
        """Copy a layer's experts from full tensors ([E, ...] per part, any device)."""
        if self.tiered:
            torch.cuda.synchronize(self.device)      # the host tier is written by the CPU: no kernel may be reading it
        self._store(layer, 0, [p.to(self.device) if not self.tiered else p for p in parts])
        torch.cuda.synchronize(self.device)

    def load_jnf(self, jnf, layers=None, verify=True, chunk=16):
        """Fill the ledger from a JNF v1 tree (``tarfa_amd.jnf.JnfModel``); layer l of the ledger
        takes JNF layer ``layers[l]`` (default: the same index).  Every expert's SHA-256 is
        checked as it is read (``verify``).

        Resident mode: experts go through two pinned staging buffers of ``chunk`` experts --
        while one buffer's copy to HBM runs on the side stream, the next chunk is read into the
        other (the reference's read_bf16 path, exact_bf16.py:163-193, with the copy overlapped).
        Tiered mode: the file is read straight into the pinned host tier the kernels read
        non-resident experts from; the experts already assigned HBM slots are then copied in on
        the side stream, and ``table(layer)`` orders the next call after them."""
        if self.int4:
            raise ValueError("JNF holds bf16 experts; fill an int4 ledger from a bf16 one (quantized_from)")
        E, dev = self.shape.num_experts, self.device
        src = list(range(self.L)) if layers is None else [int(l) for l in layers]
        if len(src) != self.L:
            raise ValueError(f"{len(src)} JNF layers for a ledger of {self.L}")
        for l, jl in enumerate(src):
            ly = jnf.layers.get(jl)
            if ly is None or (ly.num_experts, ly.hidden, ly.intermediate) != (E, self.shape.hidden,
                                                                             self.shape.intermediate):
                raise ValueError(f"JNF layer {jl} missing or not of shape {self.shape}")
        side = self._side_stream()
        side.wait_stream(torch.cuda.current_stream(dev))
        if self.tiered:
            # The CPU writes the pinned host tier directly, and kernels already queued on any
            # stream may still read it (non-resident experts), as may an earlier side-stream
            # copy into the HBM slots: wait for all of them before the first write.
            torch.cuda.synchronize(dev)
            for l, jl in enumerate(src):
                jnf.read_experts(jl, range(E), self.host[l][0], self.host[l][1], verify=verify)
                with torch.cuda.stream(side):
                    for e, sl in self.slot_of[l].items():
                        for dst, h in zip(self.hbm[l], self.host[l]):
                            dst[sl].copy_(h[e], non_blocking=True)
                    ev = torch.cuda.Event()
                    ev.record(side)
                self._pending[l] = ev
            return
        n = min(chunk, E)
        stage = [[torch.empty(n, *sh, dtype=dt, pin_memory=True) for sh, dt in self.specs] for _ in range(2)]
        done = [None, None]
        k = 0
        for l, jl in enumerate(src):
            for e0 in range(0, E, n):
                m = min(n, E - e0)
                b = k % 2
                if done[b] is not None:
                    done[b].synchronize()            # the copy that last read this buffer has finished
                jnf.read_experts(jl, range(e0, e0 + m), stage[b][0], stage[b][1], verify=verify)
                with torch.cuda.stream(side):
                    for dst, st in zip(self.hbm[l], stage[b]):
                        dst[e0:e0 + m].copy_(st[:m], non_blocking=True)
                    ev = torch.cuda.Event()
                    ev.record(side)
                done[b] = ev
                k += 1
        for ev in done:
            if ev is not None:
                ev.synchronize()

    def _store(self, l, e0, parts):
        n = parts[0].shape[0]
        if self.tiered:
            for dst, src in zip(self.host[l], parts):
                dst[e0:e0 + n].copy_(src)
            for e in range(e0, e0 + n):
                s = self.slot_of[l].get(e)
                if s is not None:
                    for dst, src in zip(self.hbm[l], parts):
                        dst[s].copy_(src[e - e0])
        else:
            for dst, src in zip(self.hbm[l], parts):
                dst[e0:e0 + n].copy_(src)

    # ------------------------------------------------------------------ tiered mode
    def _side_stream(self):
        if self._side is None:
            self._side = torch.cuda.Stream(self.device)
        return self._side

    def promote(self, layer, experts, protect=()):
        """Move ``experts`` of ``layer`` into HBM slots (tiered mode), evicting the slots whose
        experts are coldest by the last heat snapshot and not in ``protect`` or ``experts``.

        Copies run on a side stream after all work already queued on the current stream
        (a slot is never overwritten while a queued kernel may still read it); the
        table rows switch after the copies; ``table(layer)`` makes the next user wait.
        """
        if not self.tiered:
            return []
        want = [int(e) for e in dict.fromkeys(int(e) for e in experts) if int(e) not in self.slot_of[layer]]
        if not want:
            return []
        keep = set(int(e) for e in protect) | set(int(e) for e in experts)
        heat = self._heat_host[layer] if getattr(self, "_heat_host", None) is not None else None
        free = [s for s in range(self.S) if self.in_slot[layer][s] < 0]
        victims = sorted((s for s in range(self.S) if self.in_slot[layer][s] >= 0
                          and self.in_slot[layer][s] not in keep),
                         key=lambda s: (int(heat[self.in_slot[layer][s]]) if heat is not None else 0, s))
        plan = []
        for e in want:
            if free:
                s = free.pop(0)
            elif victims:
                s = victims.pop(0)
            else:
                break
            plan.append((e, s))
        if not plan:
            return []
        cur = torch.cuda.current_stream(self.device)
        side = self._side_stream()
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            for e, s in plan:
                old = self.in_slot[layer][s]
                if old >= 0:
                    del self.slot_of[layer][old]
                    self.stats["evictions"] += 1
                for dst, src in zip(self.hbm[layer], self.host[layer]):
                    dst[s].copy_(src[e], non_blocking=True)
                self.in_slot[layer][s] = e
                self.slot_of[layer][e] = s
                self.stats["promotions"] += 1
                self.stats["bytes_promoted"] += sum(t[s].numel() * t.element_size() for t in self.hbm[layer])
            rows = self._row_host(layer).pin_memory()
            self.tables[layer].copy_(rows, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(side)
        self._pending[layer] = ev
        self._keep_rows[layer] = rows     # the pinned source outlives its asynchronous copy
        return plan

    def snapshot_heat(self):
        """Host copy of the heat counters (one synchronisation), used by promote/rebalance."""
        self._heat_host = self.heat.cpu()
        return self._heat_host

    def rebalance(self):
        """Tiered mode: per layer, move the hottest experts (by a fresh heat snapshot) into HBM."""
        if not self.tiered:
            return 0
        heat = self.snapshot_heat()
        moved = 0
        for l in range(self.L):
            order = torch.argsort(heat[l], descending=True, stable=True)[:self.S].tolist()
            hot = [e for e in order if heat[l, e] > 0]
            moved += len(self.promote(l, hot, protect=hot))
        return moved

    # ------------------------------------------------------------------ heat / hotlist
    def hotlist(self, budgets=(1, 2, 4, 8)):
        """Per layer: expert counts (descending) and predicted coverage for each budget of
        resident experts (format/JNF_V1.md:40-45)."""
        heat = self.snapshot_heat()
        out = {"selections": int(heat.sum().item()), "layers": []}
        for l in range(self.L):
            h = heat[l]
            tot = int(h.sum())
            order = torch.argsort(h, descending=True, stable=True)
            counts = [(int(e), int(h[e])) for e in order.tolist() if h[e] > 0]
            cov = {str(b): round(sum(c for _, c in counts[:b]) / tot, 4) if tot else 0.0 for b in budgets}
            out["layers"].append({"layer": l, "counts": counts, "coverage": cov})
        return out


class RouteTelemetry:
    """Device-side route-reuse telemetry for L layers (tmoe_route_record); see routing_telemetry()."""

    def __init__(self, n_layers, top_k, num_experts, device="cuda"):
        self.L, self.k, self.E = n_layers, top_k, num_experts
        n = lib().tmoe_route_telemetry_bytes(n_layers, top_k, num_experts)
        if n == 0:
            raise ValueError("unsupported telemetry shape")
        self.state = torch.zeros(n, dtype=torch.uint8, device=device)
        self.ids = torch.full((n_layers, top_k), num_experts, dtype=torch.int64, device=device)

    def record(self, ids=None):
        """Record one token's routing for every layer (ids [L, k] int64 on the device)."""
        ids = self.ids if ids is None else ids
        st = lib().tmoe_route_record(ids.data_ptr(), self.L, self.k, self.E, self.state.data_ptr(),
                                     self.state.numel(), torch.cuda.current_stream(ids.device).cuda_stream)
        check(st, "tmoe_route_record")

    def counters(self):
        """[L, 8] host uint64 (steps, uses, reuse_1, 2, 4, 8, 16, distinct); one synchronisation."""
        return self.state[:self.L * 64].cpu().view(torch.int64).reshape(self.L, 8)

    def routing_telemetry(self):
        """The reference's routing_telemetry() fields (fused_int4.py:86-95), summed over layers."""
        c = self.counters().sum(0).tolist()
        uses = c[1]
        out = {"decode_steps": c[0], "expert_uses": uses, "unique_layer_experts": c[7]}
        for i, w in enumerate((1, 2, 4, 8, 16)):
            out[f"reuse_{w}"] = c[2 + i]
        out["reuse_rates"] = {str(w): round(out[f"reuse_{w}"] / max(uses, 1), 4) for w in (1, 2, 4, 8, 16)}
        return out


def zipf_logits(shape: MoEShape, n_layers, tokens, seed, s=1.1, device="cuda"):
    """Router logits [tokens, L, E] fp32 whose top-k follows Zipf(s) expert popularity per layer:
    logit = log(w(rank_l(e))) + Gumbel, w(r) = (r + 1)^-s, rank_l a seeded per-layer permutation.
    Gumbel-top-k of these logits samples k experts without replacement with probabilities
    proportional to w."""
    E = shape.num_experts
    g = torch.Generator().manual_seed(int(seed))
    ranks = torch.stack([torch.randperm(E, generator=g) for _ in range(n_layers)])          # [L, E]
    logw = -s * torch.log(ranks.double() + 1.0)
    u = torch.rand(tokens, n_layers, E, generator=g, dtype=torch.float64).clamp_(1e-300, 1.0)
    gum = -torch.log(-torch.log(u))
    return (logw[None] + gum).float().to(device), ranks
