"""Per-task timeline of the fused batch-1 decode kernel (a debug view of one call).

`DecodeTrace` switches the library's debug recording on (`tmoe_debug_decode_trace`), and
`summarize` turns the records of the last fused-decode launch into phases: for each task
group (router rows R, shared gate/up S, shared down SD, gate/up Gj and down Dj of routed
slot j) when its tasks started, when their loads returned and when they ended, the steps
of each block's routing resolution (logits seen, top-k selected, weights formed), plus the
weight bytes each 1 us bin of the call delivered (each task's bytes spread evenly from the
issue of its loads -- its start, or the moment its wave knew the routing -- to their return).  Times are microseconds after the first wave's entry
(s_memrealtime runs at 100 MHz: 10 ns resolution).

The reference has no counterpart: it times the whole decode call by wall clock
(tarfa/engine/fused_int4.py:164, 203-204).
"""
import numpy as np
import torch

from ._lib import check, lib

TICK_US = 0.01
HEADER = 16
TASK_WORDS = 8
DOWN_ROWS = 8


class DecodeTrace:
    """Context manager: fused-decode launches inside it record their timeline into a device
    buffer; `records()` copies the last launch's records to the host."""

    def __init__(self, device, nbytes=8 << 20):
        self.buf = torch.zeros(nbytes // 8, dtype=torch.int64, device=device)

    def __enter__(self):
        check(lib().tmoe_debug_decode_trace(self.buf.data_ptr(), self.buf.numel() * 8), "tmoe_debug_decode_trace")
        return self

    def __exit__(self, *exc):
        check(lib().tmoe_debug_decode_trace(None, 0), "tmoe_debug_decode_trace")
        return False

    def records(self):
        torch.cuda.synchronize()
        return self.buf.cpu().numpy().view(np.uint64).copy()


def task_bytes(kind, H, I, Is, E, q4):
    """Weight bytes one task of this kind reads (the fused kernel's task sizes)."""
    if kind == "R":
        return 4 * H * 2
    if kind == "S":
        return (8 if q4 else 4) * H * 2
    if kind == "SD":
        return DOWN_ROWS * Is * 2
    if kind == "G":
        return 8 * (H // 2 + H // 64) if q4 else 4 * H * 2
    rows = (16 if I <= 1024 else 8) if q4 else DOWN_ROWS
    return rows * (I // 2 + I // 64) if q4 else rows * I * 2


KINDS = {0: "R", 2: "S", 3: "SD", 4: "G", 5: "D"}


def summarize(rec, H, I, Is, E):
    """Phases of one traced call: a dict with the per-group table and the bandwidth bins."""
    hdr = rec[:HEADER].astype(np.int64)
    n_tasks, grid = int(hdr[0]), int(hdr[1])
    q4 = bool(hdr[11])
    t = rec[HEADER:HEADER + n_tasks * TASK_WORDS].reshape(n_tasks, TASK_WORDS).astype(np.int64)
    w = rec[HEADER + n_tasks * TASK_WORDS:HEADER + n_tasks * TASK_WORDS + grid * 4 * 2].reshape(-1, 2).astype(np.int64)
    # Each record names its task (type | (slot + 1) << 8 | idx << 16); in the XCD-slot mode's
    # per-XCD lists some record slots stay unused (start 0).
    used = t[:, 0] > 0
    t = t[used]
    ident = t[:, 7]
    tasks = [(KINDS[int(v & 0xFF)], int((v >> 8) & 0xFF) - 1 if KINDS[int(v & 0xFF)] in ("G", "D") else -1,
              int(v >> 16)) for v in ident]
    t0 = int(w[:, 0].min())
    us = lambda v: (v - t0) * TICK_US  # noqa: E731
    start, route, take, end = (us(t[:, i]) for i in range(4))
    take = np.where(t[:, 2] > 0, take, end)
    groups = {}
    for i, (kind, slot, _) in enumerate(tasks):
        groups.setdefault(kind if slot < 0 else f"{kind}{slot}", []).append(i)
    rows = []
    for name, idx in groups.items():
        idx = np.asarray(idx)
        r = route[idx][t[idx, 1] > 0]
        rows.append({
            "group": name, "tasks": int(idx.size),
            "start_first": float(start[idx].min()), "start_med": float(np.median(start[idx])),
            "start_last": float(start[idx].max()),
            "route_first": float(r.min()) if r.size else None, "route_last": float(r.max()) if r.size else None,
            "loads_med": float(np.median(take[idx] - start[idx])),
            "end_med": float(np.median(end[idx])), "end_last": float(end[idx].max()),
        })
    total = float(us(w[:, 1]).max())
    bins = np.zeros(int(np.ceil(total)) + 1)
    for i, (kind, _, _) in enumerate(tasks):
        b = task_bytes(kind, H, I, Is, E, q4)
        a = max(start[i], route[i]) if t[i, 1] > 0 else start[i]   # loads issue once the routing is known
        z = max(take[i], a + 1e-3)
        lo, hi = int(a), int(z)
        for k in range(lo, hi + 1):
            ov = min(z, k + 1) - max(a, k)
            if ov > 0:
                bins[k] += b * ov / (z - a)
    # Routing, per block that resolved it: poll start, all logits seen, top-k selected,
    # weights formed, route words in LDS.
    off = HEADER + n_tasks * TASK_WORDS + grid * 4 * 2
    b = rec[off:off + grid * 8].reshape(-1, 8).astype(np.int64)
    b = b[b[:, 0] > 0]
    routing = None
    if b.size:
        med = lambda c: float(np.median(us(b[:, c])))  # noqa: E731
        polled = bool((b[:, 1] > 0).all())   # no poll (and no stamp) when the logits are supplied
        routing = {"blocks": int(len(b)), "poll_start_med": med(0),
                   "logits_seen_med": med(1) if polled else None,
                   "logits_seen_first": float(us(b[:, 1]).min()) if polled else None, "selected_med": med(4),
                   "weights_med": med(5), "resolved_med": med(2), "resolved_first": float(us(b[:, 2]).min()),
                   "poll_rounds_med": float(np.median(b[:, 3]))}
    return {"total_us": total, "waves": int(grid * 4), "entry_last_us": float(us(w[:, 0]).max()),
            "groups": rows, "gbps_per_us": (bins / 1e3).tolist(), "routing": routing}


def format_summary(s):
    """Text table of a summary (one line per task group, then the bandwidth bins)."""
    out = [f"call {s['total_us']:.2f} us, {s['waves']} waves, last wave entered at {s['entry_last_us']:.2f} us",
           f"{'group':>6} {'tasks':>6} {'start first/med/last':>22} {'routing known':>15} "
           f"{'loads med':>9} {'end med/last':>14}"]
    for r in s["groups"]:
        rt = f"{r['route_first']:.2f}/{r['route_last']:.2f}" if r["route_first"] is not None else "-"
        out.append(f"{r['group']:>6} {r['tasks']:>6} {r['start_first']:>6.2f} {r['start_med']:>6.2f} "
                   f"{r['start_last']:>6.2f}   {rt:>15} {r['loads_med']:>9.2f} {r['end_med']:>6.2f} "
                   f"{r['end_last']:>6.2f}")
    r = s.get("routing")
    if r:
        seen = (f"logits seen {r['logits_seen_med']:.2f} (first {r['logits_seen_first']:.2f})"
                if r["logits_seen_med"] is not None else "logits supplied")
        out.append(f"routing ({r['blocks']} blocks, medians): poll start {r['poll_start_med']:.2f}, {seen}, top-k selected "
                   f"{r['selected_med']:.2f}, weights {r['weights_med']:.2f}, resolved {r['resolved_med']:.2f} "
                   f"(first {r['resolved_first']:.2f}), poll rounds {r['poll_rounds_med']:.0f}")
    out.append("weight GB/s per 1 us bin: " + " ".join(f"{v:.0f}" for v in s["gbps_per_us"]))
    return "\n".join(out)


def main(argv=None):
    """Trace the full-size layer (H=2560, E=256, I=1024, k=8, shared Is=1024) at batch 1:
    warm up over a rotation of seeded layers, then print the timeline of the last of
    `--calls` traced back-to-back calls, `--reps` times."""
    import argparse

    from . import seeded
    from .moe import MoEShape, Workspace
    from .residency import LayerWeights, ResidencyLedger

    ap = argparse.ArgumentParser(prog="python -m tarfa_amd.timeline")
    ap.add_argument("--mode", choices=["bf16", "int4"], default="bf16")
    ap.add_argument("--layers", type=int, default=12, help="seeded layers rotated (4 GB of experts each)")
    ap.add_argument("--calls", type=int, default=40)
    ap.add_argument("--reps", type=int, default=3)
    ap.add_argument("--logits", action="store_true",
                    help="supply each call a seeded router-logits row (as the 48-layer stack does)")
    a = ap.parse_args(argv)
    dev = torch.device("cuda:0")
    shape = MoEShape(2560, 256, 1024, 8, 1024)
    ledger = ResidencyLedger(shape, a.layers, dev)
    ledger.fill_seeded(1)
    tables = ledger.tables if a.mode == "bf16" else ResidencyLedger.quantized_from(ledger).tables
    layers = [LayerWeights(*seeded.make_block_weights(shape, 1, l, dev)) for l in range(a.layers)]
    xs = [seeded.make_tokens(shape, 1, 16, layer=l, device=dev) for l in range(a.layers)]
    lgs = [seeded.make_logits(shape, 2, 16, layer=l, device=dev) for l in range(a.layers)] if a.logits else None
    ws = Workspace(shape, dev)
    out = torch.empty(1, shape.hidden, dtype=torch.bfloat16, device=dev)
    fn = lib().tmoe_moe_block_bf16 if a.mode == "bf16" else lib().tmoe_moe_block_int4
    stream = torch.cuda.current_stream(dev).cuda_stream
    buf = ws.ensure(1)

    def call(s):
        # One C call per step (no Python-side checks), so calls run back to back on the GPU.
        l = s % a.layers
        ly = layers[l]
        x = xs[l][(s // a.layers) % 16]
        lg = lgs[l][(s // a.layers) % 16].data_ptr() if lgs else None
        st = fn(x.data_ptr(), 1, ly.router_w.data_ptr(), lg, tables[l].data_ptr(),
                *[t.data_ptr() for t in ly.shared], shape.hidden, shape.num_experts, shape.intermediate,
                shape.top_k, shape.shared_intermediate, out.data_ptr(), None, None, None, buf.data_ptr(),
                buf.numel(), stream)
        check(st, "moe block")

    for s in range(200):
        call(s)
    step = 200
    with DecodeTrace(dev) as tr:
        for _ in range(a.reps):
            for _ in range(a.calls):
                call(step)
                step += 1
            print(format_summary(summarize(tr.records(), shape.hidden, shape.intermediate,
                                           shape.shared_intermediate, shape.num_experts)), flush=True)
    ws.status()


if __name__ == "__main__":
    main()
