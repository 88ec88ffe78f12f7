#!/usr/bin/env python3
"""MoE-layer hot-path benchmark on one MI355X; prints ONE JSON line.

Headline (``value``): exact-BF16 decode of one token through one full-size MoE
layer (H=2560, E=256 routed experts with I=1024, top-8, one shared expert with
Is=1024), router included, µs per token-layer.  A step is one token through one
layer; steps rotate over ``--layers`` distinct seeded layers and fresh tokens so
the per-step working set (~143 MB) is never served from the 256 MB Infinity
Cache.  Inputs and weights are resident in HBM before timing starts: the 48 layers
(194 GB of bf16 experts) live in one residency ledger.

Also reported: the labelled int4 fast mode at the same shape (``int4``), the
48-layer stack decoding consecutive tokens with Zipf-popular routing (``stack``), the
T=4096 exact-BF16 prefill chunk through the same layer shape (router logits
supplied ~N(0,1)), and the reference's op sequence run on the host CPU (torch
bf16) on a bounded sample as ``cpu_baseline``.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--layers L] [--no-cpu] [--no-prefill] [--no-int4]
                    [--no-small] [--no-stack]
"""
import argparse
import ctypes
import json
import os
import statistics
import sys
import time

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense bf16 MFMA
METRIC = "MoE layer µs/token + achieved HBM GB/s (bf16 exact, int4 fast), batch 1"


def decode_bytes(s):
    """Algorithmic bytes of one decode token-layer: 8 routed experts, shared expert, router, shared gate."""
    H, E, I, k, Is = s.hidden, s.num_experts, s.intermediate, s.top_k, s.shared_intermediate
    return 2 * (k * 3 * H * I + 3 * H * Is + E * H + (H if Is else 0))


def decode_bytes_int4(s, group=128):
    """Algorithmic bytes of one int4 fast-mode token-layer: 8 routed experts as packed int4 plus
    bf16 group scales, the bf16 shared expert, router and shared gate."""
    H, E, I, k, Is = s.hidden, s.num_experts, s.intermediate, s.top_k, s.shared_intermediate
    per_expert = 3 * H * I // 2 + 2 * (3 * H * I // group)
    return k * per_expert + 2 * (3 * H * Is + E * H + (H if Is else 0))


def prefill_flops(s, T):
    H, I, k, Is = s.hidden, s.intermediate, s.top_k, s.shared_intermediate
    return 2 * T * k * 3 * H * I + 2 * T * 3 * H * Is


def prefill_weight_bytes(s):
    H, E, I, Is = s.hidden, s.num_experts, s.intermediate, s.shared_intermediate
    return 2 * (E * 3 * H * I + 3 * H * Is)


def profiled_traffic(name, key="traffic_bytes_per_launch"):
    """HBM bytes per launch recorded by the rocprofv3 FETCH_SIZE / WRITE_SIZE passes in profiles/<name>."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", name)
    try:
        for line in open(path):
            if line.startswith(key + ":"):
                return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def host_cpu():
    """(model name, physical cores, logical CPUs of the host, CPUs this process may use)."""
    model, cores = "unknown", set()
    phys = core = None
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "model name" and model == "unknown":
                model = v
            elif k == "physical id":
                phys = v
            elif k == "core id":
                core = v
            elif not k and phys is not None and core is not None:
                cores.add((phys, core))
                phys = core = None
        if phys is not None and core is not None:
            cores.add((phys, core))
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return model, len(cores) or None, os.cpu_count() or 1, usable


def leg_steps(args):
    """Timed steps of every decode leg: the headline (bf16 block), the sublayer and int4."""
    K = args.steps
    return {"decode": K,
            "layer": K if args.layer_steps is None else args.layer_steps,
            "int4": K if args.int4_steps is None else args.int4_steps}


def token_rows(L, warmup, steps):
    """Per-layer token rows every decode leg needs: step s of a leg runs layer s % L on that
    layer's token row s // L, for s < warmup + steps."""
    return (warmup + max(steps.values()) + L - 1) // L


def step_plan(L, warmup, steps):
    """(layer, row) of each of the warmup + steps launches of one leg."""
    return [(s % L, s // L) for s in range(warmup + steps)]


def cpu_threads(usable):
    return max(1, min(16, usable))     # this GPU's share of the host


def parse_args(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--layers", type=int, default=48,
                    help="resident seeded layers (48 = the whole stack, 194 GB of bf16 experts)")
    ap.add_argument("--layer-steps", type=int, default=None, help="timed steps of the sublayer leg (default --steps)")
    ap.add_argument("--int4-steps", type=int, default=None, help="timed steps of the int4 leg (default --steps)")
    ap.add_argument("--stack-tokens", type=int, default=64)
    ap.add_argument("--no-stack", action="store_true")
    ap.add_argument("--prefill-steps", type=int, default=6)
    ap.add_argument("--cpu-tokens", type=int, default=200,
                    help="decode tokens of each CPU baseline decode sample (median reported)")
    ap.add_argument("--cpu-prefill-reps", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-int4", action="store_true")
    ap.add_argument("--no-small", action="store_true")
    ap.add_argument("--small-steps", type=int, default=200,
                    help="timed steps per token count of the small-batch leg")
    ap.add_argument("--small-tokens", default="2,4,8,16", help="token counts of the small-batch leg (2..16)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run plain device copies of known size (scale for HBM byte counters)")
    return ap.parse_args(argv)


class _Timer:
    """HIP events on the launch stream (torch's current stream, which every leg launches on)."""

    def __init__(self, torch):
        self.torch = torch
        self.e0 = torch.cuda.Event(enable_timing=True)
        self.e1 = torch.cuda.Event(enable_timing=True)

    def run(self, fn, plan, warmup):
        for a in plan[:warmup]:
            fn(a)
        self.torch.cuda.synchronize()
        t0 = time.perf_counter()
        self.e0.record()
        for a in plan[warmup:]:
            fn(a)
        self.e1.record()
        self.torch.cuda.synchronize()
        return self.e0.elapsed_time(self.e1), time.perf_counter() - t0


def run(args, log):
    import torch
    from tarfa_amd import seeded
    from tarfa_amd import moe as tm
    from tarfa_amd._lib import lib
    from tarfa_amd.moe import MoEShape, Workspace
    from tarfa_amd.residency import LayerWeights, ResidencyLedger, zipf_logits
    from tarfa_amd.stack import MoEStack

    dev = torch.device("cuda:0")
    shape = MoEShape(2560, 256, 1024, 8, 1024)
    L, W = args.layers, args.warmup
    steps = leg_steps(args)
    K = steps["decode"]
    H = shape.hidden
    timer = _Timer(torch)

    # ---------------- setup: the L seeded full-size layers resident in HBM (residency ledger),
    # per-layer router / shared-expert weights and token rows for every decode leg
    t0 = time.perf_counter()
    ledger = ResidencyLedger(shape, L, dev)
    ledger.fill_seeded(1)
    layers = [LayerWeights(*seeded.make_block_weights(shape, 1, l, dev)) for l in range(L)]
    tables = [ledger.tables[l] for l in range(L)]
    rows = token_rows(L, W, steps)
    xs = [seeded.make_tokens(shape, 1, rows, layer=l, device=dev) for l in range(L)]
    ws = Workspace(shape, dev)
    out = torch.empty(1, H, dtype=torch.bfloat16, device=dev)
    ids = torch.empty(1, shape.top_k, dtype=torch.int64, device=dev)
    wts = torch.empty(1, shape.top_k, dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()
    log(f"setup {time.perf_counter() - t0:.1f}s: {L} resident layers x {prefill_weight_bytes(shape) / 1e9:.2f} GB, "
        f"{rows} token rows per layer")

    # Lean launch path: prebuilt ctypes arguments, one C call per step.
    stream = torch.cuda.current_stream(dev).cuda_stream
    wsp, wsn = ws.buf.data_ptr(), ws.buf.numel()

    def block_args(l, r, table=None):
        ly = layers[l]
        sh = [t.data_ptr() for t in ly.shared]
        return (xs[l][r].data_ptr(), 1, ly.router_w.data_ptr(), None, (tables[l] if table is None else table).data_ptr(), *sh, H,
                shape.num_experts, shape.intermediate, shape.top_k, shape.shared_intermediate, out.data_ptr(),
                ids.data_ptr(), wts.data_ptr(), None, wsp, wsn, stream)

    def launcher(fn, name):
        def go(a):
            if fn(*a):
                raise RuntimeError(f"{name} failed")
        return go

    plan = [block_args(l, r) for l, r in step_plan(L, W, K)]
    gpu_ms, wall = timer.run(launcher(lib().tmoe_moe_block_bf16, "tmoe_moe_block_bf16"), plan, W)
    ws.status()
    us = gpu_ms * 1e3 / K
    nbytes = decode_bytes(shape)
    gbs = nbytes / (us * 1e-6) / 1e9
    log(f"decode: {us:.2f} us/token-layer (wall {wall * 1e6 / K:.2f} us), {gbs:.0f} GB/s")

    result = {
        "metric": METRIC, "value": round(us, 3), "unit": "us/token-layer", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(us / 1e3, 6), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic: seeded counter-based generator (sum of twelve uniforms), weights ~N(0,0.02), x ~N(0,1)",
        "config": {"workload": "full-size exact-BF16 MoE decode layer, batch 1 (router + 8 routed SwiGLU experts "
                               "+ shared expert + combine)",
                   "hidden": H, "experts": shape.num_experts, "intermediate": shape.intermediate,
                   "top_k": shape.top_k, "shared_intermediate": shape.shared_intermediate,
                   "layers_rotated": L, "batch": 1},
        "roofline": {"kernel": "k_decode_fused (one persistent launch per token-layer)",
                     "bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic("k_decode_fused_decode_h2560_e256_i1024_k8.md"),
                     "algorithmic_bytes_per_launch": nbytes},
        "hbm_gbps": round(gbs, 1),
        "tokens_per_s_48_layers": round(1e6 / (48 * us), 2),
    }

    # The MoE sublayer (post-attention RMSNorm fused into the input, residual add into the
    # combine) on the same rotation: what the fused norm and residual cost on top.
    gen = torch.Generator().manual_seed(7)
    ln_ws = [(torch.randn(H, generator=gen) * 0.1).to(torch.bfloat16).to(dev) for _ in range(L)]
    KL = steps["layer"]

    def layer_args(l, r):
        a = block_args(l, r)
        return (a[0], 1, ln_ws[l].data_ptr(), ctypes.c_float(1e-6)) + a[2:]

    lplan = [layer_args(l, r) for l, r in step_plan(L, W, KL)]
    gpu_ms, _ = timer.run(launcher(lib().tmoe_moe_layer_bf16, "tmoe_moe_layer_bf16"), lplan, W)
    ws.status()
    us_l = gpu_ms * 1e3 / KL
    log(f"layer (RMSNorm + block + residual): {us_l:.2f} us/token-layer")
    result["layer"] = {"workload": "the MoE sublayer at the same shape, batch 1: bf16(h + block(rmsnorm(h))), the "
                                   "norm formed once per fused-decode wave, the residual added in its combine",
                       "us_per_token_layer": round(us_l, 3), "over_block_us": round(us_l - us, 3), "steps": KL}

    if args.calibrate_copy:
        # Plain device copies of a known size: under `rocprofv3 --pmc FETCH_SIZE` /
        # `WRITE_SIZE` they give the counter-to-byte scale for this GPU.
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(8):
            dst.copy_(src)
        torch.cuda.synchronize()
        result["copy_calibration_bytes"] = src.numel()
        del src, dst

    # ---------------- int4 fast mode: the same layers with their routed experts quantised (group 128)
    if not args.no_int4:
        t0 = time.perf_counter()
        q4 = ResidencyLedger.quantized_from(ledger)
        log(f"int4 setup {time.perf_counter() - t0:.1f}s")
        K4 = steps["int4"]
        plan4 = [block_args(l, r, q4.tables[l]) for l, r in step_plan(L, W, K4)]
        gpu_ms, _ = timer.run(launcher(lib().tmoe_moe_block_int4, "tmoe_moe_block_int4"), plan4, W)
        ws.status()
        us4 = gpu_ms * 1e3 / K4
        nb4 = decode_bytes_int4(shape)
        gbs4 = nb4 / (us4 * 1e-6) / 1e9
        result["int4"] = {"workload": "labelled int4 fast mode at the same layer shape, batch 1: routed experts "
                                      "int4 [-8,7] packed 2 per byte along K, bf16 scales per group of 128 "
                                      "(max|w|/7), shared expert exact bf16",
                          "us_per_token_layer": round(us4, 3), "hbm_gbps": round(gbs4, 1),
                          "frac": round(gbs4 / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_launch": nb4,
                          "traffic": profiled_traffic("k_decode_fused_int4_decode_h2560_e256_i1024_k8.md"),
                          "steps": K4, "tokens_per_s_48_layers": round(1e6 / (48 * us4), 2)}
        log(f"int4 decode: {us4:.2f} us/token-layer, {gbs4:.0f} GB/s")
        if not args.no_prefill:
            # int4 prefill: T=4096, logits supplied; weights dequantised into the MFMA fragments
            T4, P4 = 4096, args.prefill_steps
            pws4 = Workspace(shape, dev, tokens=T4)
            px4 = seeded.make_tokens(shape, 2, T4, device=dev)
            plg4 = [seeded.make_logits(shape, 2, T4, layer=l, device=dev) for l in range(min(L, P4 + 1))]
            pout4 = torch.empty(T4, H, dtype=torch.bfloat16, device=dev)
            pi4 = torch.empty(T4, shape.top_k, dtype=torch.int64, device=dev)
            pw4 = torch.empty(T4, shape.top_k, dtype=torch.bfloat16, device=dev)

            def prefill4(i):
                l = i % len(plg4)
                tm.moe_block(shape, px4, q4.tables[l], pws4, logits=plg4[l], shared=layers[l].shared, out=pout4,
                             ids=pi4, weights=pw4)

            gpu_ms, _ = timer.run(prefill4, list(range(P4 + 1)), 1)
            pws4.status()
            pus4 = gpu_ms * 1e3 / P4
            # routed: 3*H*I nibbles + one bf16 scale per 128 columns per expert; shared expert bf16
            wb4 = shape.num_experts * 3 * H * shape.intermediate * (64 + 2) // 128 + \
                2 * 3 * H * shape.shared_intermediate
            result["int4"]["prefill"] = {
                "workload": "int4 prefill chunk T=4096 through one full-size layer (logits ~N(0,1) supplied, shared "
                            "expert bf16): routed weights dequantised in registers into the MFMA fragments",
                "us_per_layer": round(pus4, 1), "tflops": round(prefill_flops(shape, T4) / (pus4 * 1e-6) / 1e12, 1),
                "weight_bytes": wb4, "weight_gbps": round(wb4 / (pus4 * 1e-6) / 1e9, 1),
                "gemm_traffic_per_launch": profiled_traffic("k_grouped_gemm_w_prefill_t4096_h2560_e256_i1024_k8.md",
                                                            "int4_traffic_bytes_per_launch")}
            log(f"int4 prefill: {pus4:.1f} us/layer")
            del pws4, px4, plg4
        del q4, plan4

    # ---------------- prefill: T = 4096 through the same layer shape, logits supplied
    if not args.no_prefill:
        T = 4096
        pws = Workspace(shape, dev, tokens=T)
        P = args.prefill_steps
        pl = [(l % L) for l in range(P + 1)]
        px = {l: seeded.make_tokens(shape, 2, T, layer=l, device=dev) for l in set(pl)}
        plg = {l: seeded.make_logits(shape, 2, T, layer=l, device=dev) for l in set(pl)}
        pout = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
        pids = torch.empty(T, shape.top_k, dtype=torch.int64, device=dev)
        pw = torch.empty(T, shape.top_k, dtype=torch.bfloat16, device=dev)

        def prefill(i):
            l = pl[i]
            tm.moe_block(shape, px[l], tables[l], pws, logits=plg[l],
                         shared=layers[l].shared, out=pout, ids=pids, weights=pw)

        gpu_ms, _ = timer.run(prefill, list(range(P + 1)), 1)
        pws.status()
        pus = gpu_ms * 1e3 / P
        fl = prefill_flops(shape, T)
        wb = prefill_weight_bytes(shape)
        tflops = fl / (pus * 1e-6) / 1e12
        wgbs = wb / (pus * 1e-6) / 1e9
        attain = min(BF16_PEAK_TFLOPS, HBM_PEAK_GBS * fl / wb / 1e3)
        result["prefill"] = {"workload": "exact-BF16 prefill chunk T=4096 through one full-size layer "
                                         "(logits ~N(0,1) supplied, shared expert included)",
                             "us_per_layer": round(pus, 1), "tflops": round(tflops, 1),
                             "mfma_frac": round(tflops / BF16_PEAK_TFLOPS, 4),
                             "weight_gbps": round(wgbs, 1), "hbm_frac": round(wgbs / HBM_PEAK_GBS, 4),
                             "attainable_tflops": round(attain, 1), "roofline_frac": round(tflops / attain, 4),
                             "flops": fl, "weight_bytes": wb, "tokens_per_s": round(T / (pus * 1e-6), 1),
                             "gemm_traffic_per_launch": profiled_traffic("k_grouped_gemm_w_prefill_t4096_h2560_e256_i1024_k8.md")}
        log(f"prefill: {pus:.1f} us/layer, {tflops:.1f} TFLOP/s, weights {wgbs:.0f} GB/s")
        del pws, px, plg

    # ---------------- small batches: T = 2..16 tokens through the full-size layer (router from
    # weights, shared expert), layers rotated as in the headline; each expert the batch hits is
    # read once, so the floor is (distinct experts + shared expert) x 3 H I bf16 + the router
    if not args.no_small:
        result["small_batch"] = small_batch(args, torch, seeded, shape, ledger, layers, tables, L, dev, lib, log)

    # ---------------- the whole stack: 48 resident layers, batch-1 decode of consecutive tokens,
    # per-layer router logits with Zipf(1.1) expert popularity (heat ledger + route telemetry on)
    if not args.no_stack:
        NT, NW = args.stack_tokens, 4
        stack = MoEStack(ledger, layers)
        ledger.heat.zero_()
        slg, _ = zipf_logits(shape, L, NT + NW, seed=11, device=dev)
        sx = seeded.make_tokens(shape, 3, NT + NW, device=dev)
        gpu_ms, _ = timer.run(lambda t: stack.decode(sx[t:t + 1], slg[t]), list(range(NW + NT)), NW)
        stack.status()
        ms_tok = gpu_ms / NT
        # logits are supplied: per layer the routed experts, the shared expert and the shared gate row are read
        tok_bytes = L * (decode_bytes(shape) - 2 * shape.num_experts * H)
        heat = ledger.heat.cpu()
        top8 = heat.sort(-1, descending=True).values[:, :8].sum(-1).double() / heat.sum(-1).double()
        result["stack"] = {"workload": f"{L}-layer MoE-only stack at the full-size layer shape, {194.1 * L / 48:.1f} GB of "
                                       "experts resident in HBM, batch-1 decode of consecutive tokens; per-layer "
                                       "router logits log(Zipf s=1.1 weight of a permuted rank) + Gumbel",
                           "layers": L, "tokens": NT, "ms_per_token": round(ms_tok, 4),
                           "tokens_per_s": round(1e3 / ms_tok, 2), "us_per_layer": round(ms_tok * 1e3 / L, 3),
                           "hbm_gbps": round(tok_bytes / (ms_tok * 1e-3) / 1e9, 1),
                           "algorithmic_bytes_per_token": tok_bytes,
                           "heat_top8_share_mean": round(float(top8.mean()), 4),
                           "routing_telemetry": stack.telemetry.routing_telemetry()}
        log(f"stack: {ms_tok:.3f} ms/token over {L} layers")
        del stack

    # ---------------- CPU baseline: the reference's op chain in torch bf16 on the host
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(args, torch, seeded, shape, ledger, layers, nbytes, dev, log)

    torch.cuda.synchronize()
    return result


def small_batch(args, torch, seeded, shape, ledger, layers, tables, L, dev, lib, log):
    """Small-batch decode (T = 2, 4, 8, 16 tokens per call) through the full-size layer:
    router + routed experts + shared expert + combine, µs per layer and against the weight
    read of the experts actually hit."""
    from tarfa_amd.moe import Workspace
    H, E, I, k, Is = shape.hidden, shape.num_experts, shape.intermediate, shape.top_k, shape.shared_intermediate
    stream = torch.cuda.current_stream(dev).cuda_stream
    fn = lib().tmoe_moe_block_bf16
    expert_b = 2 * 3 * H * I
    out = {"workload": "T tokens per call through the full-size exact-BF16 layer (router from weights, shared "
                       "expert, combine in ascending expert id), layers rotated; floor = (distinct experts hit "
                       "+ shared expert) x 3 H I bf16 + router weights at 8 TB/s", "by_tokens": {}}
    K, W = args.small_steps, 16
    for T in [int(v) for v in args.small_tokens.split(",")]:
        ws = Workspace(shape, dev, tokens=T)
        xs = [seeded.make_tokens(shape, 4, T, layer=l, device=dev) for l in range(L)]
        o = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
        ids = torch.empty(T, k, dtype=torch.int64, device=dev)
        wts = torch.empty(T, k, dtype=torch.bfloat16, device=dev)
        argv = [(xs[l].data_ptr(), T, layers[l].router_w.data_ptr(), None, tables[l].data_ptr(),
                 *[t.data_ptr() for t in layers[l].shared], H, E, I, k, Is, o.data_ptr(), ids.data_ptr(),
                 wts.data_ptr(), None, ws.buf.data_ptr(), ws.buf.numel(), stream) for l in range(L)]
        hits = []
        for l in range(min(L, 16)):
            if fn(*argv[l]):
                raise RuntimeError("tmoe_moe_block_bf16 failed")
            hits.append(len(set(ids.view(-1).tolist())))
        nh = sum(hits) / len(hits)

        def go(i):
            if fn(*argv[i % L]):
                raise RuntimeError("tmoe_moe_block_bf16 failed")

        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for i in range(W):
            go(i)
        torch.cuda.synchronize()
        e0.record()
        for i in range(W, W + K):
            go(i)
        e1.record()
        torch.cuda.synchronize()
        ws.status()
        us = e0.elapsed_time(e1) * 1e3 / K
        floor_b = (nh + (1 if Is else 0)) * expert_b + 2 * E * H
        floor_us = floor_b / (HBM_PEAK_GBS * 1e3)
        out["by_tokens"][str(T)] = {"us_per_layer": round(us, 2), "us_per_token": round(us / T, 2),
                                    "experts_hit": round(nh, 2), "weight_bytes": int(floor_b),
                                    "floor_us": round(floor_us, 2), "frac_of_floor": round(floor_us / us, 4),
                                    "steps": K}
        log(f"small batch T={T}: {us:.1f} us/layer ({us / T:.1f} us/token), {nh:.1f} experts, "
            f"{floor_us / us:.3f} of the weight-read floor")
        del ws, xs
    return out


def cpu_baseline(args, torch, seeded, shape, ledger, layers, nbytes, dev, log):
    """The reference's op chain (torch CPU bf16) on this host, on bounded samples: decode of the
    full-size layer (the headline's unit), decode of the small CPU layer (H=1024, E=32, I=512, no
    shared expert) and one T=4096 prefill chunk through the full-size layer."""
    from oracle import cpu_reference as cref
    from tarfa_amd.moe import MoEShape

    model, phys, logical, usable = host_cpu()
    nt = cpu_threads(usable)
    torch.set_num_threads(nt)
    H = shape.hidden

    def median_us(fn, reps, warm=2):
        for _ in range(warm):
            fn()
        times = []
        for _ in range(reps):
            t1 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t1)
        return statistics.median(times) * 1e6

    t_all = time.perf_counter()
    # full-size layer 0, same seeded weights as the GPU legs
    gu, dn = ledger.hbm[0][0].cpu(), ledger.hbm[0][1].cpu()
    wg = layers[0].router_w.cpu()
    shw = tuple(t.cpu() for t in layers[0].shared)
    nd = args.cpu_tokens
    xc = seeded.make_tokens(shape, 4, nd + 2, device=dev).cpu()
    it = iter(range(nd + 2))
    us1 = median_us(lambda: cref.moe_block(xc[next(it)][None], wg, shape.top_k, gu, dn, shape.num_experts, shw), nd)
    # the small CPU layer
    s0 = MoEShape(1024, 32, 512, 8, 0)
    l0 = seeded.make_layer(s0, seed=5, device=dev)
    gu0, dn0, wg0 = l0.gate_up.cpu(), l0.down.cpu(), l0.router_w.cpu()
    x0 = seeded.make_tokens(s0, 5, nd + 2, device=dev).cpu()
    it0 = iter(range(nd + 2))
    us0 = median_us(lambda: cref.moe_block(x0[next(it0)][None], wg0, s0.top_k, gu0, dn0, s0.num_experts), nd)
    # T = 4096 prefill chunk, logits supplied ~N(0,1), shared expert included
    T = 4096
    px = seeded.make_tokens(shape, 2, T, device=dev).cpu()
    plg = seeded.make_logits(shape, 2, T, device=dev).cpu()
    sp = median_us(lambda: cref.moe_block(px, wg, shape.top_k, gu, dn, shape.num_experts, shw, logits=plg),
                   args.cpu_prefill_reps) * 1e-6
    fl = prefill_flops(shape, T)
    log(f"cpu: {us1:.0f} us/token-layer (full size), {us0:.0f} us (small layer), prefill {sp:.2f} s/layer "
        f"on {nt} threads")
    return {
        "value": round(us1, 1), "unit": "us/token-layer", "cores": nt, "kind": "port",
        "sample": f"median of {nd} decode tokens through one full-size layer (same seeded weights as the GPU legs), "
                  f"torch {torch.__version__} CPU bf16 op sequence of fused_int4.py:192-194 + router + shared "
                  f"expert; also the small CPU layer (median of {nd}) and one T=4096 prefill chunk "
                  f"(fused_int4.py:239-244, median of {args.cpu_prefill_reps}); each after 2 warm-up runs",
        "gbps": round(nbytes / (us1 * 1e-6) / 1e9, 2),
        "cpu_model": model, "host_physical_cores": phys, "host_logical_cpus": logical,
        "usable_cpus": usable, "threads": nt,
        "decode_small_layer_us": round(us0, 1),
        "prefill_t4096_s_per_layer": round(sp, 3), "prefill_t4096_tflops": round(fl / sp / 1e12, 3),
        "seconds": round(time.perf_counter() - t_all, 1)}


def main(argv=None):
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the MoE layer is not sharded across "
              "GPUs in this build.", file=sys.stderr)
        return 2
    log = lambda *a: print("[bench]", *a, file=sys.stderr, flush=True)  # noqa: E731
    result = run(args, log)
    # Every device object of the run is released by now; drain the device and return the
    # cached blocks before the interpreter's exit handlers run.
    import gc
    import torch
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
