"""Parity at the workload's full sizes: the T = 4096 prefill chunk through the full-size
layer (bf16 and int4) and the 48-layer, 194 GB resident stack decoding Zipf-routed tokens.

Bars: top-k ids, the dispatch permutation, heat counters and route telemetry bit-exact
against the oracle for every token and layer; outputs within max-abs 2e-2 and rel-L2 1e-3
of the oracle (prefill: a seeded sample of tokens, each token's own experts combined in
ascending expert id plus the shared expert; stack: every layer of every token, each fed the
device's output of the layer before, experts in router order).
"""
import numpy as np
import pytest
import torch

from oracle import bf16, int4, moe
from oracle.telemetry import RouteTelemetry as OracleTelemetry
from tarfa_amd import moe as tm
from tarfa_amd import seeded
from tarfa_amd.moe import MoEShape, Workspace
from tarfa_amd.residency import LayerWeights, ResidencyLedger, zipf_logits
from tarfa_amd.stack import MoEStack
from tests._util import assert_close_bf16, expert_dicts, f32

pytestmark = pytest.mark.gpu

FULL = MoEShape(2560, 256, 1024, 8, 1024)


def u16(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("mode", ["bf16", "int4"])
def test_prefill_t4096_full_size_layer(gpu, mode):
    T, E, k = 4096, FULL.num_experts, FULL.top_k
    seed = 300 if mode == "bf16" else 301
    layer = seeded.make_layer(FULL, seed, device=gpu)
    if mode == "bf16":
        table = tm.expert_table(layer.gate_up, layer.down)
    else:
        q4 = (*tm.quantize_int4(layer.gate_up), *tm.quantize_int4(layer.down))
        table = tm.expert_table_q4(*q4)
    ws = Workspace(FULL, gpu, tokens=T)
    x = seeded.make_tokens(FULL, seed, T, device=gpu)
    logits = seeded.make_logits(FULL, seed, T, device=gpu)        # ~N(0, 1): ~128 tokens per expert
    out, ids, w = tm.moe_block(FULL, x, table, ws, logits=logits, shared=layer.shared)
    torch.cuda.synchronize()
    ws.status()
    # routing and permutation of every token, bit-exact
    ids_ref, w_ref, _ = moe.router_topk(logits.cpu().numpy(), k)
    ids_d = ids.cpu().numpy()
    assert np.array_equal(ids_d, ids_ref)
    assert np.all(np.abs(f32(w) - w_ref) <= np.abs(w_ref) * 2.0 ** -7)
    counts = np.bincount(ids_ref.ravel(), minlength=E)
    assert counts.min() > 64 and counts.max() < 256                   # near-uniform load around 128
    offsets, perm, _ = tm.dispatch(ids, E, ws)
    o_ref, p_ref = moe.dispatch(ids_ref, E)
    assert np.array_equal(offsets.cpu().numpy(), o_ref)
    assert np.array_equal(perm.cpu().numpy()[:T * k], p_ref)
    # outputs of 64 seeded tokens, 16 at a time (only their experts are copied to the host)
    sample = np.sort(np.random.default_rng(seed).choice(T, 64, replace=False))
    xs, wd, got = f32(x), f32(w), f32(out)
    sh = [f32(t) for t in layer.shared]
    for c in range(0, sample.size, 16):
        rows = sample[c:c + 16]
        if mode == "bf16":
            gu, dn = expert_dicts(layer.gate_up, layer.down, ids_d[rows])
        else:
            used = sorted(set(ids_d[rows].ravel().tolist()))
            gq, gs, dq, ds = q4
            gu = {e: bf16.to_f32(int4.dequant(gq[e].cpu().numpy(), u16(gs[e]))) for e in used}
            dn = {e: bf16.to_f32(int4.dequant(dq[e].cpu().numpy(), u16(ds[e]))) for e in used}
        ref = moe.experts_prefill(xs[rows], ids_d[rows], wd[rows], gu, dn, E)
        ref = moe.add_bf16(ref, moe.shared_expert(xs[rows], *sh))
        assert_close_bf16(got[rows], ref, f"{mode} prefill T=4096 tokens {rows[0]}..{rows[-1]}")
        del gu, dn


def test_stack_48_layers_resident_zipf_decode(gpu):
    """The 48 full-size layers (194 GB of bf16 experts) resident in HBM; 5 consecutive tokens
    with Zipf(1.1) per-layer logits; ids of every (token, layer), heat and route telemetry
    bit-exact; every token's output at every layer against the oracle (each layer's input is
    the device's output of the layer before)."""
    L, NT = 48, 5
    ledger = ResidencyLedger(FULL, L, gpu)
    ledger.fill_seeded(41)
    layers = [LayerWeights(*seeded.make_block_weights(FULL, 41, l, gpu)) for l in range(L)]
    stack = MoEStack(ledger, layers)
    logits, _ = zipf_logits(FULL, L, NT, seed=13, device=gpu)
    x0 = seeded.make_tokens(FULL, 41, NT, device=gpu)
    ref_tel = OracleTelemetry(L)
    heat = np.zeros((L, FULL.num_experts), np.int64)
    for t in range(NT):
        outs = []
        stack.decode(x0[t:t + 1], logits[t], per_layer_out=outs)
        torch.cuda.synchronize()
        ids = stack.ids.cpu().numpy()
        lg = logits[t].cpu().numpy()
        ids_ref, w_ref, _ = moe.router_topk(lg, FULL.top_k)
        assert np.array_equal(ids, ids_ref), f"token {t} ids"
        for l in range(L):
            np.add.at(heat[l], ids_ref[l], 1)
            ref_tel.record(l, ids_ref[l].tolist(), FULL.num_experts)
        for l in range(L):
            inp = f32(x0[t:t + 1]) if l == 0 else f32(outs[l - 1])
            gu, dn = expert_dicts(ledger.hbm[l][0], ledger.hbm[l][1], ids_ref[l:l + 1])
            sh = [f32(w) for w in layers[l].shared]
            ref = moe.add_bf16(moe.experts_decode(inp[0], ids_ref[l], w_ref[l], gu, dn, FULL.num_experts),
                               moe.shared_expert(inp[0], *sh))
            assert_close_bf16(f32(outs[l])[0], ref, f"stack token {t} layer {l}")
            del gu, dn
    stack.status()
    assert np.array_equal(ledger.heat.cpu().numpy(), heat)
    c = stack.telemetry.counters().numpy()
    for l in range(L):
        st = ref_tel.per_layer[l]
        assert c[l, 0] == st["decode_steps"] and c[l, 1] == st["expert_uses"], l
        assert list(c[l, 2:7]) == [st[f"reuse_{w}"] for w in (1, 2, 4, 8, 16)], l
    got, want = stack.telemetry.routing_telemetry(), ref_tel.totals()
    for key in want:
        assert got[key] == want[key], key
    # Zipf popularity: the 8 hottest experts of a layer take far more than 8/256 of the picks
    share = np.sort(heat, axis=-1)[:, ::-1][:, :8].sum(-1) / heat.sum(-1)
    assert share.mean() > 0.2
    del stack, ledger
    torch.cuda.empty_cache()
