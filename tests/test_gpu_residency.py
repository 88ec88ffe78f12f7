"""GPU tests of the residency ledger, the layer stack and the route telemetry.

Bars: route telemetry counters and heat counters bit-exact against the CPU
restatements; each layer of the stack within the layer tolerance of the oracle
(given that layer's device input) with bit-exact ids; a tiered ledger (experts
read from pinned host memory or HBM slots, promotions in between) gives
bit-identical outputs to the fully resident ledger.
"""
import numpy as np
import pytest
import torch

from oracle import moe
from oracle.telemetry import RouteTelemetry as OracleTelemetry
from tarfa_amd import moe as tm
from tarfa_amd import seeded
from tarfa_amd._lib import lib
from tarfa_amd.moe import MoEShape
from tarfa_amd.residency import LayerWeights, ResidencyLedger, RouteTelemetry, zipf_logits
from tarfa_amd.stack import MoEStack
from tests._util import assert_close_bf16, expert_dicts, f32

pytestmark = pytest.mark.gpu

SHAPE = MoEShape(1024, 32, 512, 8, 512)      # exact-fit fused variant, with a shared expert


def _layers(shape, L, seed, gpu):
    out = []
    for l in range(L):
        ly = seeded.make_layer(MoEShape(shape.hidden, shape.num_experts, 8, shape.top_k, shape.shared_intermediate),
                               seed, layer=l, device=gpu)
        out.append(LayerWeights(ly.router_w, ly.shared))
    return out


def test_kernel_reads_experts_from_pinned_host_memory(gpu):
    """Zero-copy: a dequantise launch reading packed weights and scales straight from pinned host memory."""
    g = torch.Generator().manual_seed(1)
    packed = torch.randint(0, 256, (64, 256), dtype=torch.uint8, generator=g).pin_memory()
    scales = (torch.randn(64, 4, generator=g) * 0.02).to(torch.bfloat16).pin_memory()
    ref = tm.dequant_int4(packed.to(gpu), scales.to(gpu))
    out = torch.empty(64, 512, dtype=torch.bfloat16, device=gpu)
    st = lib().tmoe_dequant_int4_bf16(packed.data_ptr(), scales.data_ptr(), 64, 512, 128, out.data_ptr(),
                                      torch.cuda.current_stream().cuda_stream)
    assert st == 0
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_route_telemetry_matches_oracle(gpu):
    L, k, E = 3, 8, 32
    rng = np.random.default_rng(4)
    tel = RouteTelemetry(L, k, E, gpu)
    ref = OracleTelemetry(L)
    for step in range(40):
        ids = np.stack([rng.choice(E if rng.random() > 0.1 else 12, size=k, replace=False)
                        for _ in range(L)]).astype(np.int64)
        if step % 7 == 3:
            ids[1, :] = E                       # every slot the sentinel: nothing recorded
        if step % 5 == 1:
            ids[0, 2] = E                       # one sentinel slot
            ids[2, 3] = ids[2, 4]               # a duplicate id (caller-supplied routing)
        if step % 11 == 6:
            ids[2, 0] = 99                      # outside [0, E]: dropped like the sentinel
        tel.record(torch.from_numpy(ids).to(gpu))
        for l in range(L):
            ref.record(l, ids[l].tolist(), E)
    c = tel.counters().numpy()
    for l in range(L):
        st = ref.per_layer[l]
        assert c[l, 0] == st["decode_steps"] and c[l, 1] == st["expert_uses"]
        assert list(c[l, 2:7]) == [st[f"reuse_{w}"] for w in (1, 2, 4, 8, 16)]
    got = tel.routing_telemetry()
    want = ref.totals()
    for key in ("decode_steps", "expert_uses", "unique_layer_experts", "reuse_1", "reuse_16"):
        assert got[key] == want[key], key


def test_stack_decode_parity_heat_and_telemetry(gpu):
    L, T = 3, 5
    ledger = ResidencyLedger(SHAPE, L, gpu)
    ledger.fill_seeded(31)
    layers = _layers(SHAPE, L, 31, gpu)
    stack = MoEStack(ledger, layers)
    logits, _ = zipf_logits(SHAPE, L, T, seed=3, device=gpu)
    x0 = seeded.make_tokens(SHAPE, 31, T, device=gpu)
    ref_tel = OracleTelemetry(L)
    hist = np.zeros((L, SHAPE.num_experts), np.int64)
    for t in range(T):
        outs = []
        stack.decode(x0[t:t + 1], logits[t], per_layer_out=outs)
        torch.cuda.synchronize()
        ids = stack.ids.cpu().numpy()
        inp = f32(x0[t:t + 1])
        for l in range(L):
            lg = logits[t, l].cpu().numpy()[None]
            ids_ref, w_ref, _ = moe.router_topk(lg, SHAPE.top_k)
            assert np.array_equal(ids[l], ids_ref[0]), f"token {t} layer {l} ids"
            gu, dn = expert_dicts(ledger.hbm[l][0], ledger.hbm[l][1], ids_ref)
            sh = [f32(w) for w in layers[l].shared]
            ref = moe.add_bf16(moe.experts_decode(inp[0], ids_ref[0], w_ref[0], gu, dn, SHAPE.num_experts),
                               moe.shared_expert(inp[0], *sh))
            assert_close_bf16(f32(outs[l])[0], ref, f"stack token {t} layer {l}")
            inp = f32(outs[l])                   # the device output is the next layer's input
            np.add.at(hist[l], ids_ref[0], 1)
            ref_tel.record(l, ids_ref[0].tolist(), SHAPE.num_experts)
    stack.status()
    assert np.array_equal(ledger.heat.cpu().numpy(), hist)
    got, want = stack.telemetry.routing_telemetry(), ref_tel.totals()
    for key in ("decode_steps", "expert_uses", "unique_layer_experts", "reuse_1", "reuse_2", "reuse_4"):
        assert got[key] == want[key], key
    hl = ledger.hotlist()
    assert hl["selections"] == L * T * SHAPE.top_k
    assert all(0 < float(d["coverage"]["8"]) <= 1.0 for d in hl["layers"])


@pytest.mark.parametrize("int4", [False, True])
def test_tiered_ledger_matches_resident(gpu, int4):
    """Experts read from pinned host memory or HBM slots, with promotions and a heat
    rebalance between tokens, give the same bits as the fully resident ledger."""
    L, T = 2, 6
    res = ResidencyLedger(SHAPE, L, gpu, int4=int4)
    res.fill_seeded(8)
    tier = ResidencyLedger(SHAPE, L, gpu, int4=int4, hbm_slots=4)
    tier.fill_seeded(8)
    assert tier.location(0, 3) == "hbm" and tier.location(0, 20) == "host"
    layers = _layers(SHAPE, L, 8, gpu)
    a, b = MoEStack(res, layers), MoEStack(tier, layers)
    logits, _ = zipf_logits(SHAPE, L, T, seed=5, device=gpu)
    x0 = seeded.make_tokens(SHAPE, 8, T, device=gpu)
    for t in range(T):
        ya = a.decode(x0[t:t + 1], logits[t]).clone()
        yb = b.decode(x0[t:t + 1], logits[t]).clone()
        assert torch.equal(ya, yb), f"token {t}"
        assert torch.equal(a.ids, b.ids)
        if t == 1:
            moved = tier.promote(0, b.ids[0].tolist())
            assert all(tier.location(0, e) == "hbm" for e, _ in moved)
            assert sum(tier.location(0, int(e)) == "hbm" for e in b.ids[0].tolist()) == min(4, SHAPE.top_k)
        if t == 3:
            assert tier.rebalance() > 0
    a.status()
    b.status()
    assert tier.stats["promotions"] > 0 and tier.stats["evictions"] > 0
    assert torch.equal(res.heat, tier.heat)


def test_jnf_filled_ledgers_match_seeded(gpu, tmp_path):
    """A JNF v1 tree written from a seeded ledger fills a resident and a tiered ledger
    (verified reads, double-buffered staging / the pinned host tier) whose decodes give the
    seeded ledger's bits, before and after promotions from the file-filled host tier."""
    from tarfa_amd.jnf import JnfModel, write_jnf
    L, T = 2, 4
    res = ResidencyLedger(SHAPE, L, gpu)
    res.fill_seeded(8)
    write_jnf(tmp_path, {l: (res.hbm[l][0], res.hbm[l][1]) for l in range(L)}, top_k=SHAPE.top_k,
              model_id="seeded-8", revision="0", tokenizer_revision="0")
    jnf = JnfModel(tmp_path, SHAPE)
    full = ResidencyLedger(SHAPE, L, gpu)
    full.load_jnf(jnf, chunk=6)                      # 32 experts in chunks of 6: a ragged last chunk
    tier = ResidencyLedger(SHAPE, L, gpu, hbm_slots=4)
    tier.load_jnf(jnf)
    torch.cuda.synchronize(gpu)
    for l in range(L):
        assert torch.equal(full.hbm[l][0], res.hbm[l][0]) and torch.equal(full.hbm[l][1], res.hbm[l][1])
    layers = _layers(SHAPE, L, 8, gpu)
    stacks = [MoEStack(g, layers) for g in (res, full, tier)]
    logits, _ = zipf_logits(SHAPE, L, T, seed=6, device=gpu)
    x0 = seeded.make_tokens(SHAPE, 8, T, device=gpu)
    for t in range(T):
        ys = [s.decode(x0[t:t + 1], logits[t]).clone() for s in stacks]
        assert torch.equal(ys[0], ys[1]) and torch.equal(ys[0], ys[2]), f"token {t}"
        if t == 1:
            assert tier.promote(1, stacks[2].ids[1].tolist())
