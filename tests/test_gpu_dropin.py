"""The drop-in boundary driven where the reference binds it: a transformers
Qwen3_5MoeSparseMoeBlock whose experts module gets libtmoe's forward installed
(tarfa/engine/fused_int4.py:262), the whole-block replacement built from the same
module, the boundary's telemetry and status poll, and workspace reuse across T.

Bars as the other parity tests: ids bit-exact; outputs within max-abs 2e-2 and rel-L2 1e-3
of the oracle at the reference's rounding points (decode in router order, prefill in
ascending expert id).
"""
import numpy as np
import pytest
import torch

from oracle import bf16, moe, rng
from tarfa_amd import experts as tx
from tarfa_amd import moe as tm
from tarfa_amd import seeded
from tarfa_amd.moe import MoEShape, Workspace
from tests._util import assert_close_bf16, f32

pytestmark = pytest.mark.gpu

BF = torch.bfloat16
SHAPE = MoEShape(1024, 32, 512, 8, 512)


def _tf_block(shape, seed, device):
    """A bf16 transformers Qwen3_5MoeSparseMoeBlock with seeded weights, on ``device``."""
    from transformers.models.qwen3_5_moe import configuration_qwen3_5_moe as C, modeling_qwen3_5_moe as M
    H, E, I, k, Is = shape.hidden, shape.num_experts, shape.intermediate, shape.top_k, shape.shared_intermediate
    cfg = C.Qwen3_5MoeTextConfig(hidden_size=H, num_experts=E, moe_intermediate_size=I, num_experts_per_tok=k,
                                 shared_expert_intermediate_size=Is, hidden_act="silu")
    blk = M.Qwen3_5MoeSparseMoeBlock(cfg).to(BF)
    layer = seeded.make_layer(shape, seed, device=device)
    with torch.no_grad():
        blk.experts.gate_up_proj.copy_(layer.gate_up.cpu())
        blk.experts.down_proj.copy_(layer.down.cpu())
        blk.gate.weight.copy_(layer.router_w.cpu())
        g, u, d, sg = layer.shared
        blk.shared_expert.gate_proj.weight.copy_(g.cpu())
        blk.shared_expert.up_proj.weight.copy_(u.cpu())
        blk.shared_expert.down_proj.weight.copy_(d.cpu())
        blk.shared_expert_gate.weight.copy_(sg.cpu().reshape(1, -1))
    return blk.to(device), layer


def _oracle_block(x, ids, w, layer, shape):
    xs = f32(x)
    gu = {e: f32(layer.gate_up[e]) for e in set(ids.reshape(-1).tolist())}
    dn = {e: f32(layer.down[e]) for e in gu}
    if xs.shape[0] == 1:
        routed = moe.experts_decode(xs[0], ids[0], w[0], gu, dn, shape.num_experts)[None]
    else:
        routed = moe.experts_prefill(xs, ids, w, gu, dn, shape.num_experts)
    return moe.add_bf16(routed, moe.shared_expert(xs, *[f32(t) for t in layer.shared]))


@pytest.mark.parametrize("T", [1, 17])
def test_install_experts_on_a_transformers_block(gpu, T):
    blk, layer = _tf_block(SHAPE, 40 + T, gpu)
    ex = blk.experts
    store = tx.ExpertStore.from_slabs(SHAPE, ex.gate_up_proj.data, ex.down_proj.data)
    tx.install_experts(ex, store)
    assert "gate_up_proj" not in dict(ex.named_parameters())
    x = seeded.make_tokens(SHAPE, 40 + T, T, device=gpu)
    with torch.no_grad():
        out = blk(x.reshape(1, T, -1)).reshape(T, -1)
        _, tw, ti = blk.gate(x)                      # the module's own routing (bf16 logits)
    torch.cuda.synchronize()
    store.check_status()
    ref = _oracle_block(x, ti.cpu().numpy(), f32(tw), layer, SHAPE)
    assert_close_bf16(f32(out), ref, f"installed experts T={T}")
    # the hidden state is not mutated and the result is a new tensor
    assert out.data_ptr() != x.data_ptr()


@pytest.mark.parametrize("T,k,j,ties", [(1, 8, 5, False), (37, 8, 5, True), (1000, 8, 1, False), (64, 16, 8, True),
                                       (5, 8, 8, False)])
def test_topk_renorm_matches_the_oracle(gpu, T, k, j, ties):
    """tmoe_topk_renorm_bf16 (fused_int4.py:157-160) bit-exact against the oracle's restatement,
    ties (equal weights keep the lower slot) included."""
    g = np.random.default_rng(T * 7 + k + j)
    vals = np.array([0.125, 0.25, 0.5], np.float32) if ties else None
    w = (g.choice(vals, (T, k)) if ties else bf16.rnd(g.uniform(0.01, 1.0, (T, k)).astype(np.float32)))
    ids = g.integers(0, 257, (T, k))
    ti = torch.from_numpy(ids).to(gpu)
    tw = torch.from_numpy(w.astype(np.float32)).to(BF).to(gpu)
    got_ids, got_w = tm.topk_renorm(ti, tw, j)
    want_ids, want_w = moe.jtopk_truncate(ids, w, j) if j < k else (ids, w)
    if j == k:                                           # nothing to cut: still the renormalised weights
        want_ids, want_w = moe.jtopk_truncate(np.pad(ids, ((0, 0), (0, 1))), np.pad(w, ((0, 0), (0, 1))), j)
    assert np.array_equal(got_ids.cpu().numpy(), want_ids)
    assert np.array_equal(f32(got_w), want_w)


@pytest.mark.parametrize("T", [1, 17])
def test_install_experts_cuts_the_routing_to_jtopk(gpu, T, monkeypatch):
    """The reference's JTOPK (environment, fused_int4.py:17) below the router's top-k: the routed
    step runs on the top-JTOPK weights renormalised, as fused_int4.py:157-160 does."""
    monkeypatch.setenv("JTOPK", "5")
    blk, layer = _tf_block(SHAPE, 80 + T, gpu)
    ex = blk.experts
    store = tx.ExpertStore.from_slabs(SHAPE, ex.gate_up_proj.data, ex.down_proj.data)
    tx.install_experts(ex, store)
    x = seeded.make_tokens(SHAPE, 80 + T, T, device=gpu)
    with torch.no_grad():
        out = blk(x.reshape(1, T, -1)).reshape(T, -1)
        _, tw, ti = blk.gate(x)
    torch.cuda.synchronize()
    store.check_status()
    ids5, w5 = moe.jtopk_truncate(ti.cpu().numpy(), f32(tw), 5)
    ref = _oracle_block(x, ids5, w5, layer, SHAPE)
    assert_close_bf16(f32(out), ref, f"JTOPK=5 T={T}")


@pytest.mark.parametrize("T", [1, 17])
def test_from_transformers_block(gpu, T):
    blk, layer = _tf_block(SHAPE, 60 + T, gpu)
    tb = tx.from_transformers_block(blk, gpu)
    x = seeded.make_tokens(SHAPE, 60 + T, T, device=gpu)
    out = tb(x.reshape(1, T, -1)).reshape(T, -1)
    torch.cuda.synchronize()
    tb.store.check_status()
    ids = tb.last_ids.cpu().numpy()
    ref_ids, _, _ = moe.router_topk(moe.router_logits(f32(x), f32(layer.router_w)), SHAPE.top_k)
    assert np.array_equal(ids, ref_ids)
    ref = _oracle_block(x, ids, f32(tb.last_weights), layer, SHAPE)
    assert_close_bf16(f32(out), ref, f"from_transformers_block T={T}")


def test_dropin_counters_route_telemetry_and_status_poll(gpu):
    shape = MoEShape(512, 16, 256, 4)
    layer = seeded.make_layer(shape, 9, device=gpu)
    store = tx.ExpertStore.from_slabs(shape, layer.gate_up, layer.down, status_poll=1)

    class _Experts(torch.nn.Module):
        pass

    mod = tx.install_experts(_Experts(), store)
    x = seeded.make_tokens(shape, 9, 3, device=gpu)
    w = torch.tensor([[0.4, 0.3, 0.2, 0.1]], device=gpu).to(BF)
    good = torch.tensor([[3, 16, 7, 1]], device=gpu)            # 16 = the skip sentinel E
    base_routes = tx.routing_telemetry()["decode_steps"]
    mod(x[:1], good, w)
    mod(x[1:2], torch.tensor([[3, 5, 7, 1]], device=gpu), w)
    mod(x, torch.tensor([[3, 5, 7, 1]] * 3, device=gpu), w.expand(3, 4).contiguous())   # a prefill call
    torch.cuda.synchronize()
    assert store.book.counts == {"decode": 2, "prefill": 1}
    t = tx.telemetry()
    assert t["decode_moe_calls"] >= 2 and t["prefill_moe_calls"] >= 1 and t["decode_moe_seconds"] > 0
    c = store.book.route.counters()[0].tolist()
    # two decode steps: {3,7,1} then {3,5,7,1}; reuse_1 = |{3,7,1}| = 3, one new expert (5)
    assert c[:3] == [2, 7, 3] and c[7] == 4
    assert tx.routing_telemetry()["decode_steps"] == base_routes + 2
    # an expert id outside [0, E] is raised by a later call once the asynchronous poll lands
    mod(x[:1], torch.tensor([[3, 99, 7, 1]], device=gpu), w)
    torch.cuda.synchronize()
    mod(x[:1], good, w)                                          # polls the bad call's status
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError, match="expert id"):
        mod(x[:1], good, w)
    with pytest.raises(RuntimeError, match="expert id"):
        store.check_status()
    store.check_status()                                         # cleared
    out = mod(x[:1], good, w)
    torch.cuda.synchronize()
    gu = {e: f32(layer.gate_up[e]) for e in (3, 7, 1)}
    dn = {e: f32(layer.down[e]) for e in gu}
    ref = moe.experts_decode(f32(x)[0], good.cpu().numpy()[0], f32(w)[0], gu, dn, 16)
    assert_close_bf16(f32(out)[0], ref, "after the error was cleared")


FULL = MoEShape(2560, 256, 1024, 8, 1024)


def test_decode_after_prefill_on_one_workspace(gpu):
    """T > 1 calls write their scratch where a T = 1 call's hand-off words used to lie; the first
    decode after them must equal a decode on a fresh workspace bit for bit (block and experts-only)."""
    layer = seeded.make_layer(FULL, 77, device=gpu)
    table = tm.expert_table(layer.gate_up, layer.down)
    x1 = seeded.make_tokens(FULL, 77, 1, device=gpu)
    ids1 = torch.tensor([[5, 200, 17, 99, 31, 250, 0, 128]], device=gpu)
    w1 = torch.tensor([[0.3, 0.2, 0.1, 0.1, 0.1, 0.08, 0.07, 0.05]], device=gpu).to(BF)
    fresh = Workspace(FULL, gpu)
    ref_blk, ref_ids, _ = tm.moe_block(FULL, x1, table, fresh, router_w=layer.router_w, shared=layer.shared)
    ref_ex = tm.experts_forward(FULL, x1, ids1, w1, table, Workspace(FULL, gpu))
    torch.cuda.synchronize()
    ref_blk, ref_ex = ref_blk.clone(), ref_ex.clone()
    ws = Workspace(FULL, gpu, tokens=32)
    for T in (2, 4, 8, 32):
        xT = seeded.make_tokens(FULL, 78, T, device=gpu)
        tm.moe_block(FULL, xT, table, ws, router_w=layer.router_w, shared=layer.shared)
        got, ids, _ = tm.moe_block(FULL, x1, table, ws, router_w=layer.router_w, shared=layer.shared)
        torch.cuda.synchronize()
        assert torch.equal(ids, ref_ids), f"ids after T={T}"
        assert torch.equal(got, ref_blk), f"block decode after a T={T} block"
        idsT = torch.stack([torch.randperm(FULL.num_experts)[:FULL.top_k] for _ in range(T)]).to(gpu)
        wT = torch.full((T, FULL.top_k), 0.125, device=gpu).to(BF)
        tm.experts_forward(FULL, xT, idsT, wT, table, ws)
        got = tm.experts_forward(FULL, x1, ids1, w1, table, ws)
        torch.cuda.synchronize()
        assert torch.equal(got, ref_ex), f"experts decode after a T={T} experts call"
    ws.status()
    fresh.status()
