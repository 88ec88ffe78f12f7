"""GPU parity of the small-batch experts path (2 <= T <= 16 tokens, bf16 experts) through the
C ABI against the oracle's T > 1 semantics (experts in ascending id, a bf16 rounding after
each add, then the shared expert; tarfa/engine/fused_int4.py:227-248).

Bars: top-k ids bit-exact; outputs within max-abs 2e-2 and rel-L2 1e-3 of the oracle.  Edge
cases the reference's index_add_ loop defines: a token listing one expert twice (each slot
adds the expert's output with its own weight), the skip sentinel E and invalid ids (reported),
one expert taking every token (a 16-row group), no expert at all (zero output, or the
residual on the layer entry), and workspace reuse across token counts.
"""
import numpy as np
import pytest
import torch

from oracle import moe
from tarfa_amd import seeded
from tarfa_amd import moe as tm
from tarfa_amd.moe import MoEShape, Workspace
from tests._util import assert_close_bf16, expert_dicts, f32

pytestmark = pytest.mark.gpu

MID = MoEShape(1024, 32, 512, 8, 512)
FULL = MoEShape(2560, 256, 1024, 8, 1024)


def _block_case(shape, T, seed, gpu, layer=None, ws=None):
    layer = layer or seeded.make_layer(shape, seed, device=gpu)
    ws = ws or Workspace(shape, gpu, tokens=T)
    table = tm.expert_table(layer.gate_up, layer.down)
    x = seeded.make_tokens(shape, seed, T, device=gpu)
    logits = seeded.make_logits(shape, seed, T, device=gpu)
    out, ids, w = tm.moe_block(shape, x, table, ws, logits=logits, shared=layer.shared)
    out, ids, w = out.clone(), ids.clone(), w.clone()
    ids_ref, w_ref, _ = moe.router_topk(logits.cpu().numpy(), shape.top_k)
    assert np.array_equal(ids.cpu().numpy(), ids_ref)
    xs = f32(x)
    gu, dn = expert_dicts(layer.gate_up, layer.down, ids_ref)
    routed = moe.experts_prefill(xs, ids_ref, f32(w), gu, dn, shape.num_experts)
    ref = routed
    if layer.shared is not None:
        ref = moe.add_bf16(routed, moe.shared_expert(xs, *[f32(t) for t in layer.shared]))
    assert_close_bf16(f32(out), ref, f"small-batch block T={T}")
    out2 = tm.experts_forward(shape, x, ids, w, table, ws)
    assert_close_bf16(f32(out2), routed, f"small-batch experts T={T}")
    ws.status()
    return layer, ws


@pytest.mark.parametrize("T", [2, 3, 4, 8, 16])
def test_small_batch_block_mid(gpu, T):
    _block_case(MID, T, 300 + T, gpu)


@pytest.mark.parametrize("T", [2, 4, 8, 16])
def test_small_batch_block_full_size(gpu, T):
    _block_case(FULL, T, 400 + T, gpu)


@pytest.mark.parametrize("shape,T,seed", [(MID, 2, 76), (MID, 6, 77), (FULL, 2, 78), (FULL, 16, 79)])
def test_small_batch_router_weights_path(gpu, shape, T, seed):
    """Router logits computed on the device (fp32 GEMV) before the small-batch experts, at the
    mid shape and at the full-size layer (H=2560, E=256) for the smallest and largest T.  At
    T = 2 the router launch also runs the shared expert's gate/up and gate, and the up launch
    its down (4-stage up tiles at H = 1024, 5-stage at H = 2560)."""
    layer = seeded.make_layer(shape, seed, device=gpu)
    ws = Workspace(shape, gpu, tokens=T)
    table = tm.expert_table(layer.gate_up, layer.down)
    x = seeded.make_tokens(shape, seed, T, device=gpu)
    out, ids, w = tm.moe_block(shape, x, table, ws, router_w=layer.router_w, shared=layer.shared)
    torch.cuda.synchronize()
    xs = f32(x)
    lg = moe.router_logits(xs, f32(layer.router_w))
    ids_ref, _, _ = moe.router_topk(lg, shape.top_k)
    clear = moe.topk_gaps(lg, shape.top_k) > 1e-4 * np.maximum(1.0, np.abs(lg).max(axis=-1))
    assert clear.all(), "seed gives a near-tie; pick another"
    assert np.array_equal(ids.cpu().numpy(), ids_ref)
    gu, dn = expert_dicts(layer.gate_up, layer.down, ids_ref)
    ref = moe.add_bf16(moe.experts_prefill(xs, ids_ref, f32(w), gu, dn, shape.num_experts),
                       moe.shared_expert(xs, *[f32(t) for t in layer.shared]))
    assert_close_bf16(f32(out), ref, f"small-batch block, device router, H={shape.hidden} T={T}")


def test_small_batch_duplicates_sentinel_hot_expert(gpu):
    """Caller ids with a repeated expert in one token, the sentinel E, and expert 5 in every
    token of a 16-token batch (one group of 16 rows)."""
    shape = MoEShape(1024, 32, 512, 4, 0)
    T = 16
    layer = seeded.make_layer(shape, 91, device=gpu)
    ws = Workspace(shape, gpu, tokens=T)
    table = tm.expert_table(layer.gate_up, layer.down)
    x = seeded.make_tokens(shape, 91, T, device=gpu)
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(0, 32, (T, 4), generator=g)
    ids[:, 0] = 5
    ids[3, 2] = ids[3, 1]                 # token 3 lists one expert twice
    ids[7, 3] = 32                        # the skip sentinel
    ids[9] = torch.tensor([5, 32, 32, 32])
    w = (torch.rand(T, 4, generator=g) * 0.5 + 0.1).to(torch.bfloat16)
    ids_d, w_d = ids.to(gpu), w.to(gpu)
    out = tm.experts_forward(shape, x, ids_d, w_d, table, ws)
    ids_np = ids.numpy()
    gu, dn = expert_dicts(layer.gate_up, layer.down, ids_np)
    ref = moe.experts_prefill(f32(x), ids_np, f32(w), gu, dn, shape.num_experts)
    assert_close_bf16(f32(out), ref, "duplicates / sentinel / hot expert")
    ws.status()                           # the sentinel is not an error
    bad = ids_d.clone()
    bad[2, 2] = 40
    tm.experts_forward(shape, x, bad, w_d, table, ws)
    with pytest.raises(RuntimeError, match="expert id"):
        ws.status()


def test_small_batch_no_expert(gpu):
    """Every slot the sentinel: no group and no shared expert, the output is written as zero."""
    shape = MoEShape(1024, 32, 512, 8, 0)
    T = 3
    layer = seeded.make_layer(shape, 12, device=gpu)
    ws = Workspace(shape, gpu, tokens=T)
    table = tm.expert_table(layer.gate_up, layer.down)
    x = seeded.make_tokens(shape, 12, T, device=gpu)
    ids = torch.full((T, 8), 32, dtype=torch.int64, device=gpu)
    w = torch.full((T, 8), 0.125, device=gpu).to(torch.bfloat16)
    out = tm.experts_forward(shape, x, ids, w, table, ws, out=torch.full_like(x, 7.0))
    assert torch.count_nonzero(out) == 0
    ws.status()


def test_small_batch_layer_entry(gpu):
    """tmoe_moe_layer_bf16 at T = 5: RMSNorm in, the block, the residual added in the combine."""
    shape, T = MID, 5
    layer = seeded.make_layer(shape, 55, device=gpu)
    gen = torch.Generator().manual_seed(55)
    ln_w = (torch.randn(shape.hidden, generator=gen) * 0.1).to(torch.bfloat16).to(gpu)
    h = (seeded.make_tokens(shape, 55, T, device=gpu).float() * 4.0).to(torch.bfloat16)
    table = tm.expert_table(layer.gate_up, layer.down)
    ws = Workspace(shape, gpu, tokens=T)
    logits = seeded.make_logits(shape, 55, T, device=gpu)
    out = tm.moe_layer(shape, h, ln_w, 1e-6, table, ws, logits=logits, shared=layer.shared)[0].clone()
    # The block on the oracle's normalised input; the device's x may differ from it by one
    # bf16 step in a few elements (its own fp32 order for mean(h^2)), hence two steps of slack.
    xn = torch.from_numpy(moe.rmsnorm(f32(h), f32(ln_w), 1e-6)).to(gpu, torch.bfloat16)
    y = tm.moe_block(shape, xn, table, Workspace(shape, gpu, tokens=T), logits=logits, shared=layer.shared)[0]
    ref = moe.moe_layer(f32(h), f32(y))
    got = f32(out)
    step = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -126))) - 7)
    assert np.all(np.abs(got - ref) <= 2e-2 + 2 * step)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 1e-3
    ws.status()


def test_small_batch_workspace_reuse(gpu):
    """One workspace through T = 16, 2, 16 (arrival counters return to zero after each call):
    the repeat gives identical bits."""
    shape = MID
    layer = seeded.make_layer(shape, 21, device=gpu)
    ws = Workspace(shape, gpu, tokens=16)
    table = tm.expert_table(layer.gate_up, layer.down)
    outs = []
    for T in (16, 2, 16):
        x = seeded.make_tokens(shape, 21, T, device=gpu)
        logits = seeded.make_logits(shape, 21, T, device=gpu)
        outs.append(tm.moe_block(shape, x, table, ws, logits=logits, shared=layer.shared)[0].clone())
    assert torch.equal(outs[0], outs[2])
    ws.status()
