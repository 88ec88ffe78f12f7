"""GPU parity of the MoE sublayer entry points (tmoe_moe_layer_bf16 / _int4):
out = bf16(h + block(bf16(rmsnorm(h) * (1 + ln_w)))), transformers
modeling_qwen3_5_moe.py:800-814, 870-875.

The reference for out is the residual add of the oracle over the block entry point run on
the oracle's normalised input (the block itself is pinned against the oracle elsewhere).
The device forms x with its own fp32 summation order for mean(h^2), so x may differ from
the oracle's by one bf16 step in a few elements: outputs are held to the bf16 bars, and
tokens whose top-k has a near-tie are left out of the routing comparison.
"""
import numpy as np
import pytest
import torch

from oracle import bf16, moe
from tarfa_amd import seeded
from tarfa_amd import moe as tm
from tarfa_amd.moe import MoEShape, Workspace
from tests._util import f32

pytestmark = pytest.mark.gpu


def _case(shape, T, seed, gpu, q4):
    layer = seeded.make_layer(shape, seed, device=gpu)
    gen = torch.Generator().manual_seed(seed)
    ln_w = (torch.randn(shape.hidden, generator=gen) * 0.1).to(torch.bfloat16).to(gpu)
    h = (seeded.make_tokens(shape, seed, T, device=gpu).float() * 4.0).to(torch.bfloat16)
    eps = 1e-6
    # The table holds raw pointers: the quantised tensors must outlive every call.
    q4w = (*tm.quantize_int4(layer.gate_up), *tm.quantize_int4(layer.down)) if q4 else None
    table = tm.expert_table_q4(*q4w) if q4 else tm.expert_table(layer.gate_up, layer.down)
    ws = Workspace(shape, gpu, tokens=T)
    out, ids, w = tm.moe_layer(shape, h, ln_w, eps, table, ws, router_w=layer.router_w, shared=layer.shared)
    out = out.clone()
    ids = ids.clone()
    x_ref = moe.rmsnorm(f32(h), f32(ln_w), eps)
    xb = torch.from_numpy(x_ref).to(gpu, torch.bfloat16)
    ws2 = Workspace(shape, gpu, tokens=T)
    yb, ids_b, _ = tm.moe_block(shape, xb, table, ws2, router_w=layer.router_w, shared=layer.shared)
    torch.cuda.synchronize()
    lg = moe.router_logits(x_ref, f32(layer.router_w))
    ids_ref, _, _ = moe.router_topk(lg, shape.top_k)
    clear = moe.topk_gaps(lg, shape.top_k) > 1e-3 * np.maximum(1.0, np.abs(lg).max(axis=-1))
    assert clear.mean() > 0.8
    assert np.array_equal(ids.cpu().numpy()[clear], ids_ref[clear])
    assert np.array_equal(ids_b.cpu().numpy()[clear], ids_ref[clear])
    ref = moe.moe_layer(f32(h), f32(yb))
    # out carries the residual stream (|h| up to ~16 here): per element the block's own bar
    # (2e-2) plus two bf16 steps at the element's magnitude (one step in x moves a few
    # block outputs slightly; the add rounds once more).
    got, want = f32(out)[clear], ref[clear]
    step = np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 2.0 ** -126))) - 7)
    err = np.abs(got - want)
    same = (bf16.bits(got) == bf16.bits(want)).mean()
    rel = np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)
    assert np.all(err <= 2e-2 + 2 * step) and same > 0.99 and rel <= 1e-3, \
        f"layer T={T} q4={q4}: max err {err.max():.3e}, bit-same {same:.4f}, rel-L2 {rel:.2e}"
    ws.status()
    del q4w
    return out


@pytest.mark.parametrize("T,q4", [(1, False), (1, True), (37, False), (300, False), (300, True)])
def test_moe_layer_matches_block_on_normalised_input(gpu, T, q4):
    # H, I multiples of 512: the fused decode kernel (T = 1), the persistent GEMM at T = 300
    shape = MoEShape(1024, 32, 512, 8, 512)
    if T == 37:
        shape = MoEShape(256, 16, 128, 4, 128)    # the register-staged GEMM
    _case(shape, T, 70 + T, gpu, q4)


def test_moe_layer_unfused_decode_fallback(gpu):
    """k = 10 has no fused decode variant: x is normalised by its own kernel, the unfused
    decode runs on it and the residual is added after."""
    _case(MoEShape(512, 32, 256, 10, 0), 1, 91, gpu, False)


def test_moe_layer_repeat_is_bit_identical(gpu):
    shape = MoEShape(1024, 32, 512, 8, 512)
    a = _case(shape, 1, 80, gpu, False)
    b = _case(shape, 1, 80, gpu, False)
    assert torch.equal(a, b)
