"""GPU parity of the int4 fast mode (quantise, dequantise, fused dequant-GEMV decode).

Bars: the device quantiser and the dequantised bf16 values are bit-exact against
the CPU oracle (oracle/int4.py); the fast-mode layer output is within max-abs
2e-2 and rel-L2 1e-3 of the oracle's int4 FFN (fp32 GEMVs, act = bf16(silu(g) * u),
fp32 weighted sum over experts in router order, one bf16 cast; shared expert in
exact bf16 added as bf16(routed + bf16(gate * shared))).  An activation whose exact
value lies within fp32 error of a bf16 rounding midpoint may round either way (the
GEMV's fp32 summation order decides); the oracle enumerates both roundings of those
(int4.ffn_candidates) and the output is held to the bar against the closest.  The reference's own
self-test criterion (tarfa/engine/moe_kernel.py:128-145: max|err| / max|ref| < 2e-2
on random packed bytes with per-row scales) is checked as well.
"""
import numpy as np
import pytest
import torch

from oracle import bf16, int4, moe
from tarfa_amd import seeded
from tarfa_amd import moe as tm
from tarfa_amd.moe import MoEShape, Workspace
from tests._util import assert_close_any_bf16, assert_close_bf16, f32

pytestmark = pytest.mark.gpu

SMALL = MoEShape(1024, 32, 512, 8, 0)
FULL = MoEShape(2560, 256, 1024, 8, 1024)


def u16(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def test_quantize_and_dequant_bit_exact_seeded_experts(gpu):
    layer = seeded.make_layer(SMALL, 21, device=gpu)
    gq, gs = tm.quantize_int4(layer.gate_up)
    dq, ds = tm.quantize_int4(layer.down)
    gw = tm.dequant_int4(gq, gs)
    for e in (0, 13, 31):
        p_ref, s_ref = int4.quantize(f32(layer.gate_up[e]), 128)
        assert np.array_equal(gq[e].cpu().numpy(), p_ref), f"gate_up packed, expert {e}"
        assert np.array_equal(u16(gs[e]), s_ref), f"gate_up scales, expert {e}"
        assert np.array_equal(u16(gw[e]), int4.dequant(p_ref, s_ref, 128)), f"gate_up dequant, expert {e}"
        p_ref, s_ref = int4.quantize(f32(layer.down[e]), 128)
        assert np.array_equal(dq[e].cpu().numpy(), p_ref), f"down packed, expert {e}"
        assert np.array_equal(u16(ds[e]), s_ref), f"down scales, expert {e}"


def test_quantize_special_groups(gpu):
    """Zero groups, exact half-way quotients (round half to even), huge and tiny magnitudes, other G."""
    K = 256
    rows = []
    rows.append(np.zeros(K, np.float32))                                   # scale 0 -> every code 0
    r = np.zeros(K, np.float32)
    r[:10] = [7.0, 2.5, -3.5, 0.5, -0.5, 6.5, -6.5, 1.5, -2.5, 3.5]         # scale bf16(7/7) = 1
    r[128:131] = [-7.0, 4.5, -4.5]
    rows.append(r)
    rows.append(np.float32(3.0e38) * np.sign(np.linspace(-1, 1, K)).astype(np.float32))
    rows.append((np.arange(K, dtype=np.float32) - 128) * np.float32(1e-38))  # fp32 denormal quotients
    rng_ = np.random.default_rng(5)
    rows.append(rng_.standard_normal(K).astype(np.float32) * np.float32(0.02))
    w = bf16.to_f32(bf16.bits(np.stack(rows)))                              # exact bf16 values
    wt = torch.from_numpy(bf16.bits(w).view(np.int16)).view(torch.bfloat16).to(gpu)
    for G in (128, 32, 256):
        p, s = tm.quantize_int4(wt, G)
        p_ref, s_ref = int4.quantize(w, G)
        assert np.array_equal(p.cpu().numpy(), p_ref), f"packed G={G}"
        assert np.array_equal(u16(s), s_ref), f"scales G={G}"
        assert np.array_equal(u16(tm.dequant_int4(p, s, G)), int4.dequant(p_ref, s_ref, G)), f"dequant G={G}"
    codes = int4.codes(tm.quantize_int4(wt, 128)[0].cpu().numpy())
    assert np.all(codes[0] == 0)
    assert list(codes[1][:10]) == [7, 2, -4, 0, 0, 6, -6, 2, -2, 4]         # ties to even


def test_dequant_every_code_and_scale_pattern(gpu):
    """16 codes x every finite bf16 scale, dequantised on the device vs the oracle table."""
    s_bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    finite = (s_bits & 0x7F80) != 0x7F80
    s_bits = s_bits[finite]
    n = s_bits.size                                           # one row per scale, 16 codes each
    packed = np.tile(np.array([0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE], np.uint8), (n, 1))
    p = torch.from_numpy(packed).to(gpu)
    s = torch.from_numpy(s_bits.view(np.int16).reshape(n, 1)).view(torch.bfloat16).to(gpu)
    got = u16(tm.dequant_int4(p, s, 16))
    assert np.array_equal(got, int4.dequant(packed, s_bits.reshape(n, 1), 16))


def _q4_layer(layer):
    gq, gs = tm.quantize_int4(layer.gate_up)
    dq, ds = tm.quantize_int4(layer.down)
    return gq, gs, dq, ds


def _host_experts(q4, ids):
    gq, gs, dq, ds = q4
    return {int(e): (gq[e].cpu().numpy(), u16(gs[e]), dq[e].cpu().numpy(), u16(ds[e]))
            for e in ids if 0 <= int(e) < gq.shape[0]}


def _int4_ref(x, ids, w, ex, num_experts):
    """oracle int4 FFN over the valid slots in router order (the sentinel is skipped): the
    admissible outputs, the first being int4.ffn itself (see int4.ffn_candidates)."""
    sel = [(ex[int(e)], wj) for e, wj in zip(ids, w) if 0 <= int(e) < num_experts]
    if not sel:
        return [np.zeros_like(x)]
    return int4.ffn_candidates(x, [s[0] for s in sel], np.array([s[1] for s in sel], np.float32))


def _int4_block_case(shape, seed, gpu):
    layer = seeded.make_layer(shape, seed, device=gpu)
    q4 = _q4_layer(layer)
    table = tm.expert_table_q4(*q4)
    ws = Workspace(shape, gpu)
    x = seeded.make_tokens(shape, seed, 1, device=gpu)
    out, ids, w = tm.moe_block(shape, x, table, ws, router_w=layer.router_w, shared=layer.shared)
    torch.cuda.synchronize()
    xs = f32(x)[0]
    lg = moe.router_logits(f32(x), f32(layer.router_w))
    ids_ref, w_ref, _ = moe.router_topk(lg, shape.top_k)
    gaps = moe.topk_gaps(lg, shape.top_k)
    assert gaps[0] > 1e-5 * max(1.0, np.abs(lg).max()), "seed with a near-tie in the top-k"
    assert np.array_equal(ids.cpu().numpy(), ids_ref)
    ex = _host_experts(q4, ids_ref[0])
    routed = _int4_ref(xs, ids_ref[0], w_ref[0], ex, shape.num_experts)
    ref = routed
    if layer.shared is not None:
        sh = moe.shared_expert(xs, *[f32(t) for t in layer.shared])
        ref = [moe.add_bf16(r, sh) for r in routed]
    assert_close_any_bf16(f32(out)[0], ref, f"int4 block seed {seed}")
    # experts.forward boundary (routed experts only)
    out2 = tm.experts_forward(shape, x, ids, w, table, ws)
    assert_close_any_bf16(f32(out2)[0], routed, f"int4 experts seed {seed}")
    ws.status()


@pytest.mark.parametrize("seed", [0, 1])
def test_int4_decode_small_layer(gpu, seed):
    _int4_block_case(SMALL, seed, gpu)


def test_int4_decode_full_size_layer(gpu):
    _int4_block_case(FULL, 200, gpu)


def test_int4_reference_self_test_criterion(gpu):
    """moe_kernel.py:128-145 at its own shape (E=8, H=3072, I=1024): random packed bytes,
    per-row scales ~N(0, 0.02) (every group of a row shares the row's scale), x ~ 0.5 N(0,1),
    softmax routing weights; max|err| / max|ref| < 2e-2, and the layer tolerance vs the oracle."""
    E, H, I = 8, 3072, 1024
    g = torch.Generator().manual_seed(0)
    gup = torch.randint(0, 256, (E, 2 * I, H // 2), dtype=torch.uint8, generator=g)
    dp = torch.randint(0, 256, (E, H, I // 2), dtype=torch.uint8, generator=g)
    gus = (torch.randn(E, 2 * I, 1, generator=g) * 0.02).to(torch.bfloat16).expand(E, 2 * I, H // 128).contiguous()
    dss = (torch.randn(E, H, 1, generator=g) * 0.02).to(torch.bfloat16).expand(E, H, I // 128).contiguous()
    x = (torch.randn(1, H, generator=g) * 0.5).to(torch.bfloat16)
    rw = torch.softmax(torch.randn(E, generator=g), 0).to(torch.bfloat16).reshape(1, E)
    shape = MoEShape(H, E, I, E, 0)
    q4 = tuple(t.to(gpu) for t in (gup, gus, dp, dss))
    table = tm.expert_table_q4(*q4)
    ws = Workspace(shape, gpu)
    ids = torch.arange(E, device=gpu).reshape(1, E)
    out = tm.experts_forward(shape, x.to(gpu), ids, rw.to(gpu), table, ws)
    got = f32(out)[0]
    ex = {e: (gup[e].numpy(), u16(gus[e]), dp[e].numpy(), u16(dss[e])) for e in range(E)}
    ref = _int4_ref(f32(x)[0], list(range(E)), f32(rw)[0], ex, E)
    # the reference's fp32 _ref_ffn (moe_kernel.py:117-125), restated in fp64
    ref64 = np.zeros(H)
    for e in range(E):
        gw = int4.codes(gup[e].numpy()) * bf16.to_f32(u16(gus[e]))[:, :1].astype(np.float64)
        dw = int4.codes(dp[e].numpy()) * bf16.to_f32(u16(dss[e]))[:, :1].astype(np.float64)
        gu = gw @ f32(x)[0].astype(np.float64)
        a = gu[:I] / (1 + np.exp(-gu[:I])) * gu[I:]
        ref64 += float(f32(rw)[0, e]) * (dw @ a)
    rel = np.abs(got - ref64).max() / np.abs(ref64).max()
    assert rel < 2e-2, rel
    assert_close_any_bf16(got, ref, "moe_kernel self-test shape")
    ws.status()


def test_int4_sentinel_and_invalid_ids(gpu):
    shape = MoEShape(512, 16, 512, 4)
    layer = seeded.make_layer(shape, 9, device=gpu)
    q4 = _q4_layer(layer)
    table = tm.expert_table_q4(*q4)
    ws = Workspace(shape, gpu)
    x = seeded.make_tokens(shape, 9, 1, device=gpu)
    ids = torch.tensor([[3, 16, 7, 1]], device=gpu)             # 16 = the skip sentinel E
    w = torch.tensor([[0.4, 0.3, 0.2, 0.1]], device=gpu).to(torch.bfloat16)
    out = tm.experts_forward(shape, x, ids, w, table, ws)
    ref = _int4_ref(f32(x)[0], [3, 16, 7, 1], f32(w)[0], _host_experts(q4, [3, 7, 1]), 16)
    assert_close_any_bf16(f32(out)[0], ref, "int4 sentinel")
    ws.status()
    bad = torch.tensor([[3, 99, 7, 1]], device=gpu)
    tm.experts_forward(shape, x, bad, w, table, ws)
    with pytest.raises(RuntimeError, match="expert id"):
        ws.status()


def test_int4_and_bf16_calls_share_a_workspace(gpu):
    """Alternating bf16 and int4 calls on one workspace (one epoch counter) stay correct."""
    shape = SMALL
    layer = seeded.make_layer(shape, 4, device=gpu)
    q4 = _q4_layer(layer)
    t16, t4 = tm.expert_table(layer.gate_up, layer.down), tm.expert_table_q4(*q4)
    ws = Workspace(shape, gpu)
    x = seeded.make_tokens(shape, 4, 1, device=gpu)
    a16 = tm.moe_block(shape, x, t16, ws, router_w=layer.router_w)[0].clone()
    a4 = tm.moe_block(shape, x, t4, ws, router_w=layer.router_w)[0].clone()
    for _ in range(3):
        assert torch.equal(tm.moe_block(shape, x, t16, ws, router_w=layer.router_w)[0], a16)
        assert torch.equal(tm.moe_block(shape, x, t4, ws, router_w=layer.router_w)[0], a4)
    ws.status()


@pytest.mark.parametrize("T,shared,I", [(37, True, 512), (300, False, 512), (2, True, 512), (1024, True, 1024)])
def test_int4_prefill_matches_dequantised_bf16_chain(gpu, T, shared, I):
    """T > 1 in int4 mode: the reference dequantises each hit expert and runs the bf16 prefill
    chain on it (tarfa/engine/fused_int4.py:249-261), so the oracle is experts_prefill on the
    dequantised weights, combined in ascending expert id; the shared expert stays bf16."""
    shape = MoEShape(1024, 32, I, 8, I if shared else 0)   # T=1024: several tiles per block
    layer = seeded.make_layer(shape, 40 + T, device=gpu)
    q4 = _q4_layer(layer)
    table = tm.expert_table_q4(*q4)
    ws = Workspace(shape, gpu, tokens=T)
    x = seeded.make_tokens(shape, 40 + T, T, device=gpu)
    out, ids, w = tm.moe_block(shape, x, table, ws, router_w=layer.router_w, shared=layer.shared)
    torch.cuda.synchronize()
    lg = moe.router_logits(f32(x), f32(layer.router_w))
    ids_ref, w_ref, _ = moe.router_topk(lg, shape.top_k)
    gaps = moe.topk_gaps(lg, shape.top_k)
    clear = gaps > 1e-5 * np.maximum(1.0, np.abs(lg).max(axis=-1))
    assert np.array_equal(ids.cpu().numpy()[clear], ids_ref[clear])
    gq, gs, dq, ds = q4
    gu = {e: bf16.to_f32(int4.dequant(gq[e].cpu().numpy(), u16(gs[e]))) for e in range(shape.num_experts)}
    dn = {e: bf16.to_f32(int4.dequant(dq[e].cpu().numpy(), u16(ds[e]))) for e in range(shape.num_experts)}
    ids_d, w_d = ids.cpu().numpy(), f32(w)          # the device routing (ties near fp32 noise resolved alike)
    ref = moe.experts_prefill(f32(x), ids_d, w_d, gu, dn, shape.num_experts)
    if shared:
        ref = moe.add_bf16(ref, moe.shared_expert(f32(x), *[f32(t) for t in layer.shared]))
    assert_close_bf16(f32(out), ref, f"int4 prefill T={T}")
    # experts.forward boundary with the same routing
    out2 = tm.experts_forward(shape, x, ids, w, table, ws)
    assert_close_bf16(f32(out2), moe.experts_prefill(f32(x), ids_d, w_d, gu, dn, shape.num_experts), "int4 experts")
    ws.status()


@pytest.mark.parametrize("mode", ["int4", "bf16"])
def test_prefill_one_cycle_tiles(gpu, mode):
    """H = I = 512: each up-GEMM tile is a single 8-stage cycle (int4: the register-staged
    kernel takes it; bf16: the whole-line kernel's shortest K, two 4-stage cycles), and at
    T = 4096 over 16 experts (208 M-chunks) every persistent block walks several tiles, so a
    tile's successor is prepared within its own cycles; the outputs against the oracle's chain
    (int4: on the dequantised weights)."""
    shape = MoEShape(512, 16, 512, 8, 0)
    T = 4096
    layer = seeded.make_layer(shape, 77, device=gpu)
    if mode == "int4":
        q4 = _q4_layer(layer)
        table = tm.expert_table_q4(*q4)
        gq, gs, dq, ds = q4
        gu = {e: bf16.to_f32(int4.dequant(gq[e].cpu().numpy(), u16(gs[e]))) for e in range(shape.num_experts)}
        dn = {e: bf16.to_f32(int4.dequant(dq[e].cpu().numpy(), u16(ds[e]))) for e in range(shape.num_experts)}
    else:
        table = tm.expert_table(layer.gate_up, layer.down)
        gu = {e: f32(layer.gate_up[e]) for e in range(shape.num_experts)}
        dn = {e: f32(layer.down[e]) for e in range(shape.num_experts)}
    ws = Workspace(shape, gpu, tokens=T)
    x = seeded.make_tokens(shape, 77, T, device=gpu)
    out, ids, w = tm.moe_block(shape, x, table, ws, router_w=layer.router_w)
    torch.cuda.synchronize()
    ref = moe.experts_prefill(f32(x), ids.cpu().numpy(), f32(w), gu, dn, shape.num_experts)
    assert_close_bf16(f32(out), ref, f"{mode} prefill H=512 T=4096")
    ws.status()
