"""CPU pins of the oracle against independent implementations (no GPU).

Each oracle function is checked against something other than its own formula:
torch's bf16 cast and op chain, transformers' Qwen3.5-MoE modules (the
third-party code the reference calls), brute-force one_hot/where, exhaustive
enumeration, a published known-answer vector, or the reference's own
known-answer criterion.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import bf16, int4, moe, rng
from tests._util import rel_l2

BF = torch.bfloat16


def tb(a):
    """numpy fp32 (bf16 values) -> torch bf16 (exact)."""
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(BF)


# ------------------------------------------------------------------ bf16

def test_bf16_rounding_matches_torch_random_patterns():
    g = np.random.default_rng(0)
    u = g.integers(0, 2 ** 32, 1 << 22, dtype=np.uint64).astype(np.uint32)
    f = u.view(np.float32)
    f = f[np.isfinite(f)]
    want = torch.from_numpy(f).to(BF).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bf16.bits(f), want)


def test_bf16_rounding_ties_and_edges():
    # exact ties (low half 0x8000) round to even; max finite rounds to inf like torch
    hi = np.arange(0, 1 << 16, dtype=np.uint32)
    f = ((hi << 16) | 0x8000).view(np.float32)
    f = f[np.isfinite(f)]
    want = torch.from_numpy(f).to(BF).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bf16.bits(f), want)
    edges = np.array([0.0, -0.0, 1e-45, -1e-45, 3.4028235e38, -3.4028235e38, np.inf, -np.inf], np.float32)
    want = torch.from_numpy(edges).to(BF).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bf16.bits(edges), want)
    assert np.isnan(bf16.to_f32(bf16.bits(np.array([np.nan], np.float32))))[0]


# ------------------------------------------------------------------ generator

def test_splitmix64_known_answer():
    # splitmix64.c (Vigna), state seeded with 1234567: first five outputs
    assert [int(v) for v in rng.hashes(1234567, 0, 5)] == [
        6457827717110365317, 3203168211198807973, 9817491932198370423,
        4593380528125082431, 16408922859458223821]


def test_generator_vectorised_equals_bigint():
    k = rng.key(42, rng.stream_id(rng.KIND_DOWN, 3, 17))
    h = rng.hashes(k, 1000, 64)
    for i in range(64):
        assert int(h[i]) == rng._mix_int(k + (1000 + i + 1) * rng.GOLDEN)
    # n16: the centred sum of the twelve 16-bit fields of hashes 3i .. 3i+2, times one fp32 constant
    z = rng.n16_f32(k, 64, 0.02, start=1000)
    for i in range(64):
        c = sum((rng._mix_int(k + (3 * (1000 + i) + j + 1) * rng.GOLDEN) >> s) & 0xFFFF
                for j in range(3) for s in (0, 16, 32, 48)) - 393210
        assert z[i] == np.float32(np.float32(c) * rng.scale16(0.02))
    # n32: the twelve 32-bit fields of hashes 6i .. 6i+5, in fp64, rounded once to fp32
    y = rng.n32_f32(k, 16, 1.0, start=77)
    for i in range(16):
        c = sum((rng._mix_int(k + (6 * (77 + i) + j + 1) * rng.GOLDEN) >> s) & 0xFFFFFFFF
                for j in range(6) for s in (0, 32)) - 6 * 0xFFFFFFFF
        assert y[i] == np.float32(c * (1.0 / rng.STD32))


def test_generator_moments_and_determinism():
    k = rng.key(7, rng.stream_id(rng.KIND_GATE_UP, 0, 1))
    a = rng.n16_f32(k, 1 << 20, 1.0)
    assert abs(a.mean()) < 5e-3 and abs(a.std() - 1.0) < 5e-3
    assert np.array_equal(a[1000:2000], rng.n16_f32(k, 1000, 1.0, start=1000))
    b = rng.n32_f32(k, 1 << 18, 1.0)
    assert abs(b.mean()) < 1e-2 and abs(b.std() - 1.0) < 1e-2
    assert np.array_equal(b[500:600], rng.n32_f32(k, 100, 1.0, start=500))
    # distinct streams are uncorrelated
    c = rng.n16_f32(rng.key(7, rng.stream_id(rng.KIND_GATE_UP, 0, 2)), 1 << 20, 1.0)
    assert abs(np.corrcoef(a, c)[0, 1]) < 5e-3


def test_generator_tails_are_close_to_normal():
    """Irwin-Hall n=12: excess kurtosis -1.2/12 = -0.1 and P(|z| > 3) = 0.002014 (the
    closed-form CDF of a sum of twelve uniforms), against 0 and 0.002700 for N(0, 1); |z| <= 6.
    The n=4 form (kurtosis -0.3, P(|z| > 3) = 0.00043, |z| <= 3.46) fails these bounds."""
    k = rng.key(9, rng.stream_id(rng.KIND_X, 0, 0))
    a = rng.n16_f32(k, 1 << 22, 1.0).astype(np.float64)
    kurt = np.mean(a ** 4) / np.mean(a ** 2) ** 2 - 3.0
    assert abs(kurt - (-0.1)) < 0.01
    tail = np.mean(np.abs(a) > 3.0)
    assert 0.0019 < tail < 0.00215
    assert np.abs(a).max() <= 6.0 + 1e-3
    b = rng.n32_f32(k, 1 << 20, 1.0).astype(np.float64)
    assert abs(np.mean(b ** 4) / np.mean(b ** 2) ** 2 - 3.0 - (-0.1)) < 0.02


# ------------------------------------------------------------------ router

@pytest.mark.parametrize("E,k", [(32, 8), (256, 8), (64, 4)])
def test_router_topk_matches_torch(E, k):
    logits = rng.tensor_f32(3, rng.KIND_LOGITS, (512, E), 1.0)
    assert np.min(moe.topk_gaps(logits, k)) > 0          # no ties: torch's order is defined
    ids, w, probs = moe.router_topk(logits, k)
    lt = torch.from_numpy(logits)
    p = torch.softmax(lt, dim=-1, dtype=torch.float)
    tv, ti = torch.topk(p, k, dim=-1)
    tv = (tv / tv.sum(dim=-1, keepdim=True)).to(BF)
    assert np.array_equal(ids, ti.numpy())
    tw = tv.float().numpy()
    assert np.mean(tw == w) > 0.99
    assert np.all(np.abs(tw - w) <= np.abs(tw) * 2.0 ** -7)   # at most one bf16 ulp apart
    assert np.allclose(probs, p.numpy(), rtol=1e-6, atol=1e-9)


def test_router_logits_and_transformers_router_fp32():
    from transformers.models.qwen3_5_moe import configuration_qwen3_5_moe as C, modeling_qwen3_5_moe as M
    H, E, k = 256, 32, 8
    cfg = C.Qwen3_5MoeTextConfig(hidden_size=H, num_experts=E, num_experts_per_tok=k, moe_intermediate_size=64)
    router = M.Qwen3_5MoeTopKRouter(cfg)
    wg = bf16.to_f32(rng.tensor_bf16(5, rng.KIND_ROUTER, (E, H), 0.02))
    x = bf16.to_f32(rng.tensor_bf16(5, rng.KIND_X, (64, H), 1.0))
    with torch.no_grad():
        router.weight.copy_(torch.from_numpy(wg))                  # fp32 module: fp32 logits
        tl, tw, ti = router(torch.from_numpy(x))
    lg = moe.router_logits(x, wg)
    np.testing.assert_allclose(lg, tl.numpy(), rtol=1e-5, atol=1e-5)
    assert np.min(moe.topk_gaps(lg, k)) > 1e-4
    ids, w, _ = moe.router_topk(lg, k)
    assert np.array_equal(ids, ti.numpy())
    np.testing.assert_allclose(w, tw.numpy(), rtol=2.0 ** -8)


def test_router_tie_breaks_to_lower_index():
    lg = np.array([[0.5, 1.0, 1.0, 0.2, 1.0, 0.9]], np.float32)
    ids, _, _ = moe.router_topk(lg, 3)
    assert ids.tolist() == [[1, 2, 4]]


@pytest.mark.parametrize("k,j", [(8, 5), (8, 1), (16, 8), (6, 4)])
def test_jtopk_truncate_matches_the_reference_lines_in_torch(k, j):
    """fused_int4.py:157-160 run in torch CPU bf16 (topk, gather, sum, divide) on untied weights
    whose kept values span few binades (the fp32 sum is then exact, so its order is moot)."""
    g = np.random.default_rng(k * 31 + j)
    for trial in range(50):
        w = bf16.rnd(g.uniform(0.02, 1.0, (7, k)).astype(np.float32))
        if any(len(set(r.tolist())) < k for r in w):
            continue                                    # torch's tie order is not defined
        ids = g.integers(0, 256, (7, k))
        tw, tid = tb(w), torch.from_numpy(ids)
        tv, ti = tw.topk(j, dim=-1)
        want_ids = torch.gather(tid, -1, ti)
        want_w = tv / tv.sum(dim=-1, keepdim=True)
        got_ids, got_w = moe.jtopk_truncate(ids, w, j)
        assert np.array_equal(got_ids, want_ids.numpy())
        assert np.array_equal(got_w, want_w.float().numpy())


def test_jtopk_truncate_ties_keep_the_lower_slot_and_passes_short_routings():
    w = bf16.rnd(np.array([[0.25, 0.5, 0.25, 0.5, 0.125, 0.25]], np.float32))
    ids = np.array([[10, 11, 12, 13, 14, 15]])
    got_ids, got_w = moe.jtopk_truncate(ids, w, 4)
    assert got_ids.tolist() == [[11, 13, 10, 12]]       # 0.5 (slots 1, 3), then 0.25 (slots 0, 2)
    s = bf16.rnd(np.float32(1.5))
    half, quarter = (np.asarray(bf16.rnd(np.float32(v) / s)).item() for v in (0.5, 0.25))
    assert got_w.tolist() == [[half] * 2 + [quarter] * 2]
    same_ids, same_w = moe.jtopk_truncate(ids, w, 6)   # k <= j: the routing is kept as it is
    assert np.array_equal(same_ids, ids) and np.array_equal(same_w, w)


# ------------------------------------------------------------------ dispatch

@pytest.mark.parametrize("T,k,E", [(1, 8, 32), (2, 2, 4), (7, 3, 5), (33, 8, 32), (64, 1, 16)])
def test_dispatch_matches_one_hot_where(T, k, E):
    g = np.random.default_rng(T * 100 + k)
    ids = np.stack([g.permutation(E)[:k] for _ in range(T)]).astype(np.int64)
    offsets, perm = moe.dispatch(ids, E)
    mask = F.one_hot(torch.from_numpy(ids), num_classes=E).permute(2, 1, 0)      # fused_int4.py:228
    hit = torch.greater(mask.sum(dim=(-1, -2)), 0).nonzero().flatten().tolist()   # :229
    rows, counts = [], np.zeros(E, np.int64)
    for e in hit:
        pos, tok = torch.where(mask[e])                                            # :241
        rows += (tok * k + pos).tolist()
        counts[e] = len(tok)
    assert perm.tolist() == rows
    assert offsets.tolist() == [0] + np.cumsum(counts).tolist()


def test_dispatch_drops_sentinel_and_out_of_range():
    ids = np.array([[0, 4], [4, 1], [2, 9]], np.int64)       # E = 4: id 4 is the sentinel, 9 invalid
    offsets, perm = moe.dispatch(ids, 4)
    assert offsets.tolist() == [0, 1, 2, 3, 3]
    assert perm.tolist() == [0, 3, 4]


# ------------------------------------------------------------------ expert compute

def _layer(seed, H, E, I, Is=0):
    gu = {e: bf16.to_f32(rng.tensor_bf16(seed, rng.KIND_GATE_UP, (2 * I, H), 0.02, 0, e)) for e in range(E)}
    dn = {e: bf16.to_f32(rng.tensor_bf16(seed, rng.KIND_DOWN, (H, I), 0.02, 0, e)) for e in range(E)}
    wg = bf16.to_f32(rng.tensor_bf16(seed, rng.KIND_ROUTER, (E, H), 0.02))
    sh = None
    if Is:
        sh = (bf16.to_f32(rng.tensor_bf16(seed, rng.KIND_SH_GATE, (Is, H), 0.02)),
              bf16.to_f32(rng.tensor_bf16(seed, rng.KIND_SH_UP, (Is, H), 0.02)),
              bf16.to_f32(rng.tensor_bf16(seed, rng.KIND_SH_DOWN, (H, Is), 0.02)),
              bf16.to_f32(rng.tensor_bf16(seed, rng.KIND_SH_GATEW, (H,), 0.02)))
    return gu, dn, wg, sh


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_decode_matches_reference_op_chain(seed):
    """The literal torch op sequence of fused_int4.py:180, 192-194 on CPU in bf16."""
    H, E, I, k = 1024, 32, 512, 8
    gu, dn, wg, _ = _layer(seed, H, E, I)
    x = bf16.to_f32(rng.tensor_bf16(seed, rng.KIND_X, (1, H), 1.0))
    ids, w, _ = moe.router_topk(moe.router_logits(x, wg), k)
    got = moe.experts_decode(x[0], ids[0], w[0], gu, dn, E)
    xt = tb(x[0])
    acc = torch.zeros_like(xt)
    rwl = tb(w[0])
    for j, e in enumerate(ids[0].tolist()):
        g, u = F.linear(xt, tb(gu[e])).chunk(2, dim=-1)
        acc = acc + rwl[j] * F.linear(F.silu(g) * u, tb(dn[e]))
    ref = acc.float().numpy()
    assert rel_l2(got, ref) <= 1e-3 and np.max(np.abs(got - ref)) <= 2e-2
    assert np.mean(got == ref) >= 0.95


def test_decode_order_matters():
    """Router order vs ascending-id order differ beyond the tolerance -- the pin is not vacuous."""
    H, E, I, k = 1024, 32, 512, 8
    gu, dn, wg, _ = _layer(11, H, E, I)
    x = bf16.to_f32(rng.tensor_bf16(11, rng.KIND_X, (1, H), 1.0))
    ids, w, _ = moe.router_topk(moe.router_logits(x, wg), k)
    a = moe.experts_decode(x[0], ids[0], w[0], gu, dn, E)
    o = np.argsort(ids[0])
    b = moe.experts_decode(x[0], ids[0][o], w[0][o], gu, dn, E)
    assert rel_l2(a, b) > 1e-3


def _tf_block(H, E, I, k, Is):
    from transformers.models.qwen3_5_moe import configuration_qwen3_5_moe as C, modeling_qwen3_5_moe as M
    cfg = C.Qwen3_5MoeTextConfig(hidden_size=H, num_experts=E, moe_intermediate_size=I, num_experts_per_tok=k,
                                 shared_expert_intermediate_size=Is, hidden_act="silu")
    return M.Qwen3_5MoeSparseMoeBlock(cfg).to(BF)


def _load_tf_block(blk, gu, dn, wg, sh):
    E = len(gu)
    with torch.no_grad():
        blk.experts.gate_up_proj.copy_(torch.stack([tb(gu[e]) for e in range(E)]))
        blk.experts.down_proj.copy_(torch.stack([tb(dn[e]) for e in range(E)]))
        blk.gate.weight.copy_(tb(wg))
        if sh is not None:
            blk.shared_expert.gate_proj.weight.copy_(tb(sh[0]))
            blk.shared_expert.up_proj.weight.copy_(tb(sh[1]))
            blk.shared_expert.down_proj.weight.copy_(tb(sh[2]))
            blk.shared_expert_gate.weight.copy_(tb(sh[3]).reshape(1, -1))


@pytest.mark.parametrize("T", [2, 16, 40])
def test_prefill_matches_transformers_eager_experts(T):
    """transformers' eager Qwen3_5MoeExperts.forward is the loop the reference restates (channel.py:44-60)."""
    H, E, I, k = 128, 8, 64, 4
    gu, dn, wg, _ = _layer(T, H, E, I)
    blk = _tf_block(H, E, I, k, 64)
    _load_tf_block(blk, gu, dn, wg, None)
    x = bf16.to_f32(rng.tensor_bf16(T, rng.KIND_X, (T, H), 1.0))
    ids, w, _ = moe.router_topk(moe.router_logits(x, wg), k)
    with torch.no_grad():
        ref = blk.experts(tb(x), torch.from_numpy(ids), tb(w)).float().numpy()
    got = moe.experts_prefill(x, ids, w, gu, dn, E)
    assert rel_l2(got, ref) <= 1e-3 and np.max(np.abs(got - ref)) <= 2e-2
    assert np.mean(got == ref) >= 0.95


def test_block_composition_matches_transformers():
    """Shared MLP, sigmoid gate and the routed-first final add (modeling_qwen3_5_moe.py:787-798)."""
    H, E, I, k, Is, T = 128, 8, 64, 2, 64, 12
    gu, dn, wg, sh = _layer(21, H, E, I, Is)
    blk = _tf_block(H, E, I, k, Is)
    _load_tf_block(blk, gu, dn, wg, sh)
    x = bf16.to_f32(rng.tensor_bf16(21, rng.KIND_X, (T, H), 1.0))
    with torch.no_grad():
        ref = blk(tb(x).reshape(1, T, H)).reshape(T, H).float().numpy()
        _, tw, ti = blk.gate(tb(x))                      # the module's own (bf16-logit) routing
    routed = moe.experts_prefill(x, ti.numpy(), tw.float().numpy(), gu, dn, E)
    got = moe.add_bf16(routed, moe.shared_expert(x, *sh))
    assert rel_l2(got, ref) <= 1e-3 and np.max(np.abs(got - ref)) <= 2e-2
    with torch.no_grad():
        s_ref = (torch.sigmoid(blk.shared_expert_gate(tb(x))) * blk.shared_expert(tb(x))).float().numpy()
    assert rel_l2(moe.shared_expert(x, *sh), s_ref) <= 1e-3


# ------------------------------------------------------------------ int4

def test_dequant_exhaustive_codes_times_all_bf16_scales():
    """16 codes x every finite bf16 scale vs torch ``q.to(bf16) * scale`` (channel_q4.py:14 with dtype bf16)."""
    sb = np.arange(1 << 16, dtype=np.uint16)
    s = bf16.to_f32(sb)
    sb = sb[np.isfinite(s)]
    packed = np.repeat(np.arange(16, dtype=np.uint8) | (np.arange(16, dtype=np.uint8)[::-1] << 4), 1)[None, :]
    packed = np.repeat(packed, sb.size, axis=0)                # [n_scales, 16] -> K = 32
    scales = sb[:, None]                                       # group = K = 32
    got = int4.dequant(packed, scales, group=32)
    q = torch.from_numpy(int4.codes(packed)).to(torch.int16)   # int16 codes like channel_q4.py:11-12
    want = (q.to(BF) * torch.from_numpy(bf16.to_f32(scales)).to(BF)).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


def test_codes_nibble_order_matches_reference_dequant():
    """Low nibble -> even k, high nibble -> odd k (moe_kernel.py:110-114 restated in torch)."""
    g = np.random.default_rng(1)
    packed = g.integers(0, 256, (8, 16), dtype=np.uint8)
    p = torch.from_numpy(packed)
    lo = (p & 0xF).to(torch.int16) - 8
    hi = ((p >> 4) & 0xF).to(torch.int16) - 8
    q = torch.stack([lo, hi], dim=-1).reshape(p.shape[0], -1)
    assert np.array_equal(int4.codes(packed), q.numpy())


def test_quantizer_invariants():
    w = bf16.to_f32(rng.tensor_bf16(9, rng.KIND_GATE_UP, (64, 512), 0.02))
    w[3, :128] = 0.0                                             # an all-zero group
    packed, sb = int4.quantize(w, 128)
    q = int4.codes(packed)
    s = np.repeat(bf16.to_f32(sb), 128, axis=-1)
    assert q.min() >= -7 and q.max() <= 7                        # s = max/7 never needs -8
    assert np.all(q[3, :128] == 0) and np.all(bf16.to_f32(sb)[3, 0] == 0)
    wh = bf16.to_f32(int4.dequant(packed, sb, 128))
    assert np.all(np.abs(w - q * s) <= s / 2 * (1 + 2.0 ** -7) + 1e-30)
    assert np.all(np.abs(wh - q * s) <= np.abs(q * s) * 2.0 ** -8)
    # exactly representable inputs round-trip
    s0 = np.float32(0.015625)
    qq = np.tile(np.arange(-7, 8, dtype=np.float32), 9)[:128]
    qq[0] = 7
    p2, s2 = int4.quantize((qq * s0)[None, :], 128)
    assert np.array_equal(int4.codes(p2)[0], qq.astype(np.int32))


def test_int4_ffn_reference_known_answer_criterion():
    """moe_kernel.py:128-145: random packed weights, fp16-like per-row scales, pass if max|err|/max|ref| < 2e-2.

    Group = K reproduces the reference's per-row scale; the reference _ref_ffn
    (moe_kernel.py:117-125) is restated in torch fp64.
    """
    torch.manual_seed(0)
    E, H, I = 4, 256, 128
    g = np.random.default_rng(0)
    gup = g.integers(0, 256, (E, 2 * I, H // 2), dtype=np.uint8)
    dp = g.integers(0, 256, (E, H, I // 2), dtype=np.uint8)
    gus = bf16.bits(g.standard_normal((E, 2 * I, 1)).astype(np.float32) * 0.02)
    ds = bf16.bits(g.standard_normal((E, H, 1)).astype(np.float32) * 0.02)
    x = bf16.rnd(g.standard_normal(H).astype(np.float32) * 0.5)
    rw = bf16.rnd(torch.softmax(torch.randn(E), 0).numpy())
    out = torch.zeros(H, dtype=torch.float64)
    for e in range(E):
        gw = torch.from_numpy(int4.codes(gup[e])).double() * torch.from_numpy(bf16.to_f32(gus[e])).double()
        dw = torch.from_numpy(int4.codes(dp[e])).double() * torch.from_numpy(bf16.to_f32(ds[e])).double()
        gu_ = gw @ torch.from_numpy(x).double()
        gg, uu = gu_.chunk(2)
        out += float(rw[e]) * (dw @ (F.silu(gg) * uu))
    ref = out.numpy()
    got = _ffn_rowscale(x, gup, gus, dp, ds, rw)
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) < 2e-2


def _ffn_rowscale(x, gup, gus, dp, ds, rw):
    """oracle int4.ffn with one scale per row: group = K for each projection."""
    E = gup.shape[0]
    y = np.zeros(x.shape[0], np.float64)
    for e in range(E):
        gu = int4.gemv_f32(gup[e], gus[e], x, group=gup.shape[2] * 2).astype(np.float64)
        inter = gu.shape[0] // 2
        gg, uu = gu[:inter], gu[inter:]
        act = bf16.rnd(((gg / (1 + np.exp(-gg))) * uu).astype(np.float32))
        d = int4.gemv_f32(dp[e], ds[e], act, group=dp.shape[2] * 2).astype(np.float64)
        y = (y + (d * float(rw[e])).astype(np.float32)).astype(np.float32).astype(np.float64)
    return bf16.rnd(y.astype(np.float32))


def test_int4_ffn_group_form_equals_rowscale_form_when_scales_repeat():
    """With every group scale of a row equal, the group-128 ffn equals the per-row form exactly."""
    g = np.random.default_rng(3)
    E, H, I = 2, 256, 128
    gup = g.integers(0, 256, (E, 2 * I, H // 2), dtype=np.uint8)
    dp = g.integers(0, 256, (E, H, I // 2), dtype=np.uint8)
    gus = bf16.bits(g.standard_normal((E, 2 * I, 1)).astype(np.float32) * 0.02)
    ds = bf16.bits(g.standard_normal((E, H, 1)).astype(np.float32) * 0.02)
    x = bf16.rnd(g.standard_normal(H).astype(np.float32))
    rw = bf16.rnd(np.array([0.6, 0.4], np.float32))
    a = _ffn_rowscale(x, gup, gus, dp, ds, rw)
    b = int4.ffn(x, [(gup[e], np.repeat(gus[e], 2, -1), dp[e], ds[e]) for e in range(E)], rw, group=128)
    assert rel_l2(a, b) < 1e-6


def _distinct_group_scales(g, shape):
    """bf16 scale bits whose groups within a row all differ: each group of a row takes its own
    binade (a per-row permutation of 2^-10 .. 2^(ng - 11)) with a random mantissa."""
    ng = shape[-1]
    rows = int(np.prod(shape[:-1]))
    exps = np.stack([g.permutation(ng) for _ in range(rows)]).reshape(shape) - 10
    s = bf16.bits((2.0 ** exps * g.uniform(1.0, 2.0, shape)).astype(np.float32))
    assert all(len(set(row.tolist())) == ng for row in s.reshape(-1, ng))
    return s


def test_int4_gemv_group_scales_closed_form():
    """gemv_f32 with a distinct scale per (row, group) against the dequantise-then-multiply closed
    form sum_k q[n,k] * s[n, k // G] * x[k] in fp64 (np.repeat expands each scale over its group).
    A scale indexed by k % n_groups (np.tile) instead of k // G misses by far more than rounding."""
    g = np.random.default_rng(11)
    N, K, G = 48, 640, 128
    packed = g.integers(0, 256, (N, K // 2), dtype=np.uint8)
    sb = _distinct_group_scales(g, (N, K // G))
    x = bf16.rnd(g.standard_normal(K).astype(np.float32))
    s = bf16.to_f32(sb).astype(np.float64)
    q = int4.codes(packed).astype(np.float64)
    ref = (q * np.repeat(s, G, axis=-1)) @ x.astype(np.float64)
    got = int4.gemv_f32(packed, sb, x, G).astype(np.float64)
    assert np.all(np.abs(got - ref) <= 2.0 ** -23 * np.abs(ref) + 1e-30)
    wrong = (q * np.tile(s, (1, G))) @ x.astype(np.float64)
    assert rel_l2(wrong, ref) > 0.1


def test_int4_gemv_group_scales_brute_force_2x256():
    """Two rows of 256 columns, two groups each, summed term by term in Python floats."""
    g = np.random.default_rng(12)
    packed = g.integers(0, 256, (2, 128), dtype=np.uint8)
    sb = _distinct_group_scales(g, (2, 2))
    x = bf16.rnd(g.standard_normal(256).astype(np.float32))
    got = int4.gemv_f32(packed, sb, x, 128)
    for n in range(2):
        acc = 0.0
        for k in range(256):
            byte = int(packed[n, k // 2])
            nib = (byte & 0xF) if k % 2 == 0 else (byte >> 4)
            scale = float(bf16.to_f32(np.array([sb[n, k // 128]], np.uint16))[0])
            acc += (nib - 8) * scale * float(x[k])
        assert abs(float(got[n]) - acc) <= 2.0 ** -23 * abs(acc) + 1e-30


def test_int4_ffn_group_scales_against_fp64_dequantised_ffn():
    """ffn with distinct group scales against the reference's _ref_ffn semantics
    (moe_kernel.py:117-125, dequantise then fp64 products) written on dequantised matrices;
    the reference's own criterion max|err| / max|ref| < 2e-2, and the rel-L2 bar of the path."""
    g = np.random.default_rng(13)
    E, H, I = 3, 512, 256
    x = bf16.rnd(g.standard_normal(H).astype(np.float32))
    rw = bf16.rnd(np.array([0.5, 0.3, 0.2], np.float32))
    experts, ref = [], np.zeros(H, np.float64)
    for e in range(E):
        gq = g.integers(0, 256, (2 * I, H // 2), dtype=np.uint8)
        dq = g.integers(0, 256, (H, I // 2), dtype=np.uint8)
        gs = _distinct_group_scales(g, (2 * I, H // 128))
        ds = _distinct_group_scales(g, (H, I // 128))
        experts.append((gq, gs, dq, ds))
        wg = int4.codes(gq) * np.repeat(bf16.to_f32(gs).astype(np.float64), 128, axis=-1)
        wd = int4.codes(dq) * np.repeat(bf16.to_f32(ds).astype(np.float64), 128, axis=-1)
        gu = torch.from_numpy(wg @ x.astype(np.float64))
        a = F.silu(gu[:I]) * gu[I:]
        ref += float(rw[e]) * (wd @ a.numpy())
    got = int4.ffn(x, experts, rw, 128).astype(np.float64)
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) < 2e-2
    assert rel_l2(got, ref) < 5e-3


def test_int4_ambiguous_roundings_known_answers():
    v = np.array([1.12109375 + 1e-7, 1.12107, 1.5, -1.12109375 - 2e-7, 3.0, 1.0], np.float32)
    idx, other, dist = int4.ambiguous_roundings(v, 2e-6)
    assert list(idx) == [0, 3]
    # 1.12109375 is the midpoint of bf16 1.1171875 (0x3F8F) and 1.125 (0x3F90)
    assert bf16.bits(v[0]) == 0x3F90 and other[0] == 0x3F8F
    assert bf16.bits(v[3]) == 0xBF90 and other[1] == 0xBF8F
    assert np.all(dist < 3e-7)
    idx, _, _ = int4.ambiguous_roundings(v, 0.0)
    assert idx.size == 0


def test_int4_ffn_candidates_first_is_ffn_and_count():
    g = np.random.default_rng(3)
    H, I, E = 256, 128, 3
    ex = []
    for e in range(E):
        gq, gs = int4.quantize(g.standard_normal((2 * I, H)).astype(np.float32) * 0.02, 128)
        dq, ds = int4.quantize(g.standard_normal((H, I)).astype(np.float32) * 0.02, 128)
        ex.append((gq, gs, dq, ds))
    x = bf16.rnd(g.standard_normal(H).astype(np.float32))
    rw = bf16.rnd(np.array([0.5, 0.3, 0.2], np.float32))
    outs = int4.ffn_candidates(x, ex, rw)
    assert np.array_equal(outs[0], int4.ffn(x, ex, rw))
    # every activation "ambiguous": 2^max_flips candidates
    outs = int4.ffn_candidates(x, ex, rw, rel=1.0, max_flips=2)
    assert len(outs) == 4
    assert np.array_equal(outs[0], int4.ffn(x, ex, rw))


# ------------------------------------------------------------------ route telemetry (a13)
def test_route_telemetry_known_answers():
    """Hand-worked sequence through the restatement of fused_int4.py:71-84."""
    from oracle.telemetry import RouteTelemetry
    t = RouteTelemetry(2)
    E = 10
    t.record(0, [1, 2, 3], E)            # nothing seen before
    t.record(0, [3, 4, 10], E)           # 10 = sentinel dropped; 3 reused from 1 step back
    t.record(0, [10, 10, 10], E)         # all sentinel: not recorded
    t.record(0, [1, 4, 5], E)            # 4 one back, 1 two back
    t.record(1, [7, 7, 8], E)            # list of 3 uses, set of 2
    st = t.per_layer[0]
    assert st["decode_steps"] == 3 and st["expert_uses"] == 3 + 2 + 3
    assert st["reuse_1"] == 1 + 1 and st["reuse_2"] == 1 + 2 and st["reuse_16"] == 3
    assert t.per_layer[1]["expert_uses"] == 3 and t.per_layer[1]["reuse_1"] == 0
    tot = t.totals()
    assert tot["unique_layer_experts"] == 5 + 2
    # 17 steps later expert 1 falls out of every window
    for s in range(16):
        t.record(0, [9], E)
    before = t.per_layer[0]["reuse_16"]
    t.record(0, [1], E)
    assert t.per_layer[0]["reuse_16"] == before


def test_expert_bytes_match_the_workload_definition():
    from tarfa_amd.moe import MoEShape
    from tarfa_amd.residency import expert_bytes
    s = MoEShape(2560, 256, 1024, 8, 1024)
    assert expert_bytes(s) == 15_728_640             # 3 x 2560 x 1024 x 2 B
    assert expert_bytes(s, int4=True) == 4_055_040   # 3,932,160 packed + 122,880 scale bytes


def test_zipf_logits_follow_the_rank_weights():
    """Gumbel-top-k of log w + Gumbel samples without replacement with P proportional to w:
    the empirical top-1 frequency of each expert matches w / sum(w) (chi-square-level check)."""
    import torch
    from tarfa_amd.moe import MoEShape
    from tarfa_amd.residency import zipf_logits
    s = MoEShape(64, 32, 8, 4)
    T = 20000
    lg, ranks = zipf_logits(s, 2, T, seed=7, device="cpu")
    assert lg.shape == (T, 2, 32) and lg.dtype == torch.float32
    top1 = lg.argmax(-1)                                     # [T, L]
    w = (ranks.double() + 1.0) ** -1.1                       # [L, E]
    p = (w / w.sum(-1, keepdim=True)).numpy()
    for l in range(2):
        freq = np.bincount(top1[:, l].numpy(), minlength=32) / T
        assert np.all(np.abs(freq - p[l]) < 5 * np.sqrt(p[l] * (1 - p[l]) / T) + 1e-3)
    # popularity by rank is monotone in the k-selection counts too (top-4 of 32)
    sel = torch.zeros(2, 32)
    for l in range(2):
        sel[l].scatter_add_(0, lg[:, l].topk(4, -1).indices.reshape(-1), torch.ones(T * 4))
        by_rank = sel[l][torch.argsort(ranks[l])]
        assert by_rank[0] > by_rank[4] > by_rank[16] > by_rank[31]


# ------------------------------------------------------------------ int4, the reference's per-row fp16 layout

def test_dequant_f16_exhaustive_codes_times_all_fp16_scales():
    """16 codes x every finite fp16 scale vs channel_q4.py:10-14 run in torch CPU fp16."""
    sb = np.arange(1 << 16, dtype=np.uint16)
    sb = sb[np.isfinite(sb.view(np.float16))]
    packed = (np.arange(16, dtype=np.uint8) | (np.arange(16, dtype=np.uint8)[::-1] << 4))[None, :]
    packed = np.repeat(packed, sb.size, axis=0)                 # [n, 16] -> K = 32, one scale per row
    got = int4.dequant_f16(packed, sb[:, None], group=32)
    p = torch.from_numpy(packed)
    lo = (p & 0xF).to(torch.int16) - 8
    hi = ((p >> 4) & 0xF).to(torch.int16) - 8
    q = torch.stack([lo, hi], dim=-1).reshape(p.shape[0], -1)
    scale = torch.from_numpy(sb.view(np.int16)).view(torch.float16)
    want = (q.to(torch.float16) * scale[:, None]).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


def _ref_ffn_fp16_rows(x, gup, gus, dp, ds, rw):
    """The reference's _ref_ffn (moe_kernel.py:117-125): fp16 dequant (channel_q4.py:10-14)
    with per-row fp16 scales, .float(), fp32 matmuls, written as the reference writes it."""
    out = torch.zeros(x.shape[0], dtype=torch.float32)
    xf = torch.from_numpy(np.asarray(x, np.float32))
    for e in range(gup.shape[0]):
        def deq(pk, sc):
            p = torch.from_numpy(pk)
            lo = (p & 0xF).to(torch.int16) - 8
            hi = ((p >> 4) & 0xF).to(torch.int16) - 8
            q = torch.stack([lo, hi], dim=-1).reshape(p.shape[0], -1)
            return q.to(torch.float16) * torch.from_numpy(sc.view(np.int16)).view(torch.float16)[:, None]
        gw, dw = deq(gup[e], gus[e]).float(), deq(dp[e], ds[e]).float()
        gu = gw @ xf
        g, u = gu.chunk(2)
        a = F.silu(g) * u
        out += float(rw[e]) * (dw @ a)
    return out.numpy()


def test_int4_ffn_rows_against_reference_ref_ffn():
    """ffn_rows vs the reference's own closed form on its per-row fp16 layout (random packed
    weights, fp16 scales ~N(0, 0.02), x ~ 0.5 N(0, 1): the data of moe_kernel.py:128-139);
    the reference's criterion max|err| / max|ref| < 2e-2 and a tighter rel-L2."""
    g = np.random.default_rng(7)
    E, H, I = 4, 512, 256
    gup = g.integers(0, 256, (E, 2 * I, H // 2), dtype=np.uint8)
    dp = g.integers(0, 256, (E, H, I // 2), dtype=np.uint8)
    gus = (g.standard_normal((E, 2 * I)) * 0.02).astype(np.float16).view(np.uint16)
    ds = (g.standard_normal((E, H)) * 0.02).astype(np.float16).view(np.uint16)
    x = bf16.rnd(g.standard_normal(H).astype(np.float32) * 0.5)
    rw = bf16.rnd(torch.softmax(torch.from_numpy(g.standard_normal(E).astype(np.float32)), 0).numpy())
    ref = _ref_ffn_fp16_rows(x, gup, gus, dp, ds, rw)
    got = int4.ffn_rows(x, [(gup[e], gus[e], dp[e], ds[e]) for e in range(E)], rw)
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) < 2e-2
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-2   # the reference's bf16 act rounding aside


def test_int4_gemv_rows_brute_force():
    """gemv_rows against a plain double loop on a 3 x 64 case with distinct row scales."""
    g = np.random.default_rng(11)
    pk = g.integers(0, 256, (3, 32), dtype=np.uint8)
    sc = np.array([0.5, -0.0625, 3.0], np.float16).view(np.uint16)
    x = g.standard_normal(64).astype(np.float32)
    got = int4.gemv_rows(pk, sc, x)
    for n in range(3):
        acc = 0.0
        for b in range(32):
            acc += ((int(pk[n, b]) & 0xF) - 8) * float(x[2 * b]) + ((int(pk[n, b]) >> 4) - 8) * float(x[2 * b + 1])
        want = np.float32(np.float32(acc) * np.float32(np.array(sc[n], np.uint16).view(np.float16)))
        assert got[n] == want


def test_int4_dequant_rows_bf16_matches_torch():
    g = np.random.default_rng(12)
    pk = g.integers(0, 256, (64, 64), dtype=np.uint8)
    sc = (g.standard_normal(64) * 0.02).astype(np.float16).view(np.uint16)
    got = int4.dequant_rows_bf16(pk, sc)
    q = torch.from_numpy(int4.codes(pk)).float()
    s = torch.from_numpy(sc.view(np.int16)).view(torch.float16).float()[:, None]
    want = (q * s).to(BF).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
