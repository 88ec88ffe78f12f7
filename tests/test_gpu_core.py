"""GPU parity of the HIP path (through the C ABI) against the CPU oracle.

Bars: bit-exact for the generator, top-k ids and the dispatch permutation;
bf16 layer outputs within max-abs 2e-2 and rel-L2 1e-3 (accumulation order:
bf16 rounding after each GEMV, SiLU, multiply, weight-scale and add; decode in
router order, prefill in ascending expert id).
"""
import numpy as np
import pytest
import torch

from oracle import bf16, moe, rng
from tarfa_amd import seeded
from tarfa_amd import moe as tm
from tarfa_amd.moe import MoEShape, Workspace
from tests._util import assert_close_bf16, expert_dicts, f32

pytestmark = pytest.mark.gpu

SMALL = MoEShape(1024, 32, 512, 8, 0)            # the reference-CPU-sized layer
FULL = MoEShape(2560, 256, 1024, 8, 1024)        # full-size layer with a shared expert


def bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def test_fill_matches_oracle_generator(gpu):
    for n, start in ((1003, 0), (4096, 77), (8, 1 << 33)):
        k = rng.key(11, rng.stream_id(rng.KIND_GATE_UP, 2, 5))
        t = torch.empty(n, dtype=torch.bfloat16, device=gpu)
        tm.fill_bf16(t, k, 0.02, start=start)
        assert np.array_equal(bits(t), rng.n16_bf16_bits(k, n, 0.02, start=start))
        f = torch.empty(n, dtype=torch.float32, device=gpu)
        tm.fill_f32(f, k, 1.0, start=start)
        assert np.array_equal(f.cpu().numpy(), rng.n32_f32(k, n, 1.0, start=start))
    layer = seeded.make_layer(SMALL, seed=3, layer=1, device=gpu)
    for e in (0, 17, 31):
        want = rng.tensor_bf16(3, rng.KIND_GATE_UP, (1024, 1024), 0.02, 1, e)
        assert np.array_equal(bits(layer.gate_up[e]), want)
        want = rng.tensor_bf16(3, rng.KIND_DOWN, (1024, 512), 0.02, 1, e)
        assert np.array_equal(bits(layer.down[e]), want)
    assert np.array_equal(bits(layer.router_w), rng.tensor_bf16(3, rng.KIND_ROUTER, (32, 1024), 0.02, 1))


def _check_routing(ids, w, logits_ref, k, what):
    """Top-k ids equal wherever the oracle's top-(k+1) gap exceeds fp32 dot-order noise."""
    ids_ref, w_ref, _ = moe.router_topk(logits_ref, k)
    gaps = moe.topk_gaps(logits_ref, k)
    clear = gaps > 1e-5 * np.maximum(1.0, np.abs(logits_ref).max(axis=-1))
    assert clear.mean() > 0.95, f"{what}: too many near-ties ({(~clear).sum()})"
    assert np.array_equal(ids[clear], ids_ref[clear]), f"{what}: top-k ids differ"
    wd = np.abs(w[clear] - w_ref[clear])
    assert np.all(wd <= np.abs(w_ref[clear]) * 2.0 ** -7), f"{what}: routing weights beyond one bf16 ulp"
    return ids_ref, w_ref


@pytest.mark.parametrize("H,E,k,T", [(1024, 32, 8, 64), (2560, 256, 8, 64), (512, 64, 4, 7), (2560, 256, 8, 1000),
                                     (1024, 32, 8, 333), (2560, 256, 8, 40), (1024, 100, 6, 200)])
def test_router_topk_multi_token(gpu, H, E, k, T):
    shape = MoEShape(H, E, 256, k)
    wg = seeded.make_layer(MoEShape(H, E, 8, k), seed=5, device=gpu).router_w
    x = seeded.make_tokens(shape, 5, T, device=gpu)
    ids, w, logits = tm.router_topk(shape, x=x, router_w=wg)
    lg_ref = moe.router_logits(f32(x), f32(wg))
    np.testing.assert_allclose(logits.cpu().numpy(), lg_ref, rtol=1e-5, atol=1e-5)
    _check_routing(ids.cpu().numpy(), f32(w), lg_ref, k, "router")
    # supplied logits: selection on identical fp32 inputs is bit-exact
    ids2, w2, _ = tm.router_topk(shape, logits=torch.from_numpy(lg_ref).to(gpu))
    ids_ref, w_ref, _ = moe.router_topk(lg_ref, k)
    assert np.array_equal(ids2.cpu().numpy(), ids_ref)
    assert np.all(np.abs(f32(w2) - w_ref) <= np.abs(w_ref) * 2.0 ** -7)


def _decode_case(shape, seed, gpu, layer=None):
    layer = layer or seeded.make_layer(shape, seed, device=gpu)
    ws = Workspace(shape, gpu)
    table = tm.expert_table(layer.gate_up, layer.down)
    x = seeded.make_tokens(shape, seed, 1, device=gpu)
    out, ids, w = tm.moe_block(shape, x, table, ws, router_w=layer.router_w, shared=layer.shared)
    torch.cuda.synchronize()
    xs = f32(x)
    lg = moe.router_logits(xs, f32(layer.router_w))
    ids_ref, w_ref = _check_routing(ids.cpu().numpy(), f32(w), lg, shape.top_k, "decode router")
    gu, dn = expert_dicts(layer.gate_up, layer.down, ids_ref)
    ref = moe.experts_decode(xs[0], ids_ref[0], w_ref[0], gu, dn, shape.num_experts)
    if layer.shared is not None:
        ref = moe.add_bf16(ref, moe.shared_expert(xs[0], *[f32(t) for t in layer.shared]))
    assert_close_bf16(f32(out)[0], ref, f"decode block seed {seed}")
    # experts.forward boundary with the oracle's routing
    out2 = tm.experts_forward(shape, x, torch.from_numpy(ids_ref).to(gpu),
                              torch.from_numpy(w_ref).to(gpu, torch.bfloat16), table, ws)
    ref2 = moe.experts_decode(xs[0], ids_ref[0], w_ref[0], gu, dn, shape.num_experts)
    assert_close_bf16(f32(out2)[0], ref2, f"decode experts seed {seed}")
    ws.status()
    return layer


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_decode_small_layer(gpu, seed):
    _decode_case(SMALL, seed, gpu)


def test_decode_full_size_layer(gpu):
    layer = _decode_case(FULL, 100, gpu)
    _decode_case(FULL, 101, gpu, layer=None)
    del layer


def test_decode_sentinel_and_invalid_ids(gpu):
    shape = MoEShape(512, 16, 256, 4)
    layer = seeded.make_layer(shape, 9, device=gpu)
    ws = Workspace(shape, gpu)
    table = tm.expert_table(layer.gate_up, layer.down)
    x = seeded.make_tokens(shape, 9, 1, device=gpu)
    ids = torch.tensor([[3, 16, 7, 1]], device=gpu)             # 16 = the skip sentinel E
    w = torch.tensor([[0.4, 0.3, 0.2, 0.1]], device=gpu).to(torch.bfloat16)
    out = tm.experts_forward(shape, x, ids, w, table, ws)
    gu, dn = expert_dicts(layer.gate_up, layer.down, ids.cpu().numpy())
    ref = moe.experts_decode(f32(x)[0], ids.cpu().numpy()[0], f32(w)[0], gu, dn, 16)
    assert_close_bf16(f32(out)[0], ref, "sentinel")
    ws.status()                                                  # the sentinel is not an error
    bad = torch.tensor([[3, 99, 7, 1]], device=gpu)
    tm.experts_forward(shape, x, bad, w, table, ws)
    with pytest.raises(RuntimeError, match="expert id"):
        ws.status()


# Fused-decode workspace layout (tarfa_amd/csrc/tmoe_ws.h): a status block (64 uint32), then
# 256-byte lines; line 0 word 0 holds the epoch, lines 2..129 are the 128 task queues, each
# with a copy of the epoch in word 16 (read by that queue's waves).
QUEUES = 128
EPOCH_BYTE = 256
EPOCH_COPIES = [256 + (2 + q) * 256 + 16 * 4 for q in range(QUEUES)]


def _epoch(ws):
    vals = [int(ws.buf[o:o + 4].cpu().view(torch.int32).numpy().view(np.uint32)[0])
            for o in [EPOCH_BYTE] + EPOCH_COPIES]
    assert len(set(vals)) == 1, f"epoch copies disagree: {sorted(set(vals))}"
    return vals[0]


def _set_epoch(ws, value):
    b = torch.tensor(list(value.to_bytes(4, "little")), dtype=torch.uint8, device=ws.buf.device)
    for o in [EPOCH_BYTE] + EPOCH_COPIES:
        ws.buf[o:o + 4] = b


def test_decode_workspace_reuse_and_epoch_wrap(gpu):
    """Back-to-back decode calls on one workspace, across the 2^32 epoch wrap.

    Hand-off words carry the call's epoch, so each call must ignore every word an
    earlier call left behind; each output is checked against the oracle.
    """
    shape = MoEShape(1024, 32, 512, 8, 512)
    layer = seeded.make_layer(shape, 21, device=gpu)
    ws = Workspace(shape, gpu)
    table = tm.expert_table(layer.gate_up, layer.down)
    xs = seeded.make_tokens(shape, 21, 9, device=gpu)
    shared = [f32(t) for t in layer.shared]

    def one(r):
        x = xs[r:r + 1]
        out, ids, w = tm.moe_block(shape, x, table, ws, router_w=layer.router_w, shared=layer.shared)
        torch.cuda.synchronize()
        xf = f32(x)
        lg = moe.router_logits(xf, f32(layer.router_w))
        ids_ref, w_ref = _check_routing(ids.cpu().numpy(), f32(w), lg, shape.top_k, f"reuse call {r}")
        gu, dn = expert_dicts(layer.gate_up, layer.down, ids_ref)
        ref = moe.add_bf16(moe.experts_decode(xf[0], ids_ref[0], w_ref[0], gu, dn, shape.num_experts),
                           moe.shared_expert(xf[0], *shared))
        assert_close_bf16(f32(out)[0], ref, f"reuse call {r}")

    assert _epoch(ws) == 0
    for r in range(4):
        one(r)
        assert _epoch(ws) == r + 1
    _set_epoch(ws, 0xFFFFFFFD)
    one(4)
    assert _epoch(ws) == 0xFFFFFFFE
    one(5)
    assert _epoch(ws) == 0                    # tag 0xFFFFFFFF: the hand-off area is zeroed, epoch restarts
    one(6)
    assert _epoch(ws) == 1
    one(7)
    ws.status()


@pytest.mark.parametrize("T,E,k", [(4096, 256, 8), (5, 32, 8), (1000, 16, 1), (300, 4, 2), (20000, 64, 8)])
def test_dispatch_bit_exact(gpu, T, E, k):
    g = np.random.default_rng(T + E)
    ids = np.stack([g.permutation(E)[:k] for _ in range(T)]).astype(np.int64)
    if T > 10:
        ids[3, 0] = E                                            # sentinel rows are skipped
    ws = Workspace(MoEShape(128, E, 64, k), gpu, tokens=T)
    offsets, perm, inv = tm.dispatch(torch.from_numpy(ids).to(gpu), E, ws)
    o_ref, p_ref = moe.dispatch(ids, E)
    assert np.array_equal(offsets.cpu().numpy(), o_ref)
    n = int(o_ref[-1])
    assert np.array_equal(perm.cpu().numpy()[:n], p_ref)
    inv_ref = np.full(T * k, -1, np.int64)
    inv_ref[p_ref] = np.arange(n)
    assert np.array_equal(inv.cpu().numpy(), inv_ref)


def test_dispatch_rejects_too_many_entries(gpu):
    """T*k above 524288 (the scatter's LDS mask) is refused before any launch."""
    T, k, E = 65537, 8, 16
    ids = torch.zeros(T, k, dtype=torch.int64, device=gpu)
    ws = Workspace(MoEShape(128, E, 64, k), gpu, tokens=T)
    with pytest.raises(RuntimeError, match="unsupported or inconsistent sizes"):
        tm.dispatch(ids, E, ws)


@pytest.mark.parametrize("T,shared", [(2, False), (37, True), (300, True)])
def test_prefill_small_block(gpu, T, shared):
    shape = MoEShape(256, 16, 128, 4, 128 if shared else 0)
    layer = seeded.make_layer(shape, 40 + T, device=gpu)
    ws = Workspace(shape, gpu, tokens=T)
    table = tm.expert_table(layer.gate_up, layer.down)
    x = seeded.make_tokens(shape, 40 + T, T, device=gpu)
    logits = seeded.make_logits(shape, 40 + T, T, device=gpu)
    out, ids, w = tm.moe_block(shape, x, table, ws, logits=logits, shared=layer.shared)
    lg = logits.cpu().numpy()
    ids_ref, w_ref, _ = moe.router_topk(lg, shape.top_k)
    assert np.array_equal(ids.cpu().numpy(), ids_ref)
    xs = f32(x)
    gu, dn = expert_dicts(layer.gate_up, layer.down, ids_ref)
    ref = moe.experts_prefill(xs, ids_ref, f32(w), gu, dn, shape.num_experts)
    if shared:
        ref = moe.add_bf16(ref, moe.shared_expert(xs, *[f32(t) for t in layer.shared]))
    assert_close_bf16(f32(out), ref, f"prefill T={T}")
    out2 = tm.experts_forward(shape, x, ids, w, table, ws)
    ref2 = moe.experts_prefill(xs, ids_ref, f32(w), gu, dn, shape.num_experts)
    assert_close_bf16(f32(out2), ref2, f"prefill experts T={T}")


def test_prefill_many_experts_with_shared_gate(gpu):
    """E = 300 (the top-k's 16-logits-per-lane variant) with a shared expert at T = 40: the
    top-k and the shared gate run in one launch; ids exact, outputs at the bf16 bars."""
    shape = MoEShape(256, 300, 128, 6, 128)
    T = 40
    layer = seeded.make_layer(shape, 83, device=gpu)
    ws = Workspace(shape, gpu, tokens=T)
    table = tm.expert_table(layer.gate_up, layer.down)
    x = seeded.make_tokens(shape, 83, T, device=gpu)
    logits = seeded.make_logits(shape, 83, T, device=gpu)
    out, ids, w = tm.moe_block(shape, x, table, ws, logits=logits, shared=layer.shared)
    ids_ref, w_ref, _ = moe.router_topk(logits.cpu().numpy(), shape.top_k)
    assert np.array_equal(ids.cpu().numpy(), ids_ref)
    xs = f32(x)
    gu, dn = expert_dicts(layer.gate_up, layer.down, ids_ref)
    ref = moe.add_bf16(moe.experts_prefill(xs, ids_ref, f32(w), gu, dn, shape.num_experts),
                       moe.shared_expert(xs, *[f32(t) for t in layer.shared]))
    assert_close_bf16(f32(out), ref, "prefill E=300 with shared gate")


def test_prefill_group_larger_than_one_tile(gpu):
    """Skewed routing: one expert receives every token (> 256 rows -> several M-chunks)."""
    shape = MoEShape(256, 8, 128, 2)
    T = 600
    layer = seeded.make_layer(shape, 77, device=gpu)
    ws = Workspace(shape, gpu, tokens=T)
    table = tm.expert_table(layer.gate_up, layer.down)
    x = seeded.make_tokens(shape, 77, T, device=gpu)
    ids = torch.stack([torch.zeros(T, dtype=torch.int64), torch.arange(T) % 7 + 1], dim=1).to(gpu)
    w = torch.full((T, 2), 0.5, device=gpu).to(torch.bfloat16)
    out = tm.experts_forward(shape, x, ids, w, table, ws)
    gu, dn = expert_dicts(layer.gate_up, layer.down, ids.cpu().numpy())
    ref = moe.experts_prefill(f32(x), ids.cpu().numpy(), f32(w), gu, dn, 8)
    assert_close_bf16(f32(out), ref, "skewed prefill")


@pytest.mark.parametrize("T,shared", [(1024, True), (700, False)])
def test_prefill_persistent_gemm_many_tiles(gpu, T, shared):
    """H and I multiples of 512 take the persistent grouped GEMM (one block per CU walking a
    tile list with its loads running on across tiles).  1024 tokens x 8 slots over 32 experts
    is ~256 rows per expert (two M-chunks each: a full one and a partial one), 8 N-tiles per
    chunk for gate/up and 4 for down: several tiles per block in both GEMMs, so the
    next-tile prefetch, the epilogue between tiles and the last tile's tail all run."""
    shape = MoEShape(1024, 32, 1024, 8, 1024 if shared else 0)
    layer = seeded.make_layer(shape, 60 + T, device=gpu)
    ws = Workspace(shape, gpu, tokens=T)
    table = tm.expert_table(layer.gate_up, layer.down)
    x = seeded.make_tokens(shape, 60 + T, T, device=gpu)
    logits = seeded.make_logits(shape, 60 + T, T, device=gpu)
    out, ids, w = tm.moe_block(shape, x, table, ws, logits=logits, shared=layer.shared)
    ids_ref, w_ref, _ = moe.router_topk(logits.cpu().numpy(), shape.top_k)
    assert np.array_equal(ids.cpu().numpy(), ids_ref)
    counts = np.bincount(ids_ref.ravel(), minlength=shape.num_experts)
    assert counts.max() > 160 and (counts % 160 != 0).any()       # multi-chunk groups, partial chunks
    xs = f32(x)
    gu, dn = expert_dicts(layer.gate_up, layer.down, ids_ref)
    ref = moe.experts_prefill(xs, ids_ref, f32(w), gu, dn, shape.num_experts)
    if shared:
        ref = moe.add_bf16(ref, moe.shared_expert(xs, *[f32(t) for t in layer.shared]))
    assert_close_bf16(f32(out), ref, f"persistent prefill T={T}")
    # the same call again on the same workspace: identical bits
    out2 = tm.moe_block(shape, x, table, ws, logits=logits, shared=layer.shared)[0]
    assert torch.equal(out2, out)


@pytest.mark.parametrize("E,k", [(32, 8), (256, 8), (8, 8), (16, 4), (512, 8)])
def test_decode_router_exact_ties(gpu, E, k):
    """The fused decode's in-kernel top-k on supplied logits with many exact ties (and +-0):
    ids bit-exact against the oracle's order (logit descending, ties to the lower index)."""
    shape = MoEShape(1024, E, 512, k, 0)
    layer = seeded.make_layer(shape, 12, device=gpu)
    table = tm.expert_table(layer.gate_up, layer.down)
    ws = Workspace(shape, gpu)
    x = seeded.make_tokens(shape, 12, 1, device=gpu)
    rng = np.random.default_rng(E + k)
    vals = np.array([0.0, -0.0, 1.5, -2.25, 3.0, 1.5, 0.75], np.float32)
    for trial in range(8):
        lg = rng.choice(vals, size=E).astype(np.float32)
        if trial == 0:
            lg[:] = 0.0
            lg[::2] = -0.0                          # every logit tied (+0 and -0 compare equal)
        if trial == 1:
            lg = np.arange(E, dtype=np.float32) % 3  # tied blocks across every lane position
        out, ids, w = tm.moe_block(shape, x, table, ws, logits=torch.from_numpy(lg[None].copy()).to(gpu))
        ids_ref, w_ref, _ = moe.router_topk(lg[None], k)
        assert np.array_equal(ids.cpu().numpy(), ids_ref), f"E={E} k={k} trial {trial}"
        assert np.all(np.abs(f32(w) - w_ref) <= np.abs(w_ref) * 2.0 ** -7)
    # fewer finite logits than slots: the rest take the sentinel E with weight 0
    lg = np.full(E, -np.inf, np.float32)
    lg[[5, 2, 7]] = [1.0, 1.0, 0.5]
    out, ids, w = tm.moe_block(shape, x, table, ws, logits=torch.from_numpy(lg[None].copy()).to(gpu))
    want = [2, 5, 7] + [E] * (k - 3)
    assert ids.cpu().numpy()[0].tolist() == want
    assert np.all(f32(w)[0, 3:] == 0) and abs(float(f32(w)[0, :3].sum()) - 1.0) < 1e-2
    ws.status()
