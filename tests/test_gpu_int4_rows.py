"""GPU parity for the reference's own int4 layout: packed nibbles with ONE fp16 scale per
row (tarfa/engine/channel_q4.py:10-14, 18, 28-38), read from its per-layer files.

Bars: the device dequantisation is bit-exact with the reference's ``dequant_int4`` (oracle
``int4.dequant_f16``, itself pinned exhaustively against torch's fp16 multiply); batch-1
outputs are within max-abs 2e-2 / rel-L2 1e-3 of the oracle's ``moe_ffn`` restatement on
this layout (``int4.ffn_rows``; closest of the candidates where an activation sits on a
bf16 midpoint); T > 1 outputs against the exact-BF16 prefill oracle on the weights
bf16((nibble - 8) * fp32(s)) (``int4.dequant_rows_bf16``).  Weights are seeded bf16
experts quantised per row with s = fp16(max|w| / 7), q = rint(w / s) (the reference ships
no quantiser).
"""
import numpy as np
import pytest
import torch

from oracle import bf16, int4, moe
from tarfa_amd import moe as tm
from tarfa_amd import seeded
from tarfa_amd.experts import ExpertStore
from tarfa_amd.int4_files import Int4LayerFile, write_layer_file
from tarfa_amd.moe import MoEShape, Workspace
from tests._util import assert_close_any_bf16, assert_close_bf16, f32

pytestmark = pytest.mark.gpu

SMALL = MoEShape(1024, 32, 512, 8, 0)
FULL = MoEShape(2560, 256, 1024, 8, 1024)


def u16(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def quantize_rows(w):
    """bf16 [..., N, K] -> (packed [..., N, K/2] u8, fp16 scales [..., N]): s = fp16(max|w|/7)."""
    wf = w.float()
    s = (wf.abs().amax(-1) / 7.0).to(torch.float16)
    sf = s.float().unsqueeze(-1)
    q = torch.where(sf == 0, torch.zeros_like(wf), torch.round(wf / sf)).clamp(-8, 7).to(torch.int32) + 8
    packed = (q[..., 0::2] | (q[..., 1::2] << 4)).to(torch.uint8)
    return packed.contiguous(), s.contiguous()


def rows_layer(layer):
    gq, gs = quantize_rows(layer.gate_up)
    dq, ds = quantize_rows(layer.down)
    return gq, gs, dq, ds


def test_dequant_f16_every_code_and_fp16_scale(gpu):
    """16 codes x every finite fp16 scale on the device vs the oracle (the reference's dequant_int4)."""
    sb = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    sb = sb[np.isfinite(sb.view(np.float16))]
    packed = np.tile(np.array([0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE], np.uint8), (sb.size, 1))
    p = torch.from_numpy(packed).to(gpu)
    s = torch.from_numpy(sb.view(np.int16)).view(torch.float16).to(gpu)
    got = u16(tm.dequant_int4_f16(p, s))
    assert np.array_equal(got, int4.dequant_f16(packed, sb[:, None], 16))


def _host(q, ids):
    gq, gs, dq, ds = q
    return {int(e): (gq[e].cpu().numpy(), u16(gs[e]), dq[e].cpu().numpy(), u16(ds[e])) for e in set(ids.tolist())
            if 0 <= int(e) < gq.shape[0]}


def _decode_case(shape, seed, gpu, from_file=None):
    layer = seeded.make_layer(shape, seed, device=gpu)
    q = rows_layer(layer)
    if from_file is not None:
        write_layer_file(from_file, *q)
        f = Int4LayerFile(from_file)
        q2 = f.load(gpu)
        for a, b in zip(q2, q):
            assert torch.equal(a, b)
        store = ExpertStore.from_int4_file(shape, from_file, gpu)
        table = store.table
    else:
        table = tm.expert_table_q4_rows(*q)
    ws = Workspace(shape, gpu)
    x = seeded.make_tokens(shape, seed, 1, device=gpu)
    out, ids, w = tm.moe_block(shape, x, table, ws, router_w=layer.router_w, shared=layer.shared)
    torch.cuda.synchronize()
    ws.status()
    xs = f32(x)[0]
    ids_ref, w_ref, _ = moe.router_topk(moe.router_logits(f32(x), f32(layer.router_w)), shape.top_k)
    assert np.array_equal(ids.cpu().numpy(), ids_ref)
    ex = _host(q, ids_ref[0])
    sel = [ex[int(e)] for e in ids_ref[0]]
    routed = int4.ffn_candidates(xs, sel, w_ref[0], gemv=int4.gemv_rows)
    assert np.array_equal(routed[0], int4.ffn_rows(xs, sel, w_ref[0]))
    ref = routed
    if layer.shared is not None:
        sh = moe.shared_expert(xs, *[f32(t) for t in layer.shared])
        ref = [moe.add_bf16(r, sh) for r in routed]
    assert_close_any_bf16(f32(out)[0], ref, f"int4 rows block seed {seed}")
    out2 = tm.experts_forward(shape, x, ids, w, table, ws)
    assert_close_any_bf16(f32(out2)[0], routed, f"int4 rows experts seed {seed}")
    ws.status()


@pytest.mark.parametrize("seed", [0, 1])
def test_rows_decode_small_layer(gpu, seed):
    _decode_case(SMALL, seed, gpu)


def test_rows_decode_full_size_layer_from_a_layer_file(gpu, tmp_path):
    _decode_case(FULL, 5, gpu, from_file=tmp_path / "layer_0.safetensors")


@pytest.mark.parametrize("T", [3, 64, 300])
def test_rows_prefill_matches_bf16_chain_on_dequantised_weights(gpu, T):
    shape = MoEShape(1024, 32, 512, 8, 512)
    layer = seeded.make_layer(shape, 40 + T, device=gpu)
    q = rows_layer(layer)
    table = tm.expert_table_q4_rows(*q)
    ws = Workspace(shape, gpu, tokens=T)
    x = seeded.make_tokens(shape, 40 + T, T, device=gpu)
    out, ids, w = tm.moe_block(shape, x, table, ws, router_w=layer.router_w, shared=layer.shared)
    torch.cuda.synchronize()
    ws.status()
    ids_d = ids.cpu().numpy()
    gu = {e: bf16.to_f32(int4.dequant_rows_bf16(q[0][e].cpu().numpy(), u16(q[1][e]))) for e in set(ids_d.ravel().tolist())}
    dn = {e: bf16.to_f32(int4.dequant_rows_bf16(q[2][e].cpu().numpy(), u16(q[3][e]))) for e in gu}
    ref = moe.experts_prefill(f32(x), ids_d, f32(w), gu, dn, shape.num_experts)
    ref = moe.add_bf16(ref, moe.shared_expert(f32(x), *[f32(t) for t in layer.shared]))
    assert_close_bf16(f32(out), ref, f"int4 rows prefill T={T}")
    # the experts.forward boundary at T > 1 (routed only), same weights
    out2 = tm.experts_forward(shape, x, ids, w, table, ws)
    ref2 = moe.experts_prefill(f32(x), ids_d, f32(w), gu, dn, shape.num_experts)
    assert_close_bf16(f32(out2), ref2, f"int4 rows experts T={T}")


def test_rows_prefill_full_size_sampled_tokens(gpu):
    """The per-row-scale prefill GEMM at the full-size layer (H=2560, E=256, I=1024, shared
    expert), T = 300: every token's ids against the oracle router, and 12 sampled tokens'
    outputs against the exact-BF16 chain on the dequantised weights of the experts they use."""
    shape, T = FULL, 300
    layer = seeded.make_layer(shape, 61, device=gpu)
    q = rows_layer(layer)
    table = tm.expert_table_q4_rows(*q)
    ws = Workspace(shape, gpu, tokens=T)
    x = seeded.make_tokens(shape, 61, T, device=gpu)
    logits = seeded.make_logits(shape, 61, T, device=gpu)
    out, ids, w = tm.moe_block(shape, x, table, ws, logits=logits, shared=layer.shared)
    torch.cuda.synchronize()
    ws.status()
    ids_d = ids.cpu().numpy()
    ids_ref, _, _ = moe.router_topk(logits.cpu().numpy(), shape.top_k)
    assert np.array_equal(ids_d, ids_ref)
    pick = np.linspace(0, T - 1, 12).astype(int)
    sel = ids_d[pick]
    gu = {e: bf16.to_f32(int4.dequant_rows_bf16(q[0][e].cpu().numpy(), u16(q[1][e]))) for e in set(sel.ravel().tolist())}
    dn = {e: bf16.to_f32(int4.dequant_rows_bf16(q[2][e].cpu().numpy(), u16(q[3][e]))) for e in gu}
    xs = f32(x)[pick]
    ref = moe.experts_prefill(xs, sel, f32(w)[pick], gu, dn, shape.num_experts)
    ref = moe.add_bf16(ref, moe.shared_expert(xs, *[f32(t) for t in layer.shared]))
    assert_close_bf16(f32(out)[pick], ref, f"int4 rows prefill full size T={T}")


def test_rows_prefill_register_staged_kernel(gpu):
    """A shape the persistent GEMM does not take (H = 640, I = 384): the register-staged
    kernel's per-row-scale path."""
    shape = MoEShape(640, 16, 384, 4, 0)
    T = 9
    layer = seeded.make_layer(shape, 77, device=gpu)
    q = rows_layer(layer)
    table = tm.expert_table_q4_rows(*q)
    ws = Workspace(shape, gpu, tokens=T)
    x = seeded.make_tokens(shape, 77, T, device=gpu)
    out, ids, w = tm.moe_block(shape, x, table, ws, router_w=layer.router_w)
    torch.cuda.synchronize()
    ws.status()
    ids_d = ids.cpu().numpy()
    gu = {e: bf16.to_f32(int4.dequant_rows_bf16(q[0][e].cpu().numpy(), u16(q[1][e]))) for e in set(ids_d.ravel().tolist())}
    dn = {e: bf16.to_f32(int4.dequant_rows_bf16(q[2][e].cpu().numpy(), u16(q[3][e]))) for e in gu}
    ref = moe.experts_prefill(f32(x), ids_d, f32(w), gu, dn, shape.num_experts)
    assert_close_bf16(f32(out), ref, "int4 rows prefill, register-staged GEMM")
