"""tmoe_moe_block_bf16_noalloc (static scratch, no workspace) against tmoe_moe_block_bf16
(caller workspace), both called through the C ABI: identical ids, weights and output bits,
on consecutive calls of shrinking size (a prefill chunk, then a single token, ...)."""
import pytest
import torch

from tarfa_amd import moe as tm
from tarfa_amd import seeded
from tarfa_amd._lib import lib
from tarfa_amd.moe import MoEShape, Workspace

pytestmark = pytest.mark.gpu

FULL = MoEShape(2560, 256, 1024, 8, 1024)
TMOE_ERR_NULL, TMOE_ERR_SCRATCH = -1, -8


def _noalloc(shape, x, layer, status, logits=None):
    T, dev = x.shape[0], x.device
    out = torch.empty_like(x)
    ids = torch.empty(T, shape.top_k, dtype=torch.int64, device=dev)
    w = torch.empty(T, shape.top_k, dtype=torch.bfloat16, device=dev)
    sh = [t.data_ptr() for t in layer.shared]
    st = lib().tmoe_moe_block_bf16_noalloc(
        x.data_ptr(), T, layer.router_w.data_ptr(), None if logits is None else logits.data_ptr(),
        layer.table.data_ptr(), *sh, shape.hidden, shape.num_experts, shape.intermediate, shape.top_k,
        shape.shared_intermediate, out.data_ptr(), ids.data_ptr(), w.data_ptr(), None, status.data_ptr(),
        torch.cuda.current_stream(dev).cuda_stream)
    return st, out, ids, w


def test_noalloc_block_matches_the_workspace_entry_point(gpu):
    layer = seeded.make_layer(FULL, 90, device=gpu)
    layer.table = tm.expert_table(layer.gate_up, layer.down)
    status = torch.zeros(1, dtype=torch.int32, device=gpu)
    for i, T in enumerate((64, 1, 5, 1)):
        x = seeded.make_tokens(FULL, 90 + i, T, device=gpu)
        logits = seeded.make_logits(FULL, 90 + i, T, device=gpu) if T == 5 else None
        st, out, ids, w = _noalloc(FULL, x, layer, status, logits)
        assert st == 0, lib().tmoe_strerror(st)
        ws = Workspace(FULL, gpu, tokens=T)
        r_out, r_ids, r_w = tm.moe_block(FULL, x, layer.table, ws, router_w=None if logits is not None else
                                         layer.router_w, logits=logits, shared=layer.shared)
        torch.cuda.synchronize()
        ws.status()
        assert int(status.item()) == 0, f"call {i} (T={T}) flagged {int(status.item())}"
        assert torch.equal(ids, r_ids), f"call {i} (T={T}) ids"
        assert torch.equal(w, r_w), f"call {i} (T={T}) weights"
        assert torch.equal(out, r_out), f"call {i} (T={T}) output"


def test_noalloc_block_rejects_what_it_cannot_hold(gpu):
    layer = seeded.make_layer(MoEShape(2560, 256, 1024, 8, 1024), 91, device=gpu)
    layer.table = tm.expert_table(layer.gate_up, layer.down)
    status = torch.zeros(1, dtype=torch.int32, device=gpu)
    x = seeded.make_tokens(FULL, 91, 221, device=gpu)          # one token past the static scratch
    assert _noalloc(FULL, x, layer, status)[0] == TMOE_ERR_SCRATCH
    assert "static scratch" in lib().tmoe_strerror(TMOE_ERR_SCRATCH).decode()
    st = lib().tmoe_moe_block_bf16_noalloc(x.data_ptr(), 1, layer.router_w.data_ptr(), None,
                                           layer.table.data_ptr(), *[t.data_ptr() for t in layer.shared],
                                           2560, 256, 1024, 8, 1024, x.data_ptr(), None, None, None, None, None)
    assert st == TMOE_ERR_NULL                                  # the status word is required
    torch.cuda.synchronize()
