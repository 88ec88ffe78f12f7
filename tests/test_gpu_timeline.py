"""The fused decode's debug timeline (tmoe_debug_decode_trace): every task of one call is
recorded once, with ordered stamps, and the summary's groups match the task list."""
import numpy as np
import pytest
import torch

from tarfa_amd import moe as tm
from tarfa_amd import seeded
from tarfa_amd.moe import MoEShape, Workspace
from tarfa_amd.timeline import HEADER, TASK_WORDS, DecodeTrace, format_summary, summarize

pytestmark = pytest.mark.gpu

FULL = MoEShape(2560, 256, 1024, 8, 1024)


def test_decode_timeline_records_every_task(gpu):
    layer = seeded.make_layer(FULL, 61, device=gpu)
    table = tm.expert_table(layer.gate_up, layer.down)
    ws = Workspace(FULL, gpu)
    x = seeded.make_tokens(FULL, 61, 1, device=gpu)
    ref, _, _ = tm.moe_block(FULL, x, table, ws, router_w=layer.router_w, shared=layer.shared)
    with DecodeTrace(gpu) as tr:
        out, _, _ = tm.moe_block(FULL, x, table, ws, router_w=layer.router_w, shared=layer.shared)
        rec = tr.records()
    ws.status()
    assert torch.equal(out, ref)                     # recording changes no result
    n, grid = int(rec[0]), int(rec[1])
    t = rec[HEADER:HEADER + n * TASK_WORDS].reshape(n, TASK_WORDS).astype(np.int64)
    assert np.all(t[:, 0] > 0), "a task was not recorded"
    assert np.all(t[:, 3] >= t[:, 0])
    took = t[:, 2] > 0
    assert np.all(t[took, 2] >= t[took, 0]) and np.all(t[took, 3] >= t[took, 2])
    assert np.all((t[:, 5] & 0xF) < 8)               # XCC ids
    s = summarize(rec, FULL.hidden, FULL.intermediate, FULL.shared_intermediate, FULL.num_experts)
    counts = {g["group"]: g["tasks"] for g in s["groups"]}
    n_r = (FULL.num_experts + 1 + 3) // 4
    assert counts["R"] == n_r and counts["S"] == 512 and counts["SD"] == FULL.hidden // 8
    for j in range(FULL.top_k):
        assert counts[f"G{j}"] == FULL.intermediate // 2 and counts[f"D{j}"] == FULL.hidden // 8
    assert sum(counts.values()) == n and s["waves"] == grid * 4
    assert "call" in format_summary(s)
