"""The HIP path against the committed golden fixtures (tests/golden/golden.json).

The device generator must reproduce the fixtures' weight digests bit for bit; the
router ids and the dispatch permutation must equal the fixtures; int4 packed codes,
scales and dequantised values are bit-exact; layer outputs are held to the layer
tolerance (max-abs 2e-2, rel-L2 1e-3).
"""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

from oracle import bf16
from tarfa_amd import moe as tm
from tarfa_amd import seeded
from tarfa_amd.moe import MoEShape, Workspace
from tests._util import assert_close_bf16, f32

pytestmark = pytest.mark.gpu

GOLDEN = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.json")))


def _sha(t):
    return hashlib.sha256(t.detach().cpu().contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def _bits(hexstr):
    return np.frombuffer(bytes.fromhex(hexstr), np.uint16)


@pytest.mark.parametrize("name", ["decode_small_layer", "decode_tiny_shared", "prefill_tiny_shared"])
def test_block_against_fixtures(gpu, name):
    for case in GOLDEN[name]:
        H, E, I, k, Is, T = (case[n] for n in ("H", "E", "I", "k", "Is", "T"))
        shape = MoEShape(H, E, I, k, Is)
        ly = seeded.make_layer(shape, case["seed"], device=gpu)
        x = seeded.make_tokens(shape, case["seed"], T, device=gpu)
        assert _sha(ly.gate_up) == case["sha256"]["gate_up"] and _sha(ly.down) == case["sha256"]["down"]
        assert _sha(ly.router_w) == case["sha256"]["router_w"] and _sha(x) == case["sha256"]["x"]
        if Is:
            assert hashlib.sha256(b"".join(t.cpu().contiguous().view(torch.uint8).numpy().tobytes()
                                           for t in ly.shared)).hexdigest() == case["sha256"]["shared"]
        ws = Workspace(shape, gpu, tokens=T)
        out, ids, w = tm.moe_block(shape, x, tm.expert_table(ly.gate_up, ly.down), ws, router_w=ly.router_w,
                                   shared=ly.shared)
        torch.cuda.synchronize()
        assert np.array_equal(ids.cpu().numpy(), np.array(case["ids"])), f"{name} ids"
        want = bf16.to_f32(_bits(case["out_bf16"])).reshape(T, H)
        assert_close_bf16(f32(out), want, f"{name} seed {case['seed']}")
        ws.status()


def test_int4_against_fixtures(gpu):
    for case in GOLDEN["int4_tiny"]:
        H, I, E, k = case["H"], case["I"], case["E"], case["k"]
        shape = MoEShape(H, E, I, k, 0)
        ly = seeded.make_layer(shape, case["seed"], device=gpu)
        gq, gs = tm.quantize_int4(ly.gate_up)
        dq, ds = tm.quantize_int4(ly.down)
        for e in range(E):
            packed = torch.cat([gq[e].reshape(-1), dq[e].reshape(-1)])
            scales = torch.cat([gs[e].reshape(-1), ds[e].reshape(-1)])
            assert _sha(packed) == case["packed_sha256"][e] and _sha(scales) == case["scales_sha256"][e]
        assert gq[0, 0].cpu().numpy().tobytes().hex() == case["expert0_gate_up_packed_row0"]
        deq = tm.dequant_int4(gq[0, :1].contiguous(), gs[0, :1].contiguous())
        assert deq.cpu().view(torch.int16).numpy().tobytes().hex() == case["expert0_gate_up_dequant_row0"]
        x = seeded.make_tokens(shape, case["seed"], 1, device=gpu)
        ids = torch.tensor([case["ids"]], device=gpu)
        w = torch.from_numpy(np.array(case["weights_bf16"], np.uint16).view(np.int16)).view(torch.bfloat16)
        ws = Workspace(shape, gpu)
        out = tm.experts_forward(shape, x, ids, w.reshape(1, k).to(gpu), tm.expert_table_q4(gq, gs, dq, ds), ws)
        assert_close_bf16(f32(out)[0], bf16.to_f32(_bits(case["ffn_bf16"])), "int4 fixture")
        ws.status()


def test_dispatch_against_fixtures(gpu):
    for case in GOLDEN["dispatch"]:
        T, k, E = case["T"], case["k"], case["E"]
        ws = Workspace(MoEShape(64, E, 8, k), gpu, tokens=T)
        offsets, perm, _ = tm.dispatch(torch.tensor(case["ids"], device=gpu), E, ws)
        assert offsets.cpu().tolist() == case["offsets"]
        n = case["offsets"][-1]
        assert perm.cpu().tolist()[:n] == case["perm"][:n]
