"""The committed golden fixtures (tests/golden/golden.json) against the CPU oracle.

The oracle must still produce every fixture bit for bit (regression pin), and the
reference's own op sequence in torch CPU bf16 (oracle/cpu_reference.py, the chain of
tarfa/engine/fused_int4.py:192-194 and :228-244) must land within the layer
tolerance of the fixture outputs (an independent pin of the oracle's rounding points).
"""
import json
import os
import sys

import numpy as np
import pytest
import torch

from oracle import bf16
from oracle import cpu_reference as cref
from tests._util import assert_close_bf16

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden as mg  # noqa: E402

GOLDEN = json.load(open(os.path.join(HERE, "golden", "golden.json")))


def _bits(hexstr):
    return np.frombuffer(bytes.fromhex(hexstr), np.uint16)


@pytest.mark.parametrize("name", ["decode_small_layer", "decode_tiny_shared", "prefill_tiny_shared"])
def test_oracle_reproduces_block_fixtures(name):
    for case in GOLDEN[name]:
        got = mg.block_case(case["seed"], case["H"], case["E"], case["I"], case["k"], case["Is"], case["T"])
        assert got == case


def test_oracle_reproduces_int4_and_dispatch_fixtures():
    for case in GOLDEN["int4_tiny"]:
        assert mg.int4_case(case["seed"], case["H"], case["I"], case["E"], case["k"]) == case
    for case in GOLDEN["dispatch"]:
        assert mg.dispatch_case(case["seed"], case["T"], case["k"], case["E"]) == case


@pytest.mark.parametrize("name", ["decode_small_layer", "decode_tiny_shared", "prefill_tiny_shared"])
def test_reference_op_chain_matches_fixtures(name):
    """torch CPU bf16 op sequence of the reference vs the fixture (oracle) outputs."""
    for case in GOLDEN[name]:
        H, E, I, k, Is, T = (case[n] for n in ("H", "E", "I", "k", "Is", "T"))
        gu, dn, wg, sh = mg.layer(case["seed"], H, E, I, Is)
        from oracle import rng
        x = rng.tensor_bf16(case["seed"], rng.KIND_X, (T, H), mg.X_STD)
        t = lambda a: torch.from_numpy(bf16.to_f32(a)).to(torch.bfloat16)  # noqa: E731
        shw = tuple(t(s) for s in sh) if sh is not None else None
        ids, _ = cref.router(t(x), t(wg), k)
        assert np.array_equal(ids.numpy(), np.array(case["ids"]))
        out = cref.moe_block(t(x), t(wg), k, t(gu), t(dn), E, shw)
        want = bf16.to_f32(_bits(case["out_bf16"])).reshape(T, H)
        assert_close_bf16(out.float().numpy(), want, f"{name} seed {case['seed']}")
