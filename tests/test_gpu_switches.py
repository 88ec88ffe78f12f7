"""The environment switches that pick an alternative kernel give the same results.

`TMOE_PREFILL_GEMM=frag` runs the bf16 prefill groups on the kernel that loads weights straight
into MFMA fragments (the default reads whole 128-byte lines and reorders them through LDS);
`TMOE_SMALLBATCH=0` sends 2 <= T <= 16 token batches to the grouped GEMM instead of the
small-batch kernels.  Both are read once per process, so the cases run in a child process with
the switches set, against the oracle at the usual bars (top-k ids bit-exact, outputs within
max-abs 2e-2 and rel-L2 1e-3).
"""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = """
import sys, torch
from tests import test_gpu_core as core
from tests.test_gpu_smallbatch import MID, _block_case
dev = torch.device("cuda:0")
for T, shared in ((1024, True), (700, False)):
    print("persistent prefill T=%d shared=%s" % (T, shared), flush=True)
    core.test_prefill_persistent_gemm_many_tiles(dev, T, shared)
for T in (2, 8, 16):
    print("small batch via grouped GEMM T=%d" % T, flush=True)
    _block_case(MID, T, 500 + T, dev)
print("switch cases passed", flush=True)
"""


def test_fragment_gemm_and_grouped_small_batch(gpu):
    env = dict(os.environ, TMOE_PREFILL_GEMM="frag", TMOE_SMALLBATCH="0")
    r = subprocess.run([sys.executable, "-c", CHILD], cwd=ROOT, env=env, capture_output=True,
                       text=True, timeout=110)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "switch cases passed" in r.stdout
