"""The oracle's RMSNorm against transformers' own Qwen3_5MoeRMSNorm (installed library,
transformers/models/qwen3_5_moe/modeling_qwen3_5_moe.py:800-814), on CPU."""
import numpy as np
import pytest
import torch

from oracle import bf16, moe


def _transformers_rmsnorm(h, w, eps):
    from transformers.models.qwen3_5_moe.modeling_qwen3_5_moe import Qwen3_5MoeRMSNorm
    m = Qwen3_5MoeRMSNorm(h.shape[-1], eps=eps)
    with torch.no_grad():
        m.weight.copy_(torch.from_numpy(w))
    with torch.no_grad():
        return m(torch.from_numpy(h).to(torch.bfloat16)).float().numpy()


@pytest.mark.parametrize("H,seed", [(1024, 0), (2560, 1), (2560, 2)])
def test_oracle_rmsnorm_matches_transformers(H, seed):
    g = np.random.default_rng(seed)
    h = bf16.rnd((g.standard_normal((64, H)) * 3.0).astype(np.float32))
    w = bf16.rnd((g.standard_normal(H) * 0.1).astype(np.float32))   # zero-centred: the scale is 1 + w
    eps = 1e-6
    ref = _transformers_rmsnorm(h, w, eps)
    got = moe.rmsnorm(h, w, eps)
    # The two differ only in the fp32 summation order of the mean: one bf16 step at most,
    # in a small fraction of the elements.
    ulp = np.abs(bf16.bits(got).astype(np.int32) - bf16.bits(ref).astype(np.int32))
    assert ulp.max() <= 1
    assert (ulp > 0).mean() < 0.01


def test_oracle_rmsnorm_closed_forms():
    """A constant row c: mean(h^2) = c^2, so x = bf16(c / sqrt(c^2 + eps) * (1 + w)); with
    w = 0 and eps = 0 that is 1 (sign of c) exactly; a zero row stays zero."""
    H = 512
    for c in (0.5, -3.0, 1024.0):
        x = moe.rmsnorm(np.full((1, H), c, np.float32), np.zeros(H, np.float32), 0.0)
        assert np.all(x == np.sign(c))
    assert np.all(moe.rmsnorm(np.zeros((2, H), np.float32), np.ones(H, np.float32), 1e-6) == 0)
    w = bf16.rnd(np.linspace(-0.5, 0.5, H).astype(np.float32))
    x = moe.rmsnorm(np.full((1, H), 2.0, np.float32), w, 0.0)
    assert np.array_equal(x[0], bf16.rnd((np.float32(1.0) + w).astype(np.float32)))
