"""Shared helpers for the parity tests (tolerances, host copies of device tensors)."""
import numpy as np

# BF16 layer-output tolerance of the workload definition.  Accumulation order of
# both sides: bf16 rounding after each GEMV, SiLU, multiply, weight-scale and add;
# decode accumulates experts in router order, prefill in ascending expert id.
MAX_ABS = 2e-2
REL_L2 = 1e-3


def f32(t):
    """Device/host torch tensor -> numpy fp32 (bf16 widened exactly)."""
    return t.detach().float().cpu().numpy()


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def assert_close_bf16(got, ref, what=""):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    mx = float(np.max(np.abs(got - ref))) if got.size else 0.0
    rl = rel_l2(got, ref)
    same = float(np.mean(got == ref)) if got.size else 1.0
    assert mx <= MAX_ABS and rl <= REL_L2, f"{what}: max-abs {mx:.3e} rel-L2 {rl:.3e} bit-same {same:.4f}"
    return mx, rl, same


def expert_dicts(gate_up, down, ids):
    """Host fp32 copies of the experts named in ``ids`` (device slabs [E,2I,H] / [E,H,I])."""
    import torch
    uniq = sorted({int(e) for e in np.asarray(ids).reshape(-1).tolist() if 0 <= int(e) < gate_up.shape[0]})
    gu, dn = {}, {}
    if uniq:
        idx = torch.tensor(uniq, device=gate_up.device)
        g = gate_up.index_select(0, idx).float().cpu().numpy()
        d = down.index_select(0, idx).float().cpu().numpy()
        for j, e in enumerate(uniq):
            gu[e], dn[e] = g[j], d[j]
    return gu, dn


def assert_close_any_bf16(got, refs, what=""):
    """assert_close_bf16 against the closest of several admissible oracle outputs (the
    oracle enumerates activations that lie on a bf16 rounding midpoint within fp32 error)."""
    best = min(range(len(refs)), key=lambda i: rel_l2(got, refs[i]))
    return assert_close_bf16(got, refs[best], f"{what} (candidate {best} of {len(refs)})")
