"""Int4 fast mode, CPU restatement (oracle, test infrastructure only).

Format (group-quantised variant of the reference's per-row format,
tarfa/engine/moe_kernel.py:10-14, tarfa/engine/channel_q4.py:10-14):

  packed [N, K/2] uint8   low nibble = even k, high nibble = odd k, value = nibble - 8
  scales [N, K/G] bf16    one scale per (row, group of G consecutive k)
  dequant  w_hat = bf16(fp32((nibble - 8) * s[n, k // G]))   (the product is exact in
           fp32: at most 3 x 8 significant bits; only the bf16 rounding is inexact)

The reference's own files carry ONE fp16 scale per row (channel_q4.py:10-14, 18, 28-38;
moe_kernel.py:10-14); ``dequant_f16``, ``gemv_rows`` and ``ffn_rows`` restate that layout.

The reference carries no quantiser (its int4 files come from outside the
repository, channel_q4.py:6).  The quantiser here is this build's definition:

  s = bf16(fp32(max_{k in group} |w| / 7))      fp32 IEEE division, then RNE to bf16
  q = clamp(rint(fp32(w / s)), -8, 7)           rint = round half to even; s == 0 -> q = 0
"""
import numpy as np

from . import bf16

rb = bf16.rnd


def quantize(w, group=128):
    """bf16 weights [N,K] (fp32 values) -> (packed [N,K/2] uint8, scale bf16 bits [N,K/G] uint16)."""
    w = np.asarray(w, np.float32)
    N, K = w.shape
    assert K % group == 0 and group % 2 == 0
    wg = w.reshape(N, K // group, group)
    amax = np.abs(wg).max(axis=-1)
    s = rb(amax / np.float32(7.0))                            # fp32 division, RNE to bf16
    with np.errstate(divide="ignore", invalid="ignore"):
        r = wg / s[..., None]                                  # fp32 / fp32, IEEE
    q = np.where(s[..., None] == 0, 0.0, np.rint(r))
    q = np.clip(q, -8, 7).astype(np.int32).reshape(N, K)
    nib = (q + 8).astype(np.uint8)
    packed = (nib[:, 0::2] | (nib[:, 1::2] << np.uint8(4))).astype(np.uint8)
    return packed, bf16.bits(s)


def codes(packed):
    """packed [N,K/2] -> signed codes [N,K] int32 (even k = low nibble)."""
    p = np.asarray(packed, np.uint8)
    lo = (p & 0xF).astype(np.int32) - 8
    hi = (p >> 4).astype(np.int32) - 8
    return np.stack([lo, hi], axis=-1).reshape(p.shape[0], -1)


def dequant(packed, scale_bits, group=128):
    """(packed, bf16 scale bits) -> dequantised bf16 bit patterns [N,K] (uint16).

    Restates channel_q4.py:10-14 / moe_kernel.py:110-114 (``q.to(dtype) * scale``)
    with a per-group instead of a per-row scale.
    """
    q = codes(packed).astype(np.float32)
    s = np.repeat(bf16.to_f32(scale_bits), group, axis=-1)
    with np.errstate(over="ignore"):                 # huge scales overflow to inf, as torch does
        return bf16.bits(q * s)


def gemv_f32(packed, scale_bits, x, group=128):
    """fp32 sum over groups of s[n,g] * sum_{k in g} q[n,k] x[k] (fp64 inside, fp32 out).

    The Triton kernel folds the per-row scale onto the fp32 dot
    (moe_kernel.py:60-63); with group scales the fold happens per group.
    """
    q = codes(packed).astype(np.float64)
    N, K = q.shape
    s = bf16.to_f32(scale_bits).astype(np.float64)
    part = (q.reshape(N, K // group, group) * np.asarray(x, np.float64).reshape(1, K // group, group)).sum(-1)
    return (part * s).sum(-1).astype(np.float32)


def ffn(x, experts, rw, group=128):
    """Labelled fast mode for one token: moe_kernel.py:90-104 with group scales.

    ``experts`` = list of (gate_up_packed, gate_up_scale, down_packed, down_scale)
    in router order; ``rw`` the bf16 routing weights.  Up projection in fp32,
    ``act = bf16(silu(g) * u)`` in fp32 (``:100``), down projection in fp32, then the
    fp32 weighted sum over experts (``:103``) and one cast to bf16 (``:104``).
    """
    x = np.asarray(x, np.float32)
    y = np.zeros(x.shape[0], np.float64)
    for (gq, gs, dq, ds), w in zip(experts, np.asarray(rw, np.float32).reshape(-1)):
        gu = gemv_f32(gq, gs, x, group).astype(np.float64)
        inter = gu.shape[0] // 2
        g, u = gu[:inter], gu[inter:]
        act = rb(((g / (1.0 + np.exp(-g))).astype(np.float32).astype(np.float64) * u).astype(np.float32))
        d = gemv_f32(dq, ds, act, group).astype(np.float64)
        y = (y + (d * np.float64(w)).astype(np.float32)).astype(np.float32).astype(np.float64)
    return rb(y.astype(np.float32))


def _act_f64(g, u):
    """silu(g) * u as ffn evaluates it, before the bf16 rounding (fp32 value, kept in fp64)."""
    return ((g / (1.0 + np.exp(-g))).astype(np.float32).astype(np.float64) * u).astype(np.float32).astype(np.float64)


def ambiguous_roundings(v, rel):
    """Where v lies within ``rel`` (relative) of a bf16 rounding midpoint: the indices, the
    bf16 value on the other side of the midpoint (uint16 bits) and the distance to it."""
    v = np.asarray(v, np.float32)
    t = v.view(np.uint32) & np.uint32(0xFFFF0000)                   # truncated toward zero
    lo = t.view(np.float32).astype(np.float64)
    hi = (t + np.uint32(0x10000)).view(np.float32).astype(np.float64)
    mid = (lo + hi) / 2
    dist = np.abs(v.astype(np.float64) - mid)
    near = (dist <= rel * np.abs(mid)) & np.isfinite(v)
    tb = (t >> np.uint32(16)).astype(np.uint16)
    other = np.where(bf16.bits(v) == tb, tb + np.uint16(1), tb).astype(np.uint16)
    idx = np.nonzero(near)[0]
    return idx, other[idx], dist[idx]


def ffn_candidates(x, experts, rw, group=128, rel=2e-6, max_flips=6, gemv=None):
    """Every output ``ffn`` can give when each activation lying within ``rel`` of a bf16
    midpoint may round either way.

    The activation ``bf16(silu(g) * u)`` is the first rounding of the int4 path; g and u
    are fp32 sums whose last bits depend on the summation order, which the reference
    leaves to its Triton kernel (moe_kernel.py:54-60).  An activation within a few fp32
    ulps of a bf16 midpoint can therefore legitimately round either way, and one such
    flip of a large activation moves every output row by ~1e-3 relative.  Returns a list
    of bf16 outputs (the first is ``ffn`` itself); at most ``max_flips`` of the closest
    cases are enumerated.  ``gemv`` (default: the group form ``gemv_f32``) takes (packed,
    scales, vector); ``gemv_rows`` gives the candidates of ``ffn_rows``.
    """
    if gemv is None:
        gemv = lambda pk, sc, v: gemv_f32(pk, sc, v, group)  # noqa: E731
    x = np.asarray(x, np.float32)
    rw = np.asarray(rw, np.float32).reshape(-1)
    acts, flips = [], []
    for j, (gq, gs, dq, ds) in enumerate(experts):
        gu = gemv(gq, gs, x).astype(np.float64)
        inter = gu.shape[0] // 2
        a = _act_f64(gu[:inter], gu[inter:]).astype(np.float32)
        acts.append(rb(a))
        idx, other, dist = ambiguous_roundings(a, rel)
        flips += [(float(d), j, int(i), float(bf16.to_f32(o))) for i, o, d in zip(idx, other, dist)]
    flips = sorted(flips)[:max_flips]
    outs = []
    for mask in range(1 << len(flips)):
        y = np.zeros(x.shape[0], np.float64)
        for j, (gq, gs, dq, ds) in enumerate(experts):
            act = acts[j].copy()
            for b, (_, jj, i, alt) in enumerate(flips):
                if jj == j and (mask >> b) & 1:
                    act[i] = alt
            d = gemv(dq, ds, act).astype(np.float64)
            y = (y + (d * np.float64(rw[j])).astype(np.float32)).astype(np.float32).astype(np.float64)
        outs.append(rb(y.astype(np.float32)))
    return outs


# ------------------------------------------------------------------ the reference's per-row fp16 layout

def f16_to_f32(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def dequant_f16(packed, scale_bits, group):
    """(packed, fp16 scale bits [N, K/G]) -> fp16 bit patterns [N, K]: channel_q4.py:10-14
    ``q.to(torch.float16) * scale[:, None]`` (G = K: the reference's per-row scale), one
    correctly rounded fp16 multiply of an exact code and an fp16 scale."""
    q = codes(packed).astype(np.float16)
    s = np.repeat(np.asarray(scale_bits, np.uint16).view(np.float16), group, axis=-1)
    with np.errstate(over="ignore", invalid="ignore"):
        return (q * s).view(np.uint16)


def gemv_rows(packed, scale_bits, x):
    """The reference kernel's row: fp32 acc = sum_k (nibble - 8) x[k] (fp64 inside, rounded
    to fp32), then y = fp32(acc * fp32(s[n])) (moe_kernel.py:54-63, per-row fp16 scale)."""
    q = codes(packed).astype(np.float64)
    acc = (q @ np.asarray(x, np.float64)).astype(np.float32)
    return (acc * f16_to_f32(np.asarray(scale_bits).reshape(-1))).astype(np.float32)


def ffn_rows(x, experts, rw):
    """moe_ffn (moe_kernel.py:90-104) on the reference's per-row fp16 layout for one token:
    ``experts`` = (gate_up_packed [2I, H/2], gate_up_scale [2I] fp16 bits, down_packed
    [H, I/2], down_scale [H] fp16 bits) in router order, ``rw`` the bf16 routing weights.
    act = bf16(silu(g) * u) in fp32 (:100; the engine dtype here is bf16), fp32 weighted
    sum over experts in router order (:103), one cast to bf16 (:104)."""
    x = np.asarray(x, np.float32)
    y = np.zeros(x.shape[0], np.float32)
    for (gq, gs, dq, ds), w in zip(experts, np.asarray(rw, np.float32).reshape(-1)):
        gu = gemv_rows(gq, gs, x).astype(np.float64)
        inter = gu.shape[0] // 2
        act = rb(_act_f64(gu[:inter], gu[inter:]).astype(np.float32))
        d = gemv_rows(dq, ds, act)
        y = (y + (d * np.float32(w)).astype(np.float32)).astype(np.float32)
    return rb(y)


def dequant_rows_bf16(packed, scale_bits):
    """The bf16 weights the exact-BF16 prefill uses for the per-row layout: the exact
    product (nibble - 8) * fp32(s[n]) rounded once to bf16 (bit patterns)."""
    q = codes(packed).astype(np.float32)
    s = f16_to_f32(np.asarray(scale_bits).reshape(-1))[:, None]
    with np.errstate(over="ignore"):
        return bf16.bits(q * s)
