"""CPU restatement of the reference's per-layer MoE step (oracle, test infrastructure only).

All tensors are fp32 numpy arrays that hold bf16-representable values, except
logits/probabilities (fp32) and ids (int64).  Dot products are taken in fp64 and
rounded to fp32 then to bf16 -- the value a bf16 ``F.linear`` with fp32
accumulation rounds to, up to the accumulation order.  Every other bf16 op of the
reference (``silu``, ``*``, ``+``) is evaluated exactly (fp64) and rounded the
same way, so the rounding points are the reference's:

  decode  (T == 1): bf16 after each GEMV, SiLU, multiply, weight-scale and add;
                    experts accumulated in router order (tarfa/engine/fused_int4.py:192-194)
  prefill (T  > 1): same rounding points; experts accumulated in ascending id
                    order via index_add_ (tarfa/engine/fused_int4.py:228-244)
"""
import numpy as np

from . import bf16

rb = bf16.rnd


def dot_bf16(a, w):
    """bf16(a @ w.T) with fp64 accumulation. a [..., K], w [N, K]."""
    return rb((np.asarray(a, np.float64) @ np.asarray(w, np.float64).T).astype(np.float32))


def silu_bf16(g):
    """torch bf16 silu: computed in fp32 from a bf16 input, rounded to bf16."""
    g = np.asarray(g, np.float64)
    return rb((g / (1.0 + np.exp(-g))).astype(np.float32))


def sigmoid_bf16(z):
    z = np.asarray(z, np.float64)
    return rb((1.0 / (1.0 + np.exp(-z))).astype(np.float32))


def mul_bf16(a, b):
    return rb((np.asarray(a, np.float64) * np.asarray(b, np.float64)).astype(np.float32))


def add_bf16(a, b):
    return rb((np.asarray(a, np.float64) + np.asarray(b, np.float64)).astype(np.float32))


# ---------------------------------------------------------------- router (a1)

def router_logits(x, wg):
    """fp32 logits of bf16 x [T,H] and bf16 router weight [E,H].

    The reference router computes ``F.linear(hidden, weight)`` in the hidden
    dtype (transformers/.../modeling_qwen3_5_moe.py:770); the logits here are fp32
    as the workload definition requires (bf16 logits tie inside the top-9 for
    12-39% of tokens, which would leave the top-8 ids ill-defined).
    """
    return (np.asarray(x, np.float64) @ np.asarray(wg, np.float64).T).astype(np.float32)


def router_topk(logits, k):
    """Softmax in fp32, top-k, renormalise, cast to bf16.

    transformers/.../modeling_qwen3_5_moe.py:771-774.  Selection is by fp32
    logit, descending, ties to the lower expert index (softmax is monotone, so
    this is torch.topk's order wherever torch's is defined; torch CPU breaks ties
    in an implementation-defined order).  Probabilities are formed in fp64 from
    the fp32 logits and rounded to fp32; the renormalised weights are rounded to
    bf16.  Returns ids [T,k] int64, weights [T,k] (bf16 values), probs [T,E] fp32.
    """
    lg = np.atleast_2d(np.asarray(logits, np.float32))
    T, E = lg.shape
    idx = np.broadcast_to(np.arange(E), (T, E))
    order = np.lexsort((idx, -lg.astype(np.float64)), axis=-1)
    ids = order[:, :k].astype(np.int64)
    l64 = lg.astype(np.float64)
    ex = np.exp(l64 - l64.max(axis=-1, keepdims=True))
    probs = (ex / ex.sum(axis=-1, keepdims=True)).astype(np.float32)
    top = np.take_along_axis(probs, ids, axis=-1).astype(np.float64)
    w = rb((top / top.sum(axis=-1, keepdims=True)).astype(np.float32))
    return ids, w, probs


def jtopk_truncate(ids, w, j):
    """The reference's re-truncation at its experts boundary, tarfa/engine/fused_int4.py:157-160:
    when a token carries more than j experts, ``tv, ti = w.topk(j)``, ``ids = gather(ids, ti)``,
    ``w = tv / tv.sum(-1, keepdim=True)`` in the weights' dtype (bf16).  Selection by weight,
    descending, equal weights keeping the lower slot first (torch's tie order is
    implementation-defined); the sum of the kept bf16 values in fp32, in the kept order, rounded
    to bf16; each quotient in fp32, rounded to bf16.  ids [T,k] int64, w [T,k] bf16 values ->
    (ids [T,j], w [T,j]); k <= j returns the inputs."""
    ids = np.atleast_2d(np.asarray(ids, np.int64))
    w = np.atleast_2d(np.asarray(w, np.float32))
    T, k = w.shape
    if k <= j:
        return ids, w
    order = np.lexsort((np.broadcast_to(np.arange(k), (T, k)), -w.astype(np.float64)), axis=-1)[:, :j]
    tv = np.take_along_axis(w, order, axis=-1)
    s = np.zeros(T, np.float32)
    for r in range(j):
        s = (s + tv[:, r]).astype(np.float32)
    out = rb((tv / rb(s)[:, None]).astype(np.float32))
    return np.take_along_axis(ids, order, axis=-1), out


def topk_gaps(logits, k):
    """Smallest gap between consecutive sorted logits among the top k+1 (per token)."""
    lg = np.sort(np.atleast_2d(np.asarray(logits, np.float64)), axis=-1)[:, ::-1]
    return np.min(lg[:, :k] - lg[:, 1:k + 1], axis=-1)


# ---------------------------------------------------------------- dispatch (a3)

def dispatch(ids, num_experts):
    """Token -> expert permutation as the reference's prefill builds it.

    ``mask = F.one_hot(ids, E).permute(2, 1, 0)`` gives ``mask[e, slot, t]``; the
    experts hit are taken in ascending id (``nonzero``) and each expert's rows
    are ``torch.where(mask[e])``, i.e. (slot, t) in lexicographic order
    (tarfa/engine/fused_int4.py:228-229, 241; channel.py:46-47, 54).  The implied
    permutation is a stable sort by expert id of the slot-major traversal of the
    [T,k] id matrix.  Ids outside [0, E) (the reference's skip sentinel ``E``,
    fused_int4.py:167) are dropped.

    Returns offsets [E+1] int32 and perm [n_valid] int32 with
    ``perm[r] = t * k + slot`` for the r-th permuted row.
    """
    ids = np.asarray(ids, np.int64)
    T, k = ids.shape
    keys = ids.T.reshape(-1)                       # slot-major traversal: j = slot*T + t
    valid = (keys >= 0) & (keys < num_experts)
    j = np.nonzero(valid)[0]
    order = j[np.argsort(keys[j], kind="stable")]
    slot, t = order // T, order % T
    counts = np.bincount(keys[j], minlength=num_experts)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    return offsets, (t * k + slot).astype(np.int32)


# ---------------------------------------------------------------- expert SwiGLU (a4, a5)

def swiglu_bf16(x, w_gate_up, w_down):
    """One expert: bf16(F.linear(bf16(silu(g)) * u, Wd)) with g, u = chunk(bf16(F.linear(x, Wgu))).

    tarfa/engine/fused_int4.py:193-194 (decode) and :242-243 (prefill);
    transformers/.../modeling_qwen3_5_moe.py:751-753.
    """
    gu = dot_bf16(x, w_gate_up)
    inter = w_gate_up.shape[0] // 2
    a = mul_bf16(silu_bf16(gu[..., :inter]), gu[..., inter:])
    return dot_bf16(a, w_down)


def experts_decode(x, ids, w, gate_up, down, num_experts=None):
    """experts.forward for one token (T == 1): bf16 chain in router order.

    ``acc = acc + w_j * F.linear(act(g) * u, Wd)`` for j in router order, the
    sentinel ``num_experts`` skipped (tarfa/engine/fused_int4.py:165-168, 180,
    192-194, 202).  ``gate_up``/``down`` map expert id -> [2I,H] / [H,I] arrays.
    """
    x = np.asarray(x, np.float32).reshape(-1)
    acc = np.zeros_like(x)
    for j, e in enumerate(np.asarray(ids).reshape(-1).tolist()):
        if num_experts is not None and not (0 <= e < num_experts):
            continue
        d = swiglu_bf16(x, gate_up[e], down[e])
        acc = add_bf16(acc, mul_bf16(np.float32(np.asarray(w).reshape(-1)[j]), d))
    return acc


def experts_prefill(x, ids, w, gate_up, down, num_experts):
    """experts.forward for T > 1: per expert in ascending id, bf16 index_add_.

    tarfa/engine/fused_int4.py:228-244 (same loop as channel.py:44-60 and
    transformers' eager Qwen3_5MoeExperts.forward, modeling_qwen3_5_moe.py:735-757).
    Each expert's contribution ``bf16(bf16(down) * w[t, slot])`` is added to
    ``out[t]`` with one bf16 rounding per add, experts in ascending id order,
    within an expert in (slot, t) order.
    """
    x = np.asarray(x, np.float32)
    ids = np.asarray(ids, np.int64)
    w = np.asarray(w, np.float32)
    T, k = ids.shape
    offsets, perm = dispatch(ids, num_experts)
    out = np.zeros_like(x)
    for e in range(num_experts):
        rows = perm[offsets[e]:offsets[e + 1]]
        if rows.size == 0:
            continue
        tok, slot = rows // k, rows % k
        d = swiglu_bf16(x[tok], gate_up[e], down[e])
        ch = mul_bf16(d, w[tok, slot][:, None])
        for r in range(rows.size):                 # sequential: a token may repeat within an expert
            out[tok[r]] = add_bf16(out[tok[r]], ch[r])
    return out


# ---------------------------------------------------------------- shared expert + combine (a6-a8)

def shared_expert(x, w_gate, w_up, w_down, w_shared_gate):
    """Shared MLP and its sigmoid gate, both bf16 (transformers/.../modeling_qwen3_5_moe.py:715-717, 794).

    Returns bf16(sigmoid(bf16(x . w_sg)) * down(bf16(silu(bf16(gate(x)))) * bf16(up(x)))).
    """
    g = dot_bf16(x, w_gate)
    u = dot_bf16(x, w_up)
    s = dot_bf16(mul_bf16(silu_bf16(g), u), w_down)
    gl = dot_bf16(x, np.asarray(w_shared_gate).reshape(1, -1))     # [..., 1]
    return mul_bf16(sigmoid_bf16(gl), s)


def moe_block(x, logits_or_wg, k, gate_up, down, num_experts, shared=None, logits_given=False):
    """SparseMoeBlock.forward with fp32 router logits (modeling_qwen3_5_moe.py:787-798).

    ``expert_output + shared_expert_output`` adds the routed result first
    (``:796``).  ``shared`` = (w_gate, w_up, w_down, w_shared_gate) or None.
    Returns out [T,H], ids, weights.
    """
    x = np.atleast_2d(np.asarray(x, np.float32))
    logits = np.asarray(logits_or_wg, np.float32) if logits_given else router_logits(x, logits_or_wg)
    ids, w, _ = router_topk(logits, k)
    if x.shape[0] == 1:
        routed = experts_decode(x[0], ids[0], w[0], gate_up, down, num_experts)[None]
    else:
        routed = experts_prefill(x, ids, w, gate_up, down, num_experts)
    if shared is not None:
        routed = add_bf16(routed, shared_expert(x, *shared))
    return routed, ids, w


# ---------------------------------------------------------------- the sublayer around the block

def rmsnorm(h, w, eps):
    """Qwen3_5MoeRMSNorm (transformers modeling_qwen3_5_moe.py:800-814, applied at :870):
    in fp32, y = h * rsqrt(mean(h^2) + eps), then bf16(y * (1 + w)).  The mean is taken in
    fp64 and rounded to fp32 (the value every fp32 summation order approximates); rsqrt as
    1 / sqrt, each step rounded to fp32."""
    h = np.asarray(h, np.float32)
    w = np.asarray(w, np.float32)
    ms = np.mean(np.asarray(h, np.float64) ** 2, axis=-1, keepdims=True).astype(np.float32)
    rs = (np.float32(1.0) / np.sqrt(ms + np.float32(eps))).astype(np.float32)
    y = (h * rs).astype(np.float32)
    return rb((y * (np.float32(1.0) + w)).astype(np.float32))


def moe_layer(h, block_out):
    """The residual add after the block (transformers modeling_qwen3_5_moe.py:875): bf16(h + y)."""
    return add_bf16(h, block_out)
