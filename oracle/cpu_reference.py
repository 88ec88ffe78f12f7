"""The reference's routed-compute step run on the host CPU in torch bf16 (oracle / CPU baseline only).

This is the reference's own op sequence with ``device='cpu'`` and dtype bf16:

  router      fp32 logits, softmax(fp32), topk, renormalise, cast     transformers/.../modeling_qwen3_5_moe.py:768-776
  decode      acc = acc + w_j * F.linear(act(g) * u, Wd), router order tarfa/engine/fused_int4.py:180, 192-194
  prefill     per expert ascending: where(mask[e]), F.linear x2,        tarfa/engine/fused_int4.py:228-244
              * w[tok, pos], index_add_
  shared      sigmoid(gate(x)) * down(silu(gate_proj x) * up_proj x)  transformers/.../modeling_qwen3_5_moe.py:715-717, 790-796

It is timed by bench.py as the CPU baseline and used by tests as an
independent pin of the numpy oracle.  Nothing in tarfa_amd imports it.
"""
import torch
import torch.nn.functional as F


def router(x, wg, k):
    logits = F.linear(x.float(), wg.float())
    p = torch.softmax(logits, dim=-1, dtype=torch.float)
    tv, ti = torch.topk(p, k, dim=-1)
    tv = tv / tv.sum(dim=-1, keepdim=True)
    return ti, tv.to(torch.bfloat16)


def experts_decode(x, ids, w, gate_up, down):
    """x [H] bf16; ids/w [k]; gate_up/down: indexable by expert id (bf16 [2I,H] / [H,I])."""
    acc = torch.zeros_like(x)
    for j, e in enumerate(ids.tolist()):
        g, u = F.linear(x, gate_up[e]).chunk(2, dim=-1)
        acc = acc + w[j] * F.linear(F.silu(g) * u, down[e])
    return acc


def experts_prefill(x, ids, w, gate_up, down, num_experts):
    out = torch.zeros_like(x)
    mask = F.one_hot(ids, num_classes=num_experts).permute(2, 1, 0)
    hit = torch.greater(mask.sum(dim=(-1, -2)), 0).nonzero().flatten().tolist()
    for e in hit:
        pos, tok = torch.where(mask[e])
        g, u = F.linear(x[tok], gate_up[e]).chunk(2, dim=-1)
        ch = F.linear(F.silu(g) * u, down[e]) * w[tok, pos, None]
        out.index_add_(0, tok, ch.to(out.dtype))
    return out


def shared(x, sg, su, sd, sgw):
    s = F.linear(F.silu(F.linear(x, sg)) * F.linear(x, su), sd)
    return torch.sigmoid(F.linear(x, sgw.reshape(1, -1))) * s


def moe_block(x, wg, k, gate_up, down, num_experts, shared_w=None, logits=None):
    """x [T,H] bf16 -> [T,H] bf16 (fp32 logits, or the supplied ``logits``)."""
    if logits is None:
        ids, w = router(x, wg, k)
    else:
        p = torch.softmax(logits, dim=-1, dtype=torch.float)
        tv, ids = torch.topk(p, k, dim=-1)
        w = (tv / tv.sum(dim=-1, keepdim=True)).to(torch.bfloat16)
    if x.shape[0] == 1:
        out = experts_decode(x[0], ids[0], w[0], gate_up, down)[None]
    else:
        out = experts_prefill(x, ids, w, gate_up, down, num_experts)
    if shared_w is not None:
        out = out + shared(x, *shared_w)
    return out
