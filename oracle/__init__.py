"""CPU oracle for the per-layer MoE hot path — TEST INFRASTRUCTURE ONLY.

This package is the checker, never the product. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it. The product path (``tarfa_amd``) never imports, links or calls
anything here and fails loudly when its HIP library is missing.

Modules
-------
bf16    IEEE round-to-nearest-even fp32 -> bf16 on uint32 bit patterns.
rng     counter-based seeded generator (splitmix64 finaliser, Irwin-Hall n=12 normal
        approximation) whose device twin is ``tarfa_amd/csrc/fill.hip``.
moe     router (fp32 logits, softmax, top-k, renorm), dispatch permutation,
        exact-BF16 expert SwiGLU for decode and prefill, shared expert, combine.
int4    builder-defined group-128 quantiser, dequantiser and the fused
        dequant-GEMV FFN semantics of the int4 fast mode, with the
        enumeration of activations that sit on a bf16 rounding midpoint; the
        reference's own per-row fp16 layout (dequant, GEMV, FFN).
telemetry  route-reuse counters of the reference's decode telemetry.
cpu_reference  the reference's op chain in torch CPU bf16 (CPU baseline, pin).

Every function cites the reference file:line it restates.  Paths
``tarfa/...`` are in the reference repository; ``transformers/...`` is the
third-party package (5.15.0) that the reference calls for its router and shared
expert.

Pinning status (each function is checked in ``tests/test_oracle.py`` and
``tests/test_golden.py`` against something other than its own formula):

* bf16 rounding       pinned: torch ``Tensor.to(bfloat16)`` on 2^24 patterns + edge cases.
* rng                 pinned: moments, determinism, device bit-equality (GPU test).
* router_topk         pinned: torch CPU softmax/topk/renorm on untied inputs.
* jtopk_truncate      pinned: torch CPU run of fused_int4.py:157-160 (topk, gather, bf16
                      sum and division) on untied inputs; ties by brute force (the kept set
                      and order under the lower-slot rule).
* dispatch            pinned: brute force ``one_hot(...).permute(2,1,0)`` + ``torch.where``.
* decode / prefill    pinned: torch CPU bf16 op chain written as the reference writes it
                      (``fused_int4.py:192-194`` / ``:239-244``) and transformers'
                      eager ``Qwen3_5MoeExperts`` / ``Qwen3_5MoeMLP`` / ``SparseMoeBlock``.
* int4 dequant        pinned: exhaustive 16 codes x every finite bf16 scale vs torch.
* int4 quantiser      pinned by invariants only (the reference ships no quantiser).
* int4 ffn            pinned: reference ``_ref_ffn`` closed form (``moe_kernel.py:117-125``)
                      reimplemented in torch fp64 with per-row scales (group = K).
* int4 ffn_candidates pinned: known answers at bf16 midpoints; first candidate == ffn.
* int4 dequant_f16    pinned: exhaustive 16 codes x every finite fp16 scale vs torch's fp16
                      ``q.to(float16) * scale`` (channel_q4.py:10-14 run in torch CPU).
* int4 gemv_rows / ffn_rows  pinned: the reference's ``_ref_ffn`` (moe_kernel.py:117-125) on
                      fp16-dequantised weights in torch fp64, and a brute-force loop.
* int4 dequant_rows_bf16     pinned: torch ``(q.float() * s.float()).to(bfloat16)``.
* telemetry           pinned: a hand-worked sequence of steps (fused_int4.py:71-84).
"""
