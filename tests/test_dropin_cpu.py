"""Host-side checks of the drop-in boundary that need no GPU: dtype rejection at install time."""
import pytest
import torch

from tarfa_amd import experts as tx


def _tf_block(dtype):
    from transformers.models.qwen3_5_moe import configuration_qwen3_5_moe as C, modeling_qwen3_5_moe as M
    cfg = C.Qwen3_5MoeTextConfig(hidden_size=64, num_experts=4, moe_intermediate_size=32, num_experts_per_tok=2,
                                 shared_expert_intermediate_size=32, hidden_act="silu")
    return M.Qwen3_5MoeSparseMoeBlock(cfg).to(dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_install_rejects_a_non_bf16_experts_module(dtype):
    """The reference engine defaults to fp16 (tarfa/engine/layered.py:14); libtmoe computes in bf16."""
    blk = _tf_block(dtype)
    with pytest.raises(TypeError, match="bfloat16"):
        tx.install_experts(blk.experts, store=None)
    # nothing was popped or rebound
    assert "gate_up_proj" in dict(blk.experts.named_parameters())
    assert "forward" not in vars(blk.experts)


def test_from_transformers_block_rejects_fp16():
    with pytest.raises(TypeError, match="bfloat16"):
        tx.from_transformers_block(_tf_block(torch.float16), device="cpu")


def test_forward_rejects_a_non_bf16_hidden_state():
    class _Store:
        pass

    fwd = tx.make_experts_forward(_Store())
    with pytest.raises(TypeError, match="bfloat16"):
        fwd(None, torch.zeros(1, 64, dtype=torch.float16), torch.zeros(1, 2, dtype=torch.int64),
            torch.zeros(1, 2))
