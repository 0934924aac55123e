"""Router oracle (test infrastructure): the reference's router op order in torch on the CPU."""
import torch

from .native import topk as emulated_topk  # noqa: F401  (re-exported restatement of torch.topk)


def qwen3_router(logits, topk, norm_topk_prob=True):
    """ferry/model.py:141-146: softmax(fp32) -> topk (sorted) -> renorm -> bf16.

    ``logits`` is the bf16 (or fp32) gate output [T, E] on the CPU.  Returns
    (weights bf16 [T, k], selected int64 [T, k], probs fp32 [T, E]).
    """
    probs = torch.softmax(logits.cpu(), dim=-1, dtype=torch.float32)
    weights, selected = torch.topk(probs, topk, dim=-1)
    if norm_topk_prob:
        weights = weights / weights.sum(-1, keepdim=True)
    return weights.to(torch.bfloat16), selected, probs


def deepseek_router(logits, topk, routed_scaling_factor=1.0):
    """Greedy DeepSeek-V2 gate (HF DeepseekV2 MoEGate, reached through ferry/model.py:151-157):
    softmax(fp32) -> topk(sorted=False) -> * routed_scaling_factor; the hook casts to bf16."""
    probs = torch.softmax(logits.cpu().float(), dim=-1)
    weights, selected = torch.topk(probs, topk, dim=-1, sorted=False)
    weights = weights * routed_scaling_factor
    return weights.to(torch.bfloat16), selected, probs
