"""Router oracle (test infrastructure): the reference's router op order on the CPU.

ferry/model.py:141-146 (Qwen3) and the greedy DeepSeek-V2 gate (model.py:151-157) compute
``softmax(logits, fp32)``, ``topk`` and (Qwen3) ``w / w.sum(-1)``.  The softmax and the sum run
through the C restatement of torch's CPU kernels (oracle/softmax.c), which the CPU tests pin
bit for bit against torch.softmax / torch.sum; this keeps the oracle identical on any host CPU
(torch picks its SIMD width per machine, and the summation order follows it).  ``torch.topk``
on those probabilities is the reference's selection itself.
"""
import torch

from .native import softmax as _softmax
from .native import topk as emulated_topk  # noqa: F401  (re-exported restatement of torch.topk)
from .native import weight_sum as _weight_sum


def softmax_fp32(logits):
    """torch.softmax(logits, -1, dtype=float32) on the CPU, bit for bit."""
    return torch.from_numpy(_softmax(logits.cpu().float().numpy()))


def qwen3_router(logits, topk, norm_topk_prob=True):
    """ferry/model.py:141-146: softmax(fp32) -> topk (sorted) -> renorm -> bf16.

    ``logits`` is the bf16 (or fp32) gate output [T, E] on the CPU.  Returns
    (weights bf16 [T, k], selected int64 [T, k], probs fp32 [T, E]).
    """
    probs = softmax_fp32(logits)
    weights, selected = torch.topk(probs, topk, dim=-1)
    if norm_topk_prob:
        weights = weights / torch.from_numpy(_weight_sum(weights.numpy())).unsqueeze(-1)
    return weights.to(torch.bfloat16), selected, probs


def deepseek_router(logits, topk, routed_scaling_factor=1.0):
    """Greedy DeepSeek-V2 gate (HF DeepseekV2 MoEGate, reached through ferry/model.py:151-157):
    softmax(fp32) -> topk(sorted=False) -> * routed_scaling_factor; the hook casts to bf16."""
    probs = softmax_fp32(logits)
    weights, selected = torch.topk(probs, topk, dim=-1, sorted=False)
    weights = weights * routed_scaling_factor
    return weights.to(torch.bfloat16), selected, probs
