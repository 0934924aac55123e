"""Dispatch / combine at world = 1 (reference: ferry/transport.py).

With one GPU the all-to-all exchanges are identities: dispatch hands the hidden states and the
routing weights in sorted-ID order to the experts, combine sums the expert outputs per token
(fp32, ascending expert ID) and casts to bf16.  Cross-GPU bytes stay zero.
"""
from . import expert_ops as ops


class Transport:
    def __init__(self, ops_module, topk, experts):
        self.ops, self.topk, self.experts = ops_module, topk, experts
        self.rank = 0
        self.dispatch_bytes = self.combine_bytes = 0

    def dispatch(self, hidden, selected, weights, layout):
        lay = layout['layout']
        return hidden, lay.w_sorted

    def combine(self, hidden, parts, layout, addend=None):
        """``parts`` is the token-major [T*k, H] bf16 output of the expert FFN; ``addend``
        (bf16 [T, H], optional) is added to the bf16 result in fp32."""
        return ops.combine(parts, hidden.shape[0], self.topk, hidden.shape[1], addend=addend)
