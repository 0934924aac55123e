"""Model geometry and MoE-layer hooks (reference: ferry/model.py).

``ModelSpec``/``read_spec``/``cache_slots`` keep the reference's fields and pooled cache
budget.  The hook factories route a MoE block through the router kernel and
``OffloadRuntime.execute``; the router GEMM (``gate``) stays a PyTorch GEMM.  Loading real
checkpoints into a pinned pool is out of scope (no checkpoints offline); the synthetic
workloads build pools of the same row format instead (ferry_amd.workloads).
"""
import json
import types
from dataclasses import dataclass
from pathlib import Path

import torch

from . import expert_ops as ops


@dataclass(frozen=True)
class ModelSpec:
    model_type: str
    moe_layers: tuple      # decoder-layer indices that hold routed experts
    experts: int           # routed experts per MoE layer
    topk: int
    hidden: int
    intermediate: int      # routed-expert intermediate size

    @property
    def layers(self):
        return len(self.moe_layers)

    @property
    def expert_elements(self):
        return 3 * self.hidden * self.intermediate

    @property
    def expert_bytes(self):
        return 2 * self.expert_elements

    def cache_slots(self, cache_ratio, world):
        """Global expert-cache budget split evenly across ranks (model.py:45-48)."""
        total = int(self.layers * self.experts * cache_ratio)
        return [total // world + (r < total % world) for r in range(world)]


def read_spec(model_path):
    """ModelSpec from an HF config.json (model.py:51-70)."""
    c = json.loads((Path(model_path) / 'config.json').read_text())
    kind = c['model_type']
    n = c['num_hidden_layers']
    if kind == 'qwen3_moe':
        step = c.get('decoder_sparse_step', 1)
        dense = set(c.get('mlp_only_layers') or [])
        layers = tuple(i for i in range(n) if i not in dense and (i + 1) % step == 0)
        experts = c['num_experts']
    elif kind == 'deepseek_v2':
        first = c['first_k_dense_replace']
        freq = c.get('moe_layer_freq', 1)
        layers = tuple(i for i in range(n) if i >= first and i % freq == 0)
        experts = c['n_routed_experts']
        if c.get('topk_method', 'greedy') != 'greedy':
            raise NotImplementedError('only greedy top-k routing is supported for DeepSeek-V2')
    else:
        raise NotImplementedError(f'unsupported model_type {kind}')
    return ModelSpec(kind, layers, experts, c['num_experts_per_tok'], c['hidden_size'],
                     c['moe_intermediate_size'])


# Shapes of the two evaluated models (HF configs of Qwen3-30B-A3B and DeepSeek-V2-Lite).
QWEN3_30B_A3B = ModelSpec('qwen3_moe', tuple(range(48)), 128, 8, 2048, 768)
DEEPSEEK_V2_LITE = ModelSpec('deepseek_v2', tuple(range(1, 27)), 64, 6, 2048, 1408)
DEEPSEEK_V2_LITE_SHARED_INTERMEDIATE = 2 * 1408


def qwen3_moe(rt, layer, flat, gate_weight, topk, norm_topk_prob=True, window=128):
    """Qwen3 MoE block on [T, H] bf16 hidden states (model.py:137-148).

    logits = flat @ gate^T (PyTorch GEMM), then the router kernel (fp32 softmax, top-k,
    renorm, bf16) and the runtime.  Returns (out [T, H], logits).
    """
    logits = flat @ gate_weight.t()
    want_probs = getattr(rt.gather, 'score', 'frequency') == 'probability'
    res = ops.router_topk(logits, topk, renorm=norm_topk_prob, return_probs=want_probs)
    weights, selected = res[0], res[1]
    tail = res[2][-window:] if want_probs else None
    return rt.execute(layer, flat, selected, weights, tail), logits


def deepseek_moe(rt, layer, flat, gate_weight, topk, shared=None, routed_scaling_factor=1.0,
                 window=128):
    """DeepSeek-V2 MoE block on [T, H] bf16 hidden states, greedy gate.

    logits = fp32(x) @ fp32(gate)^T (PyTorch fp32 GEMM, as the HF gate), then the router kernel
    (fp32 softmax, top-k sorted=False, * routed_scaling_factor, bf16 -- the HF gate plus the cast
    of ferry/model.py:157), the runtime, and the shared experts (``expert_ops.SharedExpert``)
    added in bf16 inside the combine.  Returns (out [T, H], logits).
    """
    logits = flat.float() @ gate_weight.float().t()
    want_probs = getattr(rt.gather, 'score', 'frequency') == 'probability'
    res = ops.router_topk(logits, topk, renorm=False, scale=routed_scaling_factor, sorted=False,
                          return_probs=want_probs)
    weights, selected = res[0], res[1]
    tail = res[2][-window:] if want_probs else None
    return rt.execute(layer, flat, selected, weights, tail, shared=shared), logits


def _qwen3_forward(rt, layer, spec, window):
    def forward(module, hidden_states):
        shape = hidden_states.shape
        flat = hidden_states.reshape(-1, shape[-1])
        out, logits = qwen3_moe(rt, layer, flat, module.gate.weight, spec.topk,
                                bool(getattr(module, 'norm_topk_prob', True)), window)
        return out.view(shape), logits
    return forward


def _deepseek_moe(rt, layer, window):
    def moe(module, hidden_states, topk_ids, topk_weight):
        probs = None
        if rt.gather.score == 'probability':
            tail = hidden_states[-window:]
            probs = torch.softmax(torch.nn.functional.linear(tail.float(), module.gate.weight.float()),
                                  dim=-1)
        return rt.execute(layer, hidden_states, topk_ids, topk_weight.to(torch.bfloat16), probs)
    return moe


def install_hooks(model, spec, runtime, history_window):
    """Route every MoE layer through runtime.execute (model.py:125-134, HF 4.57 module API)."""
    for layer, index in enumerate(spec.moe_layers):
        mlp = model.model.layers[index].mlp
        if spec.model_type == 'qwen3_moe':
            mlp.forward = types.MethodType(_qwen3_forward(runtime, layer, spec, history_window), mlp)
        else:
            mlp.moe = types.MethodType(_deepseek_moe(runtime, layer, history_window), mlp)
        mlp.experts = None
