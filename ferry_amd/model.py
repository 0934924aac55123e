"""Model geometry and the MoE-block hooks that route a HuggingFace model through the runtime.

Reference: ferry/model.py.  ``ModelSpec`` keeps the field names FERRY's runtime reads
(model.py:24-48: ``model_type``, ``moe_layers``, ``experts``, ``topk``, ``hidden``,
``intermediate`` and the pooled ``cache_slots`` budget); ``read_spec`` reads them from an HF
``config.json``.  ``install_hooks`` replaces the forward of every routed-expert block
(model.py:125-158) by the hot path of this package: the router GEMM stays a PyTorch GEMM, the
HIP router kernel does softmax / top-k / renormalisation, and ``OffloadRuntime.execute`` runs
the experts.  It recognises both MoE-block layouts of transformers:

* 4.57 (the reference's pin): ``block.gate`` is an ``nn.Linear`` returning logits, Qwen3's
  ``norm_topk_prob`` sits on the block and its forward returns ``(hidden, router_logits)``;
* 5.x (installed here): ``block.gate`` is a router module holding the weight (and, for Qwen3,
  ``norm_topk_prob``), the routed experts are one fused module, and the block returns the
  hidden states alone.

DeepSeek-V2 blocks keep their two shared experts: they are copied into one resident
``[gate | up | down]`` row and added inside the routed combine (``expert_ops.SharedExpert``).
Loading checkpoints into the pinned pool is in ``ferry_amd.loader``.
"""
import json
import types
from dataclasses import dataclass
from pathlib import Path

import torch
import torch.nn.functional as F

from . import expert_ops as ops


@dataclass(frozen=True)
class ModelSpec:
    """Routed-expert geometry of one model (field names as FERRY's ModelSpec)."""

    model_type: str        # 'qwen3_moe' or 'deepseek_v2'
    moe_layers: tuple      # indices of the decoder layers whose MLP is a routed-expert block
    experts: int           # routed experts per block
    topk: int              # experts per token
    hidden: int            # model width H
    intermediate: int      # routed-expert SwiGLU width I

    @property
    def layers(self):
        """Number of routed-expert blocks (pool keys are layer * experts + e)."""
        return len(self.moe_layers)

    @property
    def expert_elements(self):
        """bf16 elements of one pool / cache row: gate I x H, up I x H, down H x I."""
        return 3 * self.intermediate * self.hidden

    @property
    def expert_bytes(self):
        return self.expert_elements * 2

    def cache_slots(self, cache_ratio, world):
        """Cache slots of each rank: a pooled budget of int(layers * experts * ratio) slots
        shared by all blocks, split over the ranks, lower ranks taking the remainder."""
        budget = int(self.layers * self.experts * cache_ratio)
        share, rest = divmod(budget, world)
        return [share + (1 if rank < rest else 0) for rank in range(world)]


# HF config keys per model family: (routed experts, rule selecting the routed-expert layers)
def _qwen3_layers(cfg):
    dense = set(cfg.get('mlp_only_layers') or ())
    step = cfg.get('decoder_sparse_step', 1) or 1
    return [i for i in range(cfg['num_hidden_layers']) if i not in dense and (i + 1) % step == 0]


def _deepseek_layers(cfg):
    if cfg.get('topk_method', 'greedy') != 'greedy':
        raise NotImplementedError(f"DeepSeek-V2 topk_method {cfg['topk_method']!r}: only greedy "
                                  'routing is supported')
    first = cfg.get('first_k_dense_replace', 0)
    every = cfg.get('moe_layer_freq', 1) or 1
    return [i for i in range(first, cfg['num_hidden_layers']) if i % every == 0]


_FAMILIES = {
    'qwen3_moe': (('num_experts', 'num_local_experts'), _qwen3_layers),
    'deepseek_v2': (('n_routed_experts', 'num_local_experts'), _deepseek_layers),
}


def spec_from_config(cfg):
    """ModelSpec of an HF config (a dict, or an object with to_dict())."""
    if not isinstance(cfg, dict):
        cfg = cfg.to_dict()
    family = cfg.get('model_type')
    if family not in _FAMILIES:
        raise NotImplementedError(f'unsupported model_type {family!r}')
    expert_keys, layer_rule = _FAMILIES[family]
    experts = next((cfg[key] for key in expert_keys if cfg.get(key) is not None), None)
    if experts is None:
        raise KeyError(f'{family} config names none of {expert_keys}')
    return ModelSpec(family, tuple(layer_rule(cfg)), int(experts), int(cfg['num_experts_per_tok']),
                     int(cfg['hidden_size']), int(cfg['moe_intermediate_size']))


def read_spec(model_path):
    """ModelSpec from ``<model_path>/config.json`` (reference: model.py:51-70)."""
    return spec_from_config(json.loads((Path(model_path) / 'config.json').read_text()))


# Shapes of the two evaluated models (the HF configs of Qwen3-30B-A3B and DeepSeek-V2-Lite).
QWEN3_30B_A3B = ModelSpec('qwen3_moe', tuple(range(48)), 128, 8, 2048, 768)
DEEPSEEK_V2_LITE = ModelSpec('deepseek_v2', tuple(range(1, 27)), 64, 6, 2048, 1408)
DEEPSEEK_V2_LITE_SHARED_INTERMEDIATE = 2 * 1408


# ---------------------------------------------------------------------------------------------
# One MoE block on [T, H] hidden states
# ---------------------------------------------------------------------------------------------

def _route(rt, logits, topk, **router):
    """Router kernel on the logits; returns (weights, selected, probability tail or None)."""
    want_tail = getattr(rt.gather, 'score', 'frequency') == 'probability'
    res = ops.router_topk(logits, topk, return_probs=want_tail, **router)
    tail = res[2][-rt.window:] if want_tail else None
    return res[0], res[1], tail


def qwen3_moe(rt, layer, flat, gate_weight, topk, norm_topk_prob=True, window=None):
    """Qwen3 MoE block (reference hook: model.py:137-148): bf16 logits = x W^T (PyTorch GEMM),
    then fp32 softmax / top-k / renormalisation / bf16 in the router kernel and the experts in
    the runtime.  Returns (out [T, H], logits)."""
    logits = F.linear(flat, gate_weight)
    weights, selected, tail = _route(rt, logits, topk, renorm=norm_topk_prob)
    return rt.execute(layer, flat, selected, weights, tail), logits


def deepseek_moe(rt, layer, flat, gate_weight, topk, shared=None, routed_scaling_factor=1.0,
                 window=None):
    """DeepSeek-V2 MoE block with the greedy gate (reference hook: model.py:151-158, fed by the
    HF gate): fp32 logits = fp32(x) fp32(W)^T, fp32 softmax / top-k (sorted=False) / scaling /
    bf16 in the router kernel, the routed experts in the runtime, and the shared experts
    (``expert_ops.SharedExpert``) added in bf16 inside the combine.  Returns (out, logits)."""
    logits = F.linear(flat.float(), gate_weight.float())
    weights, selected, tail = _route(rt, logits, topk, renorm=False, sorted=False,
                                     scale=routed_scaling_factor)
    return rt.execute(layer, flat, selected, weights, tail, shared=shared), logits


# ---------------------------------------------------------------------------------------------
# Hooks
# ---------------------------------------------------------------------------------------------

def _gate_weight(block):
    return block.gate.weight


def _gate_is_linear(block):
    """transformers 4.57 layout: the block's gate is a plain linear layer (returns logits)."""
    return isinstance(block.gate, torch.nn.Linear)


def _shared_row(block):
    """The block's shared-expert MLP as one resident bf16 [gate | up | down] row."""
    mlp = block.shared_experts
    parts = [mlp.gate_proj.weight, mlp.up_proj.weight, mlp.down_proj.weight]
    row = torch.cat([p.detach().to(torch.bfloat16).reshape(-1) for p in parts])
    return ops.SharedExpert(row, mlp.gate_proj.weight.shape[1], mlp.gate_proj.weight.shape[0])


def _qwen3_block_forward(rt, layer, spec, returns_logits):
    def forward(block, hidden_states):
        shape = hidden_states.shape
        flat = hidden_states.reshape(-1, shape[-1])
        norm = getattr(block, 'norm_topk_prob', None)
        if norm is None:
            norm = getattr(block.gate, 'norm_topk_prob', True)
        out, logits = qwen3_moe(rt, layer, flat, _gate_weight(block), spec.topk, bool(norm))
        out = out.view(shape)
        return (out, logits) if returns_logits else out
    return forward


def _deepseek_block_forward(rt, layer, spec, shared, scale):
    def forward(block, hidden_states):
        shape = hidden_states.shape
        flat = hidden_states.reshape(-1, shape[-1])
        out, _ = deepseek_moe(rt, layer, flat, _gate_weight(block), spec.topk, shared=shared,
                              routed_scaling_factor=scale)
        return out.view(shape)
    return forward


def install_hooks(model, spec, runtime, history_window=128):
    """Route every routed-expert block of an HF causal LM through ``runtime.execute``
    (reference: model.py:125-134).  The blocks' routed experts are released (they live in the
    pinned pool); DeepSeek-V2's shared experts move into one resident row each.  Returns the
    hooked blocks."""
    if runtime.window != history_window:
        raise ValueError(f'history_window {history_window} differs from the runtime\'s '
                         f'{runtime.window}')
    layers = model.model.layers
    hooked = []
    for layer, index in enumerate(spec.moe_layers):
        block = layers[index].mlp
        if spec.model_type == 'qwen3_moe':
            fwd = _qwen3_block_forward(runtime, layer, spec, returns_logits=_gate_is_linear(block))
        elif spec.model_type == 'deepseek_v2':
            scale = getattr(block.gate, 'routed_scaling_factor',
                            getattr(model.config, 'routed_scaling_factor', 1.0))
            shared = _shared_row(block) if getattr(block, 'shared_experts', None) is not None else None
            fwd = _deepseek_block_forward(runtime, layer, spec, shared, float(scale))
            block.shared_experts = None
        else:
            raise NotImplementedError(spec.model_type)
        block.forward = types.MethodType(fwd, block)
        block.experts = None
        hooked.append(block)
    return hooked
