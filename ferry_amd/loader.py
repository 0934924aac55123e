"""Checkpoint loading: routed experts into the pinned host pool, everything else onto the GPU.

Reference: ferry/model.py:73-122 (``load``).  The pool is one pinned bf16 tensor
``[layers * experts, 3 * I * H]``; row ``layer * experts + e`` (layer = position of the block
among ``spec.moe_layers``) holds expert e of that block as ``[gate I x H | up I x H | down H x I]``,
the row format the cache slots and the H2D engine use.

Two on-disk spellings of the routed experts are read:
  * one tensor per projection: ``model.layers.{i}.mlp.experts.{e}.{gate,up,down}_proj.weight``
    (the published Qwen3-MoE / DeepSeek-V2 checkpoints, and what transformers 5.x writes);
  * transformers 5.x's fused in-memory form: ``model.layers.{i}.mlp.experts.gate_up_proj``
    ``[E, 2I, H]`` (gate rows first) and ``...experts.down_proj`` ``[E, H, I]``.
Tensors are read one at a time with safetensors (no pickle) and copied straight into the pool
row, so host memory holds the pool plus one tensor.
"""
import json
import re
from pathlib import Path

import torch

from .model import spec_from_config

_PER_EXPERT = re.compile(r'model\.layers\.(\d+)\.mlp\.experts\.(\d+)\.(gate|up|down)_proj\.weight')
_FUSED = re.compile(r'model\.layers\.(\d+)\.mlp\.experts\.(gate_up_proj|down_proj)')
_PART = {'gate': 0, 'up': 1, 'down': 2}


def is_routed_expert(name):
    return bool(_PER_EXPERT.fullmatch(name) or _FUSED.fullmatch(name))


def checkpoint_files(model_path):
    """{tensor name: shard file} of a safetensors checkpoint (sharded or single file)."""
    from safetensors import safe_open
    root = Path(model_path)
    index = root / 'model.safetensors.index.json'
    if index.exists():
        weight_map = json.loads(index.read_text())['weight_map']
        return {name: root / shard for name, shard in weight_map.items()}
    single = root / 'model.safetensors'
    with safe_open(str(single), framework='pt') as f:
        return {name: single for name in f.keys()}


def _pool_tensor(rows, elements, pinned):
    if pinned:
        from .hostmem import pinned_empty
        return pinned_empty((rows, elements), torch.bfloat16)
    return torch.empty((rows, elements), dtype=torch.bfloat16)


def load_pool(model_path, spec, pinned=True):
    """The pinned expert pool of a checkpoint (every routed expert of every block)."""
    from safetensors import safe_open
    E, H, I = spec.experts, spec.hidden, spec.intermediate
    block_of = {index: pos for pos, index in enumerate(spec.moe_layers)}
    pool = _pool_tensor(spec.layers * E, spec.expert_elements, pinned)
    filled = torch.zeros((spec.layers * E, 3), dtype=torch.bool)
    files = checkpoint_files(model_path)
    by_file = {}
    for name, path in files.items():
        if is_routed_expert(name):
            by_file.setdefault(path, []).append(name)
    part = I * H
    for path in sorted(by_file):
        with safe_open(str(path), framework='pt', device='cpu') as f:
            for name in sorted(by_file[path]):
                m = _PER_EXPERT.fullmatch(name)
                if m:
                    index, e, which = int(m[1]), int(m[2]), _PART[m[3]]
                    if index not in block_of or not 0 <= e < E:
                        raise ValueError(f'{name}: not a routed expert of this spec')
                    t = f.get_tensor(name)
                    want = (H, I) if which == 2 else (I, H)
                    if tuple(t.shape) != want:
                        raise ValueError(f'{name}: shape {tuple(t.shape)}, expected {want}')
                    key = block_of[index] * E + e
                    pool[key, which * part:(which + 1) * part].copy_(t.reshape(-1))
                    filled[key, which] = True
                    continue
                m = _FUSED.fullmatch(name)
                index = int(m[1])
                if index not in block_of:
                    raise ValueError(f'{name}: not a routed-expert block of this spec')
                t = f.get_tensor(name)
                base = block_of[index] * E
                if m[2] == 'gate_up_proj':
                    if tuple(t.shape) != (E, 2 * I, H):
                        raise ValueError(f'{name}: shape {tuple(t.shape)}, expected {(E, 2 * I, H)}')
                    pool[base:base + E, :2 * part].copy_(t.reshape(E, 2 * part))
                    filled[base:base + E, :2] = True
                else:
                    if tuple(t.shape) != (E, H, I):
                        raise ValueError(f'{name}: shape {tuple(t.shape)}, expected {(E, H, I)}')
                    pool[base:base + E, 2 * part:].copy_(t.reshape(E, part))
                    filled[base:base + E, 2] = True
    if not bool(filled.all()):
        key = int((~filled).any(1).nonzero()[0])
        raise ValueError(f'checkpoint lacks routed-expert weights (first: block '
                         f'{spec.moe_layers[key // E]}, expert {key % E})')
    return pool


def pool_from_model(model, spec, pinned=True):
    """The pool of an HF model already in memory (either MoE-block layout); for random-weight
    models that were never written to disk."""
    E, I, H = spec.experts, spec.intermediate, spec.hidden
    pool = _pool_tensor(spec.layers * E, spec.expert_elements, pinned)
    part = I * H
    for pos, index in enumerate(spec.moe_layers):
        experts = model.model.layers[index].mlp.experts
        rows = pool[pos * E:(pos + 1) * E]
        if hasattr(experts, 'gate_up_proj'):
            rows[:, :2 * part].copy_(experts.gate_up_proj.detach().reshape(E, 2 * part))
            rows[:, 2 * part:].copy_(experts.down_proj.detach().reshape(E, part))
        else:
            for e, mlp in enumerate(experts):
                rows[e, :part].copy_(mlp.gate_proj.weight.detach().reshape(-1))
                rows[e, part:2 * part].copy_(mlp.up_proj.weight.detach().reshape(-1))
                rows[e, 2 * part:].copy_(mlp.down_proj.weight.detach().reshape(-1))
    return pool


def _set_tensor(model, name, value):
    """Place ``value`` as the parameter or buffer ``name`` of ``model``."""
    owner_name, _, attr = name.rpartition('.')
    owner = model.get_submodule(owner_name) if owner_name else model
    if attr in owner._parameters:
        owner._parameters[attr] = torch.nn.Parameter(value, requires_grad=False)
    elif attr in owner._buffers:
        owner._buffers[attr] = value
    else:
        raise KeyError(f'{name}: no such parameter or buffer in the model')


def load(model_path, spec=None, device='cuda', pinned=True):
    """(model, pool): the HF causal LM with every tensor except the routed experts on
    ``device`` (bf16, eval mode, SDPA attention), and the pinned expert pool.

    The model is built without allocating parameters, the dense tensors of the checkpoint are
    placed one by one, the routed-expert modules are dropped (their weights live in the pool),
    and buffers computed at construction (rotary frequencies) are moved to the device.
    """
    from accelerate import init_empty_weights
    from safetensors import safe_open
    from transformers import AutoConfig, AutoModelForCausalLM
    config = AutoConfig.from_pretrained(model_path, local_files_only=True)
    config._attn_implementation = 'sdpa'
    spec = spec or spec_from_config(config)
    with init_empty_weights(include_buffers=False):
        model = AutoModelForCausalLM.from_config(config, dtype=torch.bfloat16)
    for index in spec.moe_layers:
        model.model.layers[index].mlp.experts = None
    device = resolve_device(device)
    files = checkpoint_files(model_path)
    by_file = {}
    for name, path in files.items():
        if not is_routed_expert(name):
            by_file.setdefault(path, []).append(name)
    for path in sorted(by_file):
        with safe_open(str(path), framework='pt', device='cpu') as f:
            for name in sorted(by_file[path]):
                _set_tensor(model, name, f.get_tensor(name).to(device=device, dtype=torch.bfloat16))
    if getattr(config, 'tie_word_embeddings', False) and hasattr(model, 'tie_weights'):
        model.tie_weights()
    missing = [n for n, p in model.named_parameters() if p.device != device]
    if missing:
        raise ValueError(f'checkpoint lacks {len(missing)} tensors (first: {missing[0]})')
    place_buffers(model, device)
    model.eval()
    return model, load_pool(model_path, spec, pinned=pinned)


def resolve_device(device):
    """``device`` with its index filled in ('cuda' -> 'cuda:<current>'), so that it compares
    equal to the device of the tensors placed on it."""
    return torch.empty(0, device=device).device


def place_buffers(model, device):
    """Buffers computed while the model was built on the host, moved to ``device``.  Rotary
    embeddings are recomputed there with their own init function, as the reference does
    (model.py:111-115), so that the frequencies are the device's arithmetic and
    ``original_inv_freq`` names the same buffer."""
    for module in model.modules():
        if hasattr(module, 'rope_init_fn') and hasattr(module, 'inv_freq'):
            inv, module.attention_scaling = module.rope_init_fn(module.config, device=device)
            module.register_buffer('inv_freq', inv, persistent=False)
            module.original_inv_freq = inv
    for module in model.modules():
        for key, buf in list(module._buffers.items()):
            if buf is not None and buf.device != device:
                module._buffers[key] = buf.to(device)
