"""MoE-block hooks on HuggingFace models (transformers 5.x installed; 4.57 block layout too).

Tiny Qwen3-MoE and DeepSeek-V2 models with random bf16 weights run on the GPU.  After
``install_hooks`` every routed-expert block goes through the router kernel and
``OffloadRuntime.execute``; a block's output must match the oracle (the reference op order on
the CPU, with the shared experts for DeepSeek-V2) within rel 2e-2 / abs 1e-2, with the routing
bit-exact, and match HF's own block wherever HF's GPU top-k chose the same experts.  A greedy
decode through the hooked model exercises the decoder layers' use of the hooked blocks.
"""
import copy

import pytest
import torch
import torch.nn.functional as F

from oracle.experts import moe_layer_ref, shared_mlp_ref
from oracle.router import deepseek_router, qwen3_router
from test_model_loader import tiny_deepseek_config, tiny_model, tiny_qwen3_config

pytestmark = pytest.mark.gpu

SHAPE = dict(hidden_size=256, moe_intermediate_size=128, intermediate_size=512, num_hidden_layers=3,
             num_attention_heads=4, vocab_size=512)


def _setup(family, device, cap=None):
    from ferry_amd.loader import pool_from_model
    from ferry_amd.model import spec_from_config
    from ferry_amd.quota import Topology
    from ferry_amd.runtime import OffloadRuntime
    if family == 'qwen3_moe':
        cfg = tiny_qwen3_config(num_experts=16, num_experts_per_tok=4, head_dim=64,
                                num_key_value_heads=2, **SHAPE)
    else:
        cfg = tiny_deepseek_config(n_routed_experts=16, num_experts_per_tok=4, num_key_value_heads=4,
                                   kv_lora_rank=64, qk_rope_head_dim=32, qk_nope_head_dim=32,
                                   v_head_dim=64, **SHAPE)
    model = tiny_model(cfg, seed=3).to(device)
    spec = spec_from_config(cfg)
    pool = pool_from_model(model, spec)
    cap = cap or spec.layers * spec.experts
    rt = OffloadRuntime(spec, pool, [cap], 'ferry', Topology.uniform(1, spec.experts))
    return cfg, model, spec, pool, rt


@pytest.mark.parametrize('family', ['qwen3_moe', 'deepseek_v2'])
def test_hooked_block_matches_oracle_and_hf(device, family):
    from ferry_amd import expert_ops as ops
    from ferry_amd.model import install_hooks
    cfg, model, spec, pool, rt = _setup(family, device)
    E, k, H, I = spec.experts, spec.topk, spec.hidden, spec.intermediate
    pos = 0
    block = model.model.layers[spec.moe_layers[pos]].mlp
    g = torch.Generator(device=device).manual_seed(4)
    x = torch.randn((2, 150, H), generator=g, device=device).to(torch.bfloat16)
    flat = x.reshape(-1, H)
    with torch.no_grad():
        hf_out = block(x).reshape(-1, H)
        hf_logits, hf_w, hf_sel = block.gate(flat)
    shared_row = None
    if family == 'deepseek_v2':
        m = block.shared_experts
        shared_row = torch.cat([m.gate_proj.weight.reshape(-1), m.up_proj.weight.reshape(-1),
                                m.down_proj.weight.reshape(-1)]).cpu()
    gate_w = block.gate.weight.detach().clone()
    install_hooks(model, spec, rt, history_window=128)
    with torch.no_grad():
        out = block(x)
    torch.cuda.synchronize()
    assert out.shape == x.shape and out.dtype == torch.bfloat16
    out = out.reshape(-1, H).cpu()
    # routing: the hook's router-kernel call equals the oracle on the same logits
    if family == 'qwen3_moe':
        logits = F.linear(flat, gate_w)
        w_ref, sel_ref, _ = qwen3_router(logits.cpu(), k)
        w, sel = ops.router_topk(logits, k, renorm=True)
    else:
        logits = F.linear(flat.float(), gate_w.float())
        w_ref, sel_ref, _ = deepseek_router(logits.cpu(), k)
        w, sel = ops.router_topk(logits, k, renorm=False, sorted=False)
    assert torch.equal(sel.cpu(), sel_ref) and torch.equal(w.cpu(), w_ref)
    ref = moe_layer_ref(lambda e: pool[pos * E + e], flat.cpu(), sel_ref, w_ref, E, H, I)
    if shared_row is not None:
        ref = ref + shared_mlp_ref(shared_row, flat.cpu(), H, 2 * I)
    torch.testing.assert_close(out.float(), ref.float(), rtol=2e-2, atol=1e-2)
    # HF's own block (bf16 accumulation, GPU top-k) where it picked the same experts
    same = (hf_sel.sort(-1).values.cpu() == sel_ref.sort(-1).values).all(-1)
    assert same.float().mean() > 0.9
    torch.testing.assert_close(out[same].float(), hf_out.cpu()[same].float(), rtol=4e-2, atol=2e-2)
    rt.close()


@pytest.mark.parametrize('family', ['qwen3_moe', 'deepseek_v2'])
def test_hooked_model_greedy_decode(device, family):
    """Prefill + 8 greedy decode steps with a KV cache through the hooked model, with a cache
    smaller than the experts so that fetches and evictions happen every step."""
    from ferry_amd.harness import generate
    from ferry_amd.model import install_hooks
    cfg, model, spec, pool, rt = _setup(family, device, cap=20)
    ref_model = copy.deepcopy(model)
    install_hooks(model, spec, rt)
    ids = torch.randint(0, cfg.vocab_size, (3, 40), device=device,
                        generator=torch.Generator(device=device).manual_seed(5))
    res = generate(model, ids, steps=8)
    assert len(res['tokens']) == 3 and all(len(t) == 8 for t in res['tokens'])
    assert res['release_ns'] <= res['first_ns'] <= res['end_ns']
    assert rt.h2d.copies > 0 and rt.fetches_per_rank[0] == rt.h2d.copies
    assert rt.decode_fetches_per_rank[0] > 0
    # the hooked model's first-step logits agree with HF's own (unhooked) model
    with torch.no_grad():
        a = model(input_ids=ids, logits_to_keep=1).logits[:, -1].float()
        b = ref_model(input_ids=ids, logits_to_keep=1).logits[:, -1].float()
    assert torch.isfinite(a).all()
    assert F.cosine_similarity(a, b, dim=-1).min() > 0.98
    rt.close()


def test_hooks_on_transformers_457_block_layout(device):
    """The 4.57 Qwen3 block layout (gate = nn.Linear returning logits, norm_topk_prob on the
    block, forward returning (hidden, router_logits)) gets a hook with that return type."""
    from ferry_amd.model import install_hooks
    cfg, model, spec, pool, rt = _setup('qwen3_moe', device)
    index = spec.moe_layers[0]
    new_block = model.model.layers[index].mlp
    old = torch.nn.Module()
    old.gate = torch.nn.Linear(spec.hidden, spec.experts, bias=False, device=device,
                               dtype=torch.bfloat16)
    old.gate.weight.data.copy_(new_block.gate.weight.data)
    old.norm_topk_prob = True
    old.experts = torch.nn.ModuleList()
    model.model.layers[index].mlp = old
    install_hooks(model, spec, rt)
    x = torch.randn((1, 7, spec.hidden), device=device).to(torch.bfloat16)
    out, logits = old(x)
    assert out.shape == x.shape and logits.shape == (7, spec.experts)
    torch.testing.assert_close(logits, F.linear(x.reshape(-1, spec.hidden), old.gate.weight))
    assert old.experts is None
    rt.close()
