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


def _setup(family, device, cap=None, score='frequency'):
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
    rt = OffloadRuntime(spec, pool, [cap], 'ferry', Topology.uniform(1, spec.experts),
                        eviction_score=score)
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
def test_hooked_block_probability_score(device, family):
    """eviction_score='probability' through the hooks: the hook hands the runtime the fp32
    router probabilities of the last W tokens (reference model.py:146 for Qwen3, :154-156 for
    DeepSeek-V2), the runtime's history takes them as rows, and the eviction trace equals the
    oracle's (GateHistoryRef fed the same probability rows, PlannerRef) call by call, with a
    cache small enough to evict; the block outputs match the oracle."""
    import numpy as np
    from oracle.history import GateHistoryRef
    from oracle.policy import PlannerRef
    from ferry_amd.model import install_hooks
    cap = 20     # above any one call's experts (16), below the layers' (32 or 48): evictions
    cfg, model, spec, pool, rt = _setup(family, device, cap=cap, score='probability')
    E, k, H, I = spec.experts, spec.topk, spec.hidden, spec.intermediate
    blocks = [model.model.layers[i].mlp for i in spec.moe_layers]
    gates = [b.gate.weight.detach().clone() for b in blocks]
    shared = [None] * len(blocks)
    if family == 'deepseek_v2':
        shared = [torch.cat([b.shared_experts.gate_proj.weight.reshape(-1),
                             b.shared_experts.up_proj.weight.reshape(-1),
                             b.shared_experts.down_proj.weight.reshape(-1)]).cpu() for b in blocks]
    install_hooks(model, spec, rt, history_window=128)
    hist, planner = GateHistoryRef(spec.layers, E, 128), PlannerRef(spec.layers, E, cap)
    g = torch.Generator(device=device).manual_seed(8)
    calls = 0
    for step, T in enumerate([5, 150, 1, 40, 200, 3, 9, 130, 2, 60]):
        pos = step % spec.layers
        x = torch.randn((1, T, H), generator=g, device=device).to(torch.bfloat16)
        flat = x.reshape(-1, H)
        if family == 'qwen3_moe':
            w_ref, sel_ref, probs_ref = qwen3_router(F.linear(flat, gates[pos]).cpu(), k)
        else:
            w_ref, sel_ref, probs_ref = deepseek_router(
                F.linear(flat.float(), gates[pos].float()).cpu(), k)
        with torch.no_grad():
            out = blocks[pos](x)
        out = (out[0] if isinstance(out, tuple) else out).reshape(-1, H)
        hist.update(pos, probs_ref[-min(T, 128):].numpy())
        planner.plan(rt.event - 1, pos, sel_ref.numpy(), hist.scores(pos))
        assert np.array_equal(rt.controller.slots[0], planner.slots), step
        assert np.array_equal(rt.controller.last, planner.last), step
        assert np.array_equal(rt.controller.scores, planner.scores), step
        torch.cuda.synchronize()
        ref = moe_layer_ref(lambda e: pool[pos * E + e], flat.cpu(), sel_ref, w_ref, E, H, I)
        if shared[pos] is not None:
            ref = ref + shared_mlp_ref(shared[pos], flat.cpu(), H, 2 * I)
        torch.testing.assert_close(out.cpu().float(), ref.float(), rtol=2e-2, atol=1e-2)
        calls += 1
    assert calls == 10 and rt.h2d.copies > cap
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


@pytest.mark.parametrize('family', ['qwen3_moe', 'deepseek_v2'])
def test_load_default_device_cuda(device, tmp_path, family):
    """``load(path, spec)`` with its default device='cuda' places every dense tensor on the
    current GPU (a device without an index must compare equal to 'cuda:<current>'), equal to
    the saved ones, and the pool equals the experts' rows."""
    from ferry_amd.loader import load
    from ferry_amd.model import spec_from_config
    from test_model_loader import expert_rows
    cfg = tiny_qwen3_config() if family == 'qwen3_moe' else tiny_deepseek_config()
    model = tiny_model(cfg, seed=6)
    spec = spec_from_config(cfg)
    model.save_pretrained(tmp_path)
    loaded, pool = load(tmp_path, spec)
    assert pool.is_pinned() and torch.equal(pool, expert_rows(model, spec))
    cur = torch.device('cuda', torch.cuda.current_device())
    ref = {n: t for n, t in model.state_dict().items() if '.experts.' not in n}
    got = loaded.state_dict()
    for n, t in ref.items():
        assert got[n].device == cur, n
        assert torch.equal(got[n].cpu(), t), n
    assert all(b.device == cur for b in loaded.buffers())
