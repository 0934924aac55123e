"""CPU tier: model geometry from HF configs, and loading checkpoints into the expert pool.

Tiny Qwen3-MoE and DeepSeek-V2 models are built from configs by the installed transformers
(random weights, no download), written with save_pretrained (per-expert tensor names) or as
safetensors files in transformers 5.x's fused layout, and read back: every pool row must equal
[gate | up | down] of its expert, every dense tensor must equal the saved one."""
import json

import numpy as np
import pytest
import torch


def tiny_qwen3_config(**kw):
    from transformers import Qwen3MoeConfig
    args = dict(vocab_size=256, hidden_size=64, intermediate_size=128, moe_intermediate_size=32,
                num_hidden_layers=3, num_attention_heads=4, num_key_value_heads=2, head_dim=16,
                num_experts=8, num_experts_per_tok=2, max_position_embeddings=256,
                mlp_only_layers=[1], norm_topk_prob=True)
    args.update(kw)
    return Qwen3MoeConfig(**args)


def tiny_deepseek_config(**kw):
    from transformers import DeepseekV2Config
    args = dict(vocab_size=256, hidden_size=64, intermediate_size=128, moe_intermediate_size=32,
                num_hidden_layers=3, num_attention_heads=4, num_key_value_heads=4,
                n_routed_experts=8, num_experts_per_tok=3, n_shared_experts=2,
                first_k_dense_replace=1, kv_lora_rank=16, q_lora_rank=None, qk_rope_head_dim=8,
                qk_nope_head_dim=8, v_head_dim=16, max_position_embeddings=256,
                topk_method='greedy', routed_scaling_factor=1.0)
    args.update(kw)
    return DeepseekV2Config(**args)


def tiny_model(config, seed=0):
    from transformers import AutoModelForCausalLM
    torch.manual_seed(seed)
    model = AutoModelForCausalLM.from_config(config, dtype=torch.bfloat16)
    with torch.no_grad():
        for p in model.parameters():
            p.normal_(0, 0.05)
    return model.eval()


def expert_rows(model, spec):
    """[layers * E, 3 I H] reference rows from the model's own expert parameters."""
    rows = []
    for index in spec.moe_layers:
        ex = model.model.layers[index].mlp.experts
        for e in range(spec.experts):
            gate, up = ex.gate_up_proj[e].chunk(2, dim=0)
            rows.append(torch.cat([gate.reshape(-1), up.reshape(-1), ex.down_proj[e].reshape(-1)]))
    return torch.stack(rows)


def test_read_spec_families(tmp_path):
    from ferry_amd.model import ModelSpec, read_spec, spec_from_config
    q = tiny_qwen3_config(decoder_sparse_step=1)
    (tmp_path / 'config.json').write_text(json.dumps(q.to_dict()))
    assert read_spec(tmp_path) == ModelSpec('qwen3_moe', (0, 2), 8, 2, 64, 32)
    # hub config.json spells the expert count num_experts; a sparse step skips layers
    d = q.to_dict()
    d.pop('num_local_experts', None)
    d.update(num_experts=16, decoder_sparse_step=2, mlp_only_layers=[], num_hidden_layers=6)
    assert spec_from_config(d) == ModelSpec('qwen3_moe', (1, 3, 5), 16, 2, 64, 32)
    ds = tiny_deepseek_config(num_hidden_layers=7, first_k_dense_replace=2, moe_layer_freq=2)
    assert spec_from_config(ds) == ModelSpec('deepseek_v2', (2, 4, 6), 8, 3, 64, 32)
    with pytest.raises(NotImplementedError):
        spec_from_config(tiny_deepseek_config(topk_method='group_limited_greedy', n_group=2,
                                              topk_group=1))
    with pytest.raises(NotImplementedError):
        spec_from_config(dict(model_type='mixtral'))


def test_cache_slots_pool_budget():
    from ferry_amd.model import DEEPSEEK_V2_LITE, QWEN3_30B_A3B
    assert QWEN3_30B_A3B.cache_slots(0.30, 1) == [1843]
    assert DEEPSEEK_V2_LITE.cache_slots(0.30, 1) == [499]
    assert QWEN3_30B_A3B.cache_slots(0.30, 4) == [461, 461, 461, 460]
    assert sum(DEEPSEEK_V2_LITE.cache_slots(0.5, 3)) == int(26 * 64 * 0.5)
    assert QWEN3_30B_A3B.expert_bytes == 9_437_184 and DEEPSEEK_V2_LITE.expert_bytes == 17_301_504


@pytest.mark.parametrize('family', ['qwen3_moe', 'deepseek_v2'])
def test_load_checkpoint_written_by_save_pretrained(tmp_path, family):
    from ferry_amd.loader import checkpoint_files, load, load_pool
    from ferry_amd.model import spec_from_config
    cfg = tiny_qwen3_config() if family == 'qwen3_moe' else tiny_deepseek_config()
    model = tiny_model(cfg, seed=1)
    spec = spec_from_config(cfg)
    model.save_pretrained(tmp_path)
    names = checkpoint_files(tmp_path)
    assert any('.experts.0.gate_proj.weight' in n for n in names)   # per-expert on disk
    want = expert_rows(model, spec)
    pool = load_pool(tmp_path, spec, pinned=False)
    assert pool.shape == (spec.layers * spec.experts, spec.expert_elements)
    assert torch.equal(pool, want)
    loaded, pool2 = load(tmp_path, spec, device='cpu', pinned=False)
    assert torch.equal(pool2, want)
    ref = {n: t for n, t in model.state_dict().items() if '.experts.' not in n}
    got = loaded.state_dict()
    assert not any('.experts.' in n for n in got)
    for n, t in ref.items():
        assert torch.equal(got[n], t), n
    for index in spec.moe_layers:
        assert loaded.model.layers[index].mlp.experts is None
    assert all(b.device.type == 'cpu' for b in loaded.buffers())


def test_load_fused_layout_and_sharded_index(tmp_path):
    """transformers 5.x's fused expert tensors, split over two shards with an index file."""
    from safetensors.torch import save_file
    from ferry_amd.loader import load_pool, pool_from_model
    from ferry_amd.model import spec_from_config
    cfg = tiny_qwen3_config()
    model = tiny_model(cfg, seed=2)
    spec = spec_from_config(cfg)
    sd = {n: t.contiguous() for n, t in model.state_dict().items()}
    names = sorted(sd)
    half = len(names) // 2
    shards = {'a.safetensors': names[:half], 'b.safetensors': names[half:]}
    for shard, keys in shards.items():
        save_file({k: sd[k] for k in keys}, str(tmp_path / shard))
    (tmp_path / 'model.safetensors.index.json').write_text(json.dumps(
        dict(metadata={}, weight_map={k: s for s, keys in shards.items() for k in keys})))
    assert any(n.endswith('experts.gate_up_proj') for n in names)
    pool = load_pool(tmp_path, spec, pinned=False)
    assert torch.equal(pool, expert_rows(model, spec))
    assert torch.equal(pool_from_model(model, spec, pinned=False), pool)


def test_load_rejects_incomplete_or_mismatched(tmp_path):
    from safetensors.torch import save_file
    from ferry_amd.loader import load_pool
    from ferry_amd.model import spec_from_config
    cfg = tiny_qwen3_config()
    spec = spec_from_config(cfg)
    t = torch.zeros(spec.intermediate, spec.hidden, dtype=torch.bfloat16)
    save_file({'model.layers.0.mlp.experts.0.gate_proj.weight': t}, str(tmp_path / 'model.safetensors'))
    with pytest.raises(ValueError, match='lacks routed-expert'):
        load_pool(tmp_path, spec, pinned=False)
    save_file({'model.layers.0.mlp.experts.0.down_proj.weight': t}, str(tmp_path / 'model.safetensors'))
    with pytest.raises(ValueError, match='shape'):
        load_pool(tmp_path, spec, pinned=False)
    save_file({'model.layers.1.mlp.experts.0.up_proj.weight': t}, str(tmp_path / 'model.safetensors'))
    with pytest.raises(ValueError, match='not a routed expert'):
        load_pool(tmp_path, spec, pinned=False)   # layer 1 is a dense MLP layer here


def test_place_buffers_rebuilds_rotary_with_its_init_function():
    """transformers 4.57 rotary modules carry ``rope_init_fn``: place_buffers recomputes the
    frequencies on the target device with it and points ``original_inv_freq`` at the new
    buffer (reference model.py:111-115); other buffers are moved; 5.x modules (no
    ``rope_init_fn``) keep their values."""
    from ferry_amd.loader import place_buffers, resolve_device
    calls = []

    class Rotary457(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.config = 'cfg'
            self.register_buffer('inv_freq', torch.zeros(4), persistent=False)
            self.original_inv_freq = self.inv_freq

        def rope_init_fn(self, config, device=None):
            calls.append((config, device))
            return torch.arange(4, dtype=torch.float32, device=device) + 1, 0.5

    model = torch.nn.Module()
    model.rot = Rotary457()
    model.other = torch.nn.Module()
    model.other.register_buffer('scale', torch.ones(3, dtype=torch.float64))
    dev = resolve_device('cpu')
    place_buffers(model, dev)
    assert calls == [('cfg', dev)]
    assert torch.equal(model.rot.inv_freq, torch.tensor([1.0, 2.0, 3.0, 4.0]))
    assert model.rot.original_inv_freq is model.rot.inv_freq
    assert model.rot.attention_scaling == 0.5
    assert 'inv_freq' in model.rot._buffers and 'inv_freq' in model.rot._non_persistent_buffers_set
    assert torch.equal(model.other.scale, torch.ones(3, dtype=torch.float64))
    # a 5.x model built on the host: its rotary buffers (no rope_init_fn) are left as built
    cfg = tiny_qwen3_config()
    m5 = tiny_model(cfg, seed=1)
    before = {n: b.clone() for n, b in m5.named_buffers()}
    place_buffers(m5, dev)
    assert all(torch.equal(before[n], b) for n, b in m5.named_buffers())


def test_resolve_device_fills_the_index():
    from ferry_amd.loader import resolve_device
    assert resolve_device('cpu') == torch.device('cpu')
    assert resolve_device(torch.device('cpu')).type == 'cpu'
