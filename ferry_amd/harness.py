"""End-to-end generation timing on one GPU: greedy decoding with a KV cache, and the serving
metrics the reference reports.

Reference: scripts/run_cell.py:48-76 (``generate``: greedy steps from a common release time,
one device synchronisation and timestamp per generated token) and :147-156 with README.md:
127-138 (the metrics).  With one GPU there is no barrier or broadcast: the release time is
taken after the device has drained.  Metrics of a run of ``steps`` output tokens for
``requests`` sequences:
  TTFT = first token - release;  TPOT = (last token - first token) / (steps - 1);
  E2E = last token - release;    TPS = requests * steps / E2E.

``synthetic_model`` builds a randomly initialised HF causal LM of a given config with its
dense weights on the GPU and no routed-expert tensors (those live in the pinned pool), the
model the bench runs when no checkpoint is available.
"""
import time

import torch


def generate(model, input_ids, steps, start_delay_s=0.0):
    """Greedy decoding of ``steps`` tokens after the prompt ``input_ids`` [B, P] (all the same
    length).  Returns dict(release_ns, first_ns, end_ns, step_ns, tokens [B][steps])."""
    dev = input_ids.device
    batch = input_ids.shape[0]
    torch.cuda.synchronize(dev)
    release = time.perf_counter_ns() + int(start_delay_s * 1e9)
    while time.perf_counter_ns() < release:
        time.sleep(1e-4)
    cache, feed, seen = None, input_ids, 0
    stamps, tokens = [], []
    with torch.inference_mode():
        for _ in range(steps):
            n = feed.shape[1]
            positions = torch.arange(seen, seen + n, device=dev).expand(batch, n)
            mask = torch.ones((batch, seen + n), dtype=torch.long, device=dev)
            out = model(input_ids=feed, attention_mask=mask, position_ids=positions,
                        past_key_values=cache, use_cache=True, logits_to_keep=1)
            cache = out.past_key_values
            nxt = out.logits[:, -1].argmax(-1)
            tokens.append(nxt)
            torch.cuda.synchronize(dev)
            stamps.append(time.perf_counter_ns())
            seen += n
            feed = nxt[:, None]
    return dict(release_ns=release, first_ns=stamps[0], end_ns=stamps[-1], step_ns=stamps,
                tokens=torch.stack(tokens, 1).cpu().tolist())


def serving_metrics(result, requests, steps):
    """TTFT / TPOT / E2E in seconds and TPS in tokens/s of one ``generate`` result."""
    e2e = (result['end_ns'] - result['release_ns']) / 1e9
    ttft = (result['first_ns'] - result['release_ns']) / 1e9
    tpot = (result['end_ns'] - result['first_ns']) / 1e9 / (steps - 1) if steps > 1 else 0.0
    return dict(TTFT=ttft, TPOT=tpot, E2E=e2e, TPS=requests * steps / e2e)


def synthetic_model(config, spec, device='cuda', seed=0, std=0.02):
    """Random-weight HF causal LM of ``config`` on ``device`` (bf16, eval, SDPA attention)
    without its routed-expert tensors: weights ~ N(0, std), norm scales 1."""
    from accelerate import init_empty_weights
    from transformers import AutoModelForCausalLM
    config._attn_implementation = 'sdpa'
    with init_empty_weights(include_buffers=False):
        model = AutoModelForCausalLM.from_config(config, dtype=torch.bfloat16)
    for index in spec.moe_layers:
        model.model.layers[index].mlp.experts = None
    device = torch.device(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    for name, param in list(model.named_parameters()):
        owner_name, _, attr = name.rpartition('.')
        owner = model.get_submodule(owner_name)
        if 'norm' in attr or 'norm' in owner_name.rsplit('.', 1)[-1]:
            value = torch.ones(param.shape, dtype=torch.bfloat16, device=device)
        else:
            value = (torch.randn(param.shape, generator=gen, device=device) * std).to(torch.bfloat16)
        owner._parameters[attr] = torch.nn.Parameter(value, requires_grad=False)
    if getattr(config, 'tie_word_embeddings', False):
        model.tie_weights()
    for module in model.modules():
        for key, buf in list(module._buffers.items()):
            if buf is not None and buf.device != device:
                module._buffers[key] = buf.to(device)
    return model.eval()
