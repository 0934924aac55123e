"""Synthetic workloads of the five evaluation configurations (no checkpoints or datasets).

Every generator is seeded.  Expert weights are ~N(0, 0.02) bf16 rows in the reference's
pinned-pool format (key = layer * E + e, row = [gate I*H | up I*H | down H*I]); they are
drawn on the GPU (torch Philox, per-row seed) and copied into pinned host memory, which keeps
a 58 GB pool build to seconds.  Router logits are N(0, 1) plus a per-expert bias
log(p_rank) of a Zipf(s) popularity over a seeded permutation of the experts.
"""
from dataclasses import dataclass, replace

import numpy as np
import torch

from .model import DEEPSEEK_V2_LITE, QWEN3_30B_A3B, ModelSpec


@dataclass(frozen=True)
class Workload:
    name: str
    spec: ModelSpec
    tokens: int            # tokens per layer call
    cache_slots: int       # pooled cache slots (world = 1)
    zipf_s: float
    seed: int
    layers: int            # MoE layers exercised
    logits_dtype: torch.dtype
    renorm: bool
    sorted: bool
    shared_intermediate: int = 0   # DeepSeek shared experts (2 x 1408)
    steps: int = 1                 # decode steps (the decode loop)
    prefill_tokens: int = 0        # synthetic prefill before decode (the decode loop)


def _one_layer(spec):
    return replace(spec, moe_layers=spec.moe_layers[:1])


# the evaluated workloads, by what they are
DEEPSEEK_LAYER_T256 = Workload('deepseek_v2_lite_layer_t256_resident', _one_layer(DEEPSEEK_V2_LITE), 256,
                               64, 0.0, 0, 1, torch.float32, False, False,
                               shared_intermediate=2 * 1408)
QWEN3_DECODE_LAYER = Workload('qwen3_30b_a3b_moe_layer_decode_t16_cache38', _one_layer(QWEN3_30B_A3B), 16,
                              38, 1.1, 1, 1, torch.bfloat16, True, True)
QWEN3_PREFILL_STACK = Workload('qwen3_30b_a3b_moe_prefill_t8192_48layers', QWEN3_30B_A3B, 8192,
                               int(48 * 128 * 0.30), 1.1, 1, 48, torch.bfloat16, True, True)
DEEPSEEK_PREFILL_STACK = Workload('deepseek_v2_lite_moe_prefill_t65536_26layers', DEEPSEEK_V2_LITE, 65536,
                                  int(26 * 64 * 0.30), 0.9, 2, 26, torch.float32, False, False,
                                  shared_intermediate=2 * 1408)
QWEN3_DECODE_LOOP = Workload('qwen3_30b_a3b_decode_loop_t64_48layers', QWEN3_30B_A3B, 64,
                             int(48 * 128 * 0.30), 1.1, 1, 48, torch.bfloat16, True, True, steps=64,
                             prefill_tokens=1024)
WORKLOADS = {w.name: w for w in (DEEPSEEK_LAYER_T256, QWEN3_DECODE_LAYER, QWEN3_PREFILL_STACK,
                                 DEEPSEEK_PREFILL_STACK, QWEN3_DECODE_LOOP)}


def zipf_log_bias(experts, s, rng):
    """log popularity of each expert: Zipf(s) over ranks 1..E assigned by a permutation."""
    ranks = np.arange(1, experts + 1, dtype=np.float64)
    p = ranks ** (-s) if s > 0 else np.ones(experts)
    p /= p.sum()
    perm = rng.permutation(experts)
    bias = np.empty(experts, np.float64)
    bias[perm] = np.log(p)
    return bias.astype(np.float32)


class RouterLogits:
    """Per-layer seeded logits streams: N(0, 1) + Zipf log-popularity bias."""

    def __init__(self, workload, device='cuda'):
        w = workload
        rng = np.random.default_rng(w.seed)
        self.bias = [torch.from_numpy(zipf_log_bias(w.spec.experts, w.zipf_s, rng)).to(device)
                     for _ in range(w.layers)]
        self.gen = torch.Generator(device=device)
        self.gen.manual_seed(w.seed)
        self.dtype, self.device, self.E = w.logits_dtype, device, w.spec.experts

    def next(self, layer, tokens):
        z = torch.randn((tokens, self.E), generator=self.gen, device=self.device, dtype=torch.float32)
        return (z + self.bias[layer]).to(self.dtype)


def hidden_states(tokens, hidden, seed, device='cuda'):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return torch.randn((tokens, hidden), generator=g, device=device).to(torch.bfloat16)


def expert_rows(keys, elements, seed, device='cuda', std=0.02):
    """bf16 weight rows of the given pool keys, each from its own Philox seed (seed, key)."""
    out = torch.empty((len(keys), elements), dtype=torch.bfloat16, device=device)
    g = torch.Generator(device=device)
    for i, key in enumerate(keys):
        g.manual_seed(seed * 1_000_003 + int(key))
        out[i] = (torch.randn(elements, generator=g, device=device) * std).to(torch.bfloat16)
    return out


SHARED_KEY0 = 1 << 20   # seed keys of the shared-expert rows, disjoint from the pool keys


def shared_rows(layers, hidden, intermediate, seed, device='cuda'):
    """bf16 [layers, 3 H I] shared-expert rows ([gate | up | down], ~N(0, 0.02))."""
    return expert_rows(range(SHARED_KEY0, SHARED_KEY0 + layers), 3 * hidden * intermediate, seed,
                       device)


def router_gates(spec, layers, seed, device='cuda', std=0.02):
    """bf16 [E, H] router (gate) weights of each layer, ~N(0, std)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed * 1_000_003 + 7)
    return [(torch.randn((spec.experts, spec.hidden), generator=g, device=device) * std)
            .to(torch.bfloat16) for _ in range(layers)]


def make_pool(spec, layers, seed=0, device='cuda', chunk=32, pinned=True):
    """Host pool [layers * E, 3 H I] bf16 of ~N(0, 0.02) rows (model.py:86-106 format), pinned
    (what H2DEngine copies from) or pageable (the source of a PackedPool, which holds its own
    pinned copy: pinned host memory is limited, about a quarter of RAM on MI355X hosts)."""
    from .hostmem import pinned_empty
    n = layers * spec.experts
    shape = (n, spec.expert_elements)
    pool = pinned_empty(shape, torch.bfloat16) if pinned else torch.empty(shape, dtype=torch.bfloat16)
    for k0 in range(0, n, chunk):
        keys = range(k0, min(n, k0 + chunk))
        pool[k0:k0 + len(keys)].copy_(expert_rows(keys, spec.expert_elements, seed, device))
    torch.cuda.synchronize()
    return pool


def feasible_topk_sets(logits_np, k, cap):
    """Number of distinct experts per call (numpy stable top-k on the logits) <= cap - 1.

    The reference aborts (quota.py:63 assert) when a layer's active set exceeds the cache;
    decode streams skip such calls.  The margin of one slot covers a boundary tie that the
    exact top-k may resolve differently from numpy.
    """
    top = np.argsort(-logits_np, axis=1, kind='stable')[:, :k]
    return len(np.unique(top)) <= cap - 1


def decode_loop_routing(workload, seed=None, steps=None, keep=0.8):
    """Routing of the decode loop: a synthetic prefill of ``prefill_tokens`` tokens per layer
    (independent Zipf(s) draws without duplicates), then ``steps`` decode steps of ``tokens``
    tokens from the temporal-locality process of ``temporal_routing``.  Returns a dict with
    prefill int64 [L, P, k], decode int64 [S, L, T, k] and bf16 weights of both (renormalised
    softmax of seeded N(0, 1) logits over each chosen set)."""
    w = workload
    seed = w.seed if seed is None else seed
    steps = w.steps if steps is None else steps
    E, k, L, P = w.spec.experts, w.spec.topk, w.layers, w.prefill_tokens
    rng = np.random.default_rng(seed + 7919)
    pre = np.empty((L, P, k), np.int64)
    for layer in range(L):
        p = np.exp(zipf_log_bias(E, w.zipf_s, rng).astype(np.float64))
        p /= p.sum()
        for t in range(P):
            pre[layer, t] = rng.choice(E, size=k, replace=False, p=p)
    pre_logits = rng.standard_normal((L, P, k)).astype(np.float32)
    sel, logits = temporal_routing(w, steps, w.tokens, seed, keep)

    def weights(z):
        return torch.softmax(torch.from_numpy(z), dim=-1).to(torch.bfloat16)

    return dict(prefill=pre, prefill_weights=weights(pre_logits), decode=sel,
                decode_weights=weights(logits))


def temporal_routing(workload, steps, tokens, seed, keep=0.8):
    """Routing of the 48-layer decode loop: each token keeps each previous expert with p = keep, else resamples
    from Zipf(s) without duplicates.  Returns int64 [steps, layers, tokens, k] and the fp32
    logits whose renormalised softmax over the chosen set gives the weights."""
    w = workload
    E, k, L = w.spec.experts, w.spec.topk, w.layers
    rng = np.random.default_rng(seed)
    pops = []
    for _ in range(L):
        bias = zipf_log_bias(E, w.zipf_s, rng)
        p = np.exp(bias.astype(np.float64))
        pops.append(p / p.sum())
    sel = np.empty((steps, L, tokens, k), np.int64)
    for layer in range(L):
        p = pops[layer]
        cur = np.stack([rng.choice(E, size=k, replace=False, p=p) for _ in range(tokens)])
        for s in range(steps):
            if s > 0:
                for t in range(tokens):
                    row = cur[t]
                    keep_mask = rng.random(k) < keep
                    kept = list(row[keep_mask])
                    need = k - len(kept)
                    if need:
                        q = p.copy()
                        q[kept] = 0
                        q /= q.sum()
                        kept += list(rng.choice(E, size=need, replace=False, p=q))
                    cur[t] = np.array(kept, np.int64)
            sel[s, layer] = cur
    logits = rng.standard_normal((steps, L, tokens, k)).astype(np.float32)
    return sel, logits
