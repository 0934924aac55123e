"""The Qwen3-30B-A3B decode loop (48 MoE layers, a 1024-token prefill, then 64 steps of 64
tokens; pooled cache of 30% = 1,843 slots; GateHistory W = 128 selection frequency with LRU
tie-break) through OffloadRuntime: the whole fetch / eviction sequence must equal the oracle
planner's, call by call.  The sequence depends only on the routing, so the experts are kept
small (H = 256, I = 128) to bound the pool; the routing process is the full-size one."""
from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle.experts import moe_layer_ref
from oracle.history import GateHistoryRef, frequency_rows
from oracle.policy import PlannerRef

pytestmark = pytest.mark.gpu


def test_decode_loop_eviction_sequence_bit_exact(device):
    from ferry_amd import workloads
    from ferry_amd.quota import Topology
    from ferry_amd.runtime import OffloadRuntime
    w = workloads.QWEN3_DECODE_LOOP
    spec = replace(w.spec, hidden=256, intermediate=128)
    L, E, k = w.layers, spec.experts, spec.topk
    cap = w.cache_slots
    assert (L, E, k, cap, w.tokens, w.prefill_tokens, w.steps) == (48, 128, 8, 1843, 64, 1024, 64)
    routing = workloads.decode_loop_routing(w)
    pool = workloads.make_pool(spec, L, seed=w.seed)
    rt = OffloadRuntime(spec, pool, [cap], 'ferry', Topology.uniform(1, E))
    planner = PlannerRef(L, E, cap)
    hist = GateHistoryRef(L, E, 128)
    g = torch.Generator(device=device)
    g.manual_seed(w.seed)
    xs = {T: torch.randn((T, spec.hidden), generator=g, device=device).to(torch.bfloat16)
          for T in (w.prefill_tokens, w.tokens)}
    calls = [(routing['prefill'][layer], routing['prefill_weights'][layer], layer) for layer in range(L)]
    calls += [(routing['decode'][s, layer], routing['decode_weights'][s, layer], layer)
              for s in range(w.steps) for layer in range(L)]
    total_fetches = evictions = 0
    for i, (sel_np, wts, layer) in enumerate(calls):
        sel = torch.from_numpy(np.ascontiguousarray(sel_np))
        before = planner.slots.copy()
        out = rt.execute(layer, xs[sel.shape[0]], sel.to(device), wts.to(device), None)
        hist.update(layer, frequency_rows(sel_np, E, 128))
        fetches, _ = planner.plan(i, layer, sel_np, hist.scores(layer))
        assert np.array_equal(rt.controller.slots[0], planner.slots), f'call {i} (layer {layer})'
        assert np.array_equal(rt.controller.last, planner.last), f'call {i}'
        assert np.array_equal(rt.controller.scores, planner.scores), f'call {i}'
        total_fetches += len(fetches)
        evictions += int(np.sum(before[fetches[:, 2]] >= 0)) if len(fetches) else 0
        if i % 401 == 0 or i == len(calls) - 1:
            torch.cuda.synchronize()
            ref = moe_layer_ref(lambda e: pool[layer * E + e], xs[sel.shape[0]].cpu(), sel, wts, E,
                                spec.hidden, spec.intermediate)
            torch.testing.assert_close(out.cpu().float(), ref.float(), rtol=2e-2, atol=1e-2)
    rt.h2d.synchronize()
    assert rt.h2d.copies == total_fetches == int(rt.fetches_per_rank.sum())
    decode_calls = w.steps * L
    # the decode phase refetches experts evicted by the other layers (~70 per layer-step)
    assert int(rt.decode_fetches_per_rank.sum()) > 30 * decode_calls
    assert evictions > 0.9 * total_fetches - cap
    rt.close()


def test_decode_steps_full_expert_shape(device):
    """The decode loop's call shapes with full-size Qwen3-30B-A3B experts (H = 2048, I = 768): a
    1024-token prefill and three 64-token decode steps over 4 layers of the temporal-locality
    routing, with a cache small enough to fetch and evict every step.  Every token's output is
    checked against the oracle, and the eviction sequence against the oracle planner."""
    from ferry_amd import workloads
    from ferry_amd.quota import Topology
    from ferry_amd.runtime import OffloadRuntime
    w = replace(workloads.QWEN3_DECODE_LOOP, layers=4)
    spec = replace(w.spec, moe_layers=w.spec.moe_layers[:4])
    L, E, k, H, I = 4, spec.experts, spec.topk, spec.hidden, spec.intermediate
    assert (H, I, w.tokens, w.prefill_tokens) == (2048, 768, 64, 1024)
    cap = 160
    routing = workloads.decode_loop_routing(w, steps=3)
    pool = workloads.make_pool(spec, L, seed=w.seed)
    rt = OffloadRuntime(spec, pool, [cap], 'ferry', Topology.uniform(1, E))
    planner, hist = PlannerRef(L, E, cap), GateHistoryRef(L, E, 128)
    g = torch.Generator(device=device)
    g.manual_seed(11)
    calls = [(routing['prefill'][layer], routing['prefill_weights'][layer], layer) for layer in range(L)]
    calls += [(routing['decode'][s, layer], routing['decode_weights'][s, layer], layer)
              for s in range(3) for layer in range(L)]
    for i, (sel_np, wts, layer) in enumerate(calls):
        T = sel_np.shape[0]
        print(f'call {i}: layer {layer}, {T} tokens', flush=True)
        x = torch.randn((T, H), generator=g, device=device).to(torch.bfloat16)
        sel = torch.from_numpy(np.ascontiguousarray(sel_np))
        out = rt.execute(layer, x, sel.to(device), wts.to(device), None)
        hist.update(layer, frequency_rows(sel_np, E, 128))
        planner.plan(i, layer, sel_np, hist.scores(layer))
        assert np.array_equal(rt.controller.slots[0], planner.slots), f'call {i}'
        if T <= 64:   # every decode token; the prefill calls are covered by the layer tests
            torch.cuda.synchronize()
            ref = moe_layer_ref(lambda e: pool[layer * E + e], x.cpu(), sel, wts, E, H, I)
            torch.testing.assert_close(out.cpu().float(), ref.float(), rtol=2e-2, atol=1e-2)
    assert rt.decode_fetches_per_rank[0] > 0
    rt.close()


def test_decode_loop_full_size_48_layers_packed(device):
    """The decode loop at full size, as the bench runs it: 48 layers of full Qwen3-30B-A3B
    experts (H = 2048, I = 768; a 58 GB pool, built pageable and packed for the host link), the
    pooled cache of 1,843 slots, a 1024-token prefill and four 64-token decode steps of the
    temporal-locality routing.  The fetch / eviction trace equals the oracle planner's after
    every call; the output of every 11th call is checked on 8 of its tokens."""
    from ferry_amd import workloads
    from ferry_amd.h2d import PackedPool
    from ferry_amd.quota import Topology
    from ferry_amd.runtime import OffloadRuntime
    steps = 4
    w = workloads.QWEN3_DECODE_LOOP
    spec = w.spec
    L, E, k, H, I, cap = w.layers, spec.experts, spec.topk, spec.hidden, spec.intermediate, w.cache_slots
    assert (L, H, I, cap) == (48, 2048, 768, 1843)
    print('building the 48-layer pool', flush=True)
    routing = workloads.decode_loop_routing(w, steps=steps)
    pool = workloads.make_pool(spec, L, seed=w.seed, pinned=False)
    packed = PackedPool(pool, threads=16)
    print(f'packed pool: ratio {packed.ratio:.3f}', flush=True)
    rt = OffloadRuntime(spec, packed, [cap], 'ferry', Topology.uniform(1, E))
    planner, hist = PlannerRef(L, E, cap), GateHistoryRef(L, E, 128)
    g = torch.Generator(device=device)
    g.manual_seed(w.seed)
    xs = {T: torch.randn((T, H), generator=g, device=device).to(torch.bfloat16)
          for T in (w.prefill_tokens, w.tokens)}
    calls = [(routing['prefill'][layer], routing['prefill_weights'][layer], layer) for layer in range(L)]
    calls += [(routing['decode'][s, layer], routing['decode_weights'][s, layer], layer)
              for s in range(steps) for layer in range(L)]
    rng = np.random.default_rng(3)
    checked = 0
    total = 0
    for i, (sel_np, wts, layer) in enumerate(calls):
        sel = torch.from_numpy(np.ascontiguousarray(sel_np))
        x = xs[sel.shape[0]]
        out = rt.execute(layer, x, sel.to(device), wts.to(device), None)
        hist.update(layer, frequency_rows(sel_np, E, 128))
        fetches, _ = planner.plan(i, layer, sel_np, hist.scores(layer))
        total += len(fetches)
        assert np.array_equal(rt.controller.slots[0], planner.slots), f'call {i} (layer {layer})'
        assert np.array_equal(rt.controller.last, planner.last), f'call {i}'
        assert np.array_equal(rt.controller.scores, planner.scores), f'call {i}'
        if i % 11 == 0:
            torch.cuda.synchronize()
            pick = np.sort(rng.choice(sel.shape[0], 8, replace=False))
            ref = moe_layer_ref(lambda e: pool[layer * E + e], x.cpu()[pick], sel[pick], wts[pick],
                                E, H, I)
            torch.testing.assert_close(out.cpu()[pick].float(), ref.float(), rtol=2e-2, atol=1e-2)
            checked += 1
        if i % 48 == 47:
            print(f'call {i + 1} of {len(calls)}: {total} fetches so far', flush=True)
    rt.h2d.synchronize()
    assert rt.h2d.copies == total == int(rt.fetches_per_rank.sum())
    assert int(rt.decode_fetches_per_rank.sum()) > 30 * steps * L and checked >= 20
    rt.close()
    packed.close()
