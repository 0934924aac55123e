"""The Qwen3-30B-A3B-shaped prefill layer at full size on the HIP path.

8192 tokens, 128 experts top-8 (renormalised softmax), hidden 2048, SwiGLU intermediate 768,
bf16 router logits N(0, 1) + log Zipf(1.1) popularity (seed 1), every expert resident: the
layer the bench times.  The routing is Zipf-skewed, so one launch mixes every kernel family:
the largest expert has 7,966 rows (31 full 256-row M tiles and a partial one), dozens of
experts take the tiled MFMA kernels with a partial last M tile, and half of the experts have at
most 64 rows (small-expert kernels).

Routing indices, the weights and the permutation are checked on every token.  A token's output
depends only on its own row and its experts, so the reference op order
(expert_ops.cpp:54-83 execute_experts, :114-121 reduce_partials) is evaluated exactly on a
sample of tokens chosen to cover every partial M tile, the largest expert and every small
expert.  The layer runs twice: through ``OffloadRuntime.execute`` (experts fetched into the
cache, issued in two calls by row count) and as one ``expert_ffn`` call over all experts (the
bench's form); both must match the oracle, and each other bit for bit.
"""
from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle.experts import moe_layer_ref
from oracle.layout import layout_closed_form
from oracle.router import qwen3_router

pytestmark = pytest.mark.gpu

TILE_M = 256          # rows per M tile of the tiled kernels
SMALL_MAX_ROWS = 64   # experts up to this many rows run the small-expert kernels


def _sample_tokens(starts, rows, rng):
    """Token indices covering: every row of the last 32-row block of each partial M tile plus
    the first row of each partial tile, one row of every small expert, and the first and last
    rows of the largest expert."""
    pick = set()
    counts = np.diff(starts)
    for e, n in enumerate(counts):
        if n == 0:
            continue
        a = int(starts[e])
        if n <= SMALL_MAX_ROWS:
            pick.add(int(rows[a + rng.integers(n)]))
            continue
        last0 = (n - 1) // TILE_M * TILE_M          # first row of the last M tile
        pick.add(int(rows[a + last0]))
        blk0 = max(last0, (n - 1) // 32 * 32)         # last 32-row block that holds rows
        for p in range(blk0, n):
            pick.add(int(rows[a + p]))
    big = int(np.argmax(counts))
    pick.add(int(rows[starts[big]]))
    pick.add(int(rows[starts[big + 1] - 1]))
    return np.array(sorted(pick), np.int64)


def test_qwen3_prefill_t8192_full_layer(device):
    from ferry_amd import expert_ops as ops
    from ferry_amd import workloads
    from ferry_amd.quota import Topology
    from ferry_amd.runtime import OffloadRuntime
    w = workloads.QWEN3_PREFILL_STACK
    spec = replace(w.spec, moe_layers=w.spec.moe_layers[:1])
    E, k, H, I, T = spec.experts, spec.topk, spec.hidden, spec.intermediate, w.tokens
    assert (E, k, H, I, T) == (128, 8, 2048, 768, 8192)
    print(f'qwen3 prefill layer: T={T} E={E} k={k} H={H} I={I}', flush=True)
    logits = workloads.RouterLogits(replace(w, layers=1), device).next(0, T)
    x = workloads.hidden_states(T, H, seed=w.seed + 7, device=device)
    pool = workloads.make_pool(spec, 1, seed=w.seed)

    # 1. through the runtime: cold cache of E slots, so every active expert is fetched
    rt = OffloadRuntime(spec, pool, [E], 'ferry', Topology.uniform(1, E))
    wts, sel = ops.router_topk(logits, k)
    out_rt = rt.execute(0, x, sel, wts, None)
    torch.cuda.synchronize()

    # 2. one expert_ffn call over all experts, as the bench times the layer
    cache = pool.to(device)
    lay = ops.layout(sel, wts, E, check=True)
    act = torch.empty((T * k, I), dtype=torch.bfloat16, device=device)
    part = torch.empty((T * k, H), dtype=torch.bfloat16, device=device)
    ops.expert_ffn(cache, x, lay.w_sorted, lay.starts, lay.rows, lay.cols, np.arange(E),
                   np.arange(E, dtype=np.int32), H, I, act, part, max_rows=T)
    out_one = ops.combine(part, T, k, H)
    torch.cuda.synchronize()

    # routing on every token
    w_ref, sel_ref, _ = qwen3_router(logits.cpu(), k)
    assert torch.equal(sel.cpu(), sel_ref)
    assert torch.equal(wts.cpu(), w_ref)
    # permutation on every token
    wts_c = wts.cpu()
    ref_lay = layout_closed_form(sel_ref.numpy(), E, wts_c.view(torch.int16).numpy())
    for key in ('send_ids', 'starts', 'rows', 'cols', 'pair_pos'):
        assert np.array_equal(getattr(lay, key).cpu().numpy(), ref_lay[key]), key
    assert np.array_equal(lay.w_sorted.cpu().view(torch.int16).numpy(), ref_lay['w_sorted'])
    counts = np.diff(ref_lay['starts'])
    tiled = counts > SMALL_MAX_ROWS
    partial = tiled & (counts % TILE_M != 0)
    assert counts.max() == 7966, counts.max()
    assert partial.sum() >= 40 and ((counts > 0) & ~tiled).sum() >= 40
    print(f'tiled experts {int(tiled.sum())}, partial M tiles {int(partial.sum())}, '
          f'small experts {int(((counts > 0) & ~tiled).sum())}', flush=True)

    # the two paths compute every expert row with the same kernels
    assert torch.equal(out_rt, out_one)

    # output on the sampled tokens against the reference op order
    pick = _sample_tokens(ref_lay['starts'], ref_lay['rows'], np.random.default_rng(3))
    assert len(pick) >= 200
    ref = moe_layer_ref(lambda e: pool[e], x.cpu()[pick], sel_ref[pick], wts_c[pick], E, H, I)
    torch.testing.assert_close(out_rt.cpu()[pick].float(), ref.float(), rtol=2e-2, atol=1e-2)
    rt.close()


def _edge_tokens(starts, rows, rng):
    """A compact sample per layer: one row of every small expert; per tiled expert the first
    row of its last M tile, the first and last rows of that tile's last 32-row block and one
    random row of the tile; the largest expert's first and last rows."""
    pick = set()
    counts = np.diff(starts)
    for e, n in enumerate(counts):
        if n == 0:
            continue
        a = int(starts[e])
        if n <= SMALL_MAX_ROWS:
            pick.add(int(rows[a + rng.integers(n)]))
            continue
        last0 = (n - 1) // TILE_M * TILE_M
        blk0 = max(last0, (n - 1) // 32 * 32)
        for p in {last0, blk0, n - 1, int(rng.integers(last0, n))}:
            pick.add(int(rows[a + p]))
    big = int(np.argmax(counts))
    pick.update((int(rows[starts[big]]), int(rows[starts[big + 1] - 1])))
    return np.array(sorted(pick), np.int64)


def test_qwen3_prefill_stack_4_layers_packed_pooled_cache(device):
    """Four layers of the Qwen3-30B-A3B-shaped prefill stack (8192 tokens each, the stack's
    seeded routing) through OffloadRuntime with packed fetches and a pooled cache of 153 slots
    (30 % of 4 x 128): each layer's ~127 active experts evict most of the previous layer's, and
    its misses are copied in chunks, heaviest first.  The fetch / eviction trace equals the
    oracle's (GateHistoryRef + PlannerRef) after every layer, and each layer's output matches
    the reference op order on a sample of tokens at the tile edges."""
    from ferry_amd import expert_ops as ops
    from ferry_amd import workloads
    from ferry_amd.h2d import PackedPool
    from ferry_amd.quota import Topology
    from ferry_amd.runtime import OffloadRuntime
    from oracle.history import GateHistoryRef, frequency_rows
    from oracle.policy import PlannerRef
    w = workloads.QWEN3_PREFILL_STACK
    L = 4
    spec = replace(w.spec, moe_layers=w.spec.moe_layers[:L])
    E, k, H, I, T = spec.experts, spec.topk, spec.hidden, spec.intermediate, w.tokens
    cap = int(0.30 * L * E)
    assert cap == 153
    print(f'qwen3 prefill stack: {L} layers, T={T}, cap={cap}, packed', flush=True)
    gen = workloads.RouterLogits(replace(w, layers=L), device)
    logits = [gen.next(layer, T) for layer in range(L)]
    x = workloads.hidden_states(T, H, seed=w.seed + 7, device=device)
    pool = workloads.make_pool(spec, L, seed=w.seed, pinned=False)
    packed = PackedPool(pool, threads=16)
    rt = OffloadRuntime(spec, packed, [cap], 'ferry', Topology.uniform(1, E))
    hist, planner = GateHistoryRef(L, E, 128), PlannerRef(L, E, cap)
    rng = np.random.default_rng(5)
    misses = 0
    for layer in range(L):
        wts, sel = ops.router_topk(logits[layer], k)
        out = rt.execute(layer, x, sel, wts, None)
        w_ref, sel_ref, _ = qwen3_router(logits[layer].cpu(), k)
        assert torch.equal(sel.cpu(), sel_ref) and torch.equal(wts.cpu(), w_ref), layer
        hist.update(layer, frequency_rows(sel_ref.numpy(), E, 128))
        fetches, _ = planner.plan(rt.event - 1, layer, sel_ref.numpy(), hist.scores(layer))
        misses += len(fetches)
        assert np.array_equal(rt.controller.slots[0], planner.slots), layer
        assert np.array_equal(rt.controller.owner, planner.owner), layer
        assert np.array_equal(rt.controller.last, planner.last), layer
        assert np.array_equal(rt.controller.scores, planner.scores), layer
        torch.cuda.synchronize()
        ref_lay = layout_closed_form(sel_ref.numpy(), E, w_ref.view(torch.int16).numpy())
        pick = _edge_tokens(ref_lay['starts'], ref_lay['rows'], rng)
        ref = moe_layer_ref(lambda e: pool[layer * E + e], x.cpu()[pick], sel_ref[pick],
                            w_ref[pick], E, H, I)
        torch.testing.assert_close(out.cpu()[pick].float(), ref.float(), rtol=2e-2, atol=1e-2)
        print(f'layer {layer}: {len(fetches)} misses, {len(pick)} tokens checked', flush=True)
    assert rt.h2d.copies == misses == int(rt.fetches_per_rank.sum()) > 3 * cap
    rt.close()
    packed.close()
