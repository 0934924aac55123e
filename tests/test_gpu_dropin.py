"""The reference runtime's own call order, driven through ferry_amd's drop-in names.

FERRY's ``OffloadRuntime.execute`` (ferry/runtime.py:64-89) makes these calls per MoE layer:
RouteGather.collect -> GateHistory.update / scores -> Controller.plan -> H2DEngine.fetch ->
layer_slots -> device_layout -> Transport.dispatch (pack_dispatch -> exchange ->
unpack_dispatch) -> H2DEngine.wait_host -> execute_experts -> H2DEngine.mark_used ->
Transport.combine (reduce_partials -> exchange -> scatter_returned).  ``ReferenceOrder`` below
makes exactly those calls on ferry_amd's modules, which is what a FERRY runtime does once its
imports point at them.  Over a sequence of layer calls that forces evictions, its outputs and
eviction state must equal ferry_amd's fused runtime bit for bit, and the outputs must match the
oracle.  Each step's bytes and indices are checked against the oracle separately.
"""
import numpy as np
import pytest
import torch

from oracle.experts import execute_experts_ref, moe_layer_ref, reduce_partials_ref
from oracle.layout import layout_closed_form
from oracle.transport import pack_dispatch_ref, packets_closed_form, unpack_dispatch_ref

pytestmark = pytest.mark.gpu


class ReferenceOrder:
    """The steps of ferry/runtime.py:35-89 on ferry_amd's API mirrors (world = 1)."""

    def __init__(self, spec, pool, cap, window=128):
        from ferry_amd.metadata import GateHistory, RouteGather
        from ferry_amd.policy import Controller
        from ferry_amd.quota import Topology
        from ferry_amd.runtime import expert_ops
        from ferry_amd.transport import Transport
        self.spec, self.cap = spec, cap
        self.ops = expert_ops()
        self.cache = torch.empty((cap, spec.expert_elements), dtype=torch.bfloat16, device='cuda')
        self.controller = Controller(spec, [cap], 'ferry', Topology.uniform(1, spec.experts))
        self.gather = RouteGather(spec.topk, spec.experts, window, 'frequency')
        self.transport = Transport(self.ops, spec.topk, spec.experts)
        self.history = GateHistory(spec.layers, spec.experts, window)
        self.h2d = self.ops.H2DEngine(self.cache, pool)
        self.event = 0
        self.last_fetches = None

    def execute(self, layer, hidden, selected, weights, probs_tail):
        from ferry_amd.layout import device_layout
        from ferry_amd.policy import layer_slots
        spec = self.spec
        ids, origins, tail = self.gather.collect(selected, probs_tail)
        self.history.update(layer, tail)
        fetches, destinations, counts = self.controller.plan(
            self.event, layer, ids, origins, self.history.scores(layer))
        mine = fetches[fetches[:, 0] == 0]
        fetch_slots = mine[:, 2].tolist()
        self.h2d.fetch(fetch_slots, mine[:, 1].tolist())
        slot_of = layer_slots(self.controller.slots[0], self.cap, layer, spec.experts)
        layout = device_layout(ids, destinations, selected.shape[0], 0, spec.experts, slot_of)
        received, received_weights = self.transport.dispatch(hidden, selected, weights, layout)
        self.h2d.wait_host(fetch_slots)
        self.last_fetches = mine
        groups = layout['groups']
        slots = [g[3] for g in groups]
        parts = self.ops.execute_experts(self.cache, received, received_weights, slots,
                                         [g[1] for g in groups], [g[2] for g in groups],
                                         spec.hidden, spec.intermediate)
        self.h2d.mark_used(slots)
        self.event += 1
        return self.transport.combine(hidden, parts, layout)


def _routing(T, E, k, pool_size, rng):
    """Each token picks k distinct experts among a per-call subset of ``pool_size`` experts."""
    subset = rng.choice(E, pool_size, replace=False)
    sel = np.stack([rng.choice(subset, k, replace=False) for _ in range(T)]).astype(np.int64)
    logits = rng.standard_normal((T, k)).astype(np.float32)
    w = torch.softmax(torch.from_numpy(logits), -1).to(torch.bfloat16)
    return torch.from_numpy(sel), w


def test_reference_order_matches_fused_runtime(device):
    """Two layers, a 12-slot cache and 10 active experts per call: misses, evictions, slot
    reuse (WAR through mark_used) and calls that take the skinny, mid and tiled kernels."""
    from ferry_amd import workloads
    from ferry_amd.model import ModelSpec
    from ferry_amd.quota import Topology
    from ferry_amd.runtime import OffloadRuntime
    spec = ModelSpec('qwen3_moe', (0, 1), 32, 4, 256, 128)
    E, k, H, I, cap = spec.experts, spec.topk, spec.hidden, spec.intermediate, 12
    pool = workloads.make_pool(spec, spec.layers, seed=5)
    ref = ReferenceOrder(spec, pool, cap)
    fused = OffloadRuntime(spec, pool, [cap], 'ferry', Topology.uniform(1, E))
    rng = np.random.default_rng(11)
    g = torch.Generator().manual_seed(12)
    copies = 0
    for call, T in enumerate([16, 3, 300, 1, 64, 16, 129, 40, 16, 2]):
        layer = call % 2
        print(f'call {call}: layer {layer}, {T} tokens', flush=True)
        sel, w = _routing(T, E, k, 10, rng)
        x = torch.randn((T, H), generator=g).to(torch.bfloat16)
        xd, seld, wd = x.to(device), sel.to(device), w.to(device)
        out_ref = ref.execute(layer, xd, seld, wd, None)
        # after wait_host every fetched slot holds its pool row
        for _, key, slot in ref.last_fetches:
            assert torch.equal(ref.cache[slot].cpu(), pool[key]), (call, key, slot)
        copies += len(ref.last_fetches)
        out_fused = fused.execute(layer, xd, seld, wd, None)
        torch.cuda.synchronize()
        assert torch.equal(out_ref, out_fused), f'call {call}'
        for a, b in ((ref.controller.slots, fused.controller.slots),
                     (ref.controller.owner, fused.controller.owner),
                     (ref.controller.last, fused.controller.last)):
            assert np.array_equal(a, b), f'call {call}'
        oracle = moe_layer_ref(lambda e: pool[layer * E + e], x, sel, w, E, H, I)
        torch.testing.assert_close(out_ref.cpu().float(), oracle.float(), rtol=2e-2, atol=1e-2)
    assert ref.h2d.copies == fused.h2d.copies == copies
    assert copies > cap                 # the sequence evicted
    assert ref.transport.dispatch_bytes == ref.transport.combine_bytes == 0
    ref.h2d.synchronize()
    fused.close()


@pytest.mark.parametrize('T,E,k,H,I', [(40, 16, 4, 256, 128), (300, 64, 6, 512, 256)])
def test_dispatch_combine_steps_bit_exact(device, T, E, k, H, I):
    """device_layout, pack_dispatch, unpack_dispatch, execute_experts, reduce_partials and
    scatter_returned one by one against the oracle: bytes and indices bit-exact, expert rows
    within rel 2e-2 / abs 1e-2, the fp32 sums bit-exact on the same expert rows."""
    from ferry_amd import expert_ops as ops
    from ferry_amd.layout import device_layout
    rng = np.random.default_rng(T)
    g = torch.Generator().manual_seed(T)
    sel, w = _routing(T, E, k, E, rng)
    x = torch.randn((T, H), generator=g).to(torch.bfloat16)
    rows_w = (torch.randn((E, 3 * H * I), generator=g) * 0.02).to(torch.bfloat16)
    slot_of = rng.permutation(E)
    cache = torch.empty_like(rows_w)
    cache[torch.from_numpy(slot_of)] = rows_w
    cache = cache.to(device)

    layout = device_layout(sel.numpy(), np.zeros((T, k), np.int64), T, 0, E, slot_of)
    ref_lay = layout_closed_form(sel.numpy(), E, w.view(torch.int16).numpy())
    assert torch.equal(layout['send_idx'].cpu(), torch.arange(T))
    assert np.array_equal(layout['send_ids'].cpu().numpy(), ref_lay['send_ids'])
    assert layout['send_counts'] == layout['recv_counts'] == [T]
    groups = layout['groups']
    assert [g_[0] for g_ in groups] == [e for e in range(E) if ref_lay['counts'][e]]
    for e, r, c, slot in groups:
        a, b = ref_lay['starts'][e], ref_lay['starts'][e + 1]
        assert np.array_equal(r.cpu().numpy(), ref_lay['rows'][a:b])
        assert np.array_equal(c.cpu().numpy(), ref_lay['cols'][a:b])
        assert slot == slot_of[e]

    payload = ops.pack_dispatch(x.to(device), sel.to(device), w.to(device), layout['send_idx'],
                                layout['send_ids'], E)
    want = pack_dispatch_ref(x, sel, w, torch.arange(T), torch.from_numpy(ref_lay['send_ids']), E)
    assert torch.equal(payload.cpu(), want)
    assert np.array_equal(want.numpy(), packets_closed_form(x, ref_lay['send_ids'], ref_lay['w_sorted']))
    received, rweights = ops.unpack_dispatch(payload, H, k)
    ux, uw = unpack_dispatch_ref(want, H, k)
    assert torch.equal(received.cpu(), ux) and torch.equal(rweights.cpu(), uw)

    parts = ops.execute_experts(cache, received, rweights, [g_[3] for g_ in groups],
                                [g_[1] for g_ in groups], [g_[2] for g_ in groups], H, I)
    rows = [torch.from_numpy(ref_lay['rows'][ref_lay['starts'][e]:ref_lay['starts'][e + 1]])
            for e, _, _, _ in groups]
    cols = [torch.from_numpy(ref_lay['cols'][ref_lay['starts'][e]:ref_lay['starts'][e + 1]])
            for e, _, _, _ in groups]
    want_parts = execute_experts_ref([rows_w[e] for e, _, _, _ in groups], ux, uw, rows, cols, H, I)
    for got, exp in zip(parts, want_parts):
        torch.testing.assert_close(got.cpu().float(), exp.float(), rtol=2e-2, atol=1e-2)

    partial = ops.reduce_partials(parts, [g_[1] for g_ in groups], T, H, x.to(device))
    assert torch.equal(partial.cpu(), reduce_partials_ref([p.cpu() for p in parts], rows, T, H))
    back = ops.scatter_returned(partial, layout['send_idx'], T)
    assert torch.equal(back, partial)   # world = 1: an fp32 round trip of every row
    oracle = moe_layer_ref(lambda e: rows_w[e], x, sel, w, E, H, I)
    torch.testing.assert_close(back.cpu().float(), oracle.float(), rtol=2e-2, atol=1e-2)
