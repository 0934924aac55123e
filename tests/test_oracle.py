"""CPU tier: the oracle pinned against libraries, closed forms, hand-derived answers and the
committed golden fixtures (no GPU)."""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.experts import (execute_experts_ref, moe_fp64, moe_layer_ref, reduce_partials_ref,
                            silu_mul_ref)
from oracle.history import GateHistoryRef, closed_form_scores, frequency_rows
from oracle.layout import layout_closed_form, layout_loops
from oracle.native import topk as emulated_topk
from oracle.policy import PlannerRef, plan_layer_sorted
from oracle.router import deepseek_router, qwen3_router

GOLDEN = Path(__file__).resolve().parent / 'golden'


# ---------------------------------------------------------------------------------------------
# top-k restatement vs torch.topk on the CPU (the library the reference router calls)
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize('n,k', [(128, 8), (64, 6), (128, 1), (16, 3), (300, 4), (4096, 8), (64, 32),
                                 (128, 40), (8, 8), (256, 2)])
@pytest.mark.parametrize('sorted_', [True, False])
@pytest.mark.parametrize('quant', [None, 'bf16', 'coarse'])
def test_topk_restatement_matches_torch(n, k, sorted_, quant):
    rng = np.random.default_rng(n * 7 + k)
    x = rng.standard_normal((400, n)).astype(np.float32)
    if quant == 'bf16':
        x = torch.from_numpy(x).bfloat16().float().numpy()
    elif quant == 'coarse':
        x = np.round(x * 4) / 4
    p = torch.softmax(torch.from_numpy(x), -1)
    for largest in (True, False):
        tv, ti = torch.topk(p, k, largest=largest, sorted=sorted_)
        ov, oi = emulated_topk(p.numpy(), k, largest, sorted_)
        assert np.array_equal(ti.numpy(), oi)
        assert np.array_equal(tv.numpy(), ov)


def test_topk_nan_rows_match_torch():
    x = torch.randn((64, 128))
    x[::3, 5] = float('nan')
    x[1::3] = float('nan')
    for sorted_ in (True, False):
        tv, ti = torch.topk(x, 8, sorted=sorted_)
        _, oi = emulated_topk(x.numpy(), 8, True, sorted_)
        assert np.array_equal(ti.numpy(), oi)


def test_router_oracle_against_golden():
    d = np.load(GOLDEN / 'topk_qwen3_bf16.npz')
    logits = torch.from_numpy(d['logits']).view(torch.bfloat16)
    w, idx, probs = qwen3_router(logits, int(d['k']))
    assert np.array_equal(idx.numpy(), d['idx'])
    assert np.array_equal(w.view(torch.int16).numpy(), d['w'])
    _, oi = emulated_topk(probs.numpy(), int(d['k']), True, True)
    assert np.array_equal(oi, d['idx'])
    d = np.load(GOLDEN / 'topk_deepseek_fp32_unsorted.npz')
    w, idx, probs = deepseek_router(torch.from_numpy(d['logits']), int(d['k']))
    assert np.array_equal(idx.numpy(), d['idx'])
    _, oi = emulated_topk(probs.numpy(), int(d['k']), True, False)
    assert np.array_equal(oi, d['idx'])


def test_router_renorm_closed_form():
    logits = torch.randn((100, 128)).bfloat16()
    w, idx, probs = qwen3_router(logits, 8)
    top = torch.gather(probs, 1, idx)
    torch.testing.assert_close(w.float(), (top / top.sum(-1, keepdim=True)), rtol=2 ** -8, atol=0)
    # selection on logits = selection on probabilities (softmax is increasing)
    assert torch.equal(torch.topk(logits.float(), 8).indices.sort(1).values, idx.sort(1).values)


# ---------------------------------------------------------------------------------------------
# history
# ---------------------------------------------------------------------------------------------

def test_fp32_division_equals_float64_mean_cast():
    """score = float32(c / n) in fp32 equals the reference's float64 mean cast to float32."""
    for n in range(1, 129):
        c = np.arange(0, n + 1)
        a = (c.astype(np.float64) / n).astype(np.float32)
        b = c.astype(np.float32) / np.float32(n)
        assert np.array_equal(a, b), n


def test_history_ring_vs_closed_form():
    rng = np.random.default_rng(3)
    L, E, k, W = 3, 40, 5, 128
    h = GateHistoryRef(L, E, W)
    seen = [[] for _ in range(L)]
    for step in range(80):
        layer = step % L
        T = int(rng.choice([1, 2, 16, 64, 127, 128, 129, 300]))
        sel = np.stack([rng.choice(E, k, replace=False) for _ in range(T)])
        h.update(layer, frequency_rows(sel, E, W))
        seen[layer].extend(list(sel))
        assert np.array_equal(h.scores(layer), closed_form_scores(seen[layer], E, W))


def test_history_golden():
    d = np.load(GOLDEN / 'history.npz')
    L, E, k, W = int(d['layers']), int(d['experts']), int(d['topk']), int(d['window'])
    h = GateHistoryRef(L, E, W)
    off = 0
    for i, T in enumerate(d['sizes']):
        sel = d['selected'][off:off + T]
        off += T
        h.update(i % L, frequency_rows(sel, E, W))
        assert np.array_equal(h.scores(i % L), d['scores'][i])


def test_history_empty_scores_zero():
    h = GateHistoryRef(1, 8, 128)
    assert np.array_equal(h.scores(0), np.zeros(8, np.float32))


# ---------------------------------------------------------------------------------------------
# planner
# ---------------------------------------------------------------------------------------------

def test_planner_known_answer():
    """Hand-derived trace (E = 4, two layers, three slots)."""
    p = PlannerRef(2, 4, 3)
    f, dest = p.plan(0, 0, np.array([[0, 1]]), np.array([.5, .5, 0, 0], np.float32))
    assert f.tolist() == [[0, 0, 0], [0, 1, 1]] and dest.tolist() == [[0, 0]]
    # first empty slot for key 6; then the min (score, last, key) over keys 0 and 1 -> key 0
    f, _ = p.plan(1, 1, np.array([[2, 3]]), np.array([0, 0, .3, .3], np.float32))
    assert f.tolist() == [[0, 6, 2], [0, 7, 0]]
    # key 1 is protected (active in layer 0); keys 6 and 7 tie on (score, last) -> key 6
    f, _ = p.plan(2, 0, np.array([[1, 2]]), np.array([0, .25, .75, 0], np.float32))
    assert f.tolist() == [[0, 2, 2]]
    assert p.slots.tolist() == [7, 1, 2]
    assert p.last[[1, 2]].tolist() == [3, 3] and p.last[7] == 2
    # LRU: equal scores, older last use is evicted (key 7 last=2 vs key 1 last=3)
    f, _ = p.plan(3, 1, np.array([[0]]), np.array([0, 0, 0, 0], np.float32))
    assert f.tolist() == [[0, 4, 0]]   # key 7 (score 0 now, last 2) < key 2 (score .75)


def test_planner_scores_of_other_layers_are_stale():
    """The eviction key uses the score last planned for the victim's own layer."""
    p = PlannerRef(2, 2, 2)
    p.plan(0, 0, np.array([[0]]), np.array([.9, 0], np.float32))
    p.plan(1, 1, np.array([[0]]), np.array([.1, 0], np.float32))
    # layer-0 key 0 keeps score .9, layer-1 key 2 has .1 -> evict key 2
    f, _ = p.plan(2, 0, np.array([[1]]), np.array([.9, 0], np.float32))
    assert f.tolist() == [[0, 1, 1]]


def test_planner_overflow_asserts():
    p = PlannerRef(1, 8, 2)
    with pytest.raises(AssertionError):
        p.plan(0, 0, np.array([[0, 1, 2]]), np.zeros(8, np.float32))
    p = PlannerRef(1, 8, 3)
    p.plan(0, 0, np.array([[0, 1, 2]]), np.zeros(8, np.float32))
    with pytest.raises(AssertionError):   # all slots hold protected experts
        p.plan(1, 0, np.array([[0, 1, 2, 3]]), np.zeros(8, np.float32))


def test_planner_c_vs_sorted_formulation_random():
    rng = np.random.default_rng(0)
    for trial in range(20):
        L, E = int(rng.integers(1, 4)), int(rng.integers(2, 20))
        cap = int(rng.integers(1, 2 * E))
        ref = PlannerRef(L, E, cap)
        st = dict(slots=np.full(cap, -1, np.int64), owner=np.full(L * E, -1, np.int64),
                  last=np.zeros(L * E, np.int64), scores=np.zeros((L, E), np.float32))
        for ev in range(60):
            layer = int(rng.integers(0, L))
            k = int(rng.integers(1, min(E, 4) + 1))
            T = int(rng.integers(1, 5))
            sel = np.stack([rng.choice(E, k, replace=False) for _ in range(T)])
            gs = (rng.integers(0, 3, E) / 2).astype(np.float32)
            try:
                f1, dest = ref.plan(ev, layer, sel, gs)
            except AssertionError:
                f1 = None
            try:
                f2 = plan_layer_sorted(st, ev, layer, sel, gs)
            except AssertionError:
                f2 = None
            assert (f1 is None) == (f2 is None)
            if f1 is None:
                break
            assert np.array_equal(f1, f2)
            # invariants: misses ascending, every active expert resident, no duplicate keys
            assert list(f1[:, 1]) == sorted(f1[:, 1])
            live = ref.slots[ref.slots >= 0]
            assert len(set(live.tolist())) == len(live)
            for e in np.unique(sel):
                assert layer * E + e in live
            assert np.array_equal(dest, np.zeros_like(dest))


def test_planner_golden_trace():
    d = np.load(GOLDEN / 'planner.npz')
    L, E, cap = int(d['layers']), int(d['experts']), int(d['cap'])
    p = PlannerRef(L, E, cap)
    off = foff = 0
    for ev, T in enumerate(d['sizes']):
        sel = d['selected'][off:off + T]
        off += T
        f, _ = p.plan(ev, ev % L, sel, d['gate_scores'][ev])
        n = int(d['nfetch'][ev])
        assert np.array_equal(f, d['fetches'][foff:foff + n])
        foff += n
    assert np.array_equal(p.slots, d['final_slots'])
    assert np.array_equal(p.last, d['final_last'])


# ---------------------------------------------------------------------------------------------
# layout
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize('T,E,k', [(1, 4, 1), (7, 8, 8), (100, 64, 6), (513, 128, 8)])
def test_layout_closed_form_vs_loops(T, E, k):
    rng = np.random.default_rng(T)
    sel = np.stack([rng.choice(E, k, replace=False) for _ in range(T)])
    a, b = layout_closed_form(sel, E), layout_loops(sel, E)
    for key in ('send_ids', 'starts', 'rows', 'cols'):
        assert np.array_equal(a[key], b[key])
    # pair_pos is the inverse permutation
    assert np.array_equal(a['rows'][a['pair_pos']], np.repeat(np.arange(T), k))


def test_layout_golden():
    d = np.load(GOLDEN / 'layout.npz')
    a = layout_closed_form(d['selected'], int(d['experts']))
    for key in ('send_ids', 'starts', 'rows', 'cols', 'pair_pos'):
        assert np.array_equal(a[key], d[key])


# ---------------------------------------------------------------------------------------------
# expert FFN and combine
# ---------------------------------------------------------------------------------------------

def test_silu_mul_closed_form():
    g = torch.tensor([0.0, 1.0, -1.0, 3.5]).bfloat16()
    u = torch.tensor([2.0, 1.0, 1.0, -2.0]).bfloat16()
    want = torch.tensor([0.0, 1 / (1 + np.exp(-1)), -1 / (1 + np.exp(1)), -7.0 / (1 + np.exp(-3.5))])
    torch.testing.assert_close(silu_mul_ref(g, u).float(), want.float(), rtol=2 ** -8, atol=0)


def test_moe_oracle_vs_fp64():
    g = torch.Generator().manual_seed(1)
    T, E, k, H, I = 40, 8, 2, 64, 32
    rows_w = (torch.randn((E, 3 * H * I), generator=g) * 0.05).bfloat16()
    x = torch.randn((T, H), generator=g).bfloat16()
    logits = torch.randn((T, E), generator=g).bfloat16()
    w, sel, _ = qwen3_router(logits, k)
    out = moe_layer_ref(lambda e: rows_w[e], x, sel, w, E, H, I).float()
    exact = moe_fp64(lambda e: rows_w[e], x, sel, w, H, I).float()
    torch.testing.assert_close(out, exact, rtol=2e-2, atol=1e-2)


def test_shared_mlp_oracle_pinned():
    """HF DeepseekV2MLP restatement: a diagonal special case reduces it to the elementwise
    silu(2x) * (x / 2) (torch.nn.functional.silu); random weights agree with the fp64 SwiGLU."""
    from oracle.experts import shared_mlp_fp64, shared_mlp_ref
    H = I = 64
    eye = torch.eye(H)
    row = torch.cat([(2 * eye).reshape(-1), (0.5 * eye).reshape(-1), eye.reshape(-1)]).bfloat16()
    g = torch.Generator().manual_seed(3)
    x = torch.randn((10, H), generator=g).bfloat16()
    want = (torch.nn.functional.silu(2 * x) * (0.5 * x)).bfloat16()
    assert torch.equal(shared_mlp_ref(row, x, H, I), want)
    H, I = 128, 96
    row = (torch.randn(3 * H * I, generator=g) * 0.05).bfloat16()
    x = torch.randn((20, H), generator=g).bfloat16()
    torch.testing.assert_close(shared_mlp_ref(row, x, H, I).float(), shared_mlp_fp64(row, x, H, I).float(),
                               rtol=2e-2, atol=1e-2)


def test_reduce_partials_is_ascending_fp32_sum():
    g = torch.Generator().manual_seed(2)
    parts = [torch.randn((3, 8), generator=g).bfloat16() for _ in range(3)]
    rows = [torch.tensor([0, 2, 4]), torch.tensor([2, 3, 4]), torch.tensor([4, 0, 1])]
    got = reduce_partials_ref(parts, rows, 5, 8)
    acc = torch.zeros((5, 8))
    for p, r in zip(parts, rows):
        for i, t in enumerate(r.tolist()):
            acc[t] += p[i].float()
    assert torch.equal(got, acc.bfloat16())


def test_execute_experts_ref_weights_rows_cols():
    g = torch.Generator().manual_seed(3)
    H, I = 32, 16
    row = (torch.randn(3 * H * I, generator=g) * 0.1).bfloat16()
    x = torch.randn((4, H), generator=g).bfloat16()
    rw = torch.tensor([[0.5, 0.25], [1.0, 2.0], [0.0, 1.0], [1.0, 1.0]]).bfloat16()
    r, c = torch.tensor([1, 3]), torch.tensor([1, 0])
    out = execute_experts_ref([row], x, rw, [r], [c], H, I)[0]
    unit = execute_experts_ref([row], x, torch.ones_like(rw), [r], [c], H, I)[0]
    torch.testing.assert_close(out.float(), (unit.float() * torch.tensor([[2.0], [1.0]])).bfloat16().float())


def test_pack_dispatch_oracle_matches_closed_form():
    """The restated packet bytes (dense scatter / gather of expert_ops.cpp:88-104) equal the
    world-1 closed form [hidden | weights in sorted-ID order | sorted IDs] for distinct IDs, and
    unpacking returns the hidden rows and sorted weights; repeated IDs add their weights and a
    -1 packet ID gives weight 0 and the ID byte 255."""
    import torch
    from oracle.layout import layout_closed_form
    from oracle.transport import pack_dispatch_ref, packets_closed_form, unpack_dispatch_ref
    g = torch.Generator().manual_seed(0)
    for T, E, k, H in ((1, 8, 2, 16), (37, 64, 6, 64), (200, 128, 8, 32)):
        sel = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
        w = torch.softmax(torch.randn((T, k), generator=g), -1).to(torch.bfloat16)
        x = torch.randn((T, H), generator=g).to(torch.bfloat16)
        lay = layout_closed_form(sel.numpy(), E, w.view(torch.int16).numpy())
        send_ids = torch.from_numpy(lay['send_ids'])
        got = pack_dispatch_ref(x, sel, w, torch.arange(T), send_ids, E)
        assert got.dtype == torch.uint8 and got.shape == (T, 2 * H + 3 * k)
        assert np.array_equal(got.numpy(), packets_closed_form(x, lay['send_ids'], lay['w_sorted']))
        ux, uw = unpack_dispatch_ref(got, H, k)
        assert torch.equal(ux, x)
        assert np.array_equal(uw.view(torch.int16).numpy(), lay['w_sorted'])
    # repeated IDs add (fp32, then bf16); an invalid packet ID reads weight 0, ID byte 255
    x = torch.zeros((1, 4), dtype=torch.bfloat16)
    sel = torch.tensor([[2, 2, 5]])
    w = torch.tensor([[0.25, 0.5, 0.125]]).to(torch.bfloat16)
    p = pack_dispatch_ref(x, sel, w, torch.tensor([0]), torch.tensor([[2, 5, -1]]), 8)
    _, pw = unpack_dispatch_ref(p, 4, 3)
    assert pw.float().tolist() == [[0.75, 0.125, 0.0]]
    assert p[0, -3:].tolist() == [2, 5, 255]


# ---------------------------------------------------------------------------------------------
# torch's CPU softmax and renormalising sum, restated bit for bit (oracle/softmax.c)
# ---------------------------------------------------------------------------------------------

def _rows(E, rows, seed, dtype, scale=3.0):
    import torch
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((rows, E), generator=g) * scale
    if rows > 8:
        x[0, 0] = float('-inf')                     # exp underflows to 0
        x[1, :] = x[1, 0]                           # all equal
        x[2, E // 2] = 200.0                        # the others underflow
        x[3, -1] = -150.0
    return x.to(dtype)


@pytest.mark.parametrize('E', [1, 2, 7, 8, 15, 16, 17, 20, 64, 100, 128, 200, 256])
def test_softmax_restatement_bit_exact_vs_torch(E):
    """The restated softmax (SLEEF expf_u10, reduce_all's 16-lane sum order, reciprocal
    multiply) equals torch.softmax on the CPU bit for bit, for fp32 and bf16 logits."""
    import torch
    from oracle.native import softmax
    for dtype in (torch.float32, torch.bfloat16):
        for scale in (0.5, 3.0, 30.0):
            x = _rows(E, 600, seed=E + int(scale * 10), dtype=dtype, scale=scale)
            ref = torch.softmax(x, -1, dtype=torch.float32).numpy()
            got = softmax(x.float().numpy())
            assert np.array_equal(got.view(np.int32), ref.view(np.int32)), (E, dtype, scale)


def test_softmax_restatement_special_rows():
    """NaN and +inf logits make the whole row NaN; -inf logits give probability 0."""
    import torch
    from oracle.native import softmax
    x = torch.tensor([[1.0, float('nan'), 0.0, 2.0], [float('inf'), 0.0, 1.0, 1.0],
                      [float('-inf'), 0.0, 1.0, float('-inf')], [float('-inf')] * 4])
    ref = torch.softmax(x, -1).numpy()
    got = softmax(x.numpy())
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(got[ok].view(np.int32), ref[ok].view(np.int32))


def test_expf_restatement_within_one_ulp():
    """The restated SLEEF expf is within 1 ulp of the correctly rounded exp on a dense sweep of
    the softmax range [-104, 0] (its published error bound), and exact at the end points."""
    from oracle.native import lib
    d = np.linspace(-104.0, 0.0, 200001).astype(np.float32)
    got = np.array([lib().oracle_expf(float(v)) for v in d[::7]], np.float32)
    exact = np.exp(d[::7].astype(np.float64)).astype(np.float32)
    ulp = np.abs(got.view(np.int32).astype(np.int64) - exact.view(np.int32).astype(np.int64))
    assert ulp.max() <= 1
    assert lib().oracle_expf(0.0) == 1.0 and lib().oracle_expf(-105.0) == 0.0


@pytest.mark.parametrize('k', list(range(1, 33)))
def test_weight_sum_restatement_bit_exact_vs_torch(k):
    """The restated renormalising sum equals torch's CPU w.sum(-1) for every k <= 32, on top-k
    values in both the sorted and the unsorted output order."""
    import torch
    from oracle.native import weight_sum
    g = torch.Generator().manual_seed(k)
    p = torch.softmax(torch.randn((3000, 256), generator=g) * 2, -1)
    for srt in (True, False):
        w, _ = torch.topk(p, k, dim=-1, sorted=srt)
        ref = w.sum(-1).numpy()
        got = weight_sum(w.numpy())
        assert np.array_equal(got.view(np.int32), ref.view(np.int32)), (k, srt)


def fp32_near_tie_rows(T, E, k, seed):
    """fp32 logits with a pair of distinct values one ulp apart straddling the top-k boundary
    (positions k - 1 and k of the descending order), the case where torch's softmax can round
    two different logits to the same probability."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, E)).astype(np.float32)
    order = np.argsort(-x, axis=1, kind='stable')
    for t in range(T):
        a, b = order[t, k - 1], order[t, k]
        x[t, b] = np.nextafter(x[t, a], np.float32(-np.inf))
    return x


def test_fp32_near_ties_collapse_in_torch_and_restatement():
    """Distinct fp32 logits one ulp apart at the k boundary: torch's softmax maps many such
    pairs to equal probabilities (then torch.topk breaks the tie by its algorithm, not by the
    logit order), and the restated softmax reproduces exactly which pairs collapse."""
    import torch
    from oracle.native import softmax, topk
    for E, k in ((64, 6), (128, 8)):
        x = fp32_near_tie_rows(4000, E, k, seed=E)
        p_ref = torch.softmax(torch.from_numpy(x), -1).numpy()
        p = softmax(x)
        assert np.array_equal(p.view(np.int32), p_ref.view(np.int32))
        order = np.argsort(-x, axis=1, kind='stable')
        a = np.take_along_axis(p, order[:, k - 1:k], 1)[:, 0]
        b = np.take_along_axis(p, order[:, k:k + 1], 1)[:, 0]
        collapsed = a == b
        assert collapsed.sum() > 100, collapsed.sum()
        # on those rows the CPU top-k set is not the logit order's set in some rows
        _, idx = torch.topk(torch.from_numpy(p_ref), k, dim=-1)
        by_logit = np.sort(order[:, :k], axis=1)
        differs = (np.sort(idx.numpy(), axis=1) != by_logit).any(1)
        assert differs.sum() > 0 and not differs[~collapsed].any()
        # and the topk restatement follows torch on the collapsed probabilities
        _, oi = topk(p_ref, k, sorted=True)
        assert np.array_equal(oi, idx.numpy())


def test_router_oracle_equals_torch_op_sequence():
    """The router oracle (restated softmax and sum) equals the reference's torch op sequence
    run on this CPU: softmax(fp32), topk, w / w.sum(-1), bf16 -- indices, weights and
    probabilities bit for bit."""
    import torch
    from oracle.router import deepseek_router, qwen3_router
    g = torch.Generator().manual_seed(21)
    for E, k, dtype in ((128, 8, torch.bfloat16), (64, 6, torch.float32), (256, 32, torch.bfloat16),
                        (16, 5, torch.float32)):
        x = (torch.randn((2000, E), generator=g) * 2).to(dtype)
        w, sel, p = qwen3_router(x, k)
        p_t = torch.softmax(x, -1, dtype=torch.float32)
        w_t, sel_t = torch.topk(p_t, k, dim=-1)
        w_t = (w_t / w_t.sum(-1, keepdim=True)).to(torch.bfloat16)
        assert torch.equal(p, p_t) and torch.equal(sel, sel_t) and torch.equal(w, w_t)
        w2, sel2, _ = deepseek_router(x.float(), k)
        w2_t, sel2_t = torch.topk(torch.softmax(x.float(), -1), k, dim=-1, sorted=False)
        assert torch.equal(sel2, sel2_t) and torch.equal(w2, w2_t.to(torch.bfloat16))
