"""Parity of each HIP kernel (through the C ABI) with the CPU oracle."""
import numpy as np
import pytest
import torch

from oracle.experts import execute_experts_ref, moe_layer_ref, reduce_partials_ref
from oracle.history import GateHistoryRef, frequency_rows
from oracle.layout import layout_closed_form
from oracle.router import deepseek_router, qwen3_router

pytestmark = pytest.mark.gpu


def _ops():
    from ferry_amd import expert_ops
    return expert_ops


def _logits(T, E, dtype, seed, ties=False, zipf=0.0):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn((T, E), generator=g)
    if zipf:
        r = torch.arange(1, E + 1, dtype=torch.float64)
        p = r ** -zipf
        z = z + torch.log(p / p.sum()).float()[torch.randperm(E, generator=g)]
    if ties:
        z = torch.round(z * 3) / 3   # few distinct values per row: many ties at every position
    return z.to(dtype)


# ---------------------------------------------------------------------------------------------
# router
# ---------------------------------------------------------------------------------------------

# (128, 32), (64, 20), (256, 32): k - 1 > 16, torch's std::sort of the first k - 1 entries
# leaves the insertion-sort regime (the serial restatement); (200, 3): k * 64 <= n, the
# partial_sort regime
@pytest.mark.parametrize('E,k', [(128, 8), (64, 6), (16, 4), (256, 8), (32, 1), (8, 8), (200, 3),
                                 (128, 32), (64, 20), (256, 32)])
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
@pytest.mark.parametrize('ties', [False, True])
def test_router_sorted_matches_torch_cpu_topk(device, E, k, dtype, ties):
    ops = _ops()
    T = 777
    logits = _logits(T, E, dtype, seed=E * 31 + k, ties=ties)
    w_ref, sel_ref, p_ref = qwen3_router(logits, k)
    counter = torch.zeros(1, dtype=torch.int32, device=device)
    w, sel, probs = ops.router_topk(logits.to(device), k, renorm=True, return_probs=True,
                                    tie_counter=counter)
    torch.cuda.synchronize()
    assert torch.equal(sel.cpu(), sel_ref), 'routing indices differ from torch.topk on the CPU'
    assert torch.equal(probs.cpu(), p_ref), 'probabilities differ from torch.softmax on the CPU'
    assert torch.equal(w.cpu(), w_ref), 'renormalised weights differ from the CPU op sequence'
    if ties:
        assert int(counter.item()) > 0, 'the exact tie path was not exercised'


@pytest.mark.parametrize('E,k', [(64, 6), (128, 8), (16, 5), (128, 32), (256, 3)])
@pytest.mark.parametrize('ties', [False, True])
def test_router_unsorted_deepseek(device, E, k, ties):
    ops = _ops()
    T = 500
    logits = _logits(T, E, torch.float32, seed=7 + E, ties=ties)
    w_ref, sel_ref, _ = deepseek_router(logits, k, 1.0)
    w, sel = ops.router_topk(logits.to(device), k, renorm=False, scale=1.0, sorted=False)
    torch.cuda.synchronize()
    assert torch.equal(sel.cpu(), sel_ref)
    assert torch.equal(w.cpu(), w_ref)


@pytest.mark.parametrize('E,k,sorted_', [(64, 6, False), (128, 8, True), (128, 8, False),
                                         (64, 6, True), (256, 3, True)])
def test_router_fp32_near_ties(device, E, k, sorted_):
    """fp32 logits with distinct values one ulp apart at the top-k boundary: torch's softmax
    rounds many such pairs to one probability and torch.topk then breaks the tie by its own
    algorithm, so ranking by logit would pick another set.  The kernel ranks its probabilities,
    which equal torch's bit for bit, and matches torch's indices and weights."""
    from test_oracle import fp32_near_tie_rows
    ops = _ops()
    x = torch.from_numpy(fp32_near_tie_rows(3000, E, k, seed=E + k))
    w_ref, sel_ref, p_ref = (qwen3_router(x, k) if sorted_ else deepseek_router(x, k))
    w, sel, probs = ops.router_topk(x.to(device), k, renorm=sorted_, sorted=sorted_,
                                    return_probs=True)
    torch.cuda.synchronize()
    assert torch.equal(probs.cpu(), p_ref)
    assert torch.equal(sel.cpu(), sel_ref)
    assert torch.equal(w.cpu(), w_ref)
    # the rows exercise the hole: some pairs collapsed and changed torch's selected set
    order = np.argsort(-x.numpy(), axis=1, kind='stable')
    by_logit = np.sort(order[:, :k], axis=1)
    assert (np.sort(sel_ref.numpy(), axis=1) != by_logit).any(1).sum() > 0


def test_router_full_size_qwen3_prefill(device):
    """8192 tokens x 128 experts, Zipf(1.1)-skewed bf16 logits (the prefill shape)."""
    ops = _ops()
    logits = _logits(8192, 128, torch.bfloat16, seed=1, zipf=1.1)
    w_ref, sel_ref, _ = qwen3_router(logits, 8)
    w, sel = ops.router_topk(logits.to(device), 8)
    torch.cuda.synchronize()
    assert torch.equal(sel.cpu(), sel_ref)
    assert torch.equal(w.cpu(), w_ref)


def test_empty_and_single_token_calls(device):
    """T = 0 through layout / combine / expert FFN, and a list holding experts with no rows."""
    ops = _ops()
    E, k, H, I = 16, 4, 256, 128
    sel = torch.empty((0, k), dtype=torch.int64, device=device)
    w = torch.empty((0, k), dtype=torch.bfloat16, device=device)
    lay = ops.layout(sel, w, E)
    assert lay.starts.cpu().tolist() == [0] * (E + 1)
    out = ops.combine(torch.empty((0, H), dtype=torch.bfloat16, device=device), 0, k, H)
    assert out.shape == (0, H)
    rows_w = _pool(E, H, I, seed=21)
    cache = rows_w.to(device)
    act = torch.empty((0, I), dtype=torch.bfloat16, device=device)
    part = torch.empty((0, H), dtype=torch.bfloat16, device=device)
    ops.expert_ffn(cache, torch.empty((0, H), dtype=torch.bfloat16, device=device), lay.w_sorted,
                   lay.starts, lay.rows, lay.cols, np.arange(E), np.arange(E, dtype=np.int32), H, I,
                   act, part)
    # one token; the expert list also names experts the token did not select (no rows)
    g = torch.Generator().manual_seed(22)
    x = torch.randn((1, H), generator=g).to(torch.bfloat16)
    sel = torch.tensor([[3, 11, 0, 7]])
    wts = torch.softmax(torch.randn((1, k), generator=g), -1).to(torch.bfloat16)
    lay = ops.layout(sel.to(device), wts.to(device), E)
    act = torch.empty((k, I), dtype=torch.bfloat16, device=device)
    part = torch.empty((k, H), dtype=torch.bfloat16, device=device)
    ops.expert_ffn(cache, x.to(device), lay.w_sorted, lay.starts, lay.rows, lay.cols, np.arange(E),
                   np.arange(E, dtype=np.int32), H, I, act, part)
    got = ops.combine(part, 1, k, H).cpu().float()
    ref = moe_layer_ref(lambda e: rows_w[e], x, sel, wts, E, H, I).float()
    torch.testing.assert_close(got, ref, rtol=2e-2, atol=1e-2)


def test_router_empty_and_errors(device):
    ops = _ops()
    w, sel = ops.router_topk(torch.empty((0, 64), dtype=torch.bfloat16, device=device), 6)
    assert w.shape == (0, 6) and sel.shape == (0, 6)
    with pytest.raises(RuntimeError):
        ops.router_topk(torch.zeros((4, 300), dtype=torch.bfloat16, device=device), 8)
    with pytest.raises(RuntimeError):
        ops.router_topk(torch.zeros((4, 16), dtype=torch.bfloat16, device=device), 17)


# ---------------------------------------------------------------------------------------------
# layout
# ---------------------------------------------------------------------------------------------

def _selected(T, E, k, seed, zipf=0.0):
    logits = _logits(T, E, torch.float32, seed, zipf=zipf)
    return torch.topk(logits, k, dim=-1).indices.contiguous()


@pytest.mark.parametrize('T,E,k', [(1, 8, 2), (16, 128, 8), (1000, 64, 6), (1024, 128, 8),
                                   (1025, 128, 8), (4097, 512, 16), (65536, 64, 6), (8192, 128, 8)])
def test_layout_bit_exact(device, T, E, k):
    ops = _ops()
    sel = _selected(T, E, k, seed=T + E, zipf=1.1)
    w = torch.randn((T, k)).to(torch.bfloat16)
    ref = layout_closed_form(sel.numpy(), E, w.view(torch.int16).numpy())
    lay = ops.layout(sel.to(device), w.to(device), E)
    torch.cuda.synchronize()
    assert np.array_equal(lay.send_ids.cpu().numpy(), ref['send_ids'])
    assert np.array_equal(lay.w_sorted.cpu().view(torch.int16).numpy(), ref['w_sorted'])
    assert np.array_equal(lay.starts.cpu().numpy(), ref['starts'])
    assert np.array_equal(lay.rows.cpu().numpy(), ref['rows'])
    assert np.array_equal(lay.cols.cpu().numpy(), ref['cols'])
    assert np.array_equal(lay.pair_pos.cpu().numpy(), ref['pair_pos'])


@pytest.mark.parametrize('T', [5, 3000])   # one-block and three-kernel layouts
def test_layout_flags_invalid_ids(device, T):
    """Tokens with an out-of-range or a repeated expert ID are counted by the kernel and
    ``layout(check=True)`` raises; valid routing passes the check with a zero count."""
    ops = _ops()
    E, k = 32, 4
    sel = _selected(T, E, k, seed=T)
    lay = ops.layout(sel.to(device), None, E, check=True)
    assert ops.layout_errors(lay) == 0
    for bad, count in (((0, 1), 40), ((T - 1, 2), -1), ((1, 0), 1)):
        s = sel.clone()
        (t, j), v = bad, count
        s[t, j] = v if v != 1 else s[t, 3]          # 40 / -1: out of range; else a repeat
        with pytest.raises(RuntimeError, match='out of'):
            ops.layout(s.to(device), None, E, check=True)
        assert ops.layout_errors(ops.layout(s.to(device), None, E)) == 1


def test_runtime_rejects_invalid_ids(device):
    """OffloadRuntime.execute raises RuntimeError on an out-of-range or repeated ID: the host
    planner validates the IDs it reads back for planning, before any expert is computed."""
    from ferry_amd.model import ModelSpec
    from ferry_amd.quota import Topology
    from ferry_amd.runtime import OffloadRuntime
    from ferry_amd import workloads
    spec = ModelSpec('qwen3_moe', (0,), 16, 4, 256, 128)
    pool = workloads.make_pool(spec, 1, seed=0)
    rt = OffloadRuntime(spec, pool, [16], 'ferry', Topology.uniform(1, 16))
    x = torch.randn((3, 256)).to(torch.bfloat16).to(device)
    w = torch.full((3, 4), 0.25, dtype=torch.bfloat16, device=device)
    good = torch.tensor([[0, 1, 2, 3], [4, 5, 6, 7], [1, 3, 5, 7]], device=device)
    rt.execute(0, x, good, w, None)
    for bad in ([[0, 1, 2, 16], [4, 5, 6, 7], [1, 3, 5, 7]],
                [[0, 1, 2, 3], [4, 5, 6, 4], [1, 3, 5, 7]]):
        with pytest.raises(RuntimeError, match='out of range|repeated'):
            rt.execute(0, x, torch.tensor(bad, device=device), w, None)
    out = rt.execute(0, x, good, w, None)   # the runtime still works afterwards
    torch.cuda.synchronize()
    assert out.shape == (3, 256)
    rt.close()


# ---------------------------------------------------------------------------------------------
# device history
# ---------------------------------------------------------------------------------------------

def test_device_history_matches_gate_history(device):
    from ferry_amd.metadata import DeviceGateHistory
    L, E, k, W = 3, 128, 8, 128
    hist = DeviceGateHistory(L, E, k, W, device)
    ref = GateHistoryRef(L, E, W)
    rng = np.random.default_rng(0)
    scores = torch.empty(E, dtype=torch.float32, device=device)
    ids = torch.empty(4096 * k, dtype=torch.uint8, device=device)
    for step, T in enumerate([1, 16, 64, 200, 3, 127, 128, 129, 16, 16, 500, 5, 1, 64]):
        layer = step % L
        sel = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int64)
        hist.update(layer, torch.from_numpy(sel).to(device), scores, ids[:T * k])
        ref.update(layer, frequency_rows(sel, E, W))
        torch.cuda.synchronize()
        assert np.array_equal(scores.cpu().numpy(), ref.scores(layer)), f'step {step}'
        assert np.array_equal(ids[:T * k].cpu().numpy(), sel.reshape(-1).astype(np.uint8))


@pytest.mark.parametrize('T', [16, 1000])
def test_history_ready_words_and_host_wait(device, T):
    """The history kernel's ready words (one per workgroup, after its host-memory writes) end
    the engine's polling wait with the IDs, scores and timeout word in place; a wait for a value
    that was not written fails once the stream passed the event, and a stale event is refused."""
    from ferry_amd.h2d import H2DEngine
    from ferry_amd.hostmem import mapped_buffer
    from ferry_amd.metadata import DeviceGateHistory
    ops = _ops()
    E, k, W = 128, 8, 128
    nw = ops.history_ready_words(T, k)
    assert nw == 1 + -(-T * k // 4096)
    status = 4 * E + (T * k + 3) // 4 * 4
    host, dptr = mapped_buffer(status + 4 + 4 * nw)
    hp = host.data_ptr()
    words = host.numpy()[status + 4:status + 4 + 4 * nw].view(np.int32)
    cache = torch.zeros((4, 1 << 12), dtype=torch.bfloat16, device=device)
    eng = H2DEngine(cache, torch.zeros((8, 1 << 12), dtype=torch.bfloat16).pin_memory())
    hist = DeviceGateHistory(1, E, k, W, device)
    ref = GateHistoryRef(1, E, W)
    rng = np.random.default_rng(T)
    stream = torch.cuda.current_stream(device)
    for value in (7, 8, 2**31 - 1):
        sel = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int64)
        hist.update(0, torch.from_numpy(sel).to(device), dptr, dptr + 4 * E, dptr + status,
                    dptr + status + 4, value)
        ev = eng.mark_used_record([0, 1], stream)
        eng.wait_ready(ev, hp + status + 4, nw, value)
        assert (words == value).all()
        ref.update(0, frequency_rows(sel, E, W))
        assert np.array_equal(host.numpy()[:4 * E].view(np.float32), ref.scores(0))
        assert np.array_equal(host.numpy()[4 * E:4 * E + T * k], sel.reshape(-1).astype(np.uint8))
        assert host.numpy()[status:status + 4].view(np.int32)[0] == ops.ffn_sync_timeouts()
        # the marked reads count as complete: a copy into slot 0 needs no wait for the event
        eng.fetch([0], [3])
        eng.wait_host([0])
    with pytest.raises(RuntimeError, match='ready words'):
        eng.wait_ready(ev, hp + status + 4, nw, 12345)
    stale = ev
    eng.mark_used_record([], stream)
    with pytest.raises(RuntimeError, match='latest'):
        eng.wait_ready(stale, hp + status + 4, nw, 2**31 - 1)
    torch.cuda.synchronize()
    eng.close()


# ---------------------------------------------------------------------------------------------
# expert FFN + combine
# ---------------------------------------------------------------------------------------------

def _pool(n, H, I, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn((n, 3 * H * I), generator=g) * 0.02).to(torch.bfloat16)


@pytest.mark.parametrize('T,E,k,H,I,zipf', [
    (16, 128, 8, 2048, 768, 1.1),     # decode layer shape (skinny kernels only)
    (300, 16, 4, 256, 128, 1.5),      # mixed skinny / tiled experts
    (700, 8, 2, 512, 256, 0.5),       # tiled-heavy
    (64, 64, 6, 2048, 1408, 0.9),     # DeepSeek-V2-Lite expert shape
])
def test_expert_ffn_and_combine_vs_oracle(device, T, E, k, H, I, zipf):
    ops = _ops()
    rows_w = _pool(E, H, I, seed=T)
    g = torch.Generator().manual_seed(T + 1)
    x = torch.randn((T, H), generator=g).to(torch.bfloat16)
    sel = _selected(T, E, k, seed=T + 2, zipf=zipf)
    w = torch.softmax(torch.randn((T, k), generator=g), -1).to(torch.bfloat16)
    # cache holds the experts in reverse slot order, to exercise slot_of
    cache = rows_w.flip(0).contiguous().to(device)
    slot_of = np.arange(E)[::-1].astype(np.int32).copy()
    lay = ops.layout(sel.to(device), w.to(device), E)
    act = torch.empty((T * k, I), dtype=torch.bfloat16, device=device)
    part = torch.empty((T * k, H), dtype=torch.bfloat16, device=device)
    active = np.unique(sel.numpy())
    ops.expert_ffn(cache, x.to(device), lay.w_sorted, lay.starts, lay.rows, lay.cols, active, slot_of,
                   H, I, act, part, out_mode=0)
    out = ops.combine(part, T, k, H)
    torch.cuda.synchronize()
    # per-(token, expert) rows vs the reference op order
    ref_lay = layout_closed_form(sel.numpy(), E, w.float().numpy())
    w_sorted = torch.from_numpy(ref_lay['w_sorted']).to(torch.bfloat16)
    groups = [e for e in range(E) if ref_lay['counts'][e] > 0]
    rows = [torch.from_numpy(ref_lay['rows'][ref_lay['starts'][e]:ref_lay['starts'][e + 1]]) for e in groups]
    cols = [torch.from_numpy(ref_lay['cols'][ref_lay['starts'][e]:ref_lay['starts'][e + 1]]) for e in groups]
    parts = execute_experts_ref([rows_w[e] for e in groups], x, w_sorted, rows, cols, H, I)
    got_part = part.cpu().float().view(T, k, H)
    for e, r, c, p in zip(groups, rows, cols, parts):
        torch.testing.assert_close(got_part[r, c], p.float(), rtol=2e-2, atol=1e-2)
    ref = reduce_partials_ref(parts, rows, T, H)
    torch.testing.assert_close(out.cpu().float(), ref.float(), rtol=2e-2, atol=1e-2)
    # the combine itself is exact: same fp32 additions in the same order as reduce_partials
    mine = reduce_partials_ref([got_part[r, c].to(torch.bfloat16) for r, c in zip(rows, cols)], rows, T, H)
    assert torch.equal(out.cpu(), mine)


@pytest.mark.parametrize('H,I,counts,split', [
    # Qwen3 expert shape: the 8-row x 128-byte weight loads of the skinny kernels (H, I multiples
    # of 256) and the mid kernel (17-64 rows), in one mixed launch and split by size
    (2048, 768, [1, 5, 16, 17, 31, 32, 33, 47, 64, 3, 0, 64], False),
    (2048, 768, [1, 5, 16, 17, 31, 32, 33, 47, 64, 3, 0, 64], True),
    (2048, 768, [1, 2, 3, 4, 8, 12, 16, 16], True),          # decode: skinny kernels only
    # decode, six experts: the one-launch kernel with 8-column up workgroups
    (2048, 768, [16, 1, 7, 3, 9, 16], True),
    # other multiples of 256: the unpipelined 8-row x 128-byte phase-1 path (the pipelined one
    # serves H = 2048)
    (1024, 256, [1, 3, 16, 9], True),
    (512, 256, [2, 16, 5], True),
    # H, I not multiples of 256: the skinny kernels' fragment-order loads
    (384, 128, [1, 9, 16, 20, 40, 64, 2], False),
    (384, 128, [1, 9, 16, 7], True),
])
def test_small_expert_kernels_vs_oracle(device, H, I, counts, split):
    """Experts of at most 64 rows: every row count class of the skinny and mid kernels, each
    expert's rows against the reference op order."""
    ops = _ops()
    E = len(counts)
    rows_w = _pool(E, H, I, seed=H + len(counts))
    g = torch.Generator().manual_seed(E)
    ids = np.concatenate([np.full(c, e, np.int64) for e, c in enumerate(counts)])
    ids = ids[np.random.default_rng(E).permutation(len(ids))]
    T = len(ids)
    sel = torch.from_numpy(ids).view(T, 1)
    w = (torch.rand((T, 1), generator=g) + 0.5).to(torch.bfloat16)
    x = torch.randn((T, H), generator=g).to(torch.bfloat16)
    lay = ops.layout(sel.to(device), w.to(device), E)
    act = torch.empty((T, I), dtype=torch.bfloat16, device=device)
    part = torch.empty((T, H), dtype=torch.bfloat16, device=device)
    ops.expert_ffn(rows_w.to(device), x.to(device), lay.w_sorted, lay.starts, lay.rows, lay.cols,
                   np.arange(E), np.arange(E, dtype=np.int32), H, I, act, part, out_mode=0,
                   max_rows=max(counts), counts=counts if split else None)
    torch.cuda.synchronize()
    got = part.cpu().float()
    for e, c in enumerate(counts):
        if c == 0:
            continue
        r = torch.from_numpy(np.nonzero(ids == e)[0])
        ref = execute_experts_ref([rows_w[e]], x, w, [r], [torch.zeros(c, dtype=torch.long)], H, I)[0]
        torch.testing.assert_close(got[r], ref.float(), rtol=2e-2, atol=1e-2,
                                   msg=lambda m: f'expert {e} ({c} rows): {m}')


def _list_rows_counts_400():
    # 400 experts: the small ones fill more than one launch's list of 256, and the 17-64-row
    # experts (issued first) outnumber it, so the split falls among them
    c = np.random.default_rng(400).integers(10, 41, 400)
    c[::20] = 70     # tiled
    c[5] = 17
    c[11] = 5
    c[13] = 0
    return [int(v) for v in c]


@pytest.mark.parametrize('counts,H,I', [
    ([200, 1, 5, 16, 17, 31, 33, 64, 0, 90, 3, 40], 2048, 768),   # tiled, mid and skinny
    ([16, 1, 7, 3, 9, 16, 0, 12], 2048, 768),       # decode sizes: the one-launch kernel
    (_list_rows_counts_400(), 256, 128),            # a list split over two launches
])
def test_expert_ffn_list_rows_bit_identical(device, counts, H, I):
    """Row counts given to the library (list_rows: separate tiled and small launches, the small
    gate/up launch's 16-column workgroups for experts of at most 16 rows) give the same bits as
    the call without them (one list, 64-column small-expert workgroups).  Counts that put an
    expert in the other small scheme still give the same bits: a 16-column workgroup of an
    expert with more rows runs its block's mid workgroup, a 64-column one of an expert with
    fewer runs four skinny passes."""
    ops = _ops()
    E = len(counts)
    rows_w = _pool(E, H, I, seed=sum(counts))
    g = torch.Generator().manual_seed(E + 5)
    ids = np.concatenate([np.full(c, e, np.int64) for e, c in enumerate(counts)])
    ids = ids[np.random.default_rng(E).permutation(len(ids))]
    T = len(ids)
    sel = torch.from_numpy(ids).view(T, 1)
    w = (torch.rand((T, 1), generator=g) + 0.5).to(torch.bfloat16)
    x = torch.randn((T, H), generator=g).to(torch.bfloat16).to(device)
    lay = ops.layout(sel.to(device), w.to(device), E)
    cache = rows_w.to(device)
    slot_of = np.arange(E, dtype=np.int32)
    variants = {'no_rows': None, 'rows': np.array(counts)}
    if max(counts) > 16:
        swapped = np.array(counts)
        swapped[counts.index(17)] = 9     # a mid expert given a skinny count
        swapped[counts.index(5)] = 20     # a skinny expert given a mid count
        variants['swapped_schemes'] = swapped
    outs = {}
    for name, c in variants.items():
        act = torch.full((T, I), float('nan'), dtype=torch.bfloat16, device=device)
        part = torch.full((T, H), float('nan'), dtype=torch.bfloat16, device=device)
        ops.expert_ffn(cache, x, lay.w_sorted, lay.starts, lay.rows, lay.cols, np.arange(E),
                       slot_of, H, I, act, part, out_mode=0, max_rows=T, counts=c)
        torch.cuda.synchronize()
        outs[name] = (act.cpu(), part.cpu())
    assert not torch.isnan(outs['no_rows'][1].float()).any()
    for name in variants:
        assert torch.equal(outs[name][0].view(torch.int16), outs['no_rows'][0].view(torch.int16)), name
        assert torch.equal(outs[name][1].view(torch.int16), outs['no_rows'][1].view(torch.int16)), name


@pytest.mark.parametrize('nbytes', [16, 4096 + 16, 3 * 32768 + 48, 5_000_000 // 16 * 16])
def test_hbm_read_xor(device, nbytes):
    """The read-ceiling kernel reads every 16-byte word once: its per-lane XOR equals numpy's."""
    ops = _ops()
    data = np.random.default_rng(nbytes).integers(0, 256, nbytes, dtype=np.uint8)
    buf = torch.from_numpy(data).to(device)
    sink = ops.hbm_read(buf)
    torch.cuda.synchronize()
    want = np.bitwise_xor.reduce(data.view(np.uint32).reshape(-1, 4), axis=0)
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32).reshape(-1, 4), axis=0)
    assert np.array_equal(got, want)
    with pytest.raises(RuntimeError, match='multiple of 16'):
        ops.hbm_read(buf[:nbytes - 8] if nbytes > 16 else buf[:8])


def test_execute_experts_api(device):
    """The reference's execute_experts signature (expert_ops.cpp:16-45) on groups of any size."""
    ops = _ops()
    H, I, cap = 256, 128, 6
    rows_w = _pool(cap, H, I, seed=3)
    cache = rows_w.to(device)
    g = torch.Generator().manual_seed(5)
    R, k = 150, 3
    x = torch.randn((R, H), generator=g).to(torch.bfloat16)
    rw = torch.rand((R, k), generator=g).to(torch.bfloat16)
    sizes = [1, 70, 0, 150, 33]
    slots = [4, 0, 2, 5, 1]
    rows = [torch.randperm(R, generator=g)[:n].sort().values for n in sizes]
    cols = [torch.randint(0, k, (n,), generator=g) for n in sizes]
    got = ops.execute_experts(cache, x.to(device), rw.to(device), slots, [r.to(device) for r in rows],
                              [c.to(device) for c in cols], H, I)
    ref = execute_experts_ref([rows_w[s] for s in slots], x, rw, rows, cols, H, I)
    assert [t.shape[0] for t in got] == sizes
    for a, b in zip(got, ref):
        torch.testing.assert_close(a.cpu().float(), b.float(), rtol=2e-2, atol=1e-2)


def test_full_layer_matches_fp64(device):
    """bf16 MoE output within rel 2e-2 / abs 1e-2 of the reference's fp32-accumulated result."""
    ops = _ops()
    from oracle.experts import moe_fp64
    T, E, k, H, I = 512, 32, 8, 1024, 256
    rows_w = _pool(E, H, I, seed=11)
    g = torch.Generator().manual_seed(12)
    x = torch.randn((T, H), generator=g).to(torch.bfloat16)
    logits = _logits(T, E, torch.bfloat16, seed=13, zipf=1.1)
    w_ref, sel_ref, _ = qwen3_router(logits, k)
    w, sel = ops.router_topk(logits.to(device), k)
    lay = ops.layout(sel, w, E)
    act = torch.empty((T * k, I), dtype=torch.bfloat16, device=device)
    part = torch.empty((T * k, H), dtype=torch.bfloat16, device=device)
    ops.expert_ffn(rows_w.to(device), x.to(device), lay.w_sorted, lay.starts, lay.rows, lay.cols,
                   np.unique(sel_ref.numpy()), np.arange(E, dtype=np.int32), H, I, act, part)
    out = ops.combine(part, T, k, H).cpu().float()
    ref = moe_layer_ref(lambda e: rows_w[e], x, sel_ref, w_ref, E, H, I).float()
    torch.testing.assert_close(out, ref, rtol=2e-2, atol=1e-2)
    exact = moe_fp64(lambda e: rows_w[e], x, sel_ref, w_ref, H, I).float()
    torch.testing.assert_close(out, exact, rtol=2e-2, atol=1e-2)


# ---------------------------------------------------------------------------------------------
# H2D engine
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize('kind', ['kernel', 'dma'])
def test_h2d_fetch_and_counters(device, kind):
    from ferry_amd import h2d
    from ferry_amd.h2d import H2DEngine
    rows, cap, width = 10, 4, 1 << 16
    pool = torch.arange(rows * width, dtype=torch.int32).view(rows, width).to(torch.bfloat16).pin_memory()
    cache = torch.zeros((cap, width), dtype=torch.bfloat16, device=device)
    eng = H2DEngine(cache, pool)
    assert eng.engine == h2d.DMA and eng.kernel_ok    # torch's pinned memory is device-mapped
    eng.engine = h2d.KERNEL if kind == 'kernel' else h2d.DMA
    eng.fetch([2, 0, 3], [7, 1, 9])
    eng.wait_host([2, 0, 3])
    assert eng.copies == 3
    assert torch.equal(cache[2].cpu(), pool[7]) and torch.equal(cache[0].cpu(), pool[1])
    assert torch.equal(cache[3].cpu(), pool[9])
    # a slot named twice in one call ends with the later row, as with copies in stream order
    eng.fetch([0, 1, 0, 2, 1], [5, 6, 7, 8, 3])
    eng.wait_host([0, 1, 2])
    for slot, key in ((0, 7), (1, 3), (2, 8)):
        assert torch.equal(cache[slot].cpu(), pool[key]), (kind, slot)
    s = torch.cuda.current_stream()
    eng.fetch([1], [4])
    eng.wait_stream([1], s)
    snap = cache[1].clone()      # ordered after the copy by the GPU-side wait
    torch.cuda.synchronize()
    assert torch.equal(snap.cpu(), pool[4])
    with pytest.raises(RuntimeError):
        eng.fetch([cap], [0])
    with pytest.raises(RuntimeError):
        H2DEngine(cache, pool.clone())   # not pinned
    eng.synchronize()
    eng.close()


@pytest.mark.parametrize('packed', [False, True])
def test_h2d_reset_in_place(device, packed):
    """reset(): a new engine's state on the same streams -- copies 0, DMA mode, no deferred
    unpack -- and fetches afterwards byte-exact, also into slots written before the reset."""
    from ferry_amd import h2d
    from ferry_amd.h2d import H2DEngine, PackedPool
    rows, cap = 8, 4
    pool = (torch.randn((rows, 3 * 256 * 128)) * 0.02).to(torch.bfloat16).pin_memory()
    cache = torch.zeros((cap, pool.shape[1]), dtype=torch.bfloat16, device=device)
    pk = PackedPool(pool) if packed else None
    eng = H2DEngine.from_packed(cache, pk) if packed else H2DEngine(cache, pool)
    if packed:
        eng.defer_last = True
    eng.fetch([0, 1, 2], [5, 6, 7])
    eng.wait_stream([0, 1, 2], torch.cuda.current_stream())
    eng.engine = h2d.KERNEL
    eng.reset()
    assert eng.copies == 0 and eng.engine == h2d.DMA and not eng.defer_last
    eng.wait_stream([0, 3], torch.cuda.current_stream())   # nothing recorded: no wait
    eng.fetch([3, 0, 1], [1, 2, 3])
    eng.wait_host([3, 0, 1])
    assert eng.copies == 3
    for slot, key in ((3, 1), (0, 2), (1, 3), (2, 7)):
        assert torch.equal(cache[slot].cpu(), pool[key]), (packed, slot)
    eng.close()


@pytest.mark.parametrize('kind', ['kernel', 'dma'])
def test_h2d_copy_waits_for_last_use(device, kind):
    """A fetch into a slot must not overwrite it before the compute that reads it ends."""
    ops = _ops()
    from ferry_amd import h2d
    from ferry_amd.h2d import H2DEngine
    H, I, T, k, E = 2048, 768, 64, 1, 2
    rows_w = _pool(2, H, I, seed=21)
    pool = rows_w.pin_memory()
    cache = torch.zeros((1, 3 * H * I), dtype=torch.bfloat16, device=device)
    eng = H2DEngine(cache, pool)
    eng.engine = h2d.KERNEL if kind == 'kernel' else h2d.DMA
    eng.fetch([0], [0])
    s = torch.cuda.current_stream()
    eng.wait_stream([0], s)
    x = torch.randn((T, H)).to(torch.bfloat16)
    sel = torch.zeros((T, 1), dtype=torch.int64)
    w = torch.ones((T, 1), dtype=torch.bfloat16)
    lay = ops.layout(sel.to(device), w.to(device), E)
    act = torch.empty((T, I), dtype=torch.bfloat16, device=device)
    part = torch.empty((T, H), dtype=torch.bfloat16, device=device)
    for _ in range(20):   # a long read of slot 0 on the compute stream
        ops.expert_ffn(cache, x.to(device), lay.w_sorted, lay.starts, lay.rows, lay.cols, [0],
                       np.zeros(E, np.int32), H, I, act, part)
    eng.mark_used([0], s)
    eng.fetch([0], [1])          # overwrite slot 0 with expert 1: must wait for the reads
    torch.cuda.synchronize()
    eng.synchronize()
    ref = execute_experts_ref([rows_w[0]], x, w, [torch.arange(T)], [torch.zeros(T, dtype=torch.long)], H, I)[0]
    torch.testing.assert_close(part.cpu().float(), ref.float(), rtol=2e-2, atol=1e-2)
    assert torch.equal(cache[0].cpu(), rows_w[1])
    eng.close()


@pytest.mark.parametrize('packed', [False, True])
def test_h2d_mark_used_record_orders_copies(device, packed):
    """mark_used_record: one event both marks the slots (a later copy into slot 0 waits for the
    reads queued before it) and, once event_synchronize returns, the host sees what the
    stream's kernels wrote to mapped host memory -- as the runtime reads its routing IDs."""
    ops = _ops()
    from ferry_amd.h2d import H2DEngine, PackedPool
    from ferry_amd.hostmem import mapped_buffer
    H, I, T, E = 2048, 768, 64, 2
    rows_w = _pool(2, H, I, seed=23)
    pool = rows_w.pin_memory()
    cache = torch.zeros((1, 3 * H * I), dtype=torch.bfloat16, device=device)
    pk = PackedPool(pool, threads=4) if packed else None
    eng = H2DEngine.from_packed(cache, pk) if packed else H2DEngine(cache, pool)
    eng.fetch([0], [0])
    s = torch.cuda.current_stream()
    eng.wait_stream([0], s)
    x = torch.randn((T, H)).to(torch.bfloat16)
    sel = torch.zeros((T, 1), dtype=torch.int64)
    w = torch.ones((T, 1), dtype=torch.bfloat16)
    lay = ops.layout(sel.to(device), w.to(device), E)
    act = torch.empty((T, I), dtype=torch.bfloat16, device=device)
    part = torch.empty((T, H), dtype=torch.bfloat16, device=device)
    for _ in range(20):   # a long read of slot 0 on the compute stream
        ops.expert_ffn(cache, x.to(device), lay.w_sorted, lay.starts, lay.rows, lay.cols, [0],
                       np.zeros(E, np.int32), H, I, act, part)
    host, dptr = mapped_buffer(4096)
    host.zero_()
    ids = torch.arange(1, 65, dtype=torch.int64, device=device).reshape(64, 1)
    hist = dict(ring=torch.zeros(128, dtype=torch.int32, device=device),
                counts=torch.zeros(E + 62, dtype=torch.int32, device=device),
                meta=torch.zeros(2, dtype=torch.int32, device=device))
    ops.history_update(ids % 64, 64, 128, 0, hist['ring'], hist['counts'], hist['meta'], dptr,
                       dptr + 4 * 64)   # scores and uint8 IDs straight into host memory
    ev = eng.mark_used_record([0], s)
    eng.event_synchronize(ev)
    assert np.array_equal(host[256:320].numpy(), (np.arange(1, 65) % 64).astype(np.uint8))
    eng.fetch([0], [1])          # overwrite slot 0 with expert 1: must wait for the reads
    torch.cuda.synchronize()
    eng.synchronize()
    ref = execute_experts_ref([rows_w[0]], x, w, [torch.arange(T)], [torch.zeros(T, dtype=torch.long)], H, I)[0]
    torch.testing.assert_close(part.cpu().float(), ref.float(), rtol=2e-2, atol=1e-2)
    assert torch.equal(cache[0].cpu(), rows_w[1])
    empty = eng.mark_used_record([], s)   # no slots: still an event to wait on
    eng.event_synchronize(empty)
    eng.close()


def test_h2d_kernel_copy_on_caller_stream(device):
    """Kernel-mode copies queued on the caller's stream -- torch's default stream, whose handle
    is 0, and a side stream -- are ordered before that stream's next kernels with no wait."""
    from ferry_amd import h2d
    from ferry_amd.h2d import H2DEngine
    rows, cap, width = 12, 6, 3 * 64 * 128
    pool = torch.randn((rows, width)).to(torch.bfloat16).pin_memory()
    cache = torch.zeros((cap, width), dtype=torch.bfloat16, device=device)
    eng = H2DEngine(cache, pool)
    eng.engine = h2d.KERNEL
    default = torch.cuda.current_stream()
    assert default.cuda_stream == 0
    side = torch.cuda.Stream()
    for i, st in enumerate((default, side, default)):
        eng.set_kernel_stream(st)
        with torch.cuda.stream(st):
            eng.fetch([i, i + 3], [2 * i, 2 * i + 5])
            snap = cache[[i, i + 3]].clone()     # same stream, right after the copy kernel
        torch.cuda.synchronize()
        assert torch.equal(snap.cpu(), pool[[2 * i, 2 * i + 5]]), i
    eng.set_kernel_stream(None)
    eng.fetch([5], [11])
    eng.wait_host([5])
    assert torch.equal(cache[5].cpu(), pool[11])
    eng.close()


def test_h2d_copy_order_across_modes(device):
    """A copy into a slot follows the earlier copies into that slot whatever their kind (DMA
    lanes, copy kernel on the engine's stream or on a caller's stream); wait_stream covers every
    still-running copy into the listed slots, of either kind."""
    from ferry_amd import h2d
    from ferry_amd.h2d import H2DEngine
    rows, cap, width = 8, 4, 4 << 20          # 8 MiB rows: copies long enough to overlap
    g = torch.Generator().manual_seed(11)
    pool = torch.randint(-30000, 30000, (rows, width), generator=g, dtype=torch.int16)
    pool = pool.view(torch.bfloat16).pin_memory()
    cache = torch.zeros((cap, width), dtype=torch.bfloat16, device=device)
    eng = H2DEngine(cache, pool)
    side = torch.cuda.Stream()
    bits = lambda t: t.view(torch.int16)   # noqa: E731
    for rep in range(3):
        # write after write into slot 0: DMA, then the kernel on a side stream, then DMA
        eng.engine = h2d.DMA
        eng.fetch([0, 1], [1, 2])
        eng.engine = h2d.KERNEL
        eng.set_kernel_stream(side)
        eng.fetch([0, 2], [3, 4])
        eng.engine = h2d.DMA
        eng.fetch([3], [5])
        eng.engine = h2d.KERNEL
        eng.set_kernel_stream(None)
        eng.fetch([3], [6])
        # a consumer stream waits for slots filled by both kinds
        consumer = torch.cuda.Stream()
        eng.wait_stream([0, 1, 2, 3], consumer)
        with torch.cuda.stream(consumer):
            snap = cache.clone()
        torch.cuda.synchronize()
        want = pool[[3, 2, 4, 6]]
        assert torch.equal(bits(snap.cpu()), bits(want)), rep
        eng.synchronize()
        cache.zero_()
        torch.cuda.synchronize()
    eng.close()


def _spread_block(row, block, count, g):
    """Row with `count` values of block `block` (8192 values) spread over ~160 binades, so that
    the packed block holds hundreds of list entries."""
    out = row.clone()
    k = torch.randint(20, 100, (count,), generator=g).float()
    sign = torch.where(torch.rand(count, generator=g) < 0.5, -1.0, 1.0)
    big = torch.rand(count, generator=g) < 0.5
    out[8192 * block:8192 * block + count] = (sign * torch.exp2(torch.where(big, k, -k))
                                              * 1.25).to(torch.bfloat16)
    return out


@pytest.mark.parametrize('kind', ['dma', 'kernel'])
def test_h2d_packed_pool_fetch_byte_exact(device, kind):
    """Fetches from a packed pool write the pool rows' exact bytes: Gaussian rows, a row with
    special values (+-0, +-inf, NaN, denormals, huge: escapes), a row with hundreds of
    list entries in one block, a row of random bits (left raw);
    calls of 1 to 10 rows through 3 staging buffers (ring reuse inside a call and across calls),
    a slot named twice, a GPU-side wait, and raw fetches again after detaching.  kind 'kernel':
    the unpack kernel reads the packed rows over the link itself (no staging, no DMA)."""
    from ferry_amd import h2d
    from ferry_amd.h2d import H2DEngine, PackedPool
    mode = h2d.KERNEL if kind == 'kernel' else h2d.DMA
    rows, cap, width = 24, 10, 3 * 256 * 128
    g = torch.Generator().manual_seed(21)
    pool = (torch.randn((rows, width), generator=g) * 0.02).to(torch.bfloat16)
    vals = torch.tensor([0.0, -0.0, float('inf'), -float('inf'), float('nan'), 1e-40, 1e30, -7.0])
    pos = torch.randperm(width, generator=g)[:500]
    pool[5, pos] = vals.to(torch.bfloat16)[torch.arange(500) % len(vals)]
    pool[7] = torch.randint(-32768, 32767, (width,), generator=g, dtype=torch.int16).view(torch.bfloat16)
    pool[9] = _spread_block(pool[9], 4, 700, g)
    pool = pool.pin_memory()
    packed = PackedPool(pool, threads=4)
    assert packed.packed_rows == rows - 1 and packed.ratio > 1.3
    cache = torch.zeros((cap, width), dtype=torch.bfloat16, device=device)
    eng = H2DEngine(cache, pool)
    eng.use_packed(packed, ring_rows=3)
    eng.engine = mode
    bits = lambda t: t.view(torch.int16)   # noqa: E731
    rng = np.random.default_rng(2)
    for size in (1, 7, 10, 3, 10, 2):
        slots = rng.choice(cap, size, replace=False)
        keys = rng.choice(rows, size, replace=False)
        if size >= 7:
            keys[0] = 7          # the raw row
            keys[1] = 5          # the row with escapes
            keys[2] = 9          # the row with many list entries
        eng.fetch(slots, keys)
        eng.wait_host(slots)
        assert torch.equal(bits(cache.cpu()[slots]), bits(pool[keys])), size
    eng.fetch([4, 2, 4], [10, 11, 12])          # slot 4 twice: the later row wins
    consumer = torch.cuda.Stream()
    eng.wait_stream([4, 2], consumer)
    with torch.cuda.stream(consumer):
        snap = cache[[4, 2]].clone()
    torch.cuda.synchronize()
    assert torch.equal(bits(snap.cpu()), bits(pool[[12, 11]]))
    eng.use_packed(None)
    assert eng.engine == mode          # the raw pool serves either kind
    eng.fetch([0, 1], [3, 5])
    assert eng.groups() == [2]         # raw rows: one group
    eng.wait_host([0, 1])
    assert torch.equal(bits(cache.cpu()[[0, 1]]), bits(pool[[3, 5]]))
    other = pool.clone().pin_memory()
    with pytest.raises(RuntimeError):
        H2DEngine(cache, other).use_packed(packed)   # packed from another pool
    eng.close()
    packed.close()
    # a packed pool made from pageable memory stands alone: the source is freed before fetching
    src = pool.clone()
    assert not src.is_pinned()
    alone = PackedPool(src, threads=4)
    del src
    eng = H2DEngine.from_packed(cache, alone, ring_rows=2)
    eng.engine = mode
    slots = np.arange(cap)
    keys = rng.choice(rows, cap, replace=False)
    keys[3] = 7
    eng.fetch(slots, keys)
    eng.wait_host(slots)
    assert torch.equal(bits(cache.cpu()), bits(pool[keys]))
    with pytest.raises(RuntimeError):
        eng.use_packed(None)      # no raw pool to fall back to
    eng.close()
    alone.close()


@pytest.mark.parametrize('defer', [False, True])
def test_h2d_packed_sub_batches_and_ring_reuse(device, defer):
    """Calls large enough to go in several sub-batches (about 4, 8, 16 MiB from the call's end),
    each unpacked on the engine's unpack stream while the DMA lanes copy the next: 12 rows of
    ~2.8 MiB packed through a ring of 3 staging buffers (every staging buffer is reused inside
    a call, after the unpack that read it), a call naming a slot twice, calls back to back
    without a host wait, a raw row among packed ones, and a GPU-side wait on the caller's
    stream -- every slot holds the pool row's exact bytes."""
    from ferry_amd.h2d import H2DEngine, PackedPool
    rows, cap, width = 16, 14, (1 << 21) + 8192
    g = torch.Generator().manual_seed(5)
    pool = (torch.randn((rows, width), generator=g) * 0.02).to(torch.bfloat16)
    pool[6] = torch.randint(-32768, 32767, (width,), generator=g, dtype=torch.int16).view(torch.bfloat16)
    pool[11] = _spread_block(pool[11], 7, 500, g)
    packed = PackedPool(pool, threads=8)
    assert packed.packed_rows == rows - 1
    cache = torch.zeros((cap, width), dtype=torch.bfloat16, device=device)
    eng = H2DEngine.from_packed(cache, packed, ring_rows=3)
    eng.defer_last = defer   # the last sub-batch's unpack runs where its slots are waited for
    bits = lambda t: t.view(torch.int16)   # noqa: E731
    keys = np.array([0, 6, 1, 2, 11, 3, 4, 5, 7, 8, 9, 10])
    eng.fetch(np.arange(12), keys)
    ends = eng.groups()    # the call's sub-batches, as positions in its slot list
    assert len(ends) > 1 and ends[-1] == 12 and ends == sorted(set(ends)), ends
    eng.fetch([12, 13, 12], [13, 14, 15])      # back to back; slot 12 twice: row 15 wins
    assert eng.groups()[-1] == 3 and len(eng.groups()) >= 2   # the repeat starts a sub-batch
    eng.wait_host(np.arange(cap))
    want = pool[np.concatenate([keys, [15, 14]])]
    assert torch.equal(bits(cache.cpu()), bits(want))
    # overwrite every slot in one call (reverse order) and read it on another stream
    keys2 = np.arange(cap)[::-1].copy()
    eng.fetch(np.arange(cap), keys2)
    consumer = torch.cuda.Stream()
    eng.wait_stream(np.arange(cap), consumer)
    with torch.cuda.stream(consumer):
        snap = cache.clone()
    torch.cuda.synchronize()
    assert torch.equal(bits(snap.cpu()), bits(pool[keys2]))
    eng.close()
    packed.close()


@pytest.mark.parametrize('defer', [False, True])
def test_h2d_packed_slot_named_twice_raw_and_packed(device, defer):
    """A slot named twice in one packed DMA call, its rows in different sub-batches: raw then
    packed, packed then raw, raw then raw, and within one sub-batch -- the later row wins in
    every case (a raw row is copied by both lanes in byte ranges that differ between
    sub-batches, a packed one by the unpack stream)."""
    from ferry_amd.h2d import H2DEngine, PackedPool
    rows, cap, width = 16, 14, (1 << 21) + 8192
    g = torch.Generator().manual_seed(9)
    pool = (torch.randn((rows, width), generator=g) * 0.02).to(torch.bfloat16)
    for r in (6, 9, 13):     # random bits: stored raw
        pool[r] = torch.randint(-32768, 32767, (width,), generator=g,
                                dtype=torch.int16).view(torch.bfloat16)
    packed = PackedPool(pool, threads=8)
    assert packed.packed_rows == rows - 3
    cache = torch.zeros((cap, width), dtype=torch.bfloat16, device=device)
    eng = H2DEngine.from_packed(cache, packed, ring_rows=3)
    eng.defer_last = defer
    bits = lambda t: t.view(torch.int16)   # noqa: E731
    calls = [
        # raw then packed (slot 3), packed then raw (slot 5), raw then raw (slot 8)
        ([3, 0, 1, 2, 5, 4, 8, 7, 3, 10, 5, 11, 8],
         [6, 0, 1, 2, 3, 4, 9, 5, 7, 8, 13, 10, 6]),
        # within the first sub-batch: packed then raw, then more rows after
        ([2, 2, 6, 7, 9, 12], [1, 9, 0, 2, 3, 4]),
        # raw row last, after the slot's packed row several sub-batches earlier
        ([4, 0, 1, 5, 6, 7, 10, 11, 4], [5, 0, 1, 2, 3, 7, 8, 10, 13]),
    ]
    want = torch.zeros((cap, width), dtype=torch.bfloat16)
    for slots, keys in calls:
        for sl, k in zip(slots, keys):
            want[sl] = pool[k]
        eng.fetch(slots, keys)
        consumer = torch.cuda.Stream()
        eng.wait_stream(sorted(set(slots)), consumer)
        with torch.cuda.stream(consumer):
            snap = cache.clone()
        torch.cuda.synchronize()
        assert torch.equal(bits(snap.cpu()), bits(want)), slots
    eng.close()
    packed.close()


@pytest.mark.parametrize('kind', ['dma', 'kernel'])
@pytest.mark.parametrize('width', [2 * 8192 + 96, 32, 8192])
def test_h2d_packed_pool_ragged_widths(device, width, kind):
    """Packed rows whose length is not a whole number of 8192-value blocks (a partial last
    workgroup), a single 32-value row and one exact block unpack to the pool rows' bytes."""
    from ferry_amd import h2d
    from ferry_amd.h2d import H2DEngine, PackedPool
    rows, cap = 8, 8
    g = torch.Generator().manual_seed(width)
    pool = (torch.randn((rows, width), generator=g) * 0.02).to(torch.bfloat16)
    if width > 8192:
        pool[3] = _spread_block(pool[3], 1, 400, g)
    packed = PackedPool(pool, threads=2)
    cache = torch.zeros((cap, width), dtype=torch.bfloat16, device=device)
    eng = H2DEngine.from_packed(cache, packed, ring_rows=4)
    if kind == 'kernel':
        eng.engine = h2d.KERNEL
    keys = np.arange(rows)[::-1].copy()
    eng.fetch(np.arange(cap), keys)
    eng.wait_host(np.arange(cap))
    assert torch.equal(cache.cpu().view(torch.int16), pool[keys].view(torch.int16))
    eng.close()
    packed.close()


def test_h2d_kernel_copy_many_rows_and_ragged_widths(device):
    """The copy kernel against the DMA path: a fetch of more rows than one launch takes (300, in
    any slot order), row sizes that are and are not multiples of its 16-byte unit (the latter
    stay on DMA), and both kinds interleaved on one engine."""
    from ferry_amd import h2d
    from ferry_amd.h2d import H2DEngine
    g = torch.Generator().manual_seed(5)
    rows, cap = 320, 300
    for width in (8 * 4099, 7):          # 65,584 B rows (16-byte multiple) and 14 B rows
        pool = torch.randint(-30000, 30000, (rows, width), generator=g, dtype=torch.int16)
        pool = pool.view(torch.bfloat16).pin_memory()
        cache = torch.zeros((cap, width), dtype=torch.bfloat16, device=device)
        eng = H2DEngine(cache, pool)
        assert eng.engine == h2d.DMA
        if width % 8:
            assert not eng.kernel_ok
            with pytest.raises(RuntimeError):
                eng.engine = h2d.KERNEL
        else:
            eng.engine = h2d.KERNEL
        slots = torch.randperm(cap, generator=g).numpy()
        keys = torch.randperm(rows, generator=g)[:cap].numpy()
        bits = lambda t: t.view(torch.int16)   # noqa: E731  (random bits include NaNs)
        eng.fetch(slots, keys)
        eng.wait_host(slots)
        assert torch.equal(bits(cache.cpu()[slots]), bits(pool[keys]))
        if width % 8 == 0:
            eng.engine = h2d.DMA
            eng.fetch(slots[:50], keys[::-1][:50])
            eng.engine = h2d.KERNEL
            eng.fetch(slots[50:60], keys[:10])
            eng.wait_host(slots[:60])
            assert torch.equal(bits(cache.cpu()[slots[:50]]), bits(pool[keys[::-1][:50].copy()]))
            assert torch.equal(bits(cache.cpu()[slots[50:60]]), bits(pool[keys[:10]]))
        eng.close()


def test_h2d_packed_kernel_mode_many_rows(device):
    """Kernel-mode packed fetches of more rows than one unpack launch holds (150 rows: three
    launches), raw rows among them, a slot named twice (a new launch, the later row wins), then
    DMA-mode packed fetches into the same slots and kernel-mode ones again, ordered by the
    engine: every slot holds the pool row's exact bytes."""
    from ferry_amd import h2d
    from ferry_amd.h2d import H2DEngine, PackedPool
    rows, cap, width = 180, 160, 4 * 8192 + 64
    g = torch.Generator().manual_seed(17)
    pool = (torch.randn((rows, width), generator=g) * 0.02).to(torch.bfloat16)
    for r in (3, 77, 140):
        pool[r] = torch.randint(-32768, 32767, (width,), generator=g,
                                dtype=torch.int16).view(torch.bfloat16)
    pool[5] = _spread_block(pool[5], 2, 600, g)
    packed = PackedPool(pool, threads=8)
    assert packed.packed_rows == rows - 3
    cache = torch.zeros((cap, width), dtype=torch.bfloat16, device=device)
    eng = H2DEngine.from_packed(cache, packed, ring_rows=5)
    eng.engine = h2d.KERNEL
    bits = lambda t: t.view(torch.int16)   # noqa: E731
    slots = torch.randperm(cap, generator=g).numpy()[:150]
    keys = torch.randperm(rows, generator=g).numpy()[:150]
    keys[:4] = [3, 77, 140, 5]
    eng.fetch(slots, keys)
    eng.wait_host(slots)
    assert torch.equal(bits(cache.cpu()[slots]), bits(pool[keys]))
    a, b = int(slots[40]), int(slots[41])
    eng.fetch([a, b, a], [100, 101, 102])      # slot a twice: row 102 wins
    eng.engine = h2d.DMA
    eng.fetch(slots[:20], keys[::-1][:20].copy())
    eng.engine = h2d.KERNEL
    eng.fetch(slots[20:30], keys[:10])
    eng.wait_host(np.concatenate([[a, b], slots[:30]]))
    got = cache.cpu()
    assert torch.equal(bits(got[[a, b]]), bits(pool[[102, 101]]))
    assert torch.equal(bits(got[slots[:20]]), bits(pool[keys[::-1][:20].copy()]))
    assert torch.equal(bits(got[slots[20:30]]), bits(pool[keys[:10]]))
    eng.close()
    packed.close()


def test_h2d_packed_deferred_last_unpack(device):
    """With defer_last, the last sub-batch of a packed call is unpacked by the first wait_stream
    that names one of its slots (on that stream); a wait_stream on other slots leaves it pending;
    the next fetch, wait_host or synchronize queues a pending one on the unpack stream; turning
    the option off queues it too.  Every slot holds the pool row's exact bytes."""
    from ferry_amd.h2d import H2DEngine, PackedPool
    rows, cap, width = 12, 10, (1 << 20) + 4096
    g = torch.Generator().manual_seed(9)
    pool = (torch.randn((rows, width), generator=g) * 0.02).to(torch.bfloat16)
    pool[4] = torch.randint(-32768, 32767, (width,), generator=g,
                            dtype=torch.int16).view(torch.bfloat16)
    packed = PackedPool(pool, threads=8)
    cache = torch.zeros((cap, width), dtype=torch.bfloat16, device=device)
    eng = H2DEngine.from_packed(cache, packed, ring_rows=4)
    eng.defer_last = True
    bits = lambda t: t.view(torch.int16)   # noqa: E731
    consumer = torch.cuda.Stream()
    # 1: the consumer waits for the fetched slots (resolves on the consumer stream)
    eng.fetch([0, 1, 2, 3, 4, 5], [0, 1, 2, 3, 4, 5])
    eng.wait_stream([0, 1, 2, 3, 4, 5], consumer)
    with torch.cuda.stream(consumer):
        snap = cache[:6].clone()
    torch.cuda.synchronize()
    assert torch.equal(bits(snap.cpu()), bits(pool[:6]))
    # 2: a wait on other slots leaves the pending unpack; the next fetch queues it
    eng.fetch([6, 7], [6, 7])
    eng.wait_stream([0], consumer)
    eng.fetch([8], [8])
    eng.wait_host([6, 7, 8])
    assert torch.equal(bits(cache.cpu()[6:9]), bits(pool[6:9]))
    # 3: synchronize queues it; the raw row (4) among deferred ones
    eng.fetch([9, 0], [4, 11])
    eng.synchronize()
    assert torch.equal(bits(cache.cpu()[[9, 0]]), bits(pool[[4, 11]]))
    # 4: turning the option off queues it; later calls unpack on the engine's stream
    eng.fetch([1, 2], [10, 9])
    eng.defer_last = False
    eng.fetch([3], [7])
    eng.wait_host([1, 2, 3])
    assert torch.equal(bits(cache.cpu()[[1, 2, 3]]), bits(pool[[10, 9, 7]]))
    eng.close()
    packed.close()
