"""End-to-end parity of OffloadRuntime.execute with the oracle: output (toleranced) and the
fetch/eviction trace (bit-exact), through the fused HIP path."""
import numpy as np
import pytest
import torch

from oracle.experts import moe_layer_ref
from oracle.history import GateHistoryRef, frequency_rows
from oracle.policy import PlannerRef
from oracle.router import qwen3_router

pytestmark = pytest.mark.gpu


def _run(device, spec, cap, calls, tokens_of, seed, zipf, overlap=True, check_every=1,
         gate_scale=8.0, copy='dma', score='frequency', pack=False):
    """``calls`` layer calls through OffloadRuntime against the oracle: GateHistoryRef fed with
    the reference's history rows (one-hot rows of the last min(T, W) tokens for the frequency
    score; those tokens' fp32 router probabilities for the probability score, metadata.py:
    55-59,77-78) and PlannerRef; the planner state bit-exact after every call, the output
    within tolerance every ``check_every`` calls."""
    from ferry_amd import workloads
    from ferry_amd.quota import Topology
    from ferry_amd.runtime import OffloadRuntime
    pool = workloads.make_pool(spec, spec.layers, seed=seed)
    rt = OffloadRuntime(spec, pool, [cap], 'ferry', Topology.uniform(1, spec.experts),
                        overlap=overlap, copy=copy, eviction_score=score, pack=pack)
    planner = PlannerRef(spec.layers, spec.experts, cap)
    hist = GateHistoryRef(spec.layers, spec.experts, 128)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    rng = np.random.default_rng(seed)
    gates = []
    for _ in range(spec.layers):
        gw = torch.randn((spec.experts, spec.hidden), generator=g, device=device) * 0.02
        gates.append(gw.to(torch.bfloat16))
    biases = [torch.from_numpy(workloads.zipf_log_bias(spec.experts, zipf, rng)).to(device)
              for _ in range(spec.layers)]
    skipped = 0
    for call in range(calls):
        layer = call % spec.layers
        T = tokens_of(call)
        x = torch.randn((T, spec.hidden), generator=g, device=device).to(torch.bfloat16)
        if gate_scale:
            z = x.float() @ gates[layer].float().t() * gate_scale
        else:   # N(0, 1) logits as in the synthetic decode stream
            z = torch.randn((T, spec.experts), generator=g, device=device)
        logits = (z + biases[layer]).to(torch.bfloat16)
        w_ref, sel_ref, probs_ref = qwen3_router(logits.cpu(), spec.topk)
        if len(np.unique(sel_ref.numpy())) > cap:
            skipped += 1
            continue   # the reference asserts on such a call (quota.py:63)
        from ferry_amd import expert_ops as ops
        if score == 'probability':
            w, sel, probs = ops.router_topk(logits, spec.topk, return_probs=True)
            out = rt.execute(layer, x, sel, w, probs[-128:])
            rows = probs_ref[-min(T, 128):].numpy()          # fp32 rows, as gathered
        else:
            w, sel = ops.router_topk(logits, spec.topk)
            out = rt.execute(layer, x, sel, w, None)
            rows = frequency_rows(sel_ref.numpy(), spec.experts, 128)
        # oracle: history -> plan -> trace
        hist.update(layer, rows)
        fetches, _ = planner.plan(rt.event - 1, layer, sel_ref.numpy(), hist.scores(layer))
        assert np.array_equal(rt.controller.slots[0], planner.slots), f'call {call}: slots differ'
        assert np.array_equal(rt.controller.last, planner.last)
        assert np.array_equal(rt.controller.scores, planner.scores)
        if call % check_every == 0:
            torch.cuda.synchronize()
            ref = moe_layer_ref(lambda e: pool[layer * spec.experts + e], x.cpu(), sel_ref, w_ref,
                                spec.experts, spec.hidden, spec.intermediate)
            torch.testing.assert_close(out.cpu().float(), ref.float(), rtol=2e-2, atol=1e-2)
    rt.close()
    return rt, skipped


def test_runtime_small_evicting(device):
    from ferry_amd.model import ModelSpec
    spec = ModelSpec('qwen3_moe', (0, 1, 2), 32, 4, 256, 128)
    rt, skipped = _run(device, spec, cap=20, calls=60,
                       tokens_of=lambda c: [3, 16, 40, 1, 130][c % 5], seed=5, zipf=1.0)
    assert rt.h2d.copies == int(rt.fetches_per_rank.sum()) > 20   # evictions happened


@pytest.mark.parametrize('pack', [False, True])
def test_runtime_probability_score_evicting(device, pack):
    """eviction_score='probability' (the reference's Eq. 12 score, run_cell.py:187): the
    history rows are the fp32 router probabilities of the last min(T, W) tokens; calls shorter
    and longer than W, with evictions every few calls; the planner state (slots, owners, last
    use, scores) bit-exact with the oracle after every call, outputs within tolerance."""
    from ferry_amd.model import ModelSpec
    spec = ModelSpec('qwen3_moe', (0, 1, 2), 32, 4, 256, 128)
    # 32 slots hold any one call's experts but not three layers' (96 keys): evictions
    rt, skipped = _run(device, spec, cap=32, calls=45,
                       tokens_of=lambda c: [3, 16, 40, 1, 200][c % 5], seed=7, zipf=1.0,
                       score='probability', pack=pack, check_every=3)
    assert rt.gather.score == 'probability'
    assert skipped == 0 and rt.h2d.copies == int(rt.fetches_per_rank.sum()) > 64


def test_runtime_mixed_copy_modes(device):
    """copy='kernel': prefill-sized calls (DMA copies, chunked) and decode-sized calls (copy
    kernel on the compute stream) interleaved on one runtime: every call against the oracle,
    the eviction trace bit-exact."""
    from ferry_amd.model import ModelSpec
    spec = ModelSpec('qwen3_moe', (0, 1), 32, 4, 256, 128)
    rt, _ = _run(device, spec, cap=24, calls=12, tokens_of=lambda c: [4096, 16, 5000, 3][c % 4],
                 seed=8, zipf=0.8, copy='kernel')
    assert rt._kernel_copy and rt.h2d.copies > 24


def test_runtime_small_evicting_copy_kernel(device):
    from ferry_amd.model import ModelSpec
    spec = ModelSpec('qwen3_moe', (0, 1, 2), 32, 4, 256, 128)
    rt, _ = _run(device, spec, cap=20, calls=40, tokens_of=lambda c: [3, 16, 40, 1, 130][c % 5],
                 seed=5, zipf=1.0, copy='kernel')
    assert rt.h2d.copies == int(rt.fetches_per_rank.sum()) > 20


@pytest.mark.parametrize('tokens', [16, 64])
def test_runtime_on_stream_matches_dma_overlap(device, tokens):
    """The decode path with the copy kernel on the compute stream (one FFN launch after the
    copy) and the DMA path (resident experts first, then the fetched ones) give bit-identical
    outputs and the same fetch trace."""
    from dataclasses import replace

    from ferry_amd import expert_ops as ops
    from ferry_amd import workloads
    from ferry_amd.model import QWEN3_30B_A3B
    from ferry_amd.quota import Topology
    from ferry_amd.runtime import OffloadRuntime
    spec = replace(QWEN3_30B_A3B, moe_layers=(0, 1))
    pool = workloads.make_pool(spec, spec.layers, seed=3)
    bias = torch.from_numpy(workloads.zipf_log_bias(spec.experts, 1.1, np.random.default_rng(0)))
    cap = 80      # above any call's distinct experts (<= 62 at 64 tokens), below two layers'
    runs = []
    for copy in ('kernel', 'dma'):
        rt = OffloadRuntime(spec, pool, [cap], 'ferry', Topology.uniform(1, spec.experts),
                            copy=copy)
        assert rt._kernel_copy == (copy == 'kernel')
        g = torch.Generator(device=device)
        g.manual_seed(4)
        outs = []
        for call in range(8):
            x = torch.randn((tokens, spec.hidden), generator=g, device=device).to(torch.bfloat16)
            z = torch.randn((tokens, spec.experts), generator=g, device=device) + bias.to(device)
            w, sel = ops.router_topk(z.to(torch.bfloat16), spec.topk)
            assert len(torch.unique(sel)) <= cap
            outs.append(rt.execute(call % 2, x, sel, w, None).cpu())
        runs.append((outs, rt.controller.slots[0].copy(), rt.h2d.copies))
        rt.close()
    (a, slots_a, n_a), (b, slots_b, n_b) = runs
    assert n_a == n_b > cap and np.array_equal(slots_a, slots_b)
    for i, (u, v) in enumerate(zip(a, b)):
        assert torch.equal(u, v), i


@pytest.mark.parametrize('tokens', [16, 2048])
def test_runtime_packed_pool_matches_raw(device, tokens):
    """OffloadRuntime(pack=True) -- misses copied as packed rows and unpacked on the GPU -- gives
    bit-identical outputs and the same fetch trace as raw fetches, on decode-sized and on
    chunked prefill-sized calls; so does split_fetch=True (a packed decode call's fetched experts
    computed sub-batch by sub-batch as they are unpacked)."""
    from dataclasses import replace

    from ferry_amd import expert_ops as ops
    from ferry_amd import workloads
    from ferry_amd.model import QWEN3_30B_A3B
    from ferry_amd.quota import Topology
    from ferry_amd.runtime import OffloadRuntime
    spec = replace(QWEN3_30B_A3B, moe_layers=(0, 1))
    pool = workloads.make_pool(spec, spec.layers, seed=3)
    bias = torch.from_numpy(workloads.zipf_log_bias(spec.experts, 1.1, np.random.default_rng(0)))
    cap = 200 if tokens > 64 else 80
    from ferry_amd.h2d import PackedPool
    runs = []
    for pack in ('packed_pool', True, 'split', False):
        if pack == 'packed_pool':   # the runtime given a PackedPool of a pageable pool
            src = workloads.make_pool(spec, spec.layers, seed=3, pinned=False)
            rt = OffloadRuntime(spec, PackedPool(src), [cap], 'ferry',
                                Topology.uniform(1, spec.experts))
            del src
        elif pack == 'split':
            rt = OffloadRuntime(spec, pool, [cap], 'ferry', Topology.uniform(1, spec.experts),
                                pack=True, split_fetch=True)
        else:
            rt = OffloadRuntime(spec, pool, [cap], 'ferry', Topology.uniform(1, spec.experts),
                                pack=pack)
        if pack:
            assert rt.packed.ratio > 1.3
        g = torch.Generator(device=device)
        g.manual_seed(4)
        outs = []
        sub_batches = 0
        for call in range(6):
            x = torch.randn((tokens, spec.hidden), generator=g, device=device).to(torch.bfloat16)
            z = torch.randn((tokens, spec.experts), generator=g, device=device) + bias.to(device)
            w, sel = ops.router_topk(z.to(torch.bfloat16), spec.topk)
            outs.append(rt.execute(call % 2, x, sel, w, None).cpu())
            sub_batches = max(sub_batches, len(rt.h2d.groups()))
        if pack == 'split' and tokens <= 64:
            assert sub_batches >= 2   # the fetched experts did run in several launches
        runs.append((outs, rt.controller.slots[0].copy(), rt.h2d.copies))
        rt.close()
    base_outs, base_slots, base_n = runs[-1]
    for outs, slots, n in runs[:-1]:
        assert n == base_n > 0 and np.array_equal(slots, base_slots)
        for i, (u, v) in enumerate(zip(outs, base_outs)):
            assert torch.equal(u, v), i


def test_runtime_packed_reset_and_serial(device):
    """A reset in the middle of a run (the engine reset in place, not rebuilt) and the serial
    mode, with packed fetches: outputs, eviction state and copy counts equal the raw, overlapped
    run's, call by call."""
    from dataclasses import replace

    from ferry_amd import expert_ops as ops
    from ferry_amd import workloads
    from ferry_amd.model import QWEN3_30B_A3B
    from ferry_amd.quota import Topology
    from ferry_amd.runtime import OffloadRuntime
    spec = replace(QWEN3_30B_A3B, moe_layers=(0, 1))
    pool = workloads.make_pool(spec, spec.layers, seed=5)
    bias = torch.from_numpy(workloads.zipf_log_bias(spec.experts, 1.1, np.random.default_rng(1)))
    runs = []
    for pack, overlap in ((True, True), (True, False), (False, True)):
        rt = OffloadRuntime(spec, pool, [80], 'ferry', Topology.uniform(1, spec.experts), pack=pack,
                            overlap=overlap)
        streams = [id(rt.h2d)]
        g = torch.Generator(device=device)
        g.manual_seed(9)
        outs, copies = [], []
        for call in range(8):
            if call == 4:
                rt.reset()
                streams.append(id(rt.h2d))
                assert rt.h2d.copies == 0
            x = torch.randn((16, spec.hidden), generator=g, device=device).to(torch.bfloat16)
            z = torch.randn((16, spec.experts), generator=g, device=device) + bias.to(device)
            w, sel = ops.router_topk(z.to(torch.bfloat16), spec.topk)
            outs.append(rt.execute(call % 2, x, sel, w, None).cpu())
            copies.append(rt.h2d.copies)
        assert streams[0] == streams[1]   # the same engine object after the reset
        runs.append((outs, rt.controller.slots[0].copy(), copies))
        rt.close()
    base_outs, base_slots, base_copies = runs[-1]
    for outs, slots, copies in runs[:-1]:
        assert copies == base_copies and np.array_equal(slots, base_slots)
        for i, (u, v) in enumerate(zip(outs, base_outs)):
            assert torch.equal(u, v), i


def test_runtime_serial_mode(device):
    from ferry_amd.model import ModelSpec
    spec = ModelSpec('qwen3_moe', (0, 1), 16, 4, 256, 128)
    rt, _ = _run(device, spec, cap=9, calls=20, tokens_of=lambda c: 8, seed=6, zipf=1.2,
                 overlap=False)
    assert rt.serial_wait_ns >= 0


def test_runtime_qwen3_decode_shape(device):
    """The Qwen3-30B-A3B decode layer: 16 tokens, 128 experts top-8, cache of 38."""
    from ferry_amd.model import QWEN3_30B_A3B
    from dataclasses import replace
    spec = replace(QWEN3_30B_A3B, moe_layers=(0,))
    rt, skipped = _run(device, spec, cap=38, calls=24, tokens_of=lambda c: 16, seed=1, zipf=1.1,
                       check_every=3, gate_scale=0.0)
    assert skipped < 4 and rt.h2d.copies > 38


def test_h2d_profiler_writes_loadable_topology(device, tmp_path):
    """The H2D profiler measures expert-sized copies through the fetch engine and on one stream
    and writes a topology file that Topology and OffloadRuntime accept."""
    from ferry_amd.h2dprof import main
    from ferry_amd.quota import Topology
    out = tmp_path / 'topo.json'
    doc = main(['--output', str(out), '--expert-bytes', str(4 << 20), '--experts', '16',
                '--copies', '16', '--repeats', '3'])
    m = doc['measured']
    assert 1.0 < m['engine_gib_per_s'] < 200.0 and 1.0 < m['single_stream_gib_per_s'] < 200.0
    assert 1.0 < m['kernel_gib_per_s'] < 200.0
    assert len(m['samples']['engine']) == 3
    topo = Topology(out, 1, 16)
    assert topo.lut[:, 0].tolist() == list(range(17))


@pytest.mark.parametrize('family', ['qwen3', 'deepseek'])
def test_fused_decode_ffn_matches_two_launch_path(device, family):
    """The one-launch decode FFN (every expert at most 16 rows, both phases) against the
    two-launch path (the phases called separately) on the Qwen3-30B-A3B and DeepSeek-V2-Lite
    expert shapes, bit for bit, over calls that reuse the activation buffer; no wait of the
    fused launch gave up."""
    from ferry_amd import expert_ops as ops
    from ferry_amd import workloads
    from ferry_amd.model import DEEPSEEK_V2_LITE, QWEN3_30B_A3B
    spec = QWEN3_30B_A3B if family == 'qwen3' else DEEPSEEK_V2_LITE
    E, k, H, I = spec.experts, spec.topk, spec.hidden, spec.intermediate
    cache = workloads.expert_rows(range(40), spec.expert_elements, seed=9, device=device)
    slot_of = np.full(E, -1, np.int32)
    experts = np.random.default_rng(0).choice(E, 40, replace=False)
    slot_of[experts] = np.arange(40)
    g = torch.Generator(device=device)
    g.manual_seed(3)
    act = torch.empty((64 * k, I), dtype=torch.bfloat16, device=device)
    timeouts0 = ops.ffn_sync_timeouts()
    for T in (16, 1, 64 // 8, 16, 3):
        sel = torch.stack([torch.from_numpy(np.random.default_rng(T + i).choice(experts, k, replace=False))
                           for i in range(T)]).to(device)
        w = torch.softmax(torch.randn((T, k), generator=g, device=device), -1).to(torch.bfloat16)
        x = torch.randn((T, H), generator=g, device=device).to(torch.bfloat16)
        lay = ops.layout(sel, w, E, check=True)
        active = np.unique(sel.cpu().numpy())
        counts = np.bincount(sel.cpu().numpy().reshape(-1), minlength=E)
        assert counts.max() <= 16
        fused = torch.empty((T * k, H), dtype=torch.bfloat16, device=device)
        two = torch.empty_like(fused)
        args = (cache, x, lay.w_sorted, lay.starts, lay.rows, lay.cols, active, slot_of, H, I)
        ops.expert_ffn(*args, act[:T * k], fused, experts=E, counts=counts)
        ops.expert_ffn(*args, act[:T * k], two, experts=E, counts=counts, phases=ops.PHASE_UP)
        ops.expert_ffn(*args, act[:T * k], two, experts=E, counts=counts, phases=ops.PHASE_DOWN)
        torch.cuda.synchronize()
        assert torch.equal(fused, two), T
    assert ops.ffn_sync_timeouts() == timeouts0


def test_runtime_raises_after_decode_ffn_timeout(device):
    """A one-launch decode FFN whose down phase gives up -- forced from the host with a spin
    limit of 0, so that every workgroup still exits normally -- leaves its experts' rows
    unwritten.  The runtime must not pass that off as a layer output: the next call raises at
    its routing readback, as do reset() and close(); after the error the runtime works again
    and matches the oracle."""
    from ferry_amd import expert_ops as ops
    from ferry_amd import workloads
    from ferry_amd.model import ModelSpec
    from ferry_amd.quota import Topology
    from ferry_amd.runtime import OffloadRuntime
    spec = ModelSpec('qwen3_moe', (0, 1), 32, 4, 256, 128)
    pool = workloads.make_pool(spec, spec.layers, seed=12)
    rt = OffloadRuntime(spec, pool, [64], 'ferry', Topology.uniform(1, spec.experts))
    g = torch.Generator(device=device)
    g.manual_seed(2)
    T = 8
    x = torch.randn((T, spec.hidden), generator=g, device=device).to(torch.bfloat16)
    logits = torch.randn((T, spec.experts), generator=g, device=device).to(torch.bfloat16)
    w, sel = ops.router_topk(logits, spec.topk)
    w_ref, sel_ref, _ = qwen3_router(logits.cpu(), spec.topk)

    def check(out, layer):
        torch.cuda.synchronize()
        ref = moe_layer_ref(lambda e: pool[layer * spec.experts + e], x.cpu(), sel_ref, w_ref,
                            spec.experts, spec.hidden, spec.intermediate)
        torch.testing.assert_close(out.cpu().float(), ref.float(), rtol=2e-2, atol=1e-2)

    check(rt.execute(0, x, sel, w, None), 0)
    try:
        ops.ffn_set_sync_spin_limit(0)
        rt.execute(1, x, sel, w, None)       # the fused launch's down waits give up at once
    finally:
        ops.ffn_set_sync_spin_limit(None)
    with pytest.raises(RuntimeError, match='gave up'):
        rt.execute(0, x, sel, w, None)
    rt.reset()                               # the error was reported: a clean reset
    check(rt.execute(1, x, sel, w, None), 1)
    check(rt.execute(1, x, sel, w, None), 1)  # resident now: the other launch path
    try:
        ops.ffn_set_sync_spin_limit(0)
        rt.execute(0, x, sel, w, None)
    finally:
        ops.ffn_set_sync_spin_limit(None)
    with pytest.raises(RuntimeError, match='gave up'):
        rt.reset()
    check(rt.execute(0, x, sel, w, None), 0)
    try:
        ops.ffn_set_sync_spin_limit(0)
        rt.execute(1, x, sel, w, None)
    finally:
        ops.ffn_set_sync_spin_limit(None)
    with pytest.raises(RuntimeError, match='gave up'):
        rt.close()
