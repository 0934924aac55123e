"""CPU tier: the C ABI library loads and exports every declared symbol; the host-side product
code (C++ planner, Python API mirror) matches the oracle.  No GPU compute is called here."""
import ctypes
import re
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import pytest

from oracle.history import GateHistoryRef, frequency_rows
from oracle.policy import PlannerRef

ROOT = Path(__file__).resolve().parents[1]


def _declared_symbols():
    text = (ROOT / 'include' / 'ferry_amd.h').read_text()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'\b(ferry_[a-z0-9_]+)\s*\(', text)))


def test_library_exports_every_declared_symbol():
    from ferry_amd._lib import LIB_PATH, SIGNATURES
    handle = ctypes.CDLL(str(LIB_PATH))
    declared = _declared_symbols()
    assert len(declared) >= 20
    for name in declared:
        assert hasattr(handle, name), f'{name} declared in include/ferry_amd.h but not exported'
    bound = {n for n, _, _ in SIGNATURES}
    assert set(declared) <= bound | {'ferry_timing_enable', 'ferry_timing_summary'}, \
        sorted(set(declared) - bound)


def test_abi_version_and_errors():
    from ferry_amd._lib import last_error, lib
    L = lib()
    assert L.ferry_abi_version() == 6
    # ready words of the history kernel: one per workgroup of 4096 IDs, plus the history one
    assert [L.ferry_history_ready_words(t, 8) for t in (0, 16, 512, 513, 65536)] == [1, 2, 2, 3, 129]
    assert L.ferry_history_ready_words(-1, 8) == -1 and L.ferry_history_ready_words(4, 0) == -1
    assert L.ferry_history_update(None, 1, 8, 128, 128, 0, None, None, None, None, None, None,
                                  None, 0, None) != 0
    assert L.ferry_h2d_wait_ready(None, None, None, 1, 0) != 0
    # argument validation fails before any device work
    assert L.ferry_router_topk(None, 0, 4, 300, 8, 1, 1.0, 1, None, None, None, None, None) != 0
    assert 'experts' in last_error()
    assert L.ferry_layout(None, None, 4, 20, 8, None, None, None, None, None, None, None, 0, None) != 0
    assert L.ferry_combine(None, None, 1, 1, 12, None, None) != 0
    assert 'hidden' in last_error()
    assert L.ferry_expert_ffn(None, 1, 100, 128, None, 1, 1, None, None, None, None, None, 0, None,
                              1, 1, 0, None, None, None, 0, 3, None) != 0
    # the tiled down projection needs hidden % 256 == 0 once an expert exceeds the skinny size
    assert L.ferry_expert_ffn(None, 1, 384, 128, None, 100, 1, None, None, None, None, None, 1, None,
                              1, 100, 0, None, None, None, 0, 3, None) != 0
    assert 'multiple of 256' in last_error()
    # the lower row bound may not exceed the upper one
    assert L.ferry_expert_ffn(None, 1, 256, 128, None, 100, 1, None, None, None, None, None, 1, None,
                              1, 10, 11, None, None, None, 0, 3, None) != 0
    assert 'min_rows_per_expert' in last_error()
    # weights are addressed with 32-bit offsets inside an expert's cache row
    assert L.ferry_expert_ffn(None, 1, 65536, 32768, None, 100, 1, None, None, None, None, None,
                              1, None, 1, 10, 0, None, None, None, 0, 3, None) != 0
    assert '4 GiB' in last_error()
    # row counts must lie within the row bounds (checked on the host before any device work;
    # the pointers are placeholders that are never dereferenced)
    import numpy as np
    el, so = np.arange(3, dtype=np.int32), np.arange(3, dtype=np.int32)
    rows = np.array([5, 70, 2], dtype=np.int32)
    fake = 4096
    assert L.ferry_expert_ffn(fake, 3, 256, 128, fake, 100, 1, fake, fake, fake, fake,
                              el.ctypes.data, 3, so.ctypes.data, 3, 64, 0, rows.ctypes.data,
                              fake, fake, 0, 3, None) != 0
    assert 'list_rows[1] = 70' in last_error()
    assert L.ferry_combine_add(None, None, 4, 2, 64, None, None, None) != 0
    assert 'addend' in last_error()


@dataclass(frozen=True)
class _Spec:
    layers: int
    experts: int


def test_product_planner_matches_oracle_traces():
    from ferry_amd.policy import Controller, _choose_slot, layer_slots
    from ferry_amd.quota import Topology
    rng = np.random.default_rng(1)
    for trial in range(12):
        L, E = int(rng.integers(1, 5)), int(rng.integers(2, 40))
        cap = int(rng.integers(1, 2 * E))
        ctl = Controller(_Spec(L, E), [cap], 'ferry', Topology.uniform(1, E))
        ref = PlannerRef(L, E, cap)
        for ev in range(80):
            layer = int(rng.integers(0, L))
            k = int(rng.integers(1, min(E, 8) + 1))
            T = int(rng.integers(1, 6))
            sel = np.stack([rng.choice(E, k, replace=False) for _ in range(T)])
            gs = (rng.integers(0, 5, E) / 4).astype(np.float32)
            try:
                f_ref, d_ref = ref.plan(ev, layer, sel, gs)
            except AssertionError:
                f_ref = None
            try:
                f, d, counts = ctl.plan(ev, layer, sel, np.zeros(T, np.int64), gs)
            except AssertionError:
                f = None
            assert (f is None) == (f_ref is None)
            if f is None:
                break
            assert np.array_equal(f, f_ref) and np.array_equal(d, d_ref)
            assert counts.tolist() == [len(f)]
            assert np.array_equal(ctl.slots[0], ref.slots)
            assert np.array_equal(ctl.owner, ref.owner) and np.array_equal(ctl.last, ref.last)
            assert np.array_equal(layer_slots(ctl.slots[0], cap, layer, E), ref.layer_slots(layer))
            active = np.zeros(E, np.uint8)
            active[np.unique(sel)] = 1
            from oracle.native import lib as olib
            want = olib().oracle_choose_slot(layer, active.ctypes.data, ref.slots.ctypes.data, cap,
                                             ref.last.ctypes.data, ref.scores.ctypes.data, E)
            assert _choose_slot(0, layer, active, ctl.slots, [cap], ctl.last, ctl.scores, E) == want


def test_product_planner_golden_trace():
    from ferry_amd.policy import Controller
    from ferry_amd.quota import Topology
    d = np.load(ROOT / 'tests' / 'golden' / 'planner.npz')
    L, E, cap = int(d['layers']), int(d['experts']), int(d['cap'])
    ctl = Controller(_Spec(L, E), [cap], 'ferry', Topology.uniform(1, E))
    off = foff = 0
    for ev, T in enumerate(d['sizes']):
        sel = d['selected'][off:off + T]
        off += T
        f, _, _ = ctl.plan(ev, ev % L, sel, np.zeros(T, np.int64), d['gate_scores'][ev])
        n = int(d['nfetch'][ev])
        assert np.array_equal(f, d['fetches'][foff:foff + n])
        foff += n
    assert np.array_equal(ctl.slots[0], d['final_slots'])


def test_fused_plan_fetch_matches_oracle_traces():
    """ferry_plan_fetch (uint8 IDs and float32 scores from raw host pointers, plan only when no
    fetch engine is given) makes the oracle's decisions and state updates, and returns each
    expert's demand."""
    from ferry_amd.policy import Controller
    from ferry_amd.quota import Topology
    rng = np.random.default_rng(7)
    for trial in range(8):
        L, E = int(rng.integers(1, 4)), int(rng.integers(2, 200))
        cap = int(rng.integers(1, 2 * E))
        ctl = Controller(_Spec(L, E), [cap], 'ferry', Topology.uniform(1, E))
        ref = PlannerRef(L, E, cap)
        for ev in range(60):
            layer = int(rng.integers(0, L))
            k = int(rng.integers(1, min(E, 8) + 1))
            T = int(rng.integers(1, 6))
            sel = np.stack([rng.choice(E, k, replace=False) for _ in range(T)])
            gs = (rng.integers(0, 5, E) / 4).astype(np.float32)
            try:
                f_ref, _ = ref.plan(ev, layer, sel, gs)
            except AssertionError:
                f_ref = None
            ids = np.ascontiguousarray(sel.reshape(-1).astype(np.uint8))
            try:
                f, counts = ctl.plan_fetch(ev, layer, ids.ctypes.data, T, k, gs.ctypes.data, None)
            except AssertionError:
                f = None
            assert (f is None) == (f_ref is None)
            if f is None:
                break
            assert np.array_equal(f, f_ref) and counts.tolist() == [len(f)]
            assert np.array_equal(ctl.demand, np.bincount(sel.reshape(-1), minlength=E))
            assert np.array_equal(ctl.slots[0], ref.slots)
            assert np.array_equal(ctl.owner, ref.owner) and np.array_equal(ctl.last, ref.last)


def test_planner_nan_scores_match_oracle():
    """Keys whose layer score is NaN are never evicted (every comparison with NaN is false in
    the reference's scan); the planner's one-sort slot choice matches the oracle's per-miss
    scan on traces with NaN scores, including the calls where no slot is left."""
    from ferry_amd.policy import Controller
    from ferry_amd.quota import Topology
    rng = np.random.default_rng(7)
    errors = 0
    for trial in range(40):
        L, E = int(rng.integers(1, 5)), int(rng.integers(2, 40))
        cap = int(rng.integers(1, 2 * E))
        ctl = Controller(_Spec(L, E), [cap], 'ferry', Topology.uniform(1, E))
        ref = PlannerRef(L, E, cap)
        for ev in range(40):
            layer = int(rng.integers(0, L))
            k = int(rng.integers(1, min(E, 6) + 1))
            T = int(rng.integers(1, 6))
            sel = np.stack([rng.choice(E, k, replace=False) for _ in range(T)])
            gs = (rng.integers(0, 4, E) / 4).astype(np.float32)
            gs[rng.random(E) < 0.3] = np.nan
            try:
                f_ref, _ = ref.plan(ev, layer, sel, gs)
            except AssertionError:
                f_ref = None
            ids = np.ascontiguousarray(sel.reshape(-1).astype(np.uint8))
            try:
                f, _ = ctl.plan_fetch(ev, layer, ids.ctypes.data, T, k, gs.ctypes.data, None)
            except AssertionError:
                f = None
            assert (f is None) == (f_ref is None), (trial, ev)
            if f is None:
                errors += 1
                break
            assert np.array_equal(f, f_ref) and np.array_equal(ctl.slots[0], ref.slots)
    assert errors > 0


def test_product_planner_overflow_raises_assertion():
    from ferry_amd.policy import Controller
    from ferry_amd.quota import Topology
    ctl = Controller(_Spec(1, 8), [2], 'ferry', Topology.uniform(1, 8))
    with pytest.raises(AssertionError, match='admission capacity'):
        ctl.plan(0, 0, np.array([[0, 1, 2]]), np.zeros(1, np.int64), np.zeros(8, np.float32))


def test_planner_rejects_invalid_routing_ids():
    """An expert ID outside [0, E) or repeated within a token is rejected with RuntimeError
    before any planner state changes, through both the int64 and the fused uint8 entry points
    (0xFF is what the history kernel writes for an out-of-range ID)."""
    from ferry_amd.policy import Controller
    from ferry_amd.quota import Topology
    E = 16
    ctl = Controller(_Spec(2, E), [4], 'ferry', Topology.uniform(1, E))
    ctl.plan(0, 0, np.array([[1, 2], [3, 1]]), np.zeros(2, np.int64), np.zeros(E, np.float32))
    state = (ctl.slots.copy(), ctl.owner.copy(), ctl.last.copy(), ctl.scores.copy())
    gs = np.ones(E, np.float32)
    for bad in ([[1, 16]], [[-1, 2]], [[5, 5]], [[0, 1], [2, 2]]):
        with pytest.raises(RuntimeError, match='out of range|repeated'):
            ctl.plan(1, 1, np.array(bad), np.zeros(len(bad), np.int64), gs)
    for bad in ([1, 0xFF], [7, 7]):
        ids = np.array(bad, np.uint8)
        with pytest.raises(RuntimeError, match='out of range|repeated'):
            ctl.plan_fetch(1, 1, ids.ctypes.data, 1, 2, gs.ctypes.data, None)
    for a, b in zip(state, (ctl.slots, ctl.owner, ctl.last, ctl.scores)):
        assert np.array_equal(a, b)
    # the same state still plans valid routing
    f, _, _ = ctl.plan(1, 1, np.array([[0, 5]]), np.zeros(1, np.int64), gs)
    assert f[:, 1].tolist() == [E + 0, E + 5]


def test_world_gt_1_rejected():
    from ferry_amd.policy import Controller
    from ferry_amd.quota import Topology
    with pytest.raises(NotImplementedError):
        Topology.uniform(2, 8)
    with pytest.raises(NotImplementedError):
        Controller(_Spec(1, 8), [2, 2], 'ferry', Topology.uniform(1, 8))


def test_host_gate_history_matches_oracle():
    from ferry_amd.metadata import GateHistory
    from ferry_amd.metadata import frequency_rows as rows_product
    rng = np.random.default_rng(4)
    L, E, W = 2, 24, 32
    a, b = GateHistory(L, E, W), GateHistoryRef(L, E, W)
    for step in range(40):
        layer = step % L
        T = int(rng.integers(1, 50))
        sel = np.stack([rng.choice(E, 3, replace=False) for _ in range(T)])
        assert np.array_equal(rows_product(sel, E, W), frequency_rows(sel, E, W))
        a.update(layer, rows_product(sel, E, W))
        b.update(layer, frequency_rows(sel, E, W))
        assert np.array_equal(a.scores(layer), b.scores(layer))
    # probability rows (the reference's Eq. 12 score) go through the same ring
    p = rng.random((7, E)).astype(np.float32)
    a.update(0, p)
    b.update(0, p.astype(np.float64))
    assert np.array_equal(a.scores(0), b.scores(0))


def test_model_spec_cache_budget_and_read_spec(tmp_path):
    import json
    from ferry_amd.model import DEEPSEEK_V2_LITE, QWEN3_30B_A3B, read_spec
    assert QWEN3_30B_A3B.cache_slots(0.30, 1) == [1843]
    assert DEEPSEEK_V2_LITE.cache_slots(0.30, 1) == [499]
    assert QWEN3_30B_A3B.expert_bytes == 9437184 and DEEPSEEK_V2_LITE.expert_bytes == 17301504
    cfg = dict(model_type='qwen3_moe', num_hidden_layers=48, num_experts=128, num_experts_per_tok=8,
               hidden_size=2048, moe_intermediate_size=768, decoder_sparse_step=1, mlp_only_layers=[])
    (tmp_path / 'config.json').write_text(json.dumps(cfg))
    assert read_spec(tmp_path) == QWEN3_30B_A3B
    cfg = dict(model_type='deepseek_v2', num_hidden_layers=27, n_routed_experts=64, num_experts_per_tok=6,
               hidden_size=2048, moe_intermediate_size=1408, first_k_dense_replace=1, moe_layer_freq=1)
    (tmp_path / 'config.json').write_text(json.dumps(cfg))
    assert read_spec(tmp_path) == DEEPSEEK_V2_LITE


def test_workload_generators_are_seeded():
    from ferry_amd import workloads
    a = workloads.zipf_log_bias(128, 1.1, np.random.default_rng(1))
    b = workloads.zipf_log_bias(128, 1.1, np.random.default_rng(1))
    assert np.array_equal(a, b)
    p = np.exp(a.astype(np.float64))
    assert abs(p.sum() - 1) < 1e-5 and np.isclose(p.max() / p.min(), 128 ** 1.1, rtol=1e-3)
    w = workloads.QWEN3_DECODE_LOOP
    sel, logits = workloads.temporal_routing(w, steps=3, tokens=4, seed=0)
    assert sel.shape == (3, 48, 4, 8)
    for row in sel.reshape(-1, 8):
        assert len(set(row.tolist())) == 8


def test_bench_rejects_more_than_one_gpu():
    import subprocess
    import sys
    r = subprocess.run([sys.executable, str(ROOT / 'bench.py'), '--gpus', '2'], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 2 and 'one GPU' in r.stdout


def test_topology_file_round_trip(tmp_path):
    """The world-1 topology document the H2D profiler writes loads into Topology like the
    reference's file (ferry/quota.py:80-90): one domain, quota_lut[m] = [m]; a file for another
    world size or a table too short for the model is rejected."""
    import json
    from ferry_amd.h2dprof import topology_document
    from ferry_amd.quota import Topology
    measured = dict(engine=52.5, kernel=55.0, single_stream=44.0,
                    samples=dict(engine=[52.5], kernel=[55.0], single_stream=[44.0]))
    doc = topology_document(measured, 9437184, 128, 'qwen3_moe')
    path = tmp_path / 'topo.json'
    path.write_text(json.dumps(doc))
    topo = Topology(path, 1, 128)
    assert topo.masks.tolist() == [1] and abs(topo.seconds[0] - 1 / 52.5) < 1e-15
    assert topo.lut.shape == (129, 1) and topo.lut[:, 0].tolist() == list(range(129))
    uni = Topology.uniform(1, 128)
    assert np.array_equal(uni.lut, topo.lut) and uni.masks.tolist() == [1]
    with pytest.raises(ValueError, match='rebuild'):
        Topology(path, 1, 200)
    doc['world'] = 2
    path.write_text(json.dumps(doc))
    with pytest.raises(ValueError, match='2 GPUs'):
        Topology(path, 1, 128)


def _unpack_numpy(buf, n):
    """Independent decoder of a packed row back to uint16 bf16 bits: header, sign|mantissa
    plane, two bit planes of 2-bit exponent codes against table T1 (3 = escape), the prefix
    table, the escapes' 2-bit codes against table T2 (3 = next level), their 4-bit codes against
    the window [base3, base3 + 14] (15 = list) and the (index, exponent) list."""
    magic = int(np.frombuffer(buf[:4], dtype=np.uint32)[0])
    assert magic == 0x3350414b
    t1 = np.frombuffer(buf[4:7], dtype=np.uint8).astype(np.uint16)
    t2 = np.frombuffer(buf[7:10], dtype=np.uint8).astype(np.uint16)
    base3 = int(buf[10])
    values, esc1, esc2, esc3, nbytes = (int(x) for x in np.frombuffer(buf[16:56], dtype=np.uint64))
    assert values == n and nbytes == len(buf) and nbytes % 256 == 0
    a = np.frombuffer(buf[64:64 + n], dtype=np.uint8).astype(np.uint16)
    off = 64 + n
    bits = [np.unpackbits(np.frombuffer(buf[off + k * (n // 8):off + (k + 1) * (n // 8)],
                                        dtype=np.uint8), bitorder='little') for k in range(2)]
    codes = bits[0].astype(np.uint16) | (bits[1].astype(np.uint16) << 1)
    off += 2 * (n // 8)
    nb = -(-n // 8192)
    pre = np.frombuffer(buf[off:off + 12 * (nb + 1)], dtype=np.uint32).reshape(nb + 1, 3)
    off += 12 * (nb + 1)
    esc = np.flatnonzero(codes == 3)
    assert len(esc) == esc1
    stream2 = np.unpackbits(np.frombuffer(buf[off:off + 4 * (-(-esc1 // 16))], dtype=np.uint8),
                            bitorder='little').reshape(-1, 2)
    c2 = (stream2[:, 0] | (stream2[:, 1] << 1)).astype(np.uint16)
    assert not c2[esc1:].any()
    c2 = c2[:esc1]
    off += 4 * (-(-esc1 // 16))
    esc_2 = esc[c2 == 3]
    assert len(esc_2) == esc2
    nib = np.frombuffer(buf[off:off + 4 * (-(-esc2 // 8))], dtype=np.uint8)
    c3 = np.empty(2 * len(nib), np.uint16)
    c3[0::2] = nib & 0xF
    c3[1::2] = nib >> 4
    assert not c3[esc2:].any()
    c3 = c3[:esc2]
    off += 4 * (-(-esc2 // 8))
    idx = np.frombuffer(buf[off:off + 4 * esc3], dtype=np.uint32)
    exps = np.frombuffer(buf[off + 4 * esc3:off + 5 * esc3], dtype=np.uint8).astype(np.uint16)
    assert np.all(np.diff(idx.astype(np.int64)) > 0)
    assert np.array_equal(esc_2[c3 == 15], idx)
    # the prefix table counts each level's escapes before each block
    marks = np.arange(nb + 1) * 8192
    assert np.array_equal(pre[:, 0], np.searchsorted(esc, marks))
    assert np.array_equal(pre[:, 1], np.searchsorted(esc_2, marks))
    assert np.array_equal(pre[:, 2], np.searchsorted(idx, marks))
    assert not buf[off + 5 * esc3:].strip(b'\0')   # zero tail
    e = np.empty(n, np.uint16)
    lvl1 = codes < 3
    e[lvl1] = t1[codes[lvl1]]
    lvl2 = c2 < 3
    e[esc[lvl2]] = t2[c2[lvl2]]
    e[esc_2] = base3 + c3
    e[idx] = exps
    return ((a & 0x80) << 8) | (e << 7) | (a & 0x7F)


def _heavy_block(row, block, count, g):
    """A copy of a bf16 row whose 8192-value block `block` holds `count` values spread over
    ~160 binades: most of them beyond both exponent tables and the window (list entries)."""
    import torch
    out = row.clone()
    k = torch.randint(20, 100, (count,), generator=g).float()
    sign = torch.where(torch.rand(count, generator=g) < 0.5, -1.0, 1.0)
    big = torch.rand(count, generator=g) < 0.5
    vals = sign * torch.exp2(torch.where(big, k, -k)) * 1.25
    out[8192 * block:8192 * block + count] = vals.to(torch.bfloat16)
    return out


def test_pack_row_round_trip():
    """The lossless row packing of the H2D link: packed rows decode (here with an independent
    numpy decoder) to the exact bf16 bits -- Gaussian weights at a length that is a whole number
    of 8192-value blocks and at a ragged one, special values (+-0, +-inf, NaN, denormals, huge
    and tiny values: escapes at every level), values spread over 64 binades (hundreds of
    list entries per block) -- and a row of random bits, which would not shrink, is left
    raw."""
    import torch
    from ferry_amd._lib import lib
    g = torch.Generator().manual_seed(3)
    n = 1 << 16
    gauss = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)
    ragged = (torch.randn(3 * 8192 + 96, generator=g) * 0.5).to(torch.bfloat16)
    special = gauss.clone()
    vals = torch.tensor([0.0, -0.0, float('inf'), -float('inf'), float('nan'), 1e-40, -3e-39,
                         1e30, -2e-30, 7.0], dtype=torch.float32).to(torch.bfloat16)
    pos = torch.randperm(n, generator=g)[:2000]
    special[pos] = vals[torch.arange(2000) % len(vals)]
    wide = (torch.randn(n, generator=g) * torch.exp2(torch.randint(-32, 32, (n,), generator=g)
                                                     .float())).to(torch.bfloat16)
    heavy = _heavy_block(gauss, 2, 600, g)
    for row, bound in ((gauss, 0.68), (ragged, 0.72), (special, 0.9), (heavy, 0.75), (wide, 1.0)):
        m = row.numel()
        u16 = row.view(torch.int16).numpy().view(np.uint16).copy()
        nb = ctypes.c_int64()
        st = lib().ferry_pack_row(u16.ctypes.data, m, None, 0, ctypes.byref(nb))
        if row is wide and st == 1:
            continue
        assert st == 0
        buf = np.zeros(nb.value, np.uint8)
        assert lib().ferry_pack_row(u16.ctypes.data, m, buf.ctypes.data, nb.value,
                                    ctypes.byref(nb)) == 0
        assert nb.value < bound * 2 * m
        if row is heavy:   # more list entries in one block than a workgroup stages
            assert int(np.frombuffer(buf[40:48].tobytes(), np.uint64)[0]) > 300
        assert np.array_equal(_unpack_numpy(buf.tobytes(), m), u16)
    rnd = np.random.default_rng(0).integers(0, 1 << 16, n, dtype=np.uint16)
    nb = ctypes.c_int64()
    assert lib().ferry_pack_row(rnd.ctypes.data, n, None, 0, ctypes.byref(nb)) == 1
    assert lib().ferry_pack_row(rnd.ctypes.data, 100, None, 0, ctypes.byref(nb)) == 2
    assert lib().ferry_pack_row(rnd.ctypes.data, 48, None, 0, ctypes.byref(nb)) == 2
