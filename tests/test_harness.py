"""CPU tier: the serving metrics and the repeat protocol of the generate harness.

The metrics are pinned by hand-computed values of the reference's definitions
(scripts/run_cell.py:150-154, README.md:127-134): TTFT = first - release, TPOT = (end - first)
/ (steps - 1), E2E = end - release, TPS = requests * steps / E2E.  The summary is pinned by
hand-computed means and sample standard deviations.  The protocol runs a tiny HF model on the
CPU (its own experts, no hooks) with a stand-in runtime that counts resets; the greedy tokens
must equal HF's own ``generate``.
"""
import time

import numpy as np
import pytest
import torch

from test_model_loader import tiny_model, tiny_qwen3_config


def test_serving_metrics_hand_computed():
    from ferry_amd.harness import serving_metrics
    res = dict(release_ns=1_000_000_000, first_ns=1_250_000_000, end_ns=2_510_000_000)
    m = serving_metrics(res, requests=16, steps=64)
    assert m['TTFT'] == pytest.approx(0.25, abs=1e-12)
    assert m['TPOT'] == pytest.approx(0.02, abs=1e-12)        # 1.26 s over 63 intervals
    assert m['E2E'] == pytest.approx(1.51, abs=1e-12)
    assert m['TPS'] == pytest.approx(678.1456953642384, rel=1e-12)   # 1024 tokens / 1.51 s
    one = serving_metrics(dict(release_ns=0, first_ns=5_000_000, end_ns=5_000_000), 2, 1)
    assert one == dict(TTFT=0.005, TPOT=0.0, E2E=0.005, TPS=400.0)


def test_summarize_mean_and_sample_std():
    from ferry_amd.harness import summarize

    def rec(phase, ttft, tps):
        return dict(phase=phase, TTFT=ttft, TPOT=0.5, E2E=2.0, TPS=tps)
    records = [rec('warmup', 9.0, 1.0), rec('discard', 8.0, 2.0), rec('target', 0.1, 100.0),
               rec('target', 0.2, 110.0), rec('target', 0.3, 120.0)]
    s = summarize(records)
    assert s['n'] == 3
    assert s['TTFT']['mean'] == pytest.approx(0.2) and s['TTFT']['std'] == pytest.approx(0.1)
    assert s['TPS']['mean'] == pytest.approx(110.0) and s['TPS']['std'] == pytest.approx(10.0)
    assert s['TPOT'] == dict(mean=0.5, std=0.0) and s['E2E'] == dict(mean=2.0, std=0.0)
    assert summarize([rec('target', 0.4, 5.0)])['TTFT'] == dict(mean=0.4, std=0.0)
    with pytest.raises(ValueError):
        summarize(records[:2])


class _H2D:
    def __init__(self):
        self.copies = 0
        self.synchronized = 0

    def synchronize(self):
        self.synchronized += 1


class _Transport:
    dispatch_bytes = combine_bytes = 0


class _Runtime:
    """Stand-in for OffloadRuntime: the counters the protocol reads, and reset counting."""

    def __init__(self):
        self.h2d, self.transport = _H2D(), _Transport()
        self.resets = 0
        self.fetches_per_rank = np.zeros(1, np.int64)
        self.decode_fetches_per_rank = np.zeros(1, np.int64)
        self.serial_wait_ns = 0

    def reset(self):
        self.resets += 1
        self.h2d.copies += 3          # distinct per run, so the records show which run is which
        self.fetches_per_rank[:] = self.resets


def test_run_repeats_protocol_and_greedy_tokens():
    from ferry_amd.harness import run_repeats, summarize
    model = tiny_model(tiny_qwen3_config(vocab_size=97), seed=4)
    g = torch.Generator().manual_seed(1)
    warm = torch.randint(0, 97, (2, 5), generator=g)
    target = torch.randint(0, 97, (3, 9), generator=g)
    rt = _Runtime()
    seen = []
    t0 = time.perf_counter_ns()
    recs = run_repeats(model, rt, warm, target, steps=4, repeats=3, discard=1,
                       release_delay_s=0.01, log=seen.append)
    assert [r['phase'] for r in recs] == ['warmup', 'discard', 'target', 'target', 'target']
    assert [r['repeat'] for r in recs] == [0, 1, 2, 3, 4] and seen == recs
    assert rt.resets == 5 and rt.h2d.synchronized == 5
    assert [r['h2d_copies'] for r in recs] == [3, 6, 9, 12, 15]
    assert [r['fetches_per_rank'] for r in recs] == [[1], [2], [3], [4], [5]]
    assert [r['requests'] for r in recs] == [2, 3, 3, 3, 3]
    before = t0
    for r in recs:
        # each run is released 10 ms after it is called, after the previous run ended
        assert r['release_ns'] >= before + 10_000_000
        assert r['release_ns'] <= r['first_ns'] <= r['end_ns']
        before = r['end_ns']
        assert r['output_tokens'] == 4 and r['TTFT'] == (r['first_ns'] - r['release_ns']) / 1e9
        assert r['E2E'] >= r['TTFT'] and r['TPS'] == pytest.approx(r['requests'] * 4 / r['E2E'])
        assert r['peak_allocated_bytes'] is None               # CPU run
    # greedy tokens: HF's own generate on the same prompts
    with torch.no_grad():
        want = model.generate(target, attention_mask=torch.ones_like(target), max_new_tokens=4,
                              do_sample=False, min_new_tokens=4)[:, target.shape[1]:]
    for r in recs[1:]:
        assert r['tokens'] == want.tolist()
    s = summarize(recs)
    assert s['n'] == 3
    with pytest.raises(ValueError):
        run_repeats(model, rt, warm, target, steps=2, repeats=0)
