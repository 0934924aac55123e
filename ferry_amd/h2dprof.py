"""H2D expert-fetch profiler for one GPU, and the topology file the runtime's Topology loads.

Reference: scripts/profile_h2d.py:27-45 (``measure``: expert-sized pinned-to-device copies
issued back to back on a stream held by a GPU spin until all are enqueued, timed with events,
median over repeats) and scripts/build_quota_lut.py:21-47 (domains + the Step-2 quota table,
written as the JSON that ferry/quota.py:80-90 reads).  With one GPU there is one bandwidth
domain (mask 1) and the quota of m missing experts is [m].

Three rates are measured, all in GiB/s like the reference's file:
  * ``engine``: one fetch call through this package's H2D engine in its default mode
    (``hipMemcpyAsync`` on two DMA streams), which is how ``OffloadRuntime`` copies by default;
    this is the domain's ``gib_per_s``;
  * ``kernel``: the engine's copy kernel (one launch for all rows; ``OffloadRuntime(copy=
    'kernel')`` on decode-sized calls);
  * ``single_stream``: one ``copy_`` per expert on one stream, the reference's pattern.

    python -m ferry_amd.h2dprof --output topology/mi355x_qwen3.json [--model-path DIR]
"""
import argparse
import json
import statistics
import sys
import time
from pathlib import Path

import torch

SPIN_CYCLES = 20_000_000   # GPU spin that holds the copy stream until every copy is enqueued


def _time_engine(engine, slots, keys, spin_cycles):
    s = engine.stream
    with torch.cuda.stream(s):
        torch.cuda._sleep(spin_cycles)
        start = torch.cuda.Event(enable_timing=True)
        start.record(s)
    engine.fetch(slots, keys)
    end = torch.cuda.Event(enable_timing=True)
    end.record(s)
    end.synchronize()
    return start.elapsed_time(end) / 1e3


def _time_single_stream(stream, pool, cache, copies, spin_cycles):
    with torch.cuda.stream(stream):
        torch.cuda._sleep(spin_cycles)
        start = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for i in range(copies):
            cache[i % cache.shape[0]].copy_(pool[i % pool.shape[0]], non_blocking=True)
        end = torch.cuda.Event(enable_timing=True)
        end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / 1e3


def measure(expert_bytes, copies=64, repeats=5, slots=None, pool_rows=8, device=0,
            spin_cycles=SPIN_CYCLES):
    """Median GiB/s of ``copies`` back-to-back expert copies: dict(engine, kernel, single_stream,
    samples); kernel is None when the pool cannot use the copy kernel."""
    from .h2d import KERNEL, H2DEngine
    from .hostmem import pinned_empty
    torch.cuda.set_device(device)
    elements = expert_bytes // 2
    slots = copies if slots is None else slots   # distinct slots: one fetch call, one launch
    pool = pinned_empty((pool_rows, elements), torch.bfloat16)
    pool.copy_(torch.randn((pool_rows, elements)).to(torch.bfloat16))
    cache = torch.empty((slots, elements), dtype=torch.bfloat16, device=device)
    engine = H2DEngine(cache, pool)
    kern = H2DEngine(cache, pool)
    if kern.kernel_ok:
        kern.engine = KERNEL
    else:
        kern.close()
        kern = None
    stream = torch.cuda.Stream(device=device)
    idx = list(range(copies))
    slot_seq = [i % slots for i in idx]
    key_seq = [i % pool_rows for i in idx]
    gib = copies * expert_bytes / 2 ** 30
    engines = dict(engine=engine, kernel=kern)
    kinds = ['engine', 'single_stream'] + (['kernel'] if kern is not None else [])
    # warm up every path
    for kind in kinds:
        if kind == 'single_stream':
            _time_single_stream(stream, pool, cache, 8, 0)
        else:
            _time_engine(engines[kind], slot_seq[:8], key_seq[:8], 0)
    samples = {kind: [] for kind in kinds}
    for rep in range(repeats):
        for kind in kinds[rep % len(kinds):] + kinds[:rep % len(kinds)]:
            if kind == 'single_stream':
                t = _time_single_stream(stream, pool, cache, copies, spin_cycles)
            else:
                t = _time_engine(engines[kind], slot_seq, key_seq, spin_cycles)
            samples[kind].append(gib / t)
    for e in engines.values():
        if e is not None:
            e.synchronize()
            e.close()
    return dict(engine=statistics.median(samples['engine']),
                kernel=statistics.median(samples['kernel']) if kern is not None else None,
                single_stream=statistics.median(samples['single_stream']), samples=samples)


def topology_document(measured, expert_bytes, experts, model_type=None, device=0):
    """The world-1 topology file: one domain (this GPU) and quota_lut[m] = [m], m = 0..experts."""
    return dict(world=1, physical_gpus=[device], expert_bytes=int(expert_bytes),
                model_type=model_type,
                domains=[dict(gpus=[0], mask=1, gib_per_s=float(measured['engine']),
                              per_gpu_gib_per_s=[float(measured['engine'])])],
                quota_lut=[[m] for m in range(experts + 1)],
                measured=dict(engine_gib_per_s=measured['engine'],
                              kernel_gib_per_s=measured['kernel'],
                              single_stream_gib_per_s=measured['single_stream'],
                              samples=measured['samples']))


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split('\n')[0])
    p.add_argument('--model-path', help='HF model directory: size the copies like one expert')
    p.add_argument('--expert-bytes', type=int, default=9_437_184,
                   help='copy size when no model is given (Qwen3-30B-A3B expert: 9,437,184 B)')
    p.add_argument('--experts', type=int, default=128, help='quota table length - 1 (no model)')
    p.add_argument('--output', required=True)
    p.add_argument('--copies', type=int, default=64)
    p.add_argument('--repeats', type=int, default=5)
    a = p.parse_args(argv)
    model_type = None
    if a.model_path:
        from .model import read_spec
        spec = read_spec(a.model_path)
        a.expert_bytes, a.experts, model_type = spec.expert_bytes, spec.experts, spec.model_type
    t0 = time.time()
    res = measure(a.expert_bytes, a.copies, a.repeats)
    doc = topology_document(res, a.expert_bytes, a.experts, model_type)
    out = Path(a.output)
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text(json.dumps(doc, indent=1) + '\n')
    print(f'H2D {a.expert_bytes} B copies x {a.copies}, median of {a.repeats}: engine '
          f'{res["engine"]:.2f} GiB/s, copy kernel {res["kernel"] or 0:.2f} GiB/s, single stream '
          f'{res["single_stream"]:.2f} GiB/s ({time.time() - t0:.1f} s); wrote {out}', flush=True)
    return doc


if __name__ == '__main__':
    main(sys.argv[1:])
