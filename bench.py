"""Benchmark of the per-GPU MoE hot path on one MI355X.

Default workload (the headline metric): the Qwen3-30B-A3B-shaped MoE layer in decode --
16 tokens per step, 128 experts top-8 (renormalised softmax), hidden 2048, SwiGLU
intermediate 768, bf16, a 38-slot expert cache with the other experts in pinned host memory,
router logits N(0, 1) + log Zipf(1.1) popularity (seed 1).  One step = one layer call:
router kernel -> device history + D2H of the IDs -> host planner -> H2D fetch of the misses
-> layout -> grouped SwiGLU (resident experts first) -> combine.

The timed pass runs without instrumentation; a second pass over the same stream (from an empty
cache again) collects per-launch kernel times, fetch events and host phase times.

Also reported on the same line:
  * roofline: the decode expert FFN phase-1 kernel (ffn_up_skinny: gate/up projection +
    SwiGLU, 2/3 of the expert bytes), achieved GB/s on its algorithmic bytes vs 8 TB/s,
    from HIP events around each launch on the compute stream; traffic from the committed
    FETCH_SIZE / WRITE_SIZE profile of that kernel;
  * prefill: the Qwen3-shaped 8192-token layer (experts resident), tokens/s and MFMA
    utilisation of the grouped GEMMs vs 2.5 PFLOP/s;
  * prefill_deepseek: the DeepSeek-V2-Lite-shaped 65,536-token layer with its two shared
    experts (experts resident), the same figures;
  * fetch: H2D GB/s of the expert copies and the fraction hidden behind compute;
  * cpu_baseline: the oracle's torch-CPU restatement of the reference op order on the host
    cores, on a bounded sample of the same decode stream.
With --decode-loop: the 48-layer Qwen3 decode loop (1024-token prefill, then 64-token steps,
pooled cache of 1,843 slots) as a decode_loop block.
"""
import argparse
import json
import os
import sys
import time
from dataclasses import replace
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
PCIE_PEAK_GBS = 64.0


TRAFFIC_PROFILE = ROOT / 'profiles' / 'ffn_up_skinny_decode_qwen3_t16_hbm_traffic.md'


def traffic_ratio():
    """HBM traffic / algorithmic bytes of ffn_up_skinny, from the committed counter profile
    (FETCH_SIZE + WRITE_SIZE, each scaled by a copy kernel of known size), or None."""
    try:
        for line in TRAFFIC_PROFILE.read_text().splitlines():
            if line.startswith('traffic_over_algorithmic'):
                return float(line.split('=')[1])
    except OSError:
        pass
    return None


def parse():
    p = argparse.ArgumentParser()
    p.add_argument('--gpus', type=int, default=1)
    p.add_argument('--steps', type=int, default=300)
    p.add_argument('--warmup', type=int, default=30)
    p.add_argument('--prefill-reps', type=int, default=10)
    p.add_argument('--no-prefill', action='store_true')
    p.add_argument('--no-cpu-baseline', action='store_true')
    p.add_argument('--cpu-seconds', type=float, default=15.0)
    p.add_argument('--decode-loop', action='store_true',
                   help='also run the 48-layer decode loop (1024-token prefill, then 64-token '
                        'steps; pooled 30%% cache, W = 128 eviction; a 58 GB pinned pool)')
    p.add_argument('--loop-steps', type=int, default=64)
    p.add_argument('--copy-calibration-mib', type=int, default=0,
                   help='run one plain device copy kernel of this many MiB (read and written) '
                        'before the decode loop: the reference dispatch for scaling HBM byte '
                        'counters (FETCH_SIZE / WRITE_SIZE) in profiler runs')
    return p.parse_args()


def decode_stream(w, steps, device):
    """Feasible steps of the seeded decode stream: (logits bf16 [T, E], x bf16 [T, H])."""
    from ferry_amd import workloads
    logits_gen = workloads.RouterLogits(w, device)
    g = torch.Generator(device=device)
    g.manual_seed(w.seed + 1000)
    out = []
    while len(out) < steps:
        lg = logits_gen.next(0, w.tokens)
        x = torch.randn((w.tokens, w.spec.hidden), generator=g, device=device).to(torch.bfloat16)
        if workloads.feasible_topk_sets(lg.float().cpu().numpy(), w.spec.topk, w.cache_slots):
            out.append((lg, x))
    return out


def run_decode(args, device):
    from ferry_amd import expert_ops as ops
    from ferry_amd import workloads
    from ferry_amd.quota import Topology
    from ferry_amd.runtime import OffloadRuntime
    w = workloads.CONFIGS[2]
    spec = w.spec
    pool = workloads.make_pool(spec, 1, seed=0)
    rt = OffloadRuntime(spec, pool, [w.cache_slots], 'ferry', Topology.uniform(1, spec.experts),
                        timing=False)
    stream = decode_stream(w, args.warmup + args.steps, device)

    def step(lg, x):
        wts, sel = ops.router_topk(lg, spec.topk, renorm=True)
        return rt.execute(0, x, sel, wts, None)

    # pass 1 (the measurement): no instrumentation in the timed region
    for lg, x in stream[:args.warmup]:
        step(lg, x)
    torch.cuda.synchronize()
    copies0 = rt.h2d.copies
    t0 = time.perf_counter()
    for lg, x in stream[args.warmup:]:
        step(lg, x)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    rt.h2d.synchronize()
    copies = rt.h2d.copies - copies0
    # pass 2: the same stream from an empty cache again, with per-launch kernel timing, fetch
    # events and host phase timing (same misses, same launches)
    rt.reset()
    for lg, x in stream[:args.warmup]:
        step(lg, x)
    torch.cuda.synchronize()
    rt.timing = True
    ops.timing_enable(True)
    t2 = time.perf_counter()
    for lg, x in stream[args.warmup:]:
        step(lg, x)
    torch.cuda.synchronize()
    t3 = time.perf_counter()
    ks = dict(rt.kernel_bytes)
    ks['up_launches'], ks['up_ms'] = ops.timing_summary('ffn_up_skinny')
    ks['down_launches'], ks['down_ms'] = ops.timing_summary('ffn_down_skinny')
    ks['kernels'] = {name: ops.timing_summary(name) for name in
                     ('router_kernel', 'history_kernel', 'layout_single', 'ffn_up_skinny',
                      'ffn_down_skinny', 'combine_kernel')}
    fetch_ms, exposed_ms, overlap_ms = rt.fetch_timing()   # reads the launch log: before disabling
    ops.timing_enable(False)
    elapsed = t1 - t0
    tokens = w.tokens * args.steps
    res = dict(workload=w, elapsed=elapsed, instrumented_elapsed=t3 - t2, tokens=tokens,
               copies=copies, kernels=ks, fetch_ms=fetch_ms, exposed_ms=exposed_ms,
               overlap_ms=overlap_ms,
               expert_bytes=spec.expert_bytes, samples=stream[args.warmup:],
               host_ns=dict(rt.host_ns))
    rt.close()
    del pool
    return res


def run_prefill(args, device, config=3):
    """One prefill layer with every expert resident in HBM: the Qwen3-shaped 8192-token layer
    (config 3 shape) or the DeepSeek-V2-Lite-shaped 65,536-token layer with its two shared
    experts (config 4 shape)."""
    from ferry_amd import expert_ops as ops
    from ferry_amd import workloads
    w = workloads.CONFIGS[config]
    spec = replace(w.spec, moe_layers=w.spec.moe_layers[:1])
    E, k, H, I, T = spec.experts, spec.topk, spec.hidden, spec.intermediate, w.tokens
    cache = workloads.expert_rows(range(E), spec.expert_elements, seed=w.seed, device=device)
    logits = workloads.RouterLogits(replace(w, layers=1), device).next(0, T)
    x = workloads.hidden_states(T, H, seed=w.seed + 7, device=device)
    act = torch.empty((T * k, I), dtype=torch.bfloat16, device=device)
    part = torch.empty((T * k, H), dtype=torch.bfloat16, device=device)
    slot_of = np.arange(E, dtype=np.int32)
    Is = w.shared_intermediate
    shared = None
    if Is:
        srow = workloads.shared_rows(1, H, Is, seed=w.seed, device=device)[0]
        shared = ops.SharedExpert(srow, H, Is)
        shared_out = torch.empty((T, H), dtype=torch.bfloat16, device=device)

    def layer():
        wts, sel = ops.router_topk(logits, k, renorm=w.renorm, sorted=w.sorted)
        lay = ops.layout(sel, wts, E)
        ops.expert_ffn(cache, x, lay.w_sorted, lay.starts, lay.rows, lay.cols, np.arange(E), slot_of,
                       H, I, act, part, max_rows=T)
        add = shared(x, out=shared_out) if shared is not None else None
        return ops.combine(part, T, k, H, addend=add), sel

    _, sel = layer()
    torch.cuda.synchronize()
    counts = np.bincount(sel.cpu().numpy().reshape(-1), minlength=E)
    t0 = time.perf_counter()
    for _ in range(args.prefill_reps):
        layer()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ops.timing_enable(True)
    for _ in range(args.prefill_reps):
        layer()
    torch.cuda.synchronize()
    kern = {name: ops.timing_summary(name) for name in
            ('router_kernel', 'layout_count', 'layout_scan', 'layout_scatter', 'ffn_up_skinny',
             'ffn_tiled_up', 'ffn_down_skinny', 'ffn_tiled_down', 'combine_kernel')}
    ops.timing_enable(False)
    per = lambda name: kern[name][1] / max(1, args.prefill_reps)  # noqa: E731
    up_ms = per('ffn_up_skinny') + per('ffn_tiled_up')
    down_ms = per('ffn_down_skinny') + per('ffn_tiled_down')
    flops = 2 * 3 * H * I * int(counts.sum()) + (2 * 3 * H * Is * T if Is else 0)
    gemm_ms = up_ms + down_ms
    name = ('qwen3_30b_a3b_moe_prefill_t8192_layer_resident' if config == 3 else
            'deepseek_v2_lite_moe_prefill_t65536_layer_resident_shared2')
    return dict(workload=name, tokens=T, tokens_per_s=T / ((t1 - t0) / args.prefill_reps),
                layer_ms=(t1 - t0) / args.prefill_reps * 1e3,
                gemm_ms=gemm_ms, up_ms=up_ms, down_ms=down_ms, gemm_tflop=flops / 1e12,
                mfma_tflops=flops / (gemm_ms * 1e-3) / 1e12,
                mfma_util=flops / (gemm_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
                active_experts=int((counts > 0).sum()), max_rows=int(counts.max()),
                median_rows=float(np.median(counts[counts > 0])),
                kernel_ms={name: per(name) for name in kern})


def run_decode_loop(args, device):
    """Qwen3-30B-A3B decode loop over all 48 MoE layers: a 1024-token prefill layer pass, then
    ``loop_steps`` steps of 64 tokens, routing from the seeded temporal-locality process, a pooled
    cache of 1,843 slots with GateHistory W = 128 eviction."""
    import hashlib
    from ferry_amd import workloads
    from ferry_amd.quota import Topology
    from ferry_amd.runtime import OffloadRuntime
    w = workloads.CONFIGS[5]
    spec = w.spec
    L, E, k, H, I = w.layers, spec.experts, spec.topk, spec.hidden, spec.intermediate
    t0 = time.perf_counter()
    routing = workloads.decode_loop_routing(w, steps=args.loop_steps)
    pool = workloads.make_pool(spec, L, seed=w.seed)
    setup_s = time.perf_counter() - t0
    rt = OffloadRuntime(spec, pool, [w.cache_slots], 'ferry', Topology.uniform(1, E))
    g = torch.Generator(device=device)
    g.manual_seed(w.seed)
    xs = {T: torch.randn((T, H), generator=g, device=device).to(torch.bfloat16)
          for T in (w.prefill_tokens, w.tokens)}
    digest = hashlib.sha1()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for layer in range(L):
        sel = torch.from_numpy(routing['prefill'][layer]).to(device)
        rt.execute(layer, xs[w.prefill_tokens], sel, routing['prefill_weights'][layer].to(device), None)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    prefill_copies = rt.h2d.copies
    rt.timing = True
    from ferry_amd import expert_ops as ops_timing
    ops_timing.timing_enable(True)
    t2 = time.perf_counter()
    for s in range(args.loop_steps):
        for layer in range(L):
            sel = torch.from_numpy(routing['decode'][s, layer]).to(device)
            rt.execute(layer, xs[w.tokens], sel, routing['decode_weights'][s, layer].to(device), None)
        digest.update(rt.controller.slots[0].tobytes())
    torch.cuda.synchronize()
    t3 = time.perf_counter()
    up = ops_timing.timing_summary('ffn_up_skinny')[1] + ops_timing.timing_summary('ffn_tiled_up')[1]
    down = (ops_timing.timing_summary('ffn_down_skinny')[1]
            + ops_timing.timing_summary('ffn_tiled_down')[1])
    fetch_ms, exposed_ms, overlap_ms = rt.fetch_timing()   # reads the launch log: before disabling
    ops_timing.timing_enable(False)
    copies = rt.h2d.copies - prefill_copies
    calls = args.loop_steps * L
    res = dict(
        workload=w.name, layers=L, steps=args.loop_steps, tokens_per_step=w.tokens,
        cache_slots=w.cache_slots, setup_s=setup_s,
        prefill_ms_per_layer=(t1 - t0) / L * 1e3, prefill_fetches=prefill_copies,
        decode_tokens_per_s=w.tokens * args.loop_steps / (t3 - t2),
        decode_ms_per_layer_step=(t3 - t2) / calls * 1e3,
        misses_per_layer_step=copies / calls,
        h2d_gbs=copies * spec.expert_bytes / (fetch_ms * 1e-3) / 1e9 if fetch_ms else None,
        fetch_ms_per_layer_step=fetch_ms / calls,
        fetch_hidden_frac=overlap_ms / fetch_ms if fetch_ms else None,
        fetch_exposed_frac=exposed_ms / fetch_ms if fetch_ms else None,
        ffn_ms_per_layer_step=(up + down) / calls,
        hidden_cap=min(1.0, (up + down) / fetch_ms) if fetch_ms else None,
        eviction_state_sha1=digest.hexdigest())
    rt.close()
    del pool
    return res


def cpu_baseline(dec, seconds):
    """The oracle's torch-CPU restatement of the reference op order on the decode stream."""
    from oracle.experts import execute_experts_ref, reduce_partials_ref
    from oracle.history import GateHistoryRef, frequency_rows
    from oracle.layout import layout_closed_form
    from oracle.policy import PlannerRef
    from oracle.router import qwen3_router
    from ferry_amd import workloads
    w = dec['workload']
    spec = w.spec
    cores = min(16, len(os.sched_getaffinity(0)))
    torch.set_num_threads(cores)
    E, k, H, I = spec.experts, spec.topk, spec.hidden, spec.intermediate
    pool = workloads.make_pool(spec, 1, seed=0).cpu()   # same rows as the GPU pool
    planner = PlannerRef(1, E, w.cache_slots)
    hist = GateHistoryRef(1, E, 128)
    samples = [(lg.cpu(), x.cpu()) for lg, x in dec['samples']]
    steps = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        lg, x = samples[steps % len(samples)]
        wts, sel, _ = qwen3_router(lg, k)
        hist.update(0, frequency_rows(sel.numpy(), E, 128))
        planner.plan(steps, 0, sel.numpy(), hist.scores(0))
        lay = layout_closed_form(sel.numpy(), E, wts.float().numpy())
        w_sorted = torch.from_numpy(lay['w_sorted']).to(torch.bfloat16)
        groups = [e for e in range(E) if lay['counts'][e] > 0]
        rows = [torch.from_numpy(lay['rows'][lay['starts'][e]:lay['starts'][e + 1]]) for e in groups]
        cols = [torch.from_numpy(lay['cols'][lay['starts'][e]:lay['starts'][e + 1]]) for e in groups]
        parts = execute_experts_ref([pool[e] for e in groups], x, w_sorted, rows, cols, H, I)
        reduce_partials_ref(parts, rows, x.shape[0], H)
        steps += 1
    el = time.perf_counter() - t0
    return dict(value=steps * w.tokens / el, unit='tokens/s', cores=cores, kind='port',
                sample=f'{steps} decode steps ({steps * w.tokens} tokens) cycling over the same seeded stream, '
                       f'{el:.1f} s; experts read from host memory (no H2D copy on the CPU path)')


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps(dict(error='ferry_amd runs on one GPU per process; --gpus must be 1 '
                                    '(multi-GPU expert parallelism is out of scope)')))
        sys.exit(2)
    torch.cuda.set_device(0)
    device = torch.device('cuda', 0)
    if args.copy_calibration_mib:
        n = args.copy_calibration_mib << 18   # int32 words
        src = torch.zeros(n, dtype=torch.int32, device=device)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.bitwise_not(src, out=dst)       # reads n*4 bytes, writes n*4 bytes
        torch.cuda.synchronize()
        del src, dst
    dec = run_decode(args, device)
    w = dec['workload']
    ks = dec['kernels']
    up_gbs = ks['up'] / (ks['up_ms'] * 1e-3) / 1e9
    down_gbs = ks['down'] / (ks['down_ms'] * 1e-3) / 1e9
    ffn_gbs = (ks['up'] + ks['down']) / ((ks['up_ms'] + ks['down_ms']) * 1e-3) / 1e9
    value = dec['tokens'] / dec['elapsed']
    fetch_bytes = dec['copies'] * dec['expert_bytes']
    h2d_gbs = fetch_bytes / (dec['fetch_ms'] * 1e-3) / 1e9 if dec['fetch_ms'] else None
    # fraction of the fetch time covered by compute kernels queued while the misses copy
    hidden = dec['overlap_ms'] / dec['fetch_ms'] if dec['fetch_ms'] else None
    exposed = dec['exposed_ms'] / dec['fetch_ms'] if dec['fetch_ms'] else None
    compute_ms = ks['up_ms'] + ks['down_ms']
    ratio = traffic_ratio()
    bytes_per_launch = ks['up'] / max(1, ks['up_launches'])
    line = dict(
        metric='MoE-layer tokens/sec (Qwen3-30B-A3B-shaped decode layer, 16 tok/step, 38/128 cached)',
        value=value, unit='tokens/s', n_gpus=1, steps=args.steps, warmup=args.warmup,
        ms_per_step=dec['elapsed'] / args.steps * 1e3, higher_is_better=True, scaling='weak',
        vs_baseline=None, dtype='bf16', data='synthetic',
        config=dict(workload=w.name, tokens_per_step=w.tokens, experts=w.spec.experts,
                    topk=w.spec.topk, hidden=w.spec.hidden, intermediate=w.spec.intermediate,
                    cache_slots=w.cache_slots, router='N(0,1)+log Zipf(1.1), seed 1',
                    parallelism='single GPU (one expert-parallel share)'),
        roofline=dict(kernel='ffn_up_skinny (decode gate/up + SwiGLU)', bound='hbm',
                      achieved=up_gbs, peak=HBM_PEAK_GBS, unit='GB/s', frac=up_gbs / HBM_PEAK_GBS,
                      traffic=bytes_per_launch * ratio if ratio else None,
                      traffic_over_algorithmic=ratio,
                      traffic_source=TRAFFIC_PROFILE.name if ratio else None,
                      launches=ks['up_launches'],
                      avg_launch_us=ks['up_ms'] / max(1, ks['up_launches']) * 1e3,
                      bytes_per_launch=bytes_per_launch),
        decode=dict(ffn_down_gbs=down_gbs, ffn_gbs=ffn_gbs, ffn_frac=ffn_gbs / HBM_PEAK_GBS,
                    ffn_ms_per_step=compute_ms / args.steps,
                    active_experts_per_step=ks['experts'] / args.steps,
                    misses_per_step=dec['copies'] / args.steps,
                    h2d_gbs=h2d_gbs, h2d_frac=(h2d_gbs / PCIE_PEAK_GBS) if h2d_gbs else None,
                    fetch_ms_per_step=dec['fetch_ms'] / args.steps,
                    fetch_hidden_frac=hidden,
                    fetch_exposed_frac=exposed,
                    kernel_us_per_step={n: v[1] / args.steps * 1e3 for n, v in ks['kernels'].items()},
                    host_us_per_step={n: v / args.steps / 1e3 for n, v in dec['host_ns'].items()},
                    instrumented_ms_per_step=dec['instrumented_elapsed'] / args.steps * 1e3,
                    hidden_cap=min(1.0, compute_ms / dec['fetch_ms']) if dec['fetch_ms'] else None),
    )
    if not args.no_prefill:
        line['prefill'] = run_prefill(args, device, 3)
        line['prefill_deepseek'] = run_prefill(args, device, 4)
    if args.decode_loop:
        line['decode_loop'] = run_decode_loop(args, device)
    if not args.no_cpu_baseline:
        line['cpu_baseline'] = cpu_baseline(dec, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == '__main__':
    main()
