"""Benchmark of the per-GPU MoE hot path on one MI355X.

Headline (``value``): the Qwen3-30B-A3B-shaped MoE layer in decode -- 16 tokens per step, 128
experts top-8 (renormalised softmax), hidden 2048, SwiGLU intermediate 768, bf16, a 38-slot
expert cache with the other experts in pinned host memory, router logits N(0, 1) + log
Zipf(1.1) popularity (seed 1), expert weights N(0, 0.02) bf16.  One step = one layer call:
router kernel -> device history + routing IDs to the host -> host planner -> H2D fetch of the
misses -> layout -> grouped SwiGLU (resident experts first) -> combine.  The fetch copies the
misses as packed rows (OffloadRuntime(pack=True): per value a sign|mantissa byte and a 2-bit
exponent code, the rarer exponents in two escape levels and a list, lossless, 1.49x fewer bytes
over the host link on these weights) with hipMemcpyAsync on two DMA streams, and a kernel unpacks them into the cache
slots; the outputs are bit-identical to raw fetches.  Before anything is measured, 300 steps
of the stream run untimed through a throwaway runtime (a process's first few hundred decode
steps run about 3 % slower while the HIP runtime's internal pools grow).  A first pass over the
stream collects per-launch kernel times, fetch events and host phase times; the timed pass then
runs the same stream from an empty cache again, without instrumentation.

Also on the line:
  * roofline: the decode FFN kernel (ffn_skinny_fused: gate/up + SwiGLU + down in one launch),
    achieved GB/s on its algorithmic bytes vs 8 TB/s: bytes per launch / the mean of the
    per-launch HIP-event durations of all its launches in the instrumented pass; traffic from
    the committed FETCH_SIZE / WRITE_SIZE profile of that kernel;
  * roofline_prefill: the tiled up-projection GEMM (ffn_tiled_up) of the Qwen3 prefill layer,
    TFLOP/s vs 2.5 PFLOP/s bf16, measured the same way;
  * prefill / prefill_deepseek: the Qwen3 8192-token layer and the DeepSeek-V2-Lite
    65,536-token layer (with its two shared experts), experts resident;
  * prefill_stack / prefill_stack_deepseek: those layers over the whole stack (48 / 26 layers,
    distinct seeded weights and routing per layer) through OffloadRuntime with the pooled 30 %
    cache (1,843 / 499 slots) from cold, so every layer fetches its missing experts over PCIe;
    packed fetches, with the raw-row run under ``raw``;
  * decode_loop: the 48-layer Qwen3 decode loop (1024-token prefill, then 64-token steps,
    pooled cache of 1,843, W = 128 eviction), ``--loop-steps`` steps (default 8, bounded);
    packed fetches, with the raw-row run under ``raw``;
  * generate: end-to-end greedy generation through a Qwen3-30B-A3B-shaped model with random
    weights, every MoE block hooked into OffloadRuntime (the 48-layer packed pool, pooled 30 %
    cache): the reference's serving protocol (warm-up, discarded and measured runs from an empty
    cache, 200 ms release delay) and metrics, TTFT / TPOT / E2E / TPS as mean and sample std;
  * decode_raw: the headline stream with raw rows over the host link (OffloadRuntime(pack=
    False), the reference's transfer format);
  * decode_split_fetch: the headline stream with OffloadRuntime(split_fetch=True), each packed
    call's fetched experts computed sub-batch by sub-batch as they are unpacked;
  * decode_serial_raw: the headline stream with the reference's fetch scheme (raw rows, the host
    waits for every copy before any expert runs) on this library's kernels;
  * decode_copy_kernel: the headline stream through OffloadRuntime(copy='kernel'): raw misses
    copied by one kernel launch on the compute stream, then one FFN launch (no overlap);
  * reference_pattern_gpu: the reference's own per-expert torch op order for the expert FFN
    and the combine (hipBLASLt GEMMs) timed on this GPU beside this library's launches, on the
    Qwen3 prefill layer and one decode step, every expert resident;
  * cpu_baseline: the reference's op order in torch on the host cores (all cores of the
    process's affinity), median of >= 5 repeats on the decode stream, plus one Qwen3 8192-token
    prefill layer with the 48-layer extrapolation.
"""
import argparse
import gc
import json
import os
import statistics
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
PACK_THREADS = 16   # host threads that pack a pool (the box's CPU share)

TILED_TRAFFIC_PROFILE = ROOT / 'profiles' / 'ffn_tiled_prefill_qwen3_t8192_hbm_traffic.md'
FUSED_TRAFFIC_PROFILE = ROOT / 'profiles' / 'ffn_skinny_fused_decode_qwen3_t16_hbm_traffic.md'


def profile_value(path, key):
    """``key = value`` line of a committed profile summary, or None."""
    try:
        for line in path.read_text().splitlines():
            if line.startswith(key):
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
    p.add_argument('--no-stacks', action='store_true',
                   help='skip the prefill stacks and the decode loop (they build 54 + 29 GB of '
                        'pinned expert pools)')
    p.add_argument('--no-cpu-baseline', action='store_true')
    p.add_argument('--cpu-seconds', type=float, default=20.0,
                   help='CPU time budget of the decode-stream baseline (5 repeats)')
    p.add_argument('--loop-steps', type=int, default=8, help='decode-loop steps (the reference loop runs 64)')
    p.add_argument('--no-generate', action='store_true',
                   help='skip the end-to-end generate block (TTFT / TPOT / E2E / TPS)')
    p.add_argument('--gen-batch', type=int, default=16, help='generate: requests per run')
    p.add_argument('--gen-prompt', type=int, default=512, help='generate: prompt tokens per request')
    p.add_argument('--gen-output', type=int, default=16,
                   help='generate: output tokens per request (the reference cells use 64)')
    p.add_argument('--gen-repeats', type=int, default=3, help='generate: measured runs')
    p.add_argument('--gen-discard', type=int, default=1,
                   help='generate: unreported runs on the target prompts before the measured ones')
    p.add_argument('--copy-calibration-mib', type=int, default=0,
                   help='run one plain device copy kernel of this many MiB (read and written) '
                        'before the decode pass: the reference dispatch for scaling HBM byte '
                        'counters (FETCH_SIZE / WRITE_SIZE) in profiler runs')
    return p.parse_args()


def run_stacks(args, device):
    """The two prefill stacks and the decode loop, each with packed fetches and with raw rows.
    Pinned host memory is limited (about a quarter of RAM), so the raw runs use a pinned pool
    that is freed before the same seeded pool is rebuilt in pageable memory, packed (the
    packed copy is pinned) and freed again."""
    from ferry_amd import workloads
    from ferry_amd.h2d import PackedPool
    out = {}
    for w in (workloads.QWEN3_PREFILL_STACK, workloads.DEEPSEEK_PREFILL_STACK):
        qwen3 = w is workloads.QWEN3_PREFILL_STACK
        layers = 48 if qwen3 else w.layers
        t0 = time.perf_counter()
        pool = workloads.make_pool(w.spec, layers, seed=w.seed)
        pool_s = time.perf_counter() - t0
        raw = raw_summary(run_prefill_stack(device, w, pool))
        if qwen3:
            loop_raw = raw_summary(run_decode_loop(device, args.loop_steps, pool))
        del pool
        gc.collect()
        src = workloads.make_pool(w.spec, layers, seed=w.seed, pinned=False)
        t0 = time.perf_counter()
        packed = PackedPool(src, PACK_THREADS)
        pack_s = time.perf_counter() - t0
        del src
        gc.collect()
        key = 'prefill_stack' if qwen3 else 'prefill_stack_deepseek'
        out[key] = run_prefill_stack(device, w, packed)
        out[key].update(pool_build_s=pool_s, pack_s=pack_s, pack_ratio=packed.ratio, raw=raw)
        print(f'# {key} done', file=sys.stderr, flush=True)
        if qwen3:
            out['decode_loop'] = run_decode_loop(device, args.loop_steps, packed)
            out['decode_loop']['raw'] = loop_raw
            print('# decode loop done', file=sys.stderr, flush=True)
            if not args.no_generate:
                out['generate'] = run_generate(args, device, packed)
                print('# generate done', file=sys.stderr, flush=True)
        packed.close()
        del packed
        gc.collect()
    return out


def raw_summary(block):
    """The throughput fields of a stack / loop block run with raw rows over the host link."""
    keys = ('tokens_per_s', 'decode_tokens_per_s', 'stack_ms', 'decode_ms_per_layer_step',
            'h2d_gbs', 'fetch_hidden_frac')
    return {k: block[k] for k in keys if k in block}


def launch_stats(ops, name):
    n, ms = ops.timing_summary(name)
    return dict(launches=n, total_ms=ms, avg_us=ms / n * 1e3 if n else None)


# ---------------------------------------------------------------------------------------------
# the decode layer (headline)
# ---------------------------------------------------------------------------------------------

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


def run_decode(args, device, copy='dma', pack=False, split_fetch=False, overlap=True):
    from ferry_amd import expert_ops as ops
    from ferry_amd import workloads
    from ferry_amd.quota import Topology
    from ferry_amd.runtime import OffloadRuntime
    w = workloads.QWEN3_DECODE_LAYER
    spec = w.spec
    pool = workloads.make_pool(spec, 1, seed=0)
    rt = OffloadRuntime(spec, pool, [w.cache_slots], 'ferry', Topology.uniform(1, spec.experts),
                        copy=copy, pack=pack, split_fetch=split_fetch, overlap=overlap)
    packing = None
    if rt.packed is not None:
        packing = dict(ratio=rt.packed.ratio, packed_rows=rt.packed.packed_rows,
                       packed_bytes=rt.packed.packed_bytes,
                       row_bytes=spec.expert_bytes)
    stream = decode_stream(w, args.warmup + args.steps, device)

    def step(lg, x):
        wts, sel = ops.router_topk(lg, spec.topk, renorm=True)
        return rt.execute(0, x, sel, wts, None)

    # pass 1: the stream with per-launch kernel timing, fetch events and host phase timing
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
    names = ('router_kernel', 'history_kernel', 'layout_single', 'ffn_skinny_fused', 'ffn_up_skinny',
             'ffn_down_skinny', 'combine_kernel')
    ks['launch'] = {name: launch_stats(ops, name) for name in names}
    fetch_ms, exposed_ms, overlap_ms = rt.fetch_timing()   # reads the launch log: before disabling
    critical = rt.critical_path_timing()
    host_ns = dict(rt.host_ns)
    ops.timing_enable(False)
    rt.timing = False
    # pass 2 (the measurement): the same stream from an empty cache again (same misses, same
    # launches), no instrumentation in the timed region; garbage of earlier work (pinned pools
    # among it) is collected before it
    gc.collect()
    rt.reset()
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
    res = dict(workload=w, elapsed=t1 - t0, instrumented_elapsed=t3 - t2,
               critical=critical, packing=packing,
               sync_timeouts=ops.ffn_sync_timeouts(),
               tokens=w.tokens * args.steps, copies=copies, kernels=ks, fetch_ms=fetch_ms,
               exposed_ms=exposed_ms, overlap_ms=overlap_ms, expert_bytes=spec.expert_bytes,
               samples=stream[args.warmup:], host_ns=host_ns)
    rt.close()
    del pool
    return res


def warm_up_runtime(device, steps=300):
    """``steps`` calls of the headline decode stream through a throwaway runtime, untimed, before
    anything is measured.  A process's first few hundred decode steps run about 3 % slower than
    the same steps afterwards (0.78-0.81 against 0.76 ms per step in separate processes) while the
    HIP runtime's own queue, signal and argument pools grow to their working size; a warm-up of
    a hundred steps was not enough."""
    from ferry_amd import expert_ops as ops
    from ferry_amd import workloads
    from ferry_amd.quota import Topology
    from ferry_amd.runtime import OffloadRuntime
    w = workloads.QWEN3_DECODE_LAYER
    spec = w.spec
    pool = workloads.make_pool(spec, 1, seed=0)
    rt = OffloadRuntime(spec, pool, [w.cache_slots], 'ferry', Topology.uniform(1, spec.experts),
                        pack=True)
    for lg, x in decode_stream(w, steps, device):
        wts, sel = ops.router_topk(lg, spec.topk, renorm=True)
        rt.execute(0, x, sel, wts, None)
    torch.cuda.synchronize()
    rt.close()
    del rt, pool
    # free the throwaway pools now (pinned host memory), not inside a later timed region
    gc.collect()
    torch.cuda.synchronize()


def decode_block(dec, args):
    ks = dec['kernels']
    lk = ks['launch']
    fused, up, down = lk['ffn_skinny_fused'], lk['ffn_up_skinny'], lk['ffn_down_skinny']
    ffn_ms = fused['total_ms'] + up['total_ms'] + down['total_ms']
    ffn_gbs = (ks['up'] + ks['down']) / (ffn_ms * 1e-3) / 1e9
    fetch_bytes = dec['copies'] * dec['expert_bytes']
    h2d_gbs = fetch_bytes / (dec['fetch_ms'] * 1e-3) / 1e9 if dec['fetch_ms'] else None
    if fused['launches']:
        # every decode call runs both phases in the one-launch kernel
        ratio = profile_value(FUSED_TRAFFIC_PROFILE, 'traffic_over_algorithmic')
        source = FUSED_TRAFFIC_PROFILE
        kern, name = fused, 'ffn_skinny_fused (decode gate/up + SwiGLU + down, one launch)'
        kbytes = ks['up'] + ks['down']
    else:
        ratio, source = None, None   # no committed traffic profile for the split launches
        kern, name, kbytes = up, 'ffn_up_skinny (decode gate/up + SwiGLU)', ks['up']
    achieved = kbytes / (kern['total_ms'] * 1e-3) / 1e9
    bytes_per_launch = kbytes / max(1, kern['launches'])
    roofline = dict(kernel=name, bound='hbm', achieved=achieved,
                    peak=HBM_PEAK_GBS, unit='GB/s', frac=achieved / HBM_PEAK_GBS,
                    traffic=bytes_per_launch * ratio if ratio else None,
                    traffic_over_algorithmic=ratio,
                    traffic_source=source.name if ratio else None,
                    launches=kern['launches'], avg_launch_us=kern['avg_us'],
                    bytes_per_launch=bytes_per_launch,
                    average='mean of per-launch HIP-event durations (compute stream) over every '
                            'launch of the instrumented pass; warmup launches excluded')
    block = dict(ffn_gbs=ffn_gbs, ffn_frac=ffn_gbs / HBM_PEAK_GBS, ffn_ms_per_step=ffn_ms / args.steps,
                 ffn_sync_timeouts=dec.get('sync_timeouts'),
                 active_experts_per_step=ks['experts'] / args.steps,
                 misses_per_step=dec['copies'] / args.steps,
                 h2d_gbs=h2d_gbs, h2d_frac=(h2d_gbs / PCIE_PEAK_GBS) if h2d_gbs else None,
                 fetch_ms_per_step=dec['fetch_ms'] / args.steps,
                 fetch_hidden_frac=dec['overlap_ms'] / dec['fetch_ms'] if dec['fetch_ms'] else None,
                 fetch_exposed_frac=dec['exposed_ms'] / dec['fetch_ms'] if dec['fetch_ms'] else None,
                 hidden_cap=min(1.0, ffn_ms / dec['fetch_ms']) if dec['fetch_ms'] else None,
                 kernel_us_per_step={n: v['total_ms'] / args.steps * 1e3
                                     for n, v in ks['launch'].items()},
                 kernel_avg_launch_us={n: v['avg_us'] for n, v in ks['launch'].items()},
                 host_us_per_step={n: v / args.steps / 1e3 for n, v in dec['host_ns'].items()},
                 instrumented_ms_per_step=dec['instrumented_elapsed'] / args.steps * 1e3,
                 critical_path_us={k: (v * 1e3 if k.endswith('_ms') and v is not None else v)
                                   for k, v in dec['critical'].items()})
    return roofline, block


# ---------------------------------------------------------------------------------------------
# the prefill layers: one layer, experts resident
# ---------------------------------------------------------------------------------------------

def run_prefill(args, device, w):
    """One prefill layer with every expert resident in HBM, of workload ``w``: the Qwen3-shaped
    8192-token layer (QWEN3_PREFILL_STACK's shape) or the DeepSeek-V2-Lite-shaped 65,536-token
    layer with its two shared experts (DEEPSEEK_PREFILL_STACK's shape)."""
    from ferry_amd import expert_ops as ops
    from ferry_amd import workloads
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
        # the per-expert row counts on the host, as the runtime has them from the routing it
        # reads back for its planner (one device sync per layer call): here from the layout's
        # expert starts
        rows_e = np.diff(lay.starts.cpu().numpy())
        ops.expert_ffn(cache, x, lay.w_sorted, lay.starts, lay.rows, lay.cols, np.arange(E), slot_of,
                       H, I, act, part, counts=rows_e)
        add = shared(x, out=shared_out) if shared is not None else None
        return ops.combine(part, T, k, H, addend=add), sel

    _, sel = layer()
    torch.cuda.synchronize()
    counts = np.bincount(sel.cpu().numpy().reshape(-1), minlength=E)
    gc.collect()   # earlier blocks' pinned pools are freed here, not in the timed region
    t0 = time.perf_counter()
    for _ in range(args.prefill_reps):
        layer()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ops.timing_enable(True)
    for _ in range(args.prefill_reps):
        layer()
    torch.cuda.synchronize()
    names = ('router_kernel', 'layout_count', 'layout_scan', 'layout_scatter', 'ffn_up_skinny',
             'ffn_tiled_up', 'ffn_down_skinny', 'ffn_tiled_down', 'combine_kernel')
    kern = {name: launch_stats(ops, name) for name in names}
    ops.timing_enable(False)
    # plain reads of the small experts' weight byte counts where their launches run: the
    # gate/up bytes right after a layer call (whose tiled launches leave written rows to drain)
    # and a host sync, the down bytes right after that read
    reads_after_layer = None
    n_small = int(((counts > 0) & (counts <= 64)).sum())
    if n_small:
        bufs = {'up_weights': torch.ones(n_small * 2 * I * H * 2, dtype=torch.uint8, device=device),
                'down_weights': torch.ones(n_small * I * H * 2, dtype=torch.uint8, device=device)}
        sink = torch.empty(int(bufs['up_weights'].numel() // 512) + 16, dtype=torch.uint8,
                           device=device)
        times = {name: [] for name in bufs}
        for _ in range(args.prefill_reps):
            layer()
            torch.cuda.synchronize()
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(bufs) + 1)]
            ev[0].record()
            for i, buf in enumerate(bufs.values()):
                ops.hbm_read(buf, sink)
                ev[i + 1].record()
            ev[-1].synchronize()
            for i, name in enumerate(bufs):
                times[name].append(ev[i].elapsed_time(ev[i + 1]) * 1e3)
        reads_after_layer = {name: dict(bytes=bufs[name].numel(), us=float(np.median(v)))
                             for name, v in times.items()}
        del bufs, sink
    per = lambda name: kern[name]['total_ms'] / max(1, args.prefill_reps)  # noqa: E731
    up_ms = per('ffn_up_skinny') + per('ffn_tiled_up')
    down_ms = per('ffn_down_skinny') + per('ffn_tiled_down')
    flops = 2 * 3 * H * I * int(counts.sum()) + (2 * 3 * H * Is * T if Is else 0)
    tiled_rows = int(counts[counts > 64].sum()) + (T if Is else 0)
    tiled_up_flops = 2 * 2 * H * (I * int(counts[counts > 64].sum()) + (Is * T if Is else 0))
    gemm_ms = up_ms + down_ms
    name = ('qwen3_30b_a3b_moe_prefill_t8192_layer_resident' if w is workloads.QWEN3_PREFILL_STACK else
            'deepseek_v2_lite_moe_prefill_t65536_layer_resident_shared2')
    tu = kern['ffn_tiled_up']
    # the shared experts' launches add to the tiled kernel's launch count (one per layer call)
    tiled_up_launch_flops = tiled_up_flops / max(1, tu['launches'] / args.prefill_reps)
    # algorithmic HBM bytes of one routed tiled launch: each tiled expert's weights once, each of
    # its rows read once and its output rows written once
    n_tiled, routed_rows = int((counts > 64).sum()), int(counts[counts > 64].sum())
    tiled_up_bytes = 2 * (n_tiled * 2 * I * H + routed_rows * (H + I))
    tiled_down_bytes = 2 * (n_tiled * I * H + routed_rows * (I + H))
    return dict(workload=name, tokens=T, tokens_per_s=T / ((t1 - t0) / args.prefill_reps),
                layer_ms=(t1 - t0) / args.prefill_reps * 1e3,
                gemm_ms=gemm_ms, up_ms=up_ms, down_ms=down_ms, gemm_tflop=flops / 1e12,
                mfma_tflops=flops / (gemm_ms * 1e-3) / 1e12,
                mfma_util=flops / (gemm_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
                active_experts=int((counts > 0).sum()), max_rows=int(counts.max()),
                median_rows=float(np.median(counts[counts > 0])), tiled_rows=tiled_rows,
                small_experts=int(((counts > 0) & (counts <= 64)).sum()),
                small_rows=int(counts[(counts > 0) & (counts <= 64)].sum()),
                tiled_experts=n_tiled, routed_tiled_up_bytes=tiled_up_bytes,
                routed_tiled_down_bytes=tiled_down_bytes,
                tiled_up_launch_tflop=tiled_up_launch_flops / 1e12,
                tiled_up_avg_us=tu['avg_us'], small_reads_after_layer=reads_after_layer,
                kernel_ms={n: per(n) for n in kern},
                kernel_avg_launch_us={n: v['avg_us'] for n, v in kern.items()})


def reference_pattern_gpu(device, reps=5):
    """The reference's own GPU op order for the expert FFN and the combine, restated in torch and
    timed on this GPU beside this library's kernels on the same inputs: per expert (ascending
    IDs) an index_select of its token rows, the gate and up GEMMs, fp32 silu(g) * u rounded to
    bf16, the down GEMM and the routing-weight product (execute_experts, expert_ops.cpp:13-45),
    then the fp32 index_add over the experts in ascending order and one bf16 rounding
    (reduce_partials, expert_ops.cpp:75-92).  GEMMs are torch's (hipBLASLt), with the weights
    read in place from the cache rows as the reference does.  Two workloads, every expert
    resident: the Qwen3 8192-token prefill layer and one 16-token step of the decode stream.
    Timed: FFN + combine, HIP events around the whole call, median of ``reps``; the router and
    layout are outside both timings.  ``max_abs_diff``: the two outputs' largest difference."""
    import torch.nn.functional as F

    from ferry_amd import expert_ops as ops
    from ferry_amd import workloads
    out = {}
    cases = (('qwen3_prefill_t8192', workloads.QWEN3_PREFILL_STACK),
             ('qwen3_decode_t16', workloads.QWEN3_DECODE_LAYER))
    for name, w in cases:
        spec = w.spec
        E, k, H, I = spec.experts, spec.topk, spec.hidden, spec.intermediate
        if w is workloads.QWEN3_DECODE_LAYER:
            logits, x = decode_stream(w, 1, device)[0]
        else:
            logits = workloads.RouterLogits(replace(w, layers=1), device).next(0, w.tokens)
            x = workloads.hidden_states(w.tokens, H, seed=w.seed + 7, device=device)
        T = x.shape[0]
        cache = workloads.expert_rows(range(E), spec.expert_elements, seed=w.seed, device=device)
        wts, sel = ops.router_topk(logits, k, renorm=w.renorm, sorted=w.sorted)
        lay = ops.layout(sel, wts, E)
        starts = lay.starts.cpu().numpy()
        counts = np.diff(starts)
        active = np.flatnonzero(counts)
        act = torch.empty((T * k, I), dtype=torch.bfloat16, device=device)
        part = torch.empty((T * k, H), dtype=torch.bfloat16, device=device)
        slot_of = np.arange(E, dtype=np.int32)
        groups = [(e, lay.rows[starts[e]:starts[e + 1]], lay.cols[starts[e]:starts[e + 1]])
                  for e in active]
        # the routing weights in each token's sorted-ID order: (rows, cols) index them
        w_sorted = lay.w_sorted.view(T, k)

        def ours():
            ops.expert_ffn(cache, x, lay.w_sorted, lay.starts, lay.rows, lay.cols, active,
                           slot_of, H, I, act, part, counts=counts)
            return ops.combine(part, T, k, H)

        def reference():
            acc = torch.zeros((T, H), dtype=torch.float32, device=device)
            for e, rows, cols in groups:
                row = cache[e]
                gate = row[:I * H].view(I, H)
                up = row[I * H:2 * I * H].view(I, H)
                down = row[2 * I * H:].view(H, I)
                xe = x.index_select(0, rows)
                a = (F.silu(F.linear(xe, gate).float()) * F.linear(xe, up).float()).to(torch.bfloat16)
                y = F.linear(a, down) * w_sorted[rows, cols].unsqueeze(1)
                acc.index_add_(0, rows, y.float())
            return acc.to(torch.bfloat16)

        res = {}
        outs = {}
        for label, fn in (('ours', ours), ('reference_pattern', reference)):
            outs[label] = fn()
            torch.cuda.synchronize()
            ts = []
            for _ in range(reps):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                fn()
                e1.record()
                e1.synchronize()
                ts.append(e0.elapsed_time(e1))
            res[label + '_ms'] = float(np.median(ts))
        res.update(tokens=T, active_experts=int(len(active)),
                   speedup=res['reference_pattern_ms'] / res['ours_ms'],
                   max_abs_diff=float((outs['ours'].float() - outs['reference_pattern'].float())
                                      .abs().max()))
        out[name] = res
        del cache, act, part, outs
        torch.cuda.empty_cache()
    out['note'] = ('the reference\'s per-expert torch op order on this GPU (hipBLASLt GEMMs, one '
                   'host launch sequence per expert) against this library\'s launches, same '
                   'inputs, FFN + combine only')
    return out


def gemm_ceiling(device):
    """bf16 rate of AMD's tuned library (hipBLASLt through torch.matmul) on dense GEMMs shaped
    like the largest expert of each prefill layer, and on 8192^3, measured in the same run: the
    practical ceiling against which the grouped kernels' MFMA utilisation reads."""
    shapes = {'qwen3_largest_expert_up_8192x1536x2048': (8192, 1536, 2048),
              'deepseek_largest_expert_up_57344x2816x2048': (57344, 2816, 2048),
              'dense_up_65536x1536x2048': (65536, 1536, 2048),
              'dense_down_65536x2048x768': (65536, 2048, 768),
              'dense_8192x8192x8192': (8192, 8192, 8192)}
    g = torch.Generator(device=device)
    g.manual_seed(11)
    out = {}
    for name, (m, n, k) in shapes.items():
        a = torch.randn((m, k), generator=g, device=device).to(torch.bfloat16)
        b = torch.randn((k, n), generator=g, device=device).to(torch.bfloat16)
        c = torch.empty((m, n), dtype=torch.bfloat16, device=device)
        for _ in range(3):
            torch.matmul(a, b, out=c)
        ts = []
        for _ in range(10):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            torch.matmul(a, b, out=c)
            e1.record()
            e1.synchronize()
            ts.append(e0.elapsed_time(e1))
        ms = float(np.median(ts))
        tflops = 2 * m * n * k / (ms * 1e-3) / 1e12
        out[name] = dict(tflops=tflops, frac=tflops / BF16_PEAK_TFLOPS, ms=ms)
        del a, b, c
    torch.cuda.empty_cache()
    return out


def tiled_dense(device, reps=10):
    """The tiled kernels on one dense Qwen3-shaped expert of 65,536 rows (every row routed to
    it with weight 1): the up projection 65536 x 1536 x 2048 (gate and up columns, SwiGLU
    epilogue) and the down projection 65536 x 2048 x 768 (routing-weight epilogue), M x N x K,
    each timed per launch with HIP events (median over ``reps`` back-to-back launches, and over
    launches that each follow 50 ms of idle GPU), next to hipBLASLt on the same shapes in
    gemm_ceiling_hipblaslt."""
    from ferry_amd import expert_ops as ops
    from ferry_amd import workloads
    M, H, I = 65536, 2048, 768
    cache = workloads.expert_rows([0], 3 * H * I, seed=17, device=device)
    x = workloads.hidden_states(M, H, seed=18, device=device)
    sel = torch.zeros((M, 1), dtype=torch.int64, device=device)
    lay = ops.layout(sel, torch.ones((M, 1), dtype=torch.bfloat16, device=device), 1)
    act = torch.empty((M, I), dtype=torch.bfloat16, device=device)
    out = torch.empty((M, H), dtype=torch.bfloat16, device=device)
    one = np.zeros(1, np.int32)
    res = {}
    for name, phase, flops in (('up_65536x1536x2048', ops.PHASE_UP, 2 * M * 2 * I * H),
                               ('down_65536x2048x768', ops.PHASE_DOWN, 2 * M * H * I)):
        def launch():
            ops.expert_ffn(cache, x, lay.w_sorted, lay.starts, lay.rows, lay.cols, one, one, H, I,
                           act, out, max_rows=M, phases=phase)
        for _ in range(3):
            launch()
        ts = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            launch()
            e1.record()
            e1.synchronize()
            ts.append(e0.elapsed_time(e1))
        ms = float(np.median(ts))
        tflops = flops / (ms * 1e-3) / 1e12
        # the same launch after 50 ms of idle GPU each time: the clock the chip holds for a
        # burst, against the back-to-back launches above (the MFMA loop is power-limited)
        burst = []
        for _ in range(5):
            time.sleep(0.05)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            launch()
            e1.record()
            e1.synchronize()
            burst.append(e0.elapsed_time(e1))
        bms = float(np.median(burst))
        res[name] = dict(kernel='ffn_tiled_up' if phase == ops.PHASE_UP else 'ffn_tiled_down',
                         us=ms * 1e3, tflops=tflops, frac=tflops / BF16_PEAK_TFLOPS,
                         launches_us=[round(t * 1e3, 1) for t in ts],
                         after_idle_us=bms * 1e3,
                         after_idle_tflops=flops / (bms * 1e-3) / 1e12)
    del cache, x, act, out, lay
    torch.cuda.empty_cache()
    return res


def cold_reads(device, sizes, reps=9):
    """Plain cold reads (the library's hbm_read, 32 KiB workgroups) of buffers of the given byte
    counts, each event-timed (median over ``reps``); a 1 GiB read before each repeat evicts them
    from the memory-side cache.  Returns {name: dict(bytes, us, gbs, frac)}."""
    from ferry_amd import expert_ops as ops
    flush = torch.ones(1 << 30, dtype=torch.uint8, device=device)
    bufs = {k: torch.ones(int(v) // 256 * 256, dtype=torch.uint8, device=device)
            for k, v in sizes.items()}
    sink = torch.empty(int(flush.numel() // 512) + 16, dtype=torch.uint8, device=device)
    times = {k: [] for k in bufs}
    for _ in range(reps):
        ops.hbm_read(flush, sink)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(bufs) + 1)]
        ev[0].record()
        for i, b in enumerate(bufs.values()):
            ops.hbm_read(b, sink)
            ev[i + 1].record()
        ev[-1].synchronize()
        for i, k in enumerate(bufs):
            times[k].append(ev[i].elapsed_time(ev[i + 1]) * 1e3)
    out = {}
    for k, b in bufs.items():
        us = float(np.median(times[k]))
        out[k] = dict(bytes=b.numel(), us=us, gbs=b.numel() / (us * 1e-6) / 1e9,
                      frac=b.numel() / (us * 1e-6) / 1e9 / HBM_PEAK_GBS)
    del flush, bufs
    torch.cuda.empty_cache()
    return out


def read_ceiling(device, block, expert_bytes, reps=9):
    """Plain cold reads of the byte counts of a decode step's two FFN launches (the resident
    experts', the fetched experts'), measured in the same run: the practical ceiling against
    which the decode FFN's HBM fraction reads."""
    fetched = block['misses_per_step']
    resident = block['active_experts_per_step'] - fetched
    out = cold_reads(device, {'resident_launch': resident * expert_bytes,
                              'fetched_launch': fetched * expert_bytes}, reps)
    total_b = sum(v['bytes'] for v in out.values())
    total_us = sum(v['us'] for v in out.values())
    read_gbs = total_b / (total_us * 1e-6) / 1e9
    out.update(kernel='hbm_read_kernel (plain read, 32 KiB workgroups, data cold)',
               both_gbs=read_gbs, both_frac=read_gbs / HBM_PEAK_GBS,
               ffn_over_read=block['ffn_gbs'] / read_gbs)
    return out


def small_expert_ceiling(device, pre, spec):
    """The prefill layer's small-expert launches (experts of at most 64 rows: ffn_up_skinny,
    ffn_down_skinny) against plain cold reads of their weight bytes, measured in the same run."""
    n = pre['small_experts']
    H, I = spec.hidden, spec.intermediate
    reads = cold_reads(device, {'up_weights': n * 2 * I * H * 2, 'down_weights': n * I * H * 2})
    after = pre.get('small_reads_after_layer') or {}

    def phase(name, launch_us):
        r = reads[name]
        out = dict(launch_us=launch_us, read_us=r['us'], launch_over_read=launch_us / r['us'],
                   weight_bytes=r['bytes'], launch_gbs=r['bytes'] / (launch_us * 1e-6) / 1e9,
                   read_gbs=r['gbs'])
        if name in after:
            out.update(read_after_layer_us=after[name]['us'],
                       launch_over_read_after_layer=launch_us / after[name]['us'])
        return out
    return dict(experts=n, rows=pre['small_rows'],
                up=phase('up_weights', pre['kernel_avg_launch_us']['ffn_up_skinny']),
                down=phase('down_weights', pre['kernel_avg_launch_us']['ffn_down_skinny']),
                note='launch: mean per-launch HIP-event time in the prefill block; read: the '
                     'same weight bytes read cold by hbm_read after a 1 GiB read (the token '
                     'rows, read from L2, are not in the ceiling); read_after_layer: the same '
                     'reads where the launches run: the gate/up bytes right after a layer call '
                     'and a host sync (the previous layer\'s written rows still draining), the '
                     'down bytes right after them')


def prefill_roofline(pre):
    """MFMA roofline of the tiled up-projection launch of the Qwen3 prefill layer."""
    tflops = pre['tiled_up_launch_tflop'] / (pre['tiled_up_avg_us'] * 1e-6)
    ratio = profile_value(TILED_TRAFFIC_PROFILE, 'up_traffic_over_algorithmic')
    return dict(kernel='ffn_tiled_up (prefill gate/up GEMM + SwiGLU, experts > 64 rows)',
                bound='mfma', achieved=tflops, peak=BF16_PEAK_TFLOPS, unit='TFLOP/s',
                frac=tflops / BF16_PEAK_TFLOPS,
                traffic=pre['routed_tiled_up_bytes'] * ratio if ratio else None,
                algorithmic_bytes=pre['routed_tiled_up_bytes'], traffic_over_algorithmic=ratio,
                traffic_source=TILED_TRAFFIC_PROFILE.name if ratio else None,
                flop_per_launch=pre['tiled_up_launch_tflop'] * 1e12,
                avg_launch_us=pre['tiled_up_avg_us'],
                average='mean of per-launch HIP-event durations over the instrumented repeats')


# ---------------------------------------------------------------------------------------------
# the prefill stacks over every layer, and the decode loop
# ---------------------------------------------------------------------------------------------

def run_prefill_stack(device, w, pool):
    """Every MoE layer of the model on one prefill batch through OffloadRuntime with the pooled
    30 % cache, from cold.  Pass 1 is timed; pass 2 (after a reset) records fetch events."""
    from ferry_amd import expert_ops as ops
    from ferry_amd import workloads
    from ferry_amd.quota import Topology
    from ferry_amd.runtime import OffloadRuntime
    spec = w.spec
    L, E, k, H, T = w.layers, spec.experts, spec.topk, spec.hidden, w.tokens
    gen = workloads.RouterLogits(w, device)
    logits = [gen.next(layer, T) for layer in range(L)]
    x = workloads.hidden_states(T, H, seed=w.seed + 7, device=device)
    shared = None
    if w.shared_intermediate:
        rows = workloads.shared_rows(L, H, w.shared_intermediate, seed=w.seed, device=device)
        shared = [ops.SharedExpert(rows[layer], H, w.shared_intermediate) for layer in range(L)]
    rt = OffloadRuntime(spec, pool, [w.cache_slots], 'ferry', Topology.uniform(1, E))

    def stack():
        for layer in range(L):
            wts, sel = ops.router_topk(logits[layer], k, renorm=w.renorm, sorted=w.sorted,
                                       scale=1.0)
            rt.execute(layer, x, sel, wts, None, shared=shared[layer] if shared else None)

    torch.cuda.synchronize()
    gc.collect()
    t0 = time.perf_counter()
    stack()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    copies = rt.h2d.copies
    rt.reset()
    rt.timing = True
    ops.timing_enable(True)
    t2 = time.perf_counter()
    stack()
    torch.cuda.synchronize()
    t3 = time.perf_counter()
    fetch_ms, exposed_ms, overlap_ms = rt.fetch_timing()
    ffn_ms = sum(ops.timing_summary(n)[1] for n in
                 ('ffn_skinny_fused', 'ffn_up_skinny', 'ffn_tiled_up', 'ffn_down_skinny',
                  'ffn_tiled_down'))
    ops.timing_enable(False)
    flops = rt.kernel_bytes['flops'] + (2 * 3 * H * w.shared_intermediate * T * L if shared else 0)
    rt.close()
    return dict(workload=w.name, layers=L, tokens=T, cache_slots=w.cache_slots,
                stack_ms=(t1 - t0) * 1e3, tokens_per_s=T / (t1 - t0),
                instrumented_stack_ms=(t3 - t2) * 1e3, misses_per_layer=copies / L,
                h2d_gbs=copies * spec.expert_bytes / (fetch_ms * 1e-3) / 1e9 if fetch_ms else None,
                fetch_ms_per_layer=fetch_ms / L, ffn_ms_per_layer=ffn_ms / L,
                gemm_tflop_per_layer=flops / L / 1e12,
                fetch_hidden_frac=overlap_ms / fetch_ms if fetch_ms else None,
                fetch_exposed_frac=exposed_ms / fetch_ms if fetch_ms else None,
                hidden_cap=min(1.0, ffn_ms / fetch_ms) if fetch_ms else None)


def run_decode_loop(device, steps, pool):
    """Qwen3-30B-A3B decode loop over all 48 MoE layers: a 1024-token prefill layer pass, then
    ``steps`` steps of 64 tokens, routing from the seeded temporal-locality process, a pooled
    cache of 1,843 slots with GateHistory W = 128 eviction.  The steps run twice over: the
    throughput from ``steps`` plain steps, then the fetch / compute split from ``steps`` more
    steps with per-launch timing on (which adds events of its own)."""
    import hashlib
    from ferry_amd import expert_ops as ops
    from ferry_amd import workloads
    from ferry_amd.quota import Topology
    from ferry_amd.runtime import OffloadRuntime
    w = workloads.QWEN3_DECODE_LOOP
    spec = w.spec
    L, E, H = w.layers, spec.experts, spec.hidden
    routing = workloads.decode_loop_routing(w, steps=2 * steps)
    rt = OffloadRuntime(spec, pool, [w.cache_slots], 'ferry', Topology.uniform(1, E))
    g = torch.Generator(device=device)
    g.manual_seed(w.seed)
    xs = {T: torch.randn((T, H), generator=g, device=device).to(torch.bfloat16)
          for T in (w.prefill_tokens, w.tokens)}
    digest = hashlib.sha1()
    torch.cuda.synchronize()
    gc.collect()
    t0 = time.perf_counter()
    for layer in range(L):
        sel = torch.from_numpy(routing['prefill'][layer]).to(device)
        rt.execute(layer, xs[w.prefill_tokens], sel, routing['prefill_weights'][layer].to(device), None)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    prefill_copies = rt.h2d.copies

    def steps_pass(first):
        for s in range(first, first + steps):
            for layer in range(L):
                sel = torch.from_numpy(routing['decode'][s, layer]).to(device)
                rt.execute(layer, xs[w.tokens], sel, routing['decode_weights'][s, layer].to(device),
                           None)
            if first == 0:
                digest.update(rt.controller.slots[0].tobytes())
        torch.cuda.synchronize()

    t2 = time.perf_counter()
    steps_pass(0)
    t3 = time.perf_counter()
    copies = rt.h2d.copies - prefill_copies
    rt.timing = True
    ops.timing_enable(True)
    before = rt.h2d.copies
    steps_pass(steps)
    timed_copies = rt.h2d.copies - before
    ffn = sum(ops.timing_summary(n)[1] for n in
              ('ffn_skinny_fused', 'ffn_up_skinny', 'ffn_tiled_up', 'ffn_down_skinny',
               'ffn_tiled_down'))
    fetch_ms, exposed_ms, overlap_ms = rt.fetch_timing()
    ops.timing_enable(False)
    calls = steps * L
    res = dict(
        workload=w.name, layers=L, steps=steps, tokens_per_step=w.tokens, cache_slots=w.cache_slots,
        prefill_ms_per_layer=(t1 - t0) / L * 1e3, prefill_fetches=prefill_copies,
        decode_tokens_per_s=w.tokens * steps / (t3 - t2),
        decode_ms_per_layer_step=(t3 - t2) / calls * 1e3,
        misses_per_layer_step=copies / calls,
        h2d_gbs=timed_copies * spec.expert_bytes / (fetch_ms * 1e-3) / 1e9 if fetch_ms else None,
        fetch_ms_per_layer_step=fetch_ms / calls,
        fetch_hidden_frac=overlap_ms / fetch_ms if fetch_ms else None,
        fetch_exposed_frac=exposed_ms / fetch_ms if fetch_ms else None,
        ffn_ms_per_layer_step=ffn / calls,
        hidden_cap=min(1.0, ffn / fetch_ms) if fetch_ms else None,
        eviction_state_sha1=digest.hexdigest(),
        note=('throughput, misses and eviction state from the plain steps; fetch, FFN and hidden '
              'fractions from as many further steps with per-launch timing on; the reference\'s loop runs 64 '
              'steps'))
    rt.close()
    return res


# ---------------------------------------------------------------------------------------------
# end-to-end generation: the reference's serving metrics
# ---------------------------------------------------------------------------------------------

def qwen3_30b_a3b_config():
    """The HF config of Qwen3-30B-A3B's architecture (its published config.json values)."""
    from transformers import Qwen3MoeConfig
    return Qwen3MoeConfig(
        vocab_size=151936, hidden_size=2048, intermediate_size=6144, moe_intermediate_size=768,
        num_hidden_layers=48, num_attention_heads=32, num_key_value_heads=4, head_dim=128,
        num_experts=128, num_experts_per_tok=8, norm_topk_prob=True, decoder_sparse_step=1,
        mlp_only_layers=[], max_position_embeddings=40960, rms_norm_eps=1e-6,
        tie_word_embeddings=False, rope_parameters={'rope_type': 'default', 'rope_theta': 1e6})


def run_generate(args, device, packed):
    """The reference's serving measurement (scripts/run_cell.py:124-158) on one GPU: greedy
    generation through a Qwen3-30B-A3B-shaped model with random weights (dense weights N(0,
    0.02) on the GPU; the routed experts are the 48-layer pool's rows, fetched packed into a
    pooled 30 % cache of 1,843 slots, FERRY policy, W = 128), every MoE block hooked into
    OffloadRuntime.  One warm-up run on other prompts, ``--gen-discard`` unreported runs and
    ``--gen-repeats`` measured runs on the target prompts, each from an empty cache and
    released 200 ms after it is called; TTFT / TPOT / E2E / TPS as mean and sample std."""
    from ferry_amd.harness import run_repeats, summarize, synthetic_model
    from ferry_amd.model import QWEN3_30B_A3B, install_hooks, spec_from_config
    from ferry_amd.quota import Topology
    from ferry_amd.runtime import OffloadRuntime
    cfg = qwen3_30b_a3b_config()
    spec = spec_from_config(cfg)
    assert spec == QWEN3_30B_A3B
    cap = spec.cache_slots(0.30, 1)[0]
    t0 = time.perf_counter()
    model = synthetic_model(cfg, spec, device, seed=3)
    rt = OffloadRuntime(spec, packed, [cap], 'ferry', Topology.uniform(1, spec.experts))
    install_hooks(model, spec, rt, history_window=128)
    build_s = time.perf_counter() - t0
    g = torch.Generator(device=device)
    g.manual_seed(5)
    B, P = args.gen_batch, args.gen_prompt
    warm = torch.randint(0, cfg.vocab_size, (B, P), generator=g, device=device)
    target = torch.randint(0, cfg.vocab_size, (B, P), generator=g, device=device)

    def log(rec):
        print(f"# generate run {rec['repeat']} ({rec['phase']}): TTFT {rec['TTFT']:.3f} s, "
              f"TPOT {rec['TPOT'] * 1e3:.1f} ms, TPS {rec['TPS']:.1f}, "
              f"{rec['h2d_copies']} copies", file=sys.stderr, flush=True)

    t0 = time.perf_counter()
    records = run_repeats(model, rt, warm, target, steps=args.gen_output,
                          repeats=args.gen_repeats, discard=args.gen_discard, log=log)
    wall_s = time.perf_counter() - t0
    rt.close()
    summary = summarize(records)
    keep = ('repeat', 'phase', 'TTFT', 'TPOT', 'E2E', 'TPS', 'h2d_copies',
            'decode_fetches_per_rank', 'serial_wait_s', 'peak_allocated_bytes')
    out = dict(
        workload='qwen3_30b_a3b_generate_synthetic',
        config=dict(layers=spec.layers, experts=spec.experts, topk=spec.topk,
                    hidden=spec.hidden, intermediate=spec.intermediate, vocab=cfg.vocab_size,
                    attention='32 heads x 128, 4 KV heads, SDPA', batch=B, prompt_tokens=P,
                    output_tokens=args.gen_output, cache_slots=cap, history_window=128,
                    policy='ferry', fetch='packed rows, two DMA streams',
                    weights='random: dense N(0, 0.02) seed 3; experts = the stack pool rows',
                    prompts='uniform random token IDs, seeded'),
        repeats=args.gen_repeats, discarded=args.gen_discard,
        **{key: summary[key] for key in ('TTFT', 'TPOT', 'E2E', 'TPS')},
        units=dict(TTFT='s', TPOT='s', E2E='s', TPS='tokens/s'),
        runs=[{key: r[key] for key in keep} for r in records],
        model_build_s=build_s, wall_s=wall_s,
        note=('TTFT = first token - release, TPOT = (last - first) / (output_tokens - 1), '
              'TPS = batch * output_tokens / (last - release), as scripts/run_cell.py:150-154; '
              'random weights route near-uniformly, so the expert cache hits less often than '
              'with a trained model\'s temporal locality'))
    del model
    torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------------------------------------
# CPU baseline: the reference's op order in torch on the host cores
# ---------------------------------------------------------------------------------------------

def cpu_model():
    try:
        for line in Path('/proc/cpuinfo').read_text().splitlines():
            if line.startswith('model name'):
                return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_layer(logits, x, pool_rows, planner, hist, step, E, k, H, I, renorm=True):
    """One layer call in the reference's op order (model.py:141-146, metadata.py, policy.py,
    layout.py, expert_ops.cpp:54-121) with torch / numpy on the CPU."""
    from oracle.experts import execute_experts_ref, reduce_partials_ref
    from oracle.history import frequency_rows
    from oracle.layout import layout_closed_form
    probs = torch.softmax(logits, dim=-1, dtype=torch.float32)
    wts, sel = torch.topk(probs, k, dim=-1)
    if renorm:
        wts = wts / wts.sum(-1, keepdim=True)
    wts = wts.to(torch.bfloat16)
    if planner is not None:
        hist.update(0, frequency_rows(sel.numpy(), E, 128))
        planner.plan(step, 0, sel.numpy(), hist.scores(0))
    lay = layout_closed_form(sel.numpy(), E, wts.float().numpy())
    w_sorted = torch.from_numpy(lay['w_sorted']).to(torch.bfloat16)
    groups = [e for e in range(E) if lay['counts'][e] > 0]
    rows = [torch.from_numpy(lay['rows'][lay['starts'][e]:lay['starts'][e + 1]]) for e in groups]
    cols = [torch.from_numpy(lay['cols'][lay['starts'][e]:lay['starts'][e + 1]]) for e in groups]
    parts = execute_experts_ref([pool_rows(e) for e in groups], x, w_sorted, rows, cols, H, I)
    return reduce_partials_ref(parts, rows, x.shape[0], H)


def cpu_baseline(dec, seconds, device, with_prefill=True):
    from oracle.history import GateHistoryRef
    from oracle.policy import PlannerRef
    from ferry_amd import workloads
    w = dec['workload']
    spec = w.spec
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    E, k, H, I = spec.experts, spec.topk, spec.hidden, spec.intermediate
    pool = workloads.make_pool(spec, 1, seed=0).cpu()   # same rows as the GPU pool
    samples = [(lg.cpu(), x.cpu()) for lg, x in dec['samples']]
    planner, hist = PlannerRef(1, E, w.cache_slots), GateHistoryRef(1, E, 128)
    step = 0

    def run(n):
        nonlocal step
        for _ in range(n):
            lg, x = samples[step % len(samples)]
            cpu_layer(lg, x, lambda e: pool[e], planner, hist, step, E, k, H, I)
            step += 1

    run(3)   # warm-up
    t0 = time.perf_counter()
    run(5)
    per_step = (time.perf_counter() - t0) / 5
    n = max(5, int(seconds / 5 / per_step))
    rates = []
    for _ in range(5):
        t0 = time.perf_counter()
        run(n)
        rates.append(n * w.tokens / (time.perf_counter() - t0))
    out = dict(value=statistics.median(rates), unit='tokens/s', cores=cores, kind='port',
               cpu_model=cpu_model(), repeats=[round(r, 1) for r in rates], statistic='median of 5',
               sample=f'5 repeats x {n} decode steps ({n * w.tokens} tokens) of the same seeded '
                      f'stream (the decode layer); experts read from host memory (no H2D copy on the CPU '
                      f'path)')
    if with_prefill:
        # one Qwen3 8192-token prefill layer (experts resident in host memory)
        w3 = workloads.QWEN3_PREFILL_STACK
        T = w3.tokens
        lg = workloads.RouterLogits(replace(w3, layers=1), device).next(0, T).cpu()
        x = workloads.hidden_states(T, H, seed=w3.seed + 7, device=device).cpu()
        rows3 = workloads.expert_rows(range(E), spec.expert_elements, seed=w3.seed, device=device).cpu()
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            cpu_layer(lg, x, lambda e: rows3[e], None, None, 0, E, k, H, I)
            times.append(time.perf_counter() - t0)
        layer_s = statistics.median(times)
        out['prefill_layer'] = dict(
            workload='qwen3_30b_a3b_moe_prefill_t8192_layer_resident', layer_s=layer_s,
            tokens_per_s=T / layer_s, repeats_s=[round(t, 3) for t in times],
            statistic='median of 3',
            stack_48_layers_s=48 * layer_s,
            extrapolation='48 x the median layer time (each layer has the same shape; fetches '
                          'are not modelled on the CPU path)')
    return out


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
    warm_up_runtime(device)
    dec = run_decode(args, device, pack=True)
    w = dec['workload']
    roofline, block = decode_block(dec, args)
    pk = dec['packing']
    block['packing'] = dict(
        ratio=pk['ratio'], packed_rows=pk['packed_rows'],
        link_gbs=(dec['copies'] * pk['packed_bytes'] / pk['packed_rows'])
        / (dec['fetch_ms'] * 1e-3) / 1e9 if dec['fetch_ms'] else None,
        note='the misses cross the host link as packed rows (per value a sign|mantissa byte and '
             'a 2-bit exponent code, escapes in three more levels, lossless) into staging buffers '
             'and are unpacked into the cache slots on the GPU; h2d_gbs counts expert bytes '
             'delivered, link_gbs the packed bytes copied')
    line = dict(
        metric='MoE-layer tokens/sec (Qwen3-30B-A3B-shaped decode layer, 16 tok/step, 38/128 cached)',
        value=dec['tokens'] / dec['elapsed'], unit='tokens/s', n_gpus=1, steps=args.steps,
        warmup=args.warmup, ms_per_step=dec['elapsed'] / args.steps * 1e3, higher_is_better=True,
        scaling='weak', vs_baseline=None, dtype='bf16', data='synthetic',
        config=dict(workload=w.name, tokens_per_step=w.tokens, experts=w.spec.experts,
                    topk=w.spec.topk, hidden=w.spec.hidden, intermediate=w.spec.intermediate,
                    cache_slots=w.cache_slots, router='N(0,1)+log Zipf(1.1), seed 1',
                    expert_weights='N(0, 0.02) bf16, seeded',
                    fetch='hipMemcpyAsync of packed rows on two DMA streams, unpacked on the GPU',
                    parallelism='single GPU (one expert-parallel share)'),
        roofline=roofline, decode=block)
    block['read_ceiling'] = read_ceiling(device, block, w.spec.expert_bytes)
    roofline['read_ceiling_gbs'] = block['read_ceiling']['both_gbs']
    roofline['frac_of_read_ceiling'] = roofline['achieved'] / block['read_ceiling']['both_gbs']
    print(f'# decode done: {line["value"]:.0f} tokens/s', file=sys.stderr, flush=True)
    # the same decode stream with the copy kernel on the compute stream (not the reference's
    # fetch scheme, so not the headline): one launch per fetch, then one FFN launch
    dk = run_decode(args, device, copy='kernel')
    rk, bk = decode_block(dk, args)
    line['decode_copy_kernel'] = dict(
        tokens_per_s=dk['tokens'] / dk['elapsed'], ms_per_step=dk['elapsed'] / args.steps * 1e3,
        h2d_gbs=bk['h2d_gbs'], fetch_ms_per_step=bk['fetch_ms_per_step'],
        fetch_hidden_frac=bk['fetch_hidden_frac'], ffn_kernel=rk['kernel'],
        ffn_avg_launch_us=rk['avg_launch_us'], ffn_launches=rk['launches'],
        ffn_gbs=rk['achieved'], ffn_frac=rk['frac'],
        note='copy=kernel: the misses of a step are copied by one kernel launch on the compute '
             'stream, then every active expert runs in one FFN launch (no overlap)')
    print(f'# decode (copy kernel) done: {line["decode_copy_kernel"]["tokens_per_s"]:.0f} tokens/s',
          file=sys.stderr, flush=True)
    # the headline stream with each packed call's fetched experts computed sub-batch by
    # sub-batch as the engine unpacks them (OffloadRuntime(split_fetch=True)): a shorter tail
    # after the last copy, for more and smaller FFN launches
    ds = run_decode(args, device, pack=True, split_fetch=True)
    rs, bs = decode_block(ds, args)
    line['decode_split_fetch'] = dict(
        tokens_per_s=ds['tokens'] / ds['elapsed'], ms_per_step=ds['elapsed'] / args.steps * 1e3,
        ffn_launches=rs['launches'], ffn_avg_launch_us=rs['avg_launch_us'], ffn_gbs=rs['achieved'],
        ffn_frac=rs['frac'], fetch_hidden_frac=bs['fetch_hidden_frac'],
        hidden_cap=bs['hidden_cap'], critical_path_us=bs['critical_path_us'],
        note='OffloadRuntime(pack=True, split_fetch=True): one FFN launch per unpacked '
             'sub-batch of a call\'s fetched experts instead of one after the last copy; not '
             'the headline, whose single fetched-expert launch keeps the decode FFN at a '
             'higher fraction of HBM peak')
    print(f'# decode (split fetch) done: {line["decode_split_fetch"]["tokens_per_s"]:.0f} tokens/s',
          file=sys.stderr, flush=True)
    # the same decode stream fetching raw rows, as the reference's engine does
    dr = run_decode(args, device, pack=False)
    rr, br = decode_block(dr, args)
    line['decode_raw'] = dict(
        tokens_per_s=dr['tokens'] / dr['elapsed'], ms_per_step=dr['elapsed'] / args.steps * 1e3,
        h2d_gbs=br['h2d_gbs'], fetch_ms_per_step=br['fetch_ms_per_step'],
        fetch_hidden_frac=br['fetch_hidden_frac'], ffn_frac=rr['frac'],
        note='OffloadRuntime(pack=False): raw bf16 rows over the host link')
    print(f'# decode (raw rows) done: {line["decode_raw"]["tokens_per_s"]:.0f} tokens/s',
          file=sys.stderr, flush=True)
    # the reference's fetch scheme on this library's kernels: raw rows, and the host waits for
    # every copy before any expert runs (OffloadRuntime(overlap=False, pack=False))
    dsr = run_decode(args, device, pack=False, overlap=False)
    line['decode_serial_raw'] = dict(
        tokens_per_s=dsr['tokens'] / dsr['elapsed'], ms_per_step=dsr['elapsed'] / args.steps * 1e3,
        note='OffloadRuntime(overlap=False, pack=False): the reference\'s serial fetch wait and '
             'raw rows, with this library\'s kernels')
    print(f'# decode (serial, raw rows) done: {line["decode_serial_raw"]["tokens_per_s"]:.0f} '
          'tokens/s', file=sys.stderr, flush=True)
    if not args.no_prefill:
        from ferry_amd import workloads
        line['prefill'] = run_prefill(args, device, workloads.QWEN3_PREFILL_STACK)
        line['roofline_prefill'] = prefill_roofline(line['prefill'])
        line['prefill']['small_expert_ceiling'] = small_expert_ceiling(
            device, line['prefill'], workloads.QWEN3_PREFILL_STACK.spec)
        line['prefill_deepseek'] = run_prefill(args, device, workloads.DEEPSEEK_PREFILL_STACK)
        line['gemm_ceiling_hipblaslt'] = gemm_ceiling(device)
        line['tiled_dense'] = tiled_dense(device)
        line['reference_pattern_gpu'] = reference_pattern_gpu(device)
        for key, shape in (('up_65536x1536x2048', 'dense_up_65536x1536x2048'),
                           ('down_65536x2048x768', 'dense_down_65536x2048x768')):
            line['tiled_dense'][key]['vs_hipblaslt'] = (
                line['tiled_dense'][key]['tflops'] / line['gemm_ceiling_hipblaslt'][shape]['tflops'])
        print('# prefill layers done', file=sys.stderr, flush=True)
    if not args.no_stacks:
        line.update(run_stacks(args, device))
    if not args.no_cpu_baseline:
        line['cpu_baseline'] = cpu_baseline(dec, args.cpu_seconds, device,
                                            with_prefill=not args.no_prefill)
    print(json.dumps(line), flush=True)


if __name__ == '__main__':
    main()
