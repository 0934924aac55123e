"""One-GPU offloading runtime for routed experts (reference: ferry/runtime.py).

Per MoE layer call (world = 1):
  1. history: the device window counters of the layer are updated from ``selected``; the
     same kernel writes the expert IDs (uint8) and the layer's scores straight into mapped
     host memory -- the host must know the misses to enqueue fetches;
  2. the layout kernel is enqueued before the host waits for those results, so it overlaps
     the host planning;
  3. the C++ planner picks the misses (ascending expert) and their slots (routing-aware
     eviction, bit-exact with the reference) and the H2D engine enqueues their copies on its
     own stream;
  4. the misses are copied with ``hipMemcpyAsync`` on the fetch engine's DMA streams while the
     experts already resident run; the compute stream then waits on the GPU for the copies and
     runs the fetched experts.  A prefill-sized call copies its misses in a few groups,
     heaviest expert first, each computed as soon as its copies land, so that only the
     lightest group's compute is left after the last copy; a decode-sized call runs all its
     misses in one launch after the last copy (``split_fetch=True``, with packed rows: one
     launch per sub-batch as the engine unpacks it).  ``overlap=False`` restores the
     reference's serial host wait.  ``copy='kernel'`` (not the reference's scheme) copies a
     decode-sized call's misses with one copy-kernel launch on the compute stream instead and
     then runs every active expert in one FFN launch: no idle link between copies and no
     cross-queue wait, but no overlap either (the copy kernel's host reads slow the HBM-bound
     kernels that run beside it, so nothing runs beside it);
  5. the combine kernel sums each token's k expert rows in fp32 (ascending expert ID).

The one-launch decode FFN bounds its cross-workgroup wait; a wait that gives up leaves rows
unwritten and counts a timeout on the device.  The history kernel copies that count next to the
routing IDs, so the next call raises RuntimeError when it grew (an earlier call's output is then
invalid), and so do ``reset`` and ``close``.
"""
import time

import numpy as np
import torch
import torch.distributed as dist

from . import expert_ops as ops
from .hostmem import mapped_buffer
from .metadata import DeviceGateHistory, GateHistory, RouteGather
from .policy import Controller, layer_slots
from .transport import Transport


# A layer call with at least this many (token, expert) pairs fetches its misses in up to CHUNKS
# groups, heaviest first, and computes each group as soon as its copies land.  Decode calls
# (few pairs, little compute per expert) keep one group and one launch for their misses: with
# packed rows, one launch per unpacked sub-batch (OffloadRuntime(split_fetch=True)) shortens
# the step by about 1 % but adds a launch's fixed cost of GPU time for each.
CHUNK_MIN_PAIRS = 16384
CHUNKS = 6


def expert_ops():
    """The native op module (reference: ferry/runtime.py:26-31)."""
    return ops


class OffloadRuntime:
    def __init__(self, spec, pool, capacities, policy, topology, history_window=128,
                 balance_tol_bps=200, salt=1, eviction_score='frequency', overlap=True,
                 timing=False, copy='dma', pack=False, pack_threads=16, split_fetch=False):
        if dist.is_available() and dist.is_initialized() and dist.get_world_size() != 1:
            raise NotImplementedError('ferry_amd runs on one GPU (world = 1)')
        if len(capacities) != 1:
            raise NotImplementedError('ferry_amd runs on one GPU (world = 1)')
        self.spec = spec
        self.pool = pool
        self.rank, self.world = 0, 1
        self.capacities = capacities
        self.cap = capacities[0]
        self.window = history_window
        self.overlap = overlap
        self.timing = timing
        if copy not in ('dma', 'kernel'):
            raise ValueError("copy must be 'dma' or 'kernel'")
        self.copy = copy
        # packed decode calls: compute the fetched experts sub-batch by sub-batch as the engine
        # unpacks them (one FFN launch per sub-batch) instead of in one launch after the last
        self.split_fetch = bool(split_fetch)
        # a lossless packed copy of the pool for the host link, made once; every engine of this
        # runtime fetches packed rows in DMA mode and unpacks them on the GPU
        # (pack: True, or a PackedPool of this pool built by the caller and shared; ``pool``
        # itself may be a PackedPool, whose engines need no raw pool)
        from .h2d import PackedPool
        self.packed = None
        if isinstance(pool, PackedPool):
            self.packed = pool
        elif pack is not None and pack is not False:
            self.packed = pack if isinstance(pack, PackedPool) else PackedPool(pool, pack_threads)
        self.ops = expert_ops()
        self.device = torch.device('cuda', torch.cuda.current_device())
        self.cache = torch.empty((self.cap, spec.expert_elements), dtype=torch.bfloat16,
                                 device=self.device)
        self.controller = Controller(spec, capacities, policy, topology, balance_tol_bps, salt)
        self.gather = RouteGather(spec.topk, spec.experts, history_window, eviction_score)
        self.transport = Transport(self.ops, spec.topk, spec.experts)
        # mapped host staging: [scores f32 E | IDs u8 T*k | pad | timeouts i32 | ready i32 ...]
        self._stage_host = None
        self._bufs = {}
        self._ready_seq = 0
        # calls wait for their routing IDs by polling the history kernel's ready words (False:
        # on the event recorded after that kernel)
        self._poll_ids = True
        self.h2d = None
        self.reset()

    # -- state -------------------------------------------------------------------------------

    def reset(self):
        """Empty expert cache and routing history (start of every measured run).  Raises
        RuntimeError (after the reset) if a decode FFN wait gave up since the last check."""
        self._flush_used()
        if self.h2d is not None:
            self.h2d.synchronize()
        torch.cuda.synchronize(self.device)
        late = self._timeouts_since_check()
        self.controller.reset()
        spec = self.spec
        self.history = GateHistory(spec.layers, spec.experts, self.window)
        self.device_history = DeviceGateHistory(spec.layers, spec.experts, spec.topk, self.window,
                                                self.device)
        # the engine is reset in place rather than rebuilt: a new engine's streams can land on
        # the hardware queue of this runtime's compute stream and serialise with it
        if self.h2d is not None:
            self.h2d.reset()
        elif self.packed is not None:
            self.h2d = self.ops.H2DEngine.from_packed(self.cache, self.packed)
        else:
            self.h2d = self.ops.H2DEngine(self.cache, self.pool)
        self._kernel_copy = self.copy == 'kernel' and self.h2d.kernel_ok
        self._defer_last = False
        if self.copy == 'kernel' and not self._kernel_copy:
            raise RuntimeError("copy='kernel' needs a device-mapped pool with 16-byte rows")
        self._copy_mode = None
        self.event = 0
        self.fetches_per_rank = np.zeros(self.world, np.int64)
        self.decode_fetches_per_rank = np.zeros(self.world, np.int64)
        self.serial_wait_ns = 0
        self.timings = []
        self.step_marks = []   # timing=True: (ids ready, copies queued, copies done, compute resumes)
        self.kernel_bytes = dict(up=0, down=0, flops=0, experts=0, launches=0)
        # host time per phase of execute (ns, timing=True): the planning path between the
        # wait for the routing IDs and the fetch enqueue is on the critical path of a step
        self.host_ns = dict(enqueue_before_wait=0, wait_for_ids=0, plan=0, fetch_enqueue=0,
                            enqueue_after_fetch=0)
        if late:
            raise RuntimeError(self._timeout_message(late))

    # -- decode FFN timeouts -----------------------------------------------------------------

    def _timeouts_since_check(self):
        """Device-wide decode FFN timeouts counted since the last check (reads the device)."""
        now = self.ops.ffn_sync_timeouts()
        seen = getattr(self, '_timeouts_seen', now)
        self._timeouts_seen = now
        return now - seen

    @staticmethod
    def _timeout_message(n):
        return (f'{n} wait(s) of the one-launch decode FFN gave up on this device: the rows of '
                f'those experts were not written, so the output of an earlier layer call is '
                f'invalid')

    def _status_offset(self, tokens):
        """Byte offset of the timeout word in the staging buffer of a ``tokens``-token call."""
        return 4 * self.spec.experts + (tokens * self.spec.topk + 3) // 4 * 4

    def _buffers(self, tokens):
        b = self._bufs.get(tokens)
        if b is None:
            spec, k = self.spec, self.spec.topk
            b = dict(act=torch.empty((tokens * k, spec.intermediate), dtype=torch.bfloat16,
                                     device=self.device),
                     part=torch.empty((tokens * k, spec.hidden), dtype=torch.bfloat16,
                                      device=self.device),
                     layout=None, ready_n=self.ops.history_ready_words(tokens, k))
            self._bufs[tokens] = b
        # staging layout: scores | IDs | timeout word | the history kernel's ready words
        n = self._status_offset(tokens) + 4 + 4 * b['ready_n']
        if self._stage_host is None or self._stage_host.numel() < n:
            # coherent mapped host memory: the history kernel writes the layer's scores, the
            # uint8 IDs, the timeout count and its ready words straight into it, so the host
            # needs no D2H copy
            self._stage_host, self._stage_ptr = mapped_buffer(max(n, 4096))
            self._stage_host_ptr = self._stage_host.data_ptr()
            # int32 view for the timeout word (read right after the routing readback, on the
            # path to the first copy: a torch slice and view there cost about 10 us)
            self._stage_i32 = self._stage_host.numpy().view(np.int32)
        return b

    # -- one layer call ------------------------------------------------------------------------

    def execute(self, layer, hidden, selected, weights, probs_tail, shared=None):
        """One MoE layer call (runtime.py:64-89).  ``shared`` (an ``expert_ops.SharedExpert``,
        not a reference argument) adds an always-on expert's output to every token, as
        DeepSeek-V2's block does after the routed experts; it runs while the misses copy."""
        t_enter = time.perf_counter_ns()
        spec = self.spec
        T, k = selected.shape
        E = spec.experts
        if hidden.dtype != torch.bfloat16 or hidden.dim() != 2 or hidden.shape[1] != spec.hidden:
            raise RuntimeError('hidden must be bf16 [tokens, hidden]')
        stream = torch.cuda.current_stream(self.device)
        buf = self._buffers(T)
        selected = selected.contiguous()
        weights = weights.to(torch.bfloat16).contiguous()

        # 1. history; the kernel writes scores, IDs and the device's decode FFN timeout count
        # into the mapped host staging buffer (with probability scores its scores go unused)
        frequency = self.gather.score == 'frequency'
        nbytes = 4 * E + T * k
        stage_host = self._stage_host[:nbytes]
        status = self._status_offset(T)
        # the ready words after the timeout word carry this call's number once the kernel's
        # host-memory writes are visible
        self._ready_seq = self._ready_seq % 0x7FFFFFFF + 1
        seq = self._ready_seq
        self.device_history.update(layer, selected, self._stage_ptr, self._stage_ptr + 4 * E,
                                   self._stage_ptr + status, self._stage_ptr + status + 4, seq)
        tail_host = None
        if not frequency:
            tail = min(T, self.window)
            tail_host = probs_tail[-tail:].float().to('cpu', non_blocking=True)
        if self.timing:
            # timestamp of the routing IDs (the history kernel's end) for critical_path_timing
            d2h = torch.cuda.Event(enable_timing=True)
            d2h.record(stream)
        # one event both releases the IDs to the host and marks the slots that the previous call
        # read on this stream (no event of their own between that call's kernels)
        pend = self._pending_used
        if pend is not None and pend[1] != stream.cuda_stream:
            self._flush_used()
            pend = None
        self._pending_used = None
        ids_event = self.h2d.mark_used_record(pend[0] if pend is not None else [], stream)
        if self._poll_ids:
            # poll the history kernel's ready words: they are seen about 5 us before the event's
            # wait returns, and they show the previous call's slot reads complete
            words, nw = self._stage_host_ptr + status + 4, buf['ready_n']
            wait_ids = lambda: self.h2d.wait_ready(ids_event, words, nw, seq)   # noqa: E731
        else:
            wait_ids = lambda: self.h2d.event_synchronize(ids_event)   # noqa: E731

        # 2. layout (overlaps the host planning)
        buf['layout'] = self.ops.layout(selected, weights, E, out=buf['layout'])
        lay = buf['layout']
        chunked = T * k >= CHUNK_MIN_PAIRS
        on_stream = self.overlap and not chunked and self._kernel_copy
        # packed decode calls: the last sub-batch's unpack runs on this stream right after the
        # copies (one cross-queue wait before the fetched experts, not two)
        defer = (self.packed is not None and self.overlap and not chunked and not on_stream
                 and not self.timing)
        if defer != self._defer_last:
            self.h2d.defer_last = defer
            self._defer_last = defer

        # 3. plan + fetch
        t_sync = time.perf_counter_ns()
        wait_ids()
        t_ready = time.perf_counter_ns()
        count = int(self._stage_i32[status // 4])
        if count != self._timeouts_seen:
            late, self._timeouts_seen = count - self._timeouts_seen, count
            raise RuntimeError(self._timeout_message(late))
        self._set_copy_mode(on_stream, stream)
        # with chunks or timing the copies are queued here; otherwise the planner's native call
        # queues them itself, right after planning
        queue_here = chunked or self.timing
        if frequency:
            fetches, counts = self.controller.plan_fetch(
                self.event, layer, self._stage_ptr + 4 * E, T, k, self._stage_ptr,
                None if queue_here else self.h2d.handle)
        else:
            self.history.update(layer, tail_host.numpy())
            scores = self.history.scores(layer)
            ids = stage_host.numpy()[4 * E:].astype(np.int64).reshape(T, k)
            fetches, _, counts = self.controller.plan(self.event, layer, ids, np.zeros(T, np.int64),
                                                      scores)
            queue_here = True
        t_plan = time.perf_counter_ns()
        if frequency:
            counts_e = self.controller.demand.copy()   # counted by the planner in its ID pass
        else:
            counts_e = np.bincount(ids.reshape(-1), minlength=E)
        missing_keys = fetches[:, 1] - layer * E
        # copy order: heaviest expert first, so that the compute left after the last copy is
        # the lightest (the planner's slot choices do not depend on the order of the copies)
        if chunked and len(fetches) > 1:
            order = np.argsort(-counts_e[missing_keys], kind='stable')
            groups = [g for g in np.array_split(order, min(CHUNKS, len(fetches))) if len(g)]
        else:
            groups = [np.arange(len(fetches))]
        timing = self.timing and len(fetches) > 0
        if timing:
            copy_stream = stream if on_stream else self.h2d.stream
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
            ev[0].record(copy_stream)
        if queue_here and len(fetches):
            for g in groups:
                self.h2d.fetch(fetches[g, 2], fetches[g, 1])
        if (self.split_fetch and not chunked and not on_stream and self.packed is not None
                and len(fetches) > 1):
            # each sub-batch's experts run as soon as the engine has unpacked it, so only the
            # last sub-batch's experts follow the call's last copy
            ends = self.h2d.groups()
            if len(ends) > 1:
                groups = [np.arange(a, b) for a, b in zip([0] + ends[:-1], ends)]
        t_fetch = time.perf_counter_ns()
        self.fetches_per_rank += counts
        if self.event >= spec.layers:
            self.decode_fetches_per_rank += counts
        if timing:
            ev[1].record(copy_stream)

        # 4. experts: resident first, then the fetched ones (chunk by chunk as they land)
        slot_of = layer_slots(self.controller.slots[0], self.cap, layer, E)
        active = counts_e > 0
        missing = np.zeros(E, bool)
        missing[missing_keys] = True
        resident_list = np.flatnonzero(active & ~missing)
        slot32 = slot_of.astype(np.int32)
        common = (self.cache, hidden.contiguous(), lay.w_sorted, lay.starts, lay.rows, lay.cols)
        if not self.timing:
            # the reads below are marked by the next call's ID event on this stream (or by
            # _flush_used); set before they are queued, so that a call that fails part-way still
            # orders later copies into these slots after whatever it queued
            self._pending_used = (slot_of[np.flatnonzero(active)], stream.cuda_stream, stream)
        if not self.overlap and len(fetches):
            started = time.perf_counter_ns()
            self.h2d.wait_host(fetches[:, 2])
            self.serial_wait_ns += time.perf_counter_ns() - started
        mark = self.ops.timing_mark() if timing else 0
        waits = []
        if on_stream:
            # the copies are queued on this stream (the wait on their events costs nothing);
            # resident rows may come from DMA copies of earlier calls
            active_list = np.flatnonzero(active)
            self.h2d.wait_stream(slot_of[active_list], stream)
            if timing:
                waits.append((ev[0], ev[1]))   # the copy kernel holds this stream
            self._ffn(common, active_list, slot32, buf, stream, counts_e)
        elif len(resident_list):
            self.h2d.wait_stream(slot_of[resident_list], stream)
            self._ffn(common, resident_list, slot32, buf, stream, counts_e)
        shared_out = shared(common[1], out=self._shared_out(T)) if shared is not None else None
        if len(fetches) and not on_stream:
            for g in groups:
                w0 = w1 = None
                if timing:
                    w0 = torch.cuda.Event(enable_timing=True)
                    w0.record(stream)
                self.h2d.wait_stream(fetches[g, 2], stream)
                if timing:
                    w1 = torch.cuda.Event(enable_timing=True)
                    w1.record(stream)
                    waits.append((w0, w1))
                self._ffn(common, np.sort(missing_keys[g]), slot32, buf, stream, counts_e)
        if self.timing:
            self.h2d.mark_used(slot_of[np.flatnonzero(active)], stream)
        if timing:
            self.timings.append((ev, waits, (mark, self.ops.timing_mark())))
            self.step_marks.append((d2h, ev[0], ev[1], waits[-1][1] if waits else None))
        self.event += 1

        # 5. combine (+ the shared experts' output)
        out = self.ops.combine(buf['part'], T, k, spec.hidden, addend=shared_out)
        if self.timing:
            h = self.host_ns
            h['enqueue_before_wait'] += t_sync - t_enter
            h['wait_for_ids'] += t_ready - t_sync
            h['plan'] += t_plan - t_ready       # with frequency scores: plan + fetch enqueue
            h['fetch_enqueue'] += t_fetch - t_plan
            h['enqueue_after_fetch'] += time.perf_counter_ns() - t_fetch
        return out

    def _flush_used(self):
        """Mark the slots of the last call as read, with an event of their own."""
        pend = getattr(self, '_pending_used', None)
        if pend is not None and self.h2d is not None:
            self.h2d.mark_used(pend[0], pend[2])
        self._pending_used = None

    def _set_copy_mode(self, on_stream, stream):
        """Copy kernel on ``stream`` for on-stream calls, DMA copies otherwise."""
        from .h2d import DMA, KERNEL
        mode = (on_stream, stream.cuda_stream if on_stream else None)
        if mode != self._copy_mode:
            self.h2d.engine = KERNEL if on_stream else DMA
            self.h2d.set_kernel_stream(stream if on_stream else None)
            self._copy_mode = mode

    def _shared_out(self, tokens):
        b = self._bufs[tokens]
        if 'shared' not in b:
            b['shared'] = torch.empty((tokens, self.spec.hidden), dtype=torch.bfloat16,
                                      device=self.device)
        return b['shared']

    def _ffn(self, common, expert_list, slot32, buf, stream, counts_e):
        """Phase 1 (gate/up + SwiGLU) and phase 2 (down + weight) for ``expert_list``."""
        spec = self.spec
        self.ops.expert_ffn(*common, expert_list, slot32, spec.hidden, spec.intermediate,
                            buf['act'], buf['part'], out_mode=0, experts=spec.experts,
                            counts=counts_e)
        if self.timing:
            H, I = spec.hidden, spec.intermediate
            rows = int(counts_e[expert_list].sum())
            d = len(expert_list)
            # algorithmic bytes: weights read once, x / activation rows read, outputs written
            self.kernel_bytes['up'] += d * 2 * I * H * 2 + rows * (H * 2 + I * 2)
            self.kernel_bytes['down'] += d * H * I * 2 + rows * (I * 2 + H * 2 + 2)
            self.kernel_bytes['flops'] += 2 * 3 * H * I * rows
            self.kernel_bytes['experts'] += d
            self.kernel_bytes['launches'] += 1

    def fetch_timing(self):
        """(total fetch ms, exposed wait ms, overlapped compute ms) over the layer calls recorded
        with timing=True.  fetch: first copy start to last copy end on the copy stream.  exposed:
        how long the compute stream stalled on the copies.  overlapped: the time, inside each
        call's fetch window, covered by the compute kernels of that call (resident experts,
        shared experts, and missing experts whose copies landed early); it needs the library's
        per-launch timing (expert_ops.timing_enable)."""
        torch.cuda.synchronize(self.device)
        fetch = exposed = overlapped = 0.0
        for ev, waits, (m0, m1) in self.timings:
            fetch += ev[0].elapsed_time(ev[1])
            exposed += sum(max(0.0, a.elapsed_time(b)) for a, b in waits)
            overlapped += self.ops.timing_overlap(m0, m1, ev[0], ev[1])
        return fetch, exposed, overlapped

    def critical_path_timing(self):
        """Mean GPU-side gaps (ms) over the calls with copies recorded with timing=True: from the
        routing IDs being written (the history kernel's end) to the copies being queued (the
        host reads the IDs and plans in between), and from the last copy's end to the compute
        stream resuming after its wait for the copies."""
        torch.cuda.synchronize(self.device)
        plan, resume = [], []
        for d2h, q, done, w1 in self.step_marks:
            plan.append(d2h.elapsed_time(q))
            if w1 is not None:
                resume.append(done.elapsed_time(w1))
        mean = lambda v: sum(v) / len(v) if v else None   # noqa: E731
        return dict(ids_to_copy_queue_ms=mean(plan), copy_end_to_compute_ms=mean(resume),
                    calls=len(plan))

    def close(self):
        """Drain the runtime's work; raises RuntimeError if a decode FFN wait gave up since the
        last check."""
        self._flush_used()
        if self.h2d is not None:
            self.h2d.synchronize()
        torch.cuda.synchronize(self.device)
        late = self._timeouts_since_check()
        if late:
            raise RuntimeError(self._timeout_message(late))
