"""Python face of the HIP kernels (libferry_amd.so) with the reference's native-op names.

Reference: ``expert_ops()`` of ferry/runtime.py:26-31, i.e. the pybind11 module of
ferry/csrc/expert_ops.cpp:144-157 (execute_experts, pack_dispatch, unpack_dispatch,
reduce_partials, scatter_returned, H2DEngine).  The same names and argument meanings are kept
so that call sites written against the reference work unchanged; the fused hot-path entry
points (router_topk, layout, expert_ffn, combine, history_update) are exposed next to them.
All tensors are CUDA (HIP) tensors; every op runs on the current stream.
"""
import numpy as np
import torch

from ._lib import check, lib
from ._lib import check as _check_status
from .h2d import H2DEngine

__all__ = ['execute_experts', 'pack_dispatch', 'unpack_dispatch', 'reduce_partials',
           'scatter_returned', 'H2DEngine', 'router_topk', 'layout', 'expert_ffn', 'combine',
           'SharedExpert', 'history_update', 'history_ready_words', 'current_stream', 'PHASE_UP',
           'PHASE_DOWN', 'PHASE_BOTH']

MAX_EXPERTS = 512


def timing_enable(on=True):
    """Per-launch kernel timing: every kernel launch of the library gets a start/stop HIP event
    pair bracketing exactly that dispatch (hipExtLaunchKernel).  Turning it on clears the log."""
    check(lib().ferry_timing_enable(int(bool(on))), 'timing_enable')


def timing_summary(kernel):
    """(launches, total ms) of the timed launches of ``kernel`` (e.g. 'ffn_up_skinny')."""
    import ctypes
    n = ctypes.c_int64()
    ms = ctypes.c_double()
    check(lib().ferry_timing_summary(kernel.encode(), ctypes.byref(n), ctypes.byref(ms)),
          'timing_summary')
    return int(n.value), float(ms.value)


def timing_mark():
    """Position in the per-launch timing log (the number of launches recorded so far)."""
    return int(lib().ferry_timing_mark())


def timing_range(begin, end):
    """Summed ms of the timed launches at log positions [begin, end)."""
    import ctypes
    ms = ctypes.c_double()
    check(lib().ferry_timing_range(int(begin), int(end), ctypes.byref(ms)), 'timing_range')
    return float(ms.value)


def timing_overlap(begin, end, t0, t1):
    """ms that the timed launches at log positions [begin, end) overlap the window between
    two timing-enabled torch.cuda.Events (e.g. the first and last copy of a fetch)."""
    import ctypes
    ms = ctypes.c_double()
    check(lib().ferry_timing_overlap(int(begin), int(end), t0.cuda_event, t1.cuda_event,
                                     ctypes.byref(ms)), 'timing_overlap')
    return float(ms.value)


def current_stream(device=None):
    return torch.cuda.current_stream(device).cuda_stream


def _dev(t, name, dtype=None, contiguous=True):
    if not isinstance(t, torch.Tensor) or t.device.type != 'cuda':
        raise RuntimeError(f'{name} must be a CUDA tensor')
    if dtype is not None and t.dtype != dtype:
        raise RuntimeError(f'{name} must be {dtype}, got {t.dtype}')
    if contiguous and not t.is_contiguous():
        raise RuntimeError(f'{name} must be contiguous')
    return t.data_ptr()


# ------------------------------------------------------------------------------------------
# Hot-path entry points
# ------------------------------------------------------------------------------------------

def router_topk(logits, topk, renorm=True, scale=1.0, sorted=True, return_probs=False,
                tie_counter=None):
    """Softmax (fp32) + top-k + optional renorm, * scale, cast to bf16.

    Reference: ferry/model.py:141-146 (Qwen3: ``softmax(logits, -1, fp32)``, ``topk(k)``,
    ``w / w.sum(-1)``, ``.to(bf16)``) and the greedy DeepSeek-V2 gate reaching
    ferry/model.py:151-157 (``topk(sorted=False)``, ``* routed_scaling_factor``).
    Returns (weights bf16 [T, k], selected int64 [T, k]) and the fp32 probabilities when
    ``return_probs``.  Index selection is exactly torch's CPU ``topk``, ties included.
    """
    if logits.dim() != 2:
        raise RuntimeError('logits must be [tokens, experts]')
    dt = {torch.bfloat16: 0, torch.float32: 1}.get(logits.dtype)
    if dt is None:
        raise RuntimeError('logits must be bf16 or fp32')
    T, E = logits.shape
    idx = torch.empty((T, topk), dtype=torch.int64, device=logits.device)
    w = torch.empty((T, topk), dtype=torch.bfloat16, device=logits.device)
    probs = torch.empty((T, E), dtype=torch.float32, device=logits.device) if return_probs else None
    check(lib().ferry_router_topk(
        _dev(logits, 'logits'), dt, T, E, topk, int(bool(renorm)), float(scale), int(bool(sorted)),
        idx.data_ptr(), w.data_ptr(), probs.data_ptr() if probs is not None else None,
        _dev(tie_counter, 'tie_counter', torch.int32) if tie_counter is not None else None,
        current_stream(logits.device)), 'router_topk')
    return (w, idx, probs) if return_probs else (w, idx)


class Layout:
    """Device layout of one layer call (ferry/layout.py:12-94 at world = 1)."""

    __slots__ = ('tokens', 'topk', 'experts', 'send_ids', 'w_sorted', 'starts', 'rows', 'cols',
                 'pair_pos', 'workspace')


def layout_workspace_bytes(tokens, topk, experts):
    return int(lib().ferry_layout_workspace_bytes(tokens, topk, experts))


def layout_errors(lay):
    """Number of tokens of the last ``layout`` call into ``lay`` that had an expert ID outside
    [0, experts) or a repeated ID (waits for that call)."""
    return int(lay.workspace[:4].view(torch.int32).item())


def layout(selected, weights, experts, out=None, check=False):
    """Sorted packet IDs/weights, per-expert starts and the stable (rows, cols) permutation.

    Every token's IDs must be distinct and in [0, experts).  The kernel counts the tokens that
    break this; ``check=True`` waits for the result and raises RuntimeError when any did.
    """
    T, k = selected.shape
    dev = selected.device
    lay = out if out is not None else Layout()
    if out is None:
        lay.send_ids = torch.empty((T, k), dtype=torch.int64, device=dev)
        lay.w_sorted = torch.empty((T, k), dtype=torch.bfloat16, device=dev)
        lay.starts = torch.empty(experts + 1, dtype=torch.int64, device=dev)
        lay.rows = torch.empty(T * k, dtype=torch.int64, device=dev)
        lay.cols = torch.empty(T * k, dtype=torch.int64, device=dev)
        lay.pair_pos = torch.empty(T * k, dtype=torch.int32, device=dev)
        lay.workspace = torch.empty(layout_workspace_bytes(T, k, experts), dtype=torch.uint8,
                                    device=dev)
    lay.tokens, lay.topk, lay.experts = T, k, experts
    _check_status(lib().ferry_layout(
        _dev(selected, 'selected', torch.int64),
        _dev(weights, 'weights', torch.bfloat16) if weights is not None else None,
        T, k, experts, lay.send_ids.data_ptr(), lay.w_sorted.data_ptr(), lay.starts.data_ptr(),
        lay.rows.data_ptr(), lay.cols.data_ptr(), lay.pair_pos.data_ptr(),
        lay.workspace.data_ptr(), lay.workspace.numel(), current_stream(dev)), 'layout')
    if check:
        bad = layout_errors(lay)
        if bad:
            raise RuntimeError(f'layout: {bad} token(s) with an expert ID out of [0, {experts}) '
                               'or repeated')
    return lay


PHASE_UP, PHASE_DOWN, PHASE_BOTH = 1, 2, 3
SKINNY_MAX_ROWS = 64   # experts with at most this many rows run the small-expert kernels


def expert_ffn(cache, x, w_sorted, starts, rows, cols, expert_list, slot_of, hidden,
               intermediate, act, out, out_mode=0, max_rows=None, experts=None, phases=PHASE_BOTH,
               counts=None):
    """Grouped SwiGLU over cache slots for the experts in ``expert_list`` (host ints).

    phases: PHASE_UP (gate/up + SwiGLU into ``act``), PHASE_DOWN (down + routing weight from
    ``act`` into ``out``) or PHASE_BOTH.  ``counts`` (optional, host, indexed by expert) holds
    the row count of every expert, ``starts[e+1] - starts[e]``: the library then issues the
    experts with at most 64 rows (small-expert kernels, 17-64 rows first) and the larger ones
    (tiled kernels) as separate launches with exact row bounds, and skips experts without rows.
    """
    R, k = w_sorted.shape
    el = np.ascontiguousarray(expert_list, dtype=np.int32)
    so = np.ascontiguousarray(slot_of, dtype=np.int32)
    E = int(experts if experts is not None else len(so))
    args = (_dev(cache, 'cache', torch.bfloat16), cache.shape[0], hidden, intermediate,
            _dev(x, 'x', torch.bfloat16), R, k, _dev(w_sorted, 'w_sorted', torch.bfloat16),
            _dev(starts, 'starts', torch.int64), _dev(rows, 'rows', torch.int64),
            _dev(cols, 'cols', torch.int64))
    tail = (_dev(act, 'act', torch.bfloat16), _dev(out, 'out', torch.bfloat16), int(out_mode),
            int(phases), current_stream(x.device))

    if counts is None:
        check(lib().ferry_expert_ffn(*args, el.ctypes.data, len(el), so.ctypes.data, E,
                                     int(max_rows if max_rows is not None else R), 0, None, *tail),
              'expert_ffn')
        return out
    c = np.ascontiguousarray(np.asarray(counts, dtype=np.int64)[el], dtype=np.int32)
    if len(c):
        check(lib().ferry_expert_ffn(*args, el.ctypes.data, len(el), so.ctypes.data, E,
                                     int(c.max()), int(c.min()), c.ctypes.data, *tail),
              'expert_ffn')
    return out


def ffn_sync_timeouts():
    """Waits of the one-launch decode FFN that gave up on the current device (expected 0)."""
    import ctypes
    n = ctypes.c_int64()
    check(lib().ferry_expert_ffn_sync_timeouts(ctypes.byref(n)), 'ffn_sync_timeouts')
    return int(n.value)


def ffn_set_sync_spin_limit(limit):
    """How often a one-launch decode FFN's down phase polls for its up phase before it gives up
    (launches after the call): None or < 0 restores the default; 0 makes every wait give up at
    once, to check how a timeout is reported (no reference counterpart)."""
    check(lib().ferry_expert_ffn_set_sync_spin_limit(-1 if limit is None else int(limit)),
          'ffn_set_sync_spin_limit')


def hbm_read(buf, sink=None):
    """Read every byte of ``buf`` (a contiguous CUDA tensor, nbytes a multiple of 16) once at the
    HBM read rate, on the current stream: the measured read ceiling for the memory-bound
    kernels (no reference counterpart).  Returns ``sink`` (uint8, created when not given): one
    16-byte record per wavefront, the XOR of the 16-byte words it read."""
    if not (isinstance(buf, torch.Tensor) and buf.is_cuda and buf.is_contiguous()):
        raise RuntimeError('hbm_read: buf must be a contiguous CUDA tensor')
    nbytes = buf.numel() * buf.element_size()
    need = int(lib().ferry_hbm_read_sink_bytes(nbytes))
    if sink is None:
        sink = torch.empty(max(need, 16), dtype=torch.uint8, device=buf.device)
    st = torch.cuda.current_stream(buf.device).cuda_stream
    check(lib().ferry_hbm_read(buf.data_ptr(), nbytes, sink.data_ptr(), sink.numel(), st), 'hbm_read')
    return sink


def combine(part, tokens, topk, hidden, pair_pos=None, out=None, addend=None):
    """out[t] = bf16(sum_j fp32(part[src(t, j)])), j ascending (expert_ops.cpp:75-92).

    With ``addend`` (bf16 [tokens, hidden]) the result is bf16(fp32(out[t]) + fp32(addend[t])),
    the bf16 addition of the DeepSeek-V2 shared-expert output.
    """
    if out is None:
        out = torch.empty((tokens, hidden), dtype=torch.bfloat16, device=part.device)
    pp = _dev(pair_pos, 'pair_pos', torch.int32) if pair_pos is not None else None
    stream = current_stream(part.device)
    if addend is None:
        check(lib().ferry_combine(_dev(part, 'part', torch.bfloat16), pp, tokens, topk, hidden,
                                  _dev(out, 'out', torch.bfloat16), stream), 'combine')
    else:
        if addend.shape != (tokens, hidden):
            raise RuntimeError('addend must be bf16 [tokens, hidden]')
        check(lib().ferry_combine_add(_dev(part, 'part', torch.bfloat16), pp, tokens, topk, hidden,
                                      _dev(addend, 'addend', torch.bfloat16),
                                      _dev(out, 'out', torch.bfloat16), stream), 'combine_add')
    return out


class SharedExpert:
    """Always-on SwiGLU expert applied to every token (DeepSeek-V2 shared experts).

    Not in the reference runtime: HF's DeepseekV2MoE adds ``shared_experts(residuals)``
    (a DeepseekV2MLP of intermediate n_shared * moe_intermediate, bf16 nn.Linear layers) to
    the routed output (transformers 4.57 modeling_deepseek_v2; installed analogue
    modeling_deepseek_v2.py:126-151).  Here the MLP runs on the grouped SwiGLU kernels as one
    expert whose rows are all tokens with routing weight 1, from one weight row
    ``[gate I*H | up I*H | down H*I]`` (the cache row format) resident in HBM.  The SwiGLU
    rounding is the routed experts' (silu(g) * u in fp32, one bf16 rounding).
    """

    def __init__(self, row, hidden, intermediate):
        if row.dtype != torch.bfloat16 or row.numel() != 3 * hidden * intermediate:
            raise RuntimeError('shared expert row must be bf16 [3 * intermediate * hidden]')
        self.row = row.reshape(1, -1).contiguous()
        self.hidden, self.intermediate = hidden, intermediate
        self._bufs = {}

    def _buffers(self, T, device):
        b = self._bufs.get(T)
        if b is None:
            b = dict(starts=torch.tensor([0, T], dtype=torch.int64, device=device),
                     rows=torch.arange(T, dtype=torch.int64, device=device),
                     cols=torch.zeros(T, dtype=torch.int64, device=device),
                     w=torch.ones((T, 1), dtype=torch.bfloat16, device=device),
                     act=torch.empty((T, self.intermediate), dtype=torch.bfloat16, device=device))
            self._bufs[T] = b
        return b

    def __call__(self, x, out=None):
        """bf16 [T, H] -> bf16 [T, H] = down(silu(x Wg^T) * (x Wu^T))."""
        T = x.shape[0]
        if out is None:
            out = torch.empty((T, self.hidden), dtype=torch.bfloat16, device=x.device)
        if T == 0:
            return out
        b = self._buffers(T, x.device)
        return expert_ffn(self.row, x.contiguous(), b['w'], b['starts'], b['rows'], b['cols'], [0],
                          np.zeros(1, np.int32), self.hidden, self.intermediate, b['act'], out,
                          out_mode=1, experts=1, counts=[T])


def history_update(selected, experts, window, layer, ring, counts, meta, scores, ids_out=None,
                   timeouts_out=None, ready_out=None, ready_value=0):
    """Device GateHistory update of ``layer`` (ferry/metadata.py:15-38, frequency rows).

    ``scores`` (fp32 [E]), ``ids_out`` (uint8 [T*k]) and ``timeouts_out`` (int32 [1]: the
    device's count of one-launch decode FFN waits that gave up, as ``ffn_sync_timeouts``) are
    CUDA tensors or raw device addresses (ints), e.g. of a mapped host buffer that the kernel
    writes directly.  ``ready_out`` (device address of ``history_ready_words(T, k)`` int32
    words, with ``ids_out``) receives ``ready_value`` in every word once the launch's other
    writes are visible to the host."""
    T, k = selected.shape
    sp = scores if isinstance(scores, int) else _dev(scores, 'scores', torch.float32)
    ip = (ids_out if isinstance(ids_out, int) or ids_out is None
          else _dev(ids_out, 'ids_out', torch.uint8))
    tp = (timeouts_out if isinstance(timeouts_out, int) or timeouts_out is None
          else _dev(timeouts_out, 'timeouts_out', torch.int32))
    rp = (ready_out if isinstance(ready_out, int) or ready_out is None
          else _dev(ready_out, 'ready_out', torch.int32))
    check(lib().ferry_history_update(
        _dev(selected, 'selected', torch.int64), T, k, experts, window, layer,
        _dev(ring, 'ring', torch.int32), _dev(counts, 'counts', torch.int32),
        _dev(meta, 'meta', torch.int32), sp, ip, tp, rp, int(ready_value),
        current_stream(selected.device)),
        'history_update')


def history_ready_words(tokens, topk):
    """Number of int32 ready words ``history_update`` writes for a call of ``tokens``."""
    return int(lib().ferry_history_ready_words(int(tokens), int(topk)))


# ------------------------------------------------------------------------------------------
# The reference's pybind names (ferry/csrc/expert_ops.cpp:144-157)
# ------------------------------------------------------------------------------------------

def execute_experts(cache, input, routing_weights, slots, rows, cols, hidden, intermediate):
    """Routed-expert MLPs of every (slot, rows, cols) group (expert_ops.cpp:16-45).

    Output i is ``down(silu(x Wg^T) * (x Wu^T)) * routing_weights[rows[i], cols[i]]`` for
    ``x = input[rows[i]]``, one bf16 [len(rows[i]), hidden] tensor per group.
    """
    _dev(cache, 'cache', torch.bfloat16)
    if cache.dim() != 2 or cache.shape[1] != 3 * hidden * intermediate:
        raise RuntimeError('cache must be [cap, 3 * hidden * intermediate]')
    if input.dim() != 2 or input.shape[1] != hidden:
        raise RuntimeError('input must be [rows, hidden]')
    if routing_weights.dim() != 2 or routing_weights.shape[0] != input.shape[0]:
        raise RuntimeError('routing_weights must be [rows, topk]')
    if not (len(slots) == len(rows) == len(cols)):
        raise RuntimeError('slots, rows and cols must have the same length')
    G = len(slots)
    if G == 0:
        return []
    if G > MAX_EXPERTS:
        raise RuntimeError(f'at most {MAX_EXPERTS} groups per call')
    for s in slots:
        if not 0 <= int(s) < cache.shape[0]:
            raise RuntimeError('slot out of range')
    sizes = [int(r.numel()) for r in rows]
    dev = input.device
    starts = torch.tensor(np.concatenate([[0], np.cumsum(sizes)]), dtype=torch.int64, device=dev)
    rows_cat = torch.cat([r.reshape(-1) for r in rows]).to(torch.int64).contiguous()
    cols_cat = torch.cat([c.reshape(-1) for c in cols]).to(torch.int64).contiguous()
    P = int(sum(sizes))
    act = torch.empty((max(P, 1), intermediate), dtype=torch.bfloat16, device=dev)
    out = torch.empty((max(P, 1), hidden), dtype=torch.bfloat16, device=dev)
    expert_ffn(cache, input.contiguous(), routing_weights.contiguous(), starts, rows_cat, cols_cat,
               np.arange(G), np.asarray(slots, np.int32), hidden, intermediate, act, out,
               out_mode=1, experts=G, counts=sizes)
    return list(out[:P].split(sizes))


def pack_dispatch(hidden, selected, weights, send_idx, send_ids, experts):
    """Dispatch packet rows ``[x (2H B) | weights in send_ids order (2k B) | IDs (k B)]``.

    Reference: expert_ops.cpp:88-104, on the ``ferry_pack_dispatch`` kernel.  At world = 1 the
    packet never leaves the GPU (the fused path reads the routing weights in send_ids order
    straight from the layout kernel); this gives callers of the reference's Transport the same
    bytes.
    """
    n, k = send_ids.shape
    T, H = hidden.shape
    payload = torch.empty((n, 2 * H + 3 * k), dtype=torch.uint8, device=hidden.device)
    check(lib().ferry_pack_dispatch(
        _dev(hidden, 'hidden', torch.bfloat16), T, H, _dev(selected, 'selected', torch.int64),
        _dev(weights, 'weights', torch.bfloat16), selected.shape[1],
        _dev(send_idx, 'send_idx', torch.int64), _dev(send_ids, 'send_ids', torch.int64), n, k,
        experts, payload.data_ptr(), current_stream(hidden.device)), 'pack_dispatch')
    return payload


def unpack_dispatch(raw, hidden, topk):
    """Split packet rows back into bf16 [m, H] hidden states and [m, k] weights
    (expert_ops.cpp:106-111), as two strided device copies."""
    m = raw.shape[0]
    if raw.dim() != 2 or raw.shape[1] != 2 * hidden + 3 * topk:
        raise RuntimeError('raw must be uint8 [m, 2 * hidden + 3 * topk]')
    x = torch.empty((m, hidden), dtype=torch.bfloat16, device=raw.device)
    w = torch.empty((m, topk), dtype=torch.bfloat16, device=raw.device)
    check(lib().ferry_unpack_dispatch(_dev(raw, 'raw', torch.uint8), m, hidden, topk,
                                      x.data_ptr(), w.data_ptr(), current_stream(raw.device)),
          'unpack_dispatch')
    return [x, w]


def reduce_partials(parts, rows, received, hidden, like):
    """fp32 sum of expert outputs per received row, ascending group order, then bf16 (:76-83)."""
    if len(parts) == 0:
        return torch.zeros((received, hidden), dtype=torch.bfloat16, device=like.device)
    part = torch.cat([p.reshape(-1, hidden) for p in parts]).to(torch.bfloat16).contiguous()
    rows_cat = torch.cat([r.reshape(-1) for r in rows]).to(torch.int64)
    # the j-th occurrence (in group order) of each row is its j-th term
    order = torch.argsort(rows_cat, stable=True)
    counts = torch.bincount(rows_cat, minlength=received)
    k = max(int(counts.max().item()) if counts.numel() else 1, 1)
    first = torch.cumsum(counts, 0) - counts
    rank = torch.arange(order.numel(), device=like.device) - first[rows_cat[order]]
    pair_pos = torch.full((received * k,), -1, dtype=torch.int32, device=like.device)
    pair_pos[rows_cat[order] * k + rank] = order.to(torch.int32)
    return combine(part, received, k, hidden, pair_pos=pair_pos)


def scatter_returned(returned, send_idx, tokens):
    """Add returned rows back to their tokens in fp32 (expert_ops.cpp:86-92)."""
    output = torch.zeros((tokens, returned.shape[1]), dtype=torch.float32, device=returned.device)
    if returned.shape[0]:
        output.index_add_(0, send_idx, returned.float())
    return output.to(returned.dtype)
