"""Layout oracle at world = 1 (test infrastructure).

``layout_closed_form`` is the world-1 closed form of ferry/layout.py:12-94 with numpy (sort,
bincount, cumsum, stable argsort).  ``layout_loops`` restates build_layout's loops literally
(insertion sort per packet, counting-sort cursor) for small inputs; the two pin each other.
"""
import numpy as np


def layout_closed_form(selected, experts, weights=None):
    sel = np.asarray(selected, np.int64)
    T, k = sel.shape
    order = np.argsort(sel, axis=1, kind='stable')
    send_ids = np.take_along_axis(sel, order, axis=1)
    counts = np.bincount(send_ids.reshape(-1), minlength=experts)
    starts = np.zeros(experts + 1, np.int64)
    np.cumsum(counts, out=starts[1:])
    flat = np.argsort(send_ids.reshape(-1), kind='stable')
    rows, cols = np.divmod(flat, k)
    out = dict(send_idx=np.arange(T), send_ids=send_ids, counts=counts, starts=starts,
               rows=rows.astype(np.int64), cols=cols.astype(np.int64))
    if weights is not None:
        out['w_sorted'] = np.take_along_axis(np.asarray(weights), order, axis=1)
    pair_pos = np.empty(T * k, np.int64)
    pair_pos[flat] = np.arange(T * k)
    out['pair_pos'] = pair_pos
    return out


def layout_loops(selected, experts):
    """ferry/layout.py:12-75 at world = 1, rank 0, as plain loops."""
    sel = [list(map(int, r)) for r in np.asarray(selected)]
    T, k = len(sel), (len(sel[0]) if sel else 0)
    recv_ids = []
    counts = [0] * experts
    for t in range(T):
        scratch = []
        for e in sel[t]:
            pos = len(scratch)
            scratch.append(e)
            while pos > 0 and scratch[pos - 1] > e:
                scratch[pos] = scratch[pos - 1]
                pos -= 1
            scratch[pos] = e
        recv_ids.append(scratch)
        for e in scratch:
            counts[e] += 1
    starts = [0] * (experts + 1)
    for e in range(experts):
        starts[e + 1] = starts[e] + counts[e]
    rows = [0] * starts[-1]
    cols = [0] * starts[-1]
    cursor = starts[:-1]
    for row in range(T):
        for col in range(k):
            e = recv_ids[row][col]
            rows[cursor[e]] = row
            cols[cursor[e]] = col
            cursor[e] += 1
    return dict(send_ids=np.array(recv_ids, np.int64).reshape(T, k), starts=np.array(starts),
                rows=np.array(rows, np.int64), cols=np.array(cols, np.int64))
