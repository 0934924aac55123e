"""GateHistory oracle (test infrastructure).

Restates ferry/metadata.py:15-38 (the ring of W float64 rows per layer) and the frequency
rows of RouteGather.collect at world = 1 (ferry/metadata.py:67-83), plus the closed form the
device counters implement.
"""
import numpy as np


class GateHistoryRef:
    """ferry/metadata.py:15-38."""

    def __init__(self, layers, experts, window=128):
        self.window = window
        self.rows = np.zeros((layers, window, experts), np.float64)
        self.count = np.zeros(layers, np.int64)
        self.head = np.zeros(layers, np.int64)

    def update(self, layer, probs):
        w = self.window
        if len(probs) >= w:
            self.rows[layer] = probs[-w:]
            self.count[layer] = w
            self.head[layer] = 0
            return
        for row in probs:
            self.rows[layer, self.head[layer]] = row
            self.head[layer] = (self.head[layer] + 1) % w
            self.count[layer] = min(w, self.count[layer] + 1)

    def scores(self, layer):
        n = max(1, int(self.count[layer]))
        return (self.rows[layer].sum(0) / n).astype(np.float32)


def frequency_rows(expert_ids, experts, window, world=1):
    """One-hot rows of the last min(T, ceil(W / world)) tokens (metadata.py:57, :80-82)."""
    ids = np.asarray(expert_ids, np.int64)
    tail = min(len(ids), -(-window // world))
    recent = ids[len(ids) - tail:]
    rows = np.zeros((len(recent), experts), np.float64)
    if len(recent):
        np.put_along_axis(rows, recent, 1.0, axis=1)
    return rows


def closed_form_scores(token_history, experts, window):
    """score[e] = float32(c_e / n): c_e counts e among the last n = min(W, seen) tokens."""
    recent = token_history[-window:] if len(token_history) else []
    n = max(1, len(recent))
    c = np.zeros(experts, np.int64)
    for ids in recent:
        for e in set(int(x) for x in ids):
            c[e] += 1
    return (c.astype(np.float64) / n).astype(np.float32)
