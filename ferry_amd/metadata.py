"""Routing metadata at world = 1: the selection-frequency history and the route gather.

Reference: ferry/metadata.py.  ``GateHistory`` keeps the reference's host API (numpy rows of
the W most recent routed tokens; ``scores`` = float32 of the window mean) and is what the
probability score uses.  ``DeviceGateHistory`` is the hot-path form of the default
frequency score: integer window counters on the GPU (one ring of token IDs and one count
vector per layer), updated by the ``ferry_history_update`` kernel; its scores are bit-equal
to ``GateHistory`` fed with one-hot rows.
"""
import numpy as np
import torch

from . import expert_ops as ops


class GateHistory:
    """Window of the W most recent history rows of every layer; scores = their mean
    (reference: metadata.py:15-38).  State, as the reference keeps it: ``rows`` float64
    [layers, W, E] (a ring), ``count`` / ``head`` int64 [layers], ``window``."""

    def __init__(self, layers, experts, window=128):
        self.window = window
        self.rows = np.zeros((layers, window, experts), dtype=np.float64)
        self.count = np.zeros(layers, dtype=np.int64)
        self.head = np.zeros(layers, dtype=np.int64)

    def update(self, layer, probs):
        """Append a batch of rows; a batch of W rows or more replaces the window by its last W."""
        batch = np.asarray(probs, dtype=np.float64)
        W, n = self.window, len(batch)
        if n >= W:
            self.rows[layer] = batch[n - W:]
            self.count[layer], self.head[layer] = W, 0
            return
        ring = (self.head[layer] + np.arange(n)) % W     # n < W: distinct positions
        self.rows[layer, ring] = batch
        self.head[layer] = (self.head[layer] + n) % W
        self.count[layer] = min(W, self.count[layer] + n)

    def scores(self, layer):
        """float32 of the float64 window mean of ``layer``."""
        return (self.rows[layer].sum(axis=0) / max(1, int(self.count[layer]))).astype(np.float32)


class DeviceGateHistory:
    """Frequency history on the GPU: ring of W x k IDs + int32[E] counts per layer."""

    def __init__(self, layers, experts, topk, window=128, device='cuda'):
        self.layers, self.experts, self.topk, self.window = layers, experts, topk, window
        self.ring = torch.full((layers, window, topk), -1, dtype=torch.int32, device=device)
        self.counts = torch.zeros((layers, experts), dtype=torch.int32, device=device)
        self.meta = torch.zeros((layers, 2), dtype=torch.int32, device=device)

    def update(self, layer, selected, scores_out, ids_out=None, timeouts_out=None,
               ready_out=None, ready_value=0):
        """Append the last min(T, W) tokens of ``selected`` and write the layer's scores (and,
        where given, the uint8 IDs, the device's decode-FFN timeout count and the ready words)."""
        ops.history_update(selected, self.experts, self.window, layer, self.ring, self.counts,
                           self.meta, scores_out, ids_out, timeouts_out, ready_out, ready_value)


def frequency_rows(expert_ids, experts, window, world=1):
    """One-hot history rows of the last ceil(W / world) tokens (metadata.py:55-83, world = 1)."""
    ids = np.asarray(expert_ids, np.int64)
    tail = min(len(ids), -(-window // world))
    recent = ids[len(ids) - tail:]
    rows = np.zeros((len(recent), experts), np.float64)
    if len(recent):
        np.put_along_axis(rows, recent, 1.0, axis=1)
    return rows


class RouteGather:
    """World-1 route gather: the D2H copy of the expert IDs (metadata.py:41-83).

    The all-gather is the identity at world = 1; ``collect`` returns (expert_ids int64 [T, k],
    origins int64 [T] (all 0), history rows).  The fused runtime path uses the device history
    and copies the IDs together with the scores instead.
    """

    def __init__(self, topk, experts, window, score='frequency'):
        if score not in ('frequency', 'probability'):
            raise ValueError(score)
        self.topk, self.experts, self.window, self.score = topk, experts, window, score
        self.world, self.rank = 1, 0

    def collect(self, selected, probs_tail):
        ids = selected.to(torch.uint8).cpu().numpy().astype(np.int64).reshape(-1, self.topk)
        origins = np.zeros(len(ids), np.int64)
        if self.score == 'probability':
            tail = min(len(ids), self.window)
            rows = probs_tail[-tail:].float().cpu().numpy().astype(np.float32)
        else:
            rows = frequency_rows(ids, self.experts, self.window)
        return ids, origins, rows
