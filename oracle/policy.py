"""Placement-planner oracle at world = 1 (test infrastructure).

``PlannerRef`` drives the C restatement of ferry/policy.py:130-194 (oracle_plan_layer in
ref_core.c).  ``plan_layer_sorted`` is an independent formulation used to pin it: per miss it
sorts all candidate slots by the reference's eviction key with Python's ``sorted`` instead of
scanning for a running minimum.
"""
import numpy as np

from .native import lib


class PlannerRef:
    def __init__(self, layers, experts, cap):
        self.layers, self.experts, self.cap = layers, experts, cap
        self.slots = np.full(cap, -1, np.int64)
        self.owner = np.full(layers * experts, -1, np.int64)
        self.last = np.zeros(layers * experts, np.int64)
        self.scores = np.zeros((layers, experts), np.float32)

    def plan(self, event, layer, selected, gate_scores):
        sel = np.ascontiguousarray(selected, np.int64)
        T, k = sel.shape
        gs = np.ascontiguousarray(gate_scores, np.float32)
        fetches = np.empty((self.experts, 3), np.int64)
        dest = np.empty((T, k), np.int64)
        m = lib().oracle_plan_layer(event, layer, sel.ctypes.data, T, k, gs.ctypes.data,
                                    self.slots.ctypes.data, self.cap, self.owner.ctypes.data,
                                    self.last.ctypes.data, self.scores.ctypes.data, self.experts,
                                    fetches.ctypes.data, dest.ctypes.data)
        if m < 0:
            raise AssertionError('missing experts exceed the admission capacity')
        return fetches[:m].copy(), dest

    def layer_slots(self, layer):
        out = np.empty(self.experts, np.int64)
        lib().oracle_layer_slots(self.slots.ctypes.data, self.cap, layer, self.experts, out.ctypes.data)
        return out


def plan_layer_sorted(state, event, layer, selected, gate_scores):
    """Independent formulation of one plan step on a dict state (slots/owner/last/scores)."""
    E = state['scores'].shape[1]
    state['scores'][layer] = gate_scores
    active = set(int(e) for e in np.asarray(selected).reshape(-1))
    base = layer * E
    misses = sorted(e for e in active if state['owner'][base + e] < 0)
    protected = lambda key: key // E == layer and (key % E) in active  # noqa: E731
    admissible = sum(1 for key in state['slots'] if key < 0 or not protected(key))
    if len(misses) > admissible:
        raise AssertionError('missing experts exceed the admission capacity')
    fetches = []
    for e in misses:
        slots = state['slots']
        empty = [i for i, key in enumerate(slots) if key < 0]
        if empty:
            slot = empty[0]
        else:
            cands = [(float(state['scores'].reshape(-1)[key]), int(state['last'][key]), int(key), i)
                     for i, key in enumerate(slots) if not protected(key)]
            slot = sorted(cands)[0][3]
        victim = slots[slot]
        if victim >= 0:
            state['owner'][victim] = -1
        slots[slot] = base + e
        state['owner'][base + e] = 0
        fetches.append((0, base + e, slot))
    for e in active:
        state['last'][base + e] = event + 1
    return np.array(fetches, np.int64).reshape(-1, 3)
