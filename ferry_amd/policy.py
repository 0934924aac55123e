"""Expert placement controller at world = 1 (reference: ferry/policy.py).

The planner itself is C++ in libferry_amd.so (ferry_plan_layer / ferry_choose_slot /
ferry_layer_slots); this module keeps the reference's Python names and signatures.
At world = 1 both policies send every missing expert to rank 0 (FERRY: quota_lut[m] = [m];
RANDOM: randint(0, 1) = 0), so the plan is: misses in ascending expert order, each placed by
the routing-aware eviction of _choose_slot, then ``last[active] = event + 1``.
"""
import numpy as np

from ._lib import last_error, lib

FERRY, RANDOM = 0, 1
INVALID_ROUTING = -3   # planner status: an expert ID out of range or repeated within a token
POLICIES = {'ferry': FERRY, 'random': RANDOM}


def _c(a, dtype):
    if not (isinstance(a, np.ndarray) and a.dtype == dtype and a.flags.c_contiguous):
        raise TypeError(f'expected a C-contiguous {np.dtype(dtype)} array')
    return a.ctypes.data


def _choose_slot(rank, layer, active, slots, capacities, last, scores, experts):
    """Step 4: an empty slot, else the lowest eviction score, then least-recently used
    (ferry/policy.py:109-127)."""
    if rank != 0 or len(capacities) != 1:
        raise NotImplementedError('ferry_amd runs on one GPU (world = 1)')
    act = np.ascontiguousarray(active, dtype=np.uint8)
    row = np.ascontiguousarray(slots[rank], dtype=np.int64)
    return int(lib().ferry_choose_slot(layer, act.ctypes.data, row.ctypes.data, int(capacities[rank]),
                                       _c(last, np.int64), _c(scores, np.float32), experts))


def plan_layer(event, layer, selected, origins, gate_scores, policy, slots, capacities, owner,
               last, scores, quota_lut, masks, seconds, balance_tol_bps, salt):
    """Plan one MoE layer call and update the cache state in place (ferry/policy.py:130-194).

    Returns fetches[m, 3] = (rank, key, slot), destinations [T, k] and per-rank fetch counts.
    """
    if len(capacities) != 1:
        raise NotImplementedError('ferry_amd runs on one GPU (world = 1)')
    sel = np.ascontiguousarray(selected, dtype=np.int64)
    tokens, topk = sel.shape
    experts = scores.shape[1]
    gs = np.ascontiguousarray(gate_scores, dtype=np.float32)
    if slots.dtype != np.int64 or not slots.flags.c_contiguous:
        raise TypeError('slots must be a C-contiguous int64 array')
    fetches = np.empty((experts, 3), np.int64)
    destinations = np.empty((tokens, topk), np.int64)
    m = lib().ferry_plan_layer(event, layer, sel.ctypes.data, tokens, topk, gs.ctypes.data,
                               slots.ctypes.data, int(capacities[0]), _c(owner, np.int64),
                               _c(last, np.int64), _c(scores, np.float32), experts,
                               fetches.ctypes.data, destinations.ctypes.data)
    if m == INVALID_ROUTING:
        raise RuntimeError(last_error())
    if m < 0:
        # the reference fails an assert here (quota.py:63 / policy.py:177)
        raise AssertionError(last_error())
    counts = np.array([m], np.int64)
    return fetches[:m].copy(), destinations, counts


def layer_slots(slots_row, capacity, layer, experts):
    """Slot index of every expert of ``layer`` cached on this rank, or -1 (policy.py:197-205)."""
    row = np.ascontiguousarray(slots_row, dtype=np.int64)
    lookup = np.empty(experts, np.int64)
    lib().ferry_layer_slots(row.ctypes.data, int(capacity), layer, experts, lookup.ctypes.data)
    return lookup


class Controller:
    """Placement state of the pooled expert cache and the per-layer planner call
    (reference: policy.py:208-228).  State arrays, in the reference's shapes: ``slots``
    [world, cap] (pool key per slot, -1 empty), ``owner`` / ``last`` [layers * experts]
    (rank holding the key or -1; last-use tick), ``scores`` float32 [layers, experts]."""

    def __init__(self, spec, capacities, policy, topology, balance_tol_bps=200, salt=1):
        caps = np.asarray(capacities, dtype=np.int64)
        if caps.size != 1:
            raise NotImplementedError('ferry_amd runs on one GPU (world = 1)')
        self.spec, self.capacities = spec, caps
        self.policy = POLICIES[policy]
        self.balance_tol_bps, self.salt = int(balance_tol_bps), int(salt)
        self.masks, self.seconds, self.lut = topology.masks, topology.seconds, topology.lut
        self.reset()

    def reset(self):
        """Empty cache, nothing used, zero scores."""
        keys = self.spec.layers * self.spec.experts
        self.slots = np.full((1, int(self.capacities[0])), -1, dtype=np.int64)
        self.owner = np.full(keys, -1, dtype=np.int64)
        self.last = np.zeros(keys, dtype=np.int64)
        self.scores = np.zeros((self.spec.layers, self.spec.experts), dtype=np.float32)
        # raw addresses of the state arrays for the fused native call (they never reallocate)
        self._slots_ptr, self._owner_ptr = self.slots.ctypes.data, self.owner.ctypes.data
        self._last_ptr, self._scores_ptr = self.last.ctypes.data, self.scores.ctypes.data
        self._fetch_buf = None

    def plan(self, event, layer, selected, origins, gate_scores):
        """plan_layer on this state: (fetches [m, 3], destinations, per-rank fetch counts)."""
        return plan_layer(event, layer, selected, origins, gate_scores, self.policy, self.slots,
                          self.capacities, self.owner, self.last, self.scores, self.lut,
                          self.masks, self.seconds, self.balance_tol_bps, self.salt)

    def plan_fetch(self, event, layer, ids_ptr, tokens, topk, scores_ptr, h2d_handle):
        """plan() from raw host pointers (uint8 routing IDs [tokens*topk], float32 scores [E],
        e.g. the mapped staging buffer) with the misses' copies queued on the fetch engine in
        the same native call.  Returns fetches[m, 3] (a view of a buffer reused by the next
        call) and the per-rank fetch counts; ``self.demand`` then holds each expert's
        (token, expert) pair count of the call (int64 [E], reused by the next call)."""
        experts = self.spec.experts
        if self._fetch_buf is None:
            self._fetch_buf = np.empty((experts, 3), np.int64)
            self.demand = np.zeros(experts, np.int64)
            self._fetch_ptrs = (self._fetch_buf.ctypes.data, self.demand.ctypes.data,
                                int(self.capacities[0]))
        fetch_ptr, demand_ptr, cap = self._fetch_ptrs
        m = lib().ferry_plan_fetch(event, layer, ids_ptr, tokens, topk, scores_ptr,
                                   self._slots_ptr, cap, self._owner_ptr, self._last_ptr,
                                   self._scores_ptr, experts, fetch_ptr, None, demand_ptr,
                                   h2d_handle)
        if m == -1:
            raise AssertionError(last_error())
        if m == INVALID_ROUTING:
            raise RuntimeError(last_error())
        if m < 0:
            raise RuntimeError(f'plan_fetch: {last_error()}')
        return self._fetch_buf[:m], np.array([m], np.int64)
