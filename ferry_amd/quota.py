"""Step-2 quota table at world = 1 (reference: ferry/quota.py).

With one GPU the topology-aware quota is trivial: every missing expert is fetched by rank 0,
``lut[m] = [m]``, and the only surviving rule is the capacity check of greedy_quota
(quota.py:63): more misses than admissible slots is an error.  Multi-GPU topologies are out of
scope for this one-GPU build and are rejected.
"""
import json
from pathlib import Path

import numpy as np


class Topology:
    """Profiled bandwidth domains plus the quota lookup table (world = 1 only)."""

    def __init__(self, path, world, experts):
        data = json.loads(Path(path).read_text())
        if data['world'] != world:
            raise ValueError(f"topology file is for {data['world']} GPUs, runtime has {world}")
        if world != 1:
            raise NotImplementedError('ferry_amd runs on one GPU (world = 1)')
        self.masks = np.asarray([d['mask'] for d in data['domains']], np.int64)
        self.seconds = np.asarray([1.0 / d['gib_per_s'] for d in data['domains']], np.float64)
        self.lut = np.asarray(data['quota_lut'], np.int64)
        if self.lut.shape[0] < experts + 1 or self.lut.shape[1] != world:
            raise ValueError('quota lookup table does not cover this model; rebuild it')
        assert all(int(self.lut[m].sum()) == m for m in range(len(self.lut)))
        self.gpus = data.get('physical_gpus')

    @classmethod
    def uniform(cls, world, experts):
        if world != 1:
            raise NotImplementedError('ferry_amd runs on one GPU (world = 1)')
        self = cls.__new__(cls)
        self.masks = np.asarray([1], np.int64)
        self.seconds = np.ones(1, np.float64)
        self.lut = np.arange(experts + 1, dtype=np.int64).reshape(-1, 1)
        self.gpus = None
        return self
