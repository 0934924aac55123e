"""Step-2 quota table at world = 1 (reference: ferry/quota.py).

With one GPU every missing expert is fetched by that GPU: the quota table row of m misses is
[m], and the one rule of greedy_quota that survives is its capacity check (quota.py:63), which
the planner applies.  ``Topology`` reads the topology file that ``ferry_amd.h2dprof`` writes
(the format of ferry/quota.py:80-90: ``world``, ``domains`` with ``mask`` and ``gib_per_s``,
``quota_lut``, optional ``physical_gpus``) or builds the uniform one-GPU table.  Files for more
than one GPU are rejected: the multi-GPU topology quota is not part of this one-GPU build.
"""
import json
from pathlib import Path

import numpy as np


def _one_gpu(world):
    if world != 1:
        raise NotImplementedError('ferry_amd runs on one GPU (world = 1)')


class Topology:
    """Bandwidth domains (bit masks over GPUs, seconds per GiB) and the quota lookup table."""

    def __init__(self, path, world, experts):
        doc = json.loads(Path(path).read_text())
        if doc['world'] != world:
            raise ValueError(f"topology file is for {doc['world']} GPUs, runtime has {world}")
        _one_gpu(world)
        domains = doc['domains']
        self.masks = np.array([int(d['mask']) for d in domains], dtype=np.int64)
        self.seconds = np.reciprocal(np.array([float(d['gib_per_s']) for d in domains]))
        table = np.asarray(doc['quota_lut'], dtype=np.int64)
        if table.ndim != 2 or table.shape[1] != world or table.shape[0] <= experts:
            raise ValueError('quota lookup table does not cover this model; rebuild it')
        # every row m must hand out exactly m fetches
        assert np.array_equal(table.sum(axis=1), np.arange(table.shape[0])), 'bad quota table'
        self.lut = table
        self.gpus = doc.get('physical_gpus')

    @classmethod
    def uniform(cls, world, experts):
        """One GPU, one domain of unit cost: quota_lut[m] = [m]."""
        _one_gpu(world)
        topo = cls.__new__(cls)
        topo.masks = np.ones(1, dtype=np.int64)
        topo.seconds = np.ones(1, dtype=np.float64)
        topo.lut = np.arange(experts + 1, dtype=np.int64)[:, None]
        topo.gpus = None
        return topo
