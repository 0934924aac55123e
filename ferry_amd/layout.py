"""Expert-parallel layout of one MoE layer at world = 1, built on the GPU.

Reference: ferry/layout.py (build_layout + device_layout).  The reference builds the layout
with numba on the host and uploads every index array in one blocking copy; here the HIP
layout kernel (histogram, scan, stable permute) builds the same arrays in device memory.
"""
import numpy as np
import torch

from . import expert_ops as ops


def device_layout(selected, destinations, tokens_per_rank, rank, experts, slot_of, weights=None):
    """Same contract as ferry/layout.py:78-94 at world = 1.

    ``selected`` may be a host array (as in the reference) or a CUDA tensor.  Returns
    dict(send_idx, send_ids, send_counts, recv_counts, groups) with groups =
    [(e, rows_e, cols_e, slot)] for every expert with entries, ascending; plus the device
    ``layout`` object that the fused path consumes.
    """
    if rank != 0:
        raise NotImplementedError('ferry_amd runs on one GPU (world = 1)')
    if isinstance(selected, torch.Tensor):
        sel = selected.to('cuda', torch.int64).contiguous()
    else:
        sel = torch.from_numpy(np.ascontiguousarray(selected, dtype=np.int64)).to('cuda')
    T, k = sel.shape
    if T != tokens_per_rank:
        raise NotImplementedError('ferry_amd runs on one GPU (world = 1)')
    if destinations is not None and np.any(np.asarray(destinations) != 0):
        raise AssertionError('expert scheduled on this rank is not cached here')
    lay = ops.layout(sel, weights, experts, check=True)   # the reference's index checks
    starts = lay.starts.cpu().numpy()
    groups = []
    for e in np.flatnonzero(starts[1:] > starts[:-1]):
        slot = int(slot_of[e])
        assert slot >= 0, 'expert scheduled on this rank is not cached here'
        a, b = int(starts[e]), int(starts[e + 1])
        groups.append((int(e), lay.rows[a:b], lay.cols[a:b], slot))
    return dict(send_idx=torch.arange(T, device='cuda'), send_ids=lay.send_ids,
                send_counts=[T], recv_counts=[T], groups=groups, layout=lay)
