"""Packet-format oracle (test infrastructure): the reference's dispatch bytes on the CPU.

``pack_dispatch_ref`` restates ferry/csrc/expert_ops.cpp:88-104 in torch on the CPU: the bf16
routing weights are scattered into a dense fp32 [T, E] row (repeated IDs add), cast to bf16,
gathered at the packet IDs (clamped at 0) and multiplied by the validity mask; the packet row
is [hidden row bytes | packet weight bytes | IDs as uint8].  ``unpack_dispatch_ref`` restates
:106-111.  Pinned in the tests by the world-1 closed form: with distinct IDs a packet is
[hidden[t] | the routing weights in sorted-ID order (the layout's w_sorted) | sorted IDs].
"""
import numpy as np
import torch


def pack_dispatch_ref(hidden, selected, weights, send_idx, send_ids, experts):
    T, H = hidden.shape
    n, k = send_ids.shape
    dense = torch.zeros((T, experts), dtype=torch.float32)
    dense.scatter_add_(1, selected, weights.float())
    dense = dense.to(torch.bfloat16)
    valid = send_ids >= 0
    pw = dense[send_idx.unsqueeze(1), send_ids.clamp(min=0)] * valid
    rows = [hidden.index_select(0, send_idx).view(torch.uint8).reshape(n, 2 * H),
            pw.contiguous().view(torch.uint8).reshape(n, 2 * k),
            send_ids.to(torch.uint8).reshape(n, k)]
    return torch.cat(rows, dim=1)


def unpack_dispatch_ref(raw, hidden, topk):
    m = raw.shape[0]
    # flatten before reinterpreting: a one-row slice keeps the packet pitch as its stride
    x = raw[:, :2 * hidden].contiguous().reshape(-1).view(torch.bfloat16).reshape(m, hidden)
    w = (raw[:, 2 * hidden:2 * hidden + 2 * topk].contiguous().reshape(-1).view(torch.bfloat16)
         .reshape(m, topk))
    return x, w


def packets_closed_form(hidden, send_ids, w_sorted):
    """World-1 packets of distinct-ID routing: [hidden[t] | w_sorted[t] | send_ids[t]] bytes."""
    h = np.ascontiguousarray(hidden.view(torch.int16).numpy()).view(np.uint8)
    w = np.ascontiguousarray(np.asarray(w_sorted, np.int16)).view(np.uint8)
    ids = np.asarray(send_ids).astype(np.uint8)
    return np.concatenate([h, w, ids], axis=1)
