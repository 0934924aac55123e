"""Dispatch / combine at world = 1 (reference: ferry/transport.py).

``Transport`` keeps the reference's exchange protocol: dispatch packs the token packets
(``pack_dispatch``), exchanges them and unpacks them (``unpack_dispatch``); combine sums the
expert outputs of every received row (``reduce_partials``), sends them back and adds them to
their tokens (``scatter_returned``).  With one GPU each exchange is the identity, so no byte
crosses a device and the byte counters stay 0.  The fused runtime path skips the packets and
runs the layout kernel's token-major combine instead (``expert_ops.combine``).
"""


class Transport:
    def __init__(self, ops_module, topk, experts):
        self.ops, self.topk, self.experts = ops_module, topk, experts
        self.rank = 0
        self.dispatch_bytes = self.combine_bytes = 0

    def _exchange(self, x, send_counts, recv_counts):
        """The all-to-all of one rank: everything it sends is what it receives."""
        if list(send_counts) != list(recv_counts) or len(send_counts) != 1:
            raise NotImplementedError('ferry_amd runs on one GPU (world = 1)')
        return x

    def dispatch(self, hidden, selected, weights, layout):
        """Token packets to the experts: (received hidden rows, their packet weights)
        (transport.py:22-29)."""
        packets = self.ops.pack_dispatch(hidden, selected, weights, layout['send_idx'],
                                         layout['send_ids'], self.experts)
        received = self._exchange(packets, layout['send_counts'], layout['recv_counts'])
        return self.ops.unpack_dispatch(received, hidden.shape[1], self.topk)

    def combine(self, hidden, parts, layout):
        """Expert outputs back to their tokens, fp32 sums in expert order (transport.py:31-38)."""
        rows = [g[1] for g in layout['groups']]
        partial = self.ops.reduce_partials(parts, rows, sum(layout['recv_counts']),
                                           hidden.shape[1], hidden)
        returned = self._exchange(partial, layout['recv_counts'], layout['send_counts'])
        return self.ops.scatter_returned(returned, layout['send_idx'], hidden.shape[0])
