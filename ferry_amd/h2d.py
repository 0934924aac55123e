"""H2D expert fetch engine (the reference's ``H2DEngine``, ferry/csrc/expert_ops.cpp:94-142).

Copies rows of a pinned host pool into GPU cache slots: by default with ``hipMemcpyAsync`` on
the engine's two DMA streams (``DMA``, the reference's way), or with one launch of a copy
kernel per fetch call that reads the pool through its device mapping (``KERNEL``).  A copy into a slot waits, on the GPU, for the last compute that read that
slot (``mark_used``).  ``wait_host`` blocks the host like the reference;
``wait_stream`` makes a compute stream wait on the GPU instead, which lets resident experts
run while missing ones are still in flight.
"""
import ctypes

import numpy as np
import torch

from ._lib import check, lib


def _i64(values):
    return np.ascontiguousarray(np.asarray(values, dtype=np.int64).reshape(-1))


DMA, KERNEL = 0, 1   # FERRY_H2D_DMA, FERRY_H2D_KERNEL


class H2DEngine:
    def __init__(self, cache, pool):
        if not (isinstance(cache, torch.Tensor) and cache.device.type == 'cuda' and cache.is_contiguous()):
            raise RuntimeError('cache must be a contiguous CUDA tensor')
        if not (isinstance(pool, torch.Tensor) and pool.is_pinned() and pool.is_contiguous()):
            raise RuntimeError('pool must be a contiguous pinned host tensor')
        if pool.dim() != 2 or cache.dim() != 2 or pool.shape[1] != cache.shape[1] or pool.dtype != cache.dtype:
            raise RuntimeError('pool rows must match cache rows')
        self._cache, self._pool = cache, pool   # keep both alive, like the reference
        handle = ctypes.c_void_p()
        check(lib().ferry_h2d_create(cache.data_ptr(), cache.shape[0], pool.data_ptr(), pool.shape[0],
                                     cache.shape[1] * cache.element_size(), cache.device.index or 0,
                                     ctypes.byref(handle)), 'H2DEngine')
        self._h = handle.value

    @classmethod
    def from_packed(cls, cache, packed, ring_rows=64):
        """An engine that fetches every row from ``packed`` (a PackedPool) in DMA mode; no raw
        pool is needed."""
        if not (isinstance(cache, torch.Tensor) and cache.device.type == 'cuda' and cache.is_contiguous()):
            raise RuntimeError('cache must be a contiguous CUDA tensor')
        if cache.dim() != 2 or cache.shape[1] * cache.element_size() != packed.row_bytes:
            raise RuntimeError('packed rows must match cache rows')
        eng = cls.__new__(cls)
        eng._cache, eng._pool, eng._packed = cache, None, packed
        handle = ctypes.c_void_p()
        check(lib().ferry_h2d_create_packed(cache.data_ptr(), cache.shape[0], packed.handle,
                                            cache.device.index or 0, int(ring_rows),
                                            ctypes.byref(handle)), 'H2DEngine.from_packed')
        eng._h = handle.value
        return eng

    @property
    def handle(self):
        """The native engine (ferry_h2d*), for ferry_plan_fetch."""
        return self._h

    def fetch(self, slots, keys):
        s, k = _i64(slots), _i64(keys)
        if len(s) != len(k):
            raise RuntimeError('slots and keys must have the same length')
        check(lib().ferry_h2d_fetch(self._h, s.ctypes.data, k.ctypes.data, len(s)), 'H2DEngine.fetch')

    def wait_host(self, slots):
        s = _i64(slots)
        check(lib().ferry_h2d_wait_host(self._h, s.ctypes.data, len(s)), 'H2DEngine.wait_host')

    def wait_stream(self, slots, stream=None):
        s = _i64(slots)
        st = stream if stream is not None else torch.cuda.current_stream(self._cache.device)
        check(lib().ferry_h2d_wait_stream(self._h, s.ctypes.data, len(s), st.cuda_stream),
              'H2DEngine.wait_stream')

    def mark_used(self, slots, stream=None):
        s = _i64(slots)
        st = stream if stream is not None else torch.cuda.current_stream(self._cache.device)
        check(lib().ferry_h2d_mark_used(self._h, s.ctypes.data, len(s), st.cuda_stream),
              'H2DEngine.mark_used')

    def mark_used_record(self, slots, stream=None):
        """mark_used and a host-waitable event in one record on ``stream``: returns the
        event's handle (owned by the engine, valid until the next call of this method), for
        ``event_synchronize``."""
        s = _i64(slots)
        st = stream if stream is not None else torch.cuda.current_stream(self._cache.device)
        ev = ctypes.c_void_p()
        check(lib().ferry_h2d_mark_used_record(self._h, s.ctypes.data, len(s), st.cuda_stream,
                                               ctypes.byref(ev)), 'H2DEngine.mark_used_record')
        return ev.value

    def event_synchronize(self, event):
        """Block the host until an event of ``mark_used_record`` has fired."""
        check(lib().ferry_h2d_event_synchronize(self._h, event), 'H2DEngine.event_synchronize')

    def wait_ready(self, event, words_ptr, n, value):
        """Block the host until the ``n`` int32 words at host address ``words_ptr`` hold
        ``value`` (ready words a kernel queued before ``event``, the latest event of
        ``mark_used_record``, writes after its host-memory outputs); the reads that ``event``
        marks then count as complete."""
        check(lib().ferry_h2d_wait_ready(self._h, event, words_ptr, int(n), int(value)),
              'H2DEngine.wait_ready')

    def synchronize(self):
        check(lib().ferry_h2d_synchronize(self._h), 'H2DEngine.synchronize')

    def reset(self):
        """The state of a new engine (no copies or reads recorded, ``copies`` 0, DMA mode) on the
        same streams and buffers, after all of its work has finished."""
        check(lib().ferry_h2d_reset(self._h), 'H2DEngine.reset')
        self._defer_last = False

    @property
    def engine(self):
        """How rows are copied: ``KERNEL`` or ``DMA``."""
        return int(lib().ferry_h2d_engine(self._h))

    @engine.setter
    def engine(self, kind):
        check(lib().ferry_h2d_set_engine(self._h, int(kind)), 'H2DEngine.engine')

    @property
    def defer_last(self):
        """Whether the last sub-batch of a packed fetch is unpacked on the stream that waits
        for it (``wait_stream``) instead of the engine's unpack stream."""
        return bool(getattr(self, '_defer_last', False))

    @defer_last.setter
    def defer_last(self, on):
        check(lib().ferry_h2d_set_defer_last(self._h, int(bool(on))), 'H2DEngine.defer_last')
        self._defer_last = bool(on)

    def set_kernel_stream(self, stream=None):
        """Run kernel-mode copies on ``stream`` (a torch stream; None: the engine's own).  A
        handle of 0 is HIP's null stream (torch's default stream), not the engine's."""
        handle = stream.cuda_stream if stream is not None else lib().ferry_h2d_stream(self._h)
        check(lib().ferry_h2d_set_kernel_stream(self._h, handle), 'H2DEngine.set_kernel_stream')

    def use_packed(self, packed, ring_rows=64):
        """Fetch from ``packed`` (a PackedPool of this engine's pool; None: raw rows again) in
        DMA mode, through ``ring_rows`` device staging buffers."""
        check(lib().ferry_h2d_use_packed(self._h, packed.handle if packed is not None else None,
                                         int(ring_rows)), 'H2DEngine.use_packed')
        self._packed = packed   # keep it alive while the engine uses it

    @property
    def kernel_ok(self):
        """Whether the copy kernel can serve this pool (device-mapped, 16-byte rows)."""
        cur = self.engine
        try:
            self.engine = KERNEL
        except RuntimeError:
            return False
        self.engine = cur
        return True

    @property
    def copies(self):
        return int(lib().ferry_h2d_copies(self._h))

    def groups(self):
        """Ends (exclusive positions in the call's slot list) of the last fetch call's groups
        of rows that become ready together: a packed DMA call's sub-batches, otherwise one."""
        ends = np.zeros(64, np.int64)
        n = int(lib().ferry_h2d_groups(self._h, ends.ctypes.data, len(ends)))
        if n < 0:
            check(1, 'H2DEngine.groups')
        if n > len(ends):
            ends = np.zeros(n, np.int64)
            n = int(lib().ferry_h2d_groups(self._h, ends.ctypes.data, len(ends)))
        return ends[:n].tolist()

    @property
    def stream(self):
        """The engine's copy stream as a torch.cuda.ExternalStream."""
        return torch.cuda.ExternalStream(lib().ferry_h2d_stream(self._h), device=self._cache.device)

    def close(self):
        if getattr(self, '_h', None):
            lib().ferry_h2d_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class PackedPool:
    """A lossless packed copy of a pool for the host link (ferry_pack_pool), in pinned memory:
    per value a sign|mantissa byte and a 2-bit exponent code against the row's 3 most populated
    exponents, the escapes as 2-bit codes against the next 3, their escapes as 4-bit codes
    against a window of 15 or in an (index, exponent) list -- about 10.7 bits instead of 16 for
    weights that span few binades (rows that would not shrink are kept raw; rows hold a
    multiple of 32 values).  Engines fetch it in DMA mode (staging buffers) or in kernel mode
    (the unpack kernel reads it over the link).  The source pool may be
    pageable and may be freed afterwards; engines fetch from the packed pool alone
    (``H2DEngine.from_packed``) or attach it to an engine of the same pinned pool
    (``use_packed``)."""

    def __init__(self, pool, threads=16):
        if not (isinstance(pool, torch.Tensor) and pool.device.type == 'cpu'
                and pool.is_contiguous() and pool.dim() == 2 and pool.dtype == torch.bfloat16):
            raise RuntimeError('pool must be a contiguous bf16 [rows, row] host tensor')
        self.rows, self.row_bytes = pool.shape[0], pool.shape[1] * 2
        self.pool_id = pool.data_ptr()
        handle = ctypes.c_void_p()
        check(lib().ferry_pack_pool(pool.data_ptr(), pool.shape[0], pool.shape[1] * 2,
                                    int(threads), ctypes.byref(handle)), 'PackedPool')
        self._h = handle.value
        pb, pr = ctypes.c_int64(), ctypes.c_int64()
        check(lib().ferry_packed_pool_stats(self._h, ctypes.byref(pb), ctypes.byref(pr)),
              'PackedPool')
        self.packed_bytes, self.packed_rows = pb.value, pr.value
        raw = self.packed_rows * self.row_bytes
        self.ratio = raw / self.packed_bytes if self.packed_bytes else 1.0   # over packed rows

    @property
    def handle(self):
        return self._h

    def close(self):
        if getattr(self, '_h', None):
            lib().ferry_packed_pool_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
