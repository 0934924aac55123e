"""Page-locked host memory for the expert pool and the per-call staging buffer.

Allocated with hipHostMalloc through the HIP runtime that PyTorch-ROCm already loads, and
wrapped as CPU tensors that free the memory when they are released.
"""
import ctypes
import weakref

import numpy as np
import torch

_HOST_MAPPED = 0x2          # hipHostMallocMapped
_HOST_COHERENT = 0x40000000  # hipHostMallocCoherent (fine-grained: device writes go straight to host)

_hip = None


def _runtime():
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL('libamdhip64.so')
        _hip.hipHostMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t, ctypes.c_uint]
        _hip.hipHostFree.argtypes = [ctypes.c_void_p]
        _hip.hipHostGetDevicePointer.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p,
                                                 ctypes.c_uint]
    return _hip


def _host_alloc(nbytes, flags):
    hip = _runtime()
    ptr = ctypes.c_void_p()
    rc = hip.hipHostMalloc(ctypes.byref(ptr), max(nbytes, 1), flags)
    if rc != 0:
        raise RuntimeError(f'hipHostMalloc of {nbytes} bytes failed (error {rc})')
    buf = np.ctypeslib.as_array(ctypes.cast(ptr, ctypes.POINTER(ctypes.c_uint8)), shape=(max(nbytes, 1),))
    weakref.finalize(buf, hip.hipHostFree, ptr.value)
    return buf, ptr.value


def pinned_empty(shape, dtype=torch.bfloat16):
    """Uninitialised pinned host tensor.

    torch's pinned allocator rounds every request up to a power of two, so a 58 GB expert pool
    would ask for 64 GB of page-locked memory; this allocates exactly the pool's bytes."""
    n = int(np.prod(shape)) * torch.empty((), dtype=dtype).element_size()
    buf, _ = _host_alloc(n, 0)
    return torch.from_numpy(buf)[:n].view(dtype).view(shape)


def mapped_buffer(nbytes):
    """(uint8 host tensor, device address) of a coherent host buffer that kernels write
    directly: the host reads the results after an event, with no separate D2H copy."""
    buf, hptr = _host_alloc(nbytes, _HOST_MAPPED | _HOST_COHERENT)
    dptr = ctypes.c_void_p()
    rc = _runtime().hipHostGetDevicePointer(ctypes.byref(dptr), ctypes.c_void_p(hptr), 0)
    if rc != 0:
        raise RuntimeError(f'hipHostGetDevicePointer failed (error {rc})')
    return torch.from_numpy(buf)[:nbytes], dptr.value
