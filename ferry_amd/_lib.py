"""ctypes binding of libferry_amd.so, the C ABI declared in include/ferry_amd.h.

The library is built in-tree (``make -C ferry_amd/csrc``, or ``__graft_entry__.build()``).
Loading fails loudly when it is missing: there is no fallback implementation.
"""
import ctypes
import os
from pathlib import Path

_HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get('FERRY_AMD_LIB', _HERE / 'libferry_amd.so'))

_c_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float

# (name, restype, argtypes) for every entry point of include/ferry_amd.h
SIGNATURES = [
    ('ferry_last_error', ctypes.c_char_p, []),
    ('ferry_abi_version', _i32, []),
    ('ferry_router_topk', ctypes.c_int,
     [_c_p, _i32, _i64, _i64, _i64, _i32, _f32, _i32, _c_p, _c_p, _c_p, _c_p, _c_p]),
    ('ferry_layout_workspace_bytes', _i64, [_i64, _i64, _i64]),
    ('ferry_layout', ctypes.c_int,
     [_c_p, _c_p, _i64, _i64, _i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _i64, _c_p]),
    ('ferry_layout_noalloc', ctypes.c_int,
     [_c_p, _c_p, _i64, _i64, _i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p]),
    ('ferry_expert_ffn', ctypes.c_int,
     [_c_p, _i64, _i64, _i64, _c_p, _i64, _i64, _c_p, _c_p, _c_p, _c_p, _c_p, _i32, _c_p, _i64,
      _i64, _i64, _c_p, _c_p, _c_p, _i32, _i32, _c_p]),
    ('ferry_expert_ffn_sync_timeouts', ctypes.c_int, [_c_p]),
    ('ferry_expert_ffn_set_sync_spin_limit', ctypes.c_int, [_i64]),
    ('ferry_combine', ctypes.c_int, [_c_p, _c_p, _i64, _i64, _i64, _c_p, _c_p]),
    ('ferry_pack_dispatch', ctypes.c_int,
     [_c_p, _i64, _i64, _c_p, _c_p, _i64, _c_p, _c_p, _i64, _i64, _i64, _c_p, _c_p]),
    ('ferry_unpack_dispatch', ctypes.c_int, [_c_p, _i64, _i64, _i64, _c_p, _c_p, _c_p]),
    ('ferry_combine_add', ctypes.c_int, [_c_p, _c_p, _i64, _i64, _i64, _c_p, _c_p, _c_p]),
    ('ferry_history_update', ctypes.c_int,
     [_c_p, _i64, _i64, _i64, _i64, _i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _i32, _c_p]),
    ('ferry_history_ready_words', _i64, [_i64, _i64]),
    ('ferry_plan_layer', _i64,
     [_i64, _i64, _c_p, _i64, _i64, _c_p, _c_p, _i64, _c_p, _c_p, _c_p, _i64, _c_p, _c_p]),
    ('ferry_plan_fetch', _i64,
     [_i64, _i64, _c_p, _i64, _i64, _c_p, _c_p, _i64, _c_p, _c_p, _c_p, _i64, _c_p, _c_p, _c_p,
      _c_p]),
    ('ferry_choose_slot', _i64, [_i64, _c_p, _c_p, _i64, _c_p, _c_p, _i64]),
    ('ferry_layer_slots', None, [_c_p, _i64, _i64, _i64, _c_p]),
    ('ferry_h2d_create', ctypes.c_int, [_c_p, _i64, _c_p, _i64, _i64, _i32, ctypes.POINTER(_c_p)]),
    ('ferry_h2d_destroy', ctypes.c_int, [_c_p]),
    ('ferry_h2d_fetch', ctypes.c_int, [_c_p, _c_p, _c_p, _i64]),
    ('ferry_h2d_wait_host', ctypes.c_int, [_c_p, _c_p, _i64]),
    ('ferry_h2d_wait_stream', ctypes.c_int, [_c_p, _c_p, _i64, _c_p]),
    ('ferry_h2d_mark_used', ctypes.c_int, [_c_p, _c_p, _i64, _c_p]),
    ('ferry_h2d_mark_used_record', ctypes.c_int, [_c_p, _c_p, _i64, _c_p, ctypes.POINTER(_c_p)]),
    ('ferry_h2d_event_synchronize', ctypes.c_int, [_c_p, _c_p]),
    ('ferry_h2d_wait_ready', ctypes.c_int, [_c_p, _c_p, _c_p, _i64, _i32]),
    ('ferry_h2d_synchronize', ctypes.c_int, [_c_p]),
    ('ferry_h2d_reset', ctypes.c_int, [_c_p]),
    ('ferry_h2d_copies', _i64, [_c_p]),
    ('ferry_h2d_groups', _i64, [_c_p, _c_p, _i64]),
    ('ferry_h2d_stream', _c_p, [_c_p]),
    ('ferry_h2d_set_engine', ctypes.c_int, [_c_p, _i32]),
    ('ferry_h2d_set_defer_last', ctypes.c_int, [_c_p, _i32]),
    ('ferry_h2d_engine', _i32, [_c_p]),
    ('ferry_h2d_set_kernel_stream', ctypes.c_int, [_c_p, _c_p]),
    ('ferry_pack_pool', ctypes.c_int, [_c_p, _i64, _i64, _i32, ctypes.POINTER(_c_p)]),
    ('ferry_packed_pool_stats', ctypes.c_int, [_c_p, _c_p, _c_p]),
    ('ferry_packed_pool_destroy', ctypes.c_int, [_c_p]),
    ('ferry_h2d_use_packed', ctypes.c_int, [_c_p, _c_p, _i64]),
    ('ferry_h2d_create_packed', ctypes.c_int, [_c_p, _i64, _c_p, _i32, _i64, ctypes.POINTER(_c_p)]),
    ('ferry_pack_row', ctypes.c_int, [_c_p, _i64, _c_p, _i64, _c_p]),
    ('ferry_timing_enable', ctypes.c_int, [_i32]),
    ('ferry_timing_mark', _i64, []),
    ('ferry_timing_range', ctypes.c_int, [_i64, _i64, _c_p]),
    ('ferry_timing_overlap', ctypes.c_int, [_i64, _i64, _c_p, _c_p, _c_p]),
    ('ferry_hbm_read_sink_bytes', ctypes.c_int64, [_i64]),
    ('ferry_hbm_read', ctypes.c_int, [_c_p, _i64, _c_p, _i64, _c_p]),
    ('ferry_timing_summary', ctypes.c_int,
     [ctypes.c_char_p, ctypes.POINTER(_i64), ctypes.POINTER(ctypes.c_double)]),
]

_lib = None


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f'{LIB_PATH} is missing: build it with `make -C {_HERE / "csrc"}` '
                               'or __graft_entry__.build() (there is no non-HIP fallback)')
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, restype, argtypes in SIGNATURES:
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def last_error():
    msg = lib().ferry_last_error()
    return msg.decode() if msg else ''


def check(status, what):
    """Raise RuntimeError with the library's message for a non-zero status."""
    if status != 0:
        raise RuntimeError(f'{what}: {last_error() or "status " + str(status)}')
    return status
