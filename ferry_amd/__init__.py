"""ferry_amd: the MI355X-native per-GPU MoE hot path of FERRY (one GPU, HIP kernels for gfx950).

Modules mirror the reference package: runtime (OffloadRuntime), metadata (GateHistory),
policy (Controller, _choose_slot), layout (device_layout), h2d (H2DEngine), transport,
model (ModelSpec, hooks) and expert_ops (the native ops).  The kernels live in
libferry_amd.so (C ABI: include/ferry_amd.h).
"""
__version__ = '0.1.0'
