"""MI355X activation-offload engine for MOSS-Image DiT training.

``activation_cpu_offload`` is a drop-in for ``training.activation_offload.activation_cpu_offload``
of RyukoMatoiFan/MOSS-Image. The work behind it is done by ``libmoss_offload.so`` (HIP kernels
for gfx950 plus the engine), loaded through :mod:`moss_offload._native`.
"""

from .activation_offload import (
    _offload_view,
    _OffloadedTensor,
    _restore_layout,
    _storage_key,
    activation_cpu_offload,
    hook_counters,
    hook_features,
    reset_hook_counters,
)
from .engine import EngineConfig, OffloadEngine, configure, get_engine, reset_engines

__all__ = [
    "activation_cpu_offload",
    "_offload_view",
    "_restore_layout",
    "_storage_key",
    "_OffloadedTensor",
    "hook_counters",
    "hook_features",
    "reset_hook_counters",
    "EngineConfig",
    "OffloadEngine",
    "configure",
    "get_engine",
    "reset_engines",
]
