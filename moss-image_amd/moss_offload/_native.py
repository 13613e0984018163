"""ctypes binding of ``include/moss_offload.h``.

The library is loaded lazily and only after ``torch`` is imported, so it binds to the HIP
runtime torch already mapped (one runtime per process; torch's streams are valid handles for
the engine). There is no fallback: if the library is missing, every offload entry point raises.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must be imported before the library, see module docstring)

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libmoss_offload.so"

MO_ABI_VERSION = 21
MO_MAX_DIMS = 8

MO_E_INVALID = 1001
MO_E_LAYOUT = 1002
MO_E_HOST_OOM = 1003
MO_E_STATE = 1004

MO_FLAG_TIMING = 0x1
MO_FLAG_KERNEL_COPY = 0x2
MO_FLAG_KERNEL_TIMING = 0x4
MO_FLAG_NO_STAGED_RESTORE = 0x8
MO_FLAG_EAGER_PACK = 0x10
MO_FLAG_HIP_DMA = 0x20
MO_FLAG_PACK_NT_LOAD = 0x40
MO_FLAG_UNPACK_CACHED_LOAD = 0x80
MO_FLAG_UNPACK_CACHED_STORE = 0x100
MO_FLAG_WIRE_CODING = 0x200
MO_FLAG_WIRE_AUTO = 0x400
MO_TENSOR_BF16_HIGH = 0x1
MO_INT8_KERNEL_REGISTERS = 0
MO_INT8_KERNEL_LDS = 1

NO_GROUP = (1 << 64) - 1


class MoTensor(ctypes.Structure):
    _fields_ = [
        ("ptr", ctypes.c_uint64),
        ("elem_bytes", ctypes.c_uint32),
        ("ndim", ctypes.c_uint32),
        ("size", ctypes.c_int64 * MO_MAX_DIMS),
        ("stride", ctypes.c_int64 * MO_MAX_DIMS),
        ("flags", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
    ]


class MoConfig(ctypes.Structure):
    _fields_ = [
        ("stage_slot_bytes", ctypes.c_uint64),
        ("stage_slots", ctypes.c_uint32),
        ("restore_slots", ctypes.c_uint32),
        ("host_limit_bytes", ctypes.c_uint64),
        ("host_chunk_bytes", ctypes.c_uint64),
        ("flags", ctypes.c_uint32),
        ("copy_kernel_blocks", ctypes.c_uint32),
        ("d2h_engine", ctypes.c_uint32),
        ("h2d_engine", ctypes.c_uint32),
        ("wire_device_limit", ctypes.c_uint64),
        ("commit_batch_bytes", ctypes.c_uint64),
        ("stage_slots_max", ctypes.c_uint32),
        ("restore_slots_max", ctypes.c_uint32),
        ("restore_small_slots", ctypes.c_uint32),
    ]


class MoRef(ctypes.Structure):
    _fields_ = [("group", ctypes.c_uint64), ("entry", ctypes.c_uint32), ("reserved", ctypes.c_uint32)]


class MoStats(ctypes.Structure):
    _fields_ = [
        (name, ctypes.c_uint64)
        for name in (
            "groups_created",
            "groups_live",
            "entries_live",
            "bytes_packed",
            "bytes_unpacked",
            "bytes_d2h",
            "bytes_h2d",
            "pack_launches",
            "unpack_launches",
            "d2h_copies",
            "h2d_copies",
            "host_bytes_in_use",
            "host_bytes_peak",
            "host_bytes_reserved",
            "stage_slot_waits",
            "host_blocks",
        )
    ] + [("host_block_ms", ctypes.c_double)] + [
        (name, ctypes.c_uint64)
        for name in (
            "prefetch_issued",
            "prefetch_hits",
            "restore_fetches",
            "staged_hits",
            "bytes_staged",
        )
    ] + [
        ("d2h_ms", ctypes.c_double),
        ("h2d_ms", ctypes.c_double),
        ("timed_d2h_bytes", ctypes.c_uint64),
        ("timed_h2d_bytes", ctypes.c_uint64),
        ("copy_failures", ctypes.c_uint64),
        ("pack_ms", ctypes.c_double),
        ("unpack_ms", ctypes.c_double),
        ("timed_pack_bytes", ctypes.c_uint64),
        ("timed_unpack_bytes", ctypes.c_uint64),
        ("timed_pack_launches", ctypes.c_uint64),
        ("timed_unpack_launches", ctypes.c_uint64),
        ("timed_pack_hbm_bytes", ctypes.c_uint64),
        ("timed_unpack_hbm_bytes", ctypes.c_uint64),
        ("wire_segments", ctypes.c_uint64),
        ("wire_raw_bytes", ctypes.c_uint64),
        ("wire_bytes", ctypes.c_uint64),
        ("device_ring_bytes", ctypes.c_uint64),
        ("wire_fallbacks", ctypes.c_uint64),
        ("ahead_restored", ctypes.c_uint64),
        ("ahead_not_resident", ctypes.c_uint64),
        ("ahead_in_flight", ctypes.c_uint64),
        ("restore_slots_big", ctypes.c_uint64),
        ("restore_slots_small", ctypes.c_uint64),
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


class MoStreamerStats(ctypes.Structure):
    _fields_ = [
        ("fills", ctypes.c_uint64),
        ("bytes", ctypes.c_uint64),
        ("timed_bytes", ctypes.c_uint64),
        ("busy_ms", ctypes.c_double),
        ("host_blocks", ctypes.c_uint64),
        ("host_block_ms", ctypes.c_double),
        ("copy_failures", ctypes.c_uint64),
        ("writebacks", ctypes.c_uint64),
        ("writeback_bytes", ctypes.c_uint64),
        ("timed_writeback_bytes", ctypes.c_uint64),
        ("writeback_busy_ms", ctypes.c_double),
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


class MoGradaccStats(ctypes.Structure):
    _fields_ = [
        ("calls", ctypes.c_uint64),
        ("chunks", ctypes.c_uint64),
        ("bytes", ctypes.c_uint64),
        ("elements", ctypes.c_uint64),
        ("d2h_done_bytes", ctypes.c_uint64),
        ("d2h_ms", ctypes.c_double),
        ("accumulate_ms", ctypes.c_double),
        ("host_blocks", ctypes.c_uint64),
        ("host_block_ms", ctypes.c_double),
        ("pending_chunks", ctypes.c_uint64),
        ("copy_failures", ctypes.c_uint64),
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


class EngineError(RuntimeError):
    """A non-zero status from the engine library, with its message."""

    def __init__(self, call: str, status: int, message: str) -> None:
        super().__init__(f"{call} failed with status {status}: {message}")
        self.status = status


_P = ctypes.POINTER
_u64 = ctypes.c_uint64

# name -> (restype, argtypes); mirrors include/moss_offload.h
SIGNATURES: dict[str, tuple] = {
    "mo_abi_version": (ctypes.c_int, []),
    "mo_last_error": (ctypes.c_char_p, []),
    "mo_payload_layout": (ctypes.c_int, [_P(MoTensor), ctypes.c_int, _P(_u64), _P(_u64)]),
    "mo_gather": (ctypes.c_int, [_P(MoTensor), ctypes.c_int, _u64, _P(_u64), _u64]),
    "mo_scatter": (ctypes.c_int, [_P(MoTensor), ctypes.c_int, _u64, _P(_u64), _u64]),
    "mo_link_copy": (ctypes.c_int, [_u64, _u64, _u64, ctypes.c_int, ctypes.c_uint32, _u64]),
    "mo_pack_to_host": (ctypes.c_int, [_P(MoTensor), ctypes.c_int, _u64, _u64, _P(_u64), _u64]),
    "mo_create": (ctypes.c_int, [ctypes.c_int, _P(MoConfig), _P(ctypes.c_void_p)]),
    "mo_destroy": (ctypes.c_int, [ctypes.c_void_p]),
    "mo_pack": (ctypes.c_int, [ctypes.c_void_p, _P(MoTensor), ctypes.c_int, _u64, _P(MoRef)]),
    "mo_pack_progress": (ctypes.c_int, [ctypes.c_void_p, _P(_u64), _P(_u64)]),
    "mo_pack_flush": (ctypes.c_int, [ctypes.c_void_p]),
    "mo_equal": (ctypes.c_int, [ctypes.c_void_p, _u64, _u64, _u64, _u64, _P(_u64)]),
    "mo_equal_result": (ctypes.c_int, [ctypes.c_void_p, _u64, ctypes.c_int, _P(ctypes.c_int)]),
    "mo_equal_discard": (ctypes.c_int, [ctypes.c_void_p, _u64]),
    "mo_commit": (ctypes.c_int, [ctypes.c_void_p, _u64, _P(_u64)]),
    "mo_prefetch": (ctypes.c_int, [ctypes.c_void_p, _u64, _u64]),
    "mo_prefetch_entry": (ctypes.c_int, [ctypes.c_void_p, _u64, ctypes.c_uint32, _u64]),
    "mo_prefetch_groups": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(_u64), ctypes.c_uint32, _u64]),
    "mo_unpack": (ctypes.c_int, [ctypes.c_void_p, _u64, _P(_u64), ctypes.c_uint32, _u64]),
    "mo_unpack_groups": (
        ctypes.c_int,
        [ctypes.c_void_p, _P(_u64), _P(_u64), _P(ctypes.c_uint32), ctypes.c_uint32, _u64, _P(ctypes.c_uint32)],
    ),
    "mo_release": (ctypes.c_int, [ctypes.c_void_p, _u64]),
    "mo_group_info": (
        ctypes.c_int,
        [ctypes.c_void_p, _u64, _P(ctypes.c_uint32), _P(_u64), _P(ctypes.c_int)],
    ),
    "mo_synchronize": (ctypes.c_int, [ctypes.c_void_p]),
    "mo_get_stats": (ctypes.c_int, [ctypes.c_void_p, _P(MoStats)]),
    "mo_reset_stats": (ctypes.c_int, [ctypes.c_void_p]),
    "mo_trim": (ctypes.c_int, [ctypes.c_void_p]),
    "mo_link_name": (ctypes.c_char_p, [ctypes.c_void_p]),
    "mo_pinned_alloc": (ctypes.c_int, [_u64, _P(_u64)]),
    "mo_pinned_free": (ctypes.c_int, [_u64]),
    "mo_streamer_create": (ctypes.c_int, [ctypes.c_int, ctypes.c_uint32, ctypes.c_uint32, _P(ctypes.c_void_p)]),
    "mo_streamer_destroy": (ctypes.c_int, [ctypes.c_void_p]),
    "mo_streamer_fill": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, _u64, _u64, _u64]),
    "mo_streamer_writeback": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, _u64, _u64, _u64]),
    "mo_streamer_acquire": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, _u64]),
    "mo_streamer_release": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, _u64]),
    "mo_streamer_attach": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, _u64, _u64]),
    "mo_streamer_stage": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int64, _u64, _u64, ctypes.c_int64,
                                         _P(ctypes.c_uint32), _P(_u64), _P(ctypes.c_int)]),
    "mo_streamer_pin": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, _u64]),
    "mo_streamer_unpin": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, _u64, _u64]),
    "mo_streamer_mark_dirty": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, _u64, ctypes.c_int]),
    "mo_streamer_evict": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32]),
    "mo_streamer_slot_info": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, _P(ctypes.c_int64),
                                             _P(ctypes.c_uint32), _P(ctypes.c_int), _P(_u64)]),
    "mo_streamer_synchronize": (ctypes.c_int, [ctypes.c_void_p]),
    "mo_streamer_get_stats": (ctypes.c_int, [ctypes.c_void_p, _P(MoStreamerStats)]),
    "mo_streamer_reset_stats": (ctypes.c_int, [ctypes.c_void_p]),
    "mo_gradacc_create": (ctypes.c_int, [ctypes.c_int, ctypes.c_uint32, _u64, ctypes.c_uint32, ctypes.c_uint32,
                                         _P(ctypes.c_void_p)]),
    "mo_gradacc_destroy": (ctypes.c_int, [ctypes.c_void_p]),
    "mo_gradacc_accumulate": (ctypes.c_int, [ctypes.c_void_p, _u64, ctypes.c_uint32, _u64, ctypes.c_uint32, _u64,
                                             _u64]),
    "mo_gradacc_wait": (ctypes.c_int, [ctypes.c_void_p, _u64]),
    "mo_gradacc_get_stats": (ctypes.c_int, [ctypes.c_void_p, _P(MoGradaccStats)]),
    "mo_gradacc_reset_stats": (ctypes.c_int, [ctypes.c_void_p]),
    "mo_int8_decode": (ctypes.c_int, [_u64, _u64, _u64, ctypes.c_uint32, ctypes.c_uint32, _u64]),
    "mo_wire_capacity": (_u64, [_u64]),
    "mo_wire_encode": (ctypes.c_int, [_u64, _u64, _u64, _u64, _u64, _u64]),
    "mo_wire_decode": (ctypes.c_int, [_u64, _u64, _u64, _u64, _u64]),
    "mo_int8_linear_forward": (ctypes.c_int, [_u64, _u64, _u64, _u64, _u64, ctypes.c_uint32, ctypes.c_uint32,
                                              ctypes.c_uint32, _u64, _u64, _u64]),
    "mo_int8_forward_workspace_bytes": (_u64, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]),
    "mo_int8_linear_backward": (ctypes.c_int, [_u64, _u64, _u64, _u64, ctypes.c_uint32, ctypes.c_uint32,
                                               ctypes.c_uint32, _u64, _u64, _u64]),
    "mo_int8_backward_workspace_bytes": (_u64, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]),
    "mo_int8_set_kernel": (ctypes.c_int, [ctypes.c_uint32]),
    "mo_int8_launch_plan": (ctypes.c_int, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                           ctypes.c_uint32, _P(ctypes.c_uint32), _P(ctypes.c_uint32)]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Load (once) and return the engine library; raise if it is not built."""

    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        lib_path = Path(path) if path is not None else LIB_PATH
        if not lib_path.exists():
            raise RuntimeError(
                f"moss_offload native library not found at {lib_path}; build it with "
                "`python -m moss_offload.build` (hipcc, gfx950). There is no fallback path."
            )
        lib = ctypes.CDLL(str(lib_path))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.mo_abi_version()
        if version != MO_ABI_VERSION:
            raise RuntimeError(f"moss_offload ABI {version} != expected {MO_ABI_VERSION}; rebuild the library")
        _lib = lib
        return lib


def check(call: str, status: int) -> None:
    """Raise :class:`EngineError` for a non-zero status."""

    if status != 0:
        message = _lib.mo_last_error().decode(errors="replace") if _lib is not None else ""
        raise EngineError(call, status, message)


def describe(tensor: torch.Tensor, out: MoTensor, ptr: int | None = None, flags: int = 0) -> MoTensor:
    """Fill ``out`` with the view ``tensor`` (address, element size, sizes, strides, flags)."""

    shape = tensor.shape
    stride = tensor.stride()
    ndim = len(shape)
    if ndim > MO_MAX_DIMS:
        raise ValueError(f"tensor has {ndim} dims; the engine supports at most {MO_MAX_DIMS}")
    out.ptr = tensor.data_ptr() if ptr is None else ptr
    out.elem_bytes = tensor.element_size()
    out.ndim = ndim
    out.flags = flags
    out.reserved = 0
    for i in range(ndim):
        out.size[i] = shape[i]
        out.stride[i] = stride[i]
    return out
