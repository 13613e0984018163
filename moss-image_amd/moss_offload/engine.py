"""Host-side policy around the native engine: groups, handle lifetimes, restore and prefetch.

The native engine (``libmoss_offload.so``) owns the device staging ring, pinned host pool,
copy streams, events and kernels. This layer decides *when* to call it:

- one **group** per block of saves (the context commits at every block boundary),
- one **handle** per saved tensor; a group is released when its last handle dies, which is
  when the autograd graph drops the saved variable (backward, ``retain_graph`` or not, or a
  graph that is never backpropagated),
- **restore**: the first unpack of a group restores every live entry of that group in one
  unpack launch and keeps them until asked for (one H2D + one scatter per segment instead of
  one per tensor),
- **prefetch**: after a group is restored, the next ``prefetch_depth`` groups backward will
  need (each the youngest older live group: saves are consumed last-in first-out) are fetched
  on the host link while the current block computes, nearest first, a farther group only when
  all of it fits in the free restore slots.
"""

from __future__ import annotations

import atexit
import bisect
import ctypes
import threading
from collections import deque
from dataclasses import dataclass, fields

import torch

from . import _native


LINKS = ("sdma", "hipdma")
_MAX_SLOTS = 64  # staging plus restore slots, the library's limit
WIRE_CODINGS = {"off": 0, "on": _native.MO_FLAG_WIRE_CODING, "auto": _native.MO_FLAG_WIRE_AUTO}


@dataclass
class EngineConfig:
    """Sizes and switches of one device engine (see ``mo_config`` in moss_offload.h)."""

    stage_slot_bytes: int = 128 << 20
    stage_slots: int = 4
    # sixteen restore slots: a non-checkpointed block's coded saves span about five slots at
    # 128 MiB, and with four the H2D of a block's later segments waited for its earlier
    # segments' unpacks to run on the GPU (regime B 0.708 -> 0.645 s/it at six). With a
    # checkpointed block's one small segment per group, the slots bound how far ahead of the
    # GPU the backward's H2D can run: the trainer's thread runs several blocks ahead of the GPU,
    # and a slot is free only once the GPU has scattered its previous group. At eight, about a
    # third of the groups a restore could take along (restore_ahead_bytes) were still in
    # flight when asked for; at sixteen (prefetch_depth 16) none were, the unpack launches of a
    # 1024^2 checkpointed step grew from 48 to 132 MB (4.85 -> 5.78 TB/s) and the trainer's
    # thread blocked for an H2D 12 instead of 93 times per leg. Config 4 not checkpointed (24
    # blocks at 2048^2) went from 2.89 to 2.60 s/it. Wire-coded segments take at most the first
    # max(8, segments of their block + 2) slots (the engine's own rule): config 3 not
    # checkpointed runs 0.650 s/it with it against 0.665 on all sixteen and 0.654 with eight
    # slots in all. The cost is 1 GiB more device memory at 128 MiB slots (a checkpoint-only
    # trainer can take 32 MiB slots instead).
    restore_slots: int = 16
    # Ring growth for large blocks: at the commit of a group of n segments the engine grows the
    # restore ring to n + 2 slots and the staging ring to ceil(n / 3), up to these caps (0:
    # fixed rings). A 2048^2 block not checkpointed spans about 23 coded segments: with the
    # fixed 4 + 16 slots its restore fetched its last segments one at a time, each behind an
    # earlier one's scatter, and the D2H queue ran dry while attention held the next gather
    # (config 4 not checkpointed 2.60 s/it; grown to 8 + 32, 2.33). A 1024^2 block (about 11
    # segments) grows nothing. The grown slots cost device memory only where blocks are that
    # large (128 MiB each, plus a wire buffer each while coding).
    stage_slots_max: int = 8
    restore_slots_max: int = 32
    # Small restore slots (a quarter of stage_slot_bytes) for checkpointed blocks: once eight
    # groups in a row were committed with only raw segments that fit one (a checkpointed
    # 1024^2 block's inputs, 28 MB), the restore ring gains up to this many, and those segments
    # take them before a full-size slot. Nonzero also gives every restore slot past the first
    # two its device memory at first use, and trim() frees them once no group is live. A
    # checkpointed step then holds its prefetched blocks in 32 MiB slots instead of sixteen of
    # 128 MiB. 0: the restore slots are allocated up front and there are no small ones.
    restore_small_slots: int = 24
    host_limit_bytes: int = 0
    host_chunk_bytes: int = 1 << 30
    timing: bool = False
    kernel_timing: bool = False
    kernel_copy: bool = False
    # Host-link transport: "sdma" drives the SDMA engines through the HSA runtime (an issuer
    # thread orders copies; an unpack waits on the host for its H2D), "hipdma" enqueues the same
    # DMA copies on dedicated HIP streams ordered by hipStreamWaitEvent only (an unpack never
    # blocks the host). kernel_copy=True overrides both with the copy-kernel comparison.
    link: str = "sdma"
    # Cache policy of the kernels (measured choices are the defaults): non-temporal loads of the
    # saved tensors in pack, of the payload in unpack, and streaming stores of restored tensors.
    # Pack's non-temporal loads (MO_FLAG_PACK_NT_LOAD; the bare C ABI reads with ordinary loads
    # unless it is set): with gathers batched per segment and per commit, in-step pack went
    # 5.63 -> 5.91 TB/s in config 3 checkpointed, 5.12 -> 5.53 not checkpointed, 5.67 -> 5.93 in
    # config 5 unpacked, and 5.75 -> 5.87 on the block microbench, step times unchanged. (With
    # one gather per save they had slowed in-step pack: the forward still read the saves.)
    pack_nt_load: bool = True
    unpack_nt_load: bool = True
    unpack_nt_store: bool = True
    # Lossless wire coding of staging segments on the SDMA link (MO_FLAG_WIRE_*): "off", "on"
    # (every segment of at least 256 KiB), "auto" (only segments that close while at least two
    # staging slots of D2H bytes are queued, i.e. while the link sets the pace). Coded segments
    # cross the link in fewer bytes (bfloat16 activations: about 0.66) for HBM-bound coding
    # kernels and one wire buffer per staging and restore slot, allocated on first use.
    wire_coding: str = "auto"
    # Cap on the device bytes of the wire buffers (0: none). Where the buffers would pass it, or
    # their allocation fails, segments cross raw (stats "wire_fallbacks") and the engine tries
    # again at the next forward; the step never fails for want of them.
    wire_device_limit: int = 0
    copy_kernel_blocks: int = 16
    d2h_engine: int = 0
    h2d_engine: int = 0
    staged_restore: bool = True
    prefetch: bool = True
    # Groups prefetched ahead of backward: after a group is restored, up to `prefetch_depth`
    # groups backward will need next are queued for H2D into free restore slots, in that order
    # (mo_prefetch_groups: a farther group only when all of it fits). With small groups (a
    # checkpointed block's inputs) this lets the trainer's thread run that many blocks ahead of
    # the GPU without waiting for an H2D.
    prefetch_depth: int = 16
    # When autograd asks for a group, the groups backward needs next are scattered in the same
    # kernel launch if their bytes are on the device or on their way (H2D landed or handed to
    # the copy engine, or still staged),
    # up to this many payload bytes in all: a checkpointed block's inputs (about 30 MB at
    # 1024^2) are too small for one launch to reach the HBM copy rate, several together are
    # not (96 MiB: 93 MB launches at 5.43 TB/s; 192 MiB: 132 MB at 5.78 TB/s). Their restored
    # tensors wait in the cache until asked for. 0: one group per unpack.
    restore_ahead_bytes: int = 192 << 20
    dedupe: bool = True
    # Gather kernels of consecutive saves are launched together, one kernel per staging segment
    # when it closes (before its D2H), instead of one per save: fewer, larger launches that run
    # nearer the HBM copy rate. The engine keeps each save's source tensor alive until its
    # kernel is launched (at most one staging slot of saves). False: launch at every save.
    batch_packs: bool = True
    # A checkpointed block's saves (one group, about 30 MB at 1024^2) are gathered by one
    # launch too small to reach the HBM copy rate. A group's segment closed by its commit
    # waits instead, gathers and all, for the next groups' until this many bytes (or the
    # staging slot's end); then one launch gathers them all and their D2Hs follow in order.
    # Any restore, prefetch, release or synchronize sends the waiting segments first. Off
    # while wire coding is on (the link sets the pace there). 0: every commit sends its own.
    commit_batch_bytes: int = 128 << 20
    # A float32 save that is the untouched output of a bfloat16 -> float32 cast (every element's
    # low 16 bits are zero) crosses the link as its high halves: the same bits in half the bytes
    # (MO_TENSOR_BF16_HIGH). The hook decides from the autograd graph; False copies it whole.
    narrow_bf16_casts: bool = True
    # A save that is the output of torch.mul over saves already held (two tensors of one shape,
    # or a tensor and a Python number), or a dense view of one, is recomputed on unpack by the
    # same torch.mul instead of crossing the link. False offloads it like any other save.
    recompute_products: bool = True
    # A save that is a cast of the same autograd output as a cast already offloaded (RMSNorm's
    # two tokens.float(), say) is compared with it on the device (mo_equal); if the bytes are
    # equal it restores from the earlier save's payload, else it stays on the device as saved.
    # False offloads it like any other save.
    alias_equal_casts: bool = True
    # Saves made inside the last `keep_last_blocks` blocks of `model.layers` stay on the device
    # (0: offload every block, as the reference does). Backward needs them first, so offloading
    # them only sends them out and straight back; keeping them trades device memory for link
    # time in both directions. Restores stay bitwise: a kept save is the saved tensor itself.
    keep_last_blocks: int = 0
    # Each consumer of a deduplicated save (one payload saved by several autograd nodes) gets a
    # tensor of its own, as the reference's restore does: while another consumer is still to
    # take it, a take is a device copy, and the last consumer gets the restored tensor itself.
    # False hands all of them the one restored tensor, as autograd does without hooks.
    private_restores: bool = True

    def __post_init__(self) -> None:
        if self.link not in LINKS:
            raise ValueError(f"link must be one of {LINKS}, got {self.link!r}")
        if self.wire_coding not in WIRE_CODINGS:
            raise ValueError(f"wire_coding must be one of {tuple(WIRE_CODINGS)}, got {self.wire_coding!r}")
        for name in ("stage_slot_bytes", "stage_slots", "restore_slots", "stage_slots_max", "restore_slots_max",
                     "restore_small_slots",
                     "host_limit_bytes", "host_chunk_bytes",
                     "copy_kernel_blocks", "d2h_engine", "h2d_engine", "prefetch_depth", "keep_last_blocks",
                     "wire_device_limit", "restore_ahead_bytes", "commit_batch_bytes"):
            value = getattr(self, name)
            if isinstance(value, bool) or not isinstance(value, int) or value < 0:
                raise ValueError(f"{name} must be a non-negative integer, got {value!r}")

    def native(self) -> _native.MoConfig:
        cfg = _native.MoConfig()
        cfg.stage_slot_bytes = self.stage_slot_bytes
        cfg.stage_slots = self.stage_slots
        cfg.restore_slots = self.restore_slots
        cfg.host_limit_bytes = self.host_limit_bytes
        cfg.host_chunk_bytes = self.host_chunk_bytes
        cfg.flags = (
            (_native.MO_FLAG_TIMING if self.timing else 0)
            | (_native.MO_FLAG_KERNEL_COPY if self.kernel_copy else 0)
            | (_native.MO_FLAG_KERNEL_TIMING if self.kernel_timing else 0)
            | (0 if self.staged_restore else _native.MO_FLAG_NO_STAGED_RESTORE)
            | (0 if self.batch_packs else _native.MO_FLAG_EAGER_PACK)
            | (_native.MO_FLAG_HIP_DMA if self.link == "hipdma" else 0)
            | (_native.MO_FLAG_PACK_NT_LOAD if self.pack_nt_load else 0)
            | (0 if self.unpack_nt_load else _native.MO_FLAG_UNPACK_CACHED_LOAD)
            | (0 if self.unpack_nt_store else _native.MO_FLAG_UNPACK_CACHED_STORE)
            | WIRE_CODINGS[self.wire_coding]
        )
        cfg.copy_kernel_blocks = self.copy_kernel_blocks
        cfg.d2h_engine = self.d2h_engine
        cfg.h2d_engine = self.h2d_engine
        cfg.wire_device_limit = self.wire_device_limit
        cfg.commit_batch_bytes = self.commit_batch_bytes
        # a cap below the ring's own size means no growth (the library rejects a cap below it),
        # and the caps give way to the configured rings within the library's 64 slots
        stage_max = max(self.stage_slots_max, self.stage_slots) if self.stage_slots_max else self.stage_slots
        restore_max = max(self.restore_slots_max, self.restore_slots) if self.restore_slots_max else self.restore_slots
        restore_max = max(self.restore_slots, min(restore_max, _MAX_SLOTS - stage_max))
        stage_max = max(self.stage_slots, min(stage_max, _MAX_SLOTS - restore_max))
        cfg.stage_slots_max = stage_max
        cfg.restore_slots_max = restore_max
        cfg.restore_small_slots = max(0, min(self.restore_small_slots, _MAX_SLOTS - stage_max - restore_max))
        return cfg


def _span(t: torch.Tensor) -> int:
    """Elements from the lowest to the highest address of ``t`` (non-negative strides), or 0."""

    if t.numel() == 0:
        return 0
    return 1 + sum((size - 1) * stride for size, stride in zip(t.shape, t.stride()) if size > 1)


class _EntryState:
    __slots__ = ("refs", "readers", "dtype", "payload_shape", "stride", "nbytes", "restored", "restored_version")

    def __init__(self, dtype, payload_shape, stride, nbytes):
        self.refs = 0
        self.readers = 0  # references whose restore goes to an autograd consumer
        self.dtype = dtype
        self.payload_shape = payload_shape
        self.stride = stride
        self.nbytes = nbytes
        self.restored: torch.Tensor | None = None
        self.restored_version = 0


class _GroupState:
    __slots__ = ("gid", "entries", "live", "committed")

    def __init__(self, gid: int):
        self.gid = gid
        self.entries: list[_EntryState] = []
        self.live = 0
        self.committed = False


class OffloadEngine:
    """One native engine bound to one device."""

    def __init__(self, device: torch.device, config: EngineConfig | None = None) -> None:
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("the offload engine runs on a HIP device")
        self.index = self.device.index if self.device.index is not None else torch.cuda.current_device()
        self.config = config or EngineConfig()
        self._lib = _native.load()
        handle = ctypes.c_void_p()
        cfg = self.config.native()
        _native.check("mo_create", self._lib.mo_create(self.index, ctypes.byref(cfg), ctypes.byref(handle)))
        self._handle = handle
        self._lock = threading.RLock()
        self._groups: dict[int, _GroupState] = {}
        self._live: list[int] = []  # live group ids, ascending (creation order)
        self._desc = (_native.MoTensor * 1)()
        self._ref = (_native.MoRef * 1)()
        self._gid_out = ctypes.c_uint64()
        # sources of gathers not launched yet, as (pack call number, tensor, its version at the
        # save), oldest first
        self._held: deque[tuple[int, torch.Tensor, int]] = deque()
        self._calls = ctypes.c_uint64()
        self._launched = ctypes.c_uint64()
        self._committed_calls = 0  # pack calls made before the last commit (their groups are committed)
        # restores that asked for groups ahead, the groups offered, the groups restored ahead
        self._ahead_counts = {"restores": 0, "offered": 0, "restored": 0, "alone": 0}

    # ------------------------------------------------------------------ forward
    def pack(self, source: torch.Tensor, stream: int, narrow: bool = False) -> tuple[int, int]:
        """Gather ``source`` into the open group; return ``(group, entry)`` with one reference.

        ``narrow``: ``source`` is float32 with exact bfloat16 values; only its high halves are
        kept (MO_TENSOR_BF16_HIGH), and the restore writes them back with zero low halves."""

        with self._lock:
            _native.describe(source, self._desc[0], flags=_native.MO_TENSOR_BF16_HIGH if narrow else 0)
            _native.check("mo_pack", self._lib.mo_pack(self._handle, self._desc, 1, stream, self._ref))
            gid, idx = int(self._ref[0].group), int(self._ref[0].entry)
            group = self._groups.get(gid)
            if group is None:
                group = self._groups[gid] = _GroupState(gid)
                self._live.append(gid)
            if idx != len(group.entries):
                raise RuntimeError(f"engine entry index {idx} out of sync with group {gid}")
            entry = _EntryState(source.dtype, tuple(source.shape), tuple(source.stride()),
                                source.numel() * (2 if narrow else source.element_size()))
            entry.refs = entry.readers = 1
            group.entries.append(entry)
            group.live += 1
            if self.config.batch_packs:
                self._hold(source)  # after the bookkeeping: it may raise for an earlier save
            return gid, idx

    def commit(self, stream: int) -> int | None:
        """Close the open group (D2H starts); return its id or None."""

        with self._lock:
            _native.check("mo_commit", self._lib.mo_commit(self._handle, stream, ctypes.byref(self._gid_out)))
            gid = int(self._gid_out.value)
            group = self._groups.get(gid)
            if group is not None:
                group.committed = True
            if self._held:
                self._hold()
            self._committed_calls = self._calls.value if self._held else self._committed_calls
            return None if gid == _native.NO_GROUP else gid

    def acquire(self, gid: int, idx: int, reader: bool = True) -> bool:
        """Add a reference to a live entry (a deduplicated save, or with ``reader=False`` an
        input that a recomputed save reads). False if it is gone."""

        with self._lock:
            group = self._groups.get(gid)
            if group is None or idx >= len(group.entries) or group.entries[idx].refs <= 0:
                return False
            group.entries[idx].refs += 1
            group.entries[idx].readers += 1 if reader else 0
            group.live += 1
            return True

    def drop(self, gid: int, idx: int, reader: bool = True) -> None:
        """Remove one reference (as taken); release the group when none is left."""

        with self._lock:
            group = self._groups.get(gid)
            if group is None:
                return
            entry = group.entries[idx]
            entry.refs -= 1
            entry.readers -= 1 if reader else 0
            group.live -= 1
            if entry.refs <= 0:
                entry.restored = None
            if group.live <= 0:
                del self._groups[gid]
                pos = bisect.bisect_left(self._live, gid)
                if pos < len(self._live) and self._live[pos] == gid:
                    del self._live[pos]
                _native.check("mo_release", self._lib.mo_release(self._handle, gid))
                if self._held:
                    # Releasing the open group drops its pending gathers: their sources were
                    # never read, so a later in-place change to them is no error. Gathers of
                    # committed groups that waited (commit_batch_bytes) ran in the release, and
                    # are checked.
                    self._hold(check_upto=self._committed_calls)

    def _hold(self, source: torch.Tensor | None = None, check_upto: int | None = None) -> None:
        """Keep ``source`` (of the pack call just made) alive while its gather is pending, and
        let go of the sources whose gathers the engine has launched. Launched kernels are
        stream-ordered before anything that later reuses their memory.

        A pending gather reads its source when it is launched, not at the save. A source that
        was modified in place in between (its version counter moved: autograd's own test of a
        saved tensor, which it skips while saved-tensor hooks are installed) would be offloaded
        with its new bytes, where a copy at the save keeps the old ones. That raises here: the
        same program without offloading fails autograd's check in backward, and
        ``batch_packs=False`` copies at the save. ``check_upto``: check only the sources of pack
        calls numbered at most that (the others' gathers were dropped, not run)."""

        _native.check("mo_pack_progress", self._lib.mo_pack_progress(
            self._handle, ctypes.byref(self._calls), ctypes.byref(self._launched)))
        if source is not None and self._calls.value > self._launched.value:
            self._held.append((self._calls.value, source, source._version))
        launched = self._launched.value
        while self._held and self._held[0][0] <= launched:
            call, tensor, version = self._held.popleft()
            if (check_upto is None or call <= check_upto) and tensor._version != version:
                raise RuntimeError(
                    "a tensor saved for backward was modified in place before the offload engine "
                    "gathered it (autograd would reject this without offloading); "
                    "use moss_offload.configure(batch_packs=False) to copy every save at once")

    def flush(self) -> None:
        """Launch every pending gather kernel now."""

        with self._lock:
            _native.check("mo_pack_flush", self._lib.mo_pack_flush(self._handle))
            if self._held:
                self._hold()

    # ------------------------------------------------------------------ equality checks
    def equal(self, a: torch.Tensor, b: torch.Tensor, stream: int) -> int:
        """Start a device-side byte comparison of two dense tensors of one size on ``stream``;
        returns its ticket, or 0 when no check could be started. Both must stay unchanged
        until the result is known."""

        nbytes = a.numel() * a.element_size()
        if nbytes != b.numel() * b.element_size() or not (a.is_contiguous() and b.is_contiguous()):
            raise ValueError("equal() compares two contiguous tensors of the same byte size")
        ticket = _native._u64(0)
        with self._lock:
            _native.check("mo_equal", self._lib.mo_equal(
                self._handle, a.data_ptr(), b.data_ptr(), nbytes, stream, ctypes.byref(ticket)))
        return ticket.value

    def equal_result(self, ticket: int, wait: bool) -> int:
        """0 while the check runs (``wait`` False), 1 equal, 2 different; 1 and 2 free the ticket."""

        state = ctypes.c_int(0)
        with self._lock:
            _native.check("mo_equal_result", self._lib.mo_equal_result(
                self._handle, ticket, 1 if wait else 0, ctypes.byref(state)))
        return state.value

    def equal_discard(self, ticket: int) -> None:
        with self._lock:
            _native.check("mo_equal_discard", self._lib.mo_equal_discard(self._handle, ticket))

    # ------------------------------------------------------------------ backward
    def restore(self, gid: int, idx: int, stream: int, reader: bool = True) -> torch.Tensor:
        """Return entry ``idx`` of group ``gid`` as a device tensor of its packed layout: for an
        autograd consumer (``reader``) one of its own, for an internal read (``reader=False``,
        a recomputed save's input, read at once) possibly the one other readers get too."""

        with self._lock:
            group = self._groups.get(gid)
            if group is None:
                raise RuntimeError(f"offloaded group {gid} was already released")
            entry = group.entries[idx]
            cached = self._take_cached(entry, reader, stream)
            if cached is not None:
                return cached
            # Backward takes groups youngest first. An entry of a group asked for while a younger
            # group still waits is a save that later blocks share (one RoPE table or modulation
            # saved by every block, kept once by deduplication). If its group is larger than one
            # restore-ahead launch (a non-checkpointed block's saves), that entry is restored
            # alone, from the segments that hold it, and the rest of the group waits for its own
            # turn: restored whole now, it would hold device memory for the whole backward and
            # take the link from the groups backward needs first. A small group (a checkpointed
            # block's inputs) is restored whole as before.
            alone = (self._younger_waiting(gid) and
                     sum(e.nbytes for e in group.entries if e.refs > 0 and e.restored is None) >
                     max(self.config.restore_ahead_bytes, 1))
            groups = [group] if alone else [group] + self._ahead(gid)
            counts = (ctypes.c_uint32 * len(groups))(*(len(g.entries) for g in groups))
            dst = (ctypes.c_uint64 * sum(counts))()
            made, base = [], 0
            for k, g in enumerate(groups):
                mine = []
                for j, other in enumerate(g.entries):
                    if (k or j != idx) and (alone or other.refs <= 0 or other.restored is not None):
                        continue
                    tensor = torch.empty_strided(other.payload_shape, other.stride, dtype=other.dtype,
                                                 device=self.device)
                    mine.append((other, tensor))
                    if other.nbytes:
                        dst[base + j] = tensor.data_ptr()
                made.append(mine)
                base += len(g.entries)
            unpacked = (ctypes.c_uint32 * len(groups))()
            gids = (ctypes.c_uint64 * len(groups))(*(g.gid for g in groups))
            _native.check("mo_unpack_groups", self._lib.mo_unpack_groups(self._handle, gids, dst, counts, len(groups),
                                                                         stream, unpacked))
            self._ahead_counts["restores"] += 1
            self._ahead_counts["alone"] += alone
            self._ahead_counts["offered"] += len(groups) - 1
            self._ahead_counts["restored"] += sum(unpacked[k] for k in range(1, len(groups)))
            for k, mine in enumerate(made):
                if unpacked[k]:  # the first group always is
                    for other, tensor in mine:
                        other.restored = tensor
                        other.restored_version = tensor._version
            if self._held:  # unpacking the open group commits it
                self._hold()
            if self.config.prefetch and not alone:
                self._prefetch_after(gid, stream, max(1, self.config.prefetch_depth))
            return self._take_cached(entry, reader, stream)

    def _ahead(self, gid: int) -> list[_GroupState]:
        """Groups backward needs after ``gid``, nearest first, whose live entries not yet
        restored hold at most ``restore_ahead_bytes`` in all."""

        budget = self.config.restore_ahead_bytes
        out = []
        if budget <= 0:
            return out
        for nxt in self._predict_chain(gid, max(1, self.config.prefetch_depth)):
            g = self._groups[nxt]
            size = sum(e.nbytes for e in g.entries if e.refs > 0 and e.restored is None)
            if size > budget:
                break
            budget -= size
            out.append(g)
        return out

    def prefetch(self, gid: int, stream: int, ahead: bool = False) -> None:
        """Queue H2D of group ``gid``'s segments into free restore slots; with ``ahead``, also of
        the ``prefetch_depth - 1`` groups backward will need after it."""

        with self._lock:
            if gid in self._groups:
                more = self._predict_chain(gid, max(1, self.config.prefetch_depth) - 1) if ahead else []
                self._prefetch_groups([gid] + more, stream)

    def prefetch_entry(self, gid: int, idx: int, stream: int) -> None:
        """Queue H2D of the segments holding entry ``idx`` of group ``gid`` (a save later blocks
        share, restored alone while its group is not due yet)."""

        with self._lock:
            group = self._groups.get(gid)
            if group is not None and idx < len(group.entries) and group.entries[idx].restored is None:
                _native.check("mo_prefetch_entry", self._lib.mo_prefetch_entry(self._handle, gid, idx, stream))

    def _prefetch_after(self, gid: int, stream: int, count: int) -> None:
        self._prefetch_groups(self._predict_chain(gid, count), stream)

    def _predict_chain(self, gid: int, count: int) -> list[int]:
        """Up to ``count`` groups backward will need after ``gid``, nearest first."""

        order, nxt = [], gid
        for _ in range(count):
            nxt = self._predict_next(nxt)
            if nxt is None:
                break
            order.append(nxt)
        return order

    def _prefetch_groups(self, order: list[int], stream: int) -> None:
        if order:
            ids = (ctypes.c_uint64 * len(order))(*order)
            _native.check("mo_prefetch_groups", self._lib.mo_prefetch_groups(self._handle, ids, len(order), stream))

    def _take_cached(self, entry: _EntryState, reader: bool, stream: int | None = None) -> torch.Tensor | None:
        """The cached restore of ``entry``, handed out once per reference.

        The last reference takes the tensor itself. An autograd consumer while another is still
        to come gets a device copy (``private_restores``), so that no consumer can see another's
        in-place write, as with the reference's restore, which copies for each unpack. Internal
        reads share the cached tensor; a take finds it changed (its version moved) only if a
        consumer wrote it in place, and then the entry is restored again from its host copy.

        With ``stream``, a copy of a layout without gaps (its bytes are the entry's payload in
        storage order) runs as the engine's scatter kernel on that stream (a 28 MiB one-piece
        scatter takes 9-11 us) instead of the runtime's device copy that ``copy_`` makes (23 us
        on average for the 479 such copies of a 1024^2 step not checkpointed). Step times
        measured the same either way."""

        tensor = entry.restored
        if tensor is None:
            return None
        if tensor._version != entry.restored_version:
            entry.restored = None
            return None
        if entry.refs <= 1:
            entry.restored = None
            return tensor
        if reader and entry.readers > 1 and self.config.private_restores:
            copy = torch.empty_strided(entry.payload_shape, entry.stride, dtype=entry.dtype, device=self.device)
            if (stream is not None and copy.is_cuda and copy.numel() == _span(copy)
                    and torch.cuda.current_device() == self.device.index):  # the kernel runs on the current device
                _native.describe(copy, self._desc[0])
                _native.check("mo_scatter", self._lib.mo_scatter(self._desc, 1, tensor.data_ptr(), None, stream))
                return copy
            return copy.copy_(tensor)
        return tensor

    @staticmethod
    def _waiting(group: _GroupState | None) -> bool:
        """A committed group with an entry still to restore."""

        return group is not None and group.committed and any(
            e.refs > 0 and e.restored is None and e.nbytes for e in group.entries)

    def _predict_next(self, gid: int) -> int | None:
        """The group backward needs next: the youngest live group older than ``gid``."""

        pos = bisect.bisect_left(self._live, gid) - 1
        while pos >= 0:
            cand = self._groups.get(self._live[pos])
            if self._waiting(cand):
                return cand.gid
            pos -= 1
        return None

    def _younger_waiting(self, gid: int) -> bool:
        """Whether a live group younger than ``gid`` still has an entry to restore."""

        pos = len(self._live) - 1
        while pos >= 0 and self._live[pos] > gid:
            if self._waiting(self._groups.get(self._live[pos])):
                return True
            pos -= 1
        return False

    def group_bytes(self, gid: int) -> int:
        """Payload bytes of the entries of ``gid`` still to restore (0 for an unknown group)."""

        with self._lock:
            group = self._groups.get(gid)
            if group is None:
                return 0
            return sum(e.nbytes for e in group.entries if e.refs > 0 and e.restored is None)

    def committed(self, gid: int) -> bool:
        """Whether ``gid`` is a known, committed group."""

        with self._lock:
            group = self._groups.get(gid)
            return group is not None and group.committed

    # ------------------------------------------------------------------ housekeeping
    def synchronize(self) -> None:
        with self._lock:
            _native.check("mo_synchronize", self._lib.mo_synchronize(self._handle))
            if self._held:
                self._hold()

    def stats(self) -> dict:
        with self._lock:
            out = _native.MoStats()
            _native.check("mo_get_stats", self._lib.mo_get_stats(self._handle, ctypes.byref(out)))
            result = out.as_dict()
            result["py_groups_live"] = len(self._groups)
            for key, value in self._ahead_counts.items():
                result[f"py_ahead_{key}"] = value
            return result

    def reset_stats(self) -> None:
        with self._lock:
            _native.check("mo_reset_stats", self._lib.mo_reset_stats(self._handle))
            self._ahead_counts = dict.fromkeys(self._ahead_counts, 0)

    def trim(self) -> None:
        with self._lock:
            _native.check("mo_trim", self._lib.mo_trim(self._handle))

    def live_groups(self) -> int:
        with self._lock:
            return len(self._groups)

    def link_name(self) -> str:
        with self._lock:
            return self._lib.mo_link_name(self._handle).decode()

    def close(self) -> None:
        with self._lock:
            if self._handle:
                _native.check("mo_destroy", self._lib.mo_destroy(self._handle))
                self._handle = ctypes.c_void_p()
                self._held.clear()
                self._groups.clear()
                self._live.clear()


_ENGINES: dict[int, OffloadEngine] = {}
_ENGINES_LOCK = threading.Lock()
_DEFAULT_CONFIG = EngineConfig()


def configure(**overrides) -> EngineConfig:
    """Set the configuration used by engines created from now on; return it.

    Existing engines keep theirs (see :func:`reset_engines`).
    """

    global _DEFAULT_CONFIG
    names = {f.name for f in fields(EngineConfig)}
    unknown = set(overrides) - names
    if unknown:
        raise ValueError(f"unknown engine options: {sorted(unknown)}")
    values = {f.name: getattr(_DEFAULT_CONFIG, f.name) for f in fields(EngineConfig)}
    values.update(overrides)
    _DEFAULT_CONFIG = EngineConfig(**values)
    return _DEFAULT_CONFIG


def get_engine(device: torch.device) -> OffloadEngine:
    """The engine of ``device``, created on first use with the current configuration."""

    index = device.index if device.index is not None else torch.cuda.current_device()
    with _ENGINES_LOCK:
        engine = _ENGINES.get(index)
        if engine is None:
            engine = OffloadEngine(torch.device("cuda", index), _DEFAULT_CONFIG)
            _ENGINES[index] = engine
        return engine


def reset_engines() -> None:
    """Destroy every engine (no live handles may remain); the next use creates new ones."""

    with _ENGINES_LOCK:
        for engine in _ENGINES.values():
            if engine.live_groups():
                raise RuntimeError("cannot reset an engine that still holds offloaded activations")
        for engine in _ENGINES.values():
            engine.close()
        _ENGINES.clear()


@atexit.register
def _close_engines_at_exit() -> None:
    # Release streams, events, staging memory and pinned host memory while the HIP runtime is
    # still fully alive, instead of leaving them to process teardown. Handles that outlive
    # this (graphs still referenced at exit) find their engine closed and do nothing.
    with _ENGINES_LOCK:
        for engine in _ENGINES.values():
            try:
                engine.close()
            except Exception:
                pass
        _ENGINES.clear()
