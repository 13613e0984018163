"""Drop-in replacement for MOSS-Image's ``training/activation_offload.py``.

Same public surface and decisions as the reference:

- ``activation_cpu_offload(model, enabled, device)`` (reference :80-149) returns
  ``nullcontext()`` unless ``enabled``, ``device.type == "cuda"`` (true for HIP devices on
  PyTorch-ROCm) and grad mode is on (:92-93); otherwise a context that installs a
  saved-tensor ``pack``/``unpack`` hook pair for the model's forward.
- Parameter-, buffer- and streamer-staging-backed saves stay resident (:95-118), and so do
  layouts the reference cannot offload (:119-121, :32-61).
- ``_offload_view`` (:32-61), ``_restore_layout`` (:64-77) and ``_storage_key`` (:27-29) keep
  their signatures and results.

What changes is the mechanism behind ``pack``/``unpack``: instead of one pinned tensor, one
``copy_`` on the compute stream and one event per save, saves are gathered by a HIP pack
kernel into a device staging ring and leave in one DMA per block segment on a dedicated copy
stream; backward restores whole blocks with one H2D per segment, prefetched one block ahead,
and a HIP unpack kernel scatters them into freshly allocated tensors with the original
strides. Block boundaries come from forward hooks on ``model.layers``.
"""

from __future__ import annotations

import collections
import threading
import warnings
import weakref
from contextlib import nullcontext
from typing import ContextManager

import torch
from torch import nn

from . import _native
from .engine import OffloadEngine, get_engine

try:  # a weak reference to a storage that does not keep it alive
    from torch.multiprocessing.reductions import StorageWeakRef
except ImportError:  # pragma: no cover
    StorageWeakRef = None


def _storage_key(tensor: torch.Tensor) -> tuple[str, int | None, int]:
    """Identity of a tensor's storage: ``(device type, device index, storage data_ptr)``.

    Restates ``training/activation_offload.py:27-29``.
    """

    device = tensor.device
    return device.type, device.index, tensor.untyped_storage().data_ptr()


def _offload_view(tensor: torch.Tensor) -> tuple[torch.Tensor, tuple[int, ...]] | None:
    """Return ``(source, payload_shape)`` for a view that can be copied densely, else None.

    Restates ``training/activation_offload.py:32-61``: a negative stride keeps the tensor
    resident; expanded (stride-0, size > 1) dimensions are narrowed to one element; the
    remaining dimensions of size > 1, taken in increasing stride order, must each start at or
    beyond the extent covered by the smaller ones, or the layout overlaps and stays resident.
    """

    sizes = tuple(tensor.shape)
    strides = tuple(tensor.stride())
    payload_shape = list(sizes)
    source = tensor
    for dim in range(len(sizes)):
        stride = strides[dim]
        if stride < 0:
            return None
        if stride == 0 and sizes[dim] > 1:
            source = source.narrow(dim, 0, 1)
            payload_shape[dim] = 1
    extent = 1
    for stride, size in sorted(
        (strides[dim], payload_shape[dim]) for dim in range(len(sizes)) if payload_shape[dim] > 1
    ):
        if stride < extent:
            return None
        extent += (size - 1) * stride
    return source, tuple(payload_shape)


def _payload_key(source: torch.Tensor) -> tuple[int, tuple[tuple[int, int], ...], int]:
    """The bytes a payload holds, independent of the view that names them.

    ``(byte offset in the storage, ((size, byte stride), ...), element size)``: the dimensions
    of size > 1 in storage order (decreasing stride), adjacent ones merged where the outer
    stride equals the inner extent. Two views of one storage with equal keys have identical
    payloads over the same bytes (a ``[1,H,T,hd]`` transposed view and the ``[1,T,D]`` view of
    the same attention output, say), so one copy serves both.
    """

    es = source.element_size()
    dims = sorted(((size, stride * es) for size, stride in zip(source.shape, source.stride()) if size > 1),
                  key=lambda d: -d[1])
    merged: list[tuple[int, int]] = []
    for size, stride in dims:
        if merged and merged[-1][1] == size * stride:
            merged[-1] = (merged[-1][0] * size, stride)
        else:
            merged.append((size, stride))
    return source.storage_offset() * es, tuple(merged), es


def _bf16_exact(tensor: torch.Tensor, source: torch.Tensor) -> bool:
    """True when ``tensor`` is the untouched output of a bfloat16 -> float32 cast, so that the low
    16 bits of every element are zero and its high halves alone restore it bit for bit.

    Read from the autograd graph: the tensor's node is ``ToCopyBackward0`` and the gradient
    its input receives is bfloat16 (the cast's source dtype). ``_version == 0``: nothing,
    autograd-visible or under ``no_grad``, has written it since the cast. The payload must also
    be dense in storage order and 16-byte aligned (the engine's narrowing path).
    """

    if tensor.dtype != torch.float32 or source is not tensor or tensor._version != 0:
        return False
    fn = tensor.grad_fn
    if fn is None or type(fn).__name__ != "ToCopyBackward0" or tensor.data_ptr() % 16:
        return False
    try:
        node, nr = fn.next_functions[0]
        if node is None or node._input_metadata[nr].dtype != torch.bfloat16:
            return False
    except (AttributeError, IndexError, RuntimeError):  # private autograd API absent or changed
        return False
    dims = _payload_key(source)[1]
    return len(dims) <= 1 and (not dims or dims[0][1] == 4)


def _restore_layout(
    payload: torch.Tensor,
    device: torch.device,
    shape: tuple[int, ...],
    stride: tuple[int, ...],
    payload_shape: tuple[int, ...],
    *,
    non_blocking: bool,
) -> torch.Tensor:
    """Copy a dense payload into a tensor with the original (padded/expanded) layout.

    Restates ``training/activation_offload.py:64-77``: allocate ``empty_strided(payload_shape,
    stride)``, fill it from the dense, logically ordered ``payload`` with ``Tensor.copy_`` and
    return the ``as_strided(shape, stride)`` view. This is the reference's utility, kept for
    callers and tests that import it; the offload hooks do not use it (their payloads are in
    storage order and are restored by the engine's unpack kernel).
    """

    restored = torch.empty_strided(payload_shape, stride, dtype=payload.dtype, device=device)
    restored.copy_(payload, non_blocking=non_blocking)
    return restored.as_strided(shape, stride)


class _OffloadedTensor:
    """Handle returned by ``pack`` for an offloaded save (reference :17-24).

    The reference's handle owns a pinned CPU tensor and a CUDA event. This one owns one
    reference to ``(group, entry)`` in the device engine, which holds the payload in pinned
    host memory; dropping the handle (the autograd graph freeing the saved variable) drops
    the reference. ``shape``, ``stride`` and ``payload_shape`` mean what they mean in the
    reference. ``group is None`` marks a save with no elements.
    """

    __slots__ = ("engine", "group", "entry", "device", "dtype", "shape", "stride", "payload_shape", "reader")

    def __init__(self, engine, group, entry, device, dtype, shape, stride, payload_shape, reader=True):
        self.engine = engine
        self.group = group
        self.entry = entry
        self.device = device
        self.dtype = dtype
        self.shape = shape
        self.stride = stride
        self.payload_shape = payload_shape
        self.reader = reader  # False: held by a recomputed save for its replay, not by autograd

    def __del__(self):
        engine = self.engine
        if engine is not None and self.group is not None:
            try:
                engine.drop(self.group, self.entry, self.reader)
            except Exception:  # interpreter shutdown or engine already closed
                pass


class _DerivedTensor:
    """Handle for a save that is recomputed on unpack instead of offloaded.

    The save is an elementwise product of saves this context already holds (``torch.mul`` of two
    tensors of one shape and dtype, or of a tensor and a Python number), or a dense view of
    such a product. Unpack restores the inputs and replays the same ``torch.mul`` call: a
    deterministic elementwise kernel on the same bits, so the result is the saved tensor bit
    for bit, with no bytes over the host link. ``inputs`` are handles of this context
    (offloaded, derived or resident tensors) that each hold their own reference.
    """

    __slots__ = ("inputs", "scalar", "shape", "stride")

    def __init__(self, inputs, scalar, shape, stride):
        self.inputs = inputs
        self.scalar = scalar
        self.shape = shape
        self.stride = stride


_SETTLE_LOCK = threading.Lock()
_ALIAS_MIN_BYTES = 1 << 20  # smaller casts are offloaded: the check would cost more than the copy


class _CheckedAlias:
    """Handle for a save compared, on the device, with an earlier save of this context that has
    the same origin: a second cast of the same autograd output (the two ``tokens.float()`` of
    RMSNorm, ``training/model.py:171``). The graph cannot prove such casts equal (the source may
    have been written under ``no_grad`` in between), so the engine compares the bytes
    (``mo_equal``) while this handle keeps the save alive. Equal: ``target`` (a reference to
    the earlier save's entry) restores it and the save is let go. Different: the save stays on
    the device as saved, like a layout the reference keeps resident."""

    __slots__ = ("engine", "ticket", "target", "tensor")

    def __init__(self, engine, ticket, target, tensor):
        self.engine = engine
        self.ticket = ticket
        self.target = target
        self.tensor = tensor

    def settle(self, wait: bool) -> bool:
        """Take the result if it is known (or ``wait``); True once settled."""

        with _SETTLE_LOCK:  # forward polls on the caller's thread, unpack on autograd's
            if self.ticket:
                state = self.engine.equal_result(self.ticket, wait)
                if state == 0:
                    return False
                self.ticket = 0
                if state == 1:
                    self.tensor = None
                else:
                    self.target = None
            return True

    def __del__(self):
        if self.ticket:
            try:
                self.engine.equal_discard(self.ticket)
            except Exception:  # interpreter shutdown or engine already closed
                pass


def _cast_origin(tensor: torch.Tensor):
    """``(autograd node, output index)`` of the tensor a cast was made from, if ``tensor`` is
    the untouched output of a dtype cast (``ToCopyBackward0``) of a tensor that requires grad."""

    fn = tensor.grad_fn
    if fn is None or tensor._version != 0 or type(fn).__name__ != "ToCopyBackward0":
        return None
    try:
        edge = fn.next_functions[0]
    except (AttributeError, IndexError, RuntimeError):  # private autograd API absent or changed
        return None
    return edge if edge[0] is not None else None


_VIEW_NODES = ("ViewBackward0", "UnsafeViewBackward0", "ReshapeAliasBackward0")

# What the pack hook did with each save, summed over every context of the process:
#   resident      kept on the device (non-CUDA, parameter/buffer/staging storage, layout the
#                 reference keeps resident, keep_last_blocks)
#   offloaded     a new engine entry (its payload crosses the link)
#   narrowed      of those, float32 casts sent as their bfloat16 high halves
#   deduplicated  a view of bytes already offloaded: a second reference to that entry
#   derived       a torch.mul product recomputed on unpack (nothing crosses the link)
#   aliased       a second cast compared on the device with an earlier one
#   empty         a save with no elements
_COUNTS: collections.Counter = collections.Counter()


def hook_counters() -> dict[str, int]:
    """What the pack hook did with the saves it has seen (see ``_COUNTS``)."""

    return dict(_COUNTS)


def reset_hook_counters() -> None:
    _COUNTS.clear()


def hook_features() -> dict[str, bool]:
    """Which graph-reading features of the pack hook work on the running torch.

    Narrowed casts, recomputed products and aliased equal casts read private autograd state
    (``ToCopyBackward0`` input metadata, ``MulBackward0``'s saved scalar, node edges). Each
    fails closed: when the state is missing the save is offloaded whole. This probes each on a
    tiny CPU graph, so a torch upgrade that removes one shows here instead of only as more
    bytes over the link.
    """

    out = {}
    source = torch.ones(8, dtype=torch.bfloat16, requires_grad=True)
    cast = source.float()
    out["narrow_bf16_casts"] = _bf16_exact(cast, cast)
    out["alias_equal_casts"] = _cast_origin(cast) is not None
    base = torch.ones(8, requires_grad=True) * 1.0
    try:
        product = base * 3.0
        fn = product.grad_fn
        ok = type(fn).__name__ == "MulBackward0" and fn._raw_saved_other.unpack_hook is None
        other = fn._saved_other
        ok = ok and isinstance(other, torch.Tensor) and other.dim() == 0 and float(other) == 3.0
        ok = ok and fn.next_functions[0][0] is base.grad_fn
    except (AttributeError, IndexError, RuntimeError):
        ok = False
    out["recompute_products"] = bool(ok)
    return out


_REPORTED = False


def _report_features(config) -> None:
    """Warn once per process about a configured feature the running torch cannot support."""

    global _REPORTED
    if _REPORTED:
        return
    _REPORTED = True
    features = hook_features()
    missing = [name for name, ok in features.items() if getattr(config, name, False) and not ok]
    if missing:
        warnings.warn(
            "activation offload: " + ", ".join(missing) + " unavailable on torch " + torch.__version__
            + " (private autograd state missing); those saves are offloaded whole",
            RuntimeWarning,
            stacklevel=3,
        )


def _numel(shape) -> int:
    n = 1
    for size in shape:
        n *= size
    return n


class _ActivationOffload:
    """The context returned for an enabled offload: hooks + block boundaries + dedupe."""

    def __init__(self, model: nn.Module, device: torch.device, engine: OffloadEngine | None = None) -> None:
        self.model = model
        self.device = device
        # the device's shared engine, unless a caller brings its own (a second transport, say)
        self.engine: OffloadEngine = engine if engine is not None else get_engine(device)
        # Reference :95-99: storages of CUDA parameters and buffers stay resident.
        self.resident_storages = {
            _storage_key(tensor)
            for tensor in (*model.parameters(), *model.buffers())
            if tensor.device.type == "cuda" and tensor.untyped_storage().nbytes()
        }
        self.dedupe = self.engine.config.dedupe and StorageWeakRef is not None
        self.narrow = self.engine.config.narrow_bf16_casts
        self.recompute = self.engine.config.recompute_products
        self.alias = getattr(self.engine.config, "alias_equal_casts", False)
        _report_features(self.engine.config)
        # cast origin (autograd node, output index) -> (handle, weak ref, version, stream) of an
        # offloaded cast, and the aliases whose device comparison has no result yet
        self._casts: dict[tuple, tuple] = {}
        self._pending: list[_CheckedAlias] = []
        # (autograd node, output index) -> (handle, weak ref, version at the save) of every save
        # packed so far: the inputs a later product can be recomputed from
        self._made: dict[tuple, tuple] = {}
        self._seen: dict[tuple, tuple] = {}
        # saves a later block made again: (group, entry) -> None, in the order first seen
        self._shared: dict[tuple[int, int], None] = {}
        self._hooks = torch.autograd.graph.saved_tensors_hooks(self.pack, self.unpack)
        self._block_handles: list = []
        # keep_last_blocks: block index of each layer, and the first index whose saves stay
        self._layer_index: dict[int, int] = {}
        self._keep_from: int | None = None
        self._block: int | None = None  # the block running now (between its forward hooks)

    # ------------------------------------------------------------------ context
    def __enter__(self):
        layers = getattr(self.model, "layers", None)
        if isinstance(layers, (nn.ModuleList, nn.Sequential)):
            keep = max(0, int(self.engine.config.keep_last_blocks))
            if keep:
                self._layer_index = {id(layer): i for i, layer in enumerate(layers)}
                self._keep_from = len(layers) - keep
            for layer in layers:
                self._block_handles.append(layer.register_forward_pre_hook(self._boundary))
                self._block_handles.append(layer.register_forward_hook(self._boundary_post))
        self._hooks.__enter__()
        return self

    def __exit__(self, *exc):
        try:
            self._hooks.__exit__(*exc)
        finally:
            for handle in self._block_handles:
                handle.remove()
            self._block_handles.clear()
            self._seen.clear()
            self._made.clear()
            self._casts.clear()
            self._poll()
        stream = torch.cuda.current_stream(self.device).cuda_stream
        last = self.engine.commit(stream)
        # the forward is over: gathers still waiting for later commits run now, their segments
        # go to the host, and the engine lets go of their sources (which would otherwise keep
        # the forward's graph alive until the next engine call)
        self.engine.flush()
        if self.engine.config.prefetch and exc[0] is None:
            # Backward starts with the last group, and with every group holding a save that
            # later blocks made again (e.g. one RoPE table checkpointed with every block): start
            # bringing them back now, those first, then the groups backward needs after the
            # last one (which would otherwise take every free slot before a shared group got
            # one). Segments still in the staging ring are skipped. A shared group larger than
            # one restore-ahead launch (a non-checkpointed block's whole saved set) is not
            # fetched whole: only the segments holding its shared saves, which backward restores
            # alone (fetched on demand instead, such a segment queued behind the next block's
            # prefetch: 21 ms a step at 2048^2).
            limit = max(self.engine.config.restore_ahead_bytes, 1)
            small, entries = [], []
            for gid in sorted({g for g, _ in self._shared} - {last}, reverse=True):
                if self.engine.group_bytes(gid) <= limit:
                    small.append(gid)
                else:
                    entries.extend((g, i) for g, i in self._shared if g == gid)
            for gid in ([last] if last is not None else []) + small:
                self.engine.prefetch(gid, stream)
            for gid, idx in entries:
                self.engine.prefetch_entry(gid, idx, stream)
            if last is not None:
                self.engine.prefetch(last, stream, ahead=True)
        self._shared.clear()
        return False

    def _boundary(self, module, args):
        self.engine.commit(torch.cuda.current_stream(self.device).cuda_stream)
        self._block = self._layer_index.get(id(module))

    def _boundary_post(self, module, args, output):
        self.engine.commit(torch.cuda.current_stream(self.device).cuda_stream)
        self._block = None

    # ------------------------------------------------------------------ hooks
    def is_weight_backed(self, tensor: torch.Tensor) -> bool:
        """Reference :101-114: parameters, buffers and the streamers' staging buffers."""

        key = _storage_key(tensor)
        if key in self.resident_storages:
            return True
        manager = getattr(self.model, "block_swap_manager", None)
        owned = getattr(manager, "owned_cuda_buffers", None)
        if not callable(owned):
            return False
        return any(buffer.device.type == "cuda" and _storage_key(buffer) == key for buffer in owned())

    def pack(self, tensor: torch.Tensor):
        if tensor.device.type != "cuda" or tensor.layout != torch.strided or self.is_weight_backed(tensor):
            _COUNTS["resident"] += 1
            return tensor
        if self._keep_from is not None and self._block is not None and self._block >= self._keep_from:
            _COUNTS["resident"] += 1
            return tensor  # keep_last_blocks: needed first by backward
        view = _offload_view(tensor)
        if view is None or tensor.dim() > _native.MO_MAX_DIMS:
            _COUNTS["resident"] += 1
            return tensor
        source, payload_shape = view
        shape, stride = tuple(tensor.shape), tuple(tensor.stride())
        device = tensor.device
        if source.numel() == 0:
            _COUNTS["empty"] += 1
            return _OffloadedTensor(None, None, 0, device, tensor.dtype, shape, stride, payload_shape)
        if self._pending:
            self._poll()
        if self.recompute:
            derived = self._derive(tensor)
            if derived is not None:
                _COUNTS["derived"] += 1
                self._remember(tensor, derived)
                return derived
        stream = torch.cuda.current_stream(device).cuda_stream
        origin = _cast_origin(tensor) if self.alias else None
        if origin is not None:
            alias = self._alias(tensor, origin, stream)
            if alias is not None:
                _COUNTS["aliased"] += 1
                self._remember(tensor, alias)
                return alias
        key = None
        if self.dedupe:
            # by payload bytes, not by view: any view of the same bytes in the same storage order
            # reuses the entry (unpack re-strides the restored storage to the asking view)
            key = (tensor.untyped_storage().data_ptr(), _payload_key(source), tensor.dtype)
            hit = self._seen.get(key)
            if hit is not None:
                ref, version, gid, idx = hit
                if not ref.expired() and version == tensor._version and self.engine.acquire(gid, idx):
                    _COUNTS["deduplicated"] += 1
                    if self.engine.committed(gid):  # saved again by a later block
                        self._shared[(gid, idx)] = None
                    handle = _OffloadedTensor(self.engine, gid, idx, device, tensor.dtype, shape, stride, payload_shape)
                    self._remember(tensor, handle)
                    return handle
        narrow = self.narrow and _bf16_exact(tensor, source)
        gid, idx = self.engine.pack(source, stream, narrow=narrow)
        _COUNTS["offloaded"] += 1
        _COUNTS["narrowed"] += narrow
        if key is not None:
            self._seen[key] = (StorageWeakRef(tensor.untyped_storage()), tensor._version, gid, idx)
        handle = _OffloadedTensor(self.engine, gid, idx, device, tensor.dtype, shape, stride, payload_shape)
        self._remember(tensor, handle)
        if origin is not None:
            self._casts[origin] = (handle, weakref.ref(tensor), tensor._version, stream)
        return handle

    # ------------------------------------------------------------------ equal casts
    def _alias(self, tensor: torch.Tensor, origin, stream: int) -> _CheckedAlias | None:
        """A ``_CheckedAlias`` of an earlier offloaded cast of the same origin, with the device
        comparison of the two started, if that cast is still alive, unchanged and laid out
        the same; else None."""

        rec = self._casts.get(origin)
        if rec is None:
            return None
        handle, ref, version, rec_stream = rec
        earlier = ref()
        if earlier is None or earlier._version != version or earlier is tensor:
            return None
        if tensor.numel() * tensor.element_size() < _ALIAS_MIN_BYTES:
            return None
        if (earlier.dtype != tensor.dtype or earlier.shape != tensor.shape or not tensor.is_contiguous()
                or not earlier.is_contiguous() or tensor.data_ptr() % 16 or earlier.data_ptr() % 16):
            return None
        # the comparison runs on the stream the earlier cast was offloaded from, which orders it
        # before any reuse of that cast's memory once the engine lets go of it
        if stream != rec_stream:
            return None
        target = self._own(handle, reader=True)
        if target is None:
            return None
        ticket = self.engine.equal(earlier, tensor, stream)
        if not ticket:
            return None
        alias = _CheckedAlias(self.engine, ticket, target, tensor)
        self._pending.append(alias)
        return alias

    def _poll(self) -> None:
        self._pending = [alias for alias in self._pending if not alias.settle(False)]

    # ------------------------------------------------------------------ recomputed products
    def _remember(self, tensor: torch.Tensor, handle) -> None:
        if self.recompute and tensor.grad_fn is not None:
            meta = (tensor.dtype, tuple(tensor.shape), tensor.is_contiguous())
            self._made[(tensor.grad_fn, tensor.output_nr)] = (handle, weakref.ref(tensor), tensor._version, meta)

    def _held_input(self, edge):
        """The handle and (dtype, shape, contiguous) of a product's input, if this context saved
        it and, while the tensor lives, it is unchanged since (its version counter).

        A freed input cannot change any more. Between its save and its death it could only have
        been written in place, which autograd rejects in backward without offloading (the node
        that saved it needs the saved value), so a step valid without offloading never does it;
        the reference model's products (SiTU-GLU temporaries) are consumed at once."""

        node, nr = edge
        if node is None:
            return None
        rec = self._made.get((node, nr))
        if rec is None:
            return None
        handle, ref, version, meta = rec
        tensor = ref()
        if tensor is not None and tensor._version != version:
            return None
        return handle, meta

    def _own(self, handle, reader: bool = False):
        """A reference of a derived or alias handle's own to an input handle: ``reader`` when its
        restore goes to autograd (an alias's target), not when a replay only reads it."""

        if isinstance(handle, _OffloadedTensor) and handle.group is not None:
            if not self.engine.acquire(handle.group, handle.entry, reader=reader):
                return None
            return _OffloadedTensor(handle.engine, handle.group, handle.entry, handle.device, handle.dtype,
                                    handle.shape, handle.stride, handle.payload_shape, reader=reader)
        return handle  # a derived handle (owns its inputs) or a resident tensor

    def _derive(self, tensor: torch.Tensor) -> _DerivedTensor | None:
        """A ``_DerivedTensor`` for ``tensor`` if it is the untouched output of a ``torch.mul``
        (or a dense view of one) whose inputs this context saved unchanged, else None."""

        fn = tensor.grad_fn
        if fn is None or tensor._version != 0 or not tensor.is_contiguous():
            return None
        name = type(fn).__name__
        if name in _VIEW_NODES:
            # a view that covers its whole storage densely: the product it views, reshaped
            if tensor.storage_offset() != 0 or tensor.numel() * tensor.element_size() != tensor.untyped_storage().nbytes():
                return None
            fn = fn.next_functions[0][0]
            if fn is None or type(fn).__name__ != "MulBackward0":
                return None
        elif name != "MulBackward0":
            return None
        try:
            edges = fn.next_functions
            a = self._held_input(edges[0])
            if a is None:
                return None
            if edges[1][0] is None:
                # a Python number is saved as a 0-dim CPU tensor without the hooks; a tensor that
                # went through them would be unpacked by reading it, so it is left alone
                if fn._raw_saved_other.unpack_hook is not None:
                    return None
                other = fn._saved_other
                if not (isinstance(other, torch.Tensor) and other.dim() == 0 and other.device.type == "cpu"):
                    return None
                scalar, inputs = other.item(), [a]
            else:
                b = self._held_input(edges[1])
                if b is None:
                    return None
                scalar, inputs = None, [a, b]
        except (AttributeError, IndexError, RuntimeError):  # private autograd API absent or changed
            return None
        numel = tensor.numel()
        for _, (dtype, shape, contiguous) in inputs:
            if dtype != tensor.dtype or not contiguous or _numel(shape) != numel:
                return None
        if len(inputs) == 2 and inputs[0][1][1] != inputs[1][1][1]:
            return None
        owned = []
        for handle, _ in inputs:
            mine = self._own(handle)
            if mine is None:
                return None
            owned.append(mine)
        return _DerivedTensor(tuple(owned), scalar, tuple(tensor.shape), tuple(tensor.stride()))

    def unpack(self, saved):
        if isinstance(saved, torch.Tensor):
            return saved
        if isinstance(saved, _DerivedTensor):
            args = [self.unpack(h) for h in saved.inputs]
            product = torch.mul(args[0], saved.scalar if saved.scalar is not None else args[1])
            return product.as_strided(saved.shape, saved.stride)
        if isinstance(saved, _CheckedAlias):
            saved.settle(True)
            return saved.tensor if saved.tensor is not None else self.unpack(saved.target)
        if saved.group is None:
            restored = torch.empty_strided(saved.payload_shape, saved.stride, dtype=saved.dtype, device=saved.device)
        else:
            stream = torch.cuda.current_stream(saved.device).cuda_stream
            restored = saved.engine.restore(saved.group, saved.entry, stream, saved.reader)
        return restored.as_strided(saved.shape, saved.stride)


def activation_cpu_offload(
    model: nn.Module,
    enabled: bool,
    device: torch.device,
) -> ContextManager[object]:
    """Offload tensors saved by autograd to pinned host memory.

    Reference ``training/activation_offload.py:80-149``. Parameter-backed tensors remain
    resident. HIP events order the asynchronous device-to-host copies before backward
    restores a tensor.
    """

    if not enabled or device.type != "cuda" or not torch.is_grad_enabled():
        return nullcontext()
    return _ActivationOffload(model, device)
