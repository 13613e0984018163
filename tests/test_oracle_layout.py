"""Pins the layout half of the oracle and checks the drop-in's layout helpers against it (CPU).

- The reference's own known-answer tests (tests/golden/layout_kats.json, from
  training/tests/test_packed_features.py:201-235).
- Brute force: for small random layouts, ``offload_view`` must agree with an enumeration of
  storage offsets (the stride-nested walk must be strictly increasing; oracle/layout.py), an
  accepted layout must never overlap, and the restored tensor must equal the original.
- Planted mistakes in a copy of the oracle must be caught by the same checks.
"""

from __future__ import annotations

import json
import random
from pathlib import Path

import numpy as np
import pytest
import torch

from moss_offload import _offload_view, _restore_layout, _storage_key
from oracle import layout, reference_hooks

KATS = json.loads((Path(__file__).parent / "golden" / "layout_kats.json").read_text())["cases"]


def _backing(name: str) -> torch.Tensor:
    return {"arange64": torch.arange(64, dtype=torch.float32), "arange5": torch.arange(5, dtype=torch.float32)}[name]


def _make(case) -> torch.Tensor:
    backing = _backing(case["backing"])
    if case["backing"] == "arange5":
        return backing.view(1, 5).expand(*case["shape"])
    return backing.as_strided(tuple(case["shape"]), tuple(case["stride"]))


@pytest.mark.parametrize("impl", ["oracle", "dropin"])
@pytest.mark.parametrize("case", KATS, ids=[c["name"] for c in KATS])
def test_reference_layout_kats(case, impl) -> None:
    offload_view = reference_hooks.offload_view if impl == "oracle" else _offload_view
    restore_layout = reference_hooks.restore_layout if impl == "oracle" else _restore_layout
    tensor = _make(case)
    assert tuple(tensor.stride()) == tuple(case["stride"])
    view = offload_view(tensor)
    if not case["offloadable"]:
        assert view is None
        return
    assert view is not None
    source, payload_shape = view
    assert list(payload_shape) == case["payload_shape"]
    restored = restore_layout(
        source.contiguous(), torch.device("cpu"), tuple(tensor.shape), tuple(tensor.stride()), payload_shape,
        non_blocking=False,
    )
    assert list(restored.stride()) == case["restored_stride"]
    assert restored.reshape(-1).tolist() == case["values"]
    assert reference_hooks.bitwise_equal(restored, tensor)


def _random_layouts(count: int, seed: int):
    rng = random.Random(seed)
    for _ in range(count):
        ndim = rng.randint(0, 4)
        shape = [rng.choice([1, 1, 2, 3, 4]) for _ in range(ndim)]
        stride = [rng.choice([-2, 0, 1, 2, 3, 4, 5, 6, 8, 12, 16, 24]) for _ in range(ndim)]
        yield tuple(shape), tuple(stride)


def _tensor(shape, stride):
    """A view with the given layout over a large enough backing (non-negative strides only)."""

    span = 1 + sum((s - 1) * abs(st) for s, st in zip(shape, stride))
    backing = torch.arange(span + 8, dtype=torch.float32) * 1.5 - 3.0
    return backing.as_strided(shape, stride, 0)


@pytest.mark.parametrize("impl", ["oracle", "dropin"])
def test_offload_view_matches_brute_force(impl) -> None:
    offload_view = reference_hooks.offload_view if impl == "oracle" else _offload_view
    checked = offloadable = interleaved = 0
    for shape, stride in _random_layouts(3000, seed=11):
        if any(s < 0 for s in stride):
            # torch cannot build negative strides; the rule is a plain sign test.
            continue
        tensor = _tensor(shape, stride)
        view = offload_view(tensor)
        assert (view is not None) == layout.offloadable(shape, stride), (shape, stride)
        checked += 1
        if view is None:
            interleaved += layout.interleaved_overlap_free(shape, stride)
            continue
        assert not layout.overlaps(shape, stride)  # the rule is sound
        offloadable += 1
        source, payload_shape = view
        assert payload_shape == layout.narrowed_shape(shape, stride)
        flat = tensor.untyped_storage()
        flat = torch.tensor([], dtype=torch.float32).set_(flat).numpy()
        expected = layout.logical_payload(flat, 0, shape, stride)
        assert np.array_equal(source.contiguous().reshape(-1).numpy(), expected)
        restored = reference_hooks.restore_layout(
            source.contiguous(), torch.device("cpu"), shape, stride, payload_shape, non_blocking=False
        )
        assert restored.stride() == tensor.stride()
        assert reference_hooks.bitwise_equal(restored, tensor)
    assert checked > 1500 and offloadable > 300
    # The reference rule is conservative: some overlap-free interleaved layouts stay resident.
    assert interleaved > 0


def _mutant_strict(tensor):
    """The overlap walk with ``<=`` instead of ``<``: wrongly rejects dense layouts."""

    shape = list(tensor.shape)
    extent = 1
    for stride, size in sorted((st, sz) for sz, st in zip(shape, tensor.stride()) if sz > 1):
        if stride <= extent:
            return None
        extent += (size - 1) * stride
    return tensor, tuple(shape)


def _mutant_no_narrow(tensor):
    """Forgets to narrow expanded dims: stride 0 then counts as overlap."""

    if any(st == 0 and sz > 1 for sz, st in zip(tensor.shape, tensor.stride())):
        return None
    return reference_hooks.offload_view(tensor)


def _mutant_extent(tensor):
    """Adds ``size * stride`` instead of ``(size - 1) * stride`` to the extent."""

    shape = list(tensor.shape)
    source = tensor
    for dim, (size, stride) in enumerate(zip(tensor.shape, tensor.stride())):
        if stride == 0 and size > 1:
            source = source.narrow(dim, 0, 1)
            shape[dim] = 1
    extent = 1
    for stride, size in sorted((st, sz) for sz, st in zip(shape, tensor.stride()) if sz > 1):
        if stride < extent:
            return None
        extent += size * stride
    return source, tuple(shape)


@pytest.mark.parametrize("mutant", [_mutant_strict, _mutant_no_narrow, _mutant_extent])
def test_planted_layout_mistakes_are_caught(mutant) -> None:
    disagreements = 0
    for shape, stride in _random_layouts(3000, seed=12):
        if any(s < 0 for s in stride):
            continue
        tensor = _tensor(shape, stride)
        got = mutant(tensor) is not None
        if got != layout.offloadable(shape, stride):
            disagreements += 1
    assert disagreements > 0


def test_storage_key_is_per_storage() -> None:
    base = torch.zeros(16)
    assert _storage_key(base[2:]) == _storage_key(base) == reference_hooks.storage_key(base)
    assert _storage_key(torch.zeros(16)) != _storage_key(base)
