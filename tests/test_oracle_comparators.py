"""Pins the bitwise comparators every parity claim rests on: the oracle's ``bits`` /
``bitwise_equal`` (``oracle/reference_hooks.py``) and the GPU tests' ``bits_cpu`` /
``assert_bitwise`` (``tests/gpu_util.py``).

The reference's bar for restored activations is exact equality
(training/tests/test_offload_inputs.py:43-46, test_packed_features.py:201-235). "Exact" here
means the stored bits of every logical element: ``-0.0`` differs from ``+0.0`` and a NaN
equals a NaN of the same payload only, which ``torch.equal`` gets wrong both ways. Each case
below states its answer from the IEEE-754 encodings; planted comparators built on
``torch.equal``, on ``allclose``, or without the shape or dtype check must each get one wrong.
"""

from __future__ import annotations

import pytest
import torch

from gpu_util import assert_bitwise, bits_cpu
from oracle.reference_hooks import bits, bitwise_equal


def _from_bits(words, dtype):
    width = {torch.float32: torch.int32, torch.float64: torch.int64, torch.bfloat16: torch.int16,
             torch.float16: torch.int16}[dtype]
    return torch.tensor(words, dtype=torch.int64).to(width).view(dtype)


def _cases():
    """(label, a, b, bitwise equal?)"""

    cases = []
    for dtype in (torch.float32, torch.float64, torch.bfloat16, torch.float16):
        zero = torch.zeros(3, dtype=dtype)
        cases.append((f"{dtype} -0.0 vs +0.0", -zero, zero, False))
        cases.append((f"{dtype} +0.0 vs +0.0", zero, zero.clone(), True))
    # NaN payloads written bit by bit: quiet NaN, the same again, and one with another payload
    nan_words = {
        torch.float32: (0x7FC00000, 0x7FC00001),
        torch.float64: (0x7FF8000000000000, 0x7FF8000000000001),
        torch.bfloat16: (0x7FC0, 0x7FC1),
        torch.float16: (0x7E00, 0x7E01),
    }
    for dtype, (quiet, other) in nan_words.items():
        a = _from_bits([quiet, 1], dtype)
        cases.append((f"{dtype} same NaN payload", a, a.clone(), True))
        cases.append((f"{dtype} different NaN payloads", a, _from_bits([other, 1], dtype), False))
    # the lowest mantissa bit of one element
    x = torch.randn(64, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    y = x.clone()
    y.view(torch.int16)[17] ^= 1
    cases.append(("bf16 one low bit", x, y, False))
    # bool compares its stored byte: a 2 stored under a bool is not the True that 1 is
    t = torch.tensor([True, False, True])
    cases.append(("bool equal", t, t.clone(), True))
    cases.append(("bool different", t, torch.tensor([True, True, True]), False))
    cases.append(("bool stored byte 2 vs 1", torch.tensor([2, 0, 1], dtype=torch.uint8).view(torch.bool), t, False))
    # dtype and shape must match, whatever the bits
    f = torch.arange(6, dtype=torch.float32)
    cases.append(("float32 vs its int32 bits", f, f.view(torch.int32), False))
    cases.append(("shape [6] vs [2,3]", f, f.view(2, 3), False))
    cases.append(("shape [1,6] vs [6]", f.view(1, 6), f, False))
    cases.append(("empty (0,3) vs (3,0)", torch.empty(0, 3), torch.empty(3, 0), False))
    cases.append(("empty (0,3) vs (0,3)", torch.empty(0, 3), torch.empty(0, 3), True))
    # logical elements, not storage: a transposed view equals its contiguous copy, not its storage
    m = torch.arange(12, dtype=torch.float32).view(3, 4)
    cases.append(("transposed view vs contiguous copy", m.t(), m.t().contiguous(), True))
    cases.append(("transposed view vs storage order", m.t(), m.view(4, 3), False))
    cases.append(("0-d", torch.tensor(1.5), torch.tensor(1.5), True))
    cases.append(("0-d -0.0", torch.tensor(-0.0), torch.tensor(0.0), False))
    return cases


CASES = _cases()


def _assert_bitwise_bool(a, b) -> bool:
    try:
        assert_bitwise(a, b)
    except AssertionError:
        return False
    return True


COMPARATORS = {
    "oracle.bitwise_equal": bitwise_equal,
    "gpu_util.assert_bitwise": _assert_bitwise_bool,
}


@pytest.mark.parametrize("name", sorted(COMPARATORS))
@pytest.mark.parametrize("label,a,b,expected", CASES, ids=[c[0] for c in CASES])
def test_comparator_case(name, label, a, b, expected) -> None:
    assert COMPARATORS[name](a, b) is expected, label
    assert COMPARATORS[name](b, a) is expected, f"{label} (swapped)"


def test_bits_views_agree() -> None:
    for dtype in (torch.float32, torch.bfloat16, torch.float16, torch.float64, torch.int64, torch.uint8, torch.bool):
        t = torch.arange(8).to(dtype)
        assert torch.equal(bits(t), bits_cpu(t))
        assert bits(t).element_size() == t.element_size()


MUTANTS = {
    "torch.equal": lambda a, b: a.shape == b.shape and a.dtype == b.dtype and torch.equal(a, b),
    "allclose(equal_nan)": lambda a, b: a.shape == b.shape and a.dtype == b.dtype
    and (a.numel() == 0 or torch.allclose(a.float(), b.float(), rtol=0, atol=0, equal_nan=True)),
    "no dtype check": lambda a, b: a.shape == b.shape and a.element_size() == b.element_size()
    and torch.equal(bits(a), bits(b)),
    "no shape check": lambda a, b: a.dtype == b.dtype and a.numel() == b.numel()
    and torch.equal(bits(a).reshape(-1), bits(b).reshape(-1)),
    "bool by value": lambda a, b: a.shape == b.shape and a.dtype == b.dtype
    and torch.equal(a.to(torch.uint8) if a.dtype == torch.bool else bits(a),
                    b.to(torch.uint8) if b.dtype == torch.bool else bits(b)),
    "storage order": lambda a, b: a.shape == b.shape and a.dtype == b.dtype
    and torch.equal(torch.as_strided(a, (a.numel(),), (1,)).view(bits(a).dtype) if a.numel() else bits(a),
                    torch.as_strided(b, (b.numel(),), (1,)).view(bits(b).dtype) if b.numel() else bits(b)),
}


@pytest.mark.parametrize("mutant", sorted(MUTANTS))
def test_planted_comparators_fail_a_case(mutant) -> None:
    wrong = []
    for label, a, b, expected in CASES:
        try:
            got = bool(MUTANTS[mutant](a, b))
        except (RuntimeError, TypeError):
            got = None
        if got is not expected:
            wrong.append(label)
    assert wrong, f"planted comparator {mutant!r} passes every case"
