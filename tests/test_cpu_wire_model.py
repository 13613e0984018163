"""The numpy model of the engine's wire coding (``tests/wire_model.py``, format in
``csrc/mo_wire.h``): lossless on every 16-bit pattern class, sizes as the format fixes them,
and the library's ``mo_wire_capacity`` equal to the model's worst case."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import wire_model as wm


def _bf16_bytes(values: torch.Tensor) -> bytes:
    return values.to(torch.bfloat16).contiguous().view(torch.int16).numpy().tobytes()


@pytest.mark.parametrize("raw_bytes", [0, 1, 2, 1023, 1024, 1025, 32 * 1024, 32 * 1024 + 1024 + 7, 200_000])
def test_round_trip_random_bits(raw_bytes) -> None:
    rng = np.random.default_rng(raw_bytes)
    raw = rng.integers(0, 256, raw_bytes, dtype=np.uint8).tobytes()
    stream, defined = wm.encode(raw)
    assert len(stream) <= wm.max_coded(raw_bytes) <= wm.capacity(raw_bytes)
    assert int(np.frombuffer(stream[:8], "<u8")[0]) == len(stream)
    assert wm.decode(stream, raw_bytes) == raw


def test_special_values_and_widths() -> None:
    special = torch.tensor([0.0, -0.0, float("inf"), -float("inf"), float("nan"), 1e-40, -1e-40, 3.0e38, 1.0])
    gauss = torch.randn(64 * 512, generator=torch.Generator().manual_seed(1))
    parts = [
        special.repeat(600),                # every exponent class, width 8
        torch.full((512,), 1.5),            # one exponent: width 0
        torch.full((512,), -2.0 ** -130),   # subnormal bf16, width 0
        gauss,                              # activations: widths 3-5
    ]
    raw = b"".join(_bf16_bytes(p) for p in parts)
    # NaN payloads: every mantissa pattern with exponent 255
    nan_words = (np.arange(256, dtype=np.uint16) | 0x7F80).astype("<u2").tobytes() * 2
    raw += nan_words + bytes(range(7))
    stream, _ = wm.encode(raw)
    assert wm.decode(stream, len(raw)) == raw
    # width 0 block: 512 sign-mantissa bytes only; Gaussian blocks code to about 0.7 of raw
    g = _bf16_bytes(gauss)
    gs, _ = wm.encode(g)
    assert len(gs) < 0.75 * len(g)
    flat = _bf16_bytes(torch.full((32 * 512,), 1.5))
    fs, _ = wm.encode(flat)
    assert len(fs) == wm.tiles_start(len(flat)) + wm.TILE_HEADER + 32 * 512


def test_choice_rule_closed_forms() -> None:
    """The block coding the format fixes, on blocks whose best coding is known by hand."""

    e = np.full(512, 120, np.uint32)
    assert wm.choose(e) == (0, 120, 0)                       # one exponent
    e[::2] = 121
    assert wm.choose(e) == (1, 120, 0)                       # two values, no escapes: 1 bit
    e[:4] = 200                                              # four far outliers
    # 1-bit window {120} + 258 escapes: 512 + 64 + 272 bytes; 2-bit window {120, 121, 122} + 4
    # escapes: 512 + 128 + 16 = 656 bytes, the smallest; width 8: 1024 bytes
    assert wm.block_coded(2, 4) < min(wm.block_coded(1, 258), wm.block_coded(8, 0))
    assert wm.choose(e) == (2, 120, 4)
    e[:4] = 123                                              # now all inside 2 bits, no escapes:
    assert wm.choose(e) == (2, 120, 0)                       # 512 + 128 bytes
    e[:4] = 124                                              # one past it: escapes (656 bytes) beat
    assert wm.choose(e) == (2, 120, 4)                       # 3 bits without them (704 bytes)
    rnd = np.random.default_rng(0).integers(0, 256, 512).astype(np.uint32)
    assert wm.choose(rnd)[0] == 8                            # random exponents: raw bytes


def test_planted_mistakes_are_caught() -> None:
    """A decoder that drops the sign, or mis-orders the packed exponent bits, fails the round
    trip on ordinary activations (so the round-trip checks above pin the format)."""

    raw = _bf16_bytes(torch.randn(4 * 512, generator=torch.Generator().manual_seed(2)))
    stream, _ = wm.encode(raw)
    s = bytearray(stream)
    # flip the first block's sign-mantissa byte 0 sign bit
    t0 = int(np.frombuffer(stream[16:20], "<u4")[0])
    s[t0 + wm.TILE_HEADER] ^= 0x80
    assert wm.decode(bytes(s), len(raw)) != raw
    s = bytearray(stream)
    w = (int(np.frombuffer(stream[t0:t0 + 4], "<u4")[0]) >> 8) & 0xF
    assert w > 0
    s[t0 + wm.TILE_HEADER + 512] ^= 0x01  # lowest bit of word 0's exponent code
    assert wm.decode(bytes(s), len(raw)) != raw


def test_library_capacity_matches_the_model() -> None:
    from moss_offload import _native

    lib = _native.load()
    for n in [0, 1, 1024, 32 * 1024, 32 * 1024 + 1, 128 << 20, (1 << 31)]:
        assert lib.mo_wire_capacity(n) == wm.capacity(n), n
