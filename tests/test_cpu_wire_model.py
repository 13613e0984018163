"""The numpy model of the engine's wire coding (``tests/wire_model.py``, format in
``csrc/mo_wire.h``): lossless on every 16-bit pattern class, sizes as the format fixes them, the
frequency normalisation and the rANS coder pinned by closed forms, and the library's
``mo_wire_capacity`` equal to the model's worst case."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import wire_model as wm


def _bf16_bytes(values: torch.Tensor) -> bytes:
    return values.to(torch.bfloat16).contiguous().view(torch.int16).numpy().tobytes()


def _tile_head(stream: bytes, tile: int) -> tuple[int, int, int, int]:
    """(offset, mode, nsym, stream words) of one tile."""

    off = int(np.frombuffer(stream[16 + 4 * tile:20 + 4 * tile], "<u4")[0])
    h0, nwords = np.frombuffer(stream[off:off + 8], "<u4")
    return off, int(h0) & 3, (int(h0) >> 8) & 0x1FF, int(nwords)


@pytest.mark.parametrize("raw_bytes", [0, 1, 2, 1023, 1024, 1025, 32 * 1024, 32 * 1024 + 1024 + 7, 200_000])
def test_round_trip_random_bits(raw_bytes) -> None:
    rng = np.random.default_rng(raw_bytes)
    raw = rng.integers(0, 256, raw_bytes, dtype=np.uint8).tobytes()
    stream, defined = wm.encode(raw)
    assert len(stream) <= wm.max_coded(raw_bytes) <= wm.capacity(raw_bytes)
    assert int(np.frombuffer(stream[:8], "<u8")[0]) == len(stream)
    assert wm.decode(stream, raw_bytes) == raw
    for t in range(wm.tiles_of(raw_bytes)):  # random exponents do not code smaller: raw tiles
        assert _tile_head(stream, t)[1] == wm.MODE_RAW


def test_special_values_and_modes() -> None:
    special = torch.tensor([0.0, -0.0, float("inf"), -float("inf"), float("nan"), 1e-40, -1e-40, 3.0e38, 1.0])
    gauss = torch.randn(64 * 512, generator=torch.Generator().manual_seed(1))
    parts = [
        special.repeat(600),                # every exponent class
        torch.full((512,), 1.5),            # one exponent
        torch.full((512,), -2.0 ** -130),   # subnormal bf16
        gauss,                              # activations
    ]
    raw = b"".join(_bf16_bytes(p) for p in parts)
    # NaN payloads: every mantissa pattern with exponent 255
    nan_words = (np.arange(256, dtype=np.uint16) | 0x7F80).astype("<u2").tobytes() * 2
    raw += nan_words + bytes(range(7))
    stream, _ = wm.encode(raw)
    assert wm.decode(stream, len(raw)) == raw
    # Gaussian bfloat16: exponent entropy about 2.7 bits, so about (8 + 2.7) / 16 of raw
    g = _bf16_bytes(gauss)
    gs, _ = wm.encode(g)
    assert len(gs) < 0.69 * len(g)
    # one exponent: one table entry, no stream words, 64 states
    flat = _bf16_bytes(torch.full((32 * 512,), 1.5))
    fs, _ = wm.encode(flat)
    off, mode, nsym, nwords = _tile_head(fs, 0)
    assert (mode, nsym, nwords) == (wm.MODE_RANS, 1, 0)
    assert len(fs) == wm.tiles_start(len(flat)) + wm.TILE_HEADER + 32 * 512 + 16 + 4 * wm.LANES
    states = np.frombuffer(fs[off + 16 + 32 * 512 + 16:off + 16 + 32 * 512 + 16 + 256], "<u4")
    assert (states == wm.STATE_LOW).all()  # a symbol of frequency 4096 leaves every state alone


def test_normalisation_closed_forms() -> None:
    def f_of(counts: dict[int, int], n: int):
        c = np.zeros(256, np.int64)
        for e, k in counts.items():
            c[e] = k
        f = wm.normalize(c, n)
        return None if f is None else {e: int(f[e]) for e in np.flatnonzero(f)}

    assert f_of({120: 512}, 512) == {120: 4096}                          # one exponent
    assert f_of({120: 256, 121: 256}, 512) == {120: 2048, 121: 2048}      # exact halves
    assert f_of({120: 300, 121: 200, 122: 12}, 512) == {120: 2400, 121: 1600, 122: 96}  # exact: 8 c
    # n = 1536: floor(8 c / 3) sums to 4095; the most frequent exponent takes the missing 1
    assert f_of({120: 1000, 121: 500, 122: 36}, 1536) == {120: 2667, 121: 1333, 122: 96}
    # a rare exponent keeps frequency 1 (floor(8 / 32) = 0), taken from the most frequent
    assert f_of({120: 16383, 200: 1}, 16384) == {120: 4095, 200: 1}
    # ties: the smallest exponent takes the adjustment (floor(8 * 512 / 3) = 1365 three times)
    assert f_of({120: 512, 121: 512, 122: 512}, 1536) == {120: 1366, 121: 1365, 122: 1365}
    assert f_of({120: 512, 121: 513, 122: 511}, 1536) == {120: 1365, 121: 1369, 122: 1362}
    # 200 singletons each raised to 1 push the sum past 4096 by more than the largest frequency
    counts = {e: 1 for e in range(200)}
    counts.update({200 + i: (16384 - 200) // 56 + (1 if i < (16384 - 200) % 56 else 0) for i in range(56)})
    assert sum(counts.values()) == 16384
    assert f_of(counts, 16384) is None


def test_rans_coder_closed_forms() -> None:
    """Two exponents of frequency 2048 cost exactly one bit each: every state doubles per symbol
    (plus its symbol's cumulative frequency) and emits 16 bits each time it reaches 2^31."""

    n = 16384
    e = np.where(np.random.default_rng(4).random(n) < 0.5, 120, 121)
    f = np.zeros(256, np.int64)
    f[120] = f[121] = 2048
    stream, states = wm.rans_encode(e, f)
    # per lane: 256 symbols from 2^16 = 1 + 256 bits of state growth, 16 per word
    assert stream.size == wm.LANES * (256 // 16)
    assert ((states >= wm.STATE_LOW) & (states < 1 << 17)).all()
    assert (wm.rans_decode(stream, states, f, n) == e).all()
    # the same symbols one lane at a time, by hand: x -> 2 (x - x % 2048) + x % 2048 + cum
    lane = e[::64]  # state 0 codes words 0, 64, 128, ...
    x, words = wm.STATE_LOW, []
    for s in lane[::-1]:
        if x >= 2048 << 20:
            words.append(x & 0xFFFF)
            x >>= 16
        x = (x // 2048 << 12) + x % 2048 + (0 if s == 120 else 2048)
    assert x == states[0]
    # lane 0's words come first in each round that emits: rounds j = 15, 31, ... hold one word
    # per lane, so lane 0's k-th word is the stream's word 64 k (in ascending rounds)
    assert [int(w) for w in stream[::64]] == words[::-1]


def test_entropy_bound() -> None:
    """A tile codes its exponents within 1 % of their empirical entropy (plus the table and the
    states)."""

    rng = np.random.default_rng(5)
    e = np.clip(np.round(rng.normal(124, 1.3, 16384)), 110, 140).astype(np.int64)
    counts = np.bincount(e, minlength=256)
    p = counts[counts > 0] / e.size
    h = float(-(p * np.log2(p)).sum())
    f = wm.normalize(counts, e.size)
    stream, _ = wm.rans_encode(e, f)
    bits = 16 * stream.size + 64 * 16  # each final state holds about 16 more bits
    assert bits < 1.01 * h * e.size + 64 * 16


def test_planted_mistakes_are_caught() -> None:
    """A flipped sign byte, a damaged stream word and two swapped frequencies each fail the
    round trip on ordinary activations (so the round-trip checks above pin the format)."""

    raw = _bf16_bytes(torch.randn(4 * 512, generator=torch.Generator().manual_seed(2)))
    stream, _ = wm.encode(raw)
    off, mode, nsym, nwords = _tile_head(stream, 0)
    assert mode == wm.MODE_RANS and nsym > 2 and nwords > 0
    n = 4 * 512
    s = bytearray(stream)
    s[off + wm.TILE_HEADER] ^= 0x80  # word 0's sign
    assert wm.decode(bytes(s), len(raw)) != raw
    s = bytearray(stream)
    st = off + wm.TILE_HEADER + n + (4 * nsym + 15) // 16 * 16 + 4 * wm.LANES
    s[st] ^= 0x01  # lowest bit of the first stream word
    assert wm.decode(bytes(s), len(raw)) != raw
    s = bytearray(stream)
    tab = np.frombuffer(stream[off + 16 + n:off + 16 + n + 4 * nsym], "<u4").copy()
    i, k = int(np.argmax(tab >> 8)), int(np.argmin(tab >> 8))  # the most and least frequent
    fi, fk = tab[i] >> 8, tab[k] >> 8
    assert fi != fk
    tab[i] = (tab[i] & 0xFF) | (fk << 8)
    tab[k] = (tab[k] & 0xFF) | (fi << 8)
    s[off + 16 + n:off + 16 + n + 4 * nsym] = tab.astype("<u4").tobytes()
    assert wm.decode(bytes(s), len(raw)) != raw


def test_library_capacity_matches_the_model() -> None:
    from moss_offload import _native

    lib = _native.load()
    for n in [0, 1, 1024, 32 * 1024, 32 * 1024 + 1, 128 << 20, (1 << 31)]:
        assert lib.mo_wire_capacity(n) == wm.capacity(n), n
    assert wm.capacity(128 << 20) < 2.1 * (128 << 20)
    assert math.isclose(wm.max_coded(128 << 20) / (128 << 20), 1.0, rel_tol=1e-3)
