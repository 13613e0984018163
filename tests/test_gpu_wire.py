"""The wire-coding kernels through the C ABI (``mo_wire_encode`` / ``mo_wire_decode``).

Each case codes a device buffer, compares the coded stream byte for byte with the numpy model
(``tests/wire_model.py``) on every byte the format defines, checks the coded size the scan
kernel wrote to pinned host memory, decodes into a buffer with sentinel guard bytes on both
sides, and compares the result bitwise with the input. Inputs cover both tile modes (random
bits stay raw; one exponent, Gaussian activations, all exponent classes with NaN payloads,
infinities, signed zeros and subnormals, and exponents that change from one coder state's run
of words to the next are rANS-coded), partial tiles of 1 to 31 blocks and raw tails, and a
50 MiB Gaussian buffer.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import wire_model as wm
from moss_offload import _native

from gpu_util import requires_gpu

pytestmark = requires_gpu

DEV = torch.device("cuda", 0)


def _content(kind: str, nbytes: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    if kind == "random":
        return torch.randint(0, 256, (nbytes,), dtype=torch.uint8, generator=g)
    n = (nbytes + 1) // 2
    if kind == "gauss":
        v = torch.randn(n, generator=g).to(torch.bfloat16)
    elif kind == "flat":
        v = torch.full((n,), 3.25, dtype=torch.bfloat16)
    elif kind == "lanes":  # exponents that differ between 8-word lane groups (the coder's per-lane spans)
        blocks = (n + 511) // 512
        gen = np.random.default_rng(seed)
        e = np.repeat(120 + gen.integers(0, 4, (blocks, 64)), 8, axis=1)
        for b in range(blocks):
            lane = b // 4 % 64
            if b % 4 == 0:  # one lane holds the block's smallest exponent in all its words
                e[b, 8 * lane:8 * lane + 8] = 119
            elif b % 4 == 1:  # one lane below an otherwise constant block
                e[b] = 125
                e[b, 8 * lane:8 * lane + 8] = 124
            elif b % 4 == 2:  # one exponent per lane, 64 apart from first to last
                e[b] = np.repeat(90 + np.arange(64), 8)
            else:  # one lane of zeros in a block near 1.0
                e[b] = 127
                e[b, 8 * lane:8 * lane + 8] = 0
        sm = gen.integers(0, 1 << 16, e.shape) & 0x807F
        words = (sm | (e << 7)).reshape(-1)[:n]
        v = torch.from_numpy(words.astype(np.uint16).view(np.int16).copy()).view(torch.bfloat16)
    else:  # special: every exponent class, NaN payloads, infinities, zeros, subnormals
        words = torch.randint(0, 1 << 16, (n,), dtype=torch.int32, generator=g)
        words[::7] = 0x7F80 | (words[::7] & 0x807F)  # inf / NaN with random payloads
        words[1::11] = words[1::11] & 0x807F  # zeros and subnormals
        v = words.to(torch.int16).view(torch.bfloat16)
    return v.view(torch.uint8)[:nbytes].clone()


CASES = [
    ("random", 16), ("random", 1024), ("random", 1040), ("gauss", 32 * 1024), ("gauss", 32 * 1024 + 1024 + 16),
    ("flat", 64 * 1024), ("special", 3 * 32 * 1024 + 5 * 1024 + 496), ("gauss", (1 << 20) + 48),
    ("random", 40 * 1024 + 3), ("gauss", 0), ("lanes", 64 * 1024 * 4 + 2 * 1024), ("gauss", 3 * 1024 + 100),
    ("special", 31 * 1024),
]


@pytest.mark.parametrize("kind,nbytes", CASES)
def test_encode_matches_model_and_decodes_bitwise(kind, nbytes) -> None:
    lib = _native.load()
    stream = torch.cuda.current_stream(DEV).cuda_stream
    host_raw = _content(kind, nbytes, seed=nbytes)
    raw = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=DEV)
    raw[:nbytes].copy_(host_raw.to(DEV))
    cap = lib.mo_wire_capacity(nbytes)
    assert cap == wm.capacity(nbytes)
    wire = torch.full((cap,), 0xA5, dtype=torch.uint8, device=DEV)
    total = torch.zeros(1, dtype=torch.int64, pin_memory=True)
    _native.check("mo_wire_encode", lib.mo_wire_encode(raw.data_ptr(), nbytes, wire.data_ptr(), cap, total.data_ptr(),
                                                       stream))
    torch.cuda.synchronize()
    expected, defined = wm.encode(host_raw.numpy().tobytes())
    coded = int(total[0])
    assert coded == len(expected)
    got = wire[:coded].cpu().numpy()
    exp = np.frombuffer(expected, np.uint8)
    bad = np.nonzero((got != exp) & defined)[0]
    assert bad.size == 0, f"first differing coded byte at {bad[:8]}"

    guard = 64
    out = torch.full((nbytes + 2 * guard,), 0x3C, dtype=torch.uint8, device=DEV)
    _native.check("mo_wire_decode", lib.mo_wire_decode(wire.data_ptr(), coded, out[guard:].data_ptr(), nbytes, stream))
    torch.cuda.synchronize()
    res = out.cpu()
    assert torch.equal(res[guard:guard + nbytes], host_raw)
    assert bool((res[:guard] == 0x3C).all()) and bool((res[guard + nbytes:] == 0x3C).all())


def test_large_gaussian_buffer_round_trip_and_ratio() -> None:
    """50 MiB of Gaussian bfloat16 (an activation-like buffer): bitwise round trip, and a coded
    size of about 0.67 of the raw bytes (8 sign-mantissa bits and about 2.7 exponent bits a word)."""

    lib = _native.load()
    stream = torch.cuda.current_stream(DEV).cuda_stream
    n = 25 << 20
    g = torch.Generator(device=DEV).manual_seed(3)
    src = torch.randn(n, device=DEV, generator=g).to(torch.bfloat16)
    nbytes = 2 * n
    cap = lib.mo_wire_capacity(nbytes)
    wire = torch.empty(cap, dtype=torch.uint8, device=DEV)
    total = torch.zeros(1, dtype=torch.int64, pin_memory=True)
    _native.check("mo_wire_encode", lib.mo_wire_encode(src.data_ptr(), nbytes, wire.data_ptr(), cap, total.data_ptr(),
                                                       stream))
    out = torch.empty_like(src)
    torch.cuda.synchronize()
    coded = int(total[0])
    assert coded == int(wire[:8].cpu().view(torch.int64)[0])
    assert coded < 0.69 * nbytes
    _native.check("mo_wire_decode", lib.mo_wire_decode(wire.data_ptr(), coded, out.data_ptr(), nbytes, stream))
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), src.view(torch.int16))


def test_rejects_short_wire_buffer_and_misalignment() -> None:
    lib = _native.load()
    stream = torch.cuda.current_stream(DEV).cuda_stream
    raw = torch.zeros(4096, dtype=torch.uint8, device=DEV)
    wire = torch.zeros(lib.mo_wire_capacity(4096), dtype=torch.uint8, device=DEV)
    assert lib.mo_wire_encode(raw.data_ptr(), 4096, wire.data_ptr(), wire.numel() - 16, 0, stream) == _native.MO_E_INVALID
    assert lib.mo_wire_encode(raw.data_ptr() + 8, 4000, wire.data_ptr(), wire.numel(), 0, stream) == _native.MO_E_INVALID
    assert lib.mo_wire_decode(wire.data_ptr() + 4, 100, raw.data_ptr(), 4096, stream) == _native.MO_E_INVALID
