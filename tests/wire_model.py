"""Numpy model of the engine's wire coding (format: moss-image_amd/csrc/mo_wire.h).

Test infrastructure: the GPU tests compare the kernels' coded streams with ``encode`` byte for
byte (on the bytes the format defines) and the CPU tests check the model's own round trip.
A segment is read as little-endian 16-bit words; each 512-word block keeps a sign-mantissa
byte per word and codes the 8-bit exponent fields as offsets of ``width`` bits (0-8) from the
block's smallest exponent. Tiles of 32 blocks sit at offsets listed after a 16-byte header;
the raw tail (raw bytes % 1024) is kept as is.
"""

from __future__ import annotations

import numpy as np

BLOCK_VALS = 512
BLOCK_BYTES = 1024
TILE_BLOCKS = 32
HEADER = 16
TILE_HEADER = 2 * TILE_BLOCKS


def _align16(x: int) -> int:
    return (x + 15) & ~15


def tiles_of(raw_bytes: int) -> int:
    return (raw_bytes // BLOCK_BYTES + TILE_BLOCKS - 1) // TILE_BLOCKS


def data_start(raw_bytes: int) -> int:
    return _align16(HEADER + 4 * tiles_of(raw_bytes))


def tiles_start(raw_bytes: int) -> int:
    return _align16(data_start(raw_bytes) + raw_bytes % BLOCK_BYTES)


def block_coded(width: int) -> int:
    return BLOCK_VALS + 64 * width


def capacity(raw_bytes: int) -> int:
    return tiles_start(raw_bytes) + tiles_of(raw_bytes) * (TILE_HEADER + TILE_BLOCKS * block_coded(8))


def _widths(range_: np.ndarray) -> np.ndarray:
    r = range_.astype(np.int64)
    out = np.zeros_like(r)
    nz = r > 0
    out[nz] = np.floor(np.log2(r[nz])).astype(np.int64) + 1
    return out


def encode(raw: bytes | np.ndarray) -> tuple[bytes, np.ndarray]:
    """The coded stream of ``raw`` and a mask of the bytes the format defines (padding between
    the table, the tail and the tiles is left undefined by the kernels)."""

    buf = np.frombuffer(bytes(raw), dtype=np.uint8)
    raw_bytes = buf.size
    nblocks = raw_bytes // BLOCK_BYTES
    ntiles = tiles_of(raw_bytes)
    words = buf[: nblocks * BLOCK_BYTES].view("<u2").reshape(nblocks, BLOCK_VALS).astype(np.uint32)
    e = (words >> 7) & 0xFF
    lo = e.min(axis=1) if nblocks else np.zeros(0, np.uint32)
    hi = e.max(axis=1) if nblocks else np.zeros(0, np.uint32)
    width = _widths(hi - lo)
    sm = (((words >> 8) & 0x80) | (words & 0x7F)).astype(np.uint8)
    off = (e - lo[:, None]).astype(np.uint64)

    pieces: list[bytes] = []
    tile_sizes = []
    for t in range(ntiles):
        first, last = t * TILE_BLOCKS, min(t * TILE_BLOCKS + TILE_BLOCKS, nblocks)
        headers = np.zeros(TILE_BLOCKS, dtype="<u2")
        body = []
        for k, b in enumerate(range(first, last)):
            w = int(width[b])
            headers[k] = (w << 8) | int(lo[b])
            body.append(sm[b].tobytes())
            if w:
                o = off[b].reshape(64, 8)
                acc = np.zeros(64, dtype=np.uint64)
                for j in range(8):
                    acc |= o[:, j] << np.uint64(j * w)
                body.append(acc.astype("<u8").view(np.uint8).reshape(64, 8)[:, :w].tobytes())
        data = headers.tobytes() + b"".join(body)
        pieces.append(data)
        tile_sizes.append(len(data))

    start = tiles_start(raw_bytes)
    offsets = np.cumsum([0] + tile_sizes[:-1], dtype=np.int64) + start if ntiles else np.zeros(0, np.int64)
    total = start + sum(tile_sizes)
    out = np.zeros(total, dtype=np.uint8)
    defined = np.zeros(total, dtype=bool)
    header = np.array([total], dtype="<u8").tobytes() + np.array([raw_bytes, ntiles], dtype="<u4").tobytes()
    out[:HEADER] = np.frombuffer(header, np.uint8)
    defined[:HEADER] = True
    table = np.asarray(offsets, dtype="<u4").tobytes()
    out[HEADER:HEADER + len(table)] = np.frombuffer(table, np.uint8)
    defined[HEADER:HEADER + len(table)] = True
    ds, tail = data_start(raw_bytes), raw_bytes % BLOCK_BYTES
    out[ds:ds + tail] = buf[nblocks * BLOCK_BYTES:]
    defined[ds:ds + tail] = True
    for t in range(ntiles):
        o = int(offsets[t])
        out[o:o + tile_sizes[t]] = np.frombuffer(pieces[t], np.uint8)
        defined[o:o + tile_sizes[t]] = True
    return out.tobytes(), defined


def decode(stream: bytes, raw_bytes: int) -> bytes:
    """Raw bytes from a coded stream (the inverse of ``encode``)."""

    s = np.frombuffer(bytes(stream), dtype=np.uint8)
    nblocks = raw_bytes // BLOCK_BYTES
    ntiles = tiles_of(raw_bytes)
    out = np.zeros(raw_bytes, dtype=np.uint8)
    offsets = s[HEADER:HEADER + 4 * ntiles].view("<u4")
    words = np.zeros((nblocks, BLOCK_VALS), dtype=np.uint32)
    for t in range(ntiles):
        o = int(offsets[t])
        headers = s[o:o + TILE_HEADER].view("<u2")
        p = o + TILE_HEADER
        for k, b in enumerate(range(t * TILE_BLOCKS, min(t * TILE_BLOCKS + TILE_BLOCKS, nblocks))):
            w, lo = int(headers[k]) >> 8, int(headers[k]) & 0xFF
            sm = s[p:p + BLOCK_VALS].astype(np.uint32)
            p += BLOCK_VALS
            if w:
                packed = np.zeros((64, 8), dtype=np.uint8)
                packed[:, :w] = s[p:p + 64 * w].reshape(64, w)
                acc = packed.view("<u8").reshape(64)
                offs = np.stack([(acc >> np.uint64(j * w)) & np.uint64((1 << w) - 1) for j in range(8)], axis=1)
                offs = offs.reshape(BLOCK_VALS).astype(np.uint32)
                p += 64 * w
            else:
                offs = np.zeros(BLOCK_VALS, np.uint32)
            e = (offs + lo) & 0xFF
            words[b] = ((sm & 0x80) << 8) | (e << 7) | (sm & 0x7F)
    out[: nblocks * BLOCK_BYTES] = words.astype("<u2").view(np.uint8).reshape(-1)
    ds = data_start(raw_bytes)
    out[nblocks * BLOCK_BYTES:] = s[ds:ds + raw_bytes % BLOCK_BYTES]
    return out.tobytes()
