"""Numpy model of the engine's wire coding (format: moss-image_amd/csrc/mo_wire.h).

Test infrastructure: the GPU tests compare the kernels' coded streams with ``encode`` byte for
byte (on the bytes the format defines) and the CPU tests check the model's own round trip.
A segment is read as little-endian 16-bit words; each 512-word block keeps a sign-mantissa
byte per word and codes the 8-bit exponent fields at width 0 (all equal), 1-5 (a k-bit code
per word relative to a base, with 8-bit escapes for exponents outside the window) or 8 (the
exponents as they are), whichever codes smallest. Tiles of 32 blocks sit at offsets listed
after a 16-byte header; the raw tail (raw bytes % 1024) is kept as is.
"""

from __future__ import annotations

import numpy as np

BLOCK_VALS = 512
BLOCK_BYTES = 1024
TILE_BLOCKS = 32
HEADER = 16
TILE_HEADER = 4 * TILE_BLOCKS
BINS = 32


def _align16(x: int) -> int:
    return (x + 15) & ~15


def tiles_of(raw_bytes: int) -> int:
    return (raw_bytes // BLOCK_BYTES + TILE_BLOCKS - 1) // TILE_BLOCKS


def data_start(raw_bytes: int) -> int:
    return _align16(HEADER + 4 * tiles_of(raw_bytes))


def tiles_start(raw_bytes: int) -> int:
    return _align16(data_start(raw_bytes) + raw_bytes % BLOCK_BYTES)


def block_coded(width: int, escapes: int) -> int:
    return BLOCK_VALS + 64 * width + _align16(escapes)


def max_coded(raw_bytes: int) -> int:
    return tiles_start(raw_bytes) + tiles_of(raw_bytes) * (TILE_HEADER + TILE_BLOCKS * block_coded(8, 0))


def capacity(raw_bytes: int) -> int:
    """The wire buffer the coder needs: the largest stream, then each block's header (u32) as
    working space."""

    return _align16(max_coded(raw_bytes)) + 4 * (raw_bytes // BLOCK_BYTES)


def choose(e: np.ndarray) -> tuple[int, int, int]:
    """(width, base, escapes) of one block's 512 exponents: the smallest coded size among width
    8 and widths 1-5 over windows of exponent offsets s.. from the block minimum (2^k values
    when every exponent fits, else 2^k - 1 values plus escapes), ties to the smaller width,
    then the smaller s; width 0 when all exponents are equal."""

    lo, hi = int(e.min()), int(e.max())
    if lo == hi:
        return 0, lo, 0
    d = np.minimum(e.astype(np.int64) - lo, BINS - 1)
    hist = np.bincount(d, minlength=BINS)
    p = np.concatenate([[0], np.cumsum(hist)])  # p[i]: words in bins 0..i-1
    best = (block_coded(8, 0), 8, 0, 0)
    for k in range(1, 6):
        w = 1 << k
        for s_ in range(BINS):
            if s_ + w <= BINS - 1 and p[s_ + w] - p[s_] == BLOCK_VALS:
                esc = 0
            elif s_ + w - 1 <= BINS - 1:
                esc = BLOCK_VALS - int(p[s_ + w - 1] - p[s_])
            else:
                continue
            cand = (block_coded(k, esc), k, s_, esc)
            if cand[:3] < best[:3]:
                best = cand
    _, k, s_, esc = best
    if k == 8:
        return 8, 0, 0
    return k, lo + s_, esc


def encode(raw: bytes | np.ndarray) -> tuple[bytes, np.ndarray]:
    """The coded stream of ``raw`` and a mask of the bytes the format defines (padding between
    the table, the tail and the tiles is left undefined by the kernels)."""

    buf = np.frombuffer(bytes(raw), dtype=np.uint8)
    raw_bytes = buf.size
    nblocks = raw_bytes // BLOCK_BYTES
    ntiles = tiles_of(raw_bytes)
    words = buf[: nblocks * BLOCK_BYTES].view("<u2").reshape(nblocks, BLOCK_VALS).astype(np.uint32)
    expo = (words >> 7) & 0xFF
    sm = (((words >> 8) & 0x80) | (words & 0x7F)).astype(np.uint8)

    pieces: list[bytes] = []
    tile_sizes = []
    for t in range(ntiles):
        first, last = t * TILE_BLOCKS, min(t * TILE_BLOCKS + TILE_BLOCKS, nblocks)
        headers = np.zeros(TILE_BLOCKS, dtype="<u4")
        body = []
        for j, b in enumerate(range(first, last)):
            e = expo[b]
            k, base, esc = choose(e)
            headers[j] = base | (k << 8) | (esc << 12)
            body.append(sm[b].tobytes())
            if k:
                if k == 8:
                    codes = e.astype(np.uint64)
                    escaped = np.zeros(BLOCK_VALS, bool)
                else:
                    limit = (1 << k) - 1 if esc else (1 << k)
                    dd = e.astype(np.int64) - base
                    escaped = (dd < 0) | (dd >= limit)
                    codes = np.where(escaped, (1 << k) - 1, dd).astype(np.uint64)
                acc = np.zeros(64, dtype=np.uint64)
                c = codes.reshape(64, 8)
                for i in range(8):
                    acc |= c[:, i] << np.uint64(i * k)
                body.append(acc.astype("<u8").view(np.uint8).reshape(64, 8)[:, :k].tobytes())
                escs = e[escaped].astype(np.uint8).tobytes()
                assert len(escs) == esc
                body.append(escs + bytes(_align16(esc) - esc))
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
        headers = s[o:o + TILE_HEADER].view("<u4")
        p = o + TILE_HEADER
        for j, b in enumerate(range(t * TILE_BLOCKS, min(t * TILE_BLOCKS + TILE_BLOCKS, nblocks))):
            h = int(headers[j])
            base, k, esc = h & 0xFF, (h >> 8) & 0xF, h >> 12
            sm = s[p:p + BLOCK_VALS].astype(np.uint32)
            p += BLOCK_VALS
            if k == 0:
                e = np.full(BLOCK_VALS, base, np.uint32)
            else:
                packed = np.zeros((64, 8), dtype=np.uint8)
                packed[:, :k] = s[p:p + 64 * k].reshape(64, k)
                acc = packed.view("<u8").reshape(64)
                codes = np.stack([(acc >> np.uint64(i * k)) & np.uint64((1 << k) - 1) for i in range(8)], axis=1)
                codes = codes.reshape(BLOCK_VALS).astype(np.uint32)
                p += 64 * k
                if k == 8:
                    e = codes
                else:
                    e = (codes + base) & 0xFF
                    if esc:
                        escaped = codes == (1 << k) - 1
                        e[escaped] = s[p:p + int(escaped.sum())]
            p += _align16(esc)
            words[b] = ((sm & 0x80) << 8) | (e << 7) | (sm & 0x7F)
    out[: nblocks * BLOCK_BYTES] = words.astype("<u2").view(np.uint8).reshape(-1)
    ds = data_start(raw_bytes)
    out[nblocks * BLOCK_BYTES:] = s[ds:ds + raw_bytes % BLOCK_BYTES]
    return out.tobytes()
