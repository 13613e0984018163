"""Numpy model of the engine's wire coding (format: moss-image_amd/csrc/mo_wire.h).

Test infrastructure: the GPU tests compare the kernels' coded streams with ``encode`` byte for
byte (on the bytes the format defines) and the CPU tests check the model's own round trip.

A segment is read as little-endian 16-bit words. Tiles of up to 32 blocks of 512 words are
coded one by one; the raw tail (raw bytes % 1024) is kept as is. A tile keeps each word's sign
and mantissa as one byte and codes the words' 8-bit exponent fields with interleaved rANS: 64
coder states, state l taking the tile's words 64 j + l (j = 0 .. words / 64 - 1), with a
frequency table of the tile's exponents normalised to 4096. A tile whose coding would not be
smaller than its raw words is stored raw.
"""

from __future__ import annotations

import numpy as np

BLOCK_VALS = 512
BLOCK_BYTES = 1024
TILE_BLOCKS = 32
HEADER = 16
TILE_HEADER = 16
LANES = 64
PROB_BITS = 12
PROB_SCALE = 1 << PROB_BITS
STATE_LOW = 1 << 16
MODE_RANS = 0
MODE_RAW = 1


def _align16(x: int) -> int:
    return (x + 15) & ~15


def tiles_of(raw_bytes: int) -> int:
    return (raw_bytes // BLOCK_BYTES + TILE_BLOCKS - 1) // TILE_BLOCKS


def tile_words(raw_bytes: int, tile: int) -> int:
    blocks = raw_bytes // BLOCK_BYTES
    return BLOCK_VALS * min(TILE_BLOCKS, blocks - tile * TILE_BLOCKS)


def data_start(raw_bytes: int) -> int:
    return _align16(HEADER + 4 * tiles_of(raw_bytes))


def tiles_start(raw_bytes: int) -> int:
    return _align16(data_start(raw_bytes) + raw_bytes % BLOCK_BYTES)


def raw_tile_size(n: int) -> int:
    return TILE_HEADER + 2 * n


def rans_tile_size(n: int, nsym: int, nwords: int) -> int:
    return TILE_HEADER + n + _align16(4 * nsym) + 4 * LANES + _align16(2 * nwords)


def max_coded(raw_bytes: int) -> int:
    """The largest coded stream: every tile raw."""

    blocks = raw_bytes // BLOCK_BYTES
    return tiles_start(raw_bytes) + TILE_HEADER * tiles_of(raw_bytes) + blocks * BLOCK_BYTES


# The coder's working space after the largest stream, per tile: a 16-byte record (mode | nsym << 8,
# stream words, coded size), the frequency table (256 u32), the final states (64 u32) and room
# for the largest rANS stream (one 16-bit word per exponent).
SCRATCH_RECORD = 16
SCRATCH_TABLE = 4 * 256
SCRATCH_STATES = 4 * LANES
SCRATCH_STREAM = 2 * BLOCK_VALS * TILE_BLOCKS
SCRATCH_TILE = SCRATCH_RECORD + SCRATCH_TABLE + SCRATCH_STATES + SCRATCH_STREAM


def scratch_offset(raw_bytes: int) -> int:
    return _align16(max_coded(raw_bytes))


def capacity(raw_bytes: int) -> int:
    """The wire buffer the coder needs: the largest stream, then its working space."""

    return scratch_offset(raw_bytes) + SCRATCH_TILE * tiles_of(raw_bytes)


def normalize(counts: np.ndarray, n: int) -> np.ndarray | None:
    """Frequencies summing to 4096 for the exponents of a tile of n words (counts: 256 bins):
    floor(c * 4096 / n), at least 1 for every exponent present, and the difference to 4096 given
    to the most frequent exponent (the smallest one on ties). None when that would leave it
    below 1 (the tile is then stored raw)."""

    c = counts.astype(np.int64)
    f = np.where(c > 0, np.maximum(1, (c * PROB_SCALE) // n), 0)
    m = int(np.argmax(c))  # first maximum: the smallest exponent among the most frequent
    f[m] += PROB_SCALE - int(f.sum())
    if f[m] < 1:
        return None
    return f


def rans_encode(e: np.ndarray, f: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(stream of 16-bit words, 64 final states) of one tile's exponents ``e`` (n words, n a
    multiple of 512) under frequencies ``f``. State l codes e[64 j + l], j = J-1 .. 0; before
    coding a symbol of frequency q it emits its low 16 bits when x >= q << 20. The words one
    round emits are stored in lane order, and rounds in ascending j, which is the order the
    decoder reads them."""

    n = e.size
    J = n // LANES
    cum = np.concatenate([[0], np.cumsum(f)[:-1]]).astype(np.uint64)
    f64 = f.astype(np.uint64)
    sym = e.reshape(J, LANES).T.astype(np.int64)  # [lane, round]
    x = np.full(LANES, STATE_LOW, dtype=np.uint64)
    rounds = []
    for j in range(J - 1, -1, -1):
        s = sym[:, j]
        q, c = f64[s], cum[s]
        emit = x >= (q << np.uint64(20))
        rounds.append((x & np.uint64(0xFFFF))[emit].astype(np.uint16))
        x = np.where(emit, x >> np.uint64(16), x)
        x = ((x // q) << np.uint64(PROB_BITS)) + (x % q) + c
    stream = np.concatenate(rounds[::-1]) if rounds else np.zeros(0, np.uint16)
    return stream.astype(np.uint16), x.astype(np.uint32)


def rans_decode(stream: np.ndarray, states: np.ndarray, f: np.ndarray, n: int) -> np.ndarray:
    J = n // LANES
    cum = np.concatenate([[0], np.cumsum(f)[:-1]]).astype(np.int64)
    lut = np.repeat(np.arange(256), f)  # slot -> symbol
    x = states.astype(np.uint64)
    out = np.zeros((LANES, J), dtype=np.int64)
    ptr = 0
    for j in range(J):
        slot = (x & np.uint64(PROB_SCALE - 1)).astype(np.int64)
        s = lut[slot]
        out[:, j] = s
        x = f[s].astype(np.uint64) * (x >> np.uint64(PROB_BITS)) + (slot - cum[s]).astype(np.uint64)
        need = x < np.uint64(STATE_LOW)
        k = int(need.sum())
        words = np.zeros(k, np.uint64)  # a damaged stream may run short: zeros, as the kernel reads
        got = stream[ptr:ptr + k]
        words[:got.size] = got
        ptr += k
        x[need] = (x[need] << np.uint64(16)) | words
    return out.T.reshape(n)  # word 64 j + l from state l, round j


def encode_tile(words: np.ndarray) -> tuple[bytes, dict]:
    """The coded bytes of one tile (16-bit words, a multiple of 512) and what was chosen."""

    n = words.size
    expo = ((words >> 7) & 0xFF).astype(np.int64)
    f = normalize(np.bincount(expo, minlength=256), n)
    raw = np.array([MODE_RAW, 0, 0, 0], "<u4").tobytes() + words.astype("<u2").tobytes()
    if f is None:
        return raw, {"mode": MODE_RAW}
    stream, states = rans_encode(expo, f)
    present = np.flatnonzero(f)
    nsym, nwords = present.size, stream.size
    if rans_tile_size(n, nsym, nwords) >= raw_tile_size(n):
        return raw, {"mode": MODE_RAW}
    sm = (((words >> 8) & 0x80) | (words & 0x7F)).astype(np.uint8)
    table = (present | (f[present] << 8)).astype("<u4").tobytes()
    body = (np.array([MODE_RANS | (nsym << 8), nwords, 0, 0], "<u4").tobytes() + sm.tobytes() + table
            + bytes(_align16(4 * nsym) - 4 * nsym) + states.astype("<u4").tobytes() + stream.astype("<u2").tobytes()
            + bytes(_align16(2 * nwords) - 2 * nwords))
    assert len(body) == rans_tile_size(n, nsym, nwords)
    return body, {"mode": MODE_RANS, "nsym": nsym, "nwords": nwords}


def decode_tile(s: np.ndarray, o: int, n: int) -> np.ndarray:
    head = s[o:o + TILE_HEADER].view("<u4")
    mode, nsym, nwords = int(head[0]) & 3, (int(head[0]) >> 8) & 0x1FF, int(head[1])
    if mode == MODE_RAW:
        return s[o + TILE_HEADER:o + TILE_HEADER + 2 * n].view("<u2").astype(np.uint32)
    p = o + TILE_HEADER
    sm = s[p:p + n].astype(np.uint32)
    p += n
    table = s[p:p + 4 * nsym].view("<u4").astype(np.int64)
    p += _align16(4 * nsym)
    states = s[p:p + 4 * LANES].view("<u4")
    p += 4 * LANES
    stream = s[p:p + 2 * nwords].view("<u2")
    f = np.zeros(256, np.int64)
    f[table & 0xFF] = table >> 8
    e = rans_decode(stream, states, f, n).astype(np.uint32)
    return ((sm & 0x80) << 8) | (e << 7) | (sm & 0x7F)


def encode(raw: bytes | np.ndarray) -> tuple[bytes, np.ndarray]:
    """The coded stream of ``raw`` and a mask of the bytes the format defines (padding between
    the table, the tail and the tiles is left undefined by the kernels)."""

    buf = np.frombuffer(bytes(raw), dtype=np.uint8)
    raw_bytes = buf.size
    nblocks = raw_bytes // BLOCK_BYTES
    ntiles = tiles_of(raw_bytes)
    words = buf[: nblocks * BLOCK_BYTES].view("<u2").astype(np.uint32)
    pieces = []
    for t in range(ntiles):
        n = tile_words(raw_bytes, t)
        pieces.append(encode_tile(words[t * TILE_BLOCKS * BLOCK_VALS:t * TILE_BLOCKS * BLOCK_VALS + n])[0])
    sizes = [len(p) for p in pieces]
    start = tiles_start(raw_bytes)
    offsets = np.cumsum([0] + sizes[:-1], dtype=np.int64) + start if ntiles else np.zeros(0, np.int64)
    total = start + sum(sizes)
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
        out[o:o + sizes[t]] = np.frombuffer(pieces[t], np.uint8)
        defined[o:o + sizes[t]] = True
    return out.tobytes(), defined


def decode(stream: bytes, raw_bytes: int) -> bytes:
    """Raw bytes from a coded stream (the inverse of ``encode``)."""

    s = np.frombuffer(bytes(stream), dtype=np.uint8)
    nblocks = raw_bytes // BLOCK_BYTES
    ntiles = tiles_of(raw_bytes)
    out = np.zeros(raw_bytes, dtype=np.uint8)
    offsets = s[HEADER:HEADER + 4 * ntiles].view("<u4")
    words = np.zeros(nblocks * BLOCK_VALS, dtype=np.uint32)
    for t in range(ntiles):
        n = tile_words(raw_bytes, t)
        first = t * TILE_BLOCKS * BLOCK_VALS
        words[first:first + n] = decode_tile(s, int(offsets[t]), n)
    out[: nblocks * BLOCK_BYTES] = words.astype("<u2").view(np.uint8)
    ds = data_start(raw_bytes)
    out[nblocks * BLOCK_BYTES:] = s[ds:ds + raw_bytes % BLOCK_BYTES]
    return out.tobytes()
