// Wire format of a coded staging segment: lossless coding of the exponent fields of 16-bit
// words, shared by the device kernels (mo_device.hip) and the host (mo_engine.cpp,
// mo_launch.cpp).
//
// A segment's payload is a byte string whose pieces start 256-byte aligned, so the bfloat16
// values it mostly holds sit on the 2-byte grid. The coder reads it as 16-bit words w =
// s(1) e(8) m(7), in tiles of up to 32 blocks of 512 words (32 KiB raw). A tile keeps each
// word's sign and mantissa as one byte and codes the 8-bit exponent fields with interleaved rANS
// (range asymmetric numeral systems): 64 coder states, state l taking the tile's words
// l*J .. l*J + J - 1 (J = the tile's words / 64), 32-bit states kept in [2^16, 2^32), 16-bit
// renormalisation words, and the tile's exponent frequencies normalised to 4096:
//   f(e) = floor(count(e) * 4096 / words) for every exponent e present, at least 1, and the
//   difference of their sum to 4096 added to the most frequent exponent (the smallest on ties).
// Coding runs over j = J-1 .. 0: state x with symbol e (frequency f, cumulative frequency c)
// first emits x & 0xffff and shifts x right by 16 when x >= f << 20, then becomes
// (x / f) << 12 | (x % f) + c. The words one round j emits are stored in lane order, and the
// rounds in ascending j; the decoder runs j = 0 .. J-1: e = the symbol whose slot range holds
// x & 4095, x = f * (x >> 12) + (x & 4095) - c, then x = x << 16 | next word while x < 2^16.
// A tile whose coding would not be smaller than its raw words is stored raw; so is a tile whose
// normalisation would leave the most frequent exponent below 1 (not seen on real data).
//
// Layout (all offsets in bytes from the start of the coded stream, little-endian):
//   [0, 16)            header: u64 total (coded bytes, header included), u32 raw bytes,
//                      u32 tiles
//   [16, 16 + 4 T)     u32 offset of each tile's data
//   data_start         the raw tail (raw bytes % kWireBlockBytes bytes, copied as is)
//   tiles_start        the tiles, each 16-byte aligned. A tile of n words:
//                        u32 mode | nsym << 8, u32 stream words, u32 0, u32 0;
//                        mode 1 (raw): the n words as they are;
//                        mode 0 (rANS): n sign-mantissa bytes (byte i: word i's bit 15 as
//                        bit 7, its bits 0-6 as bits 0-6), the frequency table (nsym u32
//                        exponent | frequency << 8, ascending exponents; cumulative frequencies
//                        follow in that order) zero-padded to 16 bytes, the 64 final states
//                        (u32), the stream's 16-bit words zero-padded to 16 bytes.
// The wire buffer a coder writes into also holds, after the largest stream, its working space:
// per tile a 16-byte record (mode | nsym << 8, stream words, first stream word, coded size),
// the frequency table, the final states and room for the largest stream, which the coding pass
// fills from the end (wire_capacity covers both).
// Plain constexpr code (callable from device code too), no HIP headers, like mo_kdesc.h.
#pragma once

#include <stdint.h>

namespace mo {

constexpr uint32_t kWireBlockVals = 512;                              // words per block
constexpr uint32_t kWireBlockBytes = 2 * kWireBlockVals;              // raw bytes per block
constexpr uint32_t kWireTileBlocks = 32;                              // blocks per tile (one coding wave)
constexpr uint32_t kWireTileVals = kWireBlockVals * kWireTileBlocks;  // 16 384 words per tile
constexpr uint32_t kWireTileRaw = kWireBlockBytes * kWireTileBlocks;  // 32 KiB raw per tile
constexpr uint32_t kWireHeader = 16;
constexpr uint32_t kWireTileHeader = 16;
constexpr uint32_t kWireLanes = 64;           // interleaved rANS states per tile
constexpr uint32_t kWireProbBits = 12;        // frequencies sum to 4096
constexpr uint32_t kWireStateLow = 1u << 16;  // states stay in [2^16, 2^32)
constexpr uint32_t kWireModeRans = 0, kWireModeRaw = 1;
constexpr uint32_t kWireTilesPerGroup = 4;   // one wave per tile, four waves a workgroup
constexpr uint32_t kWireScanThreads = 1024;  // the one workgroup of the offset scan
// Working space per tile: record, table (256 u32), states, stream (one word per exponent).
constexpr uint32_t kWireScratchTable = 16;
constexpr uint32_t kWireScratchStates = kWireScratchTable + 4 * 256;
constexpr uint32_t kWireScratchStream = kWireScratchStates + 4 * kWireLanes;
constexpr uint32_t kWireScratchTile = kWireScratchStream + 2 * kWireTileVals;

constexpr uint64_t wire_align16(uint64_t x) { return (x + 15) & ~uint64_t(15); }
constexpr uint64_t wire_blocks(uint64_t raw) { return raw / kWireBlockBytes; }
constexpr uint64_t wire_tiles(uint64_t raw) {
  return (wire_blocks(raw) + kWireTileBlocks - 1) / kWireTileBlocks;
}
// Words of tile t (a multiple of 512).
constexpr uint32_t wire_tile_words(uint64_t raw, uint64_t t) {
  return kWireBlockVals *
         (uint32_t)(wire_blocks(raw) - t * kWireTileBlocks < kWireTileBlocks ? wire_blocks(raw) - t * kWireTileBlocks
                                                                              : kWireTileBlocks);
}
constexpr uint64_t wire_data_start(uint64_t raw) { return wire_align16(kWireHeader + 4 * wire_tiles(raw)); }
constexpr uint64_t wire_tiles_start(uint64_t raw) {
  return wire_align16(wire_data_start(raw) + raw % kWireBlockBytes);
}
constexpr uint32_t wire_raw_tile(uint32_t n) { return kWireTileHeader + 2 * n; }
constexpr uint32_t wire_rans_tile(uint32_t n, uint32_t nsym, uint32_t nwords) {
  return kWireTileHeader + n + (uint32_t)wire_align16(4 * nsym) + 4 * kWireLanes + (uint32_t)wire_align16(2 * nwords);
}
// Largest coded size of `raw` bytes (every tile raw, which the coder never exceeds).
constexpr uint64_t wire_max_coded(uint64_t raw) {
  return wire_tiles_start(raw) + kWireTileHeader * wire_tiles(raw) + wire_blocks(raw) * kWireBlockBytes;
}
constexpr uint64_t wire_scratch_offset(uint64_t raw) { return wire_align16(wire_max_coded(raw)); }
// The wire buffer to provide for coding `raw` bytes: the largest stream plus the working space.
constexpr uint64_t wire_capacity(uint64_t raw) { return wire_scratch_offset(raw) + kWireScratchTile * wire_tiles(raw); }

}  // namespace mo
