// Wire format of a coded staging segment: lossless exponent-plane coding of 16-bit words,
// shared by the device kernels (mo_device.hip) and the host (mo_engine.cpp, mo_launch.cpp).
//
// A segment's payload is a byte string whose pieces start 16-byte aligned, so the bfloat16
// values it mostly holds sit on the 2-byte grid. The coder reads it as 16-bit words w =
// s(1) e(8) m(7): it keeps each word's sign and mantissa as one byte, and replaces the 8-bit
// exponent field by its offset from the smallest exponent of the word's block, in as few bits
// as the block's exponent range needs (0 to 8). Words that are not bfloat16 (float32 low
// halves, integers) code at width 8 and cost 1/512 more than raw. Decoding restores every
// word bit for bit, NaN payloads included.
//
// Layout (all offsets in bytes from the start of the coded stream, little-endian):
//   [0, 16)            header: u64 total (coded bytes, header included), u32 raw bytes,
//                      u32 tiles
//   [16, 16 + 4 T)     u32 offset of each tile's data
//   data_start         the raw tail (raw bytes % kWireBlockBytes bytes, copied as is)
//   tiles_start        the tiles, each 16-byte aligned:
//                        kWireTileBlocks u16 block headers (width << 8 | base exponent;
//                        zero for blocks past the end), then each block's data:
//                          kWireBlockVals sign-mantissa bytes (byte i: word i's bit 15 as
//                          bit 7, its bits 0-6 as bits 0-6),
//                          kWireBlockVals exponent offsets of `width` bits, 64 * width bytes:
//                          lane l of the coding wave packs words 8l..8l+7 into `width` bytes
//                          at l * width, word 8l+k in bits [k * width, (k + 1) * width) of
//                          that little-endian field.
// A block of 512 words (1 KiB raw) codes to 512 + 64 * width bytes; a tile holds 32 blocks.
// Plain constexpr code (callable from device code too), no HIP headers, like mo_kdesc.h.
#pragma once

#include <stdint.h>

namespace mo {

constexpr uint32_t kWireBlockVals = 512;                              // words per block (one wave)
constexpr uint32_t kWireBlockBytes = 2 * kWireBlockVals;              // raw bytes per block
constexpr uint32_t kWireTileBlocks = 32;                              // blocks per tile (one workgroup)
constexpr uint32_t kWireTileRaw = kWireBlockBytes * kWireTileBlocks;  // 32 KiB raw per tile
constexpr uint32_t kWireHeader = 16;
constexpr uint32_t kWireTileHeader = 2 * kWireTileBlocks;
constexpr uint32_t kWireScanThreads = 1024;  // the one workgroup of the offset scan

constexpr uint64_t wire_align16(uint64_t x) { return (x + 15) & ~uint64_t(15); }
constexpr uint64_t wire_blocks(uint64_t raw) { return raw / kWireBlockBytes; }
constexpr uint64_t wire_tiles(uint64_t raw) {
  return (wire_blocks(raw) + kWireTileBlocks - 1) / kWireTileBlocks;
}
constexpr uint64_t wire_data_start(uint64_t raw) { return wire_align16(kWireHeader + 4 * wire_tiles(raw)); }
constexpr uint64_t wire_tiles_start(uint64_t raw) {
  return wire_align16(wire_data_start(raw) + raw % kWireBlockBytes);
}
constexpr uint32_t wire_block_coded(uint32_t width) { return kWireBlockVals + 64 * width; }
// Largest coded size of `raw` bytes (every block at width 8).
constexpr uint64_t wire_capacity(uint64_t raw) {
  return wire_tiles_start(raw) + wire_tiles(raw) * (kWireTileHeader + (uint64_t)kWireTileBlocks * wire_block_coded(8));
}

}  // namespace mo
