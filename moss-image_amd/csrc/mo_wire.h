// Wire format of a coded staging segment: lossless coding of the exponent fields of 16-bit
// words, shared by the device kernels (mo_device.hip) and the host (mo_engine.cpp,
// mo_launch.cpp).
//
// A segment's payload is a byte string whose pieces start 256-byte aligned, so the bfloat16
// values it mostly holds sit on the 2-byte grid. The coder reads it as 16-bit words w =
// s(1) e(8) m(7): it keeps each word's sign and mantissa as one byte, and codes the 8-bit
// exponent field per 512-word block in one of three ways, whichever is smallest:
//   width 0       every exponent of the block equals `base`;
//   width k 1..7  (the coder uses 1..5) a k-bit code per word: code c < 2^k - 1 (or any c when the block has no
//                 escapes) stands for exponent base + c; code 2^k - 1 marks an escape, whose
//                 8-bit exponent follows in the block's escape bytes, in word order;
//   width 8       the exponent bytes as they are.
// Words that are not bfloat16 (float32 low halves, integers, random bits) take width 8 and
// cost 1/256 more than raw. Decoding restores every word bit for bit, NaN payloads included.
//
// Layout (all offsets in bytes from the start of the coded stream, little-endian):
//   [0, 16)            header: u64 total (coded bytes, header included), u32 raw bytes,
//                      u32 tiles
//   [16, 16 + 4 T)     u32 offset of each tile's data
//   data_start         the raw tail (raw bytes % kWireBlockBytes bytes, copied as is)
//   tiles_start        the tiles, each 16-byte aligned:
//                        kWireTileBlocks u32 block headers (base | width << 8 | escapes << 12;
//                        zero for blocks past the end), then each block's data:
//                          kWireBlockVals sign-mantissa bytes (byte i: word i's bit 15 as
//                          bit 7, its bits 0-6 as bits 0-6),
//                          64 * width code bytes: lane l of the coding wave packs words
//                          8l..8l+7 into `width` bytes at l * width, word 8l+k in bits
//                          [k * width, (k + 1) * width) of that little-endian field,
//                          the escapes' exponent bytes, zero-padded to a multiple of 16.
// A tile holds 32 blocks of 512 words (1 KiB raw each). The wire buffer a coder writes into
// also holds, after the largest stream, its working space: each block's header as the sizing
// pass chose it (wire_capacity covers both).
// Plain constexpr code (callable from device code too), no HIP headers, like mo_kdesc.h.
#pragma once

#include <stdint.h>

namespace mo {

constexpr uint32_t kWireBlockVals = 512;                              // words per block (one wave)
constexpr uint32_t kWireBlockBytes = 2 * kWireBlockVals;              // raw bytes per block
constexpr uint32_t kWireTileBlocks = 32;                              // blocks per tile (one workgroup)
constexpr uint32_t kWireTileRaw = kWireBlockBytes * kWireTileBlocks;  // 32 KiB raw per tile
constexpr uint32_t kWireHeader = 16;
constexpr uint32_t kWireTileHeader = 4 * kWireTileBlocks;
constexpr uint32_t kWireScanThreads = 1024;  // the one workgroup of the offset scan
constexpr uint32_t kWireBins = 32;           // exponent offsets 0..30 from the block minimum; 31 = farther

constexpr uint64_t wire_align16(uint64_t x) { return (x + 15) & ~uint64_t(15); }
constexpr uint64_t wire_blocks(uint64_t raw) { return raw / kWireBlockBytes; }
constexpr uint64_t wire_tiles(uint64_t raw) {
  return (wire_blocks(raw) + kWireTileBlocks - 1) / kWireTileBlocks;
}
constexpr uint64_t wire_data_start(uint64_t raw) { return wire_align16(kWireHeader + 4 * wire_tiles(raw)); }
constexpr uint64_t wire_tiles_start(uint64_t raw) {
  return wire_align16(wire_data_start(raw) + raw % kWireBlockBytes);
}
// Coded bytes of one block: sign-mantissa bytes, codes, padded escape bytes.
constexpr uint32_t wire_block_coded(uint32_t width, uint32_t escapes) {
  return kWireBlockVals + 64 * width + (uint32_t)wire_align16(escapes);
}
// Largest coded size of `raw` bytes (every block at width 8, which the coder never exceeds).
constexpr uint64_t wire_max_coded(uint64_t raw) {
  return wire_tiles_start(raw) + wire_tiles(raw) * (kWireTileHeader + (uint64_t)kWireTileBlocks * wire_block_coded(8, 0));
}
// The coder's working space after the largest stream: each block's header (u32), chosen once
// by the sizing pass and read by the coding pass.
constexpr uint64_t wire_scratch_offset(uint64_t raw) { return wire_align16(wire_max_coded(raw)); }
// The wire buffer to provide for coding `raw` bytes: the largest stream plus the working space.
constexpr uint64_t wire_capacity(uint64_t raw) { return wire_scratch_offset(raw) + 4 * wire_blocks(raw); }

}  // namespace mo
