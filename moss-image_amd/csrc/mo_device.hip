// Pack / unpack kernels for gfx950 (MI355X), compiled to a standalone code object
// (hipcc --genco) that the host library embeds and loads with hipModuleLoadData.
//
// One launch moves up to kMaxDesc "pieces" (a byte range of one tensor's payload) between
// strided tensor views and a dense staging payload. The payload is in storage order, so the
// tensor side is walked in address order too; nothing is transposed. The work is pure data
// movement and HBM-bound: every path aims at 128-bit coalesced loads and stores.
//
//   CONTIG  the piece is one contiguous run and 16-byte aligned: kUnroll x 16 B in flight
//           per lane, no index arithmetic.
//   RUNS    contiguous runs whose length, start and strides are multiples of 16 B: each
//           16-byte chunk is located with fast division over the canonical dimensions.
//   ELEM    anything else (misaligned bases, odd run lengths, element-strided innermost
//           dimension): elements are gathered one by one into LDS and the tile is written
//           to the payload with 128-bit stores (pack), or read from the payload with 128-bit
//           loads into LDS and scattered from there (unpack).
//   NARROW  a contiguous float32 tensor whose values are exactly bfloat16: the payload holds
//           the high 16 bits of each element (pack reads 32 B and writes 16 B a chunk; unpack
//           writes the halves back with zero low bits), so the same bits cross the host link
//           in half the bytes.
//
// Grid: one 256-lane workgroup per 16 KiB tile of payload; tiles of all pieces of the
// launch are numbered consecutively and a workgroup finds its piece from the launch's array
// of piece start tiles.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mo_kdesc.h"
#include "mo_wire.h"

// The scratch of mo_pack_to_host (size kNoAllocScratchBytes). External linkage with a C name:
// the host finds it in the loaded code object with hipModuleGetGlobal, once per device, and
// passes that address to the pack kernel like any payload buffer (a static array would have no
// symbol in the code object). Only the pack kernel writes it and the DMA reads it.
extern "C" {
__device__ __align__(256) unsigned char mo_noalloc_scratch[mo::kNoAllocScratchBytes];
}

namespace mo {

__device__ __forceinline__ uint32_t fdiv(uint32_t n, uint32_t m, uint32_t s) {
  const uint64_t t = __umulhi(m, n);
  return (uint32_t)((t + n) >> s);
}

// Address offset (bytes, relative to the tensor base) of unit `u` of a piece's tensor side.
// A unit is a 16-byte chunk (RUNS) or an element (ELEM).
__device__ __forceinline__ uint64_t unit_offset(const KDesc& d, uint32_t u) {
  uint32_t q = fdiv(u, d.inner.m, d.inner.s);
  uint64_t off = (uint64_t)(u - q * d.inner.d) * d.inner_stride;
  const uint32_t nouter = d.nouter;
#pragma unroll
  for (int k = 0; k < kMaxOuter; ++k) {
    if (k < (int)nouter) {
      const uint32_t q2 = fdiv(q, d.outer[k].m, d.outer[k].s);
      off += (uint64_t)(q - q2 * d.outer[k].d) * d.ostride[k];
      q = q2;
    }
  }
  return off;
}

// Every device pointer reaches the kernels as an integer inside a descriptor, so the compiler
// cannot infer its address space and would emit flat (generic) memory instructions. The
// accessors below name the space: global (HBM or pinned host memory) or LDS.
#define MO_GLOBAL __attribute__((address_space(1)))
#define MO_LDS __attribute__((address_space(3)))

enum Space { kG, kL };

// 16-byte values move as a native vector: uint4 is a class whose copy constructor takes a
// generic reference, which would turn the access back into a flat one.
typedef unsigned int mo_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int mo_u32x2 __attribute__((ext_vector_type(2)));

template <Space S, typename T>
__device__ __forceinline__ T ld(const char* p) {
  if (S == kG) return *(const MO_GLOBAL T*)p;
  return *(const MO_LDS T*)p;
}
template <Space S, typename T>
__device__ __forceinline__ void st(char* p, T v) {
  if (S == kG) *(MO_GLOBAL T*)p = v;
  else *(MO_LDS T*)p = v;
}
template <>
__device__ __forceinline__ uint4 ld<kG, uint4>(const char* p) {
  const mo_u32x4 x = *(const MO_GLOBAL mo_u32x4*)p;
  return make_uint4(x.x, x.y, x.z, x.w);
}
template <>
__device__ __forceinline__ uint4 ld<kL, uint4>(const char* p) {
  const mo_u32x4 x = *(const MO_LDS mo_u32x4*)p;
  return make_uint4(x.x, x.y, x.z, x.w);
}
template <>
__device__ __forceinline__ void st<kG, uint4>(char* p, uint4 v) {
  *(MO_GLOBAL mo_u32x4*)p = mo_u32x4{v.x, v.y, v.z, v.w};
}
template <>
__device__ __forceinline__ void st<kL, uint4>(char* p, uint4 v) {
  *(MO_LDS mo_u32x4*)p = mo_u32x4{v.x, v.y, v.z, v.w};
}

template <Space D, Space S>
__device__ __forceinline__ void copy_elem(char* dst, const char* src, uint32_t eb) {
  switch (eb) {
    case 1: st<D>(dst, ld<S, uint8_t>(src)); break;
    case 2: st<D>(dst, ld<S, uint16_t>(src)); break;
    case 4: st<D>(dst, ld<S, uint32_t>(src)); break;
    case 8: st<D>(dst, ld<S, uint64_t>(src)); break;
    default: st<D>(dst, ld<S, uint4>(src)); break;
  }
}

__device__ __forceinline__ uint4 ld16(const char* p) { return ld<kG, uint4>(p); }
__device__ __forceinline__ void st16(char* p, uint4 v) { st<kG>(p, v); }

// Streaming store for the staging payload: it is written once and next read by a DMA engine,
// so the write is marked non-temporal (no reuse expected in the GPU caches).
__device__ __forceinline__ void st16_stream(char* p, uint4 v) {
  const mo_u32x4 x = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(x, (MO_GLOBAL mo_u32x4*)p);
}

// Full tiles whose cache policy the launch picks at run time (KDesc.cache) use buffer
// instructions, whose cache-policy operand is an immediate of the instruction: the policy arms of
// a switch then stay separate code paths. With ordinary loads and stores the arms differ only in a
// non-temporal hint, which the optimizer treats as metadata: it merges the arms into one and drops
// the hint. The resource spans one tile: raw access, stride 0, num_records = the tile's bytes,
// word 3 = DATA_FORMAT 32 (untyped buffer access on gfx9-family targets).
constexpr int kAuxNt = 2;  // cache-policy operand: bit 1 = nt on gfx940-family targets
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const char* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, 0, (int)bytes, 0x00020000);
}

// A full CONTIG tile: kUnroll 16-byte loads a lane in flight, then the stores.
template <bool kNtLoad, bool kNtStore>
__device__ __forceinline__ void contig_tile(char* dst, const char* src, uint32_t tid) {
  const __amdgpu_buffer_rsrc_t s = tile_rsrc(src, kTileBytes), t = tile_rsrc(dst, kTileBytes);
  mo_u32x4 v[kUnroll];
#pragma unroll
  for (int k = 0; k < kUnroll; ++k)
    v[k] = __builtin_amdgcn_raw_buffer_load_b128(s, (uint32_t)(k * kThreads + tid) * 16, 0, kNtLoad ? kAuxNt : 0);
#pragma unroll
  for (int k = 0; k < kUnroll; ++k)
    __builtin_amdgcn_raw_buffer_store_b128(v[k], t, (uint32_t)(k * kThreads + tid) * 16, 0, kNtStore ? kAuxNt : 0);
}

// A full NARROW unpack tile: 8 contiguous payload bytes (4 bfloat16 values) <-> 16 contiguous
// float32 tensor bytes a lane and round, so each instruction covers one span.
template <bool kNtLoad, bool kNtStore>
__device__ __forceinline__ void widen_tile(char* tensor32, const char* payload, uint32_t tid) {
  constexpr int kRounds = 2 * kUnroll;
  const __amdgpu_buffer_rsrc_t p = tile_rsrc(payload, kTileBytes), t = tile_rsrc(tensor32, 2 * kTileBytes);
  mo_u32x2 v[kRounds];
#pragma unroll
  for (int k = 0; k < kRounds; ++k)
    v[k] = __builtin_amdgcn_raw_buffer_load_b64(p, (uint32_t)(k * kThreads + tid) * 8, 0, kNtLoad ? kAuxNt : 0);
#pragma unroll
  for (int k = 0; k < kRounds; ++k)
    __builtin_amdgcn_raw_buffer_store_b128(mo_u32x4{v[k].x << 16, v[k].x & 0xffff0000u, v[k].y << 16, v[k].y & 0xffff0000u},
                                           t, (uint32_t)(k * kThreads + tid) * 16, 0, kNtStore ? kAuxNt : 0);
}

// Payload-side store: streaming when packing (the payload is the staging buffer).
template <bool kPack>
__device__ __forceinline__ void st16_out(char* p, uint4 v) {
  if (kPack) st16_stream(p, v);
  else st16(p, v);
}

// NARROW: 8 float32 elements (two 16-byte words a, b) <-> their 8 high halves (one 16-byte word;
// element j's bits at payload bytes 2j, 2j+1, little-endian).
__device__ __forceinline__ uint4 high_halves(uint4 a, uint4 b) {
  return make_uint4((a.x >> 16) | (a.y & 0xffff0000u), (a.z >> 16) | (a.w & 0xffff0000u),
                    (b.x >> 16) | (b.y & 0xffff0000u), (b.z >> 16) | (b.w & 0xffff0000u));
}
__device__ __forceinline__ void widen(uint4 v, uint4& a, uint4& b) {
  a = make_uint4(v.x << 16, v.x & 0xffff0000u, v.y << 16, v.y & 0xffff0000u);
  b = make_uint4(v.z << 16, v.z & 0xffff0000u, v.w << 16, v.w & 0xffff0000u);
}
template <bool kPack>
__device__ __forceinline__ void narrow_chunk(char* payload16, char* tensor32) {
  if (kPack) {
    const uint4 a = ld16(tensor32), b = ld16(tensor32 + 16);
    st16_stream(payload16, high_halves(a, b));
  } else {
    uint4 a, b;
    widen(ld16(payload16), a, b);
    st16(tensor32, a);
    st16(tensor32 + 16, b);
  }
}

template <bool kPack>
__device__ __forceinline__ void copy_tile_elem(const KDesc& d, uint64_t tile_off, uint32_t tile_bytes, char* payload,
                                               char* tensor, uint32_t eb, uint32_t tid);

// One 16 KiB tile (`tile`, numbered within the launch) of piece `d`. kElem: the launch may hold
// ELEM pieces, whose LDS staging buffer every workgroup of the launch then reserves; launches
// without them use the instantiation that reserves no LDS.
template <bool kPack, bool kElem>
__device__ __forceinline__ void copy_tile(const KDesc& d, uint32_t tile) {
  const uint32_t tid = threadIdx.x;
  const uint64_t tile_off = (uint64_t)(tile - d.tile0) * kTileBytes;  // bytes into the piece
  const uint64_t left = d.nbytes - tile_off;
  const uint32_t tile_bytes = left < kTileBytes ? (uint32_t)left : kTileBytes;
  char* const payload = (char*)d.payload + tile_off;
  char* const tensor = (char*)d.tensor;
  const uint32_t eb = d.eb;

  if (d.path == kPathContig) {
    char* const t = tensor + d.first + tile_off;
    const char* src = kPack ? t : payload;
    char* dst = kPack ? payload : t;
    if (tile_bytes == kTileBytes) {
      switch (d.cache & (kCacheNtLoad | kCacheNtStore)) {
        case 0: contig_tile<false, false>(dst, src, tid); break;
        case kCacheNtLoad: contig_tile<true, false>(dst, src, tid); break;
        case kCacheNtStore: contig_tile<false, true>(dst, src, tid); break;
        default: contig_tile<true, true>(dst, src, tid); break;
      }
    } else {
      const uint32_t nvec = tile_bytes / 16;
      for (uint32_t c = tid; c < nvec; c += kThreads) st16_out<kPack>(dst + (size_t)c * 16, ld16(src + (size_t)c * 16));
      for (uint32_t b = nvec * 16 + tid * eb; b < tile_bytes; b += kThreads * eb) copy_elem<kG, kG>(dst + b, src + b, eb);
    }
    return;
  }

  if (d.path == kPathNarrow) {
    // payload offsets count bfloat16 bits; the float32 tensor side is twice as far in. A full
    // tile, measured both ways on the block microbench: pack keeps 16-byte streaming stores (a
    // lane reads the 32 tensor bytes of one payload chunk); unpack is widen_tile.
    char* const t = tensor + 2 * (d.first + tile_off);
    if (tile_bytes == kTileBytes) {
      if (kPack) {
        uint4 a[kUnroll], b[kUnroll];
#pragma unroll
        for (int k = 0; k < kUnroll; ++k) {
          a[k] = ld16(t + (size_t)(k * kThreads + tid) * 32);
          b[k] = ld16(t + (size_t)(k * kThreads + tid) * 32 + 16);
        }
#pragma unroll
        for (int k = 0; k < kUnroll; ++k) st16_stream(payload + (size_t)(k * kThreads + tid) * 16, high_halves(a[k], b[k]));
      } else {
        switch (d.cache & (kCacheNtLoad | kCacheNtStore)) {
          case 0: widen_tile<false, false>(t, payload, tid); break;
          case kCacheNtLoad: widen_tile<true, false>(t, payload, tid); break;
          case kCacheNtStore: widen_tile<false, true>(t, payload, tid); break;
          default: widen_tile<true, true>(t, payload, tid); break;
        }
      }
    } else {
      const uint32_t nvec = tile_bytes / 16;
      for (uint32_t c = tid; c < nvec; c += kThreads) narrow_chunk<kPack>(payload + (size_t)c * 16, t + (size_t)c * 32);
      for (uint32_t b = nvec * 16 + tid * 2; b < tile_bytes; b += kThreads * 2) {
        if (kPack)
          st<kG>(payload + b, (uint16_t)(ld<kG, uint32_t>(t + (size_t)b * 2) >> 16));
        else
          st<kG>(t + (size_t)b * 2, (uint32_t)ld<kG, uint16_t>(payload + b) << 16);
      }
    }
    return;
  }

  if (d.path == kPathRuns) {
    const uint32_t c0 = (uint32_t)(tile_off / 16);
    const uint32_t nchunk = tile_bytes / 16;
    const uint32_t first = (uint32_t)d.first;
    uint4 v[kUnroll];
    uint64_t toff[kUnroll];
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
      const uint32_t c = k * kThreads + tid;
      if (c < nchunk) {
        toff[k] = unit_offset(d, first + c0 + c);
        v[k] = kPack ? ld16(tensor + toff[k]) : ld16(payload + (size_t)c * 16);
      }
    }
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
      const uint32_t c = k * kThreads + tid;
      if (c < nchunk) {
        if (kPack) st16_stream(payload + (size_t)c * 16, v[k]);
        else st16(tensor + toff[k], v[k]);
      }
    }
    return;
  }

  if constexpr (kElem) copy_tile_elem<kPack>(d, tile_off, tile_bytes, payload, tensor, eb, tid);
}

// ELEM: LDS-staged element gather / scatter of one tile.
template <bool kPack>
__device__ __forceinline__ void copy_tile_elem(const KDesc& d, uint64_t tile_off, uint32_t tile_bytes, char* payload,
                                               char* tensor, uint32_t eb, uint32_t tid) {
  __shared__ uint4 lds[kTileBytes / 16];
  char* const sbuf = (char*)lds;
  const uint32_t nelem = tile_bytes / eb;
  const uint32_t e0 = (uint32_t)d.first + (uint32_t)(tile_off / eb);
  const uint32_t nvec = tile_bytes / 16;
  if (kPack) {
    for (uint32_t j = tid; j < nelem; j += kThreads)
      copy_elem<kL, kG>(sbuf + (size_t)j * eb, tensor + unit_offset(d, e0 + j), eb);
    __syncthreads();
    for (uint32_t c = tid; c < nvec; c += kThreads) st16_stream(payload + (size_t)c * 16, ld<kL, uint4>(sbuf + (size_t)c * 16));
    for (uint32_t b = nvec * 16 + tid * eb; b < tile_bytes; b += kThreads * eb) copy_elem<kG, kL>(payload + b, sbuf + b, eb);
  } else {
    for (uint32_t c = tid; c < nvec; c += kThreads) st<kL>(sbuf + (size_t)c * 16, ld16(payload + (size_t)c * 16));
    for (uint32_t b = nvec * 16 + tid * eb; b < tile_bytes; b += kThreads * eb) copy_elem<kL, kG>(sbuf + b, payload + b, eb);
    __syncthreads();
    for (uint32_t j = tid; j < nelem; j += kThreads)
      copy_elem<kG, kL>(tensor + unit_offset(d, e0 + j), sbuf + (size_t)j * eb, eb);
  }
}

// Several pieces: the workgroup's piece is the last one starting at or before its tile. The
// starts are one contiguous array (unused entries UINT32_MAX), compared without branches.
template <bool kPack, bool kElem>
__device__ __forceinline__ void copy_body(const LaunchArgs& args) {
  const uint32_t tile = blockIdx.x;
  uint32_t i = 0;
#pragma unroll
  for (int k = 1; k < kMaxDesc; ++k) i += args.tile0[k] <= tile ? 1u : 0u;
  copy_tile<kPack, kElem>(args.d[i], tile);
}

}  // namespace mo

extern "C" __global__ __launch_bounds__(mo::kThreads) void mo_pack_kernel(const mo::LaunchArgs args) {
  mo::copy_body<true, false>(args);
}

extern "C" __global__ __launch_bounds__(mo::kThreads) void mo_unpack_kernel(const mo::LaunchArgs args) {
  mo::copy_body<false, false>(args);
}

// The same with ELEM pieces in the launch (16 KiB of LDS a workgroup).
extern "C" __global__ __launch_bounds__(mo::kThreads) void mo_pack_elem_kernel(const mo::LaunchArgs args) {
  mo::copy_body<true, true>(args);
}

extern "C" __global__ __launch_bounds__(mo::kThreads) void mo_unpack_elem_kernel(const mo::LaunchArgs args) {
  mo::copy_body<false, true>(args);
}

// One piece (tile0 == 0): the same work with a single descriptor as the kernel argument, which
// cuts the argument block a launch carries from sizeof(LaunchArgs) to sizeof(KDesc). Most
// launches move one saved tensor.
extern "C" __global__ __launch_bounds__(mo::kThreads) void mo_pack1_kernel(const mo::KDesc d) {
  mo::copy_tile<true, false>(d, blockIdx.x);
}

extern "C" __global__ __launch_bounds__(mo::kThreads) void mo_unpack1_kernel(const mo::KDesc d) {
  mo::copy_tile<false, false>(d, blockIdx.x);
}

extern "C" __global__ __launch_bounds__(mo::kThreads) void mo_pack1_elem_kernel(const mo::KDesc d) {
  mo::copy_tile<true, true>(d, blockIdx.x);
}

extern "C" __global__ __launch_bounds__(mo::kThreads) void mo_unpack1_elem_kernel(const mo::KDesc d) {
  mo::copy_tile<false, true>(d, blockIdx.x);
}

// Byte equality of two ranges (both 16-byte aligned), one 16 KiB tile per workgroup. Lanes
// that see a difference write 1 to *flag (pinned host memory the host cleared before the
// launch); equal ranges write nothing. The host reads the flag once an event recorded after
// the launch has completed.
extern "C" __global__ __launch_bounds__(mo::kThreads) void mo_equal_kernel(const char* a, const char* b,
                                                                            uint64_t nbytes, uint32_t* flag) {
  using namespace mo;
  const uint32_t tid = threadIdx.x;
  const uint64_t tile_off = (uint64_t)blockIdx.x * kTileBytes;
  const uint64_t left = nbytes - tile_off;
  const char* const x = a + tile_off;
  const char* const y = b + tile_off;
  uint32_t diff = 0;
  if (left >= kTileBytes) {
    uint4 u[kUnroll], v[kUnroll];
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
      u[k] = ld16(x + (size_t)(k * kThreads + tid) * 16);
      v[k] = ld16(y + (size_t)(k * kThreads + tid) * 16);
    }
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) diff |= (u[k].x ^ v[k].x) | (u[k].y ^ v[k].y) | (u[k].z ^ v[k].z) | (u[k].w ^ v[k].w);
  } else {
    const uint32_t nvec = (uint32_t)(left / 16);
    for (uint32_t c = tid; c < nvec; c += kThreads) {
      const uint4 u = ld16(x + (size_t)c * 16), v = ld16(y + (size_t)c * 16);
      diff |= (u.x ^ v.x) | (u.y ^ v.y) | (u.z ^ v.z) | (u.w ^ v.w);
    }
    for (uint32_t i = nvec * 16 + tid; i < (uint32_t)left; i += kThreads)
      diff |= (uint32_t)(ld<kG, uint8_t>(x + i) ^ ld<kG, uint8_t>(y + i));
  }
  if (diff) st<kG>((char*)flag, 1u);
}

// Device <-> pinned-host copy through the shader engines instead of a DMA engine.
// Each lane keeps kLinkUnroll 16-byte transfers in flight; the grid strides over the buffer.
extern "C" __global__ __launch_bounds__(mo::kThreads) void mo_link_copy_kernel(char* __restrict__ dst,
                                                                                const char* __restrict__ src,
                                                                                uint64_t nbytes) {
  using namespace mo;
  const uint64_t nvec = nbytes / 16;
  const uint64_t lanes = (uint64_t)gridDim.x * kThreads;
  const uint64_t step = lanes * kLinkUnroll;
  uint64_t base = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
  for (; base + (kLinkUnroll - 1) * lanes < nvec; base += step) {
    uint4 v[kLinkUnroll];
#pragma unroll
    for (int k = 0; k < kLinkUnroll; ++k) v[k] = ld16(src + (base + k * lanes) * 16);
#pragma unroll
    for (int k = 0; k < kLinkUnroll; ++k) st16(dst + (base + k * lanes) * 16, v[k]);
  }
  for (; base < nvec; base += lanes) st16(dst + base * 16, ld16(src + base * 16));
  if (blockIdx.x == 0) {
    for (uint64_t b = nvec * 16 + threadIdx.x; b < nbytes; b += kThreads) st<kG>(dst + b, ld<kG, uint8_t>(src + b));
  }
}

// ------------------------------------------------------------------------------------------
// Wire coding of a staging segment (format in mo_wire.h): three kernels code a segment into a
// wire buffer (block sizes per tile, one-workgroup scan of the tile sizes into offsets plus
// the header and the raw tail, then the tiles), and one kernel decodes it. Each workgroup codes
// one tile of 32 blocks; each of its four waves takes 8 blocks, a lane 8 words (16 bytes) of
// a block. Every store into the wire buffer goes through a buffer resource bounded by the
// buffer's capacity, and the decoder reads the coded stream through one too, so a stream that
// arrives damaged cannot make either kernel touch memory outside its buffers.
namespace mo {

__device__ __forceinline__ uint32_t wave_min(uint32_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = min(v, (uint32_t)__shfl_xor((int)v, m, 64));
  return v;
}
__device__ __forceinline__ uint32_t wave_max(uint32_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, m, 64));
  return v;
}
// Inclusive prefix sum over the wave's lanes.
__device__ __forceinline__ uint32_t wave_scan(uint32_t v, uint32_t lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t y = (uint32_t)__shfl_up((int)v, d, 64);
    if (lane >= (uint32_t)d) v += y;
  }
  return v;
}
__device__ __forceinline__ uint32_t word_of(const uint4& v, int k) {
  const uint32_t w = k < 2 ? v.x : k < 4 ? v.y : k < 6 ? v.z : v.w;
  return (k & 1) ? w >> 16 : w & 0xffffu;
}
__device__ __forceinline__ uint32_t exponent_of(uint32_t word) { return (word >> 7) & 0xffu; }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t wire_rsrc(const char* p, uint64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, 0, (int)(bytes < 0x7fffffffull ? bytes : 0x7fffffffull),
                                           0x00020000);
}

struct WireCode {
  uint32_t width, base, escapes;
};

// Orders the wave's own LDS accesses (a wave's LDS operations execute in order; this keeps the
// compiler from moving them across).
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// The coding of one block (mo_wire.h), by one wave; `hist` and `pref` are the wave's own 32
// words of LDS each. Among width 8, and widths 1-5 with a window of offsets s.. from the
// block's smallest exponent (no escapes when every exponent fits 2^k values, else 2^k - 1
// values and escapes), it takes the smallest coded size, ties to the smaller width, then the
// smaller s.
__device__ __forceinline__ WireCode wire_choose(const uint4& v, uint32_t lane, uint32_t* hist, uint32_t* pref) {
  uint32_t lo = 255, hi = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t e = exponent_of(word_of(v, j));
    lo = min(lo, e);
    hi = max(hi, e);
  }
  lo = wave_min(lo);
  if (__all(hi == lo)) return WireCode{0, lo, 0};  // every exponent of the block equals the smallest
  if (lane < kWireBins) hist[lane] = 0;
  wave_lds_fence();
#pragma unroll
  for (int j = 0; j < 8; ++j) atomicAdd(&hist[min(exponent_of(word_of(v, j)) - lo, kWireBins - 1)], 1u);
  wave_lds_fence();
  const uint32_t h = lane < kWireBins ? hist[lane] : 0u;
  const uint32_t p = wave_scan(h, lane) - h;  // lane i < 32: words in bins 0..i-1
  if (lane < kWireBins) pref[lane] = p;
  wave_lds_fence();
  uint32_t best = (wire_block_coded(8, 0) << 16) | (8u << 8);
  uint32_t nesc[6] = {0, 0, 0, 0, 0, 0};
#pragma unroll
  for (uint32_t k = 1; k <= 5; ++k) {
    const uint32_t w = 1u << k;
    const uint32_t s = lane;
    uint32_t esc = 0xffffu;
    if (s + w - 1 <= kWireBins - 1) {
      if (s + w <= kWireBins - 1 && pref[s + w] - p == kWireBlockVals) esc = 0;
      else esc = kWireBlockVals - (pref[s + w - 1] - p);
    }
    nesc[k] = esc;
    if (esc != 0xffffu) best = min(best, (wire_block_coded(k, esc) << 16) | (k << 8) | s);
  }
  best = wave_min(best);
  const uint32_t width = (best >> 8) & 0xffu, s = best & 0xffu;
  if (width == 8) return WireCode{8, 0, 0};
  uint32_t mine = 0;
#pragma unroll
  for (uint32_t k = 1; k <= 5; ++k)
    if (k == width) mine = nesc[k];
  return WireCode{width, lo + s, (uint32_t)__shfl((int)mine, (int)s, 64)};
}

// The code of exponent e in a block coded as c; sets *escape for an escaped exponent.
__device__ __forceinline__ uint32_t wire_code_of(uint32_t e, const WireCode& c, bool* escape) {
  *escape = false;
  if (c.width == 8) return e;
  if (c.width == 0) return 0;
  const uint32_t d = e - c.base;  // wraps for e < base
  const uint32_t limit = c.escapes ? (1u << c.width) - 1u : (1u << c.width);
  if (d < limit) return d;
  *escape = true;
  return (1u << c.width) - 1u;
}

}  // namespace mo

// Pass 1: each block's coding (its header, into the working space after the largest stream)
// and the coded size of each tile, into the stream's tile table.
extern "C" __global__ __launch_bounds__(mo::kThreads) void mo_wire_sizes_kernel(const char* raw, uint64_t raw_bytes,
                                                                                 char* wire, uint64_t wire_capacity) {
  using namespace mo;
  constexpr int kWaves = kThreads / 64;
  __shared__ uint32_t hist[kWaves][kWireBins], pref[kWaves][kWireBins];
  __shared__ uint32_t part[kWaves];
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint64_t nblocks = wire_blocks(raw_bytes);
  const uint64_t tile = blockIdx.x;
  const __amdgpu_buffer_rsrc_t w = wire_rsrc(wire, wire_capacity);
  const uint64_t scratch = wire_scratch_offset(raw_bytes);
  uint4 v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint64_t b = tile * kWireTileBlocks + wave * 8 + j;
    v[j] = b < nblocks ? ld16(raw + b * kWireBlockBytes + lane * 16) : make_uint4(0, 0, 0, 0);
  }
  uint32_t sum = 0;
  for (int j = 0; j < 8; ++j) {
    const uint64_t b = tile * kWireTileBlocks + wave * 8 + j;
    const WireCode c = wire_choose(v[j], lane, hist[wave], pref[wave]);
    if (b < nblocks) {
      sum += wire_block_coded(c.width, c.escapes);
      if (lane == 0)
        __builtin_amdgcn_raw_buffer_store_b32(c.base | (c.width << 8) | (c.escapes << 12), w, (int)(scratch + 4 * b), 0,
                                              0);
    }
  }
  if (lane == 0) part[wave] = sum;
  __syncthreads();
  if (threadIdx.x == 0)
    __builtin_amdgcn_raw_buffer_store_b32(kWireTileHeader + part[0] + part[1] + part[2] + part[3], w,
                                          (int)(kWireHeader + 4 * tile), 0, 0);
}

// Pass 2 (one workgroup of kWireScanThreads): tile sizes -> tile offsets (exclusive scan from
// tiles_start), the header, the raw tail; the total also to `host_total` (pinned host memory,
// may be null), where the copy engine's issuer reads it once this kernel has completed.
extern "C" __global__ __launch_bounds__(mo::kWireScanThreads) void mo_wire_scan_kernel(const char* raw,
                                                                                        uint64_t raw_bytes, char* wire,
                                                                                        uint64_t wire_capacity,
                                                                                        uint64_t* host_total) {
  using namespace mo;
  __shared__ uint32_t sh[kWireScanThreads];
  const uint32_t tid = threadIdx.x;
  const __amdgpu_buffer_rsrc_t w = wire_rsrc(wire, wire_capacity);
  const uint64_t tiles = wire_tiles(raw_bytes);
  uint64_t carry = wire_tiles_start(raw_bytes);
  for (uint64_t base = 0; base < tiles; base += kWireScanThreads) {
    const uint64_t t = base + tid;
    const uint32_t v = t < tiles ? __builtin_amdgcn_raw_buffer_load_b32(w, (int)(kWireHeader + 4 * t), 0, 0) : 0u;
    sh[tid] = v;
    __syncthreads();
    for (uint32_t off = 1; off < kWireScanThreads; off <<= 1) {
      const uint32_t x = tid >= off ? sh[tid - off] : 0u;
      __syncthreads();
      sh[tid] += x;
      __syncthreads();
    }
    if (t < tiles)
      __builtin_amdgcn_raw_buffer_store_b32((uint32_t)(carry + sh[tid] - v), w, (int)(kWireHeader + 4 * t), 0, 0);
    const uint32_t chunk = sh[kWireScanThreads - 1];
    __syncthreads();  // every lane has read sh before the next chunk overwrites it
    carry += chunk;
  }
  const uint64_t tail = raw_bytes % kWireBlockBytes, tail_src = wire_blocks(raw_bytes) * kWireBlockBytes;
  const uint64_t data_start = wire_data_start(raw_bytes);
  for (uint64_t i = tid; i < tail; i += kWireScanThreads)
    __builtin_amdgcn_raw_buffer_store_b8(ld<kG, uint8_t>(raw + tail_src + i), w, (int)(data_start + i), 0, 0);
  if (tid == 0) {
    __builtin_amdgcn_raw_buffer_store_b32((uint32_t)carry, w, 0, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b32((uint32_t)(carry >> 32), w, 4, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b32((uint32_t)raw_bytes, w, 8, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b32((uint32_t)tiles, w, 12, 0, 0);
    if (host_total) st<kG>((char*)host_total, carry);
  }
}

// Pass 3: code each tile at its offset.
extern "C" __global__ __launch_bounds__(mo::kThreads) void mo_wire_encode_kernel(const char* raw, uint64_t raw_bytes,
                                                                                  char* wire, uint64_t wire_capacity) {
  using namespace mo;
  constexpr int kWaves = kThreads / 64;
  __shared__ uint32_t head[kWireTileBlocks], pre[kWireTileBlocks];
  __shared__ __attribute__((aligned(16))) unsigned char plane[kWaves][kWireBlockVals];
  __shared__ __attribute__((aligned(16))) unsigned char escs[kWaves][kWireBlockVals];
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint64_t nblocks = wire_blocks(raw_bytes);
  const uint64_t tile = blockIdx.x;
  const __amdgpu_buffer_rsrc_t w = wire_rsrc(wire, wire_capacity);
  const uint32_t toff = __builtin_amdgcn_raw_buffer_load_b32(w, (int)(kWireHeader + 4 * tile), 0, 0);
  const uint64_t scratch = wire_scratch_offset(raw_bytes);
  uint4 v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint64_t b = tile * kWireTileBlocks + wave * 8 + j;
    v[j] = b < nblocks ? ld16(raw + b * kWireBlockBytes + lane * 16) : make_uint4(0, 0, 0, 0);
  }
  if (threadIdx.x < kWireTileBlocks) {
    // the block codings the sizing pass chose (zero past the end)
    const uint64_t b = tile * kWireTileBlocks + threadIdx.x;
    head[threadIdx.x] = b < nblocks ? __builtin_amdgcn_raw_buffer_load_b32(w, (int)(scratch + 4 * b), 0, 0) : 0u;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t acc = 0;
    for (uint32_t k = 0; k < kWireTileBlocks; ++k) {
      pre[k] = acc;
      if (tile * kWireTileBlocks + k < nblocks) acc += wire_block_coded((head[k] >> 8) & 0xfu, head[k] >> 12);
    }
  }
  if (threadIdx.x < kWireTileBlocks)
    __builtin_amdgcn_raw_buffer_store_b32(head[threadIdx.x], w, (int)(toff + 4 * threadIdx.x), 0, 0);
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t bl = wave * 8 + j;
    const bool live = tile * kWireTileBlocks + bl < nblocks;
    const WireCode c{(head[bl] >> 8) & 0xfu, head[bl] & 0xffu, head[bl] >> 12};
    const uint32_t dst = toff + kWireTileHeader + pre[bl];
    uint32_t sm_lo = 0, sm_hi = 0, nmine = 0;
    uint64_t acc = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t word = word_of(v[j], k);
      const uint32_t sm = ((word >> 8) & 0x80u) | (word & 0x7fu);
      if (k < 4) sm_lo |= sm << (8 * k);
      else sm_hi |= sm << (8 * (k - 4));
      bool escape;
      acc |= (uint64_t)wire_code_of(exponent_of(word), c, &escape) << (k * c.width);
      nmine += escape ? 1u : 0u;
    }
    uint32_t eoff = wave_scan(nmine, lane) - nmine;  // this lane's first escape, in word order
    if (live) {
      typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
      __builtin_amdgcn_raw_buffer_store_b64(u32x2{sm_lo, sm_hi}, w, (int)(dst + 8 * lane), 0, 0);
      for (uint32_t i = 0; i < c.width; ++i) plane[wave][lane * c.width + i] = (unsigned char)(acc >> (8 * i));
      if (nmine) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          bool escape;
          const uint32_t e = exponent_of(word_of(v[j], k));
          (void)wire_code_of(e, c, &escape);
          if (escape) escs[wave][min(eoff++, kWireBlockVals - 1)] = (unsigned char)e;
        }
      }
      // zero padding after the escapes, up to the next 16 bytes
      const uint32_t padded = (uint32_t)wire_align16(c.escapes);
      for (uint32_t i = c.escapes + lane; i < padded; i += 64) escs[wave][i] = 0;
    }
    __syncthreads();
    if (live) {
      if (lane < 4 * c.width) {
        const mo_u32x4 chunk = *(const MO_LDS mo_u32x4*)(&plane[wave][16 * lane]);
        __builtin_amdgcn_raw_buffer_store_b128(chunk, w, (int)(dst + kWireBlockVals + 16 * lane), 0, 0);
      }
      if (16 * lane < c.escapes) {
        const mo_u32x4 chunk = *(const MO_LDS mo_u32x4*)(&escs[wave][16 * lane]);
        __builtin_amdgcn_raw_buffer_store_b128(chunk, w, (int)(dst + kWireBlockVals + 64 * c.width + 16 * lane), 0,
                                               0);
      }
    }
    __syncthreads();  // the LDS planes are rewritten by the next block
  }
}

// Decode a coded stream of `raw_bytes` into `raw`. Grid: max(tiles, 1) workgroups; the first
// also copies the raw tail. Reads go through a resource over [wire, wire + wire_bytes), writes
// stay inside [raw, raw + raw_bytes) whatever the stream holds.
extern "C" __global__ __launch_bounds__(mo::kThreads) void mo_wire_decode_kernel(const char* wire, uint64_t wire_bytes,
                                                                                  uint64_t raw_bytes, char* raw) {
  using namespace mo;
  constexpr int kWaves = kThreads / 64;
  __shared__ uint32_t head[kWireTileBlocks], pre[kWireTileBlocks];
  __shared__ __attribute__((aligned(16))) unsigned char plane[kWaves][kWireBlockVals];
  __shared__ __attribute__((aligned(16))) unsigned char escs[kWaves][kWireBlockVals];
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint64_t nblocks = wire_blocks(raw_bytes);
  const uint64_t tile = blockIdx.x;
  const __amdgpu_buffer_rsrc_t w = wire_rsrc(wire, wire_bytes);
  const uint32_t toff = __builtin_amdgcn_raw_buffer_load_b32(w, (int)(kWireHeader + 4 * tile), 0, 0);
  if (threadIdx.x < kWireTileBlocks) {
    const uint32_t h = __builtin_amdgcn_raw_buffer_load_b32(w, (int)(toff + 4 * threadIdx.x), 0, 0);
    // clamp what a damaged header could hold: width 0-8, escapes 0-512
    head[threadIdx.x] = (h & 0xffu) | (min((h >> 8) & 0xfu, 8u) << 8) | (min(h >> 12, kWireBlockVals) << 12);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t acc = 0;
    for (uint32_t k = 0; k < kWireTileBlocks; ++k) {
      pre[k] = acc;
      acc += wire_block_coded((head[k] >> 8) & 0xfu, head[k] >> 12);
    }
  }
  __syncthreads();
  for (int j = 0; j < 8; ++j) {
    const uint32_t bl = wave * 8 + j;
    const uint64_t b = tile * kWireTileBlocks + bl;
    const bool live = b < nblocks;
    const WireCode c{(head[bl] >> 8) & 0xfu, head[bl] & 0xffu, head[bl] >> 12};
    const uint32_t src = toff + kWireTileHeader + pre[bl];
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    u32x2 sm = {0, 0};
    if (live) {
      sm = __builtin_amdgcn_raw_buffer_load_b64(w, (int)(src + 8 * lane), 0, 0);
      if (lane < 4 * c.width)
        *(MO_LDS mo_u32x4*)(&plane[wave][16 * lane]) =
            __builtin_amdgcn_raw_buffer_load_b128(w, (int)(src + kWireBlockVals + 16 * lane), 0, 0);
      if (16 * lane < c.escapes)
        *(MO_LDS mo_u32x4*)(&escs[wave][16 * lane]) = __builtin_amdgcn_raw_buffer_load_b128(
            w, (int)(src + kWireBlockVals + 64 * c.width + 16 * lane), 0, 0);
    }
    __syncthreads();
    uint64_t acc = 0;
    for (uint32_t i = 0; i < c.width; ++i) acc |= (uint64_t)plane[wave][lane * c.width + i] << (8 * i);
    const uint32_t mask = (1u << c.width) - 1u;
    const uint32_t esc_code = c.escapes && c.width && c.width < 8 ? mask : 0xffffffffu;
    uint32_t nmine = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) nmine += ((uint32_t)(acc >> (k * c.width)) & mask) == esc_code ? 1u : 0u;
    uint32_t eoff = wave_scan(nmine, lane) - nmine;
    if (live) {
      uint32_t out[4];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t s = ((k < 4 ? sm[0] : sm[1]) >> (8 * (k & 3))) & 0xffu;
        const uint32_t code = (uint32_t)(acc >> (k * c.width)) & mask;
        uint32_t e;
        if (c.width == 8) e = code;
        else if (code == esc_code) e = escs[wave][min(eoff++, kWireBlockVals - 1)];
        else e = (c.base + code) & 0xffu;
        const uint32_t word = ((s & 0x80u) << 8) | (e << 7) | (s & 0x7fu);
        if (k & 1) out[k >> 1] |= word << 16;
        else out[k >> 1] = word;
      }
      st16(raw + b * kWireBlockBytes + lane * 16, make_uint4(out[0], out[1], out[2], out[3]));
    }
    __syncthreads();
  }
  if (tile == 0) {
    const uint64_t tail = raw_bytes % kWireBlockBytes, tail_dst = nblocks * kWireBlockBytes;
    const uint64_t data_start = wire_data_start(raw_bytes);
    for (uint64_t i = threadIdx.x; i < tail; i += kThreads)
      st<kG>(raw + tail_dst + i, (uint8_t)__builtin_amdgcn_raw_buffer_load_b8(w, (int)(data_start + i), 0, 0));
  }
}
