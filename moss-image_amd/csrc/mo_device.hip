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
// wire buffer (each tile's exponent model and rANS stream into the working space, with its
// coded size; a one-workgroup scan of the tile sizes into offsets plus the header and the raw
// tail; then each tile assembled at its offset), and one kernel decodes it. One wave codes or
// decodes one tile, four waves a workgroup; the waves share no LDS and never wait for each
// other. Every store into the wire buffer goes through a buffer resource bounded by the
// buffer's capacity, and the decoder reads the coded stream through one too, so a stream that
// arrives damaged cannot make either kernel touch memory outside its buffers.
namespace mo {
constexpr int kWireWaves = kThreads / 64;
constexpr uint32_t kWireOob = 0x80000000u;  // a buffer offset past every wire buffer: the access is dropped
static_assert(kWireWaves == (int)kWireTilesPerGroup, "one wave per tile");

__device__ __forceinline__ uint32_t wave_max(uint32_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, m, 64));
  return v;
}
__device__ __forceinline__ uint32_t wave_sum(uint32_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += (uint32_t)__shfl_xor((int)v, m, 64);
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
// Inclusive prefix maximum over the wave's lanes (values >= 0), by DPP moves: shifts by 1, 2, 4
// and 8 lanes within each row of 16, then row 0's last lane into row 1 and row 2's into row 3,
// then lane 31 into rows 2 and 3. Lanes a move has no source for take 0.
__device__ __forceinline__ uint32_t wave_scan_max_dpp(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, false));  // row_shr:1
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, false));  // row_shr:2
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, false));  // row_shr:4
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, false));  // row_shr:8
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false));  // row_bcast:15
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false));  // row_bcast:31
  return v;
}
// Lanes below this one whose bit is set in `mask`.
__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}
__device__ __forceinline__ uint32_t word_of(const uint4& v, int k) {
  const uint32_t w = k < 2 ? v.x : k < 4 ? v.y : k < 6 ? v.z : v.w;
  return (k & 1) ? w >> 16 : w & 0xffffu;
}
__device__ __forceinline__ uint32_t exponent_of(uint32_t word) { return (word >> 7) & 0xffu; }
__device__ __forceinline__ uint32_t sign_mantissa_of(uint32_t word) { return ((word >> 8) & 0x80u) | (word & 0x7fu); }
__device__ __forceinline__ __amdgpu_buffer_rsrc_t wire_rsrc(const char* p, uint64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, 0, (int)(bytes < 0x7fffffffull ? bytes : 0x7fffffffull),
                                           0x00020000);
}
// Orders the wave's own LDS accesses (a wave's LDS operations execute in order; this keeps the
// compiler from moving them across).
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
}
// Coder table entry of one exponent: frequency (bits 0-12), cumulative frequency (bits 13-24)
// and the shift of its division magic (bits 25-28).
__device__ __forceinline__ uint32_t shift_of(uint32_t f) { return f > 1 ? 32u - (uint32_t)__clz((int)(f - 1)) : 0u; }
}  // namespace mo

// Pass 1: each tile's exponent frequencies, normalised, its rANS stream and final states in the
// working space, and the tile's coded size into the stream's tile table. One wave per tile, 3.5
// KiB of LDS a wave: the counts, then each exponent's coder entry and division magic, and one
// group's exponents. State l codes the tile's words 64 j + l, so a group of 8 rounds is 1 KiB of
// consecutive words: one 16-byte load a lane, moved to LDS, read back one byte a round.
extern "C" __global__ __launch_bounds__(mo::kThreads) void mo_wire_sizes_kernel(const char* raw, uint64_t raw_bytes,
                                                                                 char* wire, uint64_t wire_capacity) {
  using namespace mo;
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  __shared__ uint32_t counts[kWireWaves][256];
  __shared__ u32x2 coder[kWireWaves][256];  // {entry, magic}: entry = f | c << 13 | shift << 25
  __shared__ __attribute__((aligned(16))) unsigned char groups[kWireWaves][8 * kWireLanes];
  const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint64_t tile = (uint64_t)blockIdx.x * kWireTilesPerGroup + wave;
  if (tile >= wire_tiles(raw_bytes)) return;  // wave-uniform; the waves never synchronise
  const uint32_t n = wire_tile_words(raw_bytes, tile), J = n / kWireLanes, nb = n / kWireBlockVals;
  const char* src = raw + tile * kWireTileRaw;
  const __amdgpu_buffer_rsrc_t w = wire_rsrc(wire, wire_capacity);
  const uint32_t rec = (uint32_t)(wire_scratch_offset(raw_bytes) + tile * kWireScratchTile);
  MO_LDS uint32_t* const cnt = (MO_LDS uint32_t*)counts[wave];
  MO_LDS u32x2* const cod = (MO_LDS u32x2*)coder[wave];
  for (uint32_t b = lane; b < 256; b += 64) cnt[b] = 0;
  wave_lds_fence();
  // Histogram: 8 loads of 16 bytes a lane in flight; each lane adds its 8 exponents once per
  // distinct value (neighbouring words mostly share exponents, and same-address LDS atomics of
  // a wave serialise).
  for (uint32_t c0 = 0; c0 < n / 8; c0 += 8 * 64) {
    uint4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t c = c0 + 64 * i + lane;
      v[i] = c < n / 8 ? ld16(src + 16 * (uint64_t)c) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (c0 + 64 * i + lane >= n / 8) continue;
      uint32_t e[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) e[k] = exponent_of(word_of(v[i], k));
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        uint32_t same = 0;
        bool first = true;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          same += e[q] == e[k] ? 1u : 0u;
          if (q < k && e[q] == e[k]) first = false;
        }
        if (first) atomicAdd(&counts[wave][e[k]], same);
      }
    }
  }
  wave_lds_fence();
  // Normalised frequencies: lane l owns exponents 4l .. 4l + 3.
  uint32_t f[4], fsum = 0, best = 0, pres = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t e = 4 * lane + k, c = cnt[e];
    f[k] = c ? max(1u, 8u * c / nb) : 0u;  // floor(c * 4096 / n), n = 512 nb
    fsum += f[k];
    pres += c ? 1u : 0u;
    best = max(best, (c << 8) | (255u - e));  // most frequent, the smallest exponent on ties
  }
  fsum = wave_sum(fsum);
  best = wave_max(best);
  const uint32_t top_e = 255u - (best & 0xffu);
  uint32_t mine = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k)
    if (4 * lane + k == top_e) mine = f[k];
  const int adjusted = (int)__shfl((int)mine, (int)(top_e >> 2), 64) + (int)(1u << kWireProbBits) - (int)fsum;
  bool raw_tile = adjusted < 1;
#pragma unroll
  for (int k = 0; k < 4; ++k)
    if (4 * lane + k == top_e) f[k] = (uint32_t)adjusted;
  // cumulative frequencies, the table (ascending exponents) and the coder entries
  const uint32_t lsum = f[0] + f[1] + f[2] + f[3];
  uint32_t cum = wave_scan(lsum, lane) - lsum;
  const uint32_t rank_incl = wave_scan(pres, lane);
  const uint32_t nsym = (uint32_t)__shfl((int)rank_incl, 63, 64);
  uint32_t rank = rank_incl - pres;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t e = 4 * lane + k;
    if (f[k]) {
      __builtin_amdgcn_raw_buffer_store_b32(e | (f[k] << 8), w, (int)(rec + kWireScratchTable + 4 * rank), 0, 0);
      ++rank;
      const uint32_t s = shift_of(f[k]);
      cod[e] = u32x2{f[k] | (cum << 13) | (s << 25), (uint32_t)(((((uint64_t)1 << s) - f[k]) << 32) / f[k] + 1)};
    }
    cum += f[k];
  }
  wave_lds_fence();
  // rANS over j = J-1 .. 0; the stream fills the working space from its end downwards
  uint32_t x = kWireStateLow, top = J * kWireLanes;
  if (!raw_tile) {
    MO_LDS unsigned char* const grp = (MO_LDS unsigned char*)groups[wave];
    const int ngroups = (int)(J / 8);
    uint4 next = ld16(src + 1024 * (uint64_t)(ngroups - 1) + 16 * lane);
    for (int g = ngroups - 1; g >= 0; --g) {
      const uint4 v = next;
      next = ld16(src + 1024 * (uint64_t)(g > 0 ? g - 1 : 0) + 16 * lane);  // the last one is a spare
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        lo |= exponent_of(word_of(v, k)) << (8 * k);
        hi |= exponent_of(word_of(v, k + 4)) << (8 * k);
      }
      wave_lds_fence();  // the previous group's reads are done
      *(MO_LDS u32x2*)(grp + 8 * lane) = u32x2{lo, hi};
      wave_lds_fence();
#pragma unroll
      for (int r = 7; r >= 0; --r) {
        const u32x2 t = cod[grp[64 * r + lane]];
        const uint32_t fr = t[0] & 0x1fffu, c = (t[0] >> 13) & 0xfffu, s = t[0] >> 25;
        const bool emit = (uint64_t)x >= ((uint64_t)fr << 20);
        const uint64_t bal = __ballot(emit);
        const uint32_t count = (uint32_t)__popcll(bal);
        // every lane stores, a lane that emits nothing at an offset the buffer drops: a fixed
        // number of stores a group, which keeps the compiler's wait for `next` exact
        __builtin_amdgcn_raw_buffer_store_b16(
            (unsigned short)(x & 0xffffu), w,
            emit ? (int)(rec + kWireScratchStream + 2 * (top - count + lanes_below(bal))) : (int)kWireOob, 0, 0);
        x = emit ? x >> 16 : x;
        top -= count;
        const uint32_t q = (uint32_t)(((uint64_t)__umulhi(t[1], x) + x) >> s);  // x / fr
        x = (q << kWireProbBits) + (x - q * fr) + c;
      }
    }
  }
  const uint32_t nwords = J * kWireLanes - top;
  __builtin_amdgcn_raw_buffer_store_b32(x, w, (int)(rec + kWireScratchStates + 4 * lane), 0, 0);
  const uint32_t rans = wire_rans_tile(n, nsym, nwords), plain = wire_raw_tile(n);
  raw_tile = raw_tile || rans >= plain;
  if (lane == 0) {
    const uint32_t size = raw_tile ? plain : rans;
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    __builtin_amdgcn_raw_buffer_store_b128(
        u32x4{raw_tile ? kWireModeRaw : (kWireModeRans | (nsym << 8)), raw_tile ? 0u : nwords, top, size}, w,
        (int)rec, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b32(size, w, (int)(kWireHeader + 4 * tile), 0, 0);
  }
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

// Pass 3: assemble each tile at its offset (header, then the raw words, or the sign-mantissa
// bytes, table, final states and stream from the working space). One wave per tile.
extern "C" __global__ __launch_bounds__(mo::kThreads) void mo_wire_encode_kernel(const char* raw, uint64_t raw_bytes,
                                                                                  char* wire, uint64_t wire_capacity) {
  using namespace mo;
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint64_t tile = (uint64_t)blockIdx.x * kWireTilesPerGroup + wave;
  if (tile >= wire_tiles(raw_bytes)) return;
  const uint32_t n = wire_tile_words(raw_bytes, tile);
  const char* src = raw + tile * kWireTileRaw;
  const __amdgpu_buffer_rsrc_t w = wire_rsrc(wire, wire_capacity);
  const uint32_t rec = (uint32_t)(wire_scratch_offset(raw_bytes) + tile * kWireScratchTile);
  const uint32_t toff = __builtin_amdgcn_raw_buffer_load_b32(w, (int)(kWireHeader + 4 * tile), 0, 0);
  const u32x4 r = __builtin_amdgcn_raw_buffer_load_b128(w, (int)rec, 0, 0);
  const uint32_t head = r[0], nwords = r[1], first = r[2];
  if (lane == 0) __builtin_amdgcn_raw_buffer_store_b128(u32x4{head, nwords, 0u, 0u}, w, (int)toff, 0, 0);
  const uint32_t body = toff + kWireTileHeader;
  if ((head & 3u) == kWireModeRaw) {
    for (uint32_t c = lane; c < n / 8; c += 64) {
      const uint4 v = ld16(src + 16 * (uint64_t)c);
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{v.x, v.y, v.z, v.w}, w, (int)(body + 16 * c), 0, 0);
    }
    return;
  }
  const uint32_t nsym = head >> 8;
  // sign-mantissa bytes: 16 words in, 16 bytes out a lane and round
  for (uint32_t c = lane; c < n / 16; c += 64) {
    const uint4 a = ld16(src + 32 * (uint64_t)c), b = ld16(src + 32 * (uint64_t)c + 16);
    uint32_t o[4] = {0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < 16; ++k) o[k >> 2] |= sign_mantissa_of(word_of(k < 8 ? a : b, k & 7)) << (8 * (k & 3));
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{o[0], o[1], o[2], o[3]}, w, (int)(body + 16 * c), 0, 0);
  }
  // table, zero-padded to 16 bytes
  const uint32_t tab = body + n, tab_words = (uint32_t)wire_align16(4 * nsym) / 4;
  for (uint32_t i = lane; i < tab_words; i += 64) {
    const uint32_t v = i < nsym ? __builtin_amdgcn_raw_buffer_load_b32(w, (int)(rec + kWireScratchTable + 4 * i), 0, 0) : 0u;
    __builtin_amdgcn_raw_buffer_store_b32(v, w, (int)(tab + 4 * i), 0, 0);
  }
  // final states
  const uint32_t states = tab + 4 * tab_words;
  __builtin_amdgcn_raw_buffer_store_b32(
      __builtin_amdgcn_raw_buffer_load_b32(w, (int)(rec + kWireScratchStates + 4 * lane), 0, 0), w,
      (int)(states + 4 * lane), 0, 0);
  // the stream's words, zero-padded to 16 bytes
  const uint32_t stream = states + 4 * kWireLanes, padded = (uint32_t)wire_align16(2 * nwords) / 2;
  for (uint32_t i = lane; i < padded; i += 64) {
    const unsigned short v =
        i < nwords ? __builtin_amdgcn_raw_buffer_load_b16(w, (int)(rec + kWireScratchStream + 2 * (first + i)), 0, 0)
                   : (unsigned short)0;
    __builtin_amdgcn_raw_buffer_store_b16(v, w, (int)(stream + 2 * i), 0, 0);
  }
}

// Decode a coded stream of `raw_bytes` into `raw`. Grid: max(ceil(tiles / 4), 1) workgroups, one
// wave per tile; the first workgroup also copies the raw tail. 6.5 KiB of LDS a wave: the table
// entries by rank, each slot's rank, a ring of the stream's next 512 words, and one group's
// exponents: state l decodes the tile's words 64 j + l, so the exponents of 8 rounds are 1 KiB of
// consecutive words, written out as one 16-byte store a lane. Reads go through
// a resource over [wire, wire + wire_bytes), and writes stay inside [raw, raw + raw_bytes)
// whatever the stream holds: a damaged header is clamped, and table values only index the
// wave's own LDS arrays.
extern "C" __global__ __launch_bounds__(mo::kThreads) void mo_wire_decode_kernel(const char* wire, uint64_t wire_bytes,
                                                                                  uint64_t raw_bytes, char* raw) {
  using namespace mo;
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  constexpr uint32_t kSlots = 1u << kWireProbBits, kRing = 512;
  __shared__ __attribute__((aligned(16))) unsigned char slot_rank[kWireWaves][kSlots];
  __shared__ uint32_t ranks[kWireWaves][256];  // table entry -> exponent | (f - 1) << 8 | c << 20
  __shared__ __attribute__((aligned(16))) unsigned short rings[kWireWaves][kRing];
  __shared__ __attribute__((aligned(16))) unsigned char groups[kWireWaves][8 * kWireLanes];
  const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const __amdgpu_buffer_rsrc_t w = wire_rsrc(wire, wire_bytes);
  if (blockIdx.x == 0) {
    const uint64_t tail = raw_bytes % kWireBlockBytes, tail_dst = wire_blocks(raw_bytes) * kWireBlockBytes;
    const uint64_t data_start = wire_data_start(raw_bytes);
    for (uint64_t i = threadIdx.x; i < tail; i += kThreads)
      st<kG>(raw + tail_dst + i, (uint8_t)__builtin_amdgcn_raw_buffer_load_b8(w, (int)(data_start + i), 0, 0));
  }
  const uint64_t tile = (uint64_t)blockIdx.x * kWireTilesPerGroup + wave;
  if (tile >= wire_tiles(raw_bytes)) return;
  const uint32_t n = wire_tile_words(raw_bytes, tile), J = n / kWireLanes;
  char* const dst = raw + tile * kWireTileRaw;
  const uint32_t toff = __builtin_amdgcn_raw_buffer_load_b32(w, (int)(kWireHeader + 4 * tile), 0, 0);
  const uint32_t head = __builtin_amdgcn_raw_buffer_load_b32(w, (int)toff, 0, 0);
  const uint32_t body = toff + kWireTileHeader;
  if ((head & 3u) != kWireModeRans) {
    for (uint32_t c = lane; c < n / 8; c += 64) {
      const mo_u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(w, (int)(body + 16 * c), 0, 0);
      st16(dst + 16 * (uint64_t)c, make_uint4(v.x, v.y, v.z, v.w));
    }
    return;
  }
  const uint32_t nsym = min((head >> 8) & 0x1ffu, 256u);
  MO_LDS unsigned char* const sr = (MO_LDS unsigned char*)slot_rank[wave];
  MO_LDS uint32_t* const rk = (MO_LDS uint32_t*)ranks[wave];
  MO_LDS unsigned short* const ring = (MO_LDS unsigned short*)rings[wave];
  // Table entries in rank order with their cumulative frequencies; each entry's first slot is
  // marked with its rank (rank 0 starts at slot 0, where every slot's mark starts).
  const uint32_t tab = body + n;
  for (uint32_t i = lane; i < kSlots / 4; i += 64) *(MO_LDS uint32_t*)(sr + 4 * i) = 0;
  wave_lds_fence();
  uint32_t carry = 0;
#pragma unroll
  for (uint32_t k = 0; k < 4; ++k) {
    const uint32_t r = 64 * k + lane;
    const uint32_t e = r < nsym ? __builtin_amdgcn_raw_buffer_load_b32(w, (int)(tab + 4 * r), 0, 0) : 0u;
    const uint32_t f = r < nsym ? min((e >> 8) & 0x1fffu, kSlots) : 0u;
    const uint32_t incl = wave_scan(f, lane), c = carry + incl - f;
    carry += (uint32_t)__shfl((int)incl, 63, 64);
    rk[r] = (e & 0xffu) | (((f - 1) & 0xfffu) << 8) | ((c & 0xfffu) << 20);
    if (f && c < kSlots) sr[c] = (unsigned char)r;
  }
  wave_lds_fence();
  // Every slot's rank: the last mark at or before it (marks rise with the slot), 64 slots a
  // round as a prefix maximum over the round's lanes and the rounds before.
  uint32_t before = 0;
  for (uint32_t row = 0; row < kSlots / 64; ++row) {
    const uint32_t slot = 64 * row + lane;
    const uint32_t cur = max(before, wave_scan_max_dpp(sr[slot]));
    before = (uint32_t)__builtin_amdgcn_readlane((int)cur, 63);
    sr[slot] = (unsigned char)cur;
  }
  // States, and the stream's first 512 words into the ring (word i at i % 512); `next` holds
  // the 2 words this lane brings in at the next refill.
  const uint32_t states = tab + (uint32_t)wire_align16(4 * nsym);
  uint32_t x = __builtin_amdgcn_raw_buffer_load_b32(w, (int)(states + 4 * lane), 0, 0);
  const uint32_t stream = states + 4 * kWireLanes;
#pragma unroll
  for (uint32_t q = 0; q < 4; ++q)
    *(MO_LDS uint32_t*)(ring + 128 * q + 2 * lane) =
        __builtin_amdgcn_raw_buffer_load_b32(w, (int)(stream + 256 * q + 4 * lane), 0, 0);
  uint32_t next = __builtin_amdgcn_raw_buffer_load_b32(w, (int)(stream + 1024 + 4 * lane), 0, 0);
  wave_lds_fence();
  uint32_t ptr = 0, wb = 0;  // words read so far; the first word the ring still holds
  // the group's sign-mantissa bytes (words 8 l .. 8 l + 7 of its 512), one group ahead
  MO_LDS unsigned char* const grp = (MO_LDS unsigned char*)groups[wave];
  const uint32_t ngroups = J / 8;
  u32x2 sm_next = __builtin_amdgcn_raw_buffer_load_b64(w, (int)(body + 8 * lane), 0, 0);
  for (uint32_t g = 0; g < ngroups; ++g) {
    const u32x2 sm = sm_next;
    sm_next = __builtin_amdgcn_raw_buffer_load_b64(w, (int)(body + 512 * (g + 1) + 8 * lane), 0, 0);  // a spare past the last
#pragma unroll
    for (uint32_t r = 0; r < 8; ++r) {
      const uint32_t slot = x & (kSlots - 1);
      const uint32_t t = rk[sr[slot]];
      x = (((t >> 8) & 0xfffu) + 1) * (x >> kWireProbBits) + slot - (t >> 20);
      const bool need = x < kWireStateLow;
      const uint64_t bal = __ballot(need);
      const uint32_t word = ring[(ptr + lanes_below(bal)) & (kRing - 1)];
      x = need ? (x << 16) | word : x;
      ptr += (uint32_t)__popcll(bal);
      grp[64 * r + lane] = (unsigned char)t;
      if (ptr - wb >= 128) {
        // words [wb, wb + 128) are consumed: their ring quarter takes words [wb + 512, wb + 640)
        *(MO_LDS uint32_t*)(ring + (wb & (kRing - 1)) + 2 * lane) = next;
        wb += 128;
        next = __builtin_amdgcn_raw_buffer_load_b32(w, (int)(stream + 2 * (wb + kRing) + 4 * lane), 0, 0);
        wave_lds_fence();
      }
    }
    wave_lds_fence();
    const u32x2 ex = *(const MO_LDS u32x2*)(grp + 8 * lane);
    uint32_t o[4];
#pragma unroll
    for (uint32_t k = 0; k < 8; k += 2) {
      uint32_t pair = 0;
#pragma unroll
      for (uint32_t h = 0; h < 2; ++h) {
        const uint32_t i = k + h;
        const uint32_t s = (sm[i >> 2] >> (8 * (i & 3))) & 0xffu, e = (ex[i >> 2] >> (8 * (i & 3))) & 0xffu;
        pair |= (((s & 0x80u) << 8) | (e << 7) | (s & 0x7fu)) << (16 * h);
      }
      o[k >> 1] = pair;
    }
    st16(dst + 1024 * (uint64_t)g + 16 * lane, make_uint4(o[0], o[1], o[2], o[3]));
    wave_lds_fence();  // the group buffer is read before the next group writes it
  }
}
