// Weight-only int8 linear for gfx950: the forward and input-gradient GEMMs of a frozen int8
// base (per-output-channel fp32 scales), on bf16 MFMA (v_mfma_f32_32x32x16_bf16). Replaces the
// Triton kernels of training/quant_kernels.py:100-228 (_int8_linear_forward_kernel,
// _int8_linear_backward_kernel): the int8 weight tile is decoded to bf16 on its way into LDS,
// exactly as those kernels decode it, bf16(q * bf16(scale)), and no full floating-point weight
// is ever built.
//
//   C[M][NC] = A[M][R] . W'^T, W' = decode(Bq), fp32 accumulation, optional bias, bf16 output
//   forward        : A = x [rows][in],  Bq = W [out][in],  NC = out, R = in,  scale[NC]
//   input gradient : A = dy [rows][out], Bq = W [out][in], NC = in,  R = out, scale[R]
//                    (kTransB: the reduction runs along Bq's rows; the tile is transposed into
//                     LDS so that both MFMA operands are read reduction-contiguous)
//
// Tiling (Cfg): a workgroup owns a kBM x kBC output tile, split over a grid of waves; each wave
// owns (kWM x 32) x (kWC x 32) as kWM x kWC MFMA 32x32 tiles. The reduction advances 64 per
// step through a double-buffered LDS (two A tiles kBM x 64 and two decoded weight tiles
// kBC x 64, bf16). Within a step (four 16-deep MFMA slices):
//   - the A tile one step ahead is copied global -> LDS by the DMA path of buffer loads
//     (buffer_load ... lds, 16 bytes a lane), with no register round trip;
//   - the weight tile one step ahead, loaded into registers a step earlier, is decoded into the
//     other LDS buffer during slices 0-2, while the weight tile two steps ahead is loaded into
//     the other register set (two sets, alternating by step parity);
//   - after slice 2 every wave has finished its reads of this step's buffers and its writes of
//     the next step's, so the barrier sits there and slice 3 overlaps the next step's first
//     fragment reads.
// Rows of 64 bf16 are stored as eight 16-byte chunks at position chunk ^ ((row ^ row / 8) % 8),
// which keeps the fragment reads (32 rows, one chunk), the decoded writes (strided rows) and the
// DMA rows free of bank conflicts. The input-gradient weight tile is read 8 reduction rows x
// kTn columns per lane; the decode packs pairs of reduction rows into each bf16x2, which
// transposes the tile on the way into LDS.
// Per-lane global offsets are fixed for the whole reduction; the reduction position is the
// scalar offset of the buffer instructions. Tiles are numbered in groups of kGroupM row tiles
// and then XCD-aware, so that the workgroups one XCD receives (blockIdx % 8) form a contiguous
// run of a few row and column tiles in that XCD's L2.
// MFMA 32x32x16 bf16 lane layout (checked on the device): A lane l holds row l%32,
// k = 8*(l/32)+j; B lane l holds column l%32, k = 8*(l/32)+j; D register r of lane l holds
// row 8*(r/4) + 4*(l/32) + r%4, column l%32. Within a step of 64, slice q gives lane half h the
// reduction indices 32 h + 8 q + j (LDS chunk 4 h + q of a row), in every kernel of this file,
// so that all tiles add the same products in the same order and a launch plan that splits the
// rows between tiles does not change results.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace mo_gemm {

constexpr int kBR = 64;     // reduction per step (one LDS row: eight 16-byte chunks)
constexpr int kGroupM = 8;  // row tiles per group of the tile numbering
constexpr int kXcds = 8;    // MI355X: workgroup i is dispatched to XCD i % 8

template <int BM, int BC, int WAVES_M, int WAVES_C>
struct Cfg {
  static constexpr int kBM = BM, kBC = BC, kWavesM = WAVES_M;
  static constexpr int kWaves = WAVES_M * WAVES_C, kThreads = 64 * kWaves;
  static constexpr int kRowsW = BM / WAVES_M, kColsW = BC / WAVES_C;
  static constexpr int kWM = kRowsW / 32, kWC = kColsW / 32;  // MFMA tiles per wave
  static constexpr int kDma = BM / 8 / kWaves;                 // 1 KiB A blocks per wave and step
  static constexpr int kF = BC * 4 / kThreads;                 // forward: 16-byte weight pieces a lane
  static constexpr int kFcols = kThreads / 4;                  // forward: columns per piece index
  static constexpr int kTn = 8 * BC / kThreads;                // transposed: weight columns a lane
  static_assert(kDma >= 1 && BM % (8 * kWaves) == 0, "A DMA blocks must divide over the waves");
  static_assert(kF >= 1 && kFcols % 64 == 0, "forward weight pieces");
  static_assert(kTn == 4 || kTn == 8, "transposed weight columns per lane");
  static_assert(kWM >= 1 && kWC >= 1 && kWM <= 4 && kWC <= 4, "wave tile");
};

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

#define MO_LDS __attribute__((address_space(3)))

typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Raw buffer descriptors (gfx9 word 3 = 0x00020000): a read at a vector offset at or beyond
// num_records returns zero (and moves no data) and a write there is dropped. The scalar offset
// is added to the address only, so every in-range vector offset must stay in range with it.
constexpr uint32_t kOob = 0x80000000u;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, 0x00020000);
}

// s_waitcnt immediate (gfx9): wait until at most n vector-memory operations are outstanding
// (lgkm: 0 = also wait for all LDS operations, 15 = do not).
constexpr int wait_vm(int n, int lgkm) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (lgkm << 8); }

// bf16(q * bf16(s)): the product of an int8 and a bf16 is exact in fp32; one rounding to bf16.
__device__ __forceinline__ __bf16 decode(uint32_t word, int byte, float s_bf16) {
  return (__bf16)((float)(int)(int8_t)(word >> (8 * byte)) * s_bf16);
}
__device__ __forceinline__ float bf16_round(float x) { return (float)(__bf16)x; }

// Element offset of (row, 16-byte chunk) in a swizzled LDS tile of rows of 64 bf16.
__device__ __forceinline__ int swz(int row, int chunk) { return row * kBR + ((chunk ^ ((row ^ (row >> 3)) & 7)) << 3); }

template <class G, bool kTransB, bool kFullR, int kVpm>
__device__ __forceinline__ void gemm_body(const __bf16* __restrict__ A, const int8_t* __restrict__ Bq,
                                          const float* __restrict__ scale, const __bf16* __restrict__ bias,
                                          __bf16* __restrict__ C, int M, int NC, int R, int tiles_m) {
  constexpr int kBM = G::kBM, kBC = G::kBC, kWM = G::kWM, kWC = G::kWC, kDma = G::kDma, kF = G::kF,
                kFcols = G::kFcols, kTn = G::kTn;
  // two buffers of each operand; distinct objects, so their accesses are known not to alias
  __shared__ __attribute__((aligned(16))) __bf16 lds_a0[kBM * kBR];
  __shared__ __attribute__((aligned(16))) __bf16 lds_a1[kBM * kBR];
  __shared__ __attribute__((aligned(16))) __bf16 lds_b0[kBC * kBR];
  __shared__ __attribute__((aligned(16))) __bf16 lds_b1[kBC * kBR];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % G::kWavesM, wc = wave / G::kWavesM;
  const int lr = lane & 31, h = lane >> 5;

  // ---- tile numbering: XCD-aware, then grouped ----
  const int tiles = gridDim.x;
  const int tiles_c = tiles / tiles_m;
  int t;
  {
    const int b = blockIdx.x, xcd = b % kXcds, idx = b / kXcds;
    const int per = tiles / kXcds, rem = tiles % kXcds;
    t = xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
  }
  const int group_tiles = kGroupM * tiles_c;
  const int first_m = (t / group_tiles) * kGroupM;
  const int gm = min(tiles_m - first_m, kGroupM);
  const int in_group = t % group_tiles;
  const int m0 = (first_m + in_group % gm) * kBM;
  const int c0 = (in_group / gm) * kBC;

  // ---- buffer descriptors over this tile's rows of A and columns of Bq ----
  // Rows past M and columns past NC fall outside the descriptors (vector offsets). With kFullR
  // (R % 64 == 0) the reduction position is the scalar offset and stays inside a row; a step
  // past R (the odd extra step) uses the empty descriptor. Without kFullR every load checks
  // its own reduction index and carries it in the vector offset.
  const rsrc_t ra_src = make_rsrc(A + (size_t)m0 * R, (uint32_t)(min(M - m0, kBM) * R * 2));
  const rsrc_t rb_src = kTransB ? make_rsrc(Bq + c0, (uint32_t)((R - 1) * NC + (NC - c0)))
                                : make_rsrc(Bq + (size_t)c0 * R, (uint32_t)(min(NC - c0, kBC) * R));
  const rsrc_t rs_src = make_rsrc(scale, (uint32_t)((kTransB ? R : NC) * 4));
  const rsrc_t none = make_rsrc(A, 0u);

  // A by DMA: wave w fills 1 KiB blocks w * kDma + j (8 rows each); lane i writes LDS slot i % 8
  // of row 8 * block + i / 8, which holds logical chunk slot ^ swizzle(row).
  uint32_t a_off[kDma];
  int a_k[kDma];
#pragma unroll
  for (int j = 0; j < kDma; ++j) {
    const int row = (wave * kDma + j) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((row ^ (row >> 3)) & 7);
    a_k[j] = 8 * c;
    a_off[j] = (uint32_t)(row * R + 8 * c) * 2;
  }
  // Bq forward ([NC][R]): 4 lanes per column (16 int8 each), columns tid / 4 + kFcols i.
  const int f_col = tid >> 2, f_part = tid & 3;
  uint32_t f_off[kF];
#pragma unroll
  for (int i = 0; i < kF; ++i) f_off[i] = (uint32_t)((f_col + kFcols * i) * R + 16 * f_part);
  // Bq transposed ([R][NC]): lane covers reduction rows 8 t_rg + 0..7 and columns
  // kTn t_ng + 0..kTn-1 (one load of kTn bytes per row).
  const int t_rg = tid / (kBC / kTn), t_ng = tid % (kBC / kTn);
  const bool t_col_ok = c0 + kTn * t_ng < NC;  // NC % 16 == 0: all kTn columns in or out

  // LDS element offsets, loop-invariant: fragment reads [i % 2][q] (i + 2 adds 64 rows, which
  // keeps the swizzle) and decoded weight writes
  int rd_a[2][4], rd_b[2][4];
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      rd_a[p][q] = swz(wm * G::kRowsW + 32 * p + lr, 4 * h + q);
      rd_b[p][q] = swz(wc * G::kColsW + 32 * p + lr, 4 * h + q);
    }
  int wr_b[8];  // forward: [0..1] = chunks 2 f_part + 0/1 of column f_col (i adds kFcols rows);
                // transposed: [c] = column kTn t_ng + c, chunk t_rg
#pragma unroll
  for (int c = 0; c < 8; ++c)
    wr_b[c] = kTransB ? swz(kTn * t_ng + (c % kTn), t_rg) : swz(f_col, 2 * f_part + (c & 1));

  // weight tile registers, two sets (tile t in set t % 2)
  u32x4 rf[2][kF];             // forward weight bytes
  uint32_t rt[2][8][kTn / 4];  // transposed weight bytes
  float st[2][8];              // transposed: bf16-rounded scales of the lane's reduction rows
  float sf[kF];                // forward: bf16-rounded scales of the lane's columns
  if (!kTransB) {
#pragma unroll
    for (int i = 0; i < kF; ++i) {
      const int n = c0 + f_col + kFcols * i;
      sf[i] = bf16_round(__builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(rs_src, n < NC ? n * 4 : (int)kOob, 0, 0)));
    }
  }

  // A tile at reduction r0 straight into LDS.
  auto dma_a = [&](MO_LDS __bf16* As, int r0) {
    const rsrc_t src = r0 < R ? ra_src : none;
#pragma unroll
    for (int j = 0; j < kDma; ++j) {
      MO_LDS void* dst = (MO_LDS void*)(As + (wave * kDma + j) * 512);
      if (kFullR)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(src, dst, 16, a_off[j], r0 * 2, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(src, dst, 16, (r0 + a_k[j] < R) ? a_off[j] + r0 * 2 : kOob, 0, 0,
                                                 0);
    }
  };

  // Weight loads of the tile at reduction r0 into register set S.
  auto load = [&](auto set, int r0) {
    constexpr int S = decltype(set)::value;
    const rsrc_t src = r0 < R ? rb_src : none;
    if (!kTransB) {
#pragma unroll
      for (int i = 0; i < kF; ++i)
        rf[S][i] = kFullR ? __builtin_amdgcn_raw_buffer_load_b128(src, (int)f_off[i], r0, 0)
                          : __builtin_amdgcn_raw_buffer_load_b128(
                                src, (r0 + 16 * f_part < R) ? (int)(f_off[i] + r0) : (int)kOob, 0, 0);
    } else {
      const rsrc_t ssrc = r0 < R ? rs_src : none;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int rl = 8 * t_rg + i;
        const bool ok = kFullR || r0 + rl < R;
        const uint32_t off = t_col_ok ? (uint32_t)(rl * NC + kTn * t_ng) : kOob;
        const int voff = kFullR ? (int)off : (ok ? (int)(off + (uint32_t)(r0 * NC)) : (int)kOob);
        const int soff = kFullR ? r0 * NC : 0;
        if (kTn == 8) {
          const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(src, voff, soff, 0);
          rt[S][i][0] = v[0];
          rt[S][i][kTn / 8] = v[1];
        } else {
          rt[S][i][0] = __builtin_amdgcn_raw_buffer_load_b32(src, voff, soff, 0);
        }
        const int sv = kFullR ? rl * 4 : (ok ? (r0 + rl) * 4 : (int)kOob);
        st[S][i] = bf16_round(
            __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ssrc, sv, kFullR ? r0 * 4 : 0, 0)));
      }
    }
  };
  constexpr int kLoads = kTransB ? 16 : kF;  // vector-memory operations of one load()

  // Decode register set S into an LDS buffer, part p of 3 (p = -1: all parts).
  auto stage = [&](auto set, MO_LDS __bf16* Bs, int p) {
    constexpr int S = decltype(set)::value;
    if (!kTransB) {
#pragma unroll
      for (int i = 0; i < kF; ++i) {
        if (p >= 0 && i * 3 / kF != p) continue;
        bf16x8 lo, hi;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          lo[j] = decode(rf[S][i][j >> 2], j & 3, sf[i]);
          hi[j] = decode(rf[S][i][2 + (j >> 2)], j & 3, sf[i]);
        }
        *(MO_LDS bf16x8*)(Bs + wr_b[0] + i * kFcols * kBR) = lo;
        *(MO_LDS bf16x8*)(Bs + wr_b[1] + i * kFcols * kBR) = hi;
      }
    } else {
#pragma unroll
      for (int c = 0; c < kTn; ++c) {
        if (p >= 0 && c * 3 / kTn != p) continue;
        bf16x8 v;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = decode(rt[S][i][c >> 2], c & 3, st[S][i]);
        *(MO_LDS bf16x8*)(Bs + wr_b[c]) = v;
      }
    }
  };

  // Instruction interleave of one slice (kWM x kWC MFMAs): fragment reads first, two per MFMA;
  // in slice 0 the A DMA (with its M0 writes) and the weight loads; in slices 0-2 the decode
  // VALU spread over the MFMAs and the decoded-tile LDS writes last.
  auto schedule_slice = [&](int q) {
    constexpr int kMfma = 0x008, kValu = 0x002, kDsRead = 0x100, kDsWrite = 0x200, kVmem = 0x020, kSalu = 0x004;
    constexpr int kMf = kWM * kWC, kReadSlots = (kWM + kWC + 1) / 2;
    constexpr int kWrites = kTransB ? 3 : 2;
    if (kMf < 2 + kDma) return;  // too few MFMAs to interleave: leave it to the scheduler
#pragma unroll
    for (int m = 0; m < kMf; ++m) {
      __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
      if (m < kReadSlots) __builtin_amdgcn_sched_group_barrier(kDsRead, 2, 0);
      if (q == 0 && m >= 1 && m < 1 + kDma) {
        __builtin_amdgcn_sched_group_barrier(kSalu, 2, 0);
        __builtin_amdgcn_sched_group_barrier(kVmem, 1, 0);
      }
      if (q == 0 && m == 1 + kDma) __builtin_amdgcn_sched_group_barrier(kVmem, kLoads, 0);
      if (q < 3 && m >= kReadSlots) __builtin_amdgcn_sched_group_barrier(kValu, kVpm, 0);
      if (q < 3 && m >= kMf - kWrites - 1 && m < kMf - 1) __builtin_amdgcn_sched_group_barrier(kDsWrite, 1, 0);
    }
  };

  f32x16 acc[kWM][kWC];
#pragma unroll
  for (int i = 0; i < kWM; ++i)
#pragma unroll
    for (int j = 0; j < kWC; ++j) acc[i][j] = f32x16{};

  bf16x8 fa[2][kWM], fb[2][kWC];  // fragments of two slices
  auto read_frags = [&](const MO_LDS __bf16* As, const MO_LDS __bf16* Bs, int q, int slot) {
#pragma unroll
    for (int i = 0; i < kWM; ++i) fa[slot][i] = *(const MO_LDS bf16x8*)(As + rd_a[i & 1][q] + (i >> 1) * 64 * kBR);
#pragma unroll
    for (int j = 0; j < kWC; ++j) fb[slot][j] = *(const MO_LDS bf16x8*)(Bs + rd_b[j & 1][q] + (j >> 1) * 64 * kBR);
  };

  // One reduction step over (Ac, Bc); r_next is the reduction offset of the next step.
  auto step = [&](const MO_LDS __bf16* Ac, const MO_LDS __bf16* Bc, MO_LDS __bf16* An, MO_LDS __bf16* Bn, int r_next,
                  auto stage_set, auto load_set) {
#pragma unroll
    for (int q = 0; q < kBR / 16; ++q) {
      const int cq = q & 1, nq = cq ^ 1;
      if (q < 3)
        read_frags(Ac, Bc, q + 1, nq);
      else
        read_frags(An, Bn, 0, nq);  // after the barrier: the next step's buffers are complete
      if (q == 0) {
        dma_a(An, r_next);
        load(load_set, r_next + kBR);
      }
      if (q < 3) stage(stage_set, Bn, q);
#pragma unroll
      for (int i = 0; i < kWM; ++i)
#pragma unroll
        for (int j = 0; j < kWC; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[cq][i], fb[cq][j], acc[i][j], 0, 0, 0);
      schedule_slice(q);
      __builtin_amdgcn_sched_barrier(0);
      if (q == 2) {
        // this wave's A DMA has landed (only its weight loads, issued after it, may be in
        // flight) and its LDS reads and writes are done; then the whole workgroup
        __builtin_amdgcn_s_waitcnt(wait_vm(kLoads, 0));
        __syncthreads();
      }
    }
  };

  using set0 = std::integral_constant<int, 0>;
  using set1 = std::integral_constant<int, 1>;
  typedef MO_LDS __bf16* lp;
  typedef const MO_LDS __bf16* clp;
  const int steps = (R + kBR - 1) / kBR;
  dma_a((lp)lds_a0, 0);
  load(set0{}, 0);
  stage(set0{}, (lp)lds_b0, -1);
  load(set1{}, kBR);  // past R when steps == 1: zeros
  __builtin_amdgcn_s_waitcnt(wait_vm(kLoads, 0));
  __syncthreads();
  read_frags((clp)lds_a0, (clp)lds_b0, 0, 0);
  // Steps run in pairs (one per buffer) with no branch between them; an odd step count gets one
  // more step over tiles past R, which read as zeros and add nothing.
  for (int s = 0; s < steps; s += 2) {
    step((clp)lds_a0, (clp)lds_b0, (lp)lds_a1, (lp)lds_b1, (s + 1) * kBR, set1{}, set0{});
    step((clp)lds_a1, (clp)lds_b1, (lp)lds_a0, (lp)lds_b0, (s + 2) * kBR, set0{}, set1{});
  }

  // ---- epilogue: bias, bf16, store ----
  // Lanes hold consecutive columns, so each store instruction writes two contiguous 64-byte
  // row pieces.
  const rsrc_t rc_src = make_rsrc(C + (size_t)m0 * NC, (uint32_t)(min(M - m0, kBM) * NC * 2));
  // no bias: an empty descriptor, every read returns zero
  const rsrc_t rbias_src = make_rsrc(bias, bias ? (uint32_t)NC * 2 : 0u);
#pragma unroll
  for (int j = 0; j < kWC; ++j) {
    const int col = c0 + wc * G::kColsW + j * 32 + lr;
    const bool col_ok = col < NC;
    const float b = (float)__builtin_bit_cast(
        __bf16, (unsigned short)__builtin_amdgcn_raw_buffer_load_b16(rbias_src, col_ok ? col * 2 : (int)kOob, 0, 0));
#pragma unroll
    for (int i = 0; i < kWM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = wm * G::kRowsW + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);  // rows past M: outside
        const __bf16 v = (__bf16)(acc[i][j][r] + b);
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, v), rc_src,
                                              col_ok ? (int)((uint32_t)(row * NC + col) * 2) : (int)kOob, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);  // one accumulator tile at a time (register pressure)
    }
  }
}

// ---- weight in registers ----
// C[M][N] = A[M][K] . W'^T with Bq [N][K] int8 (the reduction contiguous), W' = decode(Bq), fp32
// accumulation, bf16 output (+ bias). Scales per column (forward: Bq is the weight, scale[N]) or,
// with kScaleK, per reduction index (input gradient: Bq is the transposed weight, scale[K]).
// K % 64 == 0; rows past M and columns past N read zeros and store nothing.
// With kSplit the launch holds `splits` workgroups per tile, each over `split_steps` steps of
// the reduction (the last over what remains): item t of the XCD-aware numbering takes split
// t / tiles of tile t % tiles, and stores its fp32 sums, unrounded and without bias, to plane
// `split` of P ([splits][M][N]); mo_int8_split_reduce then adds the planes in split order.
//
// A workgroup owns a 256 x 256 tile with four waves side by side: wave w owns all 256 rows and
// columns 64 w .. 64 w + 63, as 8 x 2 MFMA 32x32x16 tiles (256 accumulators). A goes global ->
// LDS by the buffer-load DMA path, double-buffered and swizzled as in gemm_body; each wave reads
// every row of it. B never enters LDS: each lane loads the int8 bytes of its two columns
// straight into registers and decodes them there into the MFMA's B fragment, so every column is
// decoded by one wave only and the LDS carries A alone (A fragment reads, 8 KiB a wave and
// slice, plus the DMA).
// Reduction order: in a step of 64, lane half h (lanes 32 h ..) takes k = 32 h + 8 q + j in
// slice q (j = 0..7), for A's fragments and B's alike. A lane's weight bytes of a step are then
// 32 contiguous bytes of its column: two 16-byte halves, half p serving slices 2 p and 2 p + 1.
// Within step s, slice q reads the A fragments and decodes the B fragments of slice q + 1 (of
// step s + 1 when q = 3) while slice q's MFMAs run. Half 0 of a column's bytes of step s is
// free once slice 1 is decoded (during slice 0), half 1 once slice 3 is (during slice 2): half 0
// of step s + 2 is loaded in slice 1 and half 1 in slice 3, into the register set of step s
// (two sets by step parity). A has three LDS buffers (96 KiB): the tile of step s + 2 (and with
// kScaleK its 64 scales) is DMA'd in slice 0 of step s into the buffer step s - 1 used, so a
// DMA has six slices to land. After slice 2 each wave waits for everything but the loads of
// step s + 2, then the workgroup meets at the one barrier of the step: slice 3 already reads
// the next step's buffer, and every wave is done with step s - 1's before its refill.
template <bool kScaleK, bool kSplit>
__device__ __forceinline__ void ws_body(const __bf16* __restrict__ A, const int8_t* __restrict__ Bq,
                                        const float* __restrict__ scale, const __bf16* __restrict__ bias,
                                        __bf16* __restrict__ C, float* __restrict__ P, int M, int N, int K,
                                        int tiles_m, int splits, int split_steps) {
  constexpr int kBM = 256, kBN = 256, kWaves = 4, kDma = kBM / 8 / kWaves;  // 8 x 1 KiB A blocks per wave
  // three buffers as distinct objects, chosen at compile time: the compiler can then tell the
  // buffer a DMA writes from the ones being read, and waits only for the DMA that was asked for
  __shared__ __attribute__((aligned(16))) __bf16 lds_a0[kBM * kBR];
  __shared__ __attribute__((aligned(16))) __bf16 lds_a1[kBM * kBR];
  __shared__ __attribute__((aligned(16))) __bf16 lds_a2[kBM * kBR];
  __shared__ __attribute__((aligned(16))) float lds_s0[kBR];
  __shared__ __attribute__((aligned(16))) float lds_s1[kBR];
  __shared__ __attribute__((aligned(16))) float lds_s2[kBR];
  auto abuf = [&](auto i) -> MO_LDS __bf16* {
    constexpr int I = decltype(i)::value;
    return (MO_LDS __bf16*)(I == 0 ? lds_a0 : I == 1 ? lds_a1 : lds_a2);
  };
  auto sbuf = [&](auto i) -> MO_LDS float* {
    constexpr int I = decltype(i)::value;
    return (MO_LDS float*)(I == 0 ? lds_s0 : I == 1 ? lds_s1 : lds_s2);
  };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 31, h = lane >> 5;

  // ---- tile numbering: XCD-aware, then grouped (as gemm_body) ----
  const int items = gridDim.x;
  const int tiles = kSplit ? items / splits : items;
  const int tiles_c = tiles / tiles_m;
  int t;
  {
    const int b = blockIdx.x, xcd = b % kXcds, idx = b / kXcds;
    const int per = items / kXcds, rem = items % kXcds;
    t = xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
  }
  const int split = kSplit ? t / tiles : 0;
  if (kSplit) t -= split * tiles;
  const int group_tiles = kGroupM * tiles_c;
  const int first_m = (t / group_tiles) * kGroupM;
  const int gm = min(tiles_m - first_m, kGroupM);
  const int in_group = t % group_tiles;
  const int m0 = (first_m + in_group % gm) * kBM;
  const int c0 = (in_group / gm) * kBN;
  // this workgroup's reduction: [k0, k0 + klen); the descriptors start at k0
  const int k0 = kSplit ? split * split_steps * kBR : 0;
  const int klen = kSplit ? min(split_steps * kBR, K - k0) : K;

  const rsrc_t ra_src = make_rsrc(A + (size_t)m0 * K + k0, (uint32_t)((min(M - m0, kBM) * K - k0) * 2));
  const rsrc_t rb_src = make_rsrc(Bq + (size_t)c0 * K + k0, (uint32_t)(min(N - c0, kBN) * K - k0));
  const rsrc_t rs_src = kScaleK ? make_rsrc(scale + k0, (uint32_t)((K - k0) * 4)) : make_rsrc(scale, (uint32_t)(N * 4));

  // A by DMA: wave w fills 1 KiB blocks w * kDma + j (8 rows each), as gemm_body.
  uint32_t a_off[kDma];
#pragma unroll
  for (int j = 0; j < kDma; ++j) {
    const int row = (wave * kDma + j) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((row ^ (row >> 3)) & 7);
    a_off[j] = (uint32_t)(row * K + 8 * c) * 2;
  }
  // A fragment of slice q, row tile i: row 32 i + lr, chunk 4 h + q (i + 2 keeps the swizzle)
  int rd_a[2][4];
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int q = 0; q < 4; ++q) rd_a[p][q] = swz(32 * p + lr, 4 * h + q);
  // B: column tile ct of the wave holds column 64 w + 32 ct + lr of the tile
  uint32_t b_off[2];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) b_off[ct] = (uint32_t)((64 * wave + 32 * ct + lr) * K + 32 * h);
  float sf[2] = {0.f, 0.f};  // forward: bf16-rounded column scales
  if (!kScaleK) {
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const int n = c0 + 64 * wave + 32 * ct + lr;
      sf[ct] = bf16_round(__builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(rs_src, n < N ? n * 4 : (int)kOob, 0, 0)));
    }
  }

  auto dma = [&](MO_LDS __bf16* As, MO_LDS float* Ss, int r0) {
    const rsrc_t src = r0 < klen ? ra_src : make_rsrc(A, 0u);
#pragma unroll
    for (int j = 0; j < kDma; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(src, (MO_LDS void*)(As + (wave * kDma + j) * 512), 16, a_off[j],
                                               r0 * 2, 0, 0);
    if (kScaleK)  // the step's 64 scales, the same bytes from every wave
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r0 < klen ? rs_src : make_rsrc(A, 0u), (MO_LDS void*)Ss, 4, lane * 4,
                                               r0 * 4, 0, 0);
  };
  constexpr int kDmaOps = kDma + (kScaleK ? 1 : 0);

  // weight bytes: raw[set][ct][half], loaded for step r0 / 64 (past K: zeros)
  u32x4 raw[2][2][2];
  auto load_half = [&](auto set, auto half, int r0) {
    constexpr int S = decltype(set)::value, H = decltype(half)::value;
    const rsrc_t src = r0 < klen ? rb_src : make_rsrc(Bq, 0u);
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
      raw[S][ct][H] = __builtin_amdgcn_raw_buffer_load_b128(src, (int)(b_off[ct] + 16 * H), r0, 0);
  };

  bf16x8 fa[2][8], fb[2][2];  // fragments of two slices
  auto read_a = [&](const MO_LDS __bf16* As, int q, int slot) {
#pragma unroll
    for (int i = 0; i < 8; ++i) fa[slot][i] = *(const MO_LDS bf16x8*)(As + rd_a[i & 1][q] + (i >> 1) * 64 * kBR);
  };
  // B fragments of slice q from register set S (scales of that step in Ss when kScaleK)
  auto decode_b = [&](auto set, const MO_LDS float* Ss, int q, int slot) {
    constexpr int S = decltype(set)::value;
    float sk[8];
    if (kScaleK) {
      const float4 lo = *(const MO_LDS float4*)(Ss + 32 * h + 8 * q);
      const float4 hi = *(const MO_LDS float4*)(Ss + 32 * h + 8 * q + 4);
      sk[0] = lo.x, sk[1] = lo.y, sk[2] = lo.z, sk[3] = lo.w, sk[4] = hi.x, sk[5] = hi.y, sk[6] = hi.z, sk[7] = hi.w;
#pragma unroll
      for (int j = 0; j < 8; ++j) sk[j] = bf16_round(sk[j]);
    }
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const u32x4 v = q < 2 ? raw[S][ct][0] : raw[S][ct][1];
      const uint32_t w0 = v[2 * (q & 1)], w1 = v[2 * (q & 1) + 1];
      bf16x8 f;
#pragma unroll
      for (int j = 0; j < 8; ++j) f[j] = decode(j < 4 ? w0 : w1, j & 3, kScaleK ? sk[j] : sf[ct]);
      fb[slot][ct] = f;
    }
  };

  f32x16 acc[8][2];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) acc[i][ct] = f32x16{};

  // Instruction interleave of one slice: an MFMA, then one of the next slice's 8 A fragment
  // reads behind each of the first 8 MFMAs, the decode VALU (about 40 ops, 56 with per-k
  // scales) spread over all 16, the DMA (with its M0 writes) in slice 0 and the weight loads in
  // slices 1 and 3.
  auto schedule = [&](int q) {
    constexpr int kMfma = 0x008, kValu = 0x002, kDsRead = 0x100, kVmem = 0x020, kSalu = 0x004;
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
      if (m < 8) __builtin_amdgcn_sched_group_barrier(kDsRead, 1, 0);
      if (kScaleK && m == 0) __builtin_amdgcn_sched_group_barrier(kDsRead, 2, 0);
      if (q == 0 && m >= 1 && m < 1 + kDmaOps) {
        __builtin_amdgcn_sched_group_barrier(kSalu, 2, 0);
        __builtin_amdgcn_sched_group_barrier(kVmem, 1, 0);
      }
      if ((q == 1 || q == 3) && m == 10) __builtin_amdgcn_sched_group_barrier(kVmem, 2, 0);
      __builtin_amdgcn_sched_group_barrier(kValu, kScaleK ? 4 : 3, 0);
    }
  };

  // Step s over buffer b (A and scales of step s), b1 = buffer of step s + 1, b2 = buffer step
  // s + 2 is DMA'd into; weights of step s in set Cur, of step s + 1 in set Nxt; r0 = 64 s.
  auto step = [&](auto b, auto b1, auto b2, int r0, auto cur, auto nxt) {
    using H0 = std::integral_constant<int, 0>;
    using H1 = std::integral_constant<int, 1>;
    const MO_LDS __bf16* Ac = abuf(b);
    const MO_LDS __bf16* An = abuf(b1);
    const MO_LDS float* Sc = sbuf(b);
    const MO_LDS float* Sn = sbuf(b1);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int cq = q & 1, nq = cq ^ 1;
      if (q < 3) {
        read_a(Ac, q + 1, nq);
        decode_b(cur, Sc, q + 1, nq);
      } else {
        read_a(An, 0, nq);  // after the barrier: the next step's A and scales are in LDS
        decode_b(nxt, Sn, 0, nq);
      }
      if (q == 0) dma(abuf(b2), sbuf(b2), r0 + 2 * kBR);
      if (q == 1) load_half(cur, H0{}, r0 + 2 * kBR);
      if (q == 3) load_half(cur, H1{}, r0 + 2 * kBR);
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
          acc[i][ct] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[cq][i], fb[cq][ct], acc[i][ct], 0, 0, 0);
      schedule(q);
      __builtin_amdgcn_sched_barrier(0);
      if (q == 2) {
        // landed: all but step s + 2's DMA (slice 0) and half-0 loads (slice 1), so step s + 1's
        // A, scales and both weight halves; then the whole workgroup (every wave is done with
        // the buffer step s + 3 will refill)
        __builtin_amdgcn_s_waitcnt(wait_vm(kDmaOps + 2, 0));
        __syncthreads();
      }
    }
  };

  using set0 = std::integral_constant<int, 0>;
  using set1 = std::integral_constant<int, 1>;
  using H0 = std::integral_constant<int, 0>;
  using H1 = std::integral_constant<int, 1>;
  typedef const MO_LDS __bf16* clp;
  typedef const MO_LDS float* csp;
  const int steps = klen / kBR;
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  using B2 = std::integral_constant<int, 2>;
  // prologue: steps 0 and 1 (A, scales and weights); step 0 must have landed
  dma(abuf(B0{}), sbuf(B0{}), 0);
  load_half(set0{}, H0{}, 0);
  load_half(set0{}, H1{}, 0);
  dma(abuf(B1{}), sbuf(B1{}), kBR);
  load_half(set1{}, H0{}, kBR);
  load_half(set1{}, H1{}, kBR);
  __builtin_amdgcn_s_waitcnt(wait_vm(kDmaOps + 4, 0));
  __syncthreads();
  read_a((clp)lds_a0, 0, 0);
  decode_b(set0{}, (csp)lds_s0, 0, 0);
  // Steps in sixes: two register sets by step parity, three LDS buffers by step modulo 3. Steps
  // past the reduction (up to five at the end) read zeros and add nothing.
  for (int s = 0; s < steps; s += 6) {
    step(B0{}, B1{}, B2{}, (s + 0) * kBR, set0{}, set1{});
    step(B1{}, B2{}, B0{}, (s + 1) * kBR, set1{}, set0{});
    step(B2{}, B0{}, B1{}, (s + 2) * kBR, set0{}, set1{});
    step(B0{}, B1{}, B2{}, (s + 3) * kBR, set1{}, set0{});
    step(B1{}, B2{}, B0{}, (s + 4) * kBR, set0{}, set1{});
    step(B2{}, B0{}, B1{}, (s + 5) * kBR, set1{}, set0{});
  }

  if (kSplit) {
    // ---- epilogue: the fp32 sums into plane `split` of P (rows past M, columns past N outside) ----
    float* Ps = P + (size_t)split * M * N;
    const rsrc_t rp_src = make_rsrc(Ps + (size_t)m0 * N, (uint32_t)(min(M - m0, kBM) * N * 4));
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const int col = c0 + 64 * wave + 32 * ct + lr;
      const bool col_ok = col < N;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          // the element read into a scalar first: a bit cast of the vector element itself
          // reads the vector's first element
          const float v = acc[i][ct][r];
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned int, v), rp_src,
                                                col_ok ? (int)((uint32_t)(row * N + col) * 4) : (int)kOob, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    return;
  }
  // ---- epilogue: bias, bf16, store (rows past M and columns past N fall outside) ----
  // Lane half h of column tile ct holds rows 4 h + .. of columns 32 ct + lr. One
  // v_permlane32_swap per pair of values gives lane l the value of row `row0` (from h = 0)
  // and column l of the wave's 64 in one register, of row `row0 + 4` (from h = 1) in the
  // other: each store instruction then writes one full 128-byte row piece.
  const rsrc_t rc_src = make_rsrc(C + (size_t)m0 * N, (uint32_t)(min(M - m0, kBM) * N * 2));
  const rsrc_t rbias_src = make_rsrc(bias, bias ? (uint32_t)N * 2 : 0u);
  float b[2];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    const int col = c0 + 64 * wave + 32 * ct + lr;
    b[ct] = (float)__builtin_bit_cast(
        __bf16, (unsigned short)__builtin_amdgcn_raw_buffer_load_b16(rbias_src, col < N ? col * 2 : (int)kOob, 0, 0));
  }
  const int out_col = c0 + 64 * wave + lane;  // after the swap: column `lane` of the wave's 64
  const bool out_ok = out_col < N;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row0 = i * 32 + 8 * (r >> 2) + (r & 3);
      const unsigned int x = __builtin_bit_cast(unsigned short, (__bf16)(acc[i][0][r] + b[0]));
      const unsigned int y = __builtin_bit_cast(unsigned short, (__bf16)(acc[i][1][r] + b[1]));
      // x' = (x lanes 0-31, y lanes 0-31): row0; y' = (x lanes 32-63, y lanes 32-63): row0 + 4
      const auto sw = __builtin_amdgcn_permlane32_swap(x, y, false, false);
      __builtin_amdgcn_raw_buffer_store_b16((unsigned short)sw[0], rc_src,
                                            out_ok ? (int)((uint32_t)(row0 * N + out_col) * 2) : (int)kOob, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b16((unsigned short)sw[1], rc_src,
                                            out_ok ? (int)((uint32_t)((row0 + 4) * N + out_col) * 2) : (int)kOob, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Configurations: forward 256 x 256 over 2 x 4 waves (two waves a SIMD); input gradient
// 256 x 256 over 2 x 2 waves; both directions 128 x 128 over 2 x 2 waves for grids too small
// or too ragged for the large tile.
using FwdLarge = Cfg<256, 256, 2, 4>;
using BwdLarge = Cfg<256, 256, 2, 2>;
using Small = Cfg<128, 128, 2, 2>;

}  // namespace mo_gemm

#define MO_GEMM_FWD(NAME, G, FULL, VPM)                                                                            \
  extern "C" __global__ __launch_bounds__(G::kThreads) void NAME(const __bf16* A, const int8_t* Bq,              \
                                                                 const float* scale, const __bf16* bias,         \
                                                                 __bf16* C, int M, int NC, int R, int tiles_m) { \
    mo_gemm::gemm_body<G, false, FULL, VPM>(A, Bq, scale, bias, C, M, NC, R, tiles_m);                          \
  }
#define MO_GEMM_BWD(NAME, G, FULL, VPM)                                                                          \
  extern "C" __global__ __launch_bounds__(G::kThreads) void NAME(const __bf16* A, const int8_t* Bq,            \
                                                                 const float* scale, __bf16* C, int M, int NC, \
                                                                 int R, int tiles_m) {                         \
    mo_gemm::gemm_body<G, true, FULL, VPM>(A, Bq, scale, nullptr, C, M, NC, R, tiles_m);                       \
  }

extern "C" __global__ __launch_bounds__(256) void mo_int8_ws_fwd(const __bf16* A, const int8_t* Bq, const float* scale,
                                                                   const __bf16* bias, __bf16* C, int M, int N, int K,
                                                                   int tiles_m) {
  mo_gemm::ws_body<false, false>(A, Bq, scale, bias, C, nullptr, M, N, K, tiles_m, 1, 0);
}
extern "C" __global__ __launch_bounds__(256) void mo_int8_ws_kscale(const __bf16* A, const int8_t* Bq,
                                                                     const float* scale, __bf16* C, int M, int N,
                                                                     int K, int tiles_m) {
  mo_gemm::ws_body<true, false>(A, Bq, scale, nullptr, C, nullptr, M, N, K, tiles_m, 1, 0);
}
// The same with the reduction split over `splits` workgroups per tile (fp32 planes into P).
extern "C" __global__ __launch_bounds__(256) void mo_int8_ws_fwd_split(const __bf16* A, const int8_t* Bq,
                                                                         const float* scale, float* P, int M, int N,
                                                                         int K, int tiles_m, int splits,
                                                                         int split_steps) {
  mo_gemm::ws_body<false, true>(A, Bq, scale, nullptr, nullptr, P, M, N, K, tiles_m, splits, split_steps);
}
extern "C" __global__ __launch_bounds__(256) void mo_int8_ws_kscale_split(const __bf16* A, const int8_t* Bq,
                                                                            const float* scale, float* P, int M,
                                                                            int N, int K, int tiles_m, int splits,
                                                                            int split_steps) {
  mo_gemm::ws_body<true, true>(A, Bq, scale, nullptr, nullptr, P, M, N, K, tiles_m, splits, split_steps);
}

// C[rows][cols] = bf16(P[0] + P[1] + ... + P[splits - 1] (+ bias)), the planes of a split
// reduction added in split order, so the result does not depend on which workgroup finished
// first. One lane per 8 consecutive elements (cols % 16 == 0); bias may be null.
extern "C" __global__ __launch_bounds__(256) void mo_int8_split_reduce(const float* P, const __bf16* bias, __bf16* C,
                                                                        uint32_t rows, uint32_t cols,
                                                                        uint32_t splits) {
  using f32x4 = float __attribute__((ext_vector_type(4)));
  const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if (i >= (uint64_t)rows * (cols / 8)) return;
  const uint64_t e = i * 8, plane = (uint64_t)rows * cols;
  f32x4 lo = *(const f32x4*)(P + e), hi = *(const f32x4*)(P + e + 4);
  for (uint32_t s = 1; s < splits; ++s) {
    lo += *(const f32x4*)(P + s * plane + e);
    hi += *(const f32x4*)(P + s * plane + e + 4);
  }
  const uint32_t col = (uint32_t)(e % cols);
  mo_gemm::u32x4 out;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float a = k < 2 ? lo[2 * k] : hi[2 * k - 4], b = k < 2 ? lo[2 * k + 1] : hi[2 * k - 3];
    if (bias) {
      a += (float)bias[col + 2 * k];
      b += (float)bias[col + 2 * k + 1];
    }
    out[k] = (uint32_t)__builtin_bit_cast(unsigned short, (__bf16)a) |
             ((uint32_t)__builtin_bit_cast(unsigned short, (__bf16)b) << 16);
  }
  *(mo_gemm::u32x4*)(C + e) = out;
}

// full: R % 64 == 0; _tail: any multiple of 16
MO_GEMM_FWD(mo_int8_linear_fwd_large, mo_gemm::FwdLarge, true, 6)
MO_GEMM_FWD(mo_int8_linear_fwd_large_tail, mo_gemm::FwdLarge, false, 6)
MO_GEMM_FWD(mo_int8_linear_fwd_small, mo_gemm::Small, true, 6)
MO_GEMM_FWD(mo_int8_linear_fwd_small_tail, mo_gemm::Small, false, 6)
MO_GEMM_BWD(mo_int8_linear_bwd_large, mo_gemm::BwdLarge, true, 6)
MO_GEMM_BWD(mo_int8_linear_bwd_large_tail, mo_gemm::BwdLarge, false, 6)
MO_GEMM_BWD(mo_int8_linear_bwd_small, mo_gemm::Small, true, 6)
MO_GEMM_BWD(mo_int8_linear_bwd_small_tail, mo_gemm::Small, false, 6)

// The decoded weight W' = bf16(q * bf16(scale)) written out whole, for calls with enough rows
// that one decode per call costs less than the fused kernels' in-tile decode: a library GEMM
// then takes W' as a plain bf16 operand. One lane per 16 weights of a row (cols % 16 == 0):
// a 16-byte int8 load and two 16-byte bf16 stores; the same decode() as the fused kernels.
extern "C" __global__ __launch_bounds__(256) void mo_int8_decode_kernel(const int8_t* q, const float* scale,
                                                                        __bf16* out, uint32_t rows,
                                                                        uint32_t cols) {
  using u32x4 = unsigned int __attribute__((ext_vector_type(4)));
  const uint32_t per_row = cols / 16;
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;  // chunk of 16 weights
  if (i >= rows * per_row) return;
  const uint32_t r = i / per_row;
  const float s = (float)(__bf16)scale[r];
  const u32x4 v = *(const u32x4*)(q + (size_t)i * 16);
  u32x4 lo, hi;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    uint32_t packed[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const unsigned short a = __builtin_bit_cast(unsigned short, mo_gemm::decode(v[w], 2 * h, s));
      const unsigned short b = __builtin_bit_cast(unsigned short, mo_gemm::decode(v[w], 2 * h + 1, s));
      packed[h] = (uint32_t)a | ((uint32_t)b << 16);
    }
    if (w < 2) {
      lo[2 * w] = packed[0];
      lo[2 * w + 1] = packed[1];
    } else {
      hi[2 * (w - 2)] = packed[0];
      hi[2 * (w - 2) + 1] = packed[1];
    }
  }
  u32x4* dst = (u32x4*)(out + (size_t)i * 16);
  dst[0] = lo;
  dst[1] = hi;
}

// Wt[in][out] = W[out][in]^T for the input gradient on the weight-in-registers kernel, which
// needs the reduction (out) contiguous. A workgroup moves a 128 x 128 tile (grid: row tiles x
// column tiles, column tiles fastest). Lane t reads 16-byte pieces of W rows 4 (t / 8) + 0..3 at
// columns 16 (t % 8) (eight lanes per 128-byte row piece), transposes the 4 x 4 byte blocks in
// registers into 4-byte words of one column and four rows, and exchanges them through LDS
// ([column][row group], 16-byte chunks XOR-swizzled by column so the word writes of a wave
// spread over the banks); then, in four passes of 32 Wt rows, lane t writes 16 bytes of Wt row
// t / 8 of the pass at rows 16 (t % 8) (eight lanes per 128-byte row piece).
// rows % 16 == 0, cols % 16 == 0.
extern "C" __global__ __launch_bounds__(256) void mo_int8_transpose_kernel(const int8_t* w, int8_t* wt,
                                                                          uint32_t rows, uint32_t cols) {
  using mo_gemm::u32x4;
  __shared__ __attribute__((aligned(16))) uint32_t tile[128 * 32];
  auto slot = [](int col, int chunk) { return col * 32 + ((chunk ^ ((col + (col >> 4)) & 7)) << 2); };
  const uint32_t tiles_c = (cols + 127) / 128;
  const uint32_t r_base = (blockIdx.x / tiles_c) * 128, c_base = (blockIdx.x % tiles_c) * 128;
  const int t = threadIdx.x, rg = t >> 3, cc = t & 7;
  u32x4 v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t r = r_base + 4 * rg + i, c = c_base + 16 * cc;
    v[i] = (r < rows && c < cols) ? *(const u32x4*)(w + ((size_t)r * cols + c)) : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      uint32_t word = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) word |= ((v[b][j] >> (8 * c)) & 0xFFu) << (8 * b);
      const int col = 16 * cc + 4 * j + c;
      tile[slot(col, rg >> 2) + (rg & 3)] = word;
    }
  __syncthreads();
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int col = 32 * p + (t >> 3), chunk = t & 7;
    const uint32_t oc = c_base + col, r = r_base + 16 * chunk;
    if (oc < cols && r < rows) *(u32x4*)(wt + ((size_t)oc * rows + r)) = *(const u32x4*)(tile + slot(col, chunk));
  }
}
