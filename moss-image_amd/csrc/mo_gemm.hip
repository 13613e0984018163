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
// Tiling: a 256-lane workgroup (4 wave64, 2 x 2) owns a 128 x 128 output tile; each wave owns
// 64 x 64 = 2 x 2 MFMA 32x32 tiles. The reduction advances 64 per step; the next step's A and
// Bq tiles are loaded into registers while the current step's MFMAs run from LDS.
// MFMA 32x32x16 bf16 lane layout (checked on the device): A lane l holds row l%32,
// k = 8*(l/32)+j; B lane l holds column l%32, k = 8*(l/32)+j; D register r of lane l holds
// row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mo_gemm {

constexpr int kThreads = 256;
constexpr int kBM = 128;  // output rows per workgroup
constexpr int kBC = 128;  // output columns per workgroup
constexpr int kBR = 64;   // reduction per step
constexpr int kLds = kBR + 8;  // LDS row pitch in bf16 (padding spreads banks)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

#define MO_GLOBAL __attribute__((address_space(1)))
#define MO_LDS __attribute__((address_space(3)))

__device__ __forceinline__ u32x4 gload16(const void* p) { return *(const MO_GLOBAL u32x4*)p; }

// bf16(q * bf16(s)): the product of an int8 and a bf16 is exact in fp32; one rounding to bf16.
__device__ __forceinline__ __bf16 decode(int q, float s_bf16) { return (__bf16)((float)q * s_bf16); }

template <bool kTransB>
__device__ __forceinline__ void gemm_body(const __bf16* __restrict__ A, const int8_t* __restrict__ Bq,
                                          const float* __restrict__ scale, const __bf16* __restrict__ bias,
                                          __bf16* __restrict__ C, int M, int NC, int R, int tiles_m) {
  __shared__ __attribute__((aligned(16))) __bf16 As[kBM * kLds];
  __shared__ __attribute__((aligned(16))) __bf16 Bs[kBC * kLds];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave & 1, wc = wave >> 1;
  const int tile_m = blockIdx.x % tiles_m;
  const int tile_c = blockIdx.x / tiles_m;
  const int m0 = tile_m * kBM, c0 = tile_c * kBC;

  // ---- global load assignment ----
  // A: 128 rows x 64 bf16; lane pair per row, 4 chunks of 8 bf16 each.
  const int a_row = tid >> 1, a_k = (tid & 1) * 32;
  // Bq, forward: 128 columns x 64 int8, lane pair per column, 2 chunks of 16.
  // Bq, transposed: 64 reduction rows x 128 columns, 4 lanes per row, 2 chunks of 16.
  const int b_col = kTransB ? (tid & 3) * 32 : tid >> 1;
  const int b_red = kTransB ? tid >> 2 : (tid & 1) * 32;

  u32x4 ra[4], rb[2];
  float rs = 0.f;  // bf16-rounded scale for this lane's Bq values

  auto load = [&](int r0) {
    const int am = m0 + a_row;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = r0 + a_k + 8 * i;
      ra[i] = (am < M && k < R) ? gload16(A + (size_t)am * R + k) : u32x4{0, 0, 0, 0};
    }
    if (!kTransB) {
      const int n = c0 + b_col;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int k = r0 + b_red + 16 * i;
        rb[i] = (n < NC && k < R) ? gload16(Bq + (size_t)n * R + k) : u32x4{0, 0, 0, 0};
      }
      rs = n < NC ? (float)(__bf16)scale[n] : 0.f;
    } else {
      const int r = r0 + b_red;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int c = c0 + b_col + 16 * i;
        rb[i] = (r < R && c < NC) ? gload16(Bq + (size_t)r * NC + c) : u32x4{0, 0, 0, 0};
      }
      rs = r < R ? (float)(__bf16)scale[r] : 0.f;
    }
  };

  auto store_lds = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) *(MO_LDS u32x4*)(As + a_row * kLds + a_k + 8 * i) = ra[i];
    if (!kTransB) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int8_t* q = (const int8_t*)&rb[i];
        bf16x8 lo, hi;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          lo[j] = decode(q[j], rs);
          hi[j] = decode(q[8 + j], rs);
        }
        *(MO_LDS bf16x8*)(Bs + b_col * kLds + b_red + 16 * i) = lo;
        *(MO_LDS bf16x8*)(Bs + b_col * kLds + b_red + 16 * i + 8) = hi;
      }
    } else {
      // transposed: Bs[column][reduction]
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int8_t* q = (const int8_t*)&rb[i];
#pragma unroll
        for (int j = 0; j < 16; ++j) *(MO_LDS __bf16*)(Bs + (b_col + 16 * i + j) * kLds + b_red) = decode(q[j], rs);
      }
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  const int steps = (R + kBR - 1) / kBR;
  load(0);
  for (int s = 0; s < steps; ++s) {
    __syncthreads();  // previous step's MFMAs are done reading LDS
    store_lds();
    __syncthreads();
    if (s + 1 < steps) load((s + 1) * kBR);  // in flight during the MFMAs below
    const int row_a = wm * 64 + (lane & 31);
    const int row_b = wc * 64 + (lane & 31);
    const int kq = 8 * (lane >> 5);
#pragma unroll
    for (int kk = 0; kk < kBR; kk += 16) {
      bf16x8 a0 = *(MO_LDS bf16x8*)(As + row_a * kLds + kk + kq);
      bf16x8 a1 = *(MO_LDS bf16x8*)(As + (row_a + 32) * kLds + kk + kq);
      bf16x8 b0 = *(MO_LDS bf16x8*)(Bs + row_b * kLds + kk + kq);
      bf16x8 b1 = *(MO_LDS bf16x8*)(Bs + (row_b + 32) * kLds + kk + kq);
      acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b1, acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b0, acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1, acc[1][1], 0, 0, 0);
    }
  }

  // ---- epilogue: bias, bf16, store ----
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = c0 + wc * 64 + j * 32 + (lane & 31);
    if (col >= NC) continue;
    const float b = bias ? (float)bias[col] : 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < M) *(MO_GLOBAL __bf16*)(C + (size_t)row * NC + col) = (__bf16)(acc[i][j][r] + b);
      }
    }
  }
}

}  // namespace mo_gemm

extern "C" __global__ __launch_bounds__(mo_gemm::kThreads) void mo_int8_linear_fwd_kernel(
    const __bf16* A, const int8_t* Bq, const float* scale, const __bf16* bias, __bf16* C, int M, int NC, int R,
    int tiles_m) {
  mo_gemm::gemm_body<false>(A, Bq, scale, bias, C, M, NC, R, tiles_m);
}

extern "C" __global__ __launch_bounds__(mo_gemm::kThreads) void mo_int8_linear_bwd_kernel(
    const __bf16* A, const int8_t* Bq, const float* scale, __bf16* C, int M, int NC, int R, int tiles_m) {
  mo_gemm::gemm_body<true>(A, Bq, scale, nullptr, C, M, NC, R, tiles_m);
}
