// Dequant-GEMM on bf16 MFMA: Y[m][n] = sum_k X[m][k] * W[n][k] for planar
// quantized W (any of Q4_0 / Q8_0 / Q6_K), bf16 X, fp32 accumulation.
//
// This is the prefill form of the reference's fused unpack + mmul
// (src/quants/q4_0/mmul.aie.h:16-90 with aie::mmul<4,8,8,bf16,bf16>,
// src/quants/common/mmul.aie.h:9-22): weights are dequantized exactly to bf16
// (the same helper as the standalone dequant) and multiplied against bf16
// inputs with fp32 accumulation, so each product term is bit-identical to the
// reference's; only the fp32 summation order differs.
//
// Tiling: a 256-thread workgroup computes a BM x BN tile of Y; its four waves
// form a 2 x 2 grid of 64 x 64 sub-tiles, each held as 4 x 4
// v_mfma_f32_16x16x32_bf16 accumulators. Per BK slice the workgroup copies the
// X tile and dequantizes the W tile into LDS, then each wave runs 2 x 16 MFMAs.
#include "common.h"
#include "dequant_impl.h"

namespace spiral {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

constexpr int kBM = 128, kBN = 128, kBK = 64;
constexpr int kLdsK = kBK + 8;  // row pitch in elements; the pad spreads rows over banks

__device__ __forceinline__ uint4 pack8(const float v[8]) {
  return make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                    pack_bf16x2(v[6], v[7]));
}

template <int TYPE, bool F32_OUT>
__global__ void __launch_bounds__(256) gemm_kernel(const uint8_t* __restrict__ w, int64_t n_rows,
                                                   int64_t k, const uint16_t* __restrict__ x, int64_t ldx,
                                                   int64_t m, void* __restrict__ y, int64_t ldy) {
  __shared__ __align__(16) uint16_t As[kBM * kLdsK];
  __shared__ __align__(16) uint16_t Bs[kBN * kLdsK];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kBM;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kBN;
  const int64_t nb = k / block_elems(TYPE);

  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  for (int64_t k0 = 0; k0 < k; k0 += kBK) {
    // X tile: 128 rows x 64 k as 16-byte pieces (8 threads per row).
#pragma unroll
    for (int it = 0; it < (kBM * kBK / 8) / 256; ++it) {
      const int i = tid + 256 * it;
      const int r = i >> 3, c = i & 7;
      const int64_t gm = m0 + r, gk = k0 + 8 * c;
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (gm < m && gk < k) v = *reinterpret_cast<const uint4*>(x + gm * ldx + gk);
      *reinterpret_cast<uint4*>(&As[r * kLdsK + 8 * c]) = v;
    }
    // W tile: 128 rows x 64 k, dequantized exactly to bf16.
#pragma unroll
    for (int it = 0; it < (kBN * kBK / 8) / 256; ++it) {
      const int i = tid + 256 * it;
      const int r = i >> 3, c = i & 7;
      const int64_t gn = n0 + r, g = (k0 >> 3) + c;
      float v[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
      if (gn < n_rows && 8 * g < k) dequant8<TYPE>(w, n_rows, nb, gn, g, v);
      *reinterpret_cast<uint4*>(&Bs[r * kLdsK + 8 * c]) = pack8(v);
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 32) {
      // Operand layout of v_mfma_f32_16x16x32_bf16: lane l holds row (l % 16)
      // of A and column (l % 16) of B at k = 8 * (l / 16) .. + 7.
      bf16x8_t a[4], b[4];
      const int kq = kk + 8 * (lane >> 4);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        a[i] = *reinterpret_cast<const bf16x8_t*>(&As[(wm * 64 + 16 * i + (lane & 15)) * kLdsK + kq]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        b[j] = *reinterpret_cast<const bf16x8_t*>(&Bs[(wn * 64 + 16 * j + (lane & 15)) * kLdsK + kq]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }

  // Accumulator layout: lane l holds D[4 * (l / 16) + e][l % 16], e < 4.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t gn = n0 + wn * 64 + 16 * j + (lane & 15);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t gm = m0 + wm * 64 + 16 * i + 4 * (lane >> 4) + e;
        if (gm < m && gn < n_rows) {
          if constexpr (F32_OUT)
            static_cast<float*>(y)[gm * ldy + gn] = acc[i][j][e];
          else
            static_cast<__bf16*>(y)[gm * ldy + gn] = static_cast<__bf16>(acc[i][j][e]);
        }
      }
    }
  }
}

template <int TYPE>
int launch_gemm(const void* w, int64_t n_rows, int64_t k, const uint16_t* x, int64_t ldx, int64_t m,
                void* y, int y_type, int64_t ldy, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(ceil_div(n_rows, kBN)), static_cast<unsigned>(ceil_div(m, kBM)));
  const uint8_t* W = static_cast<const uint8_t*>(w);
  if (y_type == SPIRAL_TYPE_F32)
    hipLaunchKernelGGL((gemm_kernel<TYPE, true>), grid, dim3(256), 0, s, W, n_rows, k, x, ldx, m, y, ldy);
  else
    hipLaunchKernelGGL((gemm_kernel<TYPE, false>), grid, dim3(256), 0, s, W, n_rows, k, x, ldx, m, y, ldy);
  return launch_status();
}

}  // namespace

// Y = X W^T; arguments validated by the caller.
int gemm(int type, const void* w, int64_t n_rows, int64_t k, const uint16_t* x, int64_t ldx, int64_t m,
         void* y, int y_type, int64_t ldy, hipStream_t s) {
  switch (type) {
    case SPIRAL_TYPE_Q4_0: return launch_gemm<SPIRAL_TYPE_Q4_0>(w, n_rows, k, x, ldx, m, y, y_type, ldy, s);
    case SPIRAL_TYPE_Q8_0: return launch_gemm<SPIRAL_TYPE_Q8_0>(w, n_rows, k, x, ldx, m, y, y_type, ldy, s);
    case SPIRAL_TYPE_Q6_K: return launch_gemm<SPIRAL_TYPE_Q6_K>(w, n_rows, k, x, ldx, m, y, y_type, ldy, s);
    default: return SPIRAL_ERR_TYPE;
  }
}

}  // namespace spiral
