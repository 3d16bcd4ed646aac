// Dequant-GEMM on bf16 MFMA: Y[m][n] = sum_k X[m][k] * W[n][k] for planar
// quantized W (any of Q4_0 / Q8_0 / Q6_K), bf16 X, fp32 accumulation.
//
// This is the prefill form of the reference's fused unpack + mmul
// (src/quants/q4_0/mmul.aie.h:16-90 with aie::mmul<4,8,8,bf16,bf16>,
// src/quants/common/mmul.aie.h:9-22): weights are dequantized exactly to bf16
// and multiplied against bf16 inputs with fp32 accumulation, so each product
// term equals the reference's; only the fp32 summation order differs.
//
// Tiling (gfx950, wave64, v_mfma_f32_16x16x32_bf16, 16 cycles each):
//  - One workgroup per 128 (m) x 64 (n) tile of Y; m = 512, n = 4096 gives
//    256 tiles, one per CU.
//  - A k step is 128 wide. Its W tile (64 rows x 128 k) is dequantized once
//    per workgroup into LDS (double-buffered, one barrier per step): each of
//    the 512 threads turns one 16-element piece.
//  - 8 waves: wave w owns rows 32 (w % 4) .. + 31 (2 x 4 MFMA tiles) for the
//    64-wide k half w / 4 of every step. Each SIMD thus runs two waves over
//    the same rows and interleaves their instruction streams; the halves are
//    summed through LDS at the end.
//  - X goes straight from global memory into the MFMA A-operand layout with
//    buffer loads (fixed per-lane offset + scalar per-step offset; each
//    element of X is read by one wave of the workgroup, no LDS).
//  - X fragments and packed weights are requested RING - 1 steps ahead in a
//    register ring; step s + 1's weights are dequantized while step s's
//    MFMAs run.
//  - Workgroups are numbered so that each XCD (dispatch is round-robin over
//    the 8 XCDs) gets a contiguous range of tiles that share X rows in its L2.
#include <algorithm>

#include "common.h"
#include "dequant_impl.h"

namespace spiral {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

constexpr int kBM = 128, kBN = 64, kBK = 128, kThreads = 512;
constexpr int kPitch = kBK + 8;  // LDS row pitch in bf16; the pad spreads rows over banks
constexpr int kRing = 4;
constexpr int64_t kMaxBufferBytes = int64_t(1) << 31;  // buffer offsets are 32-bit

// Tile index for workgroup b of `grid`: consecutive workgroups go to
// consecutive XCDs, so hand XCD x the tiles [x grid / 8, (x + 1) grid / 8).
__device__ __forceinline__ int64_t xcd_tile(int64_t b, int64_t grid) {
  if (grid % 8 != 0) return b;
  return (b % 8) * (grid / 8) + b / 8;
}

struct AFrag {
  uint4 v[2][2];  // [m16 block][k32 sub-step of the wave's half]
};

// X fragments of a wave's 32 rows for its 64-wide half of a k step (k0 =
// start of the half): lane l holds row (l % 16) of each 16-row block at
// k = 8 (l / 16) .. + 7 of each 32-k sub-step. voff[i] is the lane's byte
// offset of its row of block i (rows past m clamped to m - 1: their outputs
// are never stored). Sub-steps at or past `nsub` are zero (the k tail).
__device__ __forceinline__ void load_a(AFrag& a, __amdgpu_buffer_rsrc_t X, const uint32_t (&voff)[2], int64_t k0,
                                       int nsub = 2) {
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int s = 0; s < 2; ++s)
      a.v[i][s] = s < nsub ? bload16(X, voff[i], static_cast<uint32_t>(k0 + 32 * s) * 2u) : make_uint4(0u, 0u, 0u, 0u);
}

template <int TYPE>
__device__ __forceinline__ void store_b(const Piece<TYPE>& pc, const typename Piece<TYPE>::Addr& pa, uint16_t* bs,
                                        int tid) {
  uint4 o0, o1;
  pc.dequant(pa, o0, o1);
  uint16_t* dst = bs + (tid >> 3) * kPitch + 16 * (tid & 7);
  *reinterpret_cast<uint4*>(dst) = o0;
  *reinterpret_cast<uint4*>(dst + 8) = o1;
}

__device__ __forceinline__ bf16x8_t read_b(const uint16_t* bs, int j, int s, int lane) {
  return *reinterpret_cast<const bf16x8_t*>(bs + (16 * j + (lane & 15)) * kPitch + 32 * s + 8 * (lane >> 4));
}

// The wave's two K32 sub-steps (sub-steps 2 h and 2 h + 1 of the 128-wide
// LDS tile) against all 64 columns.
__device__ __forceinline__ void mfma_step(f32x4_t (&acc)[2][4], const AFrag& a, const uint16_t* bs, int h,
                                          int lane) {
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    bf16x8_t b[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) b[j] = read_b(bs, j, 2 * h + s, lane);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const bf16x8_t av = __builtin_bit_cast(bf16x8_t, a.v[i][s]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, b[j], acc[i][j], 0, 0, 0);
    }
  }
}

template <int TYPE, int RING>
struct Pipe {
  AFrag a[RING];
  Piece<TYPE> pc[RING];
};

// One pipelined step s (ring slot d = s % RING): request step s + RING - 1
// (clamped to the last full step) into the slot of step s - 1, multiply
// step s, dequantize step s + 1 into the other LDS buffer.
template <int TYPE, int RING>
__device__ __forceinline__ void gemm_step(f32x4_t (&acc)[2][4], Pipe<TYPE, RING>& pp, uint16_t* bs0, int d,
                                          int64_t s, int64_t full, __amdgpu_buffer_rsrc_t X,
                                          const uint32_t (&voff)[2], const Planes& P,
                                          const typename Piece<TYPE>::Addr& pa, int h, int tid, int lane) {
  const int64_t ahead = min(s + RING - 1, full - 1) * kBK;
  load_a(pp.a[(d + RING - 1) % RING], X, voff, ahead + 64 * h);
  pp.pc[(d + RING - 1) % RING].load(P, pa, ahead);
  mfma_step(acc, pp.a[d], bs0 + (s & 1) * (kBN * kPitch), h, lane);
  store_b<TYPE>(pp.pc[(d + 1) % RING], pa, bs0 + ((s + 1) & 1) * (kBN * kPitch), tid);
  __syncthreads();
}

// 8 waves: wave w computes rows 32 (w % 4) .. + 31 of the tile over the
// k-half h = w / 4 of every step; the two halves are summed through LDS at
// the end. The two waves of a SIMD (w and w + 4) share rows, so each SIMD
// interleaves two instruction streams over the same MFMA tiles.
template <int TYPE, int RING, bool F32_OUT>
__global__ void __launch_bounds__(kThreads) gemm_kernel(const uint8_t* __restrict__ w, int64_t n_rows, int64_t k,
                                                        const uint16_t* __restrict__ x, int64_t ldx, int64_t m,
                                                        void* __restrict__ y, int64_t ldy, int64_t n_tiles_n) {
  __shared__ __align__(16) uint16_t Bs[2 * kBN * kPitch];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int mw = wave & 3, h = wave >> 2;
  const int64_t tile = xcd_tile(blockIdx.x, gridDim.x);
  const int64_t m0 = (tile / n_tiles_n) * kBM, n0 = (tile % n_tiles_n) * kBN;
  const int64_t row0 = m0 + 32 * mw;
  const int64_t nb = k / block_elems(TYPE);
  const int64_t full = k / kBK;
  const int tail = static_cast<int>(k - full * kBK);  // 0, 32, 64 or 96

  const __amdgpu_buffer_rsrc_t X = buffer_rsrc(x, static_cast<uint32_t>(m * ldx * 2));
  uint32_t voff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
    voff[i] = static_cast<uint32_t>((min(row0 + 16 * i + (lane & 15), m - 1) * ldx + 8 * (lane >> 4)) * 2);
  const Planes P = make_planes<TYPE>(w, n_rows, nb);
  const typename Piece<TYPE>::Addr pa = Piece<TYPE>::addr(min(n0 + (tid >> 3), n_rows - 1), nb, tid & 7);

  f32x4_t acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  if (full > 0) {
    // Ring slot s % RING holds step s's X fragments and packed weights; step
    // s's weights are dequantized into buffer s & 1 during step s - 1.
    Pipe<TYPE, RING> pp;
#pragma unroll
    for (int i = 0; i < RING - 1; ++i) {
      const int64_t k0 = min<int64_t>(i, full - 1) * kBK;
      load_a(pp.a[i], X, voff, k0 + 64 * h);
      pp.pc[i].load(P, pa, k0);
    }
    store_b<TYPE>(pp.pc[0], pa, Bs, tid);
    __syncthreads();
    int64_t s0 = 0;
    for (; s0 + RING <= full; s0 += RING) {
#pragma unroll
      for (int d = 0; d < RING; ++d)
        gemm_step<TYPE, RING>(acc, pp, Bs, d, s0 + d, full, X, voff, P, pa, h, tid, lane);
    }
#pragma unroll
    for (int d = 0; d < RING - 1; ++d) {
      if (s0 + d < full) gemm_step<TYPE, RING>(acc, pp, Bs, d, s0 + d, full, X, voff, P, pa, h, tid, lane);
    }
  }
  if (tail > 0) {
    // k tail of 32, 64 or 96: pieces past it and X sub-steps past it are zero.
    Piece<TYPE> pt;
    AFrag at;
    if (16 * (tid & 7) < tail)
      pt.load(P, pa, full * kBK);
    else
      pt.zero();
    load_a(at, X, voff, full * kBK + 64 * h, min(2, max(0, tail / 32 - 2 * h)));
    store_b<TYPE>(pt, pa, Bs, tid);
    __syncthreads();
    mfma_step(acc, at, Bs, h, lane);
    __syncthreads();
  }

  // Sum the two k-halves: waves 4..7 park their accumulators in LDS (the
  // weight buffers are free after the last barrier), waves 0..3 add them.
  float* red = reinterpret_cast<float*>(Bs) + mw * (2 * 4 * 4 * 64);
  if (h == 1) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) red[((i * 4 + j) * 4 + e) * 64 + lane] = acc[i][j][e];
  }
  __syncthreads();
  if (h == 1) return;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[i][j][e] += red[((i * 4 + j) * 4 + e) * 64 + lane];

  // Accumulator layout: lane l holds D[4 (l / 16) + e][l % 16], e < 4.
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t gn = n0 + 16 * j + (lane & 15);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t gm = row0 + 16 * i + 4 * (lane >> 4) + e;
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
int launch_gemm(const void* w, int64_t n_rows, int64_t k, const uint16_t* x, int64_t ldx, int64_t m, void* y,
                int y_type, int64_t ldy, hipStream_t s) {
  // Weight planes are addressed with 32-bit offsets (the largest plane is at
  // most 16/18 of the tensor); X is launched in chunks of rows that keep its
  // offsets below 2 GiB.
  if (spiral_tensor_bytes(TYPE, n_rows, k) >= kMaxBufferBytes * 2) return SPIRAL_ERR_SHAPE;
  const int64_t chunk = std::max<int64_t>(kBM, (kMaxBufferBytes / (ldx * 2)) / kBM * kBM);
  const int64_t tn = ceil_div(n_rows, kBN);
  const uint8_t* W = static_cast<const uint8_t*>(w);
  const int64_t ysz = y_type == SPIRAL_TYPE_F32 ? 4 : 2;
  for (int64_t mo = 0; mo < m; mo += chunk) {
    const int64_t mc = std::min(chunk, m - mo);
    const int64_t tm = ceil_div(mc, kBM);
    if (tn * tm > INT32_MAX) return SPIRAL_ERR_SHAPE;
    const dim3 grid(static_cast<unsigned>(tn * tm));
    const uint16_t* xc = x + mo * ldx;
    void* yc = static_cast<uint8_t*>(y) + mo * ldy * ysz;
    if (y_type == SPIRAL_TYPE_F32)
      hipLaunchKernelGGL((gemm_kernel<TYPE, kRing, true>), grid, dim3(kThreads), 0, s, W, n_rows, k, xc, ldx, mc, yc, ldy, tn);
    else
      hipLaunchKernelGGL((gemm_kernel<TYPE, kRing, false>), grid, dim3(kThreads), 0, s, W, n_rows, k, xc, ldx, mc, yc, ldy, tn);
    const int rc = launch_status();
    if (rc != SPIRAL_OK) return rc;
  }
  return SPIRAL_OK;
}

}  // namespace

// Y = X W^T; arguments validated by the caller (k a multiple of the block, x
// rows 16-byte aligned with ldx a multiple of 8).
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
