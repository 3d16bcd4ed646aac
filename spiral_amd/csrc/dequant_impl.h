// Exact dequantization of 8 consecutive elements of one planar row. Shared by
// the standalone dequant / GET_ROWS kernels and the GEMM B-tile loaders, so
// the fused products and the standalone dequant use one code path.
#pragma once

#include "common.h"

namespace spiral {

// Eight dequantized values of group g (elements 8g..8g+7) of row n.
template <int TYPE>
__device__ __forceinline__ void dequant8(const uint8_t* __restrict__ w, int64_t n_rows,
                                         int64_t nb, int64_t n, int64_t g, float v[8]) {
  if constexpr (TYPE == SPIRAL_TYPE_Q4_0) {
    const PlanarQ4_0 P(w, n_rows, nb);
    const int64_t b = g >> 2;
    const int p = static_cast<int>(g & 3);
    // Elements 0..15 of a block are the low nibbles of qs[0..15], 16..31 the
    // high nibbles (src/quants/tests/formats/q4_0.py:56-58).
    const uint2 q = *reinterpret_cast<const uint2*>(P.qs + (n * nb + b) * 16 + 8 * (p & 1));
    const int shift = (p >> 1) * 4;
    const float d = fp16_scale(P.d[n * nb + b]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = static_cast<float>(static_cast<int>((q.x >> (8 * j + shift)) & 15u) - 8) * d;
      v[j + 4] = static_cast<float>(static_cast<int>((q.y >> (8 * j + shift)) & 15u) - 8) * d;
    }
  } else if constexpr (TYPE == SPIRAL_TYPE_Q8_0) {
    const PlanarQ8_0 P(w, n_rows, nb);
    const int64_t b = g >> 2;
    const int p = static_cast<int>(g & 3);
    const uint2 q = *reinterpret_cast<const uint2*>(P.qs + (n * nb + b) * 32 + 8 * p);
    const float d = fp16_scale(P.d[n * nb + b]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = static_cast<float>(static_cast<int8_t>(q.x >> (8 * j))) * d;
      v[j + 4] = static_cast<float>(static_cast<int8_t>(q.y >> (8 * j))) * d;
    }
  } else {
    // Element e = 128h + 32j + l of a super-block takes the low (j < 2) or
    // high nibble of ql[64h + 32(j&1) + l], bits 2j..2j+1 of qh[32h + l] and
    // sub-scale sc[8h + l/16 + 2j] (src/quants/tests/formats/q6_k.py:69-95).
    const PlanarQ6_K P(w, n_rows, nb);
    const int64_t sb = g >> 5;
    const int t = static_cast<int>(g & 31);
    const int h = t >> 4, j = (t >> 2) & 3, l0 = (t & 3) * 8;
    const int64_t blk = n * nb + sb;
    const uint2 lo = *reinterpret_cast<const uint2*>(P.ql + blk * 128 + 64 * h + 32 * (j & 1) + l0);
    const uint2 hi = *reinterpret_cast<const uint2*>(P.qh + blk * 64 + 32 * h + l0);
    const float ds = fp16_scale(P.d[blk]) * static_cast<float>(P.sc[blk * 16 + 8 * h + (l0 >> 4) + 2 * j]);
    const int ls = (j >> 1) * 4, hs = 2 * j;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int q0 = static_cast<int>(((lo.x >> (8 * e + ls)) & 15u) | (((hi.x >> (8 * e + hs)) & 3u) << 4));
      const int q1 = static_cast<int>(((lo.y >> (8 * e + ls)) & 15u) | (((hi.y >> (8 * e + hs)) & 3u) << 4));
      v[e] = ds * static_cast<float>(q0 - 32);
      v[e + 4] = ds * static_cast<float>(q1 - 32);
    }
  }
}

}  // namespace spiral
