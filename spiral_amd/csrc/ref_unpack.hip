// The reference's device entry points, on the GPU, over its record layout:
// quants_unpack_all (src/quants/tests/unpack.aie.cc:21-45) and
// quants_unpack_mmul_all (src/quants/tests/mmul.aie.cc:20-35).
//
// Record layouts are those written by quants_<fmt>_repack (repack_ref.cpp).
// Values: the signed code times the decoded fp16 scale (times the int8
// sub-scale for Q6_K), rounded once to bf16 -- bit-identical to the
// reference's split-scale arithmetic, as for the planar kernels.
#include "common.h"

namespace spiral {
namespace {

struct RefGeom {
  int record_rows, record_bytes;
};
__host__ __device__ constexpr RefGeom ref_geom(int type) {
  return type == SPIRAL_TYPE_Q4_0 ? RefGeom{64, 288} : type == SPIRAL_TYPE_Q8_0 ? RefGeom{256, 2176} : RefGeom{256, 1680};
}

// Row `row` (k within the record) of one record: the 8 column values.
template <int TYPE>
__device__ __forceinline__ void ref_row8(const uint8_t* __restrict__ rec, int row, float v[8]) {
  if constexpr (TYPE == SPIRAL_TYPE_Q4_0) {
    const int blk = row >> 5, br = row & 31;
    const uint4 dv = *reinterpret_cast<const uint4*>(rec + 16 * blk);
    const uint32_t q = *reinterpret_cast<const uint32_t*>(rec + 32 + 128 * blk + 4 * br);
    const uint32_t d[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int s = static_cast<int>((q >> (4 * c)) & 15u);
      const int code = s >= 8 ? s - 16 : s;  // stored as (q - 8) & 15
      v[c] = static_cast<float>(code) * fp16_scale((c & 1) ? (d[c >> 1] >> 16) : (d[c >> 1] & 0xffffu));
    }
  } else if constexpr (TYPE == SPIRAL_TYPE_Q8_0) {
    const int blk = row >> 5, br = row & 31;
    const uint4 dv = *reinterpret_cast<const uint4*>(rec + 2048 + 16 * blk);
    const uint2 q = *reinterpret_cast<const uint2*>(rec + 256 * blk + 8 * br);
    const uint32_t d[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const uint32_t word = c < 4 ? q.x : q.y;
      const int code = static_cast<int8_t>((word >> (8 * (c & 3))) & 0xffu);
      v[c] = static_cast<float>(code) * fp16_scale((c & 1) ? (d[c >> 1] >> 16) : (d[c >> 1] & 0xffffu));
    }
  } else {
    const int ch = row >> 6, cr = row & 63;
    const uint8_t* chunk = rec + 384 * ch;
    const uint32_t lo = *reinterpret_cast<const uint32_t*>(chunk + 4 * cr);
    const uint32_t hi = *reinterpret_cast<const uint16_t*>(chunk + 256 + 2 * cr);
    const uint2 sc = *reinterpret_cast<const uint2*>(rec + 1536 + 32 * ch + 8 * (cr >> 4));
    const uint4 dv = *reinterpret_cast<const uint4*>(rec + 1664);
    const uint32_t d[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int q = static_cast<int>(((lo >> (4 * c)) & 15u) | (((hi >> (2 * c)) & 3u) << 4));
      const int s = static_cast<int8_t>(((c < 4 ? sc.x : sc.y) >> (8 * (c & 3))) & 0xffu);
      const float ds = fp16_scale((c & 1) ? (d[c >> 1] >> 16) : (d[c >> 1] & 0xffffu)) * static_cast<float>(s);
      v[c] = ds * static_cast<float>(q - 32);
    }
  }
}

// One thread per (record, row): 8 bf16 outputs, one 16-byte store. The
// output of record i starts at i * record_rows * 8, rows of 8 columns.
template <int TYPE>
__global__ void __launch_bounds__(256) ref_unpack_kernel(const uint8_t* __restrict__ packed, int64_t records,
                                                         uint16_t* __restrict__ out) {
  constexpr RefGeom G = ref_geom(TYPE);
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= records * G.record_rows) return;
  const int64_t rec = i / G.record_rows;
  const int row = static_cast<int>(i % G.record_rows);
  float v[8];
  ref_row8<TYPE>(packed + rec * G.record_bytes, row, v);
  uint4 o;
  o.x = pack_bf16x2(v[0], v[1]);
  o.y = pack_bf16x2(v[2], v[3]);
  o.z = pack_bf16x2(v[4], v[5]);
  o.w = pack_bf16x2(v[6], v[7]);
  reinterpret_cast<uint4*>(out)[i] = o;
}

// One workgroup per 8-column tile: out[tile][v][c] = sum_k in[v][k] * W[k][c]
// for the four input vectors. Each thread takes k rows tid, tid + 256, ...;
// a workgroup reduction finishes the 32 sums. Weights are the exact bf16
// values; inputs are bf16 in the reference's [k/8][4][8] tiling.
template <int TYPE>
__global__ void __launch_bounds__(256) ref_mmul_kernel(const uint8_t* __restrict__ packed, int64_t rows,
                                                       const uint16_t* __restrict__ inputs,
                                                       float* __restrict__ outputs) {
  constexpr RefGeom G = ref_geom(TYPE);
  __shared__ float red[8][32];
  const int64_t tile = blockIdx.x;
  const int64_t row_records = rows / G.record_rows;
  float acc[4][8];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[a][c] = 0.0f;
  for (int64_t k = threadIdx.x; k < rows; k += blockDim.x) {
    const int64_t r = k / G.record_rows;
    float wv[8];
    ref_row8<TYPE>(packed + (tile * row_records + r) * G.record_bytes, static_cast<int>(k % G.record_rows), wv);
    // Weights are rounded to bf16 as the reference's unpack does.
#pragma unroll
    for (int c = 0; c < 8; c += 2) {
      const uint32_t p = pack_bf16x2(wv[c], wv[c + 1]);
      wv[c] = bf16_lo(p);
      wv[c + 1] = bf16_hi(p);
    }
    const uint16_t* in = inputs + (k >> 3) * 32 + (k & 7);
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const float xv = __uint_as_float(static_cast<uint32_t>(in[8 * a]) << 16);
#pragma unroll
      for (int c = 0; c < 8; ++c) acc[a][c] = __builtin_fmaf(xv, wv[c], acc[a][c]);
    }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const float s = wave_sum(acc[a][c]);
      if (lane == 0) red[wave][8 * a + c] = s;
    }
  __syncthreads();
  if (threadIdx.x < 32) {
    float s = 0.0f;
    for (int wv = 0; wv < static_cast<int>(blockDim.x >> 6); ++wv) s += red[wv][threadIdx.x];
    outputs[tile * 32 + threadIdx.x] = s;
  }
}

int check_ref(int type, const void* a, const void* b, int64_t rows, int64_t cols) {
  if (!is_quant_type(type)) return SPIRAL_ERR_TYPE;
  if (a == nullptr || b == nullptr) return SPIRAL_ERR_NULL;
  const RefGeom g = ref_geom(type);
  if (rows <= 0 || cols <= 0 || rows % g.record_rows != 0 || cols % 8 != 0) return SPIRAL_ERR_SHAPE;
  if (!aligned16(a) || !aligned16(b)) return SPIRAL_ERR_ALIGN;
  return require_device();
}

}  // namespace
}  // namespace spiral

using namespace spiral;

extern "C" {

int quants_unpack_all(int type, const void* packed, int64_t weights_rows, int64_t weights_cols, uint16_t* out,
                      void* stream) {
  int rc = check_ref(type, packed, out, weights_rows, weights_cols);
  if (rc != SPIRAL_OK) return rc;
  const RefGeom g = ref_geom(type);
  const int64_t records = (weights_rows / g.record_rows) * (weights_cols / 8);
  const dim3 grid(static_cast<unsigned>(ceil_div(records * g.record_rows, 256)));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint8_t* P = static_cast<const uint8_t*>(packed);
  if (type == SPIRAL_TYPE_Q4_0)
    hipLaunchKernelGGL(ref_unpack_kernel<SPIRAL_TYPE_Q4_0>, grid, dim3(256), 0, s, P, records, out);
  else if (type == SPIRAL_TYPE_Q8_0)
    hipLaunchKernelGGL(ref_unpack_kernel<SPIRAL_TYPE_Q8_0>, grid, dim3(256), 0, s, P, records, out);
  else
    hipLaunchKernelGGL(ref_unpack_kernel<SPIRAL_TYPE_Q6_K>, grid, dim3(256), 0, s, P, records, out);
  return launch_status();
}

int quants_unpack_mmul_all(int type, const void* packed, const uint16_t* inputs, float* outputs,
                           int64_t weights_rows, int64_t weights_cols, void* stream) {
  int rc = check_ref(type, packed, outputs, weights_rows, weights_cols);
  if (rc != SPIRAL_OK) return rc;
  if (inputs == nullptr) return SPIRAL_ERR_NULL;
  if ((reinterpret_cast<uintptr_t>(inputs) & 1u) != 0) return SPIRAL_ERR_ALIGN;
  const dim3 grid(static_cast<unsigned>(weights_cols / 8));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint8_t* P = static_cast<const uint8_t*>(packed);
  if (type == SPIRAL_TYPE_Q4_0)
    hipLaunchKernelGGL(ref_mmul_kernel<SPIRAL_TYPE_Q4_0>, grid, dim3(256), 0, s, P, weights_rows, inputs, outputs);
  else if (type == SPIRAL_TYPE_Q8_0)
    hipLaunchKernelGGL(ref_mmul_kernel<SPIRAL_TYPE_Q8_0>, grid, dim3(256), 0, s, P, weights_rows, inputs, outputs);
  else
    hipLaunchKernelGGL(ref_mmul_kernel<SPIRAL_TYPE_Q6_K>, grid, dim3(256), 0, s, P, weights_rows, inputs, outputs);
  return launch_status();
}

}  // extern "C"
