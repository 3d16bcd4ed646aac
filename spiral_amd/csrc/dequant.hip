// Exact dequantization of planar Q4_0 / Q8_0 / Q6_K weights to bf16, and the
// GET_ROWS gather built on it.
//
// Element values follow the reference's unpack semantics exactly:
//   Q4_0  bf16_rne((q - 8) * d)        src/quants/q4_0/unpack.aie.h:31-46
//   Q8_0  bf16_rne(q * d)              src/quants/q8_0/unpack.aie.h:37-52
//   Q6_K  bf16_rne(d * sc * (q - 32))  src/quants/q6_k/unpack.aie.h:33-138
// The reference reaches these values through split bf16 scale terms; every
// product here is exact in fp32 (<= 23 significant bits) so one rounding
// (v_cvt_pk_bf16_f32, round-to-nearest-even) gives the same bits.
//
// Work item: one group of 8 consecutive output elements of one row, written
// as one 16-byte non-temporal store, so consecutive lanes store consecutive
// 16 bytes and the output streams to memory without occupying L2.
// Grids larger than 2^32 - 1 workgroups, or rows longer than 2^32 - 1 groups,
// are rejected with SPIRAL_ERR_SHAPE.
#include "common.h"
#include "dequant_impl.h"

namespace spiral {
namespace {

// A workgroup covers kDequantGroups groups of 8 elements of one row; row and
// group come from the workgroup index with one 32-bit scalar division, so no
// thread divides. Each thread converts two groups 256 apart (both loads
// issued before either is used), so each store instruction of a wave still
// writes 1 KiB of consecutive bytes.
constexpr int kDequantGroups = 512;
template <int TYPE>
__global__ void __launch_bounds__(256) dequant_kernel(const uint8_t* __restrict__ w, int64_t n_rows,
                                                      int64_t nb, uint32_t groups_per_row, uint32_t wg_per_row,
                                                      uint16_t* __restrict__ out, int64_t ld_out) {
  const uint32_t row = blockIdx.x / wg_per_row;
  const uint32_t g0 = (blockIdx.x - row * wg_per_row) * kDequantGroups + threadIdx.x;
  if (g0 >= groups_per_row) return;
  const uint32_t g1 = g0 + 256;
  const bool second = g1 < groups_per_row;
  float v[2][8];
  dequant8<TYPE>(w, n_rows, nb, row, g0, v[0]);
  dequant8<TYPE>(w, n_rows, nb, row, second ? g1 : g0, v[1]);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (h == 1 && !second) break;
    uint4 o;
    o.x = pack_bf16x2(v[h][0], v[h][1]);
    o.y = pack_bf16x2(v[h][2], v[h][3]);
    o.z = pack_bf16x2(v[h][4], v[h][5]);
    o.w = pack_bf16x2(v[h][6], v[h][7]);
    store_stream16(out + row * ld_out + 8 * (h ? g1 : g0), o);
  }
}

template <int TYPE, bool F32_OUT>
__global__ void __launch_bounds__(256) get_rows_kernel(const uint8_t* __restrict__ w, int64_t n_rows,
                                                       int64_t nb, uint32_t groups_per_row, uint32_t wg_per_row,
                                                       const int32_t* __restrict__ ids, void* __restrict__ out,
                                                       int64_t ld_out) {
  const uint32_t r = blockIdx.x / wg_per_row;
  const uint32_t g = (blockIdx.x - r * wg_per_row) * 256 + threadIdx.x;
  if (g >= groups_per_row) return;
  const int64_t n = ids[r];
  float v[8];
  if (n >= 0 && n < n_rows) {
    dequant8<TYPE>(w, n_rows, nb, n, g, v);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = 0.0f;
  }
  uint4 o;
  o.x = pack_bf16x2(v[0], v[1]);
  o.y = pack_bf16x2(v[2], v[3]);
  o.z = pack_bf16x2(v[4], v[5]);
  o.w = pack_bf16x2(v[6], v[7]);
  if constexpr (F32_OUT) {
    // The F32 output carries the same exact bf16 values, widened.
    float* p = static_cast<float*>(out) + r * ld_out + 8 * g;
    store_stream16(p, make_uint4(o.x << 16, o.x & 0xffff0000u, o.y << 16, o.y & 0xffff0000u));
    store_stream16(p + 4, make_uint4(o.z << 16, o.z & 0xffff0000u, o.w << 16, o.w & 0xffff0000u));
  } else {
    store_stream16(static_cast<uint16_t*>(out) + r * ld_out + 8 * g, o);
  }
}

}  // namespace
}  // namespace spiral

using namespace spiral;

extern "C" {

int spiral_dequant_bf16(int type, const void* w, int64_t n_rows, int64_t k, uint16_t* out,
                        int64_t ld_out, void* stream) {
  if (!is_quant_type(type)) return SPIRAL_ERR_TYPE;
  if (w == nullptr || out == nullptr) return SPIRAL_ERR_NULL;
  if (n_rows <= 0 || k <= 0 || k % block_elems(type) != 0 || ld_out < k) return SPIRAL_ERR_SHAPE;
  if (!aligned16(w) || !aligned16(out) || ld_out % 8 != 0) return SPIRAL_ERR_ALIGN;
  int rc = require_device();
  if (rc != SPIRAL_OK) return rc;
  const int64_t nb = k / block_elems(type), gpr = k / 8, wpr = ceil_div(gpr, kDequantGroups);
  if (gpr + 256 > UINT32_MAX || n_rows > UINT32_MAX || n_rows * wpr > UINT32_MAX) return SPIRAL_ERR_SHAPE;
  const dim3 grid(static_cast<unsigned>(n_rows * wpr));
  const uint32_t g32 = static_cast<uint32_t>(gpr), w32 = static_cast<uint32_t>(wpr);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint8_t* W = static_cast<const uint8_t*>(w);
#define SPIRAL_DEQUANT(T) \
  hipLaunchKernelGGL(dequant_kernel<T>, grid, dim3(256), 0, s, W, n_rows, nb, g32, w32, out, ld_out)
  switch (type) {
    case SPIRAL_TYPE_Q4_0: SPIRAL_DEQUANT(SPIRAL_TYPE_Q4_0); break;
    case SPIRAL_TYPE_Q8_0: SPIRAL_DEQUANT(SPIRAL_TYPE_Q8_0); break;
    case SPIRAL_TYPE_Q4_K: SPIRAL_DEQUANT(SPIRAL_TYPE_Q4_K); break;
    case SPIRAL_TYPE_Q5_K: SPIRAL_DEQUANT(SPIRAL_TYPE_Q5_K); break;
    case SPIRAL_TYPE_IQ4_NL: SPIRAL_DEQUANT(SPIRAL_TYPE_IQ4_NL); break;
    case SPIRAL_TYPE_IQ4_XS: SPIRAL_DEQUANT(SPIRAL_TYPE_IQ4_XS); break;
    default: SPIRAL_DEQUANT(SPIRAL_TYPE_Q6_K); break;
  }
#undef SPIRAL_DEQUANT
  return launch_status();
}

int spiral_get_rows(int type, const void* w, int64_t n_rows, int64_t k, const int32_t* ids,
                    int64_t n_ids, void* out, int out_type, int64_t ld_out, void* stream) {
  if (!is_quant_type(type)) return SPIRAL_ERR_TYPE;
  if (out_type != SPIRAL_TYPE_BF16 && out_type != SPIRAL_TYPE_F32) return SPIRAL_ERR_TYPE;
  if (n_ids == 0) return SPIRAL_OK;
  if (w == nullptr || out == nullptr || ids == nullptr) return SPIRAL_ERR_NULL;
  if (n_rows <= 0 || n_ids < 0 || k <= 0 || k % block_elems(type) != 0 || ld_out < k)
    return SPIRAL_ERR_SHAPE;
  if (!aligned16(w) || !aligned16(out) || ld_out % 8 != 0) return SPIRAL_ERR_ALIGN;
  int rc = require_device();
  if (rc != SPIRAL_OK) return rc;
  const int64_t nb = k / block_elems(type), gpr = k / 8, wpr = ceil_div(gpr, 256);
  if (gpr > UINT32_MAX || n_ids * wpr > UINT32_MAX) return SPIRAL_ERR_SHAPE;
  const dim3 grid(static_cast<unsigned>(n_ids * wpr));
  const uint32_t g32 = static_cast<uint32_t>(gpr), w32 = static_cast<uint32_t>(wpr);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint8_t* W = static_cast<const uint8_t*>(w);
#define SPIRAL_GET_ROWS(T)                                                                      \
  do {                                                                                          \
    if (out_type == SPIRAL_TYPE_F32)                                                            \
      hipLaunchKernelGGL((get_rows_kernel<T, true>), grid, dim3(256), 0, s, W, n_rows, nb, g32, \
                         w32, ids, out, ld_out);                                                \
    else                                                                                        \
      hipLaunchKernelGGL((get_rows_kernel<T, false>), grid, dim3(256), 0, s, W, n_rows, nb,     \
                         g32, w32, ids, out, ld_out);                                           \
  } while (0)
  switch (type) {
    case SPIRAL_TYPE_Q4_0: SPIRAL_GET_ROWS(SPIRAL_TYPE_Q4_0); break;
    case SPIRAL_TYPE_Q8_0: SPIRAL_GET_ROWS(SPIRAL_TYPE_Q8_0); break;
    case SPIRAL_TYPE_Q4_K: SPIRAL_GET_ROWS(SPIRAL_TYPE_Q4_K); break;
    case SPIRAL_TYPE_Q5_K: SPIRAL_GET_ROWS(SPIRAL_TYPE_Q5_K); break;
    case SPIRAL_TYPE_IQ4_NL: SPIRAL_GET_ROWS(SPIRAL_TYPE_IQ4_NL); break;
    case SPIRAL_TYPE_IQ4_XS: SPIRAL_GET_ROWS(SPIRAL_TYPE_IQ4_XS); break;
    default: SPIRAL_GET_ROWS(SPIRAL_TYPE_Q6_K); break;
  }
#undef SPIRAL_GET_ROWS
  return launch_status();
}

}  // extern "C"
