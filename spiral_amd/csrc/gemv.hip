// Decode GEMV over planar quantized weights: y[n] = sum_k W[n][k] * x[k].
//
// Bandwidth-bound streaming kernel (the reference's fused unpack_mmul at
// M = 1: src/quants/q4_0/mmul.aie.h:16-90, src/quants/q8_0/mmul.aie.h:16-117,
// src/quants/q6_k/mmul.aie.h:18-84).
//
// Structure
//  - A workgroup of 4 waves stages x once into LDS in the form its format's
//    inner loop wants (see stage_x), then walks rows persistently: wave w of
//    workgroup g takes row groups w + 4g, w + 4g + 4*gridDim, ...
//  - A "task" is the unit one lane consumes per 16-byte payload load(s):
//      Q4_0: one block (16 B qs + fp16 d) = 32 weights
//      Q8_0: half a block (16 B qs + d)   = 16 weights
//      Q6_K: a quarter super-block (2x16 B ql + 16 B qh + 4 sub-scales + d)
//            = 64 weights
//    Lane l of a wave takes tasks l, l + 64, ... of its row group, so every
//    payload load instruction of the wave reads 1 KiB of contiguous bytes.
//  - Each lane keeps an fp32 partial sum per row; a wave butterfly reduction
//    finishes the row.
//
// Arithmetic (fp32 accumulation throughout):
//  - Codes are used in an unsigned offset form and the offset is removed once
//    per task with a precomputed sum of x over the task's k range:
//      sum (q - c) x = sum q' x - c' * sum x.
//  - Q4_0 builds bf16 pairs (128 + q) straight from the nibbles with one
//    and-or each and multiplies them against bf16 x pairs with
//    v_dot2_f32_bf16; Q8_0 and Q6_K convert codes with v_cvt_f32_ubyte and
//    use fp32 FMAs against fp32 x.
//  - Weights are not rounded to bf16 first (the block scale multiplies the
//    block sum), so results differ from the bf16-weight product by rounding
//    only; tests bound that difference.
#include <algorithm>

#include "common.h"

namespace spiral {
namespace {

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

constexpr int kGemvWaves = 4;
constexpr int kGemvThreads = 64 * kGemvWaves;

template <int TYPE>
struct GemvTraits;

// Q4_0: task = one block. LDS: x as bf16 pairs permuted to the nibble order
// of the and-or extraction (16 pairs per block), then one fp32 x-sum per block.
template <>
struct GemvTraits<SPIRAL_TYPE_Q4_0> {
  static __host__ __device__ int64_t tasks_per_row(int64_t k) { return k / 32; }
  static __host__ __device__ int64_t lds_bytes(int64_t k) { return k * 2 + (k / 32) * 4; }
};
// Q8_0: task = 16 codes. LDS: fp32 x, then one fp32 sum per 16 elements.
template <>
struct GemvTraits<SPIRAL_TYPE_Q8_0> {
  static __host__ __device__ int64_t tasks_per_row(int64_t k) { return k / 16; }
  static __host__ __device__ int64_t lds_bytes(int64_t k) { return k * 4 + (k / 16) * 4; }
};
// Q6_K: task = 64 codes (h, 16-lane half). LDS as Q8_0.
template <>
struct GemvTraits<SPIRAL_TYPE_Q6_K> {
  static __host__ __device__ int64_t tasks_per_row(int64_t k) { return k / 64; }
  static __host__ __device__ int64_t lds_bytes(int64_t k) { return k * 4 + (k / 16) * 4; }
};

// ---- x staging ---------------------------------------------------------------

template <int TYPE>
__device__ void stage_x(const uint16_t* __restrict__ x, int64_t k, uint8_t* lds) {
  if constexpr (TYPE == SPIRAL_TYPE_Q4_0) {
    // Block b's 32 x values become 16 bf16 pairs, in the order the task loop
    // consumes them: for qs dword i (bytes 4i..4i+3) the pairs
    // (x[4i], x[4i+2]) (x[4i+16], x[4i+18]) (x[4i+1], x[4i+3])
    // (x[4i+17], x[4i+19]) match nibble fields at bit offsets 0, 4, 8, 12.
    uint32_t* pairs = reinterpret_cast<uint32_t*>(lds);
    float* sums = reinterpret_cast<float*>(lds + k * 2);
    const int64_t nb = k / 32;
    for (int64_t b = threadIdx.x; b < nb; b += blockDim.x) {
      const uint4* src = reinterpret_cast<const uint4*>(x + b * 32);
      uint32_t v[16];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 t = src[j];
        v[4 * j + 0] = t.x; v[4 * j + 1] = t.y; v[4 * j + 2] = t.z; v[4 * j + 3] = t.w;
      }
      // v[m] holds x[2m] (low half) and x[2m+1] (high half).
      auto xe = [&](int e) -> uint32_t { return (e & 1) ? (v[e >> 1] >> 16) : (v[e >> 1] & 0xffffu); };
      float s = 0.0f;
#pragma unroll
      for (int e = 0; e < 32; ++e) s += __uint_as_float(xe(e) << 16);
      uint4* dst = reinterpret_cast<uint4*>(pairs + b * 16);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dst[i] = make_uint4(xe(4 * i) | (xe(4 * i + 2) << 16), xe(4 * i + 16) | (xe(4 * i + 18) << 16),
                            xe(4 * i + 1) | (xe(4 * i + 3) << 16), xe(4 * i + 17) | (xe(4 * i + 19) << 16));
      }
      sums[b] = s;
    }
  } else {
    float* xf = reinterpret_cast<float*>(lds);
    float* sums = reinterpret_cast<float*>(lds + k * 4);
    const int64_t nc = k / 16;
    for (int64_t c = threadIdx.x; c < nc; c += blockDim.x) {
      const uint4* src = reinterpret_cast<const uint4*>(x + c * 16);
      const uint4 a = src[0], b = src[1];
      const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      float f[16];
      float s = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        f[2 * j] = bf16_lo(w[j]);
        f[2 * j + 1] = bf16_hi(w[j]);
        s += f[2 * j] + f[2 * j + 1];
      }
      float4* dst = reinterpret_cast<float4*>(xf + c * 16);
#pragma unroll
      for (int j = 0; j < 4; ++j) dst[j] = make_float4(f[4 * j], f[4 * j + 1], f[4 * j + 2], f[4 * j + 3]);
      sums[c] = s;
    }
  }
}

// ---- per-task payload and compute -------------------------------------------

template <int TYPE>
struct Task;

template <>
struct Task<SPIRAL_TYPE_Q4_0> {
  uint4 q;
  uint32_t d;
  __device__ __forceinline__ void load(const PlanarQ4_0& P, int64_t blk) {
    q = load_stream16(reinterpret_cast<const uint4*>(P.qs) + blk);
    d = P.d[blk];
  }
  __device__ __forceinline__ float compute(const uint8_t* lds, int64_t k, int64_t t) const {
    const uint4* xp = reinterpret_cast<const uint4*>(lds) + t * 4;
    const float xs = reinterpret_cast<const float*>(lds + k * 2)[t];
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 xv = xp[i];
      const uint32_t m = 0x000F000Fu, o = 0x43004300u;
      const uint32_t t0 = (w[i] & m) | o;
      const uint32_t t1 = ((w[i] >> 4) & m) | o;
      const uint32_t t2 = ((w[i] >> 8) & m) | o;
      const uint32_t t3 = ((w[i] >> 12) & m) | o;
      s0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, t0), __builtin_bit_cast(bf16x2_t, xv.x), s0, false);
      s1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, t1), __builtin_bit_cast(bf16x2_t, xv.y), s1, false);
      s0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, t2), __builtin_bit_cast(bf16x2_t, xv.z), s0, false);
      s1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, t3), __builtin_bit_cast(bf16x2_t, xv.w), s1, false);
    }
    // bf16 (128 + q) against x: remove 136 * sum(x) to get sum (q - 8) x.
    return fp16_scale(d) * ((s0 + s1) - 136.0f * xs);
  }
};

template <>
struct Task<SPIRAL_TYPE_Q8_0> {
  uint4 q;
  uint32_t d;
  __device__ __forceinline__ void load(const PlanarQ8_0& P, int64_t blk2) {
    q = load_stream16(reinterpret_cast<const uint4*>(P.qs) + blk2);
    d = P.d[blk2 >> 1];
  }
  __device__ __forceinline__ float compute(const uint8_t* lds, int64_t k, int64_t t) const {
    const float4* xp = reinterpret_cast<const float4*>(lds) + t * 4;
    const float xs = reinterpret_cast<const float*>(lds + k * 4)[t];
    const uint32_t w[4] = {q.x ^ 0x80808080u, q.y ^ 0x80808080u, q.z ^ 0x80808080u, q.w ^ 0x80808080u};
    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 xv = xp[i];
      // (q ^ 0x80) read as unsigned is q + 128.
      s0 = __builtin_fmaf(static_cast<float>(w[i] & 0xffu), xv.x, s0);
      s1 = __builtin_fmaf(static_cast<float>((w[i] >> 8) & 0xffu), xv.y, s1);
      s0 = __builtin_fmaf(static_cast<float>((w[i] >> 16) & 0xffu), xv.z, s0);
      s1 = __builtin_fmaf(static_cast<float>(w[i] >> 24), xv.w, s1);
    }
    return fp16_scale(d) * ((s0 + s1) - 128.0f * xs);
  }
};

template <>
struct Task<SPIRAL_TYPE_Q6_K> {
  uint4 a, b, h;
  uint2 sc;
  uint32_t d;
  int half16;  // 0 or 1: which 16-element half of the 32-lane l range
  __device__ __forceinline__ void load(const PlanarQ6_K& P, int64_t sb, int u) {
    // u = 2*h + half: elements 128h + 32j + 16*half + i, i < 16, j < 4.
    const int hh = u >> 1;
    half16 = u & 1;
    const uint8_t* ql = P.ql + sb * 128 + 64 * hh + 16 * half16;
    a = load_stream16(ql);       // j = 0 (low), 2 (high)
    b = load_stream16(ql + 32);  // j = 1 (low), 3 (high)
    h = load_stream16(P.qh + sb * 64 + 32 * hh + 16 * half16);
    sc = *reinterpret_cast<const uint2*>(P.sc + sb * 16 + 8 * hh);
    d = P.d[sb];
  }
  __device__ __forceinline__ float compute(const uint8_t* lds, int64_t k, int64_t kbase) const {
    // kbase = first element of j = 0; j adds 32.
    const float* xf = reinterpret_cast<const float*>(lds);
    const float* xs = reinterpret_cast<const float*>(lds + k * 4);
    const uint32_t A[4] = {a.x, a.y, a.z, a.w}, B[4] = {b.x, b.y, b.z, b.w}, H[4] = {h.x, h.y, h.z, h.w};
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t q[4] = {
          (A[i] & 0x0F0F0F0Fu) | ((H[i] << 4) & 0x30303030u),
          (B[i] & 0x0F0F0F0Fu) | ((H[i] << 2) & 0x30303030u),
          ((A[i] >> 4) & 0x0F0F0F0Fu) | (H[i] & 0x30303030u),
          ((B[i] >> 4) & 0x0F0F0F0Fu) | ((H[i] >> 2) & 0x30303030u),
      };
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 xv = *reinterpret_cast<const float4*>(xf + kbase + 32 * j + 4 * i);
        s[j] = __builtin_fmaf(static_cast<float>(q[j] & 0xffu), xv.x, s[j]);
        s[j] = __builtin_fmaf(static_cast<float>((q[j] >> 8) & 0xffu), xv.y, s[j]);
        s[j] = __builtin_fmaf(static_cast<float>((q[j] >> 16) & 0xffu), xv.z, s[j]);
        s[j] = __builtin_fmaf(static_cast<float>(q[j] >> 24), xv.w, s[j]);
      }
    }
    // Sub-scale of group j is sc[8h + half + 2j]: bytes half, half+2, half+4,
    // half+6 of the 8 sub-scales loaded for this h.
    const uint32_t s0 = half16 ? (sc.x >> 8) : sc.x;
    const uint32_t s1 = half16 ? (sc.y >> 8) : sc.y;
    const float c0 = static_cast<float>(static_cast<int8_t>(s0 & 0xffu));
    const float c1 = static_cast<float>(static_cast<int8_t>((s0 >> 16) & 0xffu));
    const float c2 = static_cast<float>(static_cast<int8_t>(s1 & 0xffu));
    const float c3 = static_cast<float>(static_cast<int8_t>((s1 >> 16) & 0xffu));
    const int64_t c16 = kbase >> 4;
    float acc = c0 * (s[0] - 32.0f * xs[c16]);
    acc = __builtin_fmaf(c1, s[1] - 32.0f * xs[c16 + 2], acc);
    acc = __builtin_fmaf(c2, s[2] - 32.0f * xs[c16 + 4], acc);
    acc = __builtin_fmaf(c3, s[3] - 32.0f * xs[c16 + 6], acc);
    return fp16_scale(d) * acc;
  }
};

// One lane's task: where it is and its loaded payload.
template <int TYPE>
struct Slot {
  Task<TYPE> task;
  int64_t t;  // task index within its row
  __device__ __forceinline__ void load(const void* w, int64_t n_rows, int64_t nb, int64_t n,
                                       int64_t t_) {
    t = t_;
    if constexpr (TYPE == SPIRAL_TYPE_Q4_0) {
      task.load(PlanarQ4_0(w, n_rows, nb), n * nb + t);
    } else if constexpr (TYPE == SPIRAL_TYPE_Q8_0) {
      task.load(PlanarQ8_0(w, n_rows, nb), n * nb * 2 + t);
    } else {
      task.load(PlanarQ6_K(w, n_rows, nb), n * nb + (t >> 2), static_cast<int>(t & 3));
    }
  }
  __device__ __forceinline__ float compute(const uint8_t* lds, int64_t k) const {
    if constexpr (TYPE == SPIRAL_TYPE_Q6_K) {
      const int64_t kbase = (t >> 2) * 256 + ((t >> 1) & 1) * 128 + (t & 1) * 16;
      return task.compute(lds, k, kbase);
    } else {
      return task.compute(lds, k, t);
    }
  }
};

// Tasks of a row group (RPW rows) are numbered flat, f = r * T + t; lane l
// takes f = l, l + 64, ... in chunks of UNROLL. All UNROLL payload loads of a
// chunk are issued before the first is consumed; slots past the end load a
// valid task of the group's first row and are discarded.
template <int TYPE, int RPW, int UNROLL, bool F32_OUT>
__global__ void __launch_bounds__(kGemvThreads) gemv_kernel(const void* __restrict__ w, int64_t n_rows,
                                                            int64_t k, const uint16_t* __restrict__ x,
                                                            void* __restrict__ y) {
  extern __shared__ __align__(16) uint8_t lds[];
  stage_x<TYPE>(x, k, lds);
  __syncthreads();

  using Tr = GemvTraits<TYPE>;
  const int64_t nb = k / block_elems(TYPE);
  const int64_t T = Tr::tasks_per_row(k);
  const int64_t flat = RPW * T;
  const int lane = threadIdx.x & 63;
  const int64_t wave = blockIdx.x * kGemvWaves + (threadIdx.x >> 6);
  const int64_t n_waves = static_cast<int64_t>(gridDim.x) * kGemvWaves;
  const int64_t n_groups = (n_rows + RPW - 1) / RPW;

  for (int64_t g = wave; g < n_groups; g += n_waves) {
    const int64_t row0 = g * RPW;
    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
    for (int64_t f0 = lane; f0 < flat; f0 += 64 * UNROLL) {
      Slot<TYPE> slot[UNROLL];
      int rsel[UNROLL];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const int64_t f = f0 + 64 * u;
        const int64_t r = f / T;
        const bool valid = f < flat && row0 + r < n_rows;
        rsel[u] = valid ? static_cast<int>(r) : -1;
        const int64_t rr = valid ? r : 0;
        slot[u].load(w, n_rows, nb, row0 + rr, valid ? f - r * T : 0);
      }
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const float part = slot[u].compute(lds, k);
#pragma unroll
        for (int r = 0; r < RPW; ++r) acc[r] += (rsel[u] == r) ? part : 0.0f;
      }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const float v = wave_sum(acc[r]);
      if (lane == 0 && row0 + r < n_rows) {
        if constexpr (F32_OUT) {
          static_cast<float*>(y)[row0 + r] = v;
        } else {
          static_cast<__bf16*>(y)[row0 + r] = static_cast<__bf16>(v);
        }
      }
    }
  }
}

template <int TYPE, int RPW, int UNROLL>
int launch_gemv(const void* w, int64_t n_rows, int64_t k, const uint16_t* x, void* y, int y_type,
                hipStream_t s) {
  const int64_t lds = GemvTraits<TYPE>::lds_bytes(k);
  const int per_cu = static_cast<int>(std::min<int64_t>(8, std::max<int64_t>(1, (160 * 1024) / lds)));
  const int64_t groups = (n_rows + RPW - 1) / RPW;
  const int64_t want = ceil_div(groups, kGemvWaves);
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(want, static_cast<int64_t>(device_cu_count()) * per_cu));
  if (y_type == SPIRAL_TYPE_F32)
    hipLaunchKernelGGL((gemv_kernel<TYPE, RPW, UNROLL, true>), dim3(blocks), dim3(kGemvThreads), lds, s, w, n_rows, k, x, y);
  else
    hipLaunchKernelGGL((gemv_kernel<TYPE, RPW, UNROLL, false>), dim3(blocks), dim3(kGemvThreads), lds, s, w, n_rows, k, x, y);
  return launch_status();
}

}  // namespace

// Largest k the LDS-staged GEMV accepts (64 KiB of staged x).
int64_t gemv_max_k(int type) {
  int64_t k = 0;
  const int be = block_elems(type);
  if (be == 0) return 0;
  for (int64_t c = be;; c += be) {
    const int64_t lds = type == SPIRAL_TYPE_Q4_0   ? GemvTraits<SPIRAL_TYPE_Q4_0>::lds_bytes(c)
                        : type == SPIRAL_TYPE_Q8_0 ? GemvTraits<SPIRAL_TYPE_Q8_0>::lds_bytes(c)
                                                   : GemvTraits<SPIRAL_TYPE_Q6_K>::lds_bytes(c);
    if (lds > 64 * 1024) break;
    k = c;
  }
  return k;
}

// y[n] = sum_k W[n][k] x[k]; arguments validated by the caller.
int gemv(int type, const void* w, int64_t n_rows, int64_t k, const uint16_t* x, void* y, int y_type,
         hipStream_t s) {
  switch (type) {
    case SPIRAL_TYPE_Q4_0: return launch_gemv<SPIRAL_TYPE_Q4_0, 2, 2>(w, n_rows, k, x, y, y_type, s);
    case SPIRAL_TYPE_Q8_0: return launch_gemv<SPIRAL_TYPE_Q8_0, 1, 4>(w, n_rows, k, x, y, y_type, s);
    case SPIRAL_TYPE_Q6_K: return launch_gemv<SPIRAL_TYPE_Q6_K, 2, 2>(w, n_rows, k, x, y, y_type, s);
    default: return SPIRAL_ERR_TYPE;
  }
}

}  // namespace spiral
