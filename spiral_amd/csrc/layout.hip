// Canonical GGUF <-> planar layout conversion, sizes, device queries.
//
// The planar layout splits each canonical block's fields into row-major
// planes (payload planes first, fp16 d last) so that every 16-byte payload
// vector is aligned for 128-bit loads. It is the GPU counterpart of the
// reference's load-time repack (src/quants/common/repack.h:5-7,
// src/quants/TODO.md:303-334): byte-count preserving, but a pure permutation
// (subnormal scales keep their bits; the kernels decode exponent 0 as +0, the
// value the reference's flush produces).
#include <mutex>
#include <unordered_map>
#include <vector>

#include "common.h"

namespace spiral {

int require_device() {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    return SPIRAL_ERR_NO_DEVICE;
  }
  return SPIRAL_OK;
}

int device_cu_count() {
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (dev >= static_cast<int>(cache.size())) cache.resize(dev + 1, 0);
  if (cache[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cache[dev] = cus;
  }
  return cache[dev];
}

// Resident workgroups per CU of a kernel at an LDS size (occupancy API,
// cached per device, kernel and LDS size).
int blocks_per_cu(const void* kernel, int threads, int64_t lds) {
  struct Key {
    int dev;
    const void* kernel;
    int64_t lds;
    bool operator==(const Key& o) const { return dev == o.dev && kernel == o.kernel && lds == o.lds; }
  };
  struct Hash {
    size_t operator()(const Key& k) const {
      return std::hash<const void*>()(k.kernel) ^ (std::hash<int64_t>()(k.lds) * 31u) ^ static_cast<size_t>(k.dev);
    }
  };
  static std::mutex mu;
  static std::unordered_map<Key, int, Hash> cache;
  int dev = 0;
  (void)hipGetDevice(&dev);
  const Key key{dev, kernel, lds};
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, static_cast<size_t>(lds)) != hipSuccess ||
      n <= 0) {
    (void)hipGetLastError();
    n = 1;
  }
  cache.emplace(key, n);
  return n;
}

// Raises a kernel's dynamic-LDS limit to `bytes` on the current device, once
// per device and kernel (the attribute is per device; the set is guarded so
// concurrent first launches from several threads are safe).
int allow_dynamic_lds(const void* kernel, int bytes) {
  static std::mutex mu;
  static std::unordered_map<const void*, std::vector<int>> done;  // kernel -> limit set, by device
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return SPIRAL_ERR_HIP;
  }
  std::lock_guard<std::mutex> lock(mu);
  std::vector<int>& v = done[kernel];
  if (dev >= static_cast<int>(v.size())) v.resize(dev + 1, 0);
  if (v[dev] >= bytes) return SPIRAL_OK;
  if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess) {
    (void)hipGetLastError();
    return SPIRAL_ERR_HIP;
  }
  v[dev] = bytes;
  return SPIRAL_OK;
}

namespace {

__device__ __forceinline__ uint32_t u16x2(const uint16_t* p) {
  return static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 16);
}

__device__ __forceinline__ uint4 load16_u16(const uint16_t* p) {
  return make_uint4(u16x2(p), u16x2(p + 2), u16x2(p + 4), u16x2(p + 6));
}

__device__ __forceinline__ void store16_u16(uint16_t* p, uint4 v) {
  p[0] = v.x & 0xffff; p[1] = v.x >> 16; p[2] = v.y & 0xffff; p[3] = v.y >> 16;
  p[4] = v.z & 0xffff; p[5] = v.z >> 16; p[6] = v.w & 0xffff; p[7] = v.w >> 16;
}

// One thread per canonical block. Canonical blocks are only 2-byte aligned
// (18/34/210-byte strides), so they are moved as 16-bit words; the planar
// side is written with aligned 16-byte stores.
template <int TYPE>
__global__ void to_planar_kernel(const uint8_t* __restrict__ src, int64_t stride,
                                 int64_t n_rows, int64_t nb, uint8_t* __restrict__ dst) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n_rows * nb) return;
  const int64_t n = i / nb, b = i % nb;
  const int64_t total = n_rows * nb;
  if constexpr (TYPE == SPIRAL_TYPE_Q4_0 || TYPE == SPIRAL_TYPE_IQ4_NL) {
    const uint16_t* s = reinterpret_cast<const uint16_t*>(src + n * stride + b * kQ4_0Bytes);
    reinterpret_cast<uint4*>(dst)[i] = load16_u16(s + 1);
    reinterpret_cast<uint16_t*>(dst + total * 16)[i] = s[0];
  } else if constexpr (TYPE == SPIRAL_TYPE_IQ4_XS) {
    // meta = canonical bytes 0..7 (d, scales_h, scales_l), qs = the last 128
    const uint16_t* s = reinterpret_cast<const uint16_t*>(src + n * stride + b * kIQ4_XSBytes);
    uint4* qs = reinterpret_cast<uint4*>(dst) + 8 * i;
#pragma unroll
    for (int j = 0; j < 8; ++j) qs[j] = load16_u16(s + 4 + 8 * j);
    reinterpret_cast<uint2*>(dst + total * 128)[i] = make_uint2(u16x2(s), u16x2(s + 2));
  } else if constexpr (TYPE == SPIRAL_TYPE_Q8_0) {
    const uint16_t* s = reinterpret_cast<const uint16_t*>(src + n * stride + b * kQ8_0Bytes);
    uint4* q = reinterpret_cast<uint4*>(dst) + 2 * i;
    q[0] = load16_u16(s + 1);
    q[1] = load16_u16(s + 9);
    reinterpret_cast<uint16_t*>(dst + total * 32)[i] = s[0];
  } else if constexpr (is_kquant(TYPE)) {
    // meta = canonical bytes 0..15; Q5_K qh = bytes 16..47; qs = the last 128.
    constexpr bool Q5 = TYPE == SPIRAL_TYPE_Q5_K;
    const uint16_t* s = reinterpret_cast<const uint16_t*>(src + n * stride + b * block_bytes(TYPE));
    uint4* qs = reinterpret_cast<uint4*>(dst) + 8 * i;
#pragma unroll
    for (int j = 0; j < 8; ++j) qs[j] = load16_u16(s + (Q5 ? 24 : 8) + 8 * j);
    if constexpr (Q5) {
      uint4* qh = reinterpret_cast<uint4*>(dst + total * 128) + 2 * i;
      qh[0] = load16_u16(s + 8);
      qh[1] = load16_u16(s + 16);
    }
    reinterpret_cast<uint4*>(dst + total * (Q5 ? 160 : 128))[i] = load16_u16(s);
  } else {
    const uint16_t* s = reinterpret_cast<const uint16_t*>(src + n * stride + b * kQ6_KBytes);
    uint4* ql = reinterpret_cast<uint4*>(dst) + 8 * i;
    uint4* qh = reinterpret_cast<uint4*>(dst + total * 128) + 4 * i;
    uint4* sc = reinterpret_cast<uint4*>(dst + total * 192) + i;
#pragma unroll
    for (int j = 0; j < 8; ++j) ql[j] = load16_u16(s + 8 * j);
#pragma unroll
    for (int j = 0; j < 4; ++j) qh[j] = load16_u16(s + 64 + 8 * j);
    sc[0] = load16_u16(s + 96);
    reinterpret_cast<uint16_t*>(dst + total * 208)[i] = s[104];
  }
}

template <int TYPE>
__global__ void from_planar_kernel(const uint8_t* __restrict__ src, int64_t n_rows, int64_t nb,
                                   uint8_t* __restrict__ dst, int64_t stride) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n_rows * nb) return;
  const int64_t n = i / nb, b = i % nb;
  const int64_t total = n_rows * nb;
  if constexpr (TYPE == SPIRAL_TYPE_Q4_0 || TYPE == SPIRAL_TYPE_IQ4_NL) {
    uint16_t* o = reinterpret_cast<uint16_t*>(dst + n * stride + b * kQ4_0Bytes);
    o[0] = reinterpret_cast<const uint16_t*>(src + total * 16)[i];
    store16_u16(o + 1, reinterpret_cast<const uint4*>(src)[i]);
  } else if constexpr (TYPE == SPIRAL_TYPE_IQ4_XS) {
    uint16_t* o = reinterpret_cast<uint16_t*>(dst + n * stride + b * kIQ4_XSBytes);
    const uint4* qs = reinterpret_cast<const uint4*>(src) + 8 * i;
#pragma unroll
    for (int j = 0; j < 8; ++j) store16_u16(o + 4 + 8 * j, qs[j]);
    const uint2 m = reinterpret_cast<const uint2*>(src + total * 128)[i];
    o[0] = m.x & 0xffff; o[1] = m.x >> 16; o[2] = m.y & 0xffff; o[3] = m.y >> 16;
  } else if constexpr (TYPE == SPIRAL_TYPE_Q8_0) {
    uint16_t* o = reinterpret_cast<uint16_t*>(dst + n * stride + b * kQ8_0Bytes);
    const uint4* q = reinterpret_cast<const uint4*>(src) + 2 * i;
    o[0] = reinterpret_cast<const uint16_t*>(src + total * 32)[i];
    store16_u16(o + 1, q[0]);
    store16_u16(o + 9, q[1]);
  } else if constexpr (is_kquant(TYPE)) {
    constexpr bool Q5 = TYPE == SPIRAL_TYPE_Q5_K;
    uint16_t* o = reinterpret_cast<uint16_t*>(dst + n * stride + b * block_bytes(TYPE));
    const uint4* qs = reinterpret_cast<const uint4*>(src) + 8 * i;
#pragma unroll
    for (int j = 0; j < 8; ++j) store16_u16(o + (Q5 ? 24 : 8) + 8 * j, qs[j]);
    if constexpr (Q5) {
      const uint4* qh = reinterpret_cast<const uint4*>(src + total * 128) + 2 * i;
      store16_u16(o + 8, qh[0]);
      store16_u16(o + 16, qh[1]);
    }
    store16_u16(o, reinterpret_cast<const uint4*>(src + total * (Q5 ? 160 : 128))[i]);
  } else {
    uint16_t* o = reinterpret_cast<uint16_t*>(dst + n * stride + b * kQ6_KBytes);
    const uint4* ql = reinterpret_cast<const uint4*>(src) + 8 * i;
    const uint4* qh = reinterpret_cast<const uint4*>(src + total * 128) + 4 * i;
    const uint4* sc = reinterpret_cast<const uint4*>(src + total * 192) + i;
#pragma unroll
    for (int j = 0; j < 8; ++j) store16_u16(o + 8 * j, ql[j]);
#pragma unroll
    for (int j = 0; j < 4; ++j) store16_u16(o + 64 + 8 * j, qh[j]);
    store16_u16(o + 96, sc[0]);
    o[104] = reinterpret_cast<const uint16_t*>(src + total * 208)[i];
  }
}

int check_layout_args(int type, const void* a, const void* b, int64_t n_rows, int64_t k,
                      int64_t stride) {
  if (!is_quant_type(type)) return SPIRAL_ERR_TYPE;
  if (a == nullptr || b == nullptr) return SPIRAL_ERR_NULL;
  if (n_rows <= 0 || k <= 0 || k % block_elems(type) != 0) return SPIRAL_ERR_SHAPE;
  if (spiral_tensor_bytes(type, n_rows, k) == 0) return SPIRAL_ERR_SHAPE;
  int64_t span = 0;
  if (stride < spiral_row_bytes(type, k) || (stride & 1) || __builtin_mul_overflow(n_rows, stride, &span))
    return SPIRAL_ERR_SHAPE;
  if ((reinterpret_cast<uintptr_t>(a) & 1) || (reinterpret_cast<uintptr_t>(b) & 1))
    return SPIRAL_ERR_ALIGN;
  return SPIRAL_OK;
}

}  // namespace
}  // namespace spiral

using namespace spiral;

extern "C" {

const char* spiral_status_string(int status) {
  switch (status) {
    case SPIRAL_OK: return "ok";
    case SPIRAL_ERR_SHAPE: return "invalid shape";
    case SPIRAL_ERR_ALIGN: return "misaligned pointer";
    case SPIRAL_ERR_NULL: return "null pointer";
    case SPIRAL_ERR_NO_DEVICE: return "no HIP device";
    case SPIRAL_ERR_HIP: return "HIP runtime error";
    case SPIRAL_ERR_TYPE: return "unsupported type";
    case SPIRAL_ERR_CAPACITY: return "buffer too small";
    case SPIRAL_ERR_RANGE: return "index out of range";
    default: return "unknown status";
  }
}

int spiral_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

// Both return 0 for a shape the type cannot hold and for byte counts past
// INT64_MAX.
int64_t spiral_row_bytes(int type, int64_t k) {
  const int be = block_elems(type);
  if (be == 0 || k <= 0 || k % be != 0) return 0;
  int64_t bytes = 0;
  return __builtin_mul_overflow(k / be, static_cast<int64_t>(block_bytes(type)), &bytes) ? 0 : bytes;
}

int64_t spiral_tensor_bytes(int type, int64_t n_rows, int64_t k) {
  if (n_rows <= 0) return 0;
  int64_t bytes = 0;
  return __builtin_mul_overflow(n_rows, spiral_row_bytes(type, k), &bytes) ? 0 : bytes;
}

int spiral_to_planar(int type, const void* src, int64_t src_row_stride, int64_t n_rows,
                     int64_t k, void* dst, void* stream) {
  int rc = check_layout_args(type, src, dst, n_rows, k, src_row_stride);
  if (rc != SPIRAL_OK) return rc;
  if (!aligned16(dst)) return SPIRAL_ERR_ALIGN;
  if ((rc = require_device()) != SPIRAL_OK) return rc;
  const int64_t nb = k / block_elems(type);
  const int64_t total = n_rows * nb;
  const dim3 grid(static_cast<unsigned>(ceil_div(total, 256)));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint8_t* in = static_cast<const uint8_t*>(src);
  uint8_t* out = static_cast<uint8_t*>(dst);
#define SPIRAL_TO_PLANAR(T) \
  hipLaunchKernelGGL(to_planar_kernel<T>, grid, dim3(256), 0, s, in, src_row_stride, n_rows, nb, out)
  switch (type) {
    case SPIRAL_TYPE_Q4_0: SPIRAL_TO_PLANAR(SPIRAL_TYPE_Q4_0); break;
    case SPIRAL_TYPE_Q8_0: SPIRAL_TO_PLANAR(SPIRAL_TYPE_Q8_0); break;
    case SPIRAL_TYPE_Q4_K: SPIRAL_TO_PLANAR(SPIRAL_TYPE_Q4_K); break;
    case SPIRAL_TYPE_Q5_K: SPIRAL_TO_PLANAR(SPIRAL_TYPE_Q5_K); break;
    case SPIRAL_TYPE_IQ4_NL: SPIRAL_TO_PLANAR(SPIRAL_TYPE_IQ4_NL); break;
    case SPIRAL_TYPE_IQ4_XS: SPIRAL_TO_PLANAR(SPIRAL_TYPE_IQ4_XS); break;
    default: SPIRAL_TO_PLANAR(SPIRAL_TYPE_Q6_K); break;
  }
#undef SPIRAL_TO_PLANAR
  return launch_status();
}

int spiral_from_planar(int type, const void* src, int64_t n_rows, int64_t k, void* dst,
                       int64_t dst_row_stride, void* stream) {
  int rc = check_layout_args(type, src, dst, n_rows, k, dst_row_stride);
  if (rc != SPIRAL_OK) return rc;
  if (!aligned16(src)) return SPIRAL_ERR_ALIGN;
  if ((rc = require_device()) != SPIRAL_OK) return rc;
  const int64_t nb = k / block_elems(type);
  const int64_t total = n_rows * nb;
  const dim3 grid(static_cast<unsigned>(ceil_div(total, 256)));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint8_t* in = static_cast<const uint8_t*>(src);
  uint8_t* out = static_cast<uint8_t*>(dst);
#define SPIRAL_FROM_PLANAR(T) \
  hipLaunchKernelGGL(from_planar_kernel<T>, grid, dim3(256), 0, s, in, n_rows, nb, out, dst_row_stride)
  switch (type) {
    case SPIRAL_TYPE_Q4_0: SPIRAL_FROM_PLANAR(SPIRAL_TYPE_Q4_0); break;
    case SPIRAL_TYPE_Q8_0: SPIRAL_FROM_PLANAR(SPIRAL_TYPE_Q8_0); break;
    case SPIRAL_TYPE_Q4_K: SPIRAL_FROM_PLANAR(SPIRAL_TYPE_Q4_K); break;
    case SPIRAL_TYPE_Q5_K: SPIRAL_FROM_PLANAR(SPIRAL_TYPE_Q5_K); break;
    case SPIRAL_TYPE_IQ4_NL: SPIRAL_FROM_PLANAR(SPIRAL_TYPE_IQ4_NL); break;
    case SPIRAL_TYPE_IQ4_XS: SPIRAL_FROM_PLANAR(SPIRAL_TYPE_IQ4_XS); break;
    default: SPIRAL_FROM_PLANAR(SPIRAL_TYPE_Q6_K); break;
  }
#undef SPIRAL_FROM_PLANAR
  return launch_status();
}

}  // extern "C"
