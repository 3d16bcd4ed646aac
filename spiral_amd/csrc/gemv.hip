// Decode GEMV over planar quantized weights: y[n] = sum_k W[n][k] * x[k].
//
// Bandwidth-bound streaming kernel (the reference's fused unpack_mmul at
// M = 1: src/quants/q4_0/mmul.aie.h:16-90, src/quants/q8_0/mmul.aie.h:16-117,
// src/quants/q6_k/mmul.aie.h:18-84).
//
// Work split
//  - A workgroup of WAVES waves stages x once into LDS in the form its
//    format's inner loop reads. Each wave owns a contiguous, balanced range
//    of rows; row indices are wave-uniform (scalar registers), so payload
//    addresses are a scalar row base plus a 32-bit lane offset.
//  - A row is cut into T "tasks", the unit one lane consumes per 16-byte
//    payload load(s):
//      Q4_0: one block (16 B qs + fp16 d)                          = 32 weights
//      Q8_0: half a block (16 B qs + d)                            = 16 weights
//      Q6_K: a quarter super-block (2x16 B ql, 16 B qh, 4 sub-scales, d)
//                                                                  = 64 weights
//            (exact form: an eighth, 2x8 B ql and 8 B qh         = 32 weights)
//    A "unit" is J tasks per lane: tasks 64 J p + 64 j + lane of a row (pass
//    p). Each payload load instruction of a wave reads 1 KiB of contiguous
//    bytes. When one pass covers the row (T <= 64 J), every lane's x slice is
//    the same for all rows and lives in registers (XREG); otherwise it is
//    read from LDS per unit. The exact kernel can also give a row G = 16 or
//    32 lanes, so that a unit covers four or two neighbouring rows (rows of
//    up to 256 tasks that are no multiple of 64); launch_exact picks the
//    unit shape of least estimated work.
//  - Units are software-pipelined: the payload of unit u + 1 is in flight
//    while unit u is computed, and the first unit is requested before x is
//    staged, so the HBM latency of the first loads overlaps the staging.
//  - LDS holds x in 16-byte entries blocked by 64 tasks: entry e of task t
//    sits at ((t / 64) E + e) KiB + (t % 64) 16 bytes, so a wave reading
//    entry e of its 64 tasks touches 1 KiB of consecutive LDS and e is an
//    immediate offset. Per-task sums of x follow the entries.
//  - A row's fp32 partial sums are reduced across the wave (or its lane
//    group) after its last pass with DPP (six adds for 64 lanes, the total
//    in the last lane), and that lane stores y.
//
// Arithmetic (fp32 accumulation throughout). Two modes share the kernel:
//  - Exact (the default, Exact<TYPE>): every weight is the dequantized bf16
//    value, bf16_rne(code * scale), the weight the reference's fused product
//    multiplies (src/quants/q8_0/mmul.aie.h:16-117 dequantizes each tile
//    before its mmul), and the same weight the small-batch, GEMM and MoE
//    kernels use, so a row's output does not depend on the batch it is
//    decoded in. Codes become fp16 pairs with one v_perm_b32 (a byte under
//    a fixed high byte), v_fma_mix_f32 forms code * scale exactly in fp32
//    ((B + code) * s - B * s with both terms exact, or a subnormal fp16
//    code against s * 2^24), v_cvt_pk_bf16_f32 rounds two of them to
//    nearest even, and v_dot2_f32_bf16 multiplies the pair against a bf16
//    x pair.
//  - Relaxed (Fmt<TYPE>, the spiral_gemv_relaxed entry point): the block
//    scale multiplies the block's fp32 sum, so codes are never rounded to
//    bf16 weights. That is the scale-after-mmul arithmetic the reference
//    keeps out of its exact tolerance (src/quants/NOTES.md:327-330) and
//    allows only as a named mode with its own check
//    (src/quants/TODO.md:132-135). Codes are turned into small floats with
//    an exact offset removed once per task with a precomputed sum of x:
//      sum (q - c) x = sum (q + B) x - (B + c) * sum x.
//    Q4_0 and Q6_K form bf16 pairs (128 + code) with one v_perm_b32 each
//    and multiply them against bf16 x pairs with v_dot2_f32_bf16; Q8_0 codes
//    (q + 128 up to 255) do not fit a bf16 mantissa, so it builds fp16 pairs
//    (1024 + q + 128) and multiplies each half against fp32 x with
//    v_fma_mix_f32.
#include <algorithm>

#include "common.h"

namespace spiral {
namespace {

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2_t;

constexpr int64_t kMaxLds = 64 * 1024;

// fp16 pairs (1024 + byte b0, 1024 + byte b2) and (1024 + b1, 1024 + b3) of
// a dword: bytes [b, 0x64] form the fp16 0x6400 | b.
__device__ __forceinline__ f16x2_t f16_even(uint32_t w) {
  return __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, w, 0x04020400u));
}
__device__ __forceinline__ f16x2_t f16_odd(uint32_t w) {
  return __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, w, 0x04030401u));
}

// sum over the 4 bytes of w (as 1024 + byte) times x[0..3], two chains.
__device__ __forceinline__ void mix4(uint32_t w, float x0, float x1, float x2, float x3, float& s0, float& s1) {
  const f16x2_t e = f16_even(w), o = f16_odd(w);
  s0 = __builtin_fmaf(static_cast<float>(e.x), x0, s0);
  s1 = __builtin_fmaf(static_cast<float>(o.x), x1, s1);
  s0 = __builtin_fmaf(static_cast<float>(e.y), x2, s0);
  s1 = __builtin_fmaf(static_cast<float>(o.y), x3, s1);
}

// bf16 pairs (128 + b0, 128 + b1) and (128 + b2, 128 + b3) of a dword of
// bytes below 128: bytes [b, 0x43] form the bf16 0x4300 | b.
__device__ __forceinline__ uint32_t bf16_01(uint32_t w) { return __builtin_amdgcn_perm(0x43434343u, w, 0x04010400u); }
__device__ __forceinline__ uint32_t bf16_23(uint32_t w) { return __builtin_amdgcn_perm(0x43434343u, w, 0x04030402u); }

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}

// Two exact weights as a bf16 pair: the bytes of w picked by SEL under the
// high byte HI form an fp16 pair h (v_perm_b32); each half becomes
// h * s + c in one v_fma_mix_f32 (the fp16 operand is widened exactly) and
// the two sums are rounded to nearest even into one bf16 pair. Callers pick
// HI, s and c so that h * s + c is the exact code * scale.
template <uint32_t HI, uint32_t SEL>
__device__ __forceinline__ uint32_t wpair(uint32_t w, float s, float c) {
  const f16x2_t h = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(HI, w, SEL));
  return pack_bf16x2(__builtin_fmaf(static_cast<float>(h.x), s, c), __builtin_fmaf(static_cast<float>(h.y), s, c));
}
// Byte selectors: bytes 0 and 1, or 2 and 3, of w into the low bytes of the
// two halves, the high bytes from HI.
constexpr uint32_t kSel01 = 0x04010400u, kSel23 = 0x04030402u;
// High bytes: 0x64 makes the fp16 1024 + b (exponent 10, step 1), 0x54 makes
// 64 + b / 16 (exponent 6, step 1/16), 0x00 the subnormal b * 2^-24.
constexpr uint32_t kHi1024 = 0x64646464u, kHi64 = 0x54545454u, kHiSub = 0u;
constexpr float kTwo24 = 16777216.0f;

// ---- buffer access for the exact kernel --------------------------------------
// Raw buffer resources over one wave's rows of a plane. An access whose
// offset has bit 31 set lies past the buffer (a wave's span is far below
// 2 GiB): loads return zeros and stores are dropped without touching
// memory, so the loop issues every access unconditionally and the compiler
// can wait for exactly the oldest ring slot.
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
constexpr uint32_t kSkip = 0x80000000u;
constexpr int kStreamAux = 2;  // nt: payload read once

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int64_t bytes) {
  // Third dword 0x00020000: raw (untyped) 32-bit accesses on gfx9-class GPUs.
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}
// Accesses take a per-lane offset v (constant across a wave's steps, plus
// bit 31 for a lane with nothing to read) and a wave-uniform offset s (the
// row and pass, in a scalar register). A unit past a wave's last reads
// through a buffer of no records (every access out of range).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_or_none(__amdgpu_buffer_rsrc_t r, bool none) {
  return none ? __builtin_amdgcn_make_buffer_rsrc(nullptr, 0, 0, 0x00020000) : r;
}
__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s) {
  const auto x = __builtin_amdgcn_raw_buffer_load_b128(r, v, s, kStreamAux);
  return make_uint4(x[0], x[1], x[2], x[3]);
}
__device__ __forceinline__ uint2 bload8(__amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s) {
  const auto x = __builtin_amdgcn_raw_buffer_load_b64(r, v, s, 0);
  return make_uint2(x[0], x[1]);
}
__device__ __forceinline__ uint32_t bload2(__amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, v, s, 0);
}

// Blocked LDS layout (see the header): byte offset of entry 0 of task t when
// a task has E 16-byte entries; entry e adds e KiB.
__host__ __device__ __forceinline__ uint32_t lds_task(int t, int E) {
  return static_cast<uint32_t>((t >> 6) * E) * 1024u + (static_cast<uint32_t>(t & 63) << 4);
}
__host__ __device__ __forceinline__ int64_t pad64(int64_t t) { return (t + 63) & ~int64_t(63); }

template <int TYPE>
struct Fmt;

// Staging: every workgroup copies x into LDS once. Items are handed out to
// threads K_STAGE at a time with all of an item's global loads issued before
// any is used, so a thread has up to K_STAGE * 32 bytes of x in flight.
constexpr int kStageUnroll = 4;

// ---- Q4_0 ------------------------------------------------------------------
// x entries per task (block): 4 x uint4 = its 32 bf16 x in order. Sum: float.
// Codes: for qs dword i, the low nibbles are elements 4i..4i+3 and the high
// nibbles elements 16+4i..16+4i+3; masked to bytes and widened to bf16 pairs
// (128 + c) with v_perm they line up with consecutive x pairs.
template <>
struct Fmt<SPIRAL_TYPE_Q4_0> {
  static constexpr int kTaskElems = 32, kE = 4;
  static __host__ __device__ int64_t lds_bytes(int64_t k) { return pad64(k / 32) * (kE * 16 + 4); }

  struct Row {
    const uint8_t* qs;
    const uint8_t* d;
  };
  static __device__ __forceinline__ Row row(const uint8_t* w, int64_t n_rows, int64_t k, int64_t r) {
    const int64_t nb = k / 32;
    return Row{w + r * nb * 16, w + n_rows * nb * 16 + r * nb * 2};
  }
  struct Payload {
    uint4 q;
    uint32_t d;
  };
  static __device__ __forceinline__ void load(Payload& p, const Row& R, int t) {
    const uint32_t ut = static_cast<uint32_t>(t);
    p.q = load_stream16(R.qs + ut * 16u);
    p.d = *reinterpret_cast<const uint16_t*>(R.d + ut * 2u);
  }
  struct X {
    uint4 xp[4];
    float sum;
  };
  static __device__ __forceinline__ void xload(X& x, const uint8_t* lds, int T, int t) {
    const uint8_t* e = lds + lds_task(t, kE);
#pragma unroll
    for (int i = 0; i < 4; ++i) x.xp[i] = *reinterpret_cast<const uint4*>(e + 1024 * i);
    x.sum = reinterpret_cast<const float*>(lds + pad64(T) * kE * 16)[t];
  }
  // Item = task: 32 x (4 x 16 B) and their sum.
  static __device__ void stage(const uint16_t* __restrict__ x, int64_t k, uint8_t* lds) {
    const int T = static_cast<int>(k / 32);
    float* xs = reinterpret_cast<float*>(lds + pad64(T) * kE * 16);
    const uint4* src = reinterpret_cast<const uint4*>(x);
    for (int b0 = threadIdx.x; b0 < T; b0 += kStageUnroll * blockDim.x) {
      uint4 v[kStageUnroll][4];
#pragma unroll
      for (int u = 0; u < kStageUnroll; ++u) {
        const int b = b0 + u * blockDim.x;
        if (b < T)
#pragma unroll
          for (int i = 0; i < 4; ++i) v[u][i] = src[4 * b + i];
      }
#pragma unroll
      for (int u = 0; u < kStageUnroll; ++u) {
        const int b = b0 + u * blockDim.x;
        if (b >= T) break;
        float s = 0.0f;
        uint8_t* dst = lds + lds_task(b, kE);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint4 q = v[u][i];
          s += (bf16_lo(q.x) + bf16_hi(q.x)) + (bf16_lo(q.y) + bf16_hi(q.y)) + (bf16_lo(q.z) + bf16_hi(q.z)) +
               (bf16_lo(q.w) + bf16_hi(q.w));
          *reinterpret_cast<uint4*>(dst + 1024 * i) = q;
        }
        xs[b] = s;
      }
    }
  }
  static __device__ __forceinline__ float dot(const Payload& p, const X& x) {
    const uint32_t w[4] = {p.q.x, p.q.y, p.q.z, p.q.w};
    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = w[i] & 0x0F0F0F0Fu, hi = (w[i] >> 4) & 0x0F0F0F0Fu;
      const uint4 el = x.xp[i >> 1], eh = x.xp[2 + (i >> 1)];
      s0 = dot2(bf16_01(lo), (i & 1) ? el.z : el.x, s0);
      s1 = dot2(bf16_23(lo), (i & 1) ? el.w : el.y, s1);
      s0 = dot2(bf16_01(hi), (i & 1) ? eh.z : eh.x, s0);
      s1 = dot2(bf16_23(hi), (i & 1) ? eh.w : eh.y, s1);
    }
    // bf16 (128 + c) against x: remove 136 * sum(x) to get sum (c - 8) x.
    return fp16_scale(p.d) * ((s0 + s1) - 136.0f * x.sum);
  }
};

// ---- Q8_0 ------------------------------------------------------------------
// x entries per task (half block): 4 x float4 = its 16 x. Sum: float.
template <>
struct Fmt<SPIRAL_TYPE_Q8_0> {
  static constexpr int kTaskElems = 16, kE = 4;
  static __host__ __device__ int64_t lds_bytes(int64_t k) { return pad64(k / 16) * (kE * 16 + 4); }

  struct Row {
    const uint8_t* qs;
    const uint8_t* d;
  };
  static __device__ __forceinline__ Row row(const uint8_t* w, int64_t n_rows, int64_t k, int64_t r) {
    const int64_t nb = k / 32;
    return Row{w + r * nb * 32, w + n_rows * nb * 32 + r * nb * 2};
  }
  struct Payload {
    uint4 q;
    uint32_t d;
  };
  static __device__ __forceinline__ void load(Payload& p, const Row& R, int t) {
    const uint32_t ut = static_cast<uint32_t>(t);
    p.q = load_stream16(R.qs + ut * 16u);
    p.d = *reinterpret_cast<const uint16_t*>(R.d + (ut >> 1) * 2u);
  }
  struct X {
    float4 x[4];
    float sum;
  };
  static __device__ __forceinline__ void xload(X& x, const uint8_t* lds, int T, int t) {
    const uint8_t* e = lds + lds_task(t, kE);
#pragma unroll
    for (int i = 0; i < 4; ++i) x.x[i] = *reinterpret_cast<const float4*>(e + 1024 * i);
    x.sum = reinterpret_cast<const float*>(lds + pad64(T) * kE * 16)[t];
  }
  // Item = task: 16 x (2 x 16 B) widened to fp32, and their sum.
  static __device__ void stage(const uint16_t* __restrict__ x, int64_t k, uint8_t* lds) {
    const int T = static_cast<int>(k / 16);
    float* xs = reinterpret_cast<float*>(lds + pad64(T) * kE * 16);
    const uint4* src = reinterpret_cast<const uint4*>(x);
    for (int c0 = threadIdx.x; c0 < T; c0 += kStageUnroll * blockDim.x) {
      uint4 v[kStageUnroll][2];
#pragma unroll
      for (int u = 0; u < kStageUnroll; ++u) {
        const int c = c0 + u * blockDim.x;
        if (c < T) {
          v[u][0] = src[2 * c];
          v[u][1] = src[2 * c + 1];
        }
      }
#pragma unroll
      for (int u = 0; u < kStageUnroll; ++u) {
        const int c = c0 + u * blockDim.x;
        if (c >= T) break;
        const uint32_t w[8] = {v[u][0].x, v[u][0].y, v[u][0].z, v[u][0].w, v[u][1].x, v[u][1].y, v[u][1].z, v[u][1].w};
        float s = 0.0f;
        uint8_t* dst = lds + lds_task(c, kE);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float4 f = make_float4(bf16_lo(w[2 * i]), bf16_hi(w[2 * i]), bf16_lo(w[2 * i + 1]), bf16_hi(w[2 * i + 1]));
          s += (f.x + f.y) + (f.z + f.w);
          *reinterpret_cast<float4*>(dst + 1024 * i) = f;
        }
        xs[c] = s;
      }
    }
  }
  static __device__ __forceinline__ float dot(const Payload& p, const X& x) {
    // (q ^ 0x80) read as unsigned is q + 128; as fp16 1024 + q + 128.
    const uint32_t w[4] = {p.q.x ^ 0x80808080u, p.q.y ^ 0x80808080u, p.q.z ^ 0x80808080u, p.q.w ^ 0x80808080u};
    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) mix4(w[i], x.x[i].x, x.x[i].y, x.x[i].z, x.x[i].w, s0, s1);
    return fp16_scale(p.d) * ((s0 + s1) - 1152.0f * x.sum);
  }
};

// ---- Q6_K ------------------------------------------------------------------
// Task u of a row = super-block u / 4, half h = (u >> 1) & 1, 16-lane half
// s = u & 1: elements 128 h + 32 j + 16 s + i for group j < 4, i < 16.
// x entries per task: 8 x uint4; entry 2 j + (i / 8) holds the 8 bf16 x of
// group j at i / 8 * 8 .. + 7, in order. Sum: float4, one per group.
template <>
struct Fmt<SPIRAL_TYPE_Q6_K> {
  static constexpr int kTaskElems = 64, kE = 8;
  static __host__ __device__ int64_t lds_bytes(int64_t k) { return pad64(k / 64) * (kE * 16 + 16); }

  struct Row {
    const uint8_t* ql;
    const uint8_t* qh;
    const uint8_t* sc;
    const uint8_t* d;
  };
  static __device__ __forceinline__ Row row(const uint8_t* w, int64_t n_rows, int64_t k, int64_t r) {
    const int64_t nb = k / 256, tot = n_rows * nb;
    return Row{w + r * nb * 128, w + tot * 128 + r * nb * 64, w + tot * 192 + r * nb * 16, w + tot * 208 + r * nb * 2};
  }
  struct Payload {
    uint4 a, b, h;
    uint32_t sc;  // the four sub-scales of the task's groups, one per byte
    uint32_t d;
  };
  static __device__ __forceinline__ void load(Payload& p, const Row& R, int u) {
    const uint32_t uu = static_cast<uint32_t>(u);
    const uint32_t sb = uu >> 2, hh = (uu >> 1) & 1u, s = uu & 1u;
    const uint32_t lo = sb * 128u + 64u * hh + 16u * s;
    p.a = load_stream16(R.ql + lo);        // groups 0 (low nibbles) and 2 (high)
    p.b = load_stream16(R.ql + lo + 32u);  // groups 1 (low) and 3 (high)
    p.h = load_stream16(R.qh + sb * 64u + 32u * hh + 16u * s);
    // Sub-scale of group j is sc[8 h + s + 2 j]: bytes s, s+2, s+4, s+6 of
    // the 8 sub-scales of half h.
    const uint2 sc8 = *reinterpret_cast<const uint2*>(R.sc + sb * 16u + 8u * hh);
    const uint32_t l = s ? (sc8.x >> 8) : sc8.x, hi = s ? (sc8.y >> 8) : sc8.y;
    p.sc = __builtin_amdgcn_perm(hi, l, 0x06040200u);
    p.d = *reinterpret_cast<const uint16_t*>(R.d + sb * 2u);
  }
  struct X {
    uint4 x[8];
    float4 sum;
  };
  static __device__ __forceinline__ void xload(X& x, const uint8_t* lds, int T, int u) {
    const uint8_t* e = lds + lds_task(u, kE);
#pragma unroll
    for (int i = 0; i < 8; ++i) x.x[i] = *reinterpret_cast<const uint4*>(e + 1024 * i);
    x.sum = reinterpret_cast<const float4*>(lds + pad64(T) * kE * 16)[u];
  }
  // Item = (task, group): 16 x (2 x 16 B) and their sum.
  static __device__ void stage(const uint16_t* __restrict__ x, int64_t k, uint8_t* lds) {
    const int T = static_cast<int>(k / 64);
    float* xs = reinterpret_cast<float*>(lds + pad64(T) * kE * 16);
    const int items = 4 * T;
    for (int e0 = threadIdx.x; e0 < items; e0 += kStageUnroll * blockDim.x) {
      uint4 v[kStageUnroll][2];
#pragma unroll
      for (int u = 0; u < kStageUnroll; ++u) {
        const int e = e0 + u * blockDim.x;
        if (e < items) {
          const int t = e >> 2, j = e & 3;
          const uint4* src = reinterpret_cast<const uint4*>(
              x + (t >> 2) * 256 + ((t >> 1) & 1) * 128 + (t & 1) * 16 + 32 * j);
          v[u][0] = src[0];
          v[u][1] = src[1];
        }
      }
#pragma unroll
      for (int u = 0; u < kStageUnroll; ++u) {
        const int e = e0 + u * blockDim.x;
        if (e >= items) break;
        const int t = e >> 2, j = e & 3;
        float s = 0.0f;
        uint8_t* dst = lds + lds_task(t, kE) + 1024 * (2 * j);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const uint4 q = v[u][i];
          s += (bf16_lo(q.x) + bf16_hi(q.x)) + (bf16_lo(q.y) + bf16_hi(q.y)) + (bf16_lo(q.z) + bf16_hi(q.z)) +
               (bf16_lo(q.w) + bf16_hi(q.w));
          *reinterpret_cast<uint4*>(dst + 1024 * i) = q;
        }
        xs[e] = s;
      }
    }
  }
  static __device__ __forceinline__ float dot(const Payload& p, const X& x) {
    const uint32_t A[4] = {p.a.x, p.a.y, p.a.z, p.a.w}, B[4] = {p.b.x, p.b.y, p.b.z, p.b.w};
    const uint32_t H[4] = {p.h.x, p.h.y, p.h.z, p.h.w};
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      // 6-bit codes of elements 4q .. 4q+3 of each group, one per byte.
      const uint32_t c[4] = {
          (A[q] & 0x0F0F0F0Fu) | ((H[q] << 4) & 0x30303030u),
          (B[q] & 0x0F0F0F0Fu) | ((H[q] << 2) & 0x30303030u),
          ((A[q] >> 4) & 0x0F0F0F0Fu) | (H[q] & 0x30303030u),
          ((B[q] >> 4) & 0x0F0F0F0Fu) | ((H[q] >> 2) & 0x30303030u),
      };
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 xv = x.x[2 * j + (q >> 1)];
        s[j] = dot2(bf16_01(c[j]), (q & 1) ? xv.z : xv.x, s[j]);
        s[j] = dot2(bf16_23(c[j]), (q & 1) ? xv.w : xv.y, s[j]);
      }
    }
    // bf16 (128 + code) against x: remove (128 + 32) * sum(x) per group.
    const float c0 = static_cast<float>(static_cast<int8_t>(p.sc & 0xffu));
    const float c1 = static_cast<float>(static_cast<int8_t>((p.sc >> 8) & 0xffu));
    const float c2 = static_cast<float>(static_cast<int8_t>((p.sc >> 16) & 0xffu));
    const float c3 = static_cast<float>(static_cast<int8_t>(p.sc >> 24));
    float acc = c0 * (s[0] - 160.0f * x.sum.x);
    acc = __builtin_fmaf(c1, s[1] - 160.0f * x.sum.y, acc);
    acc = __builtin_fmaf(c2, s[2] - 160.0f * x.sum.z, acc);
    acc = __builtin_fmaf(c3, s[3] - 160.0f * x.sum.w, acc);
    return fp16_scale(p.d) * acc;
  }
};

// ---- Q4_K / Q5_K --------------------------------------------------------------
// Task t of a row = qs bytes 16 t .. 16 t + 15: super-block t / 8, chunk
// c = (t / 2) % 4, half h = t % 2. Its low nibbles are elements
// 64 c + 16 h + i of group 2 c, its high nibbles elements 64 c + 32 + 16 h + i
// of group 2 c + 1 (i < 16); Q5_K adds bits 2 c and 2 c + 1 of
// qh[16 h + i]. The super-block's 16-byte meta entry (fp16 d, fp16 dmin,
// the packed 6-bit scales and mins) arrives in one load.
// x entries per task: 4 x uint4 (group 2c's 16 x, then group 2c+1's);
// sums: float2 (one per group).
//   sum_i x_i (d sc q_i - dmin m) = d sc (sum x (128 + q) - 128 sum x) - dmin m sum x
template <int TYPE>
struct FmtKQ {
  static constexpr int kTaskElems = 32, kE = 4;
  static constexpr bool kQ5 = TYPE == SPIRAL_TYPE_Q5_K;
  static __host__ __device__ int64_t lds_bytes(int64_t k) { return pad64(k / 32) * (kE * 16 + 8); }

  struct Row {
    const uint8_t* qs;
    const uint8_t* qh;
    const uint8_t* meta;
  };
  static __device__ __forceinline__ Row row(const uint8_t* w, int64_t n_rows, int64_t k, int64_t r) {
    const int64_t nb = k / 256, tot = n_rows * nb;
    return Row{w + r * nb * 128, w + tot * 128 + r * nb * 32, w + tot * (kQ5 ? 160 : 128) + r * nb * 16};
  }
  struct Payload {
    uint4 q, meta, qh;
    uint32_t c2;  // 2 c: the task's low-nibble group
  };
  static __device__ __forceinline__ void load(Payload& p, const Row& R, int t) {
    const uint32_t ut = static_cast<uint32_t>(t);
    p.q = load_stream16(R.qs + ut * 16u);
    p.meta = *reinterpret_cast<const uint4*>(R.meta + (ut >> 3) * 16u);
    if constexpr (kQ5) p.qh = load_stream16(R.qh + (ut >> 3) * 32u + (ut & 1u) * 16u);
    p.c2 = ut & 6u;
  }
  struct X {
    uint4 xp[4];
    float2 sum;
  };
  static __device__ __forceinline__ void xload(X& x, const uint8_t* lds, int T, int t) {
    const uint8_t* e = lds + lds_task(t, kE);
#pragma unroll
    for (int i = 0; i < 4; ++i) x.xp[i] = *reinterpret_cast<const uint4*>(e + 1024 * i);
    x.sum = reinterpret_cast<const float2*>(lds + pad64(T) * kE * 16)[t];
  }
  // Item = task: 2 x 16 x (2 x 16 B) and (SUMS) the two sums.
  template <bool SUMS = true>
  static __device__ void stage(const uint16_t* __restrict__ x, int64_t k, uint8_t* lds) {
    const int T = static_cast<int>(k / 32);
    float2* xs = reinterpret_cast<float2*>(lds + pad64(T) * kE * 16);
    for (int b0 = threadIdx.x; b0 < T; b0 += kStageUnroll * blockDim.x) {
      uint4 v[kStageUnroll][4];
#pragma unroll
      for (int u = 0; u < kStageUnroll; ++u) {
        const int b = b0 + u * blockDim.x;
        if (b < T) {
          const uint4* src = reinterpret_cast<const uint4*>(x + (b >> 3) * 256 + ((b >> 1) & 3) * 64 + (b & 1) * 16);
          v[u][0] = src[0];
          v[u][1] = src[1];
          v[u][2] = src[4];  // + 32 elements
          v[u][3] = src[5];
        }
      }
#pragma unroll
      for (int u = 0; u < kStageUnroll; ++u) {
        const int b = b0 + u * blockDim.x;
        if (b >= T) break;
        float s[2] = {0.0f, 0.0f};
        uint8_t* dst = lds + lds_task(b, kE);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint4 q = v[u][i];
          if constexpr (SUMS)
            s[i >> 1] += (bf16_lo(q.x) + bf16_hi(q.x)) + (bf16_lo(q.y) + bf16_hi(q.y)) +
                         (bf16_lo(q.z) + bf16_hi(q.z)) + (bf16_lo(q.w) + bf16_hi(q.w));
          *reinterpret_cast<uint4*>(dst + 1024 * i) = q;
        }
        if constexpr (SUMS) xs[b] = make_float2(s[0], s[1]);
      }
    }
  }
  static __device__ __forceinline__ float dot(const Payload& p, const X& x) {
    const uint32_t w[4] = {p.q.x, p.q.y, p.q.z, p.q.w};
    const uint32_t h[4] = {p.qh.x, p.qh.y, p.qh.z, p.qh.w};
    float a0 = 0.0f, a1 = 0.0f, b0 = 0.0f, b1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t lo = w[i] & 0x0F0F0F0Fu, hi = (w[i] >> 4) & 0x0F0F0F0Fu;
      if constexpr (kQ5) {
        lo |= ((h[i] >> p.c2) & 0x01010101u) << 4;
        hi |= ((h[i] >> (p.c2 + 1)) & 0x01010101u) << 4;
      }
      const uint4 el = x.xp[i >> 1], eh = x.xp[2 + (i >> 1)];
      a0 = dot2(bf16_01(lo), (i & 1) ? el.z : el.x, a0);
      a1 = dot2(bf16_23(lo), (i & 1) ? el.w : el.y, a1);
      b0 = dot2(bf16_01(hi), (i & 1) ? eh.z : eh.x, b0);
      b1 = dot2(bf16_23(hi), (i & 1) ? eh.w : eh.y, b1);
    }
    const uint32_t sm = kq_chunk_scales(p.meta.y, p.meta.z, p.meta.w, p.c2 >> 1);
    const float d = fp16_ieee(p.meta.x & 0xffffu), dmin = fp16_ieee(p.meta.x >> 16);
    // bf16 (128 + q) against x: remove 128 * sum(x) per group.
    const float gl = static_cast<float>(sm & 0xffu) * ((a0 + a1) - 128.0f * x.sum.x);
    const float gh = static_cast<float>((sm >> 16) & 0xffu) * ((b0 + b1) - 128.0f * x.sum.y);
    const float ml = static_cast<float>((sm >> 8) & 0xffu) * x.sum.x + static_cast<float>(sm >> 24) * x.sum.y;
    return d * (gl + gh) - dmin * ml;
  }
};
template <>
struct Fmt<SPIRAL_TYPE_Q4_K> : FmtKQ<SPIRAL_TYPE_Q4_K> {};
template <>
struct Fmt<SPIRAL_TYPE_Q5_K> : FmtKQ<SPIRAL_TYPE_Q5_K> {};

// ---- IQ4_NL / IQ4_XS -------------------------------------------------------------
// Task = 32 elements with one scale: an IQ4_NL block (16 qs bytes + fp16 d)
// or an IQ4_XS sub-block (16 qs bytes; task t is sub-block t % 8 of
// super-block t / 8, whose 8-byte meta entry (d, scales_h, scales_l) eight
// lanes share). qs dword i holds elements 4i..4i+3 (low nibbles) and
// 16+4i..16+4i+3 (high nibbles). Indices become codebook bytes kv + 128
// (iq4_lut), then fp16 pairs (1024 + kv + 128) with one v_perm_b32 each,
// multiplied against fp32 x with v_fma_mix_f32 (as Q8_0):
//   sum kv x = sum (1152 + kv) x - 1152 sum x.
// x entries per task: 8 x float4 (entries 0..3 the low-nibble elements of
// qs dwords 0..3, entries 4..7 the high-nibble ones). Sum: float.
template <int TYPE>
struct FmtIQ4 {
  static constexpr int kTaskElems = 32, kE = 8;
  static constexpr bool kXS = TYPE == SPIRAL_TYPE_IQ4_XS;
  static __host__ __device__ int64_t lds_bytes(int64_t k) { return pad64(k / 32) * (kE * 16 + 4); }

  struct Row {
    const uint8_t* qs;
    const uint8_t* d;  // IQ4_NL: fp16 d plane; IQ4_XS: meta plane
  };
  static __device__ __forceinline__ Row row(const uint8_t* w, int64_t n_rows, int64_t k, int64_t r) {
    if constexpr (kXS) {
      const int64_t nb = k / 256;
      return Row{w + r * nb * 128, w + n_rows * nb * 128 + r * nb * 8};
    } else {
      const int64_t nb = k / 32;
      return Row{w + r * nb * 16, w + n_rows * nb * 16 + r * nb * 2};
    }
  }
  struct Payload {
    uint4 q;
    uint2 m;   // IQ4_XS meta; IQ4_NL: d in m.x
    int sub;   // IQ4_XS sub-block
  };
  static __device__ __forceinline__ void load(Payload& p, const Row& R, int t) {
    const uint32_t ut = static_cast<uint32_t>(t);
    p.q = load_stream16(R.qs + ut * 16u);
    if constexpr (kXS) {
      p.m = *reinterpret_cast<const uint2*>(R.d + (ut >> 3) * 8u);
      p.sub = static_cast<int>(ut & 7u);
    } else {
      p.m = make_uint2(*reinterpret_cast<const uint16_t*>(R.d + ut * 2u), 0u);
      p.sub = 0;
    }
  }
  struct X {
    float4 x[8];
    float sum;
  };
  static __device__ __forceinline__ void xload(X& x, const uint8_t* lds, int T, int t) {
    const uint8_t* e = lds + lds_task(t, kE);
#pragma unroll
    for (int i = 0; i < 8; ++i) x.x[i] = *reinterpret_cast<const float4*>(e + 1024 * i);
    x.sum = reinterpret_cast<const float*>(lds + pad64(T) * kE * 16)[t];
  }
  // Item = task: its 32 x (4 x 16 B of bf16) widened to fp32, and their sum.
  static __device__ void stage(const uint16_t* __restrict__ x, int64_t k, uint8_t* lds) {
    const int T = static_cast<int>(k / 32);
    float* xs = reinterpret_cast<float*>(lds + pad64(T) * kE * 16);
    const uint4* src = reinterpret_cast<const uint4*>(x);
    for (int b0 = threadIdx.x; b0 < T; b0 += kStageUnroll * blockDim.x) {
      uint4 v[kStageUnroll][4];
#pragma unroll
      for (int u = 0; u < kStageUnroll; ++u) {
        const int b = b0 + u * blockDim.x;
        if (b < T)
#pragma unroll
          for (int i = 0; i < 4; ++i) v[u][i] = src[4 * b + i];
      }
#pragma unroll
      for (int u = 0; u < kStageUnroll; ++u) {
        const int b = b0 + u * blockDim.x;
        if (b >= T) break;
        const uint32_t w[16] = {v[u][0].x, v[u][0].y, v[u][0].z, v[u][0].w, v[u][1].x, v[u][1].y, v[u][1].z, v[u][1].w,
                                v[u][2].x, v[u][2].y, v[u][2].z, v[u][2].w, v[u][3].x, v[u][3].y, v[u][3].z, v[u][3].w};
        float s = 0.0f;
        uint8_t* dst = lds + lds_task(b, kE);
#pragma unroll
        for (int e = 0; e < 8; ++e) {  // entry e: elements 4e .. 4e + 3 (e < 4: 0..15, else 16..31)
          const float4 f = make_float4(bf16_lo(w[2 * e]), bf16_hi(w[2 * e]), bf16_lo(w[2 * e + 1]), bf16_hi(w[2 * e + 1]));
          s += (f.x + f.y) + (f.z + f.w);
          *reinterpret_cast<float4*>(dst + 1024 * e) = f;
        }
        xs[b] = s;
      }
    }
  }
  static __device__ __forceinline__ float dot(const Payload& p, const X& x) {
    const uint32_t w[4] = {p.q.x, p.q.y, p.q.z, p.q.w};
    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 xl = x.x[i], xh = x.x[4 + i];
      mix4(iq4_lut(w[i] & 0x0F0F0F0Fu), xl.x, xl.y, xl.z, xl.w, s0, s1);
      mix4(iq4_lut((w[i] >> 4) & 0x0F0F0F0Fu), xh.x, xh.y, xh.z, xh.w, s0, s1);
    }
    const float sc = kXS ? iq4xs_scale(p.m, p.sub) : fp16_ieee(p.m.x);
    return sc * ((s0 + s1) - 1152.0f * x.sum);
  }
};
template <>
struct Fmt<SPIRAL_TYPE_IQ4_NL> : FmtIQ4<SPIRAL_TYPE_IQ4_NL> {};
template <>
struct Fmt<SPIRAL_TYPE_IQ4_XS> : FmtIQ4<SPIRAL_TYPE_IQ4_XS> {};

// ---- exact mode ----------------------------------------------------------------
// Same tasks, payload loads and (for Q4_0, Q6_K and the K-quants) the same x
// staging as the relaxed forms above; dot() multiplies bf16_rne(code * scale)
// weights. Q8_0 and IQ4 stage x as plain bf16 (no fp32 widening, no sums).

// x as bf16 in task order, ELEMS per task: entry e of task t holds its
// elements 8e .. 8e + 7, blocked as lds_task describes.
template <int ELEMS>
struct PlainX {
  static constexpr int kE = ELEMS / 8;
  static __host__ __device__ int64_t lds_bytes(int64_t k) { return pad64(k / ELEMS) * kE * 16; }
  struct X {
    uint4 xp[kE];
  };
  static __device__ __forceinline__ void xload(X& x, const uint8_t* lds, int /*T*/, int t) {
    const uint8_t* e = lds + lds_task(t, kE);
#pragma unroll
    for (int i = 0; i < kE; ++i) x.xp[i] = *reinterpret_cast<const uint4*>(e + 1024 * i);
  }
  // Item = one 16-byte entry (8 consecutive x): item e is entry e % kE of
  // task e / kE, which is x[8 e .. 8 e + 7]. Loads past the end reread the
  // last item (no branch around them) and are not stored.
  static __device__ void stage(const uint16_t* __restrict__ x, int64_t k, uint8_t* lds) {
    const uint32_t items = static_cast<uint32_t>(k / 8);
    const uint4* src = reinterpret_cast<const uint4*>(x);
    for (uint32_t e0 = threadIdx.x; e0 < items; e0 += kStageUnroll * blockDim.x) {
      uint4 v[kStageUnroll];
#pragma unroll
      for (int u = 0; u < kStageUnroll; ++u) v[u] = src[min(e0 + u * blockDim.x, items - 1)];
#pragma unroll
      for (int u = 0; u < kStageUnroll; ++u) {
        const uint32_t e = e0 + u * blockDim.x;
        if (e < items)
          *reinterpret_cast<uint4*>(lds + lds_task(static_cast<int>(e / kE), kE) + 1024u * (e % kE)) = v[u];
      }
    }
  }
};

template <int TYPE>
struct Exact;

// Interface of an exact format F (the kernel's exact branch):
//   S                 the per-task scale terms its dot product needs;
//   scale(p, special) S from the hardware fp16 conversion; sets special when
//                     a scale is one of the reference's special cases;
//   scale_rule(p)     S from the reference's bit-level scale rule (kRule
//                     formats, for a unit in which any lane set special);
//   dot(p, x, s, a0, a1) adds the task's weights times x into a0 / a1.
// A task whose terms are all zero contributes +0 (each weight is
// h * 0 + 0), which is how tasks past a row's end are masked.

// Hardware fp16 -> fp32 (v_cvt_f32_f16), which equals the reference's rule
// (fp16_scale) on exponents 1..30 and on +-0 (-0 gives weights of +0 in
// every form below); `special` records an exponent-0 non-zero (subnormal:
// the rule gives +0) or exponent-31 (the rule gives 2^16 (1.m)) pattern.
__device__ __forceinline__ float fp16_hw(_Float16 hf, bool& special) {
  // v_cmp_class mask: signaling and quiet NaN, -inf, -subnormal, +subnormal, +inf
  constexpr int kSpecial = 0x001 | 0x002 | 0x004 | 0x010 | 0x080 | 0x200;
  special |= __builtin_amdgcn_classh(hf, kSpecial);
  return static_cast<float>(hf);
}
__device__ __forceinline__ uint32_t fp16_bits(_Float16 hf) { return __builtin_bit_cast(uint16_t, hf); }
// The scale as loaded (a 16-bit buffer load), kept as a half so that the
// common path converts it directly and only the rule path takes its bits.
__device__ __forceinline__ _Float16 bload_h(__amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s) {
  return __builtin_bit_cast(_Float16, static_cast<uint16_t>(__builtin_amdgcn_raw_buffer_load_b16(r, v, s, 0)));
}

// Q4_0: low nibbles c as fp16 1024 + c, (1024 + c) d - 1032 d = (c - 8) d;
// high nibbles masked in place (byte 16 c) as fp16 64 + c, (64 + c) d - 72 d.
// Both offset terms are exact in fp32 (129 * 8 d, 9 * 8 d).
template <>
struct Exact<SPIRAL_TYPE_Q4_0> : Fmt<SPIRAL_TYPE_Q4_0> {
  static constexpr bool kRule = true;
  struct Planes {
    __amdgpu_buffer_rsrc_t qs, d;
    uint32_t nb;
  };
  // rows [r0, r1) of the planes qs[n][nb][16] | d[n][nb]
  static __device__ __forceinline__ Planes planes(const uint8_t* w, int64_t n_rows, int64_t k, int64_t r0,
                                                  int64_t r1) {
    const int64_t nb = k / 32;
    return Planes{rsrc(w + r0 * nb * 16, (r1 - r0) * nb * 16), rsrc(w + n_rows * nb * 16 + r0 * nb * 2, (r1 - r0) * nb * 2),
                  static_cast<uint32_t>(nb)};
  }
  struct Payload {
    uint4 q;
    _Float16 d;
  };
  static __device__ __forceinline__ void bload(Payload& p, const Planes& P, bool none, uint32_t rr, uint32_t tb,
                                               uint32_t lane, uint32_t lsk) {
    const uint32_t b = rr * P.nb + tb;
    p.q = bload16(rsrc_or_none(P.qs, none), (lane * 16u) | lsk, b * 16u);
    p.d = bload_h(rsrc_or_none(P.d, none), (lane * 2u) | lsk, b * 2u);
  }
  struct S {
    float d, cl, ch;
  };
  static __device__ __forceinline__ S terms(float d) { return S{d, -1032.0f * d, -72.0f * d}; }
  static __device__ __forceinline__ S scale(const Payload& p, bool& special) { return terms(fp16_hw(p.d, special)); }
  static __device__ __forceinline__ S scale_rule(const Payload& p) { return terms(fp16_scale(fp16_bits(p.d))); }
  static __device__ __forceinline__ void dot(const Payload& p, const X& x, const S& s, float& a0, float& a1) {
    const uint32_t w[4] = {p.q.x, p.q.y, p.q.z, p.q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = w[i] & 0x0F0F0F0Fu, hi = w[i] & 0xF0F0F0F0u;
      const uint4 el = x.xp[i >> 1], eh = x.xp[2 + (i >> 1)];
      a0 = dot2(wpair<kHi1024, kSel01>(lo, s.d, s.cl), (i & 1) ? el.z : el.x, a0);
      a1 = dot2(wpair<kHi1024, kSel23>(lo, s.d, s.cl), (i & 1) ? el.w : el.y, a1);
      a0 = dot2(wpair<kHi64, kSel01>(hi, s.d, s.ch), (i & 1) ? eh.z : eh.x, a0);
      a1 = dot2(wpair<kHi64, kSel23>(hi, s.d, s.ch), (i & 1) ? eh.w : eh.y, a1);
    }
  }
};

// Q8_0: q + 128 (q ^ 0x80) as fp16 1024 + q + 128, minus 1152 d (9 * 128 d).
template <>
struct Exact<SPIRAL_TYPE_Q8_0> : Fmt<SPIRAL_TYPE_Q8_0> {
  static constexpr bool kRule = true;
  struct Planes {
    __amdgpu_buffer_rsrc_t qs, d;
    uint32_t nb;
  };
  // rows [r0, r1) of the planes qs[n][nb][32] | d[n][nb]; task t = half block
  static __device__ __forceinline__ Planes planes(const uint8_t* w, int64_t n_rows, int64_t k, int64_t r0,
                                                  int64_t r1) {
    const int64_t nb = k / 32;
    return Planes{rsrc(w + r0 * nb * 32, (r1 - r0) * nb * 32), rsrc(w + n_rows * nb * 32 + r0 * nb * 2, (r1 - r0) * nb * 2),
                  static_cast<uint32_t>(nb)};
  }
  struct Payload {
    uint4 q;
    _Float16 d;
  };
  static __device__ __forceinline__ void bload(Payload& p, const Planes& P, bool none, uint32_t rr, uint32_t tb,
                                               uint32_t lane, uint32_t lsk) {
    p.q = bload16(rsrc_or_none(P.qs, none), (lane * 16u) | lsk, rr * P.nb * 32u + tb * 16u);
    p.d = bload_h(rsrc_or_none(P.d, none), ((lane >> 1) * 2u) | lsk, (rr * P.nb + (tb >> 1)) * 2u);
  }
  using XS = PlainX<16>;
  using X = XS::X;
  static __host__ __device__ int64_t lds_bytes(int64_t k) { return XS::lds_bytes(k); }
  static __device__ __forceinline__ void xload(X& x, const uint8_t* lds, int T, int t) { XS::xload(x, lds, T, t); }
  static __device__ void stage(const uint16_t* __restrict__ x, int64_t k, uint8_t* lds) { XS::stage(x, k, lds); }
  struct S {
    float d, c;
  };
  static __device__ __forceinline__ S scale(const Payload& p, bool& special) {
    const float d = fp16_hw(p.d, special);
    return S{d, -1152.0f * d};
  }
  static __device__ __forceinline__ S scale_rule(const Payload& p) {
    const float d = fp16_scale(fp16_bits(p.d));
    return S{d, -1152.0f * d};
  }
  static __device__ __forceinline__ void dot(const Payload& p, const X& x, const S& s, float& a0, float& a1) {
    const uint32_t w[4] = {p.q.x ^ 0x80808080u, p.q.y ^ 0x80808080u, p.q.z ^ 0x80808080u, p.q.w ^ 0x80808080u};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 e = x.xp[i >> 1];
      a0 = dot2(wpair<kHi1024, kSel01>(w[i], s.d, s.c), (i & 1) ? e.z : e.x, a0);
      a1 = dot2(wpair<kHi1024, kSel23>(w[i], s.d, s.c), (i & 1) ? e.w : e.y, a1);
    }
  }
};

// Q6_K: the 6-bit code q of each element as fp16 1024 + q; with the group's
// ds = d * sc, (1024 + q) ds - 1056 ds = (q - 32) ds. ds has at most 18
// significant bits (an 11-bit significand times |sc| <= 127, or 128 = 2^7),
// so 1056 ds = 33 * 32 ds has at most 24 and is exact.
//
// The exact form takes 32-element tasks (the relaxed form's are 64): task t
// of a row covers l0 .. l0 + 7 (l0 = 8 (t % 4)) of half (t / 4) % 2 of
// super-block t / 8, in all four of the half's 16-element groups. A
// 14336-wide row is then 448 tasks, seven full passes of a wave; 64-element
// tasks end such a row in a half-masked fourth pass, which costs as much VALU
// as a full one (4096 x 14336: 14.0 us against 15.5). Each lane loads 8 bytes
// of ql twice, of qh and of the sub-scales per task.
template <>
struct Exact<SPIRAL_TYPE_Q6_K> {
  static constexpr int kTaskElems = 32, kE = 4;
  static constexpr bool kRule = true;
  static __host__ __device__ int64_t lds_bytes(int64_t k) { return pad64(k / 32) * kE * 16; }
  struct X {
    uint4 x[4];  // group j's 8 x values
  };
  static __device__ __forceinline__ void xload(X& x, const uint8_t* lds, int, int t) {
    const uint8_t* e = lds + lds_task(t, kE);
#pragma unroll
    for (int i = 0; i < 4; ++i) x.x[i] = *reinterpret_cast<const uint4*>(e + 1024 * i);
  }
  // Item = (task, group): x[256 (t / 8) + 128 ((t / 4) % 2) + 32 j + 8 (t % 4)], 8 values.
  static __device__ void stage(const uint16_t* __restrict__ x, int64_t k, uint8_t* lds) {
    const int T = static_cast<int>(k / 32);
    const int items = 4 * T;
    for (int e0 = threadIdx.x; e0 < items; e0 += kStageUnroll * blockDim.x) {
      uint4 v[kStageUnroll];
#pragma unroll
      for (int u = 0; u < kStageUnroll; ++u) {
        const int e = min(e0 + u * static_cast<int>(blockDim.x), items - 1);
        const int t = e >> 2, j = e & 3;
        v[u] = *reinterpret_cast<const uint4*>(x + (t >> 3) * 256 + ((t >> 2) & 1) * 128 + 32 * j + 8 * (t & 3));
      }
#pragma unroll
      for (int u = 0; u < kStageUnroll; ++u) {
        const int e = e0 + u * static_cast<int>(blockDim.x);
        if (e < items) *reinterpret_cast<uint4*>(lds + lds_task(e >> 2, kE) + 1024 * (e & 3)) = v[u];
      }
    }
  }
  struct Planes {
    __amdgpu_buffer_rsrc_t ql, qh, sc, d;
    uint32_t nb;
  };
  // rows [r0, r1) of the planes ql[n][nb][128] | qh[..][64] | sc[..][16] | d[n][nb]
  static __device__ __forceinline__ Planes planes(const uint8_t* w, int64_t n_rows, int64_t k, int64_t r0,
                                                  int64_t r1) {
    const int64_t nb = k / 256, tot = n_rows * nb, n = r1 - r0;
    return Planes{rsrc(w + r0 * nb * 128, n * nb * 128), rsrc(w + tot * 128 + r0 * nb * 64, n * nb * 64),
                  rsrc(w + tot * 192 + r0 * nb * 16, n * nb * 16), rsrc(w + tot * 208 + r0 * nb * 2, n * nb * 2),
                  static_cast<uint32_t>(nb)};
  }
  struct Payload {
    uint2 a, b, h;
    uint2 sc8;     // the 8 sub-scales of the task's half super-block
    uint32_t odd;  // l0 >= 16: its groups' sub-scales are the odd bytes
    _Float16 d;
  };
  static __device__ __forceinline__ uint2 bload8nt(__amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t s) {
    const auto x = __builtin_amdgcn_raw_buffer_load_b64(r, v, s, kStreamAux);
    return make_uint2(x[0], x[1]);
  }
  // Lane = task tb + lane: super-block tb / 8 + lane / 8, half (lane / 4) % 2,
  // l0 = 8 (lane % 4). Loaded values are only stored here: arithmetic on them
  // would make the compiler wait for the load at once.
  static __device__ __forceinline__ void bload(Payload& p, const Planes& P, bool none, uint32_t rr, uint32_t tb,
                                               uint32_t lane, uint32_t lsk) {
    const uint32_t sb = rr * P.nb + (tb >> 3), ls = lane >> 3, hh = (lane >> 2) & 1u, q4 = lane & 3u;
    const uint32_t lo = ls * 128u + 64u * hh + 8u * q4;
    const __amdgpu_buffer_rsrc_t ql = rsrc_or_none(P.ql, none);
    p.a = bload8nt(ql, lo | lsk, sb * 128u);
    p.b = bload8nt(ql, (lo + 32u) | lsk, sb * 128u);
    p.h = bload8nt(rsrc_or_none(P.qh, none), (ls * 64u + 32u * hh + 8u * q4) | lsk, sb * 64u);
    p.sc8 = bload8(rsrc_or_none(P.sc, none), (ls * 16u + 8u * hh) | lsk, sb * 16u);
    p.odd = q4 >> 1;
    p.d = bload_h(rsrc_or_none(P.d, none), (ls * 2u) | lsk, sb * 2u);
  }
  // Sub-scale of group j is sc[8 h + l0 / 16 + 2 j]: bytes s, s + 2, s + 4,
  // s + 6 of the half's 8 sub-scales (s = odd).
  static __device__ __forceinline__ uint32_t sub_scales(const Payload& p) {
    return __builtin_amdgcn_perm(p.sc8.y, p.sc8.x, p.odd ? 0x07050301u : 0x06040200u);
  }
  struct S {
    float ds[4], c[4];
  };
  static __device__ __forceinline__ S terms(float d, uint32_t sc4) {
    S s;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s.ds[j] = d * static_cast<float>(static_cast<int8_t>((sc4 >> (8 * j)) & 0xffu));
      s.c[j] = -1056.0f * s.ds[j];
    }
    return s;
  }
  static __device__ __forceinline__ S scale(const Payload& p, bool& special) {
    return terms(fp16_hw(p.d, special), sub_scales(p));
  }
  static __device__ __forceinline__ S scale_rule(const Payload& p) {
    return terms(fp16_scale(fp16_bits(p.d)), sub_scales(p));
  }
  static __device__ __forceinline__ void dot(const Payload& p, const X& x, const S& s, float& a0, float& a1) {
    const uint32_t A[2] = {p.a.x, p.a.y}, B[2] = {p.b.x, p.b.y}, H[2] = {p.h.x, p.h.y};
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      // 6-bit codes of elements l0 + 4q .. l0 + 4q + 3 of each group, one per byte.
      const uint32_t c[4] = {
          (A[q] & 0x0F0F0F0Fu) | ((H[q] << 4) & 0x30303030u),
          (B[q] & 0x0F0F0F0Fu) | ((H[q] << 2) & 0x30303030u),
          ((A[q] >> 4) & 0x0F0F0F0Fu) | (H[q] & 0x30303030u),
          ((B[q] >> 4) & 0x0F0F0F0Fu) | ((H[q] >> 2) & 0x30303030u),
      };
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 xv = x.x[j];
        a0 = dot2(wpair<kHi1024, kSel01>(c[j], s.ds[j], s.c[j]), q ? xv.z : xv.x, a0);
        a1 = dot2(wpair<kHi1024, kSel23>(c[j], s.ds[j], s.c[j]), q ? xv.w : xv.y, a1);
      }
    }
  }
};

// Q4_K / Q5_K: weight bf16_rne(fma(d * scale, q, -dmin * min)). The code is
// the subnormal fp16 q * 2^-24, so v_fma_mix_f32 against d * scale * 2^24
// (exact) and -dmin * min rounds q * d * scale - dmin * min once, as fmaf
// does; fp16 denormals are kept (the kernels run with fp16 denormals on).
// d and dmin are IEEE binary16 (no special cases).
template <int TYPE>
struct ExactKQ : FmtKQ<TYPE> {
  using B = FmtKQ<TYPE>;
  using Payload = typename B::Payload;
  using X = typename B::X;
  static constexpr bool kRule = false;
  // The relaxed form's staging without the sums: -dmin * min is inside each
  // weight here.
  static __device__ void stage(const uint16_t* __restrict__ x, int64_t k, uint8_t* lds) {
    B::template stage<false>(x, k, lds);
  }
  static __device__ __forceinline__ void xload(X& x, const uint8_t* lds, int, int t) {
    const uint8_t* e = lds + lds_task(t, B::kE);
#pragma unroll
    for (int i = 0; i < 4; ++i) x.xp[i] = *reinterpret_cast<const uint4*>(e + 1024 * i);
  }
  struct Planes {
    __amdgpu_buffer_rsrc_t qs, qh, meta;
    uint32_t nb;
  };
  // rows [r0, r1) of the planes qs[n][nb][128] | (Q5_K) qh[..][32] | meta[..][16]
  static __device__ __forceinline__ Planes planes(const uint8_t* w, int64_t n_rows, int64_t k, int64_t r0,
                                                  int64_t r1) {
    const int64_t nb = k / 256, tot = n_rows * nb, n = r1 - r0;
    const __amdgpu_buffer_rsrc_t qs = rsrc(w + r0 * nb * 128, n * nb * 128);
    return Planes{qs, B::kQ5 ? rsrc(w + tot * 128 + r0 * nb * 32, n * nb * 32) : qs,
                  rsrc(w + tot * (B::kQ5 ? 160 : 128) + r0 * nb * 16, n * nb * 16), static_cast<uint32_t>(nb)};
  }
  static __device__ __forceinline__ void bload(Payload& p, const Planes& P, bool none, uint32_t rr, uint32_t tb,
                                               uint32_t lane, uint32_t lsk) {
    const uint32_t sb = rr * P.nb + (tb >> 3);
    p.q = bload16(rsrc_or_none(P.qs, none), (lane * 16u) | lsk, (rr * P.nb * 8u + tb) * 16u);
    p.meta = bload16(rsrc_or_none(P.meta, none), ((lane >> 3) * 16u) | lsk, sb * 16u);
    if constexpr (B::kQ5)
      p.qh = bload16(rsrc_or_none(P.qh, none), ((lane >> 3) * 32u + (lane & 1u) * 16u) | lsk, sb * 32u);
    p.c2 = lane & 6u;
  }
  struct S {
    float dl, ml, dh, mh;
  };
  static __device__ __forceinline__ S scale(const Payload& p, bool&) {
    const uint32_t sm = kq_chunk_scales(p.meta.y, p.meta.z, p.meta.w, p.c2 >> 1);
    const float d24 = fp16_ieee(p.meta.x & 0xffffu) * kTwo24, dmin = fp16_ieee(p.meta.x >> 16);
    return S{d24 * static_cast<float>(sm & 0xffu), -(dmin * static_cast<float>((sm >> 8) & 0xffu)),
             d24 * static_cast<float>((sm >> 16) & 0xffu), -(dmin * static_cast<float>(sm >> 24))};
  }
  static __device__ __forceinline__ S scale_rule(const Payload& p) {
    bool unused = false;
    return scale(p, unused);
  }
  static __device__ __forceinline__ void dot(const Payload& p, const X& x, const S& s, float& a0, float& a1) {
    const uint32_t w[4] = {p.q.x, p.q.y, p.q.z, p.q.w};
    const uint32_t h[4] = {p.qh.x, p.qh.y, p.qh.z, p.qh.w};
    // Q5_K: bit c2 (c2 + 1) of every qh byte lands on bit 4 under a rotation
    // right by c2 - 4 (c2 - 3), so one v_and_or_b32 merges it.
    const uint32_t rl = (p.c2 + 28u) & 31u, rh = (p.c2 + 29u) & 31u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t lo = w[i] & 0x0F0F0F0Fu, hi = (w[i] >> 4) & 0x0F0F0F0Fu;
      if constexpr (B::kQ5) {
        lo = and_or_b32(__builtin_amdgcn_alignbit(h[i], h[i], rl), 0x10101010u, lo);
        hi = and_or_b32(__builtin_amdgcn_alignbit(h[i], h[i], rh), 0x10101010u, hi);
      }
      const uint4 el = x.xp[i >> 1], eh = x.xp[2 + (i >> 1)];
      a0 = dot2(wpair<kHiSub, kSel01>(lo, s.dl, s.ml), (i & 1) ? el.z : el.x, a0);
      a1 = dot2(wpair<kHiSub, kSel23>(lo, s.dl, s.ml), (i & 1) ? el.w : el.y, a1);
      a0 = dot2(wpair<kHiSub, kSel01>(hi, s.dh, s.mh), (i & 1) ? eh.z : eh.x, a0);
      a1 = dot2(wpair<kHiSub, kSel23>(hi, s.dh, s.mh), (i & 1) ? eh.w : eh.y, a1);
    }
  }
};
template <>
struct Exact<SPIRAL_TYPE_Q4_K> : ExactKQ<SPIRAL_TYPE_Q4_K> {};
template <>
struct Exact<SPIRAL_TYPE_Q5_K> : ExactKQ<SPIRAL_TYPE_Q5_K> {};

// IQ4_NL / IQ4_XS: codebook bytes kv + 128 as fp16 1024 + kv + 128 against
// the (sub-)block scale s, minus 1152 s (s at most 17 significant bits).
// d is IEEE binary16 (no special cases).
template <int TYPE>
struct ExactIQ4 : FmtIQ4<TYPE> {
  using B = FmtIQ4<TYPE>;
  using Payload = typename B::Payload;
  static constexpr bool kRule = false;
  struct Planes {
    __amdgpu_buffer_rsrc_t qs, d;
    uint32_t nb;
  };
  // rows [r0, r1): IQ4_NL qs[n][nb][16] | d[n][nb]; IQ4_XS qs[n][nb][128] | meta[n][nb][8]
  static __device__ __forceinline__ Planes planes(const uint8_t* w, int64_t n_rows, int64_t k, int64_t r0,
                                                  int64_t r1) {
    const int64_t n = r1 - r0;
    if constexpr (B::kXS) {
      const int64_t nb = k / 256;
      return Planes{rsrc(w + r0 * nb * 128, n * nb * 128), rsrc(w + n_rows * nb * 128 + r0 * nb * 8, n * nb * 8),
                    static_cast<uint32_t>(nb)};
    } else {
      const int64_t nb = k / 32;
      return Planes{rsrc(w + r0 * nb * 16, n * nb * 16), rsrc(w + n_rows * nb * 16 + r0 * nb * 2, n * nb * 2),
                    static_cast<uint32_t>(nb)};
    }
  }
  static __device__ __forceinline__ void bload(Payload& p, const Planes& P, bool none, uint32_t rr, uint32_t tb,
                                               uint32_t lane, uint32_t lsk) {
    if constexpr (B::kXS) {
      p.q = bload16(rsrc_or_none(P.qs, none), (lane * 16u) | lsk, (rr * P.nb * 8u + tb) * 16u);
      p.m = bload8(rsrc_or_none(P.d, none), ((lane >> 3) * 8u) | lsk, (rr * P.nb + (tb >> 3)) * 8u);
      p.sub = static_cast<int>(lane & 7u);
    } else {
      const uint32_t b = rr * P.nb + tb;
      p.q = bload16(rsrc_or_none(P.qs, none), (lane * 16u) | lsk, b * 16u);
      p.m = make_uint2(bload2(rsrc_or_none(P.d, none), (lane * 2u) | lsk, b * 2u), 0u);
      p.sub = 0;
    }
  }
  using XS = PlainX<32>;
  static constexpr int kE = XS::kE;
  using X = typename XS::X;
  static __host__ __device__ int64_t lds_bytes(int64_t k) { return XS::lds_bytes(k); }
  static __device__ __forceinline__ void xload(X& x, const uint8_t* lds, int T, int t) { XS::xload(x, lds, T, t); }
  static __device__ void stage(const uint16_t* __restrict__ x, int64_t k, uint8_t* lds) { XS::stage(x, k, lds); }
  struct S {
    float s, c;
  };
  static __device__ __forceinline__ S scale(const Payload& p, bool&) {
    const float sc = B::kXS ? iq4xs_scale(p.m, p.sub) : fp16_ieee(p.m.x);
    return S{sc, -1152.0f * sc};
  }
  static __device__ __forceinline__ S scale_rule(const Payload& p) {
    bool unused = false;
    return scale(p, unused);
  }
  static __device__ __forceinline__ void dot(const Payload& p, const X& x, const S& s, float& a0, float& a1) {
    const uint32_t w[4] = {p.q.x, p.q.y, p.q.z, p.q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = iq4_lut(w[i] & 0x0F0F0F0Fu), hi = iq4_lut((w[i] >> 4) & 0x0F0F0F0Fu);
      const uint4 el = x.xp[i >> 1], eh = x.xp[2 + (i >> 1)];
      a0 = dot2(wpair<kHi1024, kSel01>(lo, s.s, s.c), (i & 1) ? el.z : el.x, a0);
      a1 = dot2(wpair<kHi1024, kSel23>(lo, s.s, s.c), (i & 1) ? el.w : el.y, a1);
      a0 = dot2(wpair<kHi1024, kSel01>(hi, s.s, s.c), (i & 1) ? eh.z : eh.x, a0);
      a1 = dot2(wpair<kHi1024, kSel23>(hi, s.s, s.c), (i & 1) ? eh.w : eh.y, a1);
    }
  }
};
template <>
struct Exact<SPIRAL_TYPE_IQ4_NL> : ExactIQ4<SPIRAL_TYPE_IQ4_NL> {};
template <>
struct Exact<SPIRAL_TYPE_IQ4_XS> : ExactIQ4<SPIRAL_TYPE_IQ4_XS> {};

// ---- the kernel --------------------------------------------------------------

template <class F, int J>
struct Unit {
  typename F::Payload p[J];
};

// Requests the payload of pass `pass` of row `r`; tasks past the row's end
// load task 0 (a valid address) and are masked out in compute_unit.
template <class F, int J, bool MASK>
__device__ __forceinline__ void load_unit(Unit<F, J>& U, const uint8_t* w, int64_t n_rows, int64_t k,
                                          int64_t r, int pass, int T, int lane) {
  const typename F::Row R = F::row(w, n_rows, k, r);
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int t = pass * 64 * J + 64 * j + lane;
    F::load(U.p[j], R, (!MASK || t < T) ? t : 0);
  }
}

template <bool F32_OUT>
__device__ __forceinline__ void store_y(void* y, int64_t r, float v) {
  if constexpr (F32_OUT)
    static_cast<float*>(y)[r] = v;
  else
    static_cast<__bf16*>(y)[r] = static_cast<__bf16>(v);
}

// The relaxed kernel. F: the format's relaxed arithmetic (Fmt<TYPE>).
// XREG: the row fits one pass (T <= 64 J) and each lane keeps the x of its J
// tasks in registers. MASK: some tasks of a pass fall past the row's end.
// DEPTH: units whose payload is in flight at once (a ring of DEPTH buffers).
// MINW: waves per SIMD the registers must allow (1: no cap).
template <class F, int J, int WAVES, int DEPTH, bool XREG, bool MASK, bool F32_OUT, int MINW = 1>
__global__ void __launch_bounds__(64 * WAVES, MINW) gemv_kernel(const uint8_t* __restrict__ w, int64_t n_rows,
                                                          int64_t k, const uint16_t* __restrict__ x,
                                                          void* __restrict__ y) {
  extern __shared__ __align__(16) uint8_t lds[];
  const int lane = threadIdx.x & 63;
  const int64_t wave =
      static_cast<int64_t>(blockIdx.x) * WAVES + __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int64_t n_waves = static_cast<int64_t>(gridDim.x) * WAVES;
  const int64_t r0 = wave * n_rows / n_waves, r1 = (wave + 1) * n_rows / n_waves;
  const int T = static_cast<int>(k / F::kTaskElems);
  const int passes = XREG ? 1 : (T + 64 * J - 1) / (64 * J);
  const int64_t units = (r1 - r0) * passes;

  // Unit coordinates advance one pass at a time: (rl, pl) for loads, (rc, pc)
  // for compute.
  Unit<F, J> buf[DEPTH];
  int64_t rl = r0;
  int pl = 0;
  auto advance = [&](int64_t& r, int& pass) {
    if (++pass == passes) { pass = 0; ++r; }
  };
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) {
    if (d < units) {
      load_unit<F, J, MASK>(buf[d], w, n_rows, k, rl, pl, T, lane);
      advance(rl, pl);
    }
  }
  F::stage(x, k, lds);
  __syncthreads();

  typename F::X xr[XREG ? J : 1];
  if constexpr (XREG) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int t = 64 * j + lane;
      F::xload(xr[j], lds, T, (!MASK || t < T) ? t : 0);
    }
  }

  int64_t rc = r0;
  int pc = 0;
  float acc = 0.0f;
  for (int64_t u0 = 0; u0 < units; u0 += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      const int64_t u = u0 + d;
      if (u >= units) break;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int t = pc * 64 * J + 64 * j + lane;
        const bool ok = !MASK || t < T;
        float part;
        if constexpr (XREG) {
          part = F::dot(buf[d].p[j], xr[j]);
        } else {
          typename F::X xt;
          F::xload(xt, lds, T, ok ? t : 0);
          part = F::dot(buf[d].p[j], xt);
        }
        acc += ok ? part : 0.0f;
      }
      if (pc == passes - 1) {
        const float v = wave_sum_last(acc);
        if (lane == 63) store_y<F32_OUT>(y, rc, v);
        acc = 0.0f;
      }
      advance(rc, pc);
      if (u + DEPTH < units) {
        load_unit<F, J, MASK>(buf[d], w, n_rows, k, rl, pl, T, lane);
        advance(rl, pl);
      }
    }
  }
}

// ---- the exact kernel -----------------------------------------------------------
// The same work split and unit ring as gemv_kernel, with a branch-free memory
// skeleton: payload loads, ring refills and y stores are buffer accesses
// that every lane issues on every step. A task past the row's end (bit 31 of
// the lane's offset), a unit past the wave's last (a buffer of no records)
// and a lane with nothing to store (bit 31) access nothing; skipped loads
// return zeros, so a masked task's weights are zero. With no memory access
// under a branch, the compiler waits for exactly the oldest ring slot
// instead of draining every load in flight each step. Offsets split into a
// per-lane part, fixed for the wave, and the row and pass, in a scalar
// register, so a refill costs no vector instructions.

// A unit is one pass over RG = 64 / G rows: lane group g = lane / G takes
// row rr + g, tasks tb + lane % G. A format addresses task tb + lane of row
// rr over planes that hold rows of T tasks back to back, so the group's row
// enters as the lane index g T + lane % G (tb and T are multiples of 8, which
// keeps a super-block's eight tasks within one lane index range). Lanes of a
// row past the wave's last (row_end rows from rr) or of a task past the row's
// end are skipped.
template <class F, int J, int G, bool MASK>
__device__ __forceinline__ void bload_unit(Unit<F, J>& U, const typename F::Planes& P, bool none, int rr, int pass,
                                           int T, int lane, int row_end) {
  const int gl = lane % G;
  const uint32_t vl = static_cast<uint32_t>((lane / G) * T + gl);
  const bool row_out = G < 64 && lane / G >= row_end;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int tb = pass * G * J + G * j;
    const uint32_t lsk = ((MASK && tb + gl >= T) || row_out) ? kSkip : 0u;
    F::bload(U.p[j], P, none, static_cast<uint32_t>(rr), static_cast<uint32_t>(tb), vl, lsk);
  }
}

template <class F, int J, int G, int WAVES, int DEPTH, bool XREG, bool MASK, bool F32_OUT, int MINW>
__global__ void __launch_bounds__(64 * WAVES, MINW) gemv_exact_kernel(const uint8_t* __restrict__ w, int64_t n_rows,
                                                                      int64_t k, const uint16_t* __restrict__ x,
                                                                      void* __restrict__ y) {
  extern __shared__ __align__(16) uint8_t lds[];
  constexpr int kEsize = F32_OUT ? 4 : 2;
  constexpr int RG = 64 / G;  // rows per unit
  const int lane = threadIdx.x & 63;
  const int gl = lane % G, grp = lane / G;
  const int64_t wave =
      static_cast<int64_t>(blockIdx.x) * WAVES + __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int64_t n_waves = static_cast<int64_t>(gridDim.x) * WAVES;
  // Waves take whole groups of RG rows; only the matrix's last group can be short.
  const int64_t n_groups = (n_rows + RG - 1) / RG;
  const int64_t g0 = wave * n_groups / n_waves * RG, g1 = (wave + 1) * n_groups / n_waves * RG;
  const int64_t r0 = g0 < n_rows ? g0 : n_rows, r1 = g1 < n_rows ? g1 : n_rows;
  const int rows = static_cast<int>(r1 - r0);
  const int T = static_cast<int>(k / F::kTaskElems);
  const int passes = XREG ? 1 : (T + G * J - 1) / (G * J);
  const int units = (rows + RG - 1) / RG * passes;
  const typename F::Planes P = F::planes(w, n_rows, k, r0, r1);
  const __amdgpu_buffer_rsrc_t Y = rsrc(static_cast<uint8_t*>(y) + r0 * kEsize, (r1 - r0) * kEsize);

  // Unit coordinates (first row relative to r0, pass) advance one pass at a
  // time: (rl, pl) for loads, (rc, pc) for compute.
  Unit<F, J> buf[DEPTH];
  int rl = 0, pl = 0;
  auto advance = [&](int& r, int& pass) {
    if (++pass == passes) { pass = 0; r += RG; }
  };
  // Issued slot by slot in the loop's order, so that the loop header sees
  // the same sequence of loads in flight from the prologue as from the loop.
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) {
    bload_unit<F, J, G, MASK>(buf[d], P, d >= units, rl, pl, T, lane, rows - rl);
    advance(rl, pl);
    __builtin_amdgcn_sched_barrier(0);
  }
  F::stage(x, k, lds);
  __syncthreads();

  typename F::X xr[XREG ? J : 1];
  if constexpr (XREG) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int t = G * j + gl;
      F::xload(xr[j], lds, T, t < T ? t : 0);
    }
  }

  int rc = 0, pc = 0;
  float a0 = 0.0f, a1 = 0.0f;
  auto compute = [&](const Unit<F, J>& U) {
    // The unit's scale terms first: the hardware conversion, and the
    // reference's rule for every lane when any lane of the wave holds a
    // special scale (a wave-uniform branch around arithmetic only).
    typename F::S sc[J];
    bool special = false;
#pragma unroll
    for (int j = 0; j < J; ++j) sc[j] = F::scale(U.p[j], special);
    if constexpr (F::kRule) {
      if (__builtin_amdgcn_ballot_w64(special) != 0) {
#pragma unroll
        for (int j = 0; j < J; ++j) sc[j] = F::scale_rule(U.p[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < J; ++j) {
      if constexpr (XREG) {
        F::dot(U.p[j], xr[j], sc[j], a0, a1);
      } else {
        // Whole-wave units with no masked task read x at a wave-uniform
        // 64-task block plus the lane's slot.
        const int t = (G == 64 && !MASK) ? (((pc * J + j) << 6) | lane) : pc * G * J + G * j + gl;
        typename F::X xt;
        F::xload(xt, lds, T, (!MASK || t < T) ? t : 0);
        F::dot(U.p[j], xt, sc[j], a0, a1);
      }
    }
    const bool end = XREG || pc == passes - 1;
    float v = 0.0f;
    if (end) {
      v = group_sum_last<G>(a0 + a1);
      a0 = a1 = 0.0f;
    }
    const bool store = end && gl == G - 1 && (G == 64 || grp < rows - rc);
    const uint32_t off = static_cast<uint32_t>((rc + grp) * kEsize) | (store ? 0u : kSkip);
    if constexpr (F32_OUT)
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), Y, off, 0, 0);
    else
      __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, static_cast<__bf16>(v)), Y, off, 0, 0);
    advance(rc, pc);
  };

  // Scheduling barriers keep each slot's compute apart from the refills and
  // the next slot: an instruction of the next slot hoisted into this one
  // would make the compiler wait for that slot's loads early.
  int u = 0;
  for (; u + DEPTH <= units; u += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      compute(buf[d]);
      __builtin_amdgcn_sched_barrier(0);
      bload_unit<F, J, G, MASK>(buf[d], P, u + d + DEPTH >= units, rl, pl, T, lane, rows - rl);
      advance(rl, pl);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int d = 0; d < DEPTH - 1; ++d)
    if (u + d < units) compute(buf[d]);
}

template <class F, int J, int G, int WAVES, int DEPTH, bool XREG, bool MASK, int MINW>
int launch_exact_cfg(const void* w, int64_t n_rows, int64_t k, const uint16_t* x, void* y, int y_type, hipStream_t s) {
  constexpr int RG = 64 / G;
  const int64_t lds = F::lds_bytes(k);
  const void* kern =
      y_type == SPIRAL_TYPE_F32
          ? reinterpret_cast<const void*>(gemv_exact_kernel<F, J, G, WAVES, DEPTH, XREG, MASK, true, MINW>)
          : reinterpret_cast<const void*>(gemv_exact_kernel<F, J, G, WAVES, DEPTH, XREG, MASK, false, MINW>);
  const int64_t resident = static_cast<int64_t>(device_cu_count()) * blocks_per_cu(kern, 64 * WAVES, lds);
  const int64_t n_groups = ceil_div(n_rows, RG);
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(ceil_div(n_groups, WAVES), resident));
  // A wave's rows of a plane (at most one byte per element) must stay below
  // 2 GiB: bit 31 of an offset marks a skipped access.
  if (ceil_div(n_groups, blocks * WAVES) * RG * k >= (int64_t(1) << 31)) return SPIRAL_ERR_SHAPE;
  const uint8_t* W = static_cast<const uint8_t*>(w);
  if (y_type == SPIRAL_TYPE_F32)
    hipLaunchKernelGGL((gemv_exact_kernel<F, J, G, WAVES, DEPTH, XREG, MASK, true, MINW>),
                       dim3(static_cast<unsigned>(blocks)), dim3(64 * WAVES), lds, s, W, n_rows, k, x, y);
  else
    hipLaunchKernelGGL((gemv_exact_kernel<F, J, G, WAVES, DEPTH, XREG, MASK, false, MINW>),
                       dim3(static_cast<unsigned>(blocks)), dim3(64 * WAVES), lds, s, W, n_rows, k, x, y);
  return launch_status();
}

// Units of G lanes a row and J tasks a lane. Narrow groups (G < 64) always
// read x from LDS: rows that one narrow pass covers (16 or 32 tasks) are
// too short for registers to matter, and it halves their instantiations.
template <class F, int J, int G, int WAVES, int DEPTH, int MINW = 1>
int launch_exact_j(const void* w, int64_t n_rows, int64_t k, const uint16_t* x, void* y, int y_type, hipStream_t s) {
  const int64_t T = k / F::kTaskElems;
  const bool mask = T % (G * J) != 0;
  if constexpr (G == 64) {
    if (T <= 64 * J)
      return mask ? launch_exact_cfg<F, J, G, WAVES, DEPTH, true, true, MINW>(w, n_rows, k, x, y, y_type, s)
                  : launch_exact_cfg<F, J, G, WAVES, DEPTH, true, false, MINW>(w, n_rows, k, x, y, y_type, s);
  }
  return mask ? launch_exact_cfg<F, J, G, WAVES, DEPTH, false, true, MINW>(w, n_rows, k, x, y, y_type, s)
              : launch_exact_cfg<F, J, G, WAVES, DEPTH, false, false, MINW>(w, n_rows, k, x, y, y_type, s);
}

template <class F, int J, int WAVES, int DEPTH, bool XREG, bool MASK, int MINW = 1>
int launch_cfg(const void* w, int64_t n_rows, int64_t k, const uint16_t* x, void* y, int y_type, hipStream_t s) {
  const int64_t lds = F::lds_bytes(k);
  const void* kern = y_type == SPIRAL_TYPE_F32
                         ? reinterpret_cast<const void*>(gemv_kernel<F, J, WAVES, DEPTH, XREG, MASK, true, MINW>)
                         : reinterpret_cast<const void*>(gemv_kernel<F, J, WAVES, DEPTH, XREG, MASK, false, MINW>);
  const int64_t resident = static_cast<int64_t>(device_cu_count()) * blocks_per_cu(kern, 64 * WAVES, lds);
  const unsigned blocks = static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(ceil_div(n_rows, WAVES), resident)));
  const uint8_t* W = static_cast<const uint8_t*>(w);
  if (y_type == SPIRAL_TYPE_F32)
    hipLaunchKernelGGL((gemv_kernel<F, J, WAVES, DEPTH, XREG, MASK, true, MINW>), dim3(blocks), dim3(64 * WAVES), lds,
                       s, W, n_rows, k, x, y);
  else
    hipLaunchKernelGGL((gemv_kernel<F, J, WAVES, DEPTH, XREG, MASK, false, MINW>), dim3(blocks), dim3(64 * WAVES), lds,
                       s, W, n_rows, k, x, y);
  return launch_status();
}

template <class F, int J, int WAVES, int DEPTH, int MINW = 1>
int launch_j(const void* w, int64_t n_rows, int64_t k, const uint16_t* x, void* y, int y_type, hipStream_t s) {
  const int64_t T = k / F::kTaskElems;
  const bool xreg = T <= 64 * J, mask = T % (64 * J) != 0;
  if (xreg)
    return mask ? launch_cfg<F, J, WAVES, DEPTH, true, true, MINW>(w, n_rows, k, x, y, y_type, s)
                : launch_cfg<F, J, WAVES, DEPTH, true, false, MINW>(w, n_rows, k, x, y, y_type, s);
  return mask ? launch_cfg<F, J, WAVES, DEPTH, false, true, MINW>(w, n_rows, k, x, y, y_type, s)
              : launch_cfg<F, J, WAVES, DEPTH, false, false, MINW>(w, n_rows, k, x, y, y_type, s);
}

// Relaxed mode. J = tasks per lane per unit, chosen so that rows of up to
// 64 J tasks keep x in registers; two units in flight per wave (measured best
// on MI355X for the 4096x14336 Q6_K, 14336x4096 Q8_0 and 4096x4096 Q4_0
// shapes). Q6_K keeps x in LDS (64 bf16 per task) with J = 1, in 16-wave
// workgroups (x staged once per 16 rows; 5 % faster than 8 waves on the
// 4096x14336 shape, while deeper rings, two tasks per lane and fewer
// resident workgroups were slower). Kernels whose registers allow three
// waves a SIMD but not four (Q8_0 at J = 4, 138 VGPRs; Q5_K at J = 2, 133)
// run 12-wave workgroups, one a CU, instead of leaving a third of the slots
// empty: 14336x4096 Q8_0 11.73 us against 11.83 for 8 waves and Q5_K 10.86
// against 11.65 (medians), while 4- and 6-wave workgroups and a third ring
// slot were slower for Q8_0. Those that fit four (Q4_0, Q4_K, IQ4) keep two
// 8-wave workgroups a CU: 12- and 10-wave ones were 2-20 % slower, so rows
// longer than 128 tasks (J = 4) take 12 waves only for Q8_0.
template <int TYPE>
int launch_relaxed(const void* w, int64_t n_rows, int64_t k, const uint16_t* x, void* y, int y_type, hipStream_t s) {
  using F = Fmt<TYPE>;
  const int64_t T = k / F::kTaskElems;
  if constexpr (TYPE == SPIRAL_TYPE_Q6_K) {
    return launch_j<F, 1, 16, 2>(w, n_rows, k, x, y, y_type, s);
  } else {
    if (T <= 64) return launch_j<F, 1, 8, 2>(w, n_rows, k, x, y, y_type, s);
    if (T <= 128) return launch_j<F, 2, TYPE == SPIRAL_TYPE_Q5_K ? 12 : 8, 2>(w, n_rows, k, x, y, y_type, s);
    return launch_j<F, 4, TYPE == SPIRAL_TYPE_Q8_0 ? 12 : 8, 2>(w, n_rows, k, x, y, y_type, s);
  }
}

// Exact mode: the unit shape of least estimated work, the wider on a tie.
// Whole-wave units (G = 64) give a row U = 64 J task slots a pass; rows of up
// to 256 tasks can instead take 16 or 32 lanes a row, four or two
// neighbouring rows a unit. The estimate counts each row's passes times J
// tasks a lane: a partly masked last pass costs the VALU of a full one. A
// task costs 32 (x read from LDS), 28 with x in registers (one pass) and 35
// in narrow groups, factors fitted to these MI355X timings (us):
//                          64 lanes, LDS    64 lanes, regs   narrow groups
//   262144 x 1536 Q6_K                        79.3 (J 1)      72.9 (16 x 3)
//   13824 x 5120 Q4_K       17.4 (3 passes)   19.2 (J 4)      15.9 (32 x 5)
//   27648 x 5120 Q6_K       33.6 (3 passes)                   29.8 (32 x 5)
//   14336 x 5120 IQ4_XS     19.2 (3 passes)   21.8 (J 4)      17.1 (32 x 5)
//   18944 x 3584 Q4_0                         12.4 (J 2)      13.8 (16 x 7)
// Longer rows keep whole-wave units: a unit of narrow groups reads distant
// rows in small pieces (5120 x 13824 Q6_K: 36.7 us in 16-lane groups against
// 21.3 in passes of 64).
inline int64_t exact_work(int64_t T, int G, int J) {
  const bool xreg = G == 64 && T <= 64 * J;
  const int64_t passes = xreg ? 1 : ceil_div(T, G * J);
  return passes * J * (G < 64 ? 35 : xreg ? 28 : 32) * G;  // per 64 rows
}

inline int exact_unit(int64_t T, int max_u) {
  struct Shape {
    int u, g, j;
  };
  constexpr Shape kShapes[] = {{256, 64, 4}, {128, 64, 2}, {64, 64, 1}, {32, 32, 1}, {16, 16, 1}};
  int best = 0;
  int64_t best_work = 0;
  for (const Shape& c : kShapes) {
    if (c.u > max_u || (c.g < 64 && T > 256)) continue;
    const int64_t work = exact_work(T, c.g, c.j);
    if (best == 0 || work < best_work) best = c.u, best_work = work;
  }
  return best;
}

template <int TYPE>
int launch_exact(const void* w, int64_t n_rows, int64_t k, const uint16_t* x, void* y, int y_type, hipStream_t s) {
  using F = Exact<TYPE>;
  // Q6_K: one task a lane, 16-wave workgroups (x staged once per 16 rows).
  constexpr bool kQ6 = TYPE == SPIRAL_TYPE_Q6_K;
  constexpr int WAVES = kQ6 ? 16 : 8;
  const int u = exact_unit(k / F::kTaskElems, kQ6 ? 64 : 256);
  if (u == 16) return launch_exact_j<F, 1, 16, WAVES, 2>(w, n_rows, k, x, y, y_type, s);
  if (u == 32) return launch_exact_j<F, 1, 32, WAVES, 2>(w, n_rows, k, x, y, y_type, s);
  if constexpr (!kQ6) {
    if (u == 128) return launch_exact_j<F, 2, 64, WAVES, 2>(w, n_rows, k, x, y, y_type, s);
    if (u == 256) return launch_exact_j<F, 4, 64, WAVES, 2>(w, n_rows, k, x, y, y_type, s);
  }
  return launch_exact_j<F, 1, 64, WAVES, 2>(w, n_rows, k, x, y, y_type, s);
}

template <int TYPE>
int launch_gemv(const void* w, int64_t n_rows, int64_t k, const uint16_t* x, void* y, int y_type, bool exact,
                hipStream_t s) {
  return exact ? launch_exact<TYPE>(w, n_rows, k, x, y, y_type, s) : launch_relaxed<TYPE>(w, n_rows, k, x, y, y_type, s);
}

}  // namespace

// Largest k the LDS-staged GEMV accepts (64 KiB of staged x).
template <class F>
int64_t max_k_of() {
  const int64_t per_task = F::lds_bytes(64 * F::kTaskElems) / 64;
  return (kMaxLds / per_task / 64) * 64 * F::kTaskElems;
}

template <int TYPE>
int64_t max_k_mode(bool exact) {
  return exact ? max_k_of<Exact<TYPE>>() : max_k_of<Fmt<TYPE>>();
}

int64_t gemv_max_k(int type, bool exact) {
  switch (type) {
    case SPIRAL_TYPE_Q4_0: return max_k_mode<SPIRAL_TYPE_Q4_0>(exact);
    case SPIRAL_TYPE_Q8_0: return max_k_mode<SPIRAL_TYPE_Q8_0>(exact);
    case SPIRAL_TYPE_Q6_K: return max_k_mode<SPIRAL_TYPE_Q6_K>(exact);
    case SPIRAL_TYPE_Q4_K: return max_k_mode<SPIRAL_TYPE_Q4_K>(exact);
    case SPIRAL_TYPE_Q5_K: return max_k_mode<SPIRAL_TYPE_Q5_K>(exact);
    case SPIRAL_TYPE_IQ4_NL: return max_k_mode<SPIRAL_TYPE_IQ4_NL>(exact);
    case SPIRAL_TYPE_IQ4_XS: return max_k_mode<SPIRAL_TYPE_IQ4_XS>(exact);
    default: return 0;
  }
}

// y[n] = sum_k W[n][k] x[k]; arguments validated by the caller
// (k <= gemv_max_k(type, exact)).
int gemv(int type, const void* w, int64_t n_rows, int64_t k, const uint16_t* x, void* y, int y_type, bool exact,
         hipStream_t s) {
  switch (type) {
    case SPIRAL_TYPE_Q4_0: return launch_gemv<SPIRAL_TYPE_Q4_0>(w, n_rows, k, x, y, y_type, exact, s);
    case SPIRAL_TYPE_Q8_0: return launch_gemv<SPIRAL_TYPE_Q8_0>(w, n_rows, k, x, y, y_type, exact, s);
    case SPIRAL_TYPE_Q6_K: return launch_gemv<SPIRAL_TYPE_Q6_K>(w, n_rows, k, x, y, y_type, exact, s);
    case SPIRAL_TYPE_Q4_K: return launch_gemv<SPIRAL_TYPE_Q4_K>(w, n_rows, k, x, y, y_type, exact, s);
    case SPIRAL_TYPE_Q5_K: return launch_gemv<SPIRAL_TYPE_Q5_K>(w, n_rows, k, x, y, y_type, exact, s);
    case SPIRAL_TYPE_IQ4_NL: return launch_gemv<SPIRAL_TYPE_IQ4_NL>(w, n_rows, k, x, y, y_type, exact, s);
    case SPIRAL_TYPE_IQ4_XS: return launch_gemv<SPIRAL_TYPE_IQ4_XS>(w, n_rows, k, x, y, y_type, exact, s);
    default: return SPIRAL_ERR_TYPE;
  }
}

}  // namespace spiral
