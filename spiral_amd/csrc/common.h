// Shared definitions for the gfx950 kernels: format constants, the planar
// weight layout, scalar decode helpers and host-side validation.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "spiral_quants.h"

namespace spiral {

// ---- format constants -----------------------------------------------------
// Canonical GGUF blocks (src/quants/q4_0/layout.h:11-16,
// src/quants/q8_0/layout.h:11-14, src/quants/q6_k/layout.h:11-16).
constexpr int kQ4_0Elems = 32, kQ4_0Bytes = 18;
constexpr int kQ8_0Elems = 32, kQ8_0Bytes = 34;
constexpr int kQ6_KElems = 256, kQ6_KBytes = 210;
// K-quants with 6-bit scales and mins (ggml's block_q4_K / block_q5_K, the
// formats src/quants/TODO.md:80-107 plans): d, dmin, scales[12], [qh[32]],
// qs[128].
constexpr int kQ4_KBytes = 144, kQ5_KBytes = 176;
// Codebook formats (ggml's block_iq4_nl / block_iq4_xs, the formats
// src/quants/TODO.md:109-124 plans): 4-bit indices into a 16-entry table.
constexpr int kIQ4_NLBytes = 18, kIQ4_XSBytes = 136;

constexpr __host__ __device__ bool is_kquant(int type) {
  return type == SPIRAL_TYPE_Q4_K || type == SPIRAL_TYPE_Q5_K;
}
constexpr __host__ __device__ bool is_iq4(int type) {
  return type == SPIRAL_TYPE_IQ4_NL || type == SPIRAL_TYPE_IQ4_XS;
}
constexpr __host__ __device__ int block_elems(int type) {
  return (type == SPIRAL_TYPE_Q6_K || is_kquant(type) || type == SPIRAL_TYPE_IQ4_XS) ? 256
         : (type == SPIRAL_TYPE_Q4_0 || type == SPIRAL_TYPE_Q8_0 || type == SPIRAL_TYPE_IQ4_NL) ? 32
                                                                                                   : 0;
}
constexpr __host__ __device__ int block_bytes(int type) {
  return type == SPIRAL_TYPE_Q4_0   ? kQ4_0Bytes
         : type == SPIRAL_TYPE_Q8_0 ? kQ8_0Bytes
         : type == SPIRAL_TYPE_Q6_K ? kQ6_KBytes
         : type == SPIRAL_TYPE_Q4_K ? kQ4_KBytes
         : type == SPIRAL_TYPE_Q5_K ? kQ5_KBytes
         : type == SPIRAL_TYPE_IQ4_NL ? kIQ4_NLBytes
         : type == SPIRAL_TYPE_IQ4_XS ? kIQ4_XSBytes
                                    : 0;
}
inline bool is_quant_type(int type) { return block_elems(type) != 0; }

// ---- planar layout ----------------------------------------------------------
// Plane base pointers of one planar matrix with n_rows rows of nb blocks.
struct PlanarQ4_0 {
  const uint8_t* qs;  // [n][nb][16]
  const uint16_t* d;  // [n][nb]
  __host__ __device__ PlanarQ4_0(const void* base, int64_t n_rows, int64_t nb)
      : qs(static_cast<const uint8_t*>(base)),
        d(reinterpret_cast<const uint16_t*>(qs + n_rows * nb * 16)) {}
};
struct PlanarQ8_0 {
  const int8_t* qs;   // [n][nb][32]
  const uint16_t* d;  // [n][nb]
  __host__ __device__ PlanarQ8_0(const void* base, int64_t n_rows, int64_t nb)
      : qs(static_cast<const int8_t*>(base)),
        d(reinterpret_cast<const uint16_t*>(static_cast<const uint8_t*>(base) +
                                            n_rows * nb * 32)) {}
};
struct PlanarQ6_K {
  const uint8_t* ql;  // [n][nb][128]
  const uint8_t* qh;  // [n][nb][64]
  const int8_t* sc;   // [n][nb][16]
  const uint16_t* d;  // [n][nb]
  __host__ __device__ PlanarQ6_K(const void* base, int64_t n_rows, int64_t nb)
      : ql(static_cast<const uint8_t*>(base)),
        qh(ql + n_rows * nb * 128),
        sc(reinterpret_cast<const int8_t*>(ql + n_rows * nb * 192)),
        d(reinterpret_cast<const uint16_t*>(ql + n_rows * nb * 208)) {}
};

// K-quants: the canonical block's first 16 bytes (fp16 d, fp16 dmin, the 12
// packed scale/min bytes) stay together as one 16-byte "meta" entry, so a
// lane takes every scale of a super-block in one aligned load.
//   Q4_K: qs[n][nb][128] | meta[n][nb][16]
//   Q5_K: qs[n][nb][128] | qh[n][nb][32] | meta[n][nb][16]
struct PlanarKQ {
  const uint8_t* qs;    // [n][nb][128]
  const uint8_t* qh;    // [n][nb][32] (Q5_K)
  const uint8_t* meta;  // [n][nb][16]
  __host__ __device__ PlanarKQ(int type, const void* base, int64_t n_rows, int64_t nb)
      : qs(static_cast<const uint8_t*>(base)),
        qh(qs + n_rows * nb * 128),
        meta(qs + n_rows * nb * (type == SPIRAL_TYPE_Q5_K ? 160 : 128)) {}
};

// ---- scalar decode ------------------------------------------------------------

// Block-scale decode with the reference's device rule
// (src/quants/common/scale.aie.h:14-27): exponent 0 (zero or subnormal) gives
// +0, exponent 31 gives the finite 2^16 * (1.m), otherwise IEEE binary16.
// Written as an integer select so it compiles to v_cndmask, not a branch.
__device__ __forceinline__ float fp16_scale(uint32_t h) {
  const uint32_t t = h & 0x7fffu;
  const uint32_t bits = ((h << 16) & 0x80000000u) | ((t << 13) + 0x38000000u);
  return __uint_as_float(t >= 0x400u ? bits : 0u);
}

// The same decode for a scale that only ever multiplies codes inside an FMA
// with its offset term (code * s - c * s, both exact): the hardware
// conversion agrees with fp16_scale on exponents 1..30, and its -0 for a
// -0 scale still gives every code a +0 weight. Exponents 0 (non-zero
// mantissa: the hardware keeps the subnormal) and 31 (inf / NaN there) are
// the reference's special cases; a wave in which any lane holds one takes
// the bit-level decode for all its lanes (a wave-uniform branch), so the
// common path costs one conversion and one class test instead of six
// instructions.
__device__ __forceinline__ float fp16_scale_fma(uint32_t h) {
  const _Float16 hf = __builtin_bit_cast(_Float16, static_cast<uint16_t>(h));
  // v_cmp_class mask: signaling and quiet NaN, -inf, -subnormal, +subnormal, +inf
  constexpr int kSpecial = 0x001 | 0x002 | 0x004 | 0x010 | 0x080 | 0x200;
  float f = static_cast<float>(hf);
  if (__builtin_amdgcn_ballot_w64(__builtin_amdgcn_classh(hf, kSpecial)) != 0) f = fp16_scale(h);
  return f;
}

// IEEE binary16 -> float (subnormals keep their value): the K-quants' d and
// dmin, decoded as ggml decodes them (v_cvt_f32_f16).
__device__ __forceinline__ float fp16_ieee(uint32_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

// 6-bit scale (bits 0..7) and min (bits 8..15) of group g (0..7) of a K-quant
// super-block, from the dwords s0, s1, s2 of its 12 packed bytes:
//   bytes 0..3   bits 0..5 scale of groups 0..3, bits 6..7 bits 4..5 of the
//                scale of groups 4..7
//   bytes 4..7   the same for the mins
//   bytes 8..11  bits 0..3 of the scale (low nibble) and min (high nibble)
//                of groups 4..7
__device__ __forceinline__ uint32_t kq_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int g) {
  const uint32_t sh = 8u * static_cast<uint32_t>(g & 3);
  const uint32_t a = (s0 >> sh) & 0xffu, b = (s1 >> sh) & 0xffu, c = (s2 >> sh) & 0xffu;
  const uint32_t sc = g < 4 ? (a & 63u) : ((c & 15u) | ((a >> 6) << 4));
  const uint32_t mn = g < 4 ? (b & 63u) : ((c >> 4) | ((b >> 6) << 4));
  return sc | (mn << 8);
}

// kq_scale_min of groups 2j and 2j + 1 (chunk j = 0..3: the low and high
// nibbles of 32 qs bytes) as bytes (scale 2j, min 2j, scale 2j + 1, min
// 2j + 1), with no branch on j: two v_perm_b32 gather bytes o and o + 1
// (o = 2 (j % 2)) of s0, s1 and s2, and a bit select on j / 2 picks the
// 6-bit fields (groups 0..3) or the nibbles of s2 under the top bits of s0
// and s1 (groups 4..7).
__device__ __forceinline__ uint32_t kq_chunk_scales(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t j) {
  const uint32_t sel = 0x05010400u + 2u * (j & 1u) * 0x01010101u;
  const uint32_t a = __builtin_amdgcn_perm(s1, s0, sel);       // s0[o], s1[o], s0[o + 1], s1[o + 1]
  const uint32_t c = __builtin_amdgcn_perm(s2 >> 4, s2, sel);  // s2[o] and its high nibble, the same for o + 1
  const uint32_t lo = a & 0x3F3F3F3Fu;
  const uint32_t hi = (c & 0x0F0F0F0Fu) | ((a >> 2) & 0x30303030u);
  const uint32_t m = 0u - (j >> 1);
  return (hi & m) | (lo & ~m);
}

// IQ4 codebook entries of four 4-bit indices held one per byte of c (values
// 0..15), as bytes kv + 128 (1..241) of ggml's kvalues_iq4nl
// {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113}:
// one v_perm_b32 looks up entries 0..7, one entries 8..15, and a third picks
// per byte by index bit 3.
__device__ __forceinline__ uint32_t iq4_lut(uint32_t c) {
  const uint32_t sel = c & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(0x766A5D4Fu, 0x3F2D1801u, sel);  // entries 4..7 | 0..3
  const uint32_t hi = __builtin_amdgcn_perm(0xF1D9C5B5u, 0xA6998D81u, sel);  // entries 12..15 | 8..11
  return __builtin_amdgcn_perm(hi, lo, ((c >> 1) & 0x04040404u) | 0x03020100u);
}

// IQ4_XS sub-block scale d * (ls - 32) from a super-block's first 8 bytes
// m = (d | scales_h << 16, scales_l[0..3]): ls = nibble b % 2 of
// scales_l[b / 2] | bits 2b..2b+1 of scales_h << 4. Exact in fp32.
__device__ __forceinline__ float iq4xs_scale(uint2 m, int b) {
  const uint32_t ls = ((m.y >> (4 * b)) & 15u) | (((m.x >> (16 + 2 * b)) & 3u) << 4);
  return fp16_ieee(m.x & 0xffffu) * static_cast<float>(static_cast<int>(ls) - 32);
}

// (w & mask) | hi in one v_and_or_b32, with the mask in an SGPR and hi in a
// VGPR: a gfx9 VOP3 reads at most one scalar operand and no literal, so
// written as C the compiler emits a v_and and a v_or with literals instead.
// Q4_0 nibbles become fp16 pairs this way: (w & 0x000F000F) | 0x64006400 is
// (1024 + c0, 1024 + c2) for the low nibbles of bytes 0 and 2, and the mask
// 0x00F000F0 under 0x54005400 gives their high nibbles as (64 + c).
__device__ __forceinline__ uint32_t and_or_b32(uint32_t w, uint32_t mask, uint32_t hi) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(w), "s"(mask), "v"(hi));
  return r;
}

// Two floats -> packed bf16 pair (lo in bits 0..15), round to nearest even.
// Lowers to v_cvt_pk_bf16_f32 on gfx950.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
  bf16x2_t v;
  v[0] = (__bf16)lo;
  v[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float bf16_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t pair) { return __uint_as_float(pair & 0xffff0000u); }

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte streaming load for payload read exactly once per kernel; the
// non-temporal hint keeps it from displacing reused data (x, scales) in cache.
__device__ __forceinline__ uint4 load_stream16(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(static_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// 16-byte streaming store for output written once and not read again by the
// kernel that writes it: the non-temporal hint streams it to memory instead
// of holding it in L2 (bf16 dequant: 1.3-1.4x faster than plain stores).
__device__ __forceinline__ void store_stream16(void* p, uint4 v) {
  __builtin_nontemporal_store(u32x4_t{v.x, v.y, v.z, v.w}, static_cast<u32x4_t*>(p));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// x moved across lanes by DPP control CTRL; rows outside ROW_MASK read 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xF, false));
}

// Sum over each group of G consecutive lanes (G = 16, 32 or 64) in DPP adds
// (no LDS round trips): pairs, quads, then the four quads of each 16-lane row
// (rotations by 4 and 8, after which every lane of a row holds the row's
// sum), then the rows (broadcasts of lane 15 and lane 31). A group's sum is
// exact in its last lane; other lanes may hold partial sums.
template <int G>
__device__ __forceinline__ float group_sum_last(float v) {
  static_assert(G == 16 || G == 32 || G == 64, "groups of 16, 32 or 64 lanes");
  v += dpp_f32<0xB1, 0xF>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_f32<0x4E, 0xF>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_f32<0x124, 0xF>(v);  // row_ror 4
  v += dpp_f32<0x128, 0xF>(v);  // row_ror 8
  if constexpr (G >= 32) v += dpp_f32<0x142, 0xA>(v);  // row_bcast 15: row 0 into row 1, row 2 into row 3
  if constexpr (G == 64) v += dpp_f32<0x143, 0xC>(v);  // row_bcast 31: rows 0-1 into rows 2 and 3
  return v;
}

// Sum over the wave's 64 lanes, exact in lane 63.
__device__ __forceinline__ float wave_sum_last(float v) { return group_sum_last<64>(v); }

// ---- host-side helpers ----------------------------------------------------------

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int launch_status() {
  return hipGetLastError() == hipSuccess ? SPIRAL_OK : SPIRAL_ERR_HIP;
}

// Checks that a device is visible; the first failing call is reported as
// SPIRAL_ERR_NO_DEVICE so callers can tell "no GPU" from a kernel failure.
int require_device();

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Compute units of the current device (cached per device id).
int device_cu_count();

// Workgroups of `kernel` resident per CU at `threads` threads and `lds` bytes
// of dynamic LDS (hipOccupancyMaxActiveBlocksPerMultiprocessor, cached; 1 when
// the query fails).
int blocks_per_cu(const void* kernel, int threads, int64_t lds);

// Raises `kernel`'s dynamic-LDS limit to `bytes` on the current device
// (hipFuncSetAttribute once per device and kernel, thread-safe).
int allow_dynamic_lds(const void* kernel, int bytes);

}  // namespace spiral
