// Exact dequantization helpers shared by the standalone dequant / GET_ROWS
// kernels and the GEMM / MoE weight-tile loaders, so the fused products and
// the standalone dequant cannot drift apart.
//
// Every element value is bf16_rne(exact product):
//   Q4_0  (q - 8) * d, Q8_0 q * d, Q6_K d * sc * (q - 32)
// (src/quants/q4_0/unpack.aie.h:31-46, src/quants/q8_0/unpack.aie.h:37-52,
// src/quants/q6_k/unpack.aie.h:33-138). Each product is exact in fp32
// (at most 24 significant bits), so one round-to-nearest-even conversion
// (v_cvt_pk_bf16_f32) gives the reference's bits.
#pragma once

#include "common.h"

namespace spiral {

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

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
  } else if constexpr (is_iq4(TYPE)) {
    // IQ4_NL: Q4_0's block with codebook values; IQ4_XS: eight such 32-element
    // sub-blocks per super-block, sub-block b scaled by d * (ls_b - 32).
    // Every product is exact in fp32.
    int64_t qoff;
    float dl;
    if constexpr (TYPE == SPIRAL_TYPE_IQ4_NL) {
      const int64_t b = n * nb + (g >> 2);
      qoff = b * 16;
      dl = fp16_ieee(reinterpret_cast<const uint16_t*>(w + n_rows * nb * 16)[b]);
    } else {
      const int64_t blk = n * nb + (g >> 5);
      const int sub = static_cast<int>((g & 31) >> 2);
      qoff = blk * 128 + 16 * sub;
      dl = iq4xs_scale(reinterpret_cast<const uint2*>(w + n_rows * nb * 128)[blk], sub);
    }
    const int p = static_cast<int>(g & 3);
    const uint2 q = *reinterpret_cast<const uint2*>(w + qoff + 8 * (p & 1));
    const int shift = (p >> 1) * 4;
    const uint32_t v0 = iq4_lut((q.x >> shift) & 0x0F0F0F0Fu), v1 = iq4_lut((q.y >> shift) & 0x0F0F0F0Fu);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = static_cast<float>(static_cast<int>((v0 >> (8 * j)) & 0xffu) - 128) * dl;
      v[j + 4] = static_cast<float>(static_cast<int>((v1 >> (8 * j)) & 0xffu) - 128) * dl;
    }
  } else if constexpr (is_kquant(TYPE)) {
    // Group j (32 elements) of a super-block: the low (j even) or high nibble
    // of qs[32 (j / 2) + l], Q5_K adding bit j of qh[l] as bit 4; value
    // fma(d * scale_j, q, -dmin * min_j), one rounding, then bf16 RNE.
    const PlanarKQ P(TYPE, w, n_rows, nb);
    const int64_t sb = g >> 5;
    const int t = static_cast<int>(g & 31);
    const int j = t >> 2, l0 = (t & 3) * 8;
    const int64_t blk = n * nb + sb;
    const uint2 q = *reinterpret_cast<const uint2*>(P.qs + blk * 128 + 32 * (j >> 1) + l0);
    const uint4 m = *reinterpret_cast<const uint4*>(P.meta + blk * 16);
    const uint32_t sm = kq_scale_min(m.y, m.z, m.w, j);
    const float d1 = fp16_ieee(m.x & 0xffffu) * static_cast<float>(sm & 0xffu);
    const float m1 = fp16_ieee(m.x >> 16) * static_cast<float>(sm >> 8);
    const int ns = (j & 1) * 4;
    uint2 hb = make_uint2(0u, 0u);
    if constexpr (TYPE == SPIRAL_TYPE_Q5_K) hb = *reinterpret_cast<const uint2*>(P.qh + blk * 32 + l0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t c0 = ((q.x >> (8 * e + ns)) & 15u) | (((hb.x >> (8 * e + j)) & 1u) << 4);
      const uint32_t c1 = ((q.y >> (8 * e + ns)) & 15u) | (((hb.y >> (8 * e + j)) & 1u) << 4);
      v[e] = __builtin_fmaf(d1, static_cast<float>(c0), -m1);
      v[e + 4] = __builtin_fmaf(d1, static_cast<float>(c1), -m1);
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

// ---- 16-element weight-tile pieces for the MFMA kernels -------------------
//
// A "piece" is 16 consecutive elements of one weight row starting at a
// multiple of 16: its packed bytes are loaded into registers (Piece), then
// dequantized to 16 bf16 (two uint4) and written to LDS. Splitting load and
// dequant lets a kernel keep later tiles' loads in flight while it
// multiplies the current one.
//
// Pieces are read with buffer loads: Piece::Addr fixes, per thread, the row
// and the piece's place inside a 128-element k step (pl = 0..7), and a step
// adds only scalar offsets. Offsets are 32-bit, so every plane of the
// weight tensor must stay below 4 GiB (checked by the launcher).
//
// The values equal dequant8's. The one difference is the sign of a zero
// weight (code 8 of Q4_0, 0 of Q8_0, 32 of Q6_K) under a negative scale: +0
// here, -0 in dequant8. Zero weights contribute nothing to a product, so
// the products are unaffected; the bit-exact dequant entry points use
// dequant8.

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  // Third dword 0x00020000: raw (untyped) 32-bit accesses on gfx9-class GPUs.
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

template <int TYPE>
struct Piece;

// Buffer resources over the planes of one planar weight tensor.
struct Planes {
  __amdgpu_buffer_rsrc_t a, b, c, d;
};

template <int TYPE>
__device__ __forceinline__ Planes make_planes(const uint8_t* w, int64_t n_rows, int64_t nb) {
  const int64_t tot = n_rows * nb;
  Planes P;
  if constexpr (TYPE == SPIRAL_TYPE_Q4_0 || TYPE == SPIRAL_TYPE_IQ4_NL) {
    P.a = buffer_rsrc(w, static_cast<uint32_t>(tot * 16));
    // d plane rounded up to whole dwords: a dword load of the last d (at a
    // 4-byte aligned address, so inside the same page) then reads it instead
    // of failing the range check; the 2 bytes past the plane are only ever
    // taken for blocks past the row's end, whose d is forced to 0.
    P.d = buffer_rsrc(w + tot * 16, static_cast<uint32_t>((tot * 2 + 3) & ~int64_t(3)));
    P.b = P.c = P.a;
  } else if constexpr (TYPE == SPIRAL_TYPE_Q8_0) {
    P.a = buffer_rsrc(w, static_cast<uint32_t>(tot * 32));
    P.d = buffer_rsrc(w + tot * 32, static_cast<uint32_t>(tot * 2));
    P.b = P.c = P.a;
  } else if constexpr (TYPE == SPIRAL_TYPE_IQ4_XS) {
    P.a = buffer_rsrc(w, static_cast<uint32_t>(tot * 128));  // qs
    P.c = buffer_rsrc(w + tot * 128, static_cast<uint32_t>(tot * 8));  // meta
    P.b = P.a;
    P.d = P.c;
  } else if constexpr (is_kquant(TYPE)) {
    // a: qs, b: qh (Q5_K), c: meta
    constexpr int64_t kMeta = TYPE == SPIRAL_TYPE_Q5_K ? 160 : 128;
    P.a = buffer_rsrc(w, static_cast<uint32_t>(tot * 128));
    P.b = TYPE == SPIRAL_TYPE_Q5_K ? buffer_rsrc(w + tot * 128, static_cast<uint32_t>(tot * 32)) : P.a;
    P.c = buffer_rsrc(w + tot * kMeta, static_cast<uint32_t>(tot * 16));
    P.d = P.c;
  } else {
    P.a = buffer_rsrc(w, static_cast<uint32_t>(tot * 128));
    P.b = buffer_rsrc(w + tot * 128, static_cast<uint32_t>(tot * 64));
    P.c = buffer_rsrc(w + tot * 192, static_cast<uint32_t>(tot * 16));
    P.d = buffer_rsrc(w + tot * 208, static_cast<uint32_t>(tot * 2));
  }
  return P;
}

__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint32_t bload4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
__device__ __forceinline__ uint32_t bload2(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
}
__device__ __forceinline__ uint32_t bload1(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b8(r, voff, soff, 0);
}

// Q4_0: piece 2b + h of a row is nibble h of block b's 16 qs bytes.
template <>
struct Piece<SPIRAL_TYPE_Q4_0> {
  uint4 q;
  uint32_t d;
  struct Addr {
    uint32_t qs, d;
    int hi;
  };
  // Row n, local piece pl of a 128-element step.
  static __device__ __forceinline__ Addr addr(int64_t n, int64_t nb, int pl) {
    const uint32_t b = static_cast<uint32_t>(n * nb) + (pl >> 1);
    return Addr{b * 16u, b * 2u, pl & 1};
  }
  // Step starting at element k0 (a multiple of 128).
  __device__ __forceinline__ void load(const Planes& P, const Addr& A, int64_t k0) {
    const uint32_t kb = static_cast<uint32_t>(k0 >> 5);
    q = bload16(P.a, A.qs, kb * 16u);
    d = bload2(P.d, A.d, kb * 2u);
  }
  __device__ __forceinline__ void zero() { q = make_uint4(0u, 0u, 0u, 0u); d = 0u; }
  // fp16 (1024 + c) times d minus 1032 d is (c - 8) d, exact inside the FMA.
  // High nibbles are taken in place: byte 16 c under the high byte 0x54 is
  // the fp16 64 + c, and (64 + c) d - 72 d is (c - 8) d, exact as well, with
  // no shift. The scale decode has no branch, so the compiler can spread
  // this among the MFMAs of the kernel's step.
  __device__ __forceinline__ void dequant(const Addr& A, uint4& o0, uint4& o1) const {
    const float df = fp16_scale(d), off = (A.hi ? -72.0f : -1032.0f) * df;
    const uint32_t mask = A.hi ? 0xF0F0F0F0u : 0x0F0F0F0Fu, magic = A.hi ? 0x54545454u : 0x64646464u;
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    uint32_t o[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t c = w[i] & mask;
      const f16x2_t a = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(magic, c, 0x04010400u));
      const f16x2_t b = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(magic, c, 0x04030402u));
      o[2 * i] = pack_bf16x2(__builtin_fmaf(static_cast<float>(a.x), df, off), __builtin_fmaf(static_cast<float>(a.y), df, off));
      o[2 * i + 1] = pack_bf16x2(__builtin_fmaf(static_cast<float>(b.x), df, off), __builtin_fmaf(static_cast<float>(b.y), df, off));
    }
    o0 = make_uint4(o[0], o[1], o[2], o[3]);
    o1 = make_uint4(o[4], o[5], o[6], o[7]);
  }
};

// Q8_0: piece 2b + h of a row is qs[16h .. 16h + 15] of block b.
template <>
struct Piece<SPIRAL_TYPE_Q8_0> {
  uint4 q;
  uint32_t d;
  struct Addr {
    uint32_t qs, d;
  };
  static __device__ __forceinline__ Addr addr(int64_t n, int64_t nb, int pl) {
    const uint32_t b = static_cast<uint32_t>(n * nb) + (pl >> 1);
    return Addr{b * 32u + 16u * (pl & 1), b * 2u};
  }
  __device__ __forceinline__ void load(const Planes& P, const Addr& A, int64_t k0) {
    const uint32_t kb = static_cast<uint32_t>(k0 >> 5);
    q = bload16(P.a, A.qs, kb * 32u);
    d = bload2(P.d, A.d, kb * 2u);
  }
  __device__ __forceinline__ void zero() { q = make_uint4(0u, 0u, 0u, 0u); d = 0u; }
  // (q ^ 0x80) is q + 128: fp16 (1024 + q + 128) times d minus 1152 d.
  __device__ __forceinline__ void dequant(const Addr&, uint4& o0, uint4& o1) const {
    const float df = fp16_scale(d), off = -1152.0f * df;
    const uint32_t w[4] = {q.x ^ 0x80808080u, q.y ^ 0x80808080u, q.z ^ 0x80808080u, q.w ^ 0x80808080u};
    uint32_t o[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f16x2_t a = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, w[i], 0x04010400u));
      const f16x2_t b = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, w[i], 0x04030402u));
      o[2 * i] = pack_bf16x2(__builtin_fmaf(static_cast<float>(a.x), df, off), __builtin_fmaf(static_cast<float>(a.y), df, off));
      o[2 * i + 1] = pack_bf16x2(__builtin_fmaf(static_cast<float>(b.x), df, off), __builtin_fmaf(static_cast<float>(b.y), df, off));
    }
    o0 = make_uint4(o[0], o[1], o[2], o[3]);
    o1 = make_uint4(o[4], o[5], o[6], o[7]);
  }
};

// Q6_K: a 128-element step is half h = (k0 / 128) % 2 of super-block k0 / 256;
// local piece pl covers elements 128 h + 32 j + l0 + i (j = pl / 2,
// l0 = 16 (pl % 2), i < 16) with the single sub-scale sc[8 h + pl % 2 + 2 j].
template <>
struct Piece<SPIRAL_TYPE_Q6_K> {
  uint4 lo, hb;
  uint32_t ds_bits;  // fp16 d (low 16 bits) and the int8 sub-scale (bits 16..23)
  struct Addr {
    uint32_t ql, qh, sc, d;
    int ls, hs;  // nibble shift (0 or 4) and 2-bit field shift (2 j)
  };
  static __device__ __forceinline__ Addr addr(int64_t n, int64_t nb, int pl) {
    const uint32_t blk = static_cast<uint32_t>(n * nb);
    const int j = pl >> 1, l0 = 16 * (pl & 1);
    return Addr{blk * 128u + 32u * (j & 1) + l0, blk * 64u + l0, blk * 16u + (pl & 1) + 2 * j, blk * 2u,
                (j >> 1) * 4, 2 * j};
  }
  __device__ __forceinline__ void load(const Planes& P, const Addr& A, int64_t k0) {
    const uint32_t sb = static_cast<uint32_t>(k0 >> 8), h = static_cast<uint32_t>((k0 >> 7) & 1);
    lo = bload16(P.a, A.ql, sb * 128u + 64u * h);
    hb = bload16(P.b, A.qh, sb * 64u + 32u * h);
    const uint32_t sc = bload1(P.c, A.sc, sb * 16u + 8u * h);
    ds_bits = bload2(P.d, A.d, sb * 2u) | (sc << 16);
  }
  __device__ __forceinline__ void zero() { lo = hb = make_uint4(0u, 0u, 0u, 0u); ds_bits = 0u; }
  // ds = d * sc is exact (<= 19 bits); code * ds - 32 ds is exact in the FMA
  // and fits fp32 (<= 24 bits).
  __device__ __forceinline__ void dequant(const Addr& A, uint4& o0, uint4& o1) const {
    const float ds = fp16_scale(ds_bits & 0xffffu) * static_cast<float>(static_cast<int8_t>(ds_bits >> 16));
    const float off = -32.0f * ds;
    const uint32_t L[4] = {lo.x, lo.y, lo.z, lo.w}, H[4] = {hb.x, hb.y, hb.z, hb.w};
    uint32_t o[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t c = ((L[i] >> A.ls) & 0x0F0F0F0Fu) | (((H[i] >> A.hs) & 0x03030303u) << 4);
      o[2 * i] = pack_bf16x2(__builtin_fmaf(static_cast<float>(c & 0xffu), ds, off),
                             __builtin_fmaf(static_cast<float>((c >> 8) & 0xffu), ds, off));
      o[2 * i + 1] = pack_bf16x2(__builtin_fmaf(static_cast<float>((c >> 16) & 0xffu), ds, off),
                                 __builtin_fmaf(static_cast<float>(c >> 24), ds, off));
    }
    o0 = make_uint4(o[0], o[1], o[2], o[3]);
    o1 = make_uint4(o[4], o[5], o[6], o[7]);
  }
};

// K-quants: a 128-element step is half h = (k0 / 128) % 2 of super-block
// k0 / 256; local piece pl covers elements 16 pl .. + 15 of the half, which
// lie in group j = 4 h + pl / 2: qs bytes 64 h + 32 (pl / 4) + 16 (pl % 2)
// .. + 15, nibble (pl / 2) % 2, Q5_K bit j of qh[16 (pl % 2) .. + 15]. The
// piece carries the super-block's 16-byte meta (d, dmin, packed scales).
template <int TYPE>
struct PieceKQ {
  uint4 q, meta, qh;
  int grp;  // j
  struct Addr {
    uint32_t qs, qh, meta;
    int jl, nib;  // pl / 2 and (pl / 2) % 2
  };
  static __device__ __forceinline__ Addr addr(int64_t n, int64_t nb, int pl) {
    const uint32_t blk = static_cast<uint32_t>(n * nb);
    return Addr{blk * 128u + 32u * (pl >> 2) + 16u * (pl & 1), blk * 32u + 16u * (pl & 1), blk * 16u, pl >> 1,
                (pl >> 1) & 1};
  }
  __device__ __forceinline__ void load(const Planes& P, const Addr& A, int64_t k0) {
    const uint32_t sb = static_cast<uint32_t>(k0 >> 8), h = static_cast<uint32_t>((k0 >> 7) & 1);
    q = bload16(P.a, A.qs, sb * 128u + 64u * h);
    meta = bload16(P.c, A.meta, sb * 16u);
    if constexpr (TYPE == SPIRAL_TYPE_Q5_K) qh = bload16(P.b, A.qh, sb * 32u);
    grp = 4 * static_cast<int>(h) + A.jl;
  }
  __device__ __forceinline__ void zero() { q = meta = qh = make_uint4(0u, 0u, 0u, 0u); grp = 0; }
  __device__ __forceinline__ void dequant(const Addr& A, uint4& o0, uint4& o1) const {
    const uint32_t sm = kq_scale_min(meta.y, meta.z, meta.w, grp);
    const float d1 = fp16_ieee(meta.x & 0xffffu) * static_cast<float>(sm & 0xffu);
    const float m1 = -(fp16_ieee(meta.x >> 16) * static_cast<float>(sm >> 8));
    const uint32_t Q[4] = {q.x, q.y, q.z, q.w}, H[4] = {qh.x, qh.y, qh.z, qh.w};
    uint32_t o[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t c = (A.nib ? (Q[i] >> 4) : Q[i]) & 0x0F0F0F0Fu;
      if constexpr (TYPE == SPIRAL_TYPE_Q5_K) c |= ((H[i] >> grp) & 0x01010101u) << 4;
      o[2 * i] = pack_bf16x2(__builtin_fmaf(d1, static_cast<float>(c & 0xffu), m1),
                             __builtin_fmaf(d1, static_cast<float>((c >> 8) & 0xffu), m1));
      o[2 * i + 1] = pack_bf16x2(__builtin_fmaf(d1, static_cast<float>((c >> 16) & 0xffu), m1),
                                 __builtin_fmaf(d1, static_cast<float>(c >> 24), m1));
    }
    o0 = make_uint4(o[0], o[1], o[2], o[3]);
    o1 = make_uint4(o[4], o[5], o[6], o[7]);
  }
};
template <>
struct Piece<SPIRAL_TYPE_Q4_K> : PieceKQ<SPIRAL_TYPE_Q4_K> {};
template <>
struct Piece<SPIRAL_TYPE_Q5_K> : PieceKQ<SPIRAL_TYPE_Q5_K> {};

// IQ4: 16 indices (one nibble of 16 qs bytes) -> codebook bytes (kv + 128)
// -> fp16 pairs (1024 + kv + 128), times the scale minus 1152 scale: kv times
// the scale, exact inside the FMA (the result has at most 24 bits).
__device__ __forceinline__ void iq4_dequant16(const uint4& q, int hi, float df, uint4& o0, uint4& o1) {
  const float off = -1152.0f * df;
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  uint32_t o[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t c = iq4_lut((hi ? (w[i] >> 4) : w[i]) & 0x0F0F0F0Fu);
    const f16x2_t a = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, c, 0x04010400u));
    const f16x2_t b = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, c, 0x04030402u));
    o[2 * i] = pack_bf16x2(__builtin_fmaf(static_cast<float>(a.x), df, off), __builtin_fmaf(static_cast<float>(a.y), df, off));
    o[2 * i + 1] = pack_bf16x2(__builtin_fmaf(static_cast<float>(b.x), df, off), __builtin_fmaf(static_cast<float>(b.y), df, off));
  }
  o0 = make_uint4(o[0], o[1], o[2], o[3]);
  o1 = make_uint4(o[4], o[5], o[6], o[7]);
}

// IQ4_NL: piece 2b + h of a row is nibble h of block b's 16 qs bytes (as Q4_0).
template <>
struct Piece<SPIRAL_TYPE_IQ4_NL> {
  uint4 q;
  uint32_t d;
  using Addr = Piece<SPIRAL_TYPE_Q4_0>::Addr;
  static __device__ __forceinline__ Addr addr(int64_t n, int64_t nb, int pl) {
    return Piece<SPIRAL_TYPE_Q4_0>::addr(n, nb, pl);
  }
  __device__ __forceinline__ void load(const Planes& P, const Addr& A, int64_t k0) {
    const uint32_t kb = static_cast<uint32_t>(k0 >> 5);
    q = bload16(P.a, A.qs, kb * 16u);
    d = bload2(P.d, A.d, kb * 2u);
  }
  __device__ __forceinline__ void zero() { q = make_uint4(0u, 0u, 0u, 0u); d = 0u; }
  __device__ __forceinline__ void dequant(const Addr& A, uint4& o0, uint4& o1) const {
    iq4_dequant16(q, A.hi, fp16_ieee(d), o0, o1);
  }
};

// IQ4_XS: a 128-element step is half h of super-block k0 / 256; local piece pl
// is nibble pl % 2 of sub-block 4 h + pl / 2's 16 qs bytes.
template <>
struct Piece<SPIRAL_TYPE_IQ4_XS> {
  uint4 q;
  uint2 meta;
  int sub;
  struct Addr {
    uint32_t qs, meta;
    int sl, hi;  // pl / 2 and pl % 2
  };
  static __device__ __forceinline__ Addr addr(int64_t n, int64_t nb, int pl) {
    const uint32_t blk = static_cast<uint32_t>(n * nb);
    return Addr{blk * 128u + 16u * (pl >> 1), blk * 8u, pl >> 1, pl & 1};
  }
  __device__ __forceinline__ void load(const Planes& P, const Addr& A, int64_t k0) {
    const uint32_t sb = static_cast<uint32_t>(k0 >> 8), h = static_cast<uint32_t>((k0 >> 7) & 1);
    q = bload16(P.a, A.qs, sb * 128u + 64u * h);
    meta = make_uint2(bload4(P.c, A.meta, sb * 8u), bload4(P.c, A.meta + 4u, sb * 8u));
    sub = 4 * static_cast<int>(h) + A.sl;
  }
  __device__ __forceinline__ void zero() { q = make_uint4(0u, 0u, 0u, 0u); meta = make_uint2(0u, 0u); sub = 0; }
  __device__ __forceinline__ void dequant(const Addr& A, uint4& o0, uint4& o1) const {
    iq4_dequant16(q, A.hi, iq4xs_scale(meta, sub), o0, o1);
  }
};

}  // namespace spiral
