// Per-format weight pieces of the MoE kernels: one 128-wide
// k step of one weight row for MFMA lane group g, loaded once and
// dequantized exactly to bf16 eight elements at a time, one group of eight
// for each of the step's four v_mfma_f32_16x16x32_bf16 (MFMA s takes
// elements local(g, s, 0..7) of the step from lane group g). The
// activations are staged or packed in the same order, so any kernel that
// feeds MFMA s of a step with dequant(s) and the matching activations forms
// each (row, column) sum from the same operands in the same order.
#pragma once

#include "common.h"
#include "dequant_impl.h"

namespace spiral {
namespace {

// One 128-wide k step of one weight row for lane group g:
// loaded once, then dequantized 8 elements at a time for MFMA s = 0..3.
// local(g, s, e) is the k offset inside the step of element e < 8 of MFMA s.
template <int TYPE>
struct MoePiece;

// Whether MFMA s's elements e = 0..3 (and 4..7) are the four consecutive
// elements local(g, s, 0) + {0, 2, 1, 3}: the activations of each run of
// four are then staged with the middle two swapped (stage_swap).
template <int TYPE>
constexpr bool kStageSwap = TYPE == SPIRAL_TYPE_Q4_0;

// (a0, a1, a2, a3) -> (a0, a2, a1, a3) for four bf16 in two dwords.
__device__ __forceinline__ uint2 stage_swap(uint2 v) {
  return make_uint2(__builtin_amdgcn_perm(v.y, v.x, 0x05040100u), __builtin_amdgcn_perm(v.y, v.x, 0x07060302u));
}

// Q4_0: piece = block 4 kb + g. MFMA s takes qs dword s: bytes j = 0..3
// hold elements 4s + j (low nibbles) and 16 + 4s + j (high nibbles). One
// v_and_or_b32 turns two nibbles into an fp16 pair in place: (w & 0x000F000F)
// | 0x64006400 is (1024 + c) for elements 4s and 4s + 2, (w & 0x00F000F0) |
// 0x54005400 is (64 + c) for 16 + 4s and 16 + 4s + 2 (byte 16 c under the
// high byte 0x54: exponent 6, mantissa step 1/16), and w >> 8 gives the odd
// elements the same way. (1024 + c) m - 1032 m and (64 + c) m - 72 m are
// (c - 8) m, exact inside the FMA. So MFMA s takes elements 4s, 4s + 2,
// 4s + 1, 4s + 3, then the same plus 16: the activations are staged in that
// order (kStageSwap).
template <>
struct MoePiece<SPIRAL_TYPE_Q4_0> {
  uint4 q;
  uint32_t d;
  float m, off, off_hi;  // decoded scale and offsets (prep)
  static __device__ __forceinline__ int local(int g, int s, int e) {
    return 32 * g + (e >= 4 ? 16 : 0) + 4 * s + ((e & 1) << 1) + ((e >> 1) & 1);
  }
  __device__ __forceinline__ void prep() {
    m = fp16_scale_fma(d);
    off = -1032.0f * m;
    off_hi = -72.0f * m;
  }
  // blk = block index of the lane's piece within the row's planar planes
  __device__ __forceinline__ void load(const uint8_t* we, int64_t tot, int64_t blk) {
    q = *reinterpret_cast<const uint4*>(we + blk * 16);
    d = *reinterpret_cast<const uint16_t*>(we + tot * 16 + blk * 2);
  }
  __device__ __forceinline__ void zero() { q = make_uint4(0u, 0u, 0u, 0u); d = 0u; }
  static __device__ __forceinline__ f16x2_t and_or(uint32_t w, uint32_t mask, uint32_t hi) {
    return __builtin_bit_cast(f16x2_t, and_or_b32(w, mask, hi));
  }
  __device__ __forceinline__ uint4 dequant(int s) const {
    const uint32_t w = s == 0 ? q.x : s == 1 ? q.y : s == 2 ? q.z : q.w;
    const uint32_t w8 = w >> 8;
    const f16x2_t p[4] = {and_or(w, 0x000F000Fu, 0x64006400u),    // 4s, 4s + 2
                          and_or(w8, 0x000F000Fu, 0x64006400u),   // 4s + 1, 4s + 3
                          and_or(w, 0x00F000F0u, 0x54005400u),    // 16 + (4s, 4s + 2)
                          and_or(w8, 0x00F000F0u, 0x54005400u)};  // 16 + (4s + 1, 4s + 3)
    // all eight products first, then the packs: a pack right behind the FMA
    // that feeds it costs a wait state
    float v[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float of = i < 2 ? off : off_hi;
      v[2 * i] = __builtin_fmaf(static_cast<float>(p[i].x), m, of);
      v[2 * i + 1] = __builtin_fmaf(static_cast<float>(p[i].y), m, of);
    }
    return make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                      pack_bf16x2(v[6], v[7]));
  }
};

// Q8_0: piece = block 4 kb + g; MFMA s takes qs bytes 8s .. 8s + 7.
template <>
struct MoePiece<SPIRAL_TYPE_Q8_0> {
  uint4 q0, q1;
  uint32_t d;
  float m, off;  // decoded scale and offset (prep)
  static __device__ __forceinline__ int local(int g, int s, int e) { return 32 * g + 8 * s + e; }
  __device__ __forceinline__ void prep() {
    m = fp16_scale(d);
    off = -1152.0f * m;
  }
  __device__ __forceinline__ void load(const uint8_t* we, int64_t tot, int64_t blk) {
    q0 = *reinterpret_cast<const uint4*>(we + blk * 32);
    q1 = *reinterpret_cast<const uint4*>(we + blk * 32 + 16);
    d = *reinterpret_cast<const uint16_t*>(we + tot * 32 + blk * 2);
  }
  __device__ __forceinline__ void zero() { q0 = q1 = make_uint4(0u, 0u, 0u, 0u); d = 0u; }
  __device__ __forceinline__ uint4 dequant(int s) const {
    const uint32_t w0 = (s == 0 ? q0.x : s == 1 ? q0.z : s == 2 ? q1.x : q1.z) ^ 0x80808080u;
    const uint32_t w1 = (s == 0 ? q0.y : s == 1 ? q0.w : s == 2 ? q1.y : q1.w) ^ 0x80808080u;
    const float df = m;
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t c = i ? w1 : w0;
      const f16x2_t a = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, c, 0x04010400u));
      const f16x2_t b = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, c, 0x04030402u));
      o[2 * i] = pack_bf16x2(__builtin_fmaf(static_cast<float>(a.x), df, off), __builtin_fmaf(static_cast<float>(a.y), df, off));
      o[2 * i + 1] = pack_bf16x2(__builtin_fmaf(static_cast<float>(b.x), df, off), __builtin_fmaf(static_cast<float>(b.y), df, off));
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
  }
};

// Q6_K: a 128-wide step is half h of super-block sb; piece g = elements
// 128 h + 32 g + l, l < 32 (ql[64 h + 32 (g & 1) + l] nibble g / 2, qh[32 h
// + l] bits 2g, sub-scale sc[8 h + l / 16 + 2 g]); MFMA s takes l = 8s .. 8s+7.
template <>
struct MoePiece<SPIRAL_TYPE_Q6_K> {
  uint4 l0, l1, h0, h1;
  uint32_t ds2;  // fp16 d (bits 0..15), sc for l < 16 (16..23), sc for l >= 16 (24..31)
  uint32_t sch;  // or-ed into ds2 bits 16..31 by prep (the streaming form loads it apart)
  int ls, hs;
  float m0, off0, m1, off1;  // d * sc and -1056 d * sc for l < 16 and l >= 16 (prep)
  __device__ __forceinline__ void prep() {
    ds2 |= sch << 16;
    const float d = fp16_scale(ds2 & 0xffffu);
    m0 = d * static_cast<float>(static_cast<int8_t>(ds2 >> 16));
    m1 = d * static_cast<float>(static_cast<int8_t>(ds2 >> 24));
    off0 = -1056.0f * m0;  // exact: d * sc has at most 18 significant bits, 33 has 6
    off1 = -1056.0f * m1;
  }
  static __device__ __forceinline__ int local(int g, int s, int e) { return 32 * g + 8 * s + e; }
  // sb_row = super-block index (row * nb + sb), h = half, g = group
  __device__ __forceinline__ void load(const uint8_t* we, int64_t tot, int64_t sbi, int h, int g) {
    const uint8_t* ql = we + sbi * 128 + 64 * h + 32 * (g & 1);
    const uint8_t* qh = we + tot * 128 + sbi * 64 + 32 * h;
    l0 = *reinterpret_cast<const uint4*>(ql);
    l1 = *reinterpret_cast<const uint4*>(ql + 16);
    h0 = *reinterpret_cast<const uint4*>(qh);
    h1 = *reinterpret_cast<const uint4*>(qh + 16);
    const uint32_t sc = *reinterpret_cast<const uint16_t*>(we + tot * 192 + sbi * 16 + 8 * h + 2 * g);
    ds2 = *reinterpret_cast<const uint16_t*>(we + tot * 208 + sbi * 2) | (sc << 16);
    sch = 0u;
    ls = (g >> 1) * 4;
    hs = 2 * g;
  }
  __device__ __forceinline__ void zero() { l0 = l1 = h0 = h1 = make_uint4(0u, 0u, 0u, 0u); ds2 = sch = 0u; ls = hs = 0; }
  __device__ __forceinline__ uint4 dequant(int s) const {
    const uint4 L = s < 2 ? l0 : l1, H = s < 2 ? h0 : h1;
    const uint32_t wl0 = (s & 1) ? L.z : L.x, wl1 = (s & 1) ? L.w : L.y;
    const uint32_t wh0 = (s & 1) ? H.z : H.x, wh1 = (s & 1) ? H.w : H.y;
    const float ds = s < 2 ? m0 : m1;
    const float off = s < 2 ? off0 : off1;
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      // 6-bit codes q as fp16 pairs 1024 + q: (1024 + q) ds - 1056 ds rounds
      // (q - 32) ds once, as the single-rounded FMA of the code does.
      const uint32_t c = (((i ? wl1 : wl0) >> ls) & 0x0F0F0F0Fu) | ((((i ? wh1 : wh0) >> hs) & 0x03030303u) << 4);
      const f16x2_t a = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, c, 0x04010400u));
      const f16x2_t b = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, c, 0x04030402u));
      o[2 * i] = pack_bf16x2(__builtin_fmaf(static_cast<float>(a.x), ds, off), __builtin_fmaf(static_cast<float>(a.y), ds, off));
      o[2 * i + 1] =
          pack_bf16x2(__builtin_fmaf(static_cast<float>(b.x), ds, off), __builtin_fmaf(static_cast<float>(b.y), ds, off));
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
  }
};

// Q4_K / Q5_K: a 128-wide step is half h of super-block sb; piece g = qs
// bytes 64 h + 32 (g / 2) + 16 (g % 2) .. + 15 of the super-block (chunk
// c = 2 h + g / 2), both nibbles: MFMA s < 2 takes the low nibbles of bytes
// 8 s .. 8 s + 7 (group 2 c), s >= 2 the high nibbles of bytes 8 (s - 2) ..
// (group 2 c + 1); Q5_K adds bits 2 c / 2 c + 1 of the same positions of
// qh[16 (g % 2) .. + 15]. The piece carries the super-block's meta entry.
template <int TYPE>
struct MoePieceKQ {
  uint4 q, meta, qh;
  int grp;                   // 2 c
  float d0, m0, d1, m1;      // d * scale * 2^24 and -dmin * min of groups 2 c and 2 c + 1 (prep)
  static __device__ __forceinline__ int local(int g, int s, int e) {
    return 64 * (g >> 1) + (s < 2 ? 16 * (g & 1) + 8 * s : 32 + 16 * (g & 1) + 8 * (s - 2)) + e;
  }
  __device__ __forceinline__ void prep() {
    const uint32_t sm = kq_chunk_scales(meta.y, meta.z, meta.w, static_cast<uint32_t>(grp) >> 1);
    const float d = fp16_ieee(meta.x & 0xffffu), dm = fp16_ieee(meta.x >> 16);
    d0 = d * 16777216.0f * static_cast<float>(sm & 0xffu);
    m0 = -(dm * static_cast<float>((sm >> 8) & 0xffu));
    d1 = d * 16777216.0f * static_cast<float>((sm >> 16) & 0xffu);
    m1 = -(dm * static_cast<float>(sm >> 24));
  }
  __device__ __forceinline__ void zero() { q = meta = qh = make_uint4(0u, 0u, 0u, 0u); grp = 0; }
  __device__ __forceinline__ uint4 dequant(int s) const {
    const bool hi = s >= 2;
    const uint32_t w0 = (s & 1) ? q.z : q.x, w1 = (s & 1) ? q.w : q.y;
    const uint32_t h0 = (s & 1) ? qh.z : qh.x, h1 = (s & 1) ? qh.w : qh.y;
    const float ds = hi ? d1 : d0, off = hi ? m1 : m0;
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      uint32_t c = ((i ? w1 : w0) >> (hi ? 4 : 0)) & 0x0F0F0F0Fu;
      if constexpr (TYPE == SPIRAL_TYPE_Q5_K) c |= (((i ? h1 : h0) >> (grp + (hi ? 1 : 0))) & 0x01010101u) << 4;
      // Codes q as subnormal fp16 pairs q 2^-24 against d * scale * 2^24: the
      // product is exact and the FMA with -dmin * min rounds once.
      const f16x2_t a = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0u, c, 0x04010400u));
      const f16x2_t b = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0u, c, 0x04030402u));
      o[2 * i] = pack_bf16x2(__builtin_fmaf(static_cast<float>(a.x), ds, off), __builtin_fmaf(static_cast<float>(a.y), ds, off));
      o[2 * i + 1] =
          pack_bf16x2(__builtin_fmaf(static_cast<float>(b.x), ds, off), __builtin_fmaf(static_cast<float>(b.y), ds, off));
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
  }
};
template <>
struct MoePiece<SPIRAL_TYPE_Q4_K> : MoePieceKQ<SPIRAL_TYPE_Q4_K> {};
template <>
struct MoePiece<SPIRAL_TYPE_Q5_K> : MoePieceKQ<SPIRAL_TYPE_Q5_K> {};

// IQ4_NL / IQ4_XS: piece g = 32 elements with one scale (IQ4_NL block 4 kb + g;
// IQ4_XS sub-block 4 h + g of the step's super-block half h), 16 qs bytes:
// MFMA s takes qs dword s, low nibbles (elements 4s .. 4s + 3) then high
// nibbles (16 + 4s ..), as Q4_0; indices become codebook values (iq4_lut).
template <int TYPE>
struct MoePieceIQ4 {
  uint4 q;
  uint2 meta;  // IQ4_NL: fp16 d in meta.x; IQ4_XS: d, scales_h, scales_l
  int sub;     // IQ4_XS sub-block
  float m, off;
  static __device__ __forceinline__ int local(int g, int s, int e) { return 32 * g + (e < 4 ? 4 * s + e : 12 + 4 * s + e); }
  __device__ __forceinline__ void prep() {
    m = TYPE == SPIRAL_TYPE_IQ4_XS ? iq4xs_scale(meta, sub) : fp16_ieee(meta.x & 0xffffu);
    off = -1152.0f * m;
  }
  __device__ __forceinline__ void zero() { q = make_uint4(0u, 0u, 0u, 0u); meta = make_uint2(0u, 0u); sub = 0; }
  __device__ __forceinline__ uint4 dequant(int s) const {
    const uint32_t w = s == 0 ? q.x : s == 1 ? q.y : s == 2 ? q.z : q.w;
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t c = iq4_lut((i ? (w >> 4) : w) & 0x0F0F0F0Fu);
      const f16x2_t a = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, c, 0x04010400u));
      const f16x2_t b = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, c, 0x04030402u));
      o[2 * i] = pack_bf16x2(__builtin_fmaf(static_cast<float>(a.x), m, off), __builtin_fmaf(static_cast<float>(a.y), m, off));
      o[2 * i + 1] = pack_bf16x2(__builtin_fmaf(static_cast<float>(b.x), m, off), __builtin_fmaf(static_cast<float>(b.y), m, off));
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
  }
};
template <>
struct MoePiece<SPIRAL_TYPE_IQ4_NL> : MoePieceIQ4<SPIRAL_TYPE_IQ4_NL> {};
template <>
struct MoePiece<SPIRAL_TYPE_IQ4_XS> : MoePieceIQ4<SPIRAL_TYPE_IQ4_XS> {};

// A lane's piece offsets for one weight row (lane group g), and the buffer
// loads of k step st into a MoePiece.
template <int TYPE>
struct PieceAddr;

template <>
struct PieceAddr<SPIRAL_TYPE_Q4_0> {
  uint32_t q, d;
  __device__ __forceinline__ void set(int64_t row, int64_t nb, int g) {
    q = static_cast<uint32_t>((row * nb + g) * 16);
    d = static_cast<uint32_t>((row * nb + g) * 2);
  }
  __device__ __forceinline__ void load(MoePiece<SPIRAL_TYPE_Q4_0>& pc, const Planes& P, int64_t st) const {
    pc.q = bload16(P.a, q, static_cast<uint32_t>(st) * 64u);
    pc.d = bload2(P.d, d, static_cast<uint32_t>(st) * 8u);
  }
};

template <>
struct PieceAddr<SPIRAL_TYPE_Q8_0> {
  uint32_t q, d;
  __device__ __forceinline__ void set(int64_t row, int64_t nb, int g) {
    q = static_cast<uint32_t>((row * nb + g) * 32);
    d = static_cast<uint32_t>((row * nb + g) * 2);
  }
  __device__ __forceinline__ void load(MoePiece<SPIRAL_TYPE_Q8_0>& pc, const Planes& P, int64_t st) const {
    pc.q0 = bload16(P.a, q, static_cast<uint32_t>(st) * 128u);
    pc.q1 = bload16(P.a, q + 16u, static_cast<uint32_t>(st) * 128u);
    pc.d = bload2(P.d, d, static_cast<uint32_t>(st) * 8u);
  }
};

template <>
struct PieceAddr<SPIRAL_TYPE_Q6_K> {
  uint32_t l, h, sc, d;
  int g;
  __device__ __forceinline__ void set(int64_t row, int64_t nb, int g_) {
    g = g_;
    l = static_cast<uint32_t>(row * nb * 128 + 32 * (g & 1));
    h = static_cast<uint32_t>(row * nb * 64);
    sc = static_cast<uint32_t>(row * nb * 16 + 2 * g);
    d = static_cast<uint32_t>(row * nb * 2);
  }
  // Step st is half st % 2 of super-block st / 2.
  __device__ __forceinline__ void load(MoePiece<SPIRAL_TYPE_Q6_K>& pc, const Planes& P, int64_t st) const {
    const uint32_t sb = static_cast<uint32_t>(st >> 1), hh = static_cast<uint32_t>(st & 1);
    pc.l0 = bload16(P.a, l, sb * 128u + 64u * hh);
    pc.l1 = bload16(P.a, l + 16u, sb * 128u + 64u * hh);
    pc.h0 = bload16(P.b, h, sb * 64u + 32u * hh);
    pc.h1 = bload16(P.b, h + 16u, sb * 64u + 32u * hh);
    pc.sch = bload2(P.c, sc, sb * 16u + 8u * hh);
    pc.ds2 = bload2(P.d, d, sb * 2u);
    pc.ls = (g >> 1) * 4;
    pc.hs = 2 * g;
  }
};

template <int TYPE>
struct PieceAddrKQ {
  uint32_t q, qh, meta;
  int g;
  __device__ __forceinline__ void set(int64_t row, int64_t nb, int g_) {
    g = g_;
    q = static_cast<uint32_t>(row * nb * 128 + 32 * (g >> 1) + 16 * (g & 1));
    qh = static_cast<uint32_t>(row * nb * 32 + 16 * (g & 1));
    meta = static_cast<uint32_t>(row * nb * 16);
  }
  // Step st is half st % 2 of super-block st / 2.
  __device__ __forceinline__ void load(MoePiece<TYPE>& pc, const Planes& P, int64_t st) const {
    const uint32_t sb = static_cast<uint32_t>(st >> 1), hh = static_cast<uint32_t>(st & 1);
    pc.q = bload16(P.a, q, sb * 128u + 64u * hh);
    pc.meta = bload16(P.c, meta, sb * 16u);
    if constexpr (TYPE == SPIRAL_TYPE_Q5_K) pc.qh = bload16(P.b, qh, sb * 32u);
    pc.grp = 4 * static_cast<int>(hh) + 2 * (g >> 1);
  }
};
template <>
struct PieceAddr<SPIRAL_TYPE_Q4_K> : PieceAddrKQ<SPIRAL_TYPE_Q4_K> {};
template <>
struct PieceAddr<SPIRAL_TYPE_Q5_K> : PieceAddrKQ<SPIRAL_TYPE_Q5_K> {};

template <>
struct PieceAddr<SPIRAL_TYPE_IQ4_NL> {
  uint32_t q, d;
  __device__ __forceinline__ void set(int64_t row, int64_t nb, int g) {
    q = static_cast<uint32_t>((row * nb + g) * 16);
    d = static_cast<uint32_t>((row * nb + g) * 2);
  }
  __device__ __forceinline__ void load(MoePiece<SPIRAL_TYPE_IQ4_NL>& pc, const Planes& P, int64_t st) const {
    pc.q = bload16(P.a, q, static_cast<uint32_t>(st) * 64u);
    pc.meta = make_uint2(bload2(P.d, d, static_cast<uint32_t>(st) * 8u), 0u);
    pc.sub = 0;
  }
};

template <>
struct PieceAddr<SPIRAL_TYPE_IQ4_XS> {
  uint32_t q, meta;
  int g;
  __device__ __forceinline__ void set(int64_t row, int64_t nb, int g_) {
    g = g_;
    q = static_cast<uint32_t>(row * nb * 128 + 16 * g);
    meta = static_cast<uint32_t>(row * nb * 8);
  }
  // Step st is half st % 2 of super-block st / 2: sub-block 4 (st % 2) + g.
  __device__ __forceinline__ void load(MoePiece<SPIRAL_TYPE_IQ4_XS>& pc, const Planes& P, int64_t st) const {
    const uint32_t sb = static_cast<uint32_t>(st >> 1), hh = static_cast<uint32_t>(st & 1);
    pc.q = bload16(P.a, q, sb * 128u + 64u * hh);
    pc.meta = make_uint2(bload4(P.c, meta, sb * 8u), bload4(P.c, meta + 4u, sb * 8u));
    pc.sub = 4 * static_cast<int>(hh) + g;
  }
};

}  // namespace
}  // namespace spiral
