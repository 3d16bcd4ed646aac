/*
 * quants_oracle.c -- TEST INFRASTRUCTURE ONLY (see quants_oracle.h).
 *
 * Plain C restatement of the reference's quantized-weight semantics. Each
 * function cites the reference file:line it follows. Built by oracle/Makefile
 * into oracle/liboracle.so; never linked into the product library.
 */
#include "quants_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- scalar conversions ------------------------------------------------ */

static inline float f32_from_bits(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint32_t bits_from_f32(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

static inline uint16_t le16(const uint8_t* p) {
  /* src/quants/common/repack.h:19-22: canonical blocks are little-endian. */
  return (uint16_t)(p[0] | (p[1] << 8));
}

float oq_fp16_ieee(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t mant = h & 0x3ffu;
  if (exp == 0) {
    const float v = ldexpf((float)mant, -24);
    return sign ? -v : v;
  }
  if (exp == 31) {
    return f32_from_bits(sign | 0x7f800000u | (mant << 13));
  }
  return f32_from_bits(sign | ((exp + 112u) << 23) | (mant << 13));
}

float oq_fp16_device(uint16_t h) {
  /* src/quants/common/scale.aie.h:14-27: bits = sign | (exp+112)<<23 |
   * mant<<13, selected to all-zero bits when exp == 0. exp == 31 takes the
   * same formula, giving a finite 2^16 * (1.m). */
  const uint32_t exp = (h >> 10) & 0x1fu;
  if (exp == 0) return 0.0f;
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  return f32_from_bits(sign | ((exp + 112u) << 23) | ((uint32_t)(h & 0x3ffu) << 13));
}

uint16_t oq_bf16_rne(float f) {
  /* src/quants/q4_0_hilo/repack.h:32-38: add 0x7fff + lsb, keep the top half. */
  uint32_t u = bits_from_f32(f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float oq_bf16_f32(uint16_t b) { return f32_from_bits((uint32_t)b << 16); }

void oq_fp16_device_array(const uint16_t* h, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oq_fp16_device(h[i]);
}

void oq_bf16_rne_array(const float* f, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oq_bf16_rne(f[i]);
}

static inline float bf16_round_f(float f) { return oq_bf16_f32(oq_bf16_rne(f)); }

/* ---- the reference's device arithmetic, step by step -------------------- */

static inline void split_hi_lo(float d, float* hi, float* lo) {
  /* src/quants/common/scale.aie.h:31-39: hi = bf16(d); lo = bf16(d - hi). */
  *hi = bf16_round_f(d);
  *lo = bf16_round_f(d - *hi);
}

uint16_t oq_aie_q_times_d(int q, uint16_t d_bits) {
  float hi, lo;
  split_hi_lo(oq_fp16_device(d_bits), &hi, &lo);
  const float qf = (float)q; /* int4/int8 -> bf16 is exact */
  float acc = qf * hi;       /* aie::mul: bf16 x bf16 into fp32 */
  acc = acc + qf * lo;       /* aie::mac */
  return oq_bf16_rne(acc);   /* to_vector<bfloat16> under conv_even */
}

uint16_t oq_aie_q6_k(int q_centred, int sc, uint16_t d_bits) {
  float d_hi, d_lo;
  split_hi_lo(oq_fp16_device(d_bits), &d_hi, &d_lo); /* q6_k/unpack.aie.h:20-31 */
  const float s = (float)sc;
  float p = d_hi * s; /* q6_k/unpack.aie.h:44-46 */
  p = p + d_lo * s;
  const float hi = bf16_round_f(p); /* :48-60 three successive residuals */
  const float r1 = p - hi;
  const float mid = bf16_round_f(r1);
  const float r2 = r1 - mid;
  const float lo = bf16_round_f(r2);
  const float qf = (float)q_centred;
  float acc = qf * hi; /* apply_scales, q6_k/unpack.aie.h:81-91 */
  acc = acc + qf * mid;
  acc = acc + qf * lo;
  return oq_bf16_rne(acc);
}

static inline uint16_t closed_q_times_d(int q, uint16_t d_bits) {
  return oq_bf16_rne((float)q * oq_fp16_device(d_bits));
}

static inline uint16_t closed_q6_k(int q_centred, int sc, uint16_t d_bits) {
  /* d*sc is exact in fp32 (<= 18 significant bits), and so is the product
   * with q-32 (<= 23 bits), so a single rounding remains. */
  return oq_bf16_rne((oq_fp16_device(d_bits) * (float)sc) * (float)q_centred);
}

static int is_normal_fp16(uint32_t h) {
  const uint32_t e = (h >> 10) & 0x1f;
  return e != 0 && e != 31;
}

int64_t oq_check_q_times_d(int64_t* signed_zero) {
  int64_t bad = 0, sz = 0;
#pragma omp parallel for reduction(+ : bad, sz) schedule(static)
  for (int h = 0; h < 65536; ++h) {
    if (!is_normal_fp16((uint32_t)h)) continue;
    for (int q = -128; q <= 127; ++q) {
      const uint16_t a = oq_aie_q_times_d(q, (uint16_t)h);
      const uint16_t c = closed_q_times_d(q, (uint16_t)h);
      if (a != c) {
        if (((a | c) & 0x7fffu) == 0) sz++;
        else bad++;
      }
    }
  }
  if (signed_zero) *signed_zero = sz;
  return bad;
}

int64_t oq_check_q6_k(int d_step, int64_t* signed_zero) {
  int64_t bad = 0, sz = 0;
  if (d_step < 1) d_step = 1;
#pragma omp parallel for reduction(+ : bad, sz) schedule(dynamic, 64)
  for (int h = 0; h < 65536; h += d_step) {
    if (!is_normal_fp16((uint32_t)h)) continue;
    for (int sc = -128; sc <= 127; ++sc) {
      for (int q = -32; q <= 31; ++q) {
        const uint16_t a = oq_aie_q6_k(q, sc, (uint16_t)h);
        const uint16_t c = closed_q6_k(q, sc, (uint16_t)h);
        if (a != c) {
          if (((a | c) & 0x7fffu) == 0) sz++;
          else bad++;
        }
      }
    }
  }
  if (signed_zero) *signed_zero = sz;
  return bad;
}

int64_t oq_check_split_identity(void) {
  int64_t bad = 0;
  for (int h = 0; h < 65536; ++h) {
    if (!is_normal_fp16((uint32_t)h)) continue;
    const float d = oq_fp16_device((uint16_t)h);
    float hi, lo;
    split_hi_lo(d, &hi, &lo);
    if (hi + lo != d) bad++;
  }
  return bad;
}

/* ---- canonical GGUF dequantization -------------------------------------- */

int oq_block_bytes(int type) {
  switch (type) {
    case OQ_Q4_0: return 18;  /* src/quants/q4_0/layout.h:11-12 */
    case OQ_Q8_0: return 34;  /* src/quants/q8_0/layout.h:11-12 */
    case OQ_Q6_K: return 210; /* src/quants/q6_k/layout.h:11-12 */
    case OQ_Q4_K: return 144; /* d, dmin, scales[12], qs[128] */
    case OQ_Q5_K: return 176; /* d, dmin, scales[12], qh[32], qs[128] */
    case OQ_IQ4_NL: return 18; /* d, qs[16] */
    case OQ_IQ4_XS: return 136; /* d, scales_h, scales_l[4], qs[128] */
    default: return 0;
  }
}

int oq_block_elems(int type) {
  switch (type) {
    case OQ_Q4_0: return 32;
    case OQ_Q8_0: return 32;
    case OQ_Q6_K: return 256;
    case OQ_Q4_K: return 256;
    case OQ_Q5_K: return 256;
    case OQ_IQ4_NL: return 32;
    case OQ_IQ4_XS: return 256;
    default: return 0;
  }
}

/* Exact values of one block's weights. Every product below is exact in
 * float (Q4_0 <= 15, Q8_0 <= 19, Q6_K <= 23 significant bits), so rounding
 * these to bf16 is the format's single rounding. */
static void kq_dequant(int type, const uint8_t* blk, float* yf, double* yd);

static void iq4_dequant(int type, const uint8_t* blk, double* y);

static void dequant_block_exact(int type, const uint8_t* blk, double* y) {
  if (type == OQ_Q4_K || type == OQ_Q5_K) {
    kq_dequant(type, blk, NULL, y);
  } else if (type == OQ_IQ4_NL || type == OQ_IQ4_XS) {
    iq4_dequant(type, blk, y);
  } else if (type == OQ_Q4_0) {
    /* src/quants/tests/formats/q4_0.py:53-60: low nibbles are elements 0..15,
     * high nibbles 16..31, value (q - 8) * d. */
    const float d = oq_fp16_device(le16(blk));
    const uint8_t* qs = blk + 2;
    for (int j = 0; j < 16; ++j) {
      y[j] = (double)((qs[j] & 15) - 8) * d;
      y[j + 16] = (double)((qs[j] >> 4) - 8) * d;
    }
  } else if (type == OQ_Q8_0) {
    /* src/quants/tests/formats/q8_0.py:50-58: int8 code times d. */
    const float d = oq_fp16_device(le16(blk));
    const int8_t* qs = (const int8_t*)(blk + 2);
    for (int j = 0; j < 32; ++j) y[j] = (double)qs[j] * d;
  } else {
    /* src/quants/tests/formats/q6_k.py:55-97: ql[128] qh[64] sc[16] d. */
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    const int8_t* sc = (const int8_t*)(blk + 192);
    const float d = oq_fp16_device(le16(blk + 208));
    for (int h = 0; h < 2; ++h) {
      for (int l = 0; l < 32; ++l) {
        const int lo0 = ql[64 * h + l], lo1 = ql[64 * h + 32 + l];
        const int hb = qh[32 * h + l];
        const int q[4] = {
            (lo0 & 15) | (((hb >> 0) & 3) << 4),
            (lo1 & 15) | (((hb >> 2) & 3) << 4),
            (lo0 >> 4) | (((hb >> 4) & 3) << 4),
            (lo1 >> 4) | (((hb >> 6) & 3) << 4),
        };
        for (int j = 0; j < 4; ++j) {
          const double ds = (double)d * (double)sc[8 * h + l / 16 + 2 * j];
          y[128 * h + 32 * j + l] = ds * (double)(q[j] - 32);
        }
      }
    }
  }
}

/* ---- K-quants with 6-bit scales and mins (Q4_K, Q5_K) --------------------
 *
 * The reference plans these formats but has no code or vectors for them
 * (src/quants/TODO.md:16-17,80-107): 256-element super-blocks of eight
 * 32-element groups, fp16 d and dmin, a 6-bit scale and a 6-bit min per
 * group packed into 12 bytes, element value d * scale * q - dmin * min, and
 * Q5_K's extra high bit. The byte layout is ggml's block_q4_K / block_q5_K.
 *
 * The 12 scale bytes, field by field:
 *   bytes 0..3   bits 0..5: scale of groups 0..3; bits 6..7: bits 4..5 of
 *                the scale of groups 4..7
 *   bytes 4..7   bits 0..5: min of groups 0..3; bits 6..7: bits 4..5 of the
 *                min of groups 4..7
 *   bytes 8..11  bits 0..3: bits 0..3 of the scale of groups 4..7;
 *                bits 4..7: bits 0..3 of the min of groups 4..7
 * Group g (elements 32 g .. 32 g + 31) takes the low (g even) or high (g odd)
 * nibble of qs[32 (g / 2) + l], and for Q5_K bit g of qh[l] as bit 4 of its
 * code (l < 32).
 *
 * d and dmin decode as IEEE binary16 (subnormals keep their value), as
 * ggml's dequantization does: the reference's exponent-0 flush
 * (src/quants/common/repack.h:29-34) belongs to its NPU scale loader for the
 * formats it implements, and a K-quant's dmin is often subnormal in real
 * files. d * scale and dmin * min are exact in float; the element is
 * fmaf(d * scale, q, -dmin * min), one rounding to float, then bf16 RNE. */
static void kq_scale_min(const uint8_t* s, int g, int* sc, int* mn) {
  if (g < 4) {
    *sc = s[g] & 63;
    *mn = s[4 + g] & 63;
  } else {
    const int i = g - 4;
    *sc = (s[8 + i] & 15) | ((s[i] >> 6) << 4);
    *mn = (s[8 + i] >> 4) | ((s[4 + i] >> 6) << 4);
  }
}

/* Codes (0..15 or 0..31) of the 256 elements of a K-quant super-block. */
static void kq_codes(int type, const uint8_t* blk, int* q) {
  const uint8_t* qs = blk + (type == OQ_Q5_K ? 48 : 16);
  const uint8_t* qh = blk + 16;
  for (int g = 0; g < 8; ++g) {
    for (int l = 0; l < 32; ++l) {
      const uint8_t b = qs[32 * (g / 2) + l];
      int c = (g & 1) ? (b >> 4) : (b & 15);
      if (type == OQ_Q5_K) c |= ((qh[l] >> g) & 1) << 4;
      q[32 * g + l] = c;
    }
  }
}

static void kq_dequant(int type, const uint8_t* blk, float* yf, double* yd) {
  const float d = oq_fp16_ieee(le16(blk)), dmin = oq_fp16_ieee(le16(blk + 2));
  int q[256];
  kq_codes(type, blk, q);
  for (int g = 0; g < 8; ++g) {
    int sc, mn;
    kq_scale_min(blk + 4, g, &sc, &mn);
    const float d1 = d * (float)sc, m1 = dmin * (float)mn;
    for (int l = 0; l < 32; ++l) {
      const int e = 32 * g + l;
      if (yf) yf[e] = fmaf(d1, (float)q[e], -m1);
      if (yd) yd[e] = (double)d1 * (double)q[e] - (double)m1;
    }
  }
}

static int is_kquant(int type) { return type == OQ_Q4_K || type == OQ_Q5_K; }

/* ---- IQ4_NL / IQ4_XS: 4-bit indices into a 16-entry codebook -----------
 *
 * The reference plans both (src/quants/TODO.md:109-124) with ggml's
 * kvalues_iq4nl codebook and no code or vectors. Layout (ggml block_iq4_nl,
 * block_iq4_xs): IQ4_NL {fp16 d, qs[16]} per 32 elements, element j the low
 * (j < 16) or high nibble of qs[j % 16], value d * kv[index]; IQ4_XS {fp16 d,
 * scales_h, scales_l[4], qs[128]} per 256: eight sub-blocks of 32 laid out as
 * IQ4_NL blocks, sub-block b scaled by d * (ls - 32) with the 6-bit
 * ls = (nibble b % 2 of scales_l[b / 2]) | (bits 2b..2b+1 of scales_h) << 4.
 * d decodes as IEEE binary16, as for the K-quants. Every product is exact in
 * float (d * (ls - 32) has at most 17 significant bits, kv at most 7), so
 * the element is bf16_rne(exact product). */
static const int8_t kIq4Values[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

static void iq4_dequant(int type, const uint8_t* blk, double* y) {
  const float d = oq_fp16_ieee(le16(blk));
  const int nsub = type == OQ_IQ4_XS ? 8 : 1;
  const uint8_t* qs = blk + (type == OQ_IQ4_XS ? 8 : 2);
  for (int b = 0; b < nsub; ++b) {
    float dl = d;
    if (type == OQ_IQ4_XS) {
      const int sh = le16(blk + 2);
      const int ls = ((blk[4 + b / 2] >> (4 * (b % 2))) & 15) | (((sh >> (2 * b)) & 3) << 4);
      dl = d * (float)(ls - 32);
    }
    for (int j = 0; j < 16; ++j) {
      y[32 * b + j] = (double)dl * kIq4Values[qs[16 * b + j] & 15];
      y[32 * b + 16 + j] = (double)dl * kIq4Values[qs[16 * b + j] >> 4];
    }
  }
}

static void dequant_block(int type, const uint8_t* blk, uint16_t* y) {
  if (is_kquant(type)) {
    float v[256];
    kq_dequant(type, blk, v, NULL);
    for (int j = 0; j < 256; ++j) y[j] = oq_bf16_rne(v[j]);
    return;
  }
  double v[256];
  dequant_block_exact(type, blk, v);
  const int be = oq_block_elems(type);
  for (int j = 0; j < be; ++j) y[j] = oq_bf16_rne((float)v[j]);
}

static int shape_ok(int type, int64_t n_rows, int64_t k) {
  const int be = oq_block_elems(type);
  return be > 0 && n_rows >= 0 && k > 0 && k % be == 0;
}

int oq_dequant(int type, const uint8_t* src, int64_t row_stride,
               int64_t n_rows, int64_t k, uint16_t* out, int64_t ld_out) {
  if (!shape_ok(type, n_rows, k)) return -1;
  const int be = oq_block_elems(type), bb = oq_block_bytes(type);
  const int64_t nb = k / be;
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < n_rows; ++n) {
    for (int64_t b = 0; b < nb; ++b) {
      dequant_block(type, src + n * row_stride + b * bb, out + n * ld_out + b * be);
    }
  }
  return 0;
}

int oq_dequant_f64(int type, const uint8_t* src, int64_t row_stride,
                   int64_t n_rows, int64_t k, double* out, int64_t ld_out) {
  if (!shape_ok(type, n_rows, k)) return -1;
  const int be = oq_block_elems(type), bb = oq_block_bytes(type);
  const int64_t nb = k / be;
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < n_rows; ++n) {
    for (int64_t b = 0; b < nb; ++b) {
      dequant_block_exact(type, src + n * row_stride + b * bb, out + n * ld_out + b * be);
    }
  }
  return 0;
}

void oq_matmul_f64_exact(const double* w, int64_t ldw, int64_t n_rows, int64_t k,
                         const uint16_t* x, int64_t ldx, int64_t m, double* y,
                         int64_t ldy) {
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < n_rows; ++n) {
    for (int64_t i = 0; i < m; ++i) {
      double acc = 0.0;
      for (int64_t kk = 0; kk < k; ++kk) acc += w[n * ldw + kk] * (double)oq_bf16_f32(x[i * ldx + kk]);
      y[i * ldy + n] = acc;
    }
  }
}

int oq_get_rows(int type, const uint8_t* src, int64_t row_stride,
                int64_t n_rows, int64_t k, const int32_t* ids, int64_t n_ids,
                uint16_t* out, int64_t ld_out) {
  if (!shape_ok(type, n_rows, k)) return -1;
  for (int64_t i = 0; i < n_ids; ++i) {
    if (ids[i] < 0 || ids[i] >= n_rows) return -1;
  }
  const int be = oq_block_elems(type), bb = oq_block_bytes(type);
  const int64_t nb = k / be;
  for (int64_t i = 0; i < n_ids; ++i) {
    for (int64_t b = 0; b < nb; ++b) {
      dequant_block(type, src + (int64_t)ids[i] * row_stride + b * bb,
                    out + i * ld_out + b * be);
    }
  }
  return 0;
}

/* ---- the reference's NPU record layout ---------------------------------- */

/* Record geometry per format: rows per record, bytes per record
 * (q4_0/layout.h:31-38, q8_0/layout.h:23-35, q6_k/layout.h:23-42). */
static int ref_record_rows(int type) {
  return type == OQ_Q4_0 ? 64 : (type == OQ_Q8_0 || type == OQ_Q6_K) ? 256 : 0;
}
static int ref_record_bytes(int type) {
  return type == OQ_Q4_0 ? 288 : type == OQ_Q8_0 ? 2176 : type == OQ_Q6_K ? 1680 : 0;
}

int64_t oq_ref_record_count(int type, int64_t weights_rows, int64_t weights_cols) {
  /* src/quants/q4_0/repack.h:10-18 (same rule in q8_0 and q6_k). */
  const int rr = ref_record_rows(type);
  if (rr == 0 || weights_rows <= 0 || weights_cols <= 0) return 0;
  if (weights_rows % rr != 0 || weights_cols % 8 != 0) return 0;
  /* Shapes whose record stream overflows an int64 byte count are refused
   * (the reference's product is unchecked there). */
  int64_t records, bytes;
  if (__builtin_mul_overflow(weights_rows / rr, weights_cols / 8, &records) ||
      __builtin_mul_overflow(records, (int64_t)ref_record_bytes(type), &bytes))
    return 0;
  return records;
}

int64_t oq_ref_packed_bytes(int type, int64_t weights_rows, int64_t weights_cols) {
  return oq_ref_record_count(type, weights_rows, weights_cols) * ref_record_bytes(type);
}

static int fp16_is_subnormal(uint16_t h) {
  /* src/quants/common/repack.h:29-34 */
  return (h & 0x7c00u) == 0 && (h & 0x03ffu) != 0;
}

static uint16_t flushed_scale(const uint8_t* p, int* warnings) {
  uint16_t bits = le16(p);
  if (fp16_is_subnormal(bits)) {
    bits = 0; /* q4_0/repack.h:75-80: stored as +0 */
    *warnings |= 1;
  }
  return bits;
}

static void put16(uint8_t* p, uint16_t v) {
  p[0] = (uint8_t)(v & 0xff);
  p[1] = (uint8_t)(v >> 8);
}

int64_t oq_ref_repack(int type, const uint8_t* src, int64_t src_col_stride_bytes,
                      uint8_t* dst, int64_t dst_capacity, int64_t weights_rows,
                      int64_t weights_cols, int* warnings) {
  int warn = 0;
  const int64_t records = oq_ref_record_count(type, weights_rows, weights_cols);
  const int64_t bytes = records * ref_record_bytes(type);
  if (warnings) *warnings = 0;
  /* q4_0/repack.h:33-41: validation, 0 on any failure. */
  if (records == 0 || bytes > dst_capacity || src == NULL || dst == NULL) return 0;
  const int be = oq_block_elems(type), bb = oq_block_bytes(type);
  if (src_col_stride_bytes < (weights_rows / be) * bb) return 0;

  const int64_t col_tiles = weights_cols / 8;
  const int rr = ref_record_rows(type), rb = ref_record_bytes(type);
  const int64_t row_records = weights_rows / rr;

  for (int64_t t = 0; t < col_tiles; ++t) {
    for (int64_t r = 0; r < row_records; ++r) {
      uint8_t* rec = dst + (t * row_records + r) * rb;
      if (type == OQ_Q4_0) {
        /* q4_0/repack.h:48-107: [16 fp16 scales][2 blocks x 128 B payload];
         * payload byte p*16 + row*4 + col/2, low nibble = even column, value
         * (q - 8) & 15. */
        memset(rec + 32, 0, 256);
        for (int blk = 0; blk < 2; ++blk) {
          for (int c = 0; c < 8; ++c) {
            const uint8_t* b = src + (t * 8 + c) * src_col_stride_bytes + (r * 2 + blk) * 18;
            put16(rec + blk * 16 + c * 2, flushed_scale(b, &warn));
            for (int row = 0; row < 32; ++row) {
              const int q = row < 16 ? (b[2 + row] & 15) : (b[2 + row - 16] >> 4);
              const uint8_t s = (uint8_t)((q - 8) & 15);
              uint8_t* byte = rec + 32 + blk * 128 + row * 4 + c / 2;
              *byte |= (uint8_t)((c & 1) ? (s << 4) : s);
            }
          }
        }
      } else if (type == OQ_Q8_0) {
        /* q8_0/repack.h:53-83: 8 blocks x 4 tiles x (8 rows x 8 cols int8),
         * then 8 blocks x 8 fp16 scales at byte 2048. */
        for (int blk = 0; blk < 8; ++blk) {
          for (int c = 0; c < 8; ++c) {
            const uint8_t* b = src + (t * 8 + c) * src_col_stride_bytes + (r * 8 + blk) * 34;
            put16(rec + 2048 + blk * 16 + c * 2, flushed_scale(b, &warn));
            for (int row = 0; row < 32; ++row) {
              if (b[2 + row] == 0x80u) warn |= 2;
              rec[blk * 256 + row * 8 + c] = b[2 + row];
            }
          }
        }
      } else {
        /* q6_k/repack.h:46-108: chunk c = 2*half + pair holds 64 rows; low
         * nibble plane (row*8+col, 4 bits) then 2-bit high plane; per-chunk
         * sub-scales [subgroup][col] at 1536 + 32*chunk; fp16 d at 1664. */
        memset(rec, 0, 1536);
        for (int c = 0; c < 8; ++c) {
          const uint8_t* b = src + (t * 8 + c) * src_col_stride_bytes + r * 210;
          put16(rec + 1664 + c * 2, flushed_scale(b + 208, &warn));
        }
        for (int ch = 0; ch < 4; ++ch) {
          const int half = ch / 2, pair = ch % 2;
          uint8_t* low = rec + ch * 384;
          uint8_t* high = low + 256;
          for (int c = 0; c < 8; ++c) {
            const uint8_t* b = src + (t * 8 + c) * src_col_stride_bytes + r * 210;
            for (int s = 0; s < 4; ++s) {
              rec[1536 + ch * 32 + s * 8 + c] = b[192 + half * 8 + pair * 4 + s];
            }
            for (int row = 0; row < 64; ++row) {
              const int group = row / 32, l = row % 32;
              const uint8_t qlb = b[half * 64 + group * 32 + l];
              const int nib = pair == 0 ? (qlb & 15) : (qlb >> 4);
              const int hb = (b[128 + half * 32 + l] >> (4 * pair + 2 * group)) & 3;
              const int v = nib | (hb << 4);
              const int idx = row * 8 + c;
              low[idx / 2] |= (uint8_t)((v & 15) << (4 * (idx % 2)));
              high[idx / 4] |= (uint8_t)(((v >> 4) & 3) << (2 * (idx % 4)));
            }
          }
        }
      }
    }
  }
  if (warnings) *warnings = warn;
  return bytes;
}

int oq_ref_unpack(int type, const uint8_t* packed, int64_t weights_rows,
                  int64_t weights_cols, uint16_t* out) {
  const int64_t records = oq_ref_record_count(type, weights_rows, weights_cols);
  if (records == 0) return -1;
  const int rr = ref_record_rows(type), rb = ref_record_bytes(type);
  /* unpack.aie.cc:29-43 walks records in storage order and writes one
   * [rows][8] tile block per chunk, so the output for record i starts at
   * i * rr * 8. */
  for (int64_t i = 0; i < records; ++i) {
    const uint8_t* rec = packed + i * rb;
    uint16_t* o = out + i * (int64_t)rr * 8;
    for (int row = 0; row < rr; ++row) {
      for (int c = 0; c < 8; ++c) {
        uint16_t v;
        if (type == OQ_Q4_0) {
          /* q4_0/unpack.aie.h:16-46: int4 cast of the tile byte, scale of
           * block row/32 and column c. */
          const int blk = row / 32, br = row % 32;
          const uint8_t byte = rec[32 + blk * 128 + br * 4 + c / 2];
          int q = (c & 1) ? (byte >> 4) : (byte & 15);
          if (q >= 8) q -= 16;
          v = oq_aie_q_times_d(q, le16(rec + blk * 16 + c * 2));
        } else if (type == OQ_Q8_0) {
          /* q8_0/unpack.aie.h:18-80 */
          const int blk = row / 32, br = row % 32;
          const int q = (int8_t)rec[blk * 256 + br * 8 + c];
          v = oq_aie_q_times_d(q, le16(rec + 2048 + blk * 16 + c * 2));
        } else {
          /* q6_k/unpack.aie.h:96-178: planes -> (q + 0xE0) as int8 = q - 32,
           * sub-scale [row/16][c] of the chunk, d of column c. */
          const int ch = row / 64, cr = row % 64;
          const uint8_t* low = rec + ch * 384;
          const uint8_t* high = low + 256;
          const int idx = cr * 8 + c;
          const int q = ((low[idx / 2] >> (4 * (idx % 2))) & 15) |
                        (((high[idx / 4] >> (2 * (idx % 4))) & 3) << 4);
          const int sc = (int8_t)rec[1536 + ch * 32 + (cr / 16) * 8 + c];
          v = oq_aie_q6_k(q - 32, sc, le16(rec + 1664 + c * 2));
        }
        o[row * 8 + c] = v;
      }
    }
  }
  return 0;
}

/* ---- matmul ------------------------------------------------------------- */

void oq_matmul_f64(const uint16_t* w, int64_t ldw, int64_t n_rows, int64_t k,
                   const uint16_t* x, int64_t ldx, int64_t m, double* y,
                   int64_t ldy) {
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < n_rows; ++n) {
    for (int64_t i = 0; i < m; ++i) {
      double acc = 0.0;
      for (int64_t kk = 0; kk < k; ++kk) {
        acc += (double)oq_bf16_f32(x[i * ldx + kk]) * (double)oq_bf16_f32(w[n * ldw + kk]);
      }
      y[i * ldy + n] = acc;
    }
  }
}

void oq_matmul_f32(const uint16_t* w, int64_t ldw, int64_t n_rows, int64_t k,
                   const uint16_t* x, int64_t ldx, int64_t m, float* y,
                   int64_t ldy) {
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < n_rows; ++n) {
    for (int64_t i = 0; i < m; ++i) {
      float acc = 0.0f;
      for (int64_t kk = 0; kk < k; ++kk) {
        acc += oq_bf16_f32(x[i * ldx + kk]) * oq_bf16_f32(w[n * ldw + kk]);
      }
      y[i * ldy + n] = acc;
    }
  }
}

int oq_quant_matmul_f32(int type, const uint8_t* src, int64_t row_stride,
                        int64_t n_rows, int64_t k, const uint16_t* x,
                        int64_t ldx, int64_t m, float* y, int64_t ldy,
                        int threads) {
  if (!shape_ok(type, n_rows, k)) return -1;
  const int be = oq_block_elems(type), bb = oq_block_bytes(type);
  const int64_t nb = k / be;
  float* xf = (float*)malloc(sizeof(float) * (size_t)(m * k));
  if (!xf) return -1;
  for (int64_t i = 0; i < m; ++i)
    for (int64_t kk = 0; kk < k; ++kk) xf[i * k + kk] = oq_bf16_f32(x[i * ldx + kk]);
#ifdef _OPENMP
  if (threads < 1) threads = 1;
#pragma omp parallel num_threads(threads)
#endif
  {
    uint16_t* row = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)k);
#pragma omp for schedule(static)
    for (int64_t n = 0; n < n_rows; ++n) {
      for (int64_t b = 0; b < nb; ++b) dequant_block(type, src + n * row_stride + b * bb, row + b * be);
      for (int64_t i = 0; i < m; ++i) {
        float acc = 0.0f;
        const float* xr = xf + i * k;
        for (int64_t kk = 0; kk < k; ++kk) acc += xr[kk] * oq_bf16_f32(row[kk]);
        y[i * ldy + n] = acc;
      }
    }
    free(row);
  }
  free(xf);
  return 0;
}
