/*
 * cpu_baseline.c -- TEST INFRASTRUCTURE ONLY: the CPU baseline bench.py
 * times beside the GPU (its "cpu_baseline" legs). Nothing in spiral_amd/
 * links, loads or calls it.
 *
 * It restates the reference's CPU path for this hot path as a multi-core,
 * vectorized C program: weights are dequantized to bf16 exactly as
 * src/quants/tests/formats/q4_0.py:47-60, q8_0.py:48-58 and q6_k.py:55-129
 * do (element bf16_rne(code * d), bf16_rne(d * sc * (q - 32)) for Q6_K, d
 * decoded with the reference's device rule), and
 * products accumulate bf16 weights times bf16 activations in fp32, as
 * src/quants/tests/mmul.py:104-112 does. Results equal the oracle's
 * (oracle/quants_oracle.c) up to fp32 summation order; tests/test_oracle.py
 * holds them to it.
 *
 * Hot loops carry GCC target clones (AVX-512, AVX2, baseline x86-64), picked
 * once at load time from the host CPU, so one build runs on any x86-64 host.
 * OpenMP spreads rows over `threads` threads.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define CB_CLONES __attribute__((target_clones("avx512f", "avx2", "default")))

static inline float cb_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static inline uint32_t cb_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* The reference's device scale rule (src/quants/common/scale.aie.h:14-27):
 * exponent 0 -> +0, exponent 31 -> finite 2^16 * (1.m), else IEEE. */
static inline float cb_scale(uint16_t h) {
  const uint32_t e = h & 0x7c00u;
  const uint32_t bits = ((uint32_t)(h & 0x8000u) << 16) | ((((uint32_t)h & 0x7fffu) << 13) + 0x38000000u);
  return cb_f32(e ? bits : 0u);
}

/* float -> bf16 bits, round to nearest even (finite inputs), and back. */
static inline uint32_t cb_bf16_bits(float f) {
  const uint32_t u = cb_bits(f);
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}
static inline float cb_bf16_round(float f) { return cb_f32(cb_bf16_bits(f) << 16); }

static inline uint16_t cb_le16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* A row of Q4_0 blocks -> k bf16-rounded weights as float. */
CB_CLONES static void cb_q4_0_row(const uint8_t* row, int64_t nb, float* w) {
  for (int64_t b = 0; b < nb; ++b) {
    const uint8_t* blk = row + 18 * b;
    const float d = cb_scale(cb_le16(blk));
    const uint8_t* qs = blk + 2;
    float* o = w + 32 * b;
#pragma omp simd
    for (int j = 0; j < 16; ++j) {
      o[j] = cb_bf16_round((float)((qs[j] & 15) - 8) * d);
      o[j + 16] = cb_bf16_round((float)((qs[j] >> 4) - 8) * d);
    }
  }
}

/* sum over a row of Q8_0 blocks of bf16_rne(q d) x, fp32. */
CB_CLONES static float cb_q8_0_row_dot(const uint8_t* row, int64_t nb, const float* x) {
  float acc = 0.0f;
  for (int64_t b = 0; b < nb; ++b) {
    const uint8_t* blk = row + 34 * b;
    const float d = cb_scale(cb_le16(blk));
    const int8_t* qs = (const int8_t*)(blk + 2);
    const float* xb = x + 32 * b;
    float a = 0.0f;
#pragma omp simd reduction(+ : a)
    for (int j = 0; j < 32; ++j) a += cb_bf16_round((float)qs[j] * d) * xb[j];
    acc += a;
  }
  return acc;
}

static float* cb_x_f32(const uint16_t* x, int64_t n) {
  float* xf = (float*)malloc(sizeof(float) * (size_t)n);
  if (xf)
    for (int64_t i = 0; i < n; ++i) xf[i] = cb_f32((uint32_t)x[i] << 16);
  return xf;
}

/* y[n] = sum_k W[n][k] x[k], W canonical Q8_0 rows of k/32 blocks. */
int cb_gemv_q8_0(const uint8_t* raw, int64_t n_rows, int64_t k, const uint16_t* x, float* y, int threads) {
  if (k % 32 != 0 || n_rows < 0) return -1;
  float* xf = cb_x_f32(x, k);
  if (!xf) return -1;
  const int64_t nb = k / 32;
#pragma omp parallel for schedule(static) num_threads(threads)
  for (int64_t r = 0; r < n_rows; ++r) y[r] = cb_q8_0_row_dot(raw + r * nb * 34, nb, xf);
  free(xf);
  return 0;
}

/* Canonical Q4_0 rows -> row-major bf16 out[n][k]. */
int cb_dequant_q4_0(const uint8_t* raw, int64_t n_rows, int64_t k, uint16_t* out, int threads) {
  if (k % 32 != 0 || n_rows < 0) return -1;
  const int64_t nb = k / 32;
  int fail = 0;
#pragma omp parallel num_threads(threads)
  {
    float* w = (float*)malloc(sizeof(float) * (size_t)k);
    if (!w) {
#pragma omp atomic write
      fail = 1;
    }
#pragma omp for schedule(static)
    for (int64_t r = 0; r < n_rows; ++r) {
      if (!w) continue;
      cb_q4_0_row(raw + r * nb * 18, nb, w);
      uint16_t* o = out + r * k;
      for (int64_t j = 0; j < k; ++j) o[j] = (uint16_t)(cb_bits(w[j]) >> 16);
    }
    free(w);
  }
  return fail ? -1 : 0;
}

/* Dot products of 8 weight rows with one activation row. */
CB_CLONES static void cb_dot8(const float* w, int64_t k, const float* x, float* out) {
  float a0 = 0, a1 = 0, a2 = 0, a3 = 0, a4 = 0, a5 = 0, a6 = 0, a7 = 0;
#pragma omp simd reduction(+ : a0, a1, a2, a3, a4, a5, a6, a7)
  for (int64_t i = 0; i < k; ++i) {
    const float xv = x[i];
    a0 += w[i] * xv;
    a1 += w[k + i] * xv;
    a2 += w[2 * k + i] * xv;
    a3 += w[3 * k + i] * xv;
    a4 += w[4 * k + i] * xv;
    a5 += w[5 * k + i] * xv;
    a6 += w[6 * k + i] * xv;
    a7 += w[7 * k + i] * xv;
  }
  out[0] = a0; out[1] = a1; out[2] = a2; out[3] = a3;
  out[4] = a4; out[5] = a5; out[6] = a6; out[7] = a7;
}

/* Y[m][n] = sum_k X[m][k] W[n][k]: each thread dequantizes 8 weight rows at
 * a time (bf16-rounded, held as float) and runs them against every row of X. */
int cb_gemm_q4_0(const uint8_t* raw, int64_t n_rows, int64_t k, const uint16_t* x, int64_t m, float* y,
                 int threads) {
  if (k % 32 != 0 || n_rows < 0 || m < 0) return -1;
  float* xf = cb_x_f32(x, m * k);
  if (!xf) return -1;
  const int64_t nb = k / 32, tiles = (n_rows + 7) / 8;
  int fail = 0;
#pragma omp parallel num_threads(threads)
  {
    float* w = (float*)malloc(sizeof(float) * (size_t)(8 * k));
    if (!w) {
#pragma omp atomic write
      fail = 1;
    }
#pragma omp for schedule(dynamic, 4)
    for (int64_t t = 0; t < tiles; ++t) {
      if (!w) continue;
      const int64_t r0 = 8 * t;
      for (int r = 0; r < 8; ++r) {
        const int64_t rr = r0 + r < n_rows ? r0 + r : n_rows - 1;
        cb_q4_0_row(raw + rr * nb * 18, nb, w + r * k);
      }
      float o[8];
      for (int64_t i = 0; i < m; ++i) {
        cb_dot8(w, k, xf + i * k, o);
        for (int r = 0; r < 8 && r0 + r < n_rows; ++r) y[i * n_rows + r0 + r] = o[r];
      }
    }
    free(w);
  }
  free(xf);
  return fail ? -1 : 0;
}

/* A row of Q6_K super-blocks -> k bf16-rounded weights as float
 * (src/quants/tests/formats/q6_k.py:55-129): element 128 h + 32 j + l takes
 * the low (j < 2) or high nibble of ql[64 h + 32 (j & 1) + l], bits
 * 2 j .. 2 j + 1 of qh[32 h + l] and sub-scale sc[8 h + l / 16 + 2 j]. */
CB_CLONES static void cb_q6_k_row(const uint8_t* row, int64_t nb, float* w) {
  for (int64_t b = 0; b < nb; ++b) {
    const uint8_t* blk = row + 210 * b;
    const uint8_t *ql = blk, *qh = blk + 128;
    const int8_t* sc = (const int8_t*)(blk + 192);
    const float d = cb_scale(cb_le16(blk + 208));
    float* o = w + 256 * b;
    for (int h = 0; h < 2; ++h)
      for (int j = 0; j < 4; ++j) {
        const float ds0 = d * (float)sc[8 * h + 2 * j], ds1 = d * (float)sc[8 * h + 1 + 2 * j];
#pragma omp simd
        for (int l = 0; l < 32; ++l) {
          const int q = ((ql[64 * h + 32 * (j & 1) + l] >> (4 * (j >> 1))) & 15) | (((qh[32 * h + l] >> (2 * j)) & 3) << 4);
          o[128 * h + 32 * j + l] = cb_bf16_round((l < 16 ? ds0 : ds1) * (float)(q - 32));
        }
      }
  }
}

CB_CLONES static float cb_dot(const float* w, int64_t k, const float* x) {
  float a = 0.0f;
#pragma omp simd reduction(+ : a)
  for (int64_t i = 0; i < k; ++i) a += w[i] * x[i];
  return a;
}

/* y[n] = sum_k W[n][k] x[k], W canonical Q6_K rows of k/256 super-blocks. */
int cb_gemv_q6_k(const uint8_t* raw, int64_t n_rows, int64_t k, const uint16_t* x, float* y, int threads) {
  if (k % 256 != 0 || n_rows < 0) return -1;
  float* xf = cb_x_f32(x, k);
  if (!xf) return -1;
  const int64_t nb = k / 256;
  int fail = 0;
#pragma omp parallel num_threads(threads)
  {
    float* w = (float*)malloc(sizeof(float) * (size_t)k);
    if (!w) {
#pragma omp atomic write
      fail = 1;
    }
#pragma omp for schedule(static)
    for (int64_t r = 0; r < n_rows; ++r) {
      if (!w) continue;
      cb_q6_k_row(raw + r * nb * 210, nb, w);
      y[r] = cb_dot(w, k, xf);
    }
    free(w);
  }
  free(xf);
  return fail ? -1 : 0;
}

/* Canonical Q6_K rows -> row-major bf16 out[n][k]. */
int cb_dequant_q6_k(const uint8_t* raw, int64_t n_rows, int64_t k, uint16_t* out, int threads) {
  if (k % 256 != 0 || n_rows < 0) return -1;
  const int64_t nb = k / 256;
  int fail = 0;
#pragma omp parallel num_threads(threads)
  {
    float* w = (float*)malloc(sizeof(float) * (size_t)k);
    if (!w) {
#pragma omp atomic write
      fail = 1;
    }
#pragma omp for schedule(static)
    for (int64_t r = 0; r < n_rows; ++r) {
      if (!w) continue;
      cb_q6_k_row(raw + r * nb * 210, nb, w);
      uint16_t* o = out + r * k;
      for (int64_t j = 0; j < k; ++j) o[j] = (uint16_t)(cb_bits(w[j]) >> 16);
    }
    free(w);
  }
  return fail ? -1 : 0;
}

/* MUL_MAT_ID over canonical Q4_0 experts, the grouped form of
 * src/quants/tests/mmul.py:104-112: expert e (n_rows rows of k, at
 * raw + e * expert_bytes) multiplies the activations of every (token, slot)
 * routed to it, y[t][s][:] = W[ids[t][s]] x[t][s % x_slots][:]. Each thread
 * takes whole experts; an expert's rows are dequantized once, 8 at a time,
 * and run against all of its pairs. Ids outside [0, n_expert) give zeros. */
int cb_moe_q4_0(const uint8_t* raw, int64_t expert_bytes, int64_t n_expert, int64_t n_rows, int64_t k,
                const uint16_t* x, int64_t x_slots, const int32_t* ids, int64_t n_tokens, int64_t top_k, float* y,
                int threads) {
  if (k % 32 != 0 || n_rows <= 0 || n_expert <= 0 || n_tokens < 0 || top_k <= 0) return -1;
  if (x_slots != 1 && x_slots != top_k) return -1;
  const int64_t pairs = n_tokens * top_k, nb = k / 32;
  float* xf = cb_x_f32(x, n_tokens * x_slots * k);
  int64_t* order = (int64_t*)malloc(sizeof(int64_t) * (size_t)(pairs + 1));
  int64_t* start = (int64_t*)calloc((size_t)(n_expert + 1), sizeof(int64_t));
  if (!xf || !order || !start) {
    free(xf), free(order), free(start);
    return -1;
  }
  /* pairs grouped by expert (counting sort, pair order kept) */
  for (int64_t p = 0; p < pairs; ++p) {
    const int32_t e = ids[p];
    if (e >= 0 && e < n_expert) ++start[e + 1];
    else memset(y + p * n_rows, 0, sizeof(float) * (size_t)n_rows);
  }
  for (int64_t e = 0; e < n_expert; ++e) start[e + 1] += start[e];
  {
    int64_t* fill = (int64_t*)malloc(sizeof(int64_t) * (size_t)n_expert);
    if (!fill) {
      free(xf), free(order), free(start);
      return -1;
    }
    memcpy(fill, start, sizeof(int64_t) * (size_t)n_expert);
    for (int64_t p = 0; p < pairs; ++p) {
      const int32_t e = ids[p];
      if (e >= 0 && e < n_expert) order[fill[e]++] = p;
    }
    free(fill);
  }
  const int64_t tiles = (n_rows + 7) / 8;
  int fail = 0;
#pragma omp parallel num_threads(threads)
  {
    float* w = (float*)malloc(sizeof(float) * (size_t)(8 * k));
    if (!w) {
#pragma omp atomic write
      fail = 1;
    }
#pragma omp for schedule(dynamic, 1) collapse(2)
    for (int64_t e = 0; e < n_expert; ++e)
      for (int64_t t = 0; t < tiles; ++t) {
        if (!w || start[e] == start[e + 1]) continue;
        const uint8_t* ex = raw + e * expert_bytes;
        const int64_t r0 = 8 * t;
        for (int r = 0; r < 8; ++r) {
          const int64_t rr = r0 + r < n_rows ? r0 + r : n_rows - 1;
          cb_q4_0_row(ex + rr * nb * 18, nb, w + r * k);
        }
        float o[8];
        for (int64_t i = start[e]; i < start[e + 1]; ++i) {
          const int64_t p = order[i], tok = p / top_k, slot = p % top_k;
          cb_dot8(w, k, xf + (tok * x_slots + slot % x_slots) * k, o);
          for (int r = 0; r < 8 && r0 + r < n_rows; ++r) y[p * n_rows + r0 + r] = o[r];
        }
      }
    free(w);
  }
  free(xf), free(order), free(start);
  return fail ? -1 : 0;
}
