/*
 * quants_oracle.h -- TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of the reference's GGUF block dequantization, record repack
 * and fused-matmul semantics (crlfe/spiral, src/quants). It exists to check
 * the HIP library; nothing in spiral_amd/ links, loads or calls it. Only
 * tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg use it.
 *
 * Conventions follow the reference: a weight tensor has K = weights_rows
 * (the contiguous dot-product axis, ggml ne0) and N = weights_cols (ggml rows,
 * ne1). Canonical GGUF storage is N rows of K/block_elems blocks each; row n
 * starts at n * row_stride bytes (the reference's src_col_stride_bytes,
 * src/quants/tests/common.py:208-210).
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   oq_fp16_device   IEEE binary16 via numpy for exp 1..30, explicit fixtures
 *                    for exp 0 and exp 31 (reference text).
 *   oq_bf16_rne      torch's float32->bfloat16 conversion on random and tie
 *                    patterns.
 *   oq_dequant_*     exhaustive comparison with oq_aie_* (the reference's
 *                    device arithmetic step by step), and Python exact
 *                    rational arithmetic + torch RNE on random blocks.
 *   oq_ref_repack    byte comparison with the reference's own repack.h,
 *                    compiled from /root/reference into oracle/_ref, and with
 *                    committed fixtures made from it.
 *   oq_ref_unpack    equality with the canonical dequant re-ordered into the
 *                    reference's output order.
 *   oq_matmul_f64    numpy float64 matmul on small shapes.
 *   oq_dequant Q4_K / Q5_K (no reference code or vectors exist; ggml's
 *                    published block layout): (i) the 6-bit scale/min fields
 *                    decoded from bytes packed by an independent field-wise
 *                    packer, over every (scale, min) pair at every group;
 *                    (ii) blocks whose scales and mins reduce the K-quant to
 *                    d' * (q - c) equal the Q8_0 oracle's dequant of the same
 *                    codes, element by element (pins element order, nibble
 *                    and qh bit placement, the sign of the min term); (iii)
 *                    subnormal d / dmin against numpy's IEEE binary16; (iv)
 *                    the single rounding (fmaf) against exact rationals.
 *   oq_dequant IQ4_NL / IQ4_XS (no reference code or vectors; ggml's layout
 *                    and kvalues_iq4nl codebook): IQ4_NL blocks equal the Q8_0
 *                    oracle on codes kv[index] with the same d; IQ4_XS
 *                    sub-blocks equal IQ4_NL blocks with d' = d * (ls - 32);
 *                    every 6-bit ls at every sub-block from an independent
 *                    packer; subnormal d against numpy.
 */
#ifndef SPIRAL_QUANTS_ORACLE_H
#define SPIRAL_QUANTS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (the values ggml uses for these formats). */
enum { OQ_Q4_0 = 2, OQ_Q8_0 = 8, OQ_Q4_K = 12, OQ_Q5_K = 13, OQ_Q6_K = 14, OQ_IQ4_NL = 20, OQ_IQ4_XS = 23 };

/* ---- scalar conversions ------------------------------------------------ */

/* IEEE binary16 -> binary32 (subnormals, inf and NaN handled per IEEE). */
float oq_fp16_ieee(uint16_t h);

/* The reference's device decode of a block scale
 * (src/quants/common/scale.aie.h:9-27): exp == 0 (zero or subnormal) -> +0,
 * exp == 31 -> finite sign * 2^16 * (1 + m/1024), otherwise IEEE. The host
 * repack flush of subnormal scales (src/quants/common/repack.h:29-34) maps to
 * the same +0. */
float oq_fp16_device(uint16_t h);

/* float32 -> bfloat16, round to nearest even (algorithm of
 * src/quants/q4_0_hilo/repack.h:32-38; finite inputs). */
uint16_t oq_bf16_rne(float f);
float oq_bf16_f32(uint16_t b);

/* Array forms of the two conversions above. */
void oq_fp16_device_array(const uint16_t* h, float* out, int64_t n);
void oq_bf16_rne_array(const float* f, uint16_t* out, int64_t n);

/* ---- the reference's device arithmetic, step by step -------------------- */

/* Q4_0 / Q8_0 element: split d into bf16 hi/lo (scale.aie.h:29-39), then
 * acc = q*hi; acc += q*lo in fp32; round to bf16 (q4_0/unpack.aie.h:41-45,
 * q8_0/unpack.aie.h:44-51). q is the signed code. */
uint16_t oq_aie_q_times_d(int q, uint16_t d_bits);

/* Q6_K element: d split hi/lo, p = d_hi*sc + d_lo*sc, p split into three bf16
 * terms, acc = q*hi + q*mid + q*lo, round to bf16
 * (q6_k/unpack.aie.h:33-61,81-91). q is the centred code q-32. */
uint16_t oq_aie_q6_k(int q_centred, int sc, uint16_t d_bits);

/* Exhaustive comparisons of oq_aie_* with the closed form bf16_rne(exact
 * product) over every normal fp16 d (both signs). Returns the number of value
 * mismatches; *signed_zero receives the count of cases that differ only in
 * the sign of a zero result. d_step > 1 samples every d_step-th d. */
int64_t oq_check_q_times_d(int64_t* signed_zero);
int64_t oq_check_q6_k(int d_step, int64_t* signed_zero);
/* Checks hi + lo == d exactly for every normal fp16 d; returns failures. */
int64_t oq_check_split_identity(void);

/* ---- canonical GGUF dequantization -------------------------------------- */

/* Bytes of one canonical block and the number of elements it holds. */
int oq_block_bytes(int type);
int oq_block_elems(int type);

/* Dequantize canonical rows into row-major bf16 out[n * ld_out + k].
 * Element value: bf16_rne(code * oq_fp16_device(d)) for Q4_0 (code = q-8)
 * and Q8_0; bf16_rne(oq_fp16_device(d) * sc * (q-32)) for Q6_K
 * (src/quants/tests/formats/q4_0.py:47-60, q8_0.py:48-58, q6_k.py:55-97);
 * bf16_rne(fmaf(d * scale, q, -dmin * min)) for Q4_K / Q5_K with IEEE d and
 * dmin (the plan of src/quants/TODO.md:80-107 over ggml's block layout);
 * bf16_rne(d * kv[index]) for IQ4_NL and bf16_rne(d * (ls - 32) * kv[index])
 * for IQ4_XS, IEEE d (src/quants/TODO.md:109-124, ggml's layout).
 * Returns 0, or -1 on a bad shape. */
int oq_dequant(int type, const uint8_t* src, int64_t row_stride,
               int64_t n_rows, int64_t k, uint16_t* out, int64_t ld_out);

/* Dequantize selected rows (ggml GET_ROWS) into row-major bf16. */
/* Canonical rows -> the exact (unrounded) weights as double: the values
 * that oq_dequant rounds to bf16 once. */
int oq_dequant_f64(int type, const uint8_t* src, int64_t row_stride,
                   int64_t n_rows, int64_t k, double* out, int64_t ld_out);
/* y[m, n] = sum_k x[m, k] * w[n, k] in double over double weights. */
void oq_matmul_f64_exact(const double* w, int64_t ldw, int64_t n_rows, int64_t k,
                         const uint16_t* x, int64_t ldx, int64_t m, double* y,
                         int64_t ldy);
int oq_get_rows(int type, const uint8_t* src, int64_t row_stride,
                int64_t n_rows, int64_t k, const int32_t* ids, int64_t n_ids,
                uint16_t* out, int64_t ld_out);

/* ---- the reference's NPU record layout ---------------------------------- */

/* record_count / packed_bytes / repack_weights of src/quants/<fmt>/repack.h
 * with the same argument meaning and 0-on-error convention. *warnings gets
 * bit 0 = a subnormal scale was flushed, bit 1 = an int8 -128 was seen. */
int64_t oq_ref_record_count(int type, int64_t weights_rows, int64_t weights_cols);
int64_t oq_ref_packed_bytes(int type, int64_t weights_rows, int64_t weights_cols);
int64_t oq_ref_repack(int type, const uint8_t* src, int64_t src_col_stride_bytes,
                      uint8_t* dst, int64_t dst_capacity, int64_t weights_rows,
                      int64_t weights_cols, int* warnings);

/* quants_unpack_all (src/quants/tests/unpack.aie.cc:21-45): decode records
 * into the reference output order
 * [weights_cols/8][weights_rows/record_rows][chunk][chunk_rows][8]. */
int oq_ref_unpack(int type, const uint8_t* packed, int64_t weights_rows,
                  int64_t weights_cols, uint16_t* out);

/* ---- matmul ------------------------------------------------------------- */

/* y[i * ldy + n] = sum_k x[i * ldx + k] * w[n * ldw + k] in float64 over bf16
 * inputs (the reference's check, src/quants/tests/mmul.py:104-112, in wider
 * precision). OpenMP over n. */
void oq_matmul_f64(const uint16_t* w, int64_t ldw, int64_t n_rows, int64_t k,
                   const uint16_t* x, int64_t ldx, int64_t m, double* y,
                   int64_t ldy);

/* The same with float32 accumulation in k order: the arithmetic of the
 * reference's fused mmul (fp32 accumulators over bf16 products). */
void oq_matmul_f32(const uint16_t* w, int64_t ldw, int64_t n_rows, int64_t k,
                   const uint16_t* x, int64_t ldx, int64_t m, float* y,
                   int64_t ldy);

/* Dequantize-then-multiply, streaming: y[i][n] = sum_k x[i][k] * W[n][k] with
 * W dequantized per row on the fly (no full bf16 copy). fp32 accumulation.
 * The CPU baseline for GEMV/GEMM. OpenMP over rows when threads > 1. */
int oq_quant_matmul_f32(int type, const uint8_t* src, int64_t row_stride,
                        int64_t n_rows, int64_t k, const uint16_t* x,
                        int64_t ldx, int64_t m, float* y, int64_t ldy,
                        int threads);

#ifdef __cplusplus
}
#endif

#endif
