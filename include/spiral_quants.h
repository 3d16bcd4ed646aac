/*
 * spiral_quants.h -- C ABI of libspiral_quants.so, the MI355X (gfx950)
 * implementation of spiral's quantized-weight hot path: GGUF Q4_0 / Q8_0 /
 * Q6_K (and the Q4_K / Q5_K / IQ4_NL / IQ4_XS formats the reference plans)
 * block dequantization to bf16 and the dequant-fused matrix products behind a ggml
 * backend's MUL_MAT / GET_ROWS / MUL_MAT_ID.
 *
 * Conventions
 *  - Plain C types only. Device pointers are HIP device memory; `stream` is a
 *    hipStream_t passed as void* (NULL = the null stream). Every call is
 *    asynchronous on that stream; nothing synchronizes unless stated.
 *  - Return value: spiral_status (0 = SPIRAL_OK). Validation failures are
 *    reported before anything is launched. No exceptions cross the ABI.
 *  - Shapes use ggml's naming: a weight tensor has n_rows rows (ggml ne1,
 *    the reference's weights_cols) of k elements (ggml ne0, the reference's
 *    weights_rows). A product computes y[i][n] = sum_k x[i][k] * W[n][k].
 *  - bf16 values travel as uint16_t bit patterns.
 *  - Thread-safe for calls on distinct streams. Process-wide state: per-device
 *    caches (compute-unit counts, occupancy, raised LDS limits) filled once
 *    under a lock, and the repack warning route (quants_set_repack_warn).
 */
#ifndef SPIRAL_QUANTS_H
#define SPIRAL_QUANTS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum spiral_status {
  SPIRAL_OK = 0,
  SPIRAL_ERR_SHAPE = 1,     /* k not a multiple of the block, size <= 0, bad ld */
  SPIRAL_ERR_ALIGN = 2,     /* a device pointer is not 16-byte aligned */
  SPIRAL_ERR_NULL = 3,      /* a required pointer is NULL */
  SPIRAL_ERR_NO_DEVICE = 4, /* no HIP device is visible */
  SPIRAL_ERR_HIP = 5,       /* a HIP runtime call or kernel launch failed */
  SPIRAL_ERR_TYPE = 6,      /* unsupported tensor type or op */
  SPIRAL_ERR_CAPACITY = 7,  /* a caller buffer is too small */
  SPIRAL_ERR_RANGE = 8      /* an index is outside its tensor (host-checked) */
} spiral_status;

/* Tensor type ids: the values ggml uses for these types (ggml_type). */
enum {
  SPIRAL_TYPE_F32 = 0,
  SPIRAL_TYPE_F16 = 1,
  SPIRAL_TYPE_Q4_0 = 2,
  SPIRAL_TYPE_Q8_0 = 8,
  SPIRAL_TYPE_Q4_K = 12,
  SPIRAL_TYPE_Q5_K = 13,
  SPIRAL_TYPE_Q6_K = 14,
  SPIRAL_TYPE_IQ4_NL = 20,
  SPIRAL_TYPE_IQ4_XS = 23,
  SPIRAL_TYPE_I32 = 26,
  SPIRAL_TYPE_BF16 = 30
};

const char* spiral_status_string(int status);

/* Number of visible HIP devices (0 when none); never fails. */
int spiral_device_count(void);

/* ===================================================================== *
 * 1. The reference's host repack API, per format.                        *
 *                                                                         *
 * Same argument meaning, layout and 0-on-error convention as             *
 * spiral::quants::<fmt>::record_count / packed_bytes / repack_weights     *
 * (src/quants/q4_0/repack.h:10-111, src/quants/q8_0/repack.h:10-91,      *
 * src/quants/q6_k/repack.h:11-115) and their C shim quants_record_count / *
 * quants_packed_bytes / quants_repack (src/quants/tests/repack.cc:12-33), *
 * which the reference builds once per format; here the format is part of  *
 * the name. Host memory; the output is the reference's record stream,     *
 * byte for byte. A subnormal fp16 scale is stored as +0 and one warning    *
 * line per call goes to stderr, or to the callback set below              *
 * (src/quants/common/repack.h:38-61).                                      *
 * ===================================================================== */

/* Routes the repack warning line: the reference lets a caller that compiles
 * its header redefine QUANTS_REPACK_WARN to reroute or silence the line
 * (src/quants/common/repack.h:9-14); a shared library takes a callback.
 * fn receives the line (ending in a newline) and `user`; fn == NULL restores
 * stderr; a callback that does nothing silences it. Process-wide; a repack
 * running while this is called uses either the old or the new route. */
typedef void (*quants_warn_fn)(const char* line, void* user);
void quants_set_repack_warn(quants_warn_fn fn, void* user);
int64_t quants_q4_0_record_count(int64_t weights_rows, int64_t weights_cols);
int64_t quants_q4_0_packed_bytes(int64_t weights_rows, int64_t weights_cols);
int64_t quants_q4_0_repack(const uint8_t* src, int64_t src_col_stride_bytes,
                           uint8_t* dst, int64_t dst_capacity,
                           int64_t weights_rows, int64_t weights_cols);
int64_t quants_q8_0_record_count(int64_t weights_rows, int64_t weights_cols);
int64_t quants_q8_0_packed_bytes(int64_t weights_rows, int64_t weights_cols);
int64_t quants_q8_0_repack(const uint8_t* src, int64_t src_col_stride_bytes,
                           uint8_t* dst, int64_t dst_capacity,
                           int64_t weights_rows, int64_t weights_cols);
int64_t quants_q6_k_record_count(int64_t weights_rows, int64_t weights_cols);
int64_t quants_q6_k_packed_bytes(int64_t weights_rows, int64_t weights_cols);
int64_t quants_q6_k_repack(const uint8_t* src, int64_t src_col_stride_bytes,
                           uint8_t* dst, int64_t dst_capacity,
                           int64_t weights_rows, int64_t weights_cols);

/* ===================================================================== *
 * 2. The reference's device entry points on the GPU, over its records.   *
 * ===================================================================== */

/* Replaces quants_unpack_all (src/quants/tests/unpack.aie.cc:21-45):
 * exact bf16 dequantization of a reference record stream (from
 * quants_<fmt>_repack, copied to the device) into the reference's output
 * order [weights_cols/8][weights_rows/record_rows][chunk][rows][8]. Shapes are
 * runtime arguments instead of -DQUANTS_WEIGHTS_ROWS/COLS. */
int quants_unpack_all(int type, const void* packed, int64_t weights_rows,
                      int64_t weights_cols, uint16_t* out, void* stream);

/* Replaces quants_unpack_mmul_all (src/quants/tests/mmul.aie.cc:20-35):
 * fused dequant + bf16 product with fp32 accumulation over a record stream.
 * inputs: bf16 [weights_rows/8][4][8] (four input vectors, tiled by 8 along
 * k); outputs: f32 [weights_cols/8][4][8], overwritten (the shim zeroes its
 * outputs first). */
int quants_unpack_mmul_all(int type, const void* packed,
                           const uint16_t* inputs, float* outputs,
                           int64_t weights_rows, int64_t weights_cols,
                           void* stream);

/* ===================================================================== *
 * 3. The GPU weight layout and the ggml op surface.                      *
 *                                                                         *
 * A quantized weight lives on the device in "planar" layout: the fields of *
 * the canonical GGUF blocks split into separate row-major planes, so every *
 * 16-byte payload vector is 16-byte aligned. Same byte count as the         *
 * canonical tensor; a pure permutation of its bytes.                        *
 *   Q4_0: qs[n_rows][k/32][16]  | d[n_rows][k/32] (fp16)                     *
 *   Q8_0: qs[n_rows][k/32][32]  | d[n_rows][k/32]                            *
 *   Q6_K: ql[n_rows][k/256][128] | qh[..][64] | sc[..][16] | d[n_rows][k/256] *
 *   Q4_K: qs[n_rows][k/256][128] | meta[..][16]                              *
 *   Q5_K: qs[n_rows][k/256][128] | qh[..][32] | meta[..][16]                 *
 * (meta: a K-quant block's first 16 canonical bytes, fp16 d, fp16 dmin and  *
 * the 12 packed 6-bit scale/min bytes, kept together for one 16-byte load). *
 *   IQ4_NL: as Q4_0: qs[n_rows][k/32][16] | d[n_rows][k/32]                  *
 *   IQ4_XS: qs[n_rows][k/256][128] | meta[..][8] (fp16 d, scales_h,          *
 *           scales_l[4]: the block's first 8 canonical bytes)                *
 * This is the GPU counterpart of the reference's load-time repack           *
 * (src/quants/TODO.md:303-334). Weight pointers below are planar and must be *
 * 16-byte aligned.                                                          *
 * ===================================================================== */

/* Canonical bytes per row / per tensor (also the planar size); 0 when k is
 * not a multiple of the type's block or a size is not positive. */
int64_t spiral_row_bytes(int type, int64_t k);
int64_t spiral_tensor_bytes(int type, int64_t n_rows, int64_t k);

/* Canonical GGUF rows (row n at src + n*src_row_stride) -> planar. */
int spiral_to_planar(int type, const void* src, int64_t src_row_stride,
                     int64_t n_rows, int64_t k, void* dst, void* stream);
/* Planar -> canonical GGUF rows (inverse of spiral_to_planar). */
int spiral_from_planar(int type, const void* src, int64_t n_rows, int64_t k,
                       void* dst, int64_t dst_row_stride, void* stream);

/* Exact dequantization, planar -> row-major bf16 out[n*ld_out + k]. Element
 * values are bf16_rne(code * d) (Q4_0 code q-8, Q8_0 int8) and
 * bf16_rne(d * sc * (q-32)) (Q6_K), d decoded as the reference's device does
 * (exponent 0 -> +0; src/quants/common/scale.aie.h:9-27). Bit-identical to
 * the reference's unpack (src/quants/<fmt>/unpack.aie.h).
 * Q4_K / Q5_K (planned by the reference, src/quants/TODO.md:80-107, with no
 * code to match): bf16_rne(fma(d * scale, q, -dmin * min)), d and dmin IEEE
 * binary16 (subnormals keep their value, as in ggml), one float rounding.
 * IQ4_NL / IQ4_XS (planned, src/quants/TODO.md:109-124): bf16_rne(d *
 * kv[index]) and bf16_rne(d * (ls - 32) * kv[index]) over ggml's 16-entry
 * kvalues_iq4nl codebook, d IEEE binary16; each product is exact in fp32. */
int spiral_dequant_bf16(int type, const void* w, int64_t n_rows, int64_t k,
                        uint16_t* out, int64_t ld_out, void* stream);

/* ggml GET_ROWS with quantized src0: out[i] = dequant(W[ids[i]]), out_type
 * BF16 or F32 (both carry the same exact bf16 value). ids are device int32;
 * an id outside [0, n_rows) yields a row of zeros. */
int spiral_get_rows(int type, const void* w, int64_t n_rows, int64_t k,
                    const int32_t* ids, int64_t n_ids, void* out, int out_type,
                    int64_t ld_out, void* stream);

/* ggml MUL_MAT with quantized src0: y[i][n] = sum_k x[i][k] * W[n][k] for
 * i < m, x bf16 rows of stride ldx elements, y (BF16 or F32) rows of stride ldy
 * elements. Every W[n][k] is the exact dequantized bf16 weight (the value
 * spiral_dequant_bf16 gives), multiplied by x with fp32 accumulation, as in
 * the reference's fused dequant + mmul (src/quants/q4_0/mmul.aie.h:16-90,
 * src/quants/common/mmul.aie.h:9-22); the form chosen for m only changes
 * the summation order. m == 1 runs the streaming GEMV; 2 <= m <= 16
 * (decode batches, speculative decoding) runs the weight-streaming MFMA form,
 * which reads every weight byte once; larger m runs the MFMA dequant-GEMM,
 * which first rewrites x into MFMA operand order in `workspace` (device
 * memory, 16-byte aligned, caller-owned; at least
 * spiral_mul_mat_workspace_bytes() bytes, which is 0 for m <= 16, in which
 * case workspace may be NULL). A workspace must not be shared by calls in
 * flight at the same time. The small-batch form needs y within 2 GiB
 * ((m - 1) * ldy + n_rows elements), else SPIRAL_ERR_SHAPE. */
int64_t spiral_mul_mat_workspace_bytes(int type, int64_t n_rows, int64_t k,
                                       int64_t m);
int spiral_mul_mat(int type, const void* w, int64_t n_rows, int64_t k,
                   const uint16_t* x, int64_t ldx, int64_t m, void* y,
                   int y_type, int64_t ldy, void* workspace,
                   int64_t workspace_bytes, void* stream);

/* Named relaxed mode of the single-row product (m = 1), kept apart from the
 * exact default as the reference requires of fast variants ("separate named
 * variants with explicit verification policies", src/quants/TODO.md:132-135).
 * y[n] = sum over blocks of scale * (sum_k code[n][k] * x[k]): the block
 * scale multiplies the block's fp32 sum, so weights are never rounded to
 * bf16. That is the scale-after-mmul arithmetic the reference rejects as a
 * default (src/quants/NOTES.md:327-330). Tolerance, stated and tested:
 * within 1e-4 (F32 out) of the float64 product over unrounded weights
 * code * scale; against the exact bf16-weight product it moves outputs by
 * about 1e-2 of the largest output at k = 4096..14336, so it is tested only
 * to 2e-2 there. x bf16 [k], y [n_rows] of y_type (BF16 or F32); k at most
 * spiral_gemv_relaxed_max_k(type) (0 for a type it does not take). */
int64_t spiral_gemv_relaxed_max_k(int type);
int spiral_gemv_relaxed(int type, const void* w, int64_t n_rows, int64_t k,
                        const uint16_t* x, void* y, int y_type, void* stream);

/* ggml MUL_MAT_ID with quantized, expert-stacked src0: for token t < n_tokens
 * and slot s < top_k, y[t][s][:] = W[ids[t][s]] * x[t][s % x_slots][:].
 *  w: n_expert planar matrices of [n_rows][k], expert e at w + e*expert_stride
 *     (expert_stride >= spiral_tensor_bytes, multiple of 16).
 *  x: bf16 [n_tokens][x_slots][k] with x_slots 1 (shared input) or top_k.
 *  ids: device int32 [n_tokens][top_k]; an id outside [0, n_expert) gives a
 *     zero output row.
 *  y: [n_tokens][top_k][n_rows] of y_type (BF16 or F32).
 *  workspace: device scratch of spiral_mul_mat_id_workspace_bytes() bytes
 *     for the per-expert token lists (caller-owned, no allocation here). */
int64_t spiral_mul_mat_id_workspace_bytes(int64_t n_expert, int64_t n_tokens,
                                          int64_t top_k);
int spiral_mul_mat_id(int type, const void* w, int64_t expert_stride,
                      int64_t n_expert, int64_t n_rows, int64_t k,
                      const uint16_t* x, int64_t x_slots, const int32_t* ids,
                      int64_t n_tokens, int64_t top_k, void* y, int y_type,
                      void* workspace, int64_t workspace_bytes, void* stream);

/* spiral_mul_mat_id for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops or harnesses that forbid hipMalloc). No
 * counterpart in the reference. Arguments, results and errors as
 * spiral_mul_mat_id, without the workspace: the routing lists live in a
 * library-owned device array of SPIRAL_MUL_MAT_ID_STATIC_BYTES per GPU, held
 * until the process ends. A shape whose lists need more
 * (spiral_mul_mat_id_workspace_bytes(n_expert, n_tokens, top_k) above that:
 * about 262,000 experts plus (token, slot) pairs) fails with
 * SPIRAL_ERR_CAPACITY before anything runs. Calls no hipMalloc / hipFree.
 * Every call on one GPU shares that GPU's array: calls that overlap in time
 * on one GPU (on different streams, or from different host threads) race;
 * calls ordered on one stream do not. */
#define SPIRAL_MUL_MAT_ID_STATIC_BYTES (1 << 20)
int spiral_mul_mat_id_noalloc(int type, const void* w, int64_t expert_stride,
                              int64_t n_expert, int64_t n_rows, int64_t k,
                              const uint16_t* x, int64_t x_slots,
                              const int32_t* ids, int64_t n_tokens,
                              int64_t top_k, void* y, int y_type,
                              void* stream);

/* ggml GLU variants, numbered as ggml's ggml_glu_op: out = act(a) * b over
 * the two halves (a, b) of a row of 2F values, a the first half unless
 * swapped. act: REGLU relu, GEGLU gelu (tanh form), SWIGLU silu, GEGLU_ERF
 * gelu (erf form), GEGLU_QUICK x * sigmoid(1.702 x). SWIGLU_OAI (clamped,
 * with float parameters) is not implemented. */
enum {
  SPIRAL_GLU_REGLU = 0,
  SPIRAL_GLU_GEGLU = 1,
  SPIRAL_GLU_SWIGLU = 2,
  SPIRAL_GLU_SWIGLU_OAI = 3,
  SPIRAL_GLU_GEGLU_ERF = 4,
  SPIRAL_GLU_GEGLU_QUICK = 5
};

/* spiral_mul_mat_id followed by GLU over each output row, in one pass: the
 * expert matrices have n_rows = 2F rows (gate rows [0, F), up rows [F, 2F),
 * ggml's merged gate/up layout) and y[t][s][f] = act(g) * u with
 * g = (W x)[f], u = (W x)[F + f] (act(u) * g when swapped). y is
 * [n_tokens][top_k][F] of y_type; the [.. ][2F] product is never written.
 * Other arguments as spiral_mul_mat_id. Implemented for the decode shapes
 * (spiral_mul_mat_id_glu_fits; else SPIRAL_ERR_SHAPE); SPIRAL_ERR_TYPE for an unknown or
 * unimplemented glu_op. No counterpart in the reference, whose MoE path is
 * a plan (src/quants/TODO.md:55,214-220). */
/* 1 when spiral_mul_mat_id_glu implements this expert shape (a quantized
 * type, n_rows even and positive, k a positive multiple of the block and
 * within the fused pass's limit, 4096), else 0. Pure host logic. */
int spiral_mul_mat_id_glu_fits(int type, int64_t n_rows, int64_t k);
int spiral_mul_mat_id_glu(int type, const void* w, int64_t expert_stride,
                          int64_t n_expert, int64_t n_rows, int64_t k,
                          const uint16_t* x, int64_t x_slots,
                          const int32_t* ids, int64_t n_tokens, int64_t top_k,
                          int glu_op, int swapped, void* y, int y_type,
                          void* workspace, int64_t workspace_bytes,
                          void* stream);

/* ggml GLU on its own: y[r][f] = act(x[r][f]) * x[r][F + f] (halves swapped
 * when swapped) for r < rows, f < F; x rows of 2F floats with stride ldx
 * elements, y rows of stride ldy; F32 in and out, device pointers. */
int spiral_glu(int glu_op, int swapped, const float* x, int64_t ldx,
               int64_t F, int64_t rows, float* y, int64_t ldy, void* stream);

/* ggml's split GLU form fused into MUL_MAT_ID: the gate and up experts are
 * two stacks (w_gate, w_up) of n_expert planar n_ff x k matrices at the same
 * expert_stride, as in MoE FFNs stored with separate ffn_gate_exps and
 * ffn_up_exps tensors (ggml: two MUL_MAT_ID nodes and a GLU over both).
 * y[t][s][f] = act(gate) * up (act(up) * gate when swapped), y
 * [n_tokens][top_k][n_ff], the two products never stored. Same arguments,
 * limits (spiral_mul_mat_id_glu_fits(type, 2 * n_ff, k)), workspace and
 * errors as spiral_mul_mat_id_glu; w_up 16-byte aligned. Each output equals
 * MUL_MAT_ID of each stack followed by spiral_glu_split, bit for bit. */
int spiral_mul_mat_id_glu_split(int type, const void* w_gate, const void* w_up,
                                int64_t expert_stride, int64_t n_expert,
                                int64_t n_ff, int64_t k, const uint16_t* x,
                                int64_t x_slots, const int32_t* ids,
                                int64_t n_tokens, int64_t top_k, int glu_op,
                                int swapped, void* y, int y_type,
                                void* workspace, int64_t workspace_bytes,
                                void* stream);

/* ggml's split GLU on its own: y[r][f] = act(gate[r][f]) * up[r][f]
 * (act(up) * gate when swapped), rows of stride ldg / ldu / ldy elements;
 * F32 in and out, device pointers. */
int spiral_glu_split(int glu_op, int swapped, const float* gate, int64_t ldg,
                     const float* up, int64_t ldu, int64_t F, int64_t rows,
                     float* y, int64_t ldy, void* stream);

/* SPIRAL_GLU_SWIGLU_OAI (ggml's swiglu_oai, the gpt-oss FFN), which takes two
 * parameters (ggml op_params 2 and 3) and so has entry points of its own;
 * spiral_glu and spiral_glu_split answer SPIRAL_ERR_TYPE for it. With a the
 * activated half and b the other (halves as in spiral_glu, swapped likewise):
 *   x = min(a, limit), y = clamp(b, -limit, limit),
 *   out = x / (1 + exp(-alpha x)) * (y + 1).
 * Merged rows of 2F floats (as spiral_glu) or split gate / up rows (as
 * spiral_glu_split); same arguments, checks and errors otherwise. No
 * counterpart in the reference (ggml's GLU surface, README.md:11-14). */
int spiral_glu_swiglu_oai(int swapped, float alpha, float limit,
                          const float* x, int64_t ldx, int64_t F, int64_t rows,
                          float* y, int64_t ldy, void* stream);
int spiral_glu_split_swiglu_oai(int swapped, float alpha, float limit,
                                const float* gate, int64_t ldg, const float* up,
                                int64_t ldu, int64_t F, int64_t rows, float* y,
                                int64_t ldy, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SPIRAL_QUANTS_H */
