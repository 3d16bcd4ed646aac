/*
 * spiral_ggml.h -- a ggml-backend-shaped C surface over libspiral_quants.so:
 * buffer type / buffer / tensor upload, supports_op and graph_compute for
 * MUL_MAT, GET_ROWS and MUL_MAT_ID with quantized (Q4_0 / Q8_0 / Q6_K) src0,
 * and GLU (fused into a preceding MUL_MAT_ID when possible), on one HIP
 * device.
 *
 * The reference names this surface but does not contain it: its README says
 * the NPU backend "will live in a llama.cpp fork" (README.md:11-14) and its
 * repack header is meant to be compiled into that loader
 * (src/quants/common/repack.h:5-7). ggml itself is not vendored. The types
 * below therefore mirror the public ggml-backend interface field for field
 * (ggml_tensor's type / buffer / ne / nb / op / op_params / flags / src /
 * view_src / view_offs / data / name, ggml_cgraph's
 * n_nodes / nodes, ggml_backend_buffer_i's alloc / free / get_base /
 * init_tensor / set_tensor / get_tensor / memset_tensor / clear,
 * ggml_backend_i's graph_compute / synchronize, ggml_backend_device_i's
 * supports_op) without being ABI-identical to any ggml release: a llama.cpp
 * backend shim copies its ggml_tensor fields into spiral_tensor one to one
 * (the op ids differ between ggml releases and are mapped by that shim).
 *
 * Quantized tensors are stored on the device in the library's planar layout
 * (see spiral_quants.h section 3): set_tensor converts canonical GGUF bytes
 * to planar, get_tensor converts back, so the buffer looks canonical from
 * the host. Byte counts are unchanged (the planar layout is a permutation of
 * each 2-D matrix's bytes), so ggml's allocator sizes still hold.
 *
 * Errors: functions return spiral_status codes (spiral_quants.h); nothing
 * aborts the process. Not thread-safe per backend or buffer (as ggml).
 */
#ifndef SPIRAL_GGML_H
#define SPIRAL_GGML_H

#include <stddef.h>
#include <stdint.h>

#include "spiral_quants.h"

#ifdef __cplusplus
extern "C" {
#endif

#define SPIRAL_MAX_DIMS 4
#define SPIRAL_MAX_SRC 10
#define SPIRAL_MAX_NAME 64
#define SPIRAL_MAX_OP_PARAMS 16 /* int32 words, ggml's 64 bytes */

/* ggml tensor flags this backend reads: an OUTPUT tensor is read after the
 * graph runs, so it is never fused away. */
#define SPIRAL_TENSOR_FLAG_OUTPUT 2

/* Operations this backend knows (the subset of ggml_op it takes part in).
 * NONE / VIEW / RESHAPE / PERMUTE / TRANSPOSE are no-ops at compute time, as
 * in every ggml backend. */
typedef enum spiral_op {
  SPIRAL_OP_NONE = 0,
  SPIRAL_OP_GET_ROWS = 1,
  SPIRAL_OP_MUL_MAT = 2,
  SPIRAL_OP_MUL_MAT_ID = 3,
  SPIRAL_OP_VIEW = 4,
  SPIRAL_OP_RESHAPE = 5,
  SPIRAL_OP_PERMUTE = 6,
  SPIRAL_OP_TRANSPOSE = 7,
  SPIRAL_OP_GLU = 8 /* op_params[0]: SPIRAL_GLU_* variant, op_params[1]: swapped
                      (single-tensor form only: the split form, src1 set,
                      activates src0 whatever it holds, as ggml does);
                      SWIGLU_OAI: op_params[2] alpha, [3] limit (floats) */
} spiral_op;

typedef struct spiral_buffer spiral_buffer;   /* device memory block (opaque) */
typedef struct spiral_backend spiral_backend; /* one device + stream (opaque) */

/* ggml_tensor's fields that a backend reads: type (SPIRAL_TYPE_*, the ggml
 * type ids), ne (elements per dimension, ne[0] innermost), nb (byte strides),
 * op, op_params and flags, src (the node's inputs), view_src / view_offs (for
 * a view: the tensor that owns the memory, never itself a view, and the
 * view's byte offset into it; NULL / 0 otherwise), data (device address
 * inside `buffer`).
 *
 * A quantized view is usable (as MUL_MAT / GET_ROWS / MUL_MAT_ID src0, or by
 * set_tensor / get_tensor) only when it starts whole planar matrices of its
 * source: same row length and row count as the source's matrices, and an
 * offset that is a whole number of them (for example one expert of a stack).
 * A row-range view inside a matrix is refused: the planar layout is relative
 * to each matrix's start, so its rows are not where the view's data points. */
typedef struct spiral_tensor {
  int32_t type;
  spiral_buffer* buffer;
  int64_t ne[SPIRAL_MAX_DIMS];
  size_t nb[SPIRAL_MAX_DIMS];
  int32_t op;
  int32_t op_params[SPIRAL_MAX_OP_PARAMS];
  int32_t flags;
  struct spiral_tensor* src[SPIRAL_MAX_SRC];
  struct spiral_tensor* view_src;
  size_t view_offs;
  void* data;
  char name[SPIRAL_MAX_NAME];
} spiral_tensor;

typedef struct spiral_cgraph {
  int32_t n_nodes;
  spiral_tensor** nodes;
} spiral_cgraph;

/* ---- buffer type (ggml_backend_buffer_type_i) ------------------------- */

const char* spiral_buft_name(void);
/* Alignment of tensor data inside a buffer (ggml get_alignment). */
size_t spiral_buft_alignment(void);
/* Largest single buffer (ggml get_max_size). */
size_t spiral_buft_max_size(void);
/* Bytes a tensor occupies (ggml get_alloc_size): ggml_nbytes, unchanged by
 * the planar layout. 0 for an unsupported tensor. */
size_t spiral_buft_alloc_size(const spiral_tensor* t);
/* Allocates `size` bytes of device memory on the current device
 * (ggml alloc_buffer). Returns NULL when size is 0 or allocation fails. */
spiral_buffer* spiral_buft_alloc_buffer(size_t size);

/* ---- buffer (ggml_backend_buffer_i) ------------------------------------ */

void spiral_buffer_free(spiral_buffer* buf);
void* spiral_buffer_get_base(const spiral_buffer* buf);
size_t spiral_buffer_get_size(const spiral_buffer* buf);
/* Checks that the tensor lies inside the buffer, is contiguous in its
 * innermost dimension and, when quantized, has whole rows of blocks and
 * contiguous 2-D matrices (nb[1] == row bytes, nb[2] == ne[1] * nb[1],
 * nb[3] == ne[2] * nb[2]). Sets t->buffer (ggml init_tensor). */
int spiral_buffer_init_tensor(spiral_buffer* buf, spiral_tensor* t);
/* Host -> tensor bytes [offset, offset + size) in canonical (GGUF) byte order
 * (ggml set_tensor). Quantized tensors are converted to planar on the device;
 * any byte range is accepted. Synchronous. */
int spiral_buffer_set_tensor(spiral_buffer* buf, spiral_tensor* t, const void* data, size_t offset, size_t size);
/* Tensor bytes [offset, offset + size) -> host, in canonical byte order
 * (ggml get_tensor). Synchronous. */
int spiral_buffer_get_tensor(spiral_buffer* buf, const spiral_tensor* t, void* data, size_t offset, size_t size);
/* Sets tensor bytes [offset, offset + size) to `value` (ggml memset_tensor).
 * A constant byte pattern is the same in both layouts. */
int spiral_buffer_memset_tensor(spiral_buffer* buf, spiral_tensor* t, uint8_t value, size_t offset, size_t size);
/* Sets the whole buffer to `value` (ggml clear). */
int spiral_buffer_clear(spiral_buffer* buf, uint8_t value);

/* ---- device (ggml_backend_device_i) -------------------------------------- */

/* 1 when graph_compute can run node `op` (ggml supports_op); pure host
 * logic, no device needed:
 *   MUL_MAT     src0 Q4_0/Q8_0/Q6_K in a spiral buffer (2-D matrices, planar,
 *               ne[2], ne[3] dividing src1's), src1 F32 or BF16 with
 *               contiguous rows, dst F32 [ne0 = src0 ne1, ne1 = src1 ne1, ...];
 *   GET_ROWS    src0 quantized, src1 I32 [n_rows_out, ne02, ne03], dst F32 or
 *               BF16 with contiguous rows;
 *   MUL_MAT_ID  src0 quantized [k, n, n_expert], src1 F32/BF16
 *               [k, x_slots (1 or top_k), n_tokens], src2 I32 [top_k,
 *               n_tokens], dst F32 [n, top_k, n_tokens], all contiguous;
 *   GLU         dst F32 [F, ...]; src0 F32 [2F, ...] and no src1 (the
 *               single-tensor form), or src0 and src1 F32 [F, ...] (the
 *               split form), all of one outer shape with contiguous, evenly
 *               strided rows; op_params[0] REGLU / GEGLU / SWIGLU /
 *               SWIGLU_OAI (alpha and limit as floats in op_params[2] and
 *               [3]) / GEGLU_ERF / GEGLU_QUICK, op_params[1] 0 or 1;
 *   NONE, VIEW, RESHAPE, PERMUTE, TRANSPOSE.
 * Row lengths must be multiples of the type's block (32, Q6_K 256). */
int spiral_supports_op(const spiral_tensor* op);

/* ---- backend (ggml_backend_i) -------------------------------------------- */

/* Binds HIP device `device` and creates the backend's stream (default
 * priority). NULL when the device does not exist. */
spiral_backend* spiral_backend_init(int device);
void spiral_backend_free(spiral_backend* be);
const char* spiral_backend_name(const spiral_backend* be);
/* The backend's hipStream_t (for callers that interleave their own work). */
void* spiral_backend_stream(const spiral_backend* be);
/* Runs the graph's nodes in order on the backend's stream (ggml
 * graph_compute). Fails with SPIRAL_ERR_TYPE, before launching anything, if
 * a node is not supported; device scratch (bf16 copies of F32 activations,
 * MUL_MAT_ID routing lists) is owned by the backend and grows on demand.
 * A MUL_MAT_ID node followed by a GLU node over it runs as one fused pass
 * (spiral_mul_mat_id_glu) when no other node reads the MUL_MAT_ID result,
 * it is not flagged OUTPUT, the GLU output is contiguous and
 * spiral_mul_mat_id_glu_fits() holds for its shape; the MUL_MAT_ID's own data
 * is then not written, as with ggml's fusion. Only the graph passed in is
 * searched for other readers: a caller that splits a model graph (ggml's
 * scheduler) must flag OUTPUT every MUL_MAT_ID result read in another split.
 * Asynchronous: returns when the work is queued. */
int spiral_backend_graph_compute(spiral_backend* be, const spiral_cgraph* graph);
/* Waits for the backend's stream (ggml synchronize). */
int spiral_backend_synchronize(spiral_backend* be);

#ifdef __cplusplus
}
#endif

#endif /* SPIRAL_GGML_H */
