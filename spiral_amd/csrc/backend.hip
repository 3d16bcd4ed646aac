// ggml-backend-shaped surface (include/spiral_ggml.h): buffers that keep
// quantized tensors in the planar device layout behind a canonical-bytes
// set/get interface, supports_op, and graph_compute for MUL_MAT / GET_ROWS /
// MUL_MAT_ID with quantized src0, and GLU (fused into the MUL_MAT_ID it
// follows when nothing else reads that product).
//
// The reference only names this layer (README.md:11-14; the repack headers
// are meant to be compiled into a llama.cpp loader, src/quants/common/
// repack.h:5-7): set_tensor's canonical -> planar conversion is this
// library's counterpart of that load-time repack.
#include <algorithm>
#include <cstring>
#include <new>

#include "common.h"
#include "spiral_ggml.h"

struct spiral_buffer {
  uint8_t* base;
  size_t size;
  int device;
};

struct spiral_backend {
  int device;
  hipStream_t stream;
  uint8_t* scratch;
  size_t scratch_size;
};

namespace spiral {
namespace {

constexpr size_t kAlign = 256;

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Element (or block) size in bytes and elements per block of a tensor type.
bool type_info(int type, size_t& bytes, int64_t& blck) {
  switch (type) {
    case SPIRAL_TYPE_F32: bytes = 4; blck = 1; return true;
    case SPIRAL_TYPE_F16: bytes = 2; blck = 1; return true;
    case SPIRAL_TYPE_BF16: bytes = 2; blck = 1; return true;
    case SPIRAL_TYPE_I32: bytes = 4; blck = 1; return true;
    case SPIRAL_TYPE_Q4_0: bytes = kQ4_0Bytes; blck = kQ4_0Elems; return true;
    case SPIRAL_TYPE_Q8_0: bytes = kQ8_0Bytes; blck = kQ8_0Elems; return true;
    case SPIRAL_TYPE_Q6_K: bytes = kQ6_KBytes; blck = kQ6_KElems; return true;
    case SPIRAL_TYPE_Q4_K: bytes = kQ4_KBytes; blck = 256; return true;
    case SPIRAL_TYPE_Q5_K: bytes = kQ5_KBytes; blck = 256; return true;
    case SPIRAL_TYPE_IQ4_NL: bytes = kIQ4_NLBytes; blck = 32; return true;
    case SPIRAL_TYPE_IQ4_XS: bytes = kIQ4_XSBytes; blck = 256; return true;
    default: return false;
  }
}

// ggml_nbytes.
size_t nbytes(const spiral_tensor* t) {
  size_t ts;
  int64_t blck;
  if (!type_info(t->type, ts, blck)) return 0;
  for (int i = 0; i < SPIRAL_MAX_DIMS; ++i)
    if (t->ne[i] <= 0) return 0;
  size_t n = blck == 1 ? ts : static_cast<size_t>(t->ne[0]) * t->nb[0] / static_cast<size_t>(blck);
  if (blck == 1)
    for (int i = 0; i < SPIRAL_MAX_DIMS; ++i) n += static_cast<size_t>(t->ne[i] - 1) * t->nb[i];
  else
    for (int i = 1; i < SPIRAL_MAX_DIMS; ++i) n += static_cast<size_t>(t->ne[i] - 1) * t->nb[i];
  return n;
}

bool is_quant(const spiral_tensor* t) { return is_quant_type(t->type); }

// Quantized tensors must be stacks of contiguous 2-D matrices of whole
// blocks, 16-byte aligned (the planar layout works per matrix).
bool quant_layout_ok(const spiral_tensor* t) {
  const int64_t be = block_elems(t->type), bb = block_bytes(t->type);
  if (t->ne[0] % be != 0) return false;
  const size_t row = static_cast<size_t>(t->ne[0] / be * bb);
  if (t->nb[0] != static_cast<size_t>(bb) || t->nb[1] != row) return false;
  if (t->nb[2] != row * t->ne[1] || t->nb[3] != t->nb[2] * t->ne[2]) return false;
  // Each matrix of a stack starts its own planes: 16-byte aligned.
  if (t->ne[2] * t->ne[3] > 1 && (t->nb[2] & 15) != 0) return false;
  return (reinterpret_cast<uintptr_t>(t->data) & 15) == 0;
}

// A quantized tensor's data must start whole planar matrices: the planar
// layout is relative to each matrix's start. A view (view_src set; ggml
// keeps view_src pointing at the tensor that owns the memory) passes only
// when its matrices are its source's: same row length and row count, at an
// offset of a whole number of source matrices (one expert of a stack, say).
// A row-range view inside a matrix fails.
bool planar_whole(const spiral_tensor* t) {
  if (!quant_layout_ok(t)) return false;
  const spiral_tensor* v = t->view_src;
  if (v == nullptr) return true;
  if (v->type != t->type || v->ne[0] != t->ne[0] || v->ne[1] != t->ne[1] || !quant_layout_ok(v)) return false;
  const size_t mat = v->nb[2];
  if (mat == 0 || t->view_offs % mat != 0) return false;
  return v->data == nullptr || static_cast<const uint8_t*>(v->data) + t->view_offs == t->data;
}

// Element tensor with contiguous innermost dimension.
bool rows_contiguous(const spiral_tensor* t, size_t elem) { return t->nb[0] == elem; }

bool fully_contiguous(const spiral_tensor* t, size_t elem) {
  return t->nb[0] == elem && t->nb[1] == elem * t->ne[0] && t->nb[2] == t->nb[1] * t->ne[1] &&
         t->nb[3] == t->nb[2] * t->ne[2];
}

bool in_spiral_buffer(const spiral_tensor* t) {
  if (t->buffer == nullptr || t->data == nullptr) return false;
  const uint8_t* p = static_cast<const uint8_t*>(t->data);
  return p >= t->buffer->base && p + nbytes(t) <= t->buffer->base + t->buffer->size;
}

bool act_type(int type) { return type == SPIRAL_TYPE_F32 || type == SPIRAL_TYPE_BF16; }

size_t elem_size(int type) { return type == SPIRAL_TYPE_F32 || type == SPIRAL_TYPE_I32 ? 4 : 2; }

// ---- canonical <-> planar at byte granularity ----------------------------
//
// Canonical byte o of a stack of matrices (each `rows` rows of nb blocks of
// bb bytes) -> its planar byte offset.
__host__ __device__ inline int64_t planar_offset(int type, int64_t rows, int64_t nb, int64_t o) {
  const int64_t bb = block_bytes(type);
  const int64_t mat = rows * nb * bb;
  const int64_t i = o / mat, r = o % mat;
  const int64_t blk = r / bb, j = r % bb;  // block index in the matrix, byte in the block
  const int64_t tot = rows * nb;
  int64_t p;
  if (type == SPIRAL_TYPE_Q4_0 || type == SPIRAL_TYPE_IQ4_NL)
    p = j < 2 ? tot * 16 + blk * 2 + j : blk * 16 + (j - 2);
  else if (type == SPIRAL_TYPE_IQ4_XS)
    p = j < 8 ? tot * 128 + blk * 8 + j : blk * 128 + (j - 8);
  else if (type == SPIRAL_TYPE_Q8_0)
    p = j < 2 ? tot * 32 + blk * 2 + j : blk * 32 + (j - 2);
  else if (type == SPIRAL_TYPE_Q4_K)
    p = j < 16 ? tot * 128 + blk * 16 + j : blk * 128 + (j - 16);
  else if (type == SPIRAL_TYPE_Q5_K)
    p = j < 16   ? tot * 160 + blk * 16 + j
        : j < 48 ? tot * 128 + blk * 32 + (j - 16)
                 : blk * 128 + (j - 48);
  else
    p = j < 128   ? blk * 128 + j
        : j < 192 ? tot * 128 + blk * 64 + (j - 128)
        : j < 208 ? tot * 192 + blk * 16 + (j - 192)
                  : tot * 208 + blk * 2 + (j - 208);
  return i * mat + p;
}

__global__ void scatter_kernel(int type, int64_t rows, int64_t nb, int64_t offset, int64_t size,
                               const uint8_t* __restrict__ src, uint8_t* __restrict__ planar) {
  for (int64_t b = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; b < size;
       b += static_cast<int64_t>(gridDim.x) * blockDim.x)
    planar[planar_offset(type, rows, nb, offset + b)] = src[b];
}

__global__ void gather_kernel(int type, int64_t rows, int64_t nb, int64_t offset, int64_t size,
                              const uint8_t* __restrict__ planar, uint8_t* __restrict__ dst) {
  for (int64_t b = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; b < size;
       b += static_cast<int64_t>(gridDim.x) * blockDim.x)
    dst[b] = planar[planar_offset(type, rows, nb, offset + b)];
}

// Activation rows (F32 or BF16, any row / batch strides) -> contiguous bf16
// [n3][n2][n1][n0], round to nearest even.
template <bool F32>
__global__ void to_bf16_kernel(const uint8_t* __restrict__ src, int64_t n0, int64_t n1, int64_t n2, int64_t n3,
                               int64_t s1, int64_t s2, int64_t s3, uint16_t* __restrict__ dst) {
  const int64_t total = n0 * n1 * n2 * n3;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t i0 = i % n0, r = i / n0;
    const int64_t i1 = r % n1, r2 = r / n1;
    const int64_t i2 = r2 % n2, i3 = r2 / n2;
    const uint8_t* p = src + i1 * s1 + i2 * s2 + i3 * s3;
    if constexpr (F32) {
      const float v = reinterpret_cast<const float*>(p)[i0];
      __bf16 b = static_cast<__bf16>(v);
      dst[i] = __builtin_bit_cast(uint16_t, b);
    } else {
      dst[i] = reinterpret_cast<const uint16_t*>(p)[i0];
    }
  }
}

unsigned grid_for(int64_t n) {
  return static_cast<unsigned>(std::min<int64_t>(std::max<int64_t>(ceil_div(n, 256), 1), 65536));
}

int hip_rc(hipError_t e) {
  if (e == hipSuccess) return SPIRAL_OK;
  (void)hipGetLastError();
  return SPIRAL_ERR_HIP;
}

// Bytes of bf16 activations a node needs converted into scratch (0 if its
// src1 can be used in place).
size_t act_scratch(const spiral_tensor* b) {
  if (b->type == SPIRAL_TYPE_BF16 && b->nb[1] % 16 == 0 && (reinterpret_cast<uintptr_t>(b->data) & 15) == 0 &&
      b->nb[2] % 16 == 0 && b->nb[3] % 16 == 0)
    return 0;
  return align_up(static_cast<size_t>(b->ne[0] * b->ne[1] * b->ne[2] * b->ne[3]) * 2, kAlign);
}

// Workspace of one MUL_MAT product (the batch's matrices run one after
// another on the backend's stream and share it).
size_t mul_mat_workspace(const spiral_tensor* t) {
  const spiral_tensor* a = t->src[0];
  const int64_t n = spiral_mul_mat_workspace_bytes(a->type, a->ne[1], a->ne[0], t->src[1]->ne[1]);
  return align_up(static_cast<size_t>(n > 0 ? n : 0), kAlign);
}

size_t node_scratch(const spiral_tensor* t) {
  switch (t->op) {
    case SPIRAL_OP_MUL_MAT: return act_scratch(t->src[1]) + mul_mat_workspace(t);
    case SPIRAL_OP_MUL_MAT_ID: {
      const spiral_tensor* b = t->src[1];
      const spiral_tensor* ids = t->src[2];
      size_t need = align_up(static_cast<size_t>(b->ne[0] * b->ne[1] * b->ne[2]) * 2, kAlign);
      need += align_up(static_cast<size_t>(spiral_mul_mat_id_workspace_bytes(t->src[0]->ne[2], ids->ne[1], ids->ne[0])),
                       kAlign);
      return need;
    }
    default: return 0;
  }
}

// Activations of `b` as bf16: in place when possible, else converted into
// `scratch` (contiguous). Returns the pointer and its element strides.
const uint16_t* act_bf16(const spiral_tensor* b, uint8_t* scratch, bool force_contig, hipStream_t s, int64_t& ld1,
                         int64_t& ld2, int64_t& ld3, int& rc) {
  rc = SPIRAL_OK;
  if (!force_contig && act_scratch(b) == 0) {
    ld1 = static_cast<int64_t>(b->nb[1] / 2);
    ld2 = static_cast<int64_t>(b->nb[2] / 2);
    ld3 = static_cast<int64_t>(b->nb[3] / 2);
    return static_cast<const uint16_t*>(b->data);
  }
  if (force_contig && b->type == SPIRAL_TYPE_BF16 && fully_contiguous(b, 2) &&
      (reinterpret_cast<uintptr_t>(b->data) & 15) == 0) {
    ld1 = b->ne[0];
    ld2 = b->ne[0] * b->ne[1];
    ld3 = ld2 * b->ne[2];
    return static_cast<const uint16_t*>(b->data);
  }
  uint16_t* dst = reinterpret_cast<uint16_t*>(scratch);
  const int64_t total = b->ne[0] * b->ne[1] * b->ne[2] * b->ne[3];
  const uint8_t* src = static_cast<const uint8_t*>(b->data);
  const int64_t s1 = static_cast<int64_t>(b->nb[1]), s2 = static_cast<int64_t>(b->nb[2]), s3 = static_cast<int64_t>(b->nb[3]);
  if (b->type == SPIRAL_TYPE_F32)
    hipLaunchKernelGGL(to_bf16_kernel<true>, dim3(grid_for(total)), dim3(256), 0, s, src, b->ne[0], b->ne[1], b->ne[2],
                       b->ne[3], s1, s2, s3, dst);
  else
    hipLaunchKernelGGL(to_bf16_kernel<false>, dim3(grid_for(total)), dim3(256), 0, s, src, b->ne[0], b->ne[1], b->ne[2],
                       b->ne[3], s1, s2, s3, dst);
  rc = launch_status();
  ld1 = b->ne[0];
  ld2 = b->ne[0] * b->ne[1];
  ld3 = ld2 * b->ne[2];
  return dst;
}

int compute_mul_mat(spiral_backend* be, const spiral_tensor* t) {
  const spiral_tensor* a = t->src[0];
  const spiral_tensor* b = t->src[1];
  int rc;
  int64_t ld1, ld2, ld3;
  const uint16_t* xb = act_bf16(b, be->scratch, false, be->stream, ld1, ld2, ld3, rc);
  if (rc != SPIRAL_OK) return rc;
  const int64_t r2 = b->ne[2] / a->ne[2], r3 = b->ne[3] / a->ne[3];
  uint8_t* ws = be->scratch + act_scratch(b);
  const int64_t wsb = static_cast<int64_t>(mul_mat_workspace(t));
  for (int64_t i3 = 0; i3 < b->ne[3]; ++i3) {
    for (int64_t i2 = 0; i2 < b->ne[2]; ++i2) {
      const uint8_t* w = static_cast<const uint8_t*>(a->data) + (i2 / r2) * a->nb[2] + (i3 / r3) * a->nb[3];
      const uint16_t* x = xb + i2 * ld2 + i3 * ld3;
      uint8_t* y = static_cast<uint8_t*>(t->data) + i2 * t->nb[2] + i3 * t->nb[3];
      rc = spiral_mul_mat(a->type, w, a->ne[1], a->ne[0], x, ld1, b->ne[1], y, SPIRAL_TYPE_F32,
                          static_cast<int64_t>(t->nb[1] / 4), wsb > 0 ? ws : nullptr, wsb, be->stream);
      if (rc != SPIRAL_OK) return rc;
    }
  }
  return SPIRAL_OK;
}

int compute_get_rows(spiral_backend* be, const spiral_tensor* t) {
  const spiral_tensor* a = t->src[0];
  const spiral_tensor* ids = t->src[1];
  const size_t es = elem_size(t->type);
  for (int64_t i2 = 0; i2 < ids->ne[2]; ++i2) {
    for (int64_t i1 = 0; i1 < ids->ne[1]; ++i1) {
      const uint8_t* w = static_cast<const uint8_t*>(a->data) + i1 * a->nb[2] + i2 * a->nb[3];
      const int32_t* id = reinterpret_cast<const int32_t*>(static_cast<const uint8_t*>(ids->data) + i1 * ids->nb[1] +
                                                           i2 * ids->nb[2]);
      uint8_t* out = static_cast<uint8_t*>(t->data) + i1 * t->nb[2] + i2 * t->nb[3];
      const int rc = spiral_get_rows(a->type, w, a->ne[1], a->ne[0], id, ids->ne[0], out, t->type,
                                     static_cast<int64_t>(t->nb[1] / es), be->stream);
      if (rc != SPIRAL_OK) return rc;
    }
  }
  return SPIRAL_OK;
}

int compute_mul_mat_id(spiral_backend* be, const spiral_tensor* t) {
  const spiral_tensor* a = t->src[0];
  const spiral_tensor* b = t->src[1];
  const spiral_tensor* ids = t->src[2];
  int rc;
  int64_t ld1, ld2, ld3;
  const uint16_t* x = act_bf16(b, be->scratch, true, be->stream, ld1, ld2, ld3, rc);
  if (rc != SPIRAL_OK) return rc;
  const size_t xbytes = align_up(static_cast<size_t>(b->ne[0] * b->ne[1] * b->ne[2]) * 2, kAlign);
  const int64_t wsb = spiral_mul_mat_id_workspace_bytes(a->ne[2], ids->ne[1], ids->ne[0]);
  return spiral_mul_mat_id(a->type, a->data, static_cast<int64_t>(a->nb[2]), a->ne[2], a->ne[1], a->ne[0], x,
                           b->ne[1], static_cast<const int32_t*>(ids->data), ids->ne[1], ids->ne[0], t->data,
                           SPIRAL_TYPE_F32, be->scratch + xbytes, wsb, be->stream);
}

// MUL_MAT_ID node t with the GLU node g over it as one pass: g's data
// receives act(gate) * up directly.
int compute_mul_mat_id_glu(spiral_backend* be, const spiral_tensor* t, const spiral_tensor* g) {
  const spiral_tensor* a = t->src[0];
  const spiral_tensor* b = t->src[1];
  const spiral_tensor* ids = t->src[2];
  int rc;
  int64_t ld1, ld2, ld3;
  const uint16_t* x = act_bf16(b, be->scratch, true, be->stream, ld1, ld2, ld3, rc);
  if (rc != SPIRAL_OK) return rc;
  const size_t xbytes = align_up(static_cast<size_t>(b->ne[0] * b->ne[1] * b->ne[2]) * 2, kAlign);
  const int64_t wsb = spiral_mul_mat_id_workspace_bytes(a->ne[2], ids->ne[1], ids->ne[0]);
  return spiral_mul_mat_id_glu(a->type, a->data, static_cast<int64_t>(a->nb[2]), a->ne[2], a->ne[1], a->ne[0], x,
                               b->ne[1], static_cast<const int32_t*>(ids->data), ids->ne[1], ids->ne[0],
                               g->op_params[0], g->op_params[1], g->data, SPIRAL_TYPE_F32, be->scratch + xbytes, wsb,
                               be->stream);
}

// GLU over rows of src0, or of src0 and src1 (split form); contiguous outer
// dimensions, checked by supports_op. As in ggml, op_params[1] (swapped)
// applies to the single-tensor form only: the split form always activates
// src0 (ggml_glu_split sets it to 0, and ggml's kernels ignore it there).
int compute_glu(spiral_backend* be, const spiral_tensor* t) {
  const spiral_tensor* a = t->src[0];
  const spiral_tensor* b2 = t->src[1];
  const int64_t rows = t->ne[1] * t->ne[2] * t->ne[3];
  if (t->op_params[0] == SPIRAL_GLU_SWIGLU_OAI) {
    // ggml keeps alpha and limit as floats in op_params[2] and [3].
    float alpha, limit;
    std::memcpy(&alpha, &t->op_params[2], sizeof alpha);
    std::memcpy(&limit, &t->op_params[3], sizeof limit);
    if (b2 != nullptr)
      return spiral_glu_split_swiglu_oai(0, alpha, limit, static_cast<const float*>(a->data),
                                         static_cast<int64_t>(a->nb[1] / 4), static_cast<const float*>(b2->data),
                                         static_cast<int64_t>(b2->nb[1] / 4), t->ne[0], rows,
                                         static_cast<float*>(t->data), static_cast<int64_t>(t->nb[1] / 4), be->stream);
    return spiral_glu_swiglu_oai(t->op_params[1], alpha, limit, static_cast<const float*>(a->data),
                                 static_cast<int64_t>(a->nb[1] / 4), t->ne[0], rows, static_cast<float*>(t->data),
                                 static_cast<int64_t>(t->nb[1] / 4), be->stream);
  }
  if (b2 != nullptr)
    return spiral_glu_split(t->op_params[0], 0, static_cast<const float*>(a->data),
                            static_cast<int64_t>(a->nb[1] / 4), static_cast<const float*>(b2->data),
                            static_cast<int64_t>(b2->nb[1] / 4), t->ne[0], rows, static_cast<float*>(t->data),
                            static_cast<int64_t>(t->nb[1] / 4), be->stream);
  return spiral_glu(t->op_params[0], t->op_params[1], static_cast<const float*>(a->data),
                    static_cast<int64_t>(a->nb[1] / 4), t->ne[0], rows, static_cast<float*>(t->data),
                    static_cast<int64_t>(t->nb[1] / 4), be->stream);
}

// ggml's split form fused: MUL_MAT_ID over the gate experts (g->src[0]) and
// over the up experts (g->src[1]), same activations and ids, then GLU g
// (the gate activated, whatever op_params[1] holds, as in compute_glu).
int compute_mul_mat_id_glu_split(spiral_backend* be, const spiral_tensor* g) {
  const spiral_tensor* tg = g->src[0];
  const spiral_tensor* tu = g->src[1];
  const spiral_tensor* a = tg->src[0];
  const spiral_tensor* b = tg->src[1];
  const spiral_tensor* ids = tg->src[2];
  int rc;
  int64_t ld1, ld2, ld3;
  const uint16_t* x = act_bf16(b, be->scratch, true, be->stream, ld1, ld2, ld3, rc);
  if (rc != SPIRAL_OK) return rc;
  const size_t xbytes = align_up(static_cast<size_t>(b->ne[0] * b->ne[1] * b->ne[2]) * 2, kAlign);
  const int64_t wsb = spiral_mul_mat_id_workspace_bytes(a->ne[2], ids->ne[1], ids->ne[0]);
  return spiral_mul_mat_id_glu_split(a->type, a->data, tu->src[0]->data, static_cast<int64_t>(a->nb[2]), a->ne[2],
                                     a->ne[1], a->ne[0], x, b->ne[1], static_cast<const int32_t*>(ids->data),
                                     ids->ne[1], ids->ne[0], g->op_params[0], 0, g->data, SPIRAL_TYPE_F32,
                                     be->scratch + xbytes, wsb, be->stream);
}

// Node i (MUL_MAT_ID) can run fused with node i + 1 (GLU over it): nothing
// else in the graph reads node i, it is not a graph output, the fused pass
// covers its shape, and the GLU output is contiguous (the fused pass writes
// it as packed [pair][F] rows).
bool fusable_glu(const spiral_cgraph* graph, int32_t i) {
  if (i + 1 >= graph->n_nodes) return false;
  const spiral_tensor* t = graph->nodes[i];
  const spiral_tensor* g = graph->nodes[i + 1];
  if (t->op != SPIRAL_OP_MUL_MAT_ID || g->op != SPIRAL_OP_GLU || g->src[0] != t || g->src[1] != nullptr) return false;
  if (g->op_params[0] == SPIRAL_GLU_SWIGLU_OAI) return false;  // runs unfused (its own GLU entry point)
  if ((t->flags & SPIRAL_TENSOR_FLAG_OUTPUT) != 0 || !fully_contiguous(g, 4)) return false;
  const spiral_tensor* a = t->src[0];
  if (!spiral_mul_mat_id_glu_fits(a->type, a->ne[1], a->ne[0])) return false;
  for (int32_t j = 0; j < graph->n_nodes; ++j) {
    if (j == i + 1) continue;
    for (int s = 0; s < SPIRAL_MAX_SRC; ++s)
      if (graph->nodes[j]->src[s] == t) return false;
  }
  return true;
}

// Nodes i and i + 1 (MUL_MAT_ID, either order) and i + 2 (split GLU over
// both) can run as one pass: the two products share activations and ids,
// their expert stacks have one type, shape and stride, neither product is a
// graph output or read by any other node, the fused pass covers the shape,
// and the GLU output is contiguous.
bool fusable_glu_split(const spiral_cgraph* graph, int32_t i) {
  if (i + 2 >= graph->n_nodes) return false;
  const spiral_tensor* t0 = graph->nodes[i];
  const spiral_tensor* t1 = graph->nodes[i + 1];
  const spiral_tensor* g = graph->nodes[i + 2];
  if (t0->op != SPIRAL_OP_MUL_MAT_ID || t1->op != SPIRAL_OP_MUL_MAT_ID || g->op != SPIRAL_OP_GLU) return false;
  if (g->op_params[0] == SPIRAL_GLU_SWIGLU_OAI) return false;  // runs unfused (its own GLU entry point)
  if (g->src[1] == nullptr || !((g->src[0] == t0 && g->src[1] == t1) || (g->src[0] == t1 && g->src[1] == t0)))
    return false;
  if (((t0->flags | t1->flags) & SPIRAL_TENSOR_FLAG_OUTPUT) != 0 || !fully_contiguous(g, 4)) return false;
  if (t0->src[1] != t1->src[1] || t0->src[2] != t1->src[2]) return false;
  const spiral_tensor* a0 = t0->src[0];
  const spiral_tensor* a1 = t1->src[0];
  if (a0->type != a1->type || a0->nb[2] != a1->nb[2]) return false;
  for (int d = 0; d < 3; ++d)
    if (a0->ne[d] != a1->ne[d]) return false;
  if (a0->ne[1] > INT64_MAX / 2 || !spiral_mul_mat_id_glu_fits(a0->type, 2 * a0->ne[1], a0->ne[0])) return false;
  for (int32_t j = 0; j < graph->n_nodes; ++j) {
    if (j == i + 2) continue;
    for (int s = 0; s < SPIRAL_MAX_SRC; ++s)
      if (graph->nodes[j]->src[s] == t0 || graph->nodes[j]->src[s] == t1) return false;
  }
  return true;
}

int grow_scratch(spiral_backend* be, size_t need) {
  if (need <= be->scratch_size) return SPIRAL_OK;
  int rc = hip_rc(hipStreamSynchronize(be->stream));
  if (rc != SPIRAL_OK) return rc;
  if (be->scratch != nullptr) (void)hipFree(be->scratch);
  be->scratch = nullptr;
  be->scratch_size = 0;
  void* p = nullptr;
  rc = hip_rc(hipMalloc(&p, need));
  if (rc != SPIRAL_OK) return rc;
  be->scratch = static_cast<uint8_t*>(p);
  be->scratch_size = need;
  return SPIRAL_OK;
}

// Runs on the device that owns `buf`, restoring the caller's device.
struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) (void)hipSetDevice(dev);
  }
  ~DeviceGuard() {
    if (prev >= 0) (void)hipSetDevice(prev);
  }
};

int check_range(const spiral_buffer* buf, const spiral_tensor* t, size_t offset, size_t size) {
  if (buf == nullptr || t == nullptr) return SPIRAL_ERR_NULL;
  const size_t n = nbytes(t);
  if (n == 0) return SPIRAL_ERR_TYPE;
  if (offset > n || size > n - offset) return SPIRAL_ERR_RANGE;
  const uint8_t* p = static_cast<const uint8_t*>(t->data);
  if (p < buf->base || p + n > buf->base + buf->size) return SPIRAL_ERR_RANGE;
  return SPIRAL_OK;
}

}  // namespace
}  // namespace spiral

using namespace spiral;

extern "C" {

const char* spiral_buft_name(void) { return "SPIRAL_MI355X"; }
size_t spiral_buft_alignment(void) { return kAlign; }
size_t spiral_buft_max_size(void) { return SIZE_MAX; }

size_t spiral_buft_alloc_size(const spiral_tensor* t) { return t == nullptr ? 0 : nbytes(t); }

spiral_buffer* spiral_buft_alloc_buffer(size_t size) {
  if (size == 0 || require_device() != SPIRAL_OK) return nullptr;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  void* p = nullptr;
  if (hipMalloc(&p, size) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  spiral_buffer* b = new (std::nothrow) spiral_buffer{static_cast<uint8_t*>(p), size, dev};
  if (b == nullptr) (void)hipFree(p);
  return b;
}

void spiral_buffer_free(spiral_buffer* buf) {
  if (buf == nullptr) return;
  DeviceGuard g(buf->device);
  (void)hipFree(buf->base);
  delete buf;
}

void* spiral_buffer_get_base(const spiral_buffer* buf) { return buf == nullptr ? nullptr : buf->base; }
size_t spiral_buffer_get_size(const spiral_buffer* buf) { return buf == nullptr ? 0 : buf->size; }

int spiral_buffer_init_tensor(spiral_buffer* buf, spiral_tensor* t) {
  if (buf == nullptr || t == nullptr || t->data == nullptr) return SPIRAL_ERR_NULL;
  const size_t n = nbytes(t);
  if (n == 0) return SPIRAL_ERR_TYPE;
  const uint8_t* p = static_cast<const uint8_t*>(t->data);
  if (p < buf->base || p + n > buf->base + buf->size) return SPIRAL_ERR_RANGE;
  if (is_quant(t)) {
    if (!quant_layout_ok(t)) return SPIRAL_ERR_SHAPE;
  } else if (!rows_contiguous(t, elem_size(t->type))) {
    return SPIRAL_ERR_SHAPE;
  }
  t->buffer = buf;
  return SPIRAL_OK;
}

int spiral_buffer_set_tensor(spiral_buffer* buf, spiral_tensor* t, const void* data, size_t offset, size_t size) {
  int rc = check_range(buf, t, offset, size);
  if (rc != SPIRAL_OK) return rc;
  if (size == 0) return SPIRAL_OK;
  if (data == nullptr) return SPIRAL_ERR_NULL;
  DeviceGuard g(buf->device);
  uint8_t* dst = static_cast<uint8_t*>(t->data);
  if (!is_quant(t)) return hip_rc(hipMemcpy(dst + offset, data, size, hipMemcpyHostToDevice));
  if (!planar_whole(t)) return SPIRAL_ERR_SHAPE;
  void* stage = nullptr;
  if ((rc = hip_rc(hipMalloc(&stage, size))) != SPIRAL_OK) return rc;
  rc = hip_rc(hipMemcpy(stage, data, size, hipMemcpyHostToDevice));
  const int64_t rows = t->ne[1], k = t->ne[0], nb = k / block_elems(t->type);
  const size_t mat = t->nb[2];
  if (rc == SPIRAL_OK) {
    if (offset % mat == 0 && size % mat == 0) {
      // Whole matrices: the block-parallel conversion, one call per matrix.
      for (size_t o = 0; o < size && rc == SPIRAL_OK; o += mat)
        rc = spiral_to_planar(t->type, static_cast<uint8_t*>(stage) + o, static_cast<int64_t>(t->nb[1]), rows, k,
                              dst + offset + o, nullptr);
    } else {
      hipLaunchKernelGGL(scatter_kernel, dim3(grid_for(static_cast<int64_t>(size))), dim3(256), 0, 0, t->type, rows,
                         nb, static_cast<int64_t>(offset), static_cast<int64_t>(size),
                         static_cast<const uint8_t*>(stage), dst);
      rc = launch_status();
    }
  }
  if (rc == SPIRAL_OK) rc = hip_rc(hipDeviceSynchronize());
  (void)hipFree(stage);
  return rc;
}

int spiral_buffer_get_tensor(spiral_buffer* buf, const spiral_tensor* t, void* data, size_t offset, size_t size) {
  int rc = check_range(buf, t, offset, size);
  if (rc != SPIRAL_OK) return rc;
  if (size == 0) return SPIRAL_OK;
  if (data == nullptr) return SPIRAL_ERR_NULL;
  DeviceGuard g(buf->device);
  const uint8_t* src = static_cast<const uint8_t*>(t->data);
  if (!is_quant(t)) return hip_rc(hipMemcpy(data, src + offset, size, hipMemcpyDeviceToHost));
  if (!planar_whole(t)) return SPIRAL_ERR_SHAPE;
  void* stage = nullptr;
  if ((rc = hip_rc(hipMalloc(&stage, size))) != SPIRAL_OK) return rc;
  const int64_t rows = t->ne[1], k = t->ne[0], nb = k / block_elems(t->type);
  const size_t mat = t->nb[2];
  if (offset % mat == 0 && size % mat == 0) {
    for (size_t o = 0; o < size && rc == SPIRAL_OK; o += mat)
      rc = spiral_from_planar(t->type, src + offset + o, rows, k, static_cast<uint8_t*>(stage) + o,
                              static_cast<int64_t>(t->nb[1]), nullptr);
  } else {
    hipLaunchKernelGGL(gather_kernel, dim3(grid_for(static_cast<int64_t>(size))), dim3(256), 0, 0, t->type, rows, nb,
                       static_cast<int64_t>(offset), static_cast<int64_t>(size), src, static_cast<uint8_t*>(stage));
    rc = launch_status();
  }
  if (rc == SPIRAL_OK) rc = hip_rc(hipDeviceSynchronize());
  if (rc == SPIRAL_OK) rc = hip_rc(hipMemcpy(data, stage, size, hipMemcpyDeviceToHost));
  (void)hipFree(stage);
  return rc;
}

int spiral_buffer_memset_tensor(spiral_buffer* buf, spiral_tensor* t, uint8_t value, size_t offset, size_t size) {
  const int rc = check_range(buf, t, offset, size);
  if (rc != SPIRAL_OK) return rc;
  if (size == 0) return SPIRAL_OK;
  DeviceGuard g(buf->device);
  // A constant byte range maps to constant planar bytes only when it covers
  // whole matrices; otherwise scatter it like set_tensor would.
  if (is_quant(t) && !planar_whole(t)) return SPIRAL_ERR_SHAPE;
  if (is_quant(t) && !(offset % t->nb[2] == 0 && size % t->nb[2] == 0)) {
    uint8_t* host = new (std::nothrow) uint8_t[size];
    if (host == nullptr) return SPIRAL_ERR_CAPACITY;
    std::memset(host, value, size);
    const int r = spiral_buffer_set_tensor(buf, t, host, offset, size);
    delete[] host;
    return r;
  }
  const int r = hip_rc(hipMemset(static_cast<uint8_t*>(t->data) + offset, value, size));
  return r != SPIRAL_OK ? r : hip_rc(hipDeviceSynchronize());
}

int spiral_buffer_clear(spiral_buffer* buf, uint8_t value) {
  if (buf == nullptr) return SPIRAL_ERR_NULL;
  DeviceGuard g(buf->device);
  const int r = hip_rc(hipMemset(buf->base, value, buf->size));
  return r != SPIRAL_OK ? r : hip_rc(hipDeviceSynchronize());
}

int spiral_supports_op(const spiral_tensor* t) {
  if (t == nullptr) return 0;
  switch (t->op) {
    case SPIRAL_OP_NONE:
    case SPIRAL_OP_VIEW:
    case SPIRAL_OP_RESHAPE:
    case SPIRAL_OP_PERMUTE:
    case SPIRAL_OP_TRANSPOSE:
      return 1;
    case SPIRAL_OP_MUL_MAT: {
      const spiral_tensor* a = t->src[0];
      const spiral_tensor* b = t->src[1];
      if (a == nullptr || b == nullptr || !is_quant(a) || !planar_whole(a) || !in_spiral_buffer(a)) return 0;
      if (!act_type(b->type) || !rows_contiguous(b, elem_size(b->type))) return 0;
      if (t->type != SPIRAL_TYPE_F32 || !rows_contiguous(t, 4)) return 0;
      if (b->ne[0] != a->ne[0] || t->ne[0] != a->ne[1] || t->ne[1] != b->ne[1]) return 0;
      if (t->ne[2] != b->ne[2] || t->ne[3] != b->ne[3]) return 0;
      if (b->ne[2] % a->ne[2] != 0 || b->ne[3] % a->ne[3] != 0) return 0;
      if (t->nb[1] % 4 != 0 || (reinterpret_cast<uintptr_t>(t->data) & 3) != 0) return 0;
      return 1;
    }
    case SPIRAL_OP_GET_ROWS: {
      const spiral_tensor* a = t->src[0];
      const spiral_tensor* ids = t->src[1];
      if (a == nullptr || ids == nullptr || !is_quant(a) || !planar_whole(a) || !in_spiral_buffer(a)) return 0;
      if (ids->type != SPIRAL_TYPE_I32 || !rows_contiguous(ids, 4) || ids->ne[3] != 1) return 0;
      if (ids->ne[1] != a->ne[2] || ids->ne[2] != a->ne[3]) return 0;
      if (!act_type(t->type) || !rows_contiguous(t, elem_size(t->type))) return 0;
      if (t->ne[0] != a->ne[0] || t->ne[1] != ids->ne[0] || t->ne[2] != ids->ne[1] || t->ne[3] != ids->ne[2]) return 0;
      if (t->nb[1] % 16 != 0 || t->nb[2] % 16 != 0 || t->nb[3] % 16 != 0) return 0;
      if ((reinterpret_cast<uintptr_t>(t->data) & 15) != 0 || (reinterpret_cast<uintptr_t>(ids->data) & 3) != 0) return 0;
      return 1;
    }
    case SPIRAL_OP_MUL_MAT_ID: {
      const spiral_tensor* a = t->src[0];
      const spiral_tensor* b = t->src[1];
      const spiral_tensor* ids = t->src[2];
      if (a == nullptr || b == nullptr || ids == nullptr) return 0;
      if (!is_quant(a) || !planar_whole(a) || !in_spiral_buffer(a) || a->ne[3] != 1) return 0;
      if (!act_type(b->type) || !rows_contiguous(b, elem_size(b->type)) || b->ne[3] != 1) return 0;
      if (ids->type != SPIRAL_TYPE_I32 || !fully_contiguous(ids, 4) || ids->ne[2] != 1 || ids->ne[3] != 1) return 0;
      if (t->type != SPIRAL_TYPE_F32 || !fully_contiguous(t, 4)) return 0;
      const int64_t top_k = ids->ne[0], n_tokens = ids->ne[1];
      if (b->ne[0] != a->ne[0] || (b->ne[1] != 1 && b->ne[1] != top_k) || b->ne[2] != n_tokens) return 0;
      if (t->ne[0] != a->ne[1] || t->ne[1] != top_k || t->ne[2] != n_tokens || t->ne[3] != 1) return 0;
      int64_t pairs = 0;
      if (__builtin_mul_overflow(n_tokens, top_k, &pairs) || pairs > INT32_MAX) return 0;
      return 1;
    }
    case SPIRAL_OP_GLU: {
      // Single-tensor form (src[1] NULL: halves of src0) or split form
      // (src0 and src1 of the output's shape).
      const spiral_tensor* a = t->src[0];
      const spiral_tensor* b2 = t->src[1];
      if (a == nullptr) return 0;
      const int32_t op = t->op_params[0], swapped = t->op_params[1];
      if (op != SPIRAL_GLU_REGLU && op != SPIRAL_GLU_GEGLU && op != SPIRAL_GLU_SWIGLU && op != SPIRAL_GLU_GEGLU_ERF &&
          op != SPIRAL_GLU_GEGLU_QUICK && op != SPIRAL_GLU_SWIGLU_OAI)
        return 0;
      if (swapped != 0 && swapped != 1) return 0;
      for (const spiral_tensor* u : {a, b2, t}) {
        if (u == nullptr) continue;
        if (u->type != SPIRAL_TYPE_F32 || !rows_contiguous(u, 4)) return 0;
        // Rows evenly strided across the outer dimensions (one row stride).
        if (u->nb[2] != u->ne[1] * u->nb[1] || u->nb[3] != u->ne[2] * u->nb[2]) return 0;
        if ((reinterpret_cast<uintptr_t>(u->data) & 3) != 0) return 0;
      }
      if (a->ne[0] != (b2 == nullptr ? 2 : 1) * t->ne[0]) return 0;
      for (int d = 0; d < SPIRAL_MAX_DIMS; ++d) {
        if (d > 0 && a->ne[d] != t->ne[d]) return 0;
        if (b2 != nullptr && b2->ne[d] != t->ne[d]) return 0;
      }
      return 1;
    }
    default:
      return 0;
  }
}

spiral_backend* spiral_backend_init(int device) {
  if (device < 0 || device >= spiral_device_count()) return nullptr;
  DeviceGuard g(device);
  hipStream_t s = nullptr;
  if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  spiral_backend* be = new (std::nothrow) spiral_backend{device, s, nullptr, 0};
  if (be == nullptr) (void)hipStreamDestroy(s);
  return be;
}

void spiral_backend_free(spiral_backend* be) {
  if (be == nullptr) return;
  DeviceGuard g(be->device);
  (void)hipStreamSynchronize(be->stream);
  if (be->scratch != nullptr) (void)hipFree(be->scratch);
  (void)hipStreamDestroy(be->stream);
  delete be;
}

const char* spiral_backend_name(const spiral_backend* be) { return be == nullptr ? nullptr : "SPIRAL_MI355X"; }

void* spiral_backend_stream(const spiral_backend* be) { return be == nullptr ? nullptr : be->stream; }

int spiral_backend_graph_compute(spiral_backend* be, const spiral_cgraph* graph) {
  if (be == nullptr || graph == nullptr) return SPIRAL_ERR_NULL;
  if (graph->n_nodes > 0 && graph->nodes == nullptr) return SPIRAL_ERR_NULL;
  size_t need = 0;
  for (int32_t i = 0; i < graph->n_nodes; ++i) {
    const spiral_tensor* t = graph->nodes[i];
    if (t == nullptr) return SPIRAL_ERR_NULL;
    if (!spiral_supports_op(t)) return SPIRAL_ERR_TYPE;
    need = std::max(need, node_scratch(t));
  }
  DeviceGuard g(be->device);
  int rc = grow_scratch(be, need);
  if (rc != SPIRAL_OK) return rc;
  for (int32_t i = 0; i < graph->n_nodes && rc == SPIRAL_OK; ++i) {
    const spiral_tensor* t = graph->nodes[i];
    if (fusable_glu(graph, i)) {
      rc = compute_mul_mat_id_glu(be, t, graph->nodes[i + 1]);
      ++i;
      continue;
    }
    if (fusable_glu_split(graph, i)) {
      rc = compute_mul_mat_id_glu_split(be, graph->nodes[i + 2]);
      i += 2;
      continue;
    }
    switch (t->op) {
      case SPIRAL_OP_MUL_MAT: rc = compute_mul_mat(be, t); break;
      case SPIRAL_OP_GET_ROWS: rc = compute_get_rows(be, t); break;
      case SPIRAL_OP_MUL_MAT_ID: rc = compute_mul_mat_id(be, t); break;
      case SPIRAL_OP_GLU: rc = compute_glu(be, t); break;
      default: break;  // views and no-ops
    }
  }
  return rc;
}

int spiral_backend_synchronize(spiral_backend* be) {
  if (be == nullptr) return SPIRAL_ERR_NULL;
  DeviceGuard g(be->device);
  return hip_rc(hipStreamSynchronize(be->stream));
}

}  // extern "C"
