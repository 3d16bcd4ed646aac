"""Device-tensor wrappers over the C ABI (torch is only the memory/stream
plumbing; all compute runs in libspiral_quants.so).

Every function launches on torch's current HIP stream and returns without
synchronizing. Weight tensors are uint8 device tensors in the library's
planar layout (see to_planar); bf16 data is carried in torch.bfloat16 tensors.
"""

import ctypes

import torch

from ._lib import TYPE_BF16, TYPE_F32, check, lib
from . import BLOCK_ELEMS, row_bytes


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _out_type(dtype):
    if dtype == torch.float32:
        return TYPE_F32
    if dtype == torch.bfloat16:
        return TYPE_BF16
    raise ValueError(f"unsupported output dtype {dtype}")


def _require_cuda(*ts):
    for t in ts:
        if not t.is_cuda:
            raise ValueError("expected a device tensor")


def to_planar(qtype, raw, n_rows, k, row_stride=None):
    """Canonical GGUF rows (uint8 device tensor) -> planar weight tensor."""
    _require_cuda(raw)
    stride = row_bytes(qtype, k) if row_stride is None else row_stride
    out = torch.empty(n_rows * row_bytes(qtype, k), dtype=torch.uint8, device=raw.device)
    check(lib().spiral_to_planar(qtype, _ptr(raw), stride, n_rows, k, _ptr(out), _stream()), "to_planar")
    return out


def from_planar(qtype, planar, n_rows, k, row_stride=None):
    _require_cuda(planar)
    stride = row_bytes(qtype, k) if row_stride is None else row_stride
    out = torch.zeros(n_rows * stride, dtype=torch.uint8, device=planar.device)
    check(lib().spiral_from_planar(qtype, _ptr(planar), n_rows, k, _ptr(out), stride, _stream()), "from_planar")
    return out


def dequant(qtype, w, n_rows, k, out=None):
    """Exact bf16 dequantization -> [n_rows, k] bfloat16."""
    _require_cuda(w)
    if out is None:
        out = torch.empty((n_rows, k), dtype=torch.bfloat16, device=w.device)
    check(lib().spiral_dequant_bf16(qtype, _ptr(w), n_rows, k, _ptr(out), out.stride(0), _stream()), "dequant")
    return out


def get_rows(qtype, w, n_rows, k, ids, out_dtype=torch.float32):
    _require_cuda(w, ids)
    ids = ids.to(torch.int32).contiguous()
    out = torch.empty((ids.numel(), k), dtype=out_dtype, device=w.device)
    check(lib().spiral_get_rows(qtype, _ptr(w), n_rows, k, _ptr(ids), ids.numel(), _ptr(out),
                                _out_type(out_dtype), k, _stream()), "get_rows")
    return out


def mul_mat_workspace(qtype, n_rows, k, m, device):
    """Device workspace for mul_mat (None when the GEMV runs, which needs none)."""
    n = lib().spiral_mul_mat_workspace_bytes(qtype, n_rows, k, m)
    return torch.empty(n, dtype=torch.uint8, device=device) if n > 0 else None


def mul_mat(qtype, w, n_rows, k, x, out_dtype=torch.bfloat16, out=None, workspace=None):
    """y[m, n] = sum_k x[m, k] W[n, k]; x is [m, k] bfloat16 (row stride any
    multiple of 8). workspace: from mul_mat_workspace (allocated here when
    omitted and needed)."""
    _require_cuda(w, x)
    if x.dtype != torch.bfloat16 or x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be a 2-D bfloat16 tensor with contiguous rows")
    m = x.shape[0]
    if out is None:
        out = torch.empty((m, n_rows), dtype=out_dtype, device=w.device)
    if workspace is None:
        workspace = mul_mat_workspace(qtype, n_rows, k, m, w.device)
    ws_ptr, ws_bytes = (None, 0) if workspace is None else (_ptr(workspace), workspace.numel() * workspace.element_size())
    check(lib().spiral_mul_mat(qtype, _ptr(w), n_rows, k, _ptr(x), x.stride(0), m, _ptr(out),
                               _out_type(out.dtype), out.stride(0), ws_ptr, ws_bytes, _stream()), "mul_mat")
    return out


def gemv_relaxed(qtype, w, n_rows, k, x, out_dtype=torch.bfloat16, out=None):
    """The named relaxed single-row product (spiral_gemv_relaxed): the block
    scale multiplies each block's fp32 sum, so weights are not rounded to
    bf16 first. x is [k] (or [1, k]) bfloat16; returns [1, n_rows]."""
    _require_cuda(w, x)
    x = x.reshape(-1)
    if x.dtype != torch.bfloat16 or x.numel() != k or not x.is_contiguous():
        raise ValueError("x must be k contiguous bfloat16 values")
    if out is None:
        out = torch.empty((1, n_rows), dtype=out_dtype, device=w.device)
    check(lib().spiral_gemv_relaxed(qtype, _ptr(w), n_rows, k, _ptr(x), _ptr(out), _out_type(out.dtype),
                                    _stream()), "gemv_relaxed")
    return out


def mul_mat_id_workspace(n_expert, n_tokens, top_k, device):
    n = lib().spiral_mul_mat_id_workspace_bytes(n_expert, n_tokens, top_k)
    return torch.empty(max(n, 16), dtype=torch.uint8, device=device)


def mul_mat_id(qtype, w, expert_stride, n_expert, n_rows, k, x, ids, out_dtype=torch.bfloat16,
               workspace=None, out=None):
    """y[t, s] = W[ids[t, s]] x[t, s % x_slots]; x is [n_tokens, x_slots, k]
    bfloat16, ids [n_tokens, top_k] int32, y [n_tokens, top_k, n_rows]."""
    _require_cuda(w, x, ids)
    n_tokens, top_k = ids.shape
    x_slots = x.shape[1]
    ids = ids.to(torch.int32).contiguous()
    x = x.contiguous()
    if workspace is None:
        workspace = mul_mat_id_workspace(n_expert, n_tokens, top_k, w.device)
    if out is None:
        out = torch.empty((n_tokens, top_k, n_rows), dtype=out_dtype, device=w.device)
    check(lib().spiral_mul_mat_id(qtype, _ptr(w), expert_stride, n_expert, n_rows, k, _ptr(x), x_slots,
                                  _ptr(ids), n_tokens, top_k, _ptr(out), _out_type(out.dtype),
                                  _ptr(workspace), workspace.numel(), _stream()), "mul_mat_id")
    return out


# ggml GLU variants (ggml_glu_op numbering). SWIGLU_OAI (3) takes alpha and
# limit (gpt-oss uses 1.702 and 7.0) and runs only as a standalone GLU.
GLU_REGLU, GLU_GEGLU, GLU_SWIGLU, GLU_SWIGLU_OAI, GLU_GEGLU_ERF, GLU_GEGLU_QUICK = range(6)


def mul_mat_id_glu(qtype, w, expert_stride, n_expert, n_rows, k, x, ids, glu_op=GLU_SWIGLU, swapped=False,
                   out_dtype=torch.bfloat16, workspace=None, out=None):
    """MUL_MAT_ID + GLU in one pass: W rows [0, F) gate, [F, 2F) up (n_rows =
    2F); y[t, s, f] = act(gate) * up (act(up) * gate when swapped), y
    [n_tokens, top_k, F]."""
    _require_cuda(w, x, ids)
    n_tokens, top_k = ids.shape
    x_slots = x.shape[1]
    ids = ids.to(torch.int32).contiguous()
    x = x.contiguous()
    if workspace is None:
        workspace = mul_mat_id_workspace(n_expert, n_tokens, top_k, w.device)
    if out is None:
        out = torch.empty((n_tokens, top_k, n_rows // 2), dtype=out_dtype, device=w.device)
    check(lib().spiral_mul_mat_id_glu(qtype, _ptr(w), expert_stride, n_expert, n_rows, k, _ptr(x), x_slots,
                                      _ptr(ids), n_tokens, top_k, glu_op, int(swapped), _ptr(out),
                                      _out_type(out.dtype), _ptr(workspace), workspace.numel(), _stream()),
          "mul_mat_id_glu")
    return out


def mul_mat_id_glu_split(qtype, w_gate, w_up, expert_stride, n_expert, n_ff, k, x, ids, glu_op=GLU_SWIGLU,
                         swapped=False, out_dtype=torch.bfloat16, workspace=None, out=None):
    """ggml's split form in one pass: gate experts w_gate and up experts w_up
    (n_expert planar n_ff x k matrices each, same stride); y[t, s, f] =
    act(gate) * up (act(up) * gate when swapped), y [n_tokens, top_k, n_ff]."""
    _require_cuda(w_gate, w_up, x, ids)
    n_tokens, top_k = ids.shape
    x_slots = x.shape[1]
    ids = ids.to(torch.int32).contiguous()
    x = x.contiguous()
    if workspace is None:
        workspace = mul_mat_id_workspace(n_expert, n_tokens, top_k, w_gate.device)
    if out is None:
        out = torch.empty((n_tokens, top_k, n_ff), dtype=out_dtype, device=w_gate.device)
    check(lib().spiral_mul_mat_id_glu_split(qtype, _ptr(w_gate), _ptr(w_up), expert_stride, n_expert, n_ff, k,
                                            _ptr(x), x_slots, _ptr(ids), n_tokens, top_k, glu_op, int(swapped),
                                            _ptr(out), _out_type(out.dtype), _ptr(workspace), workspace.numel(),
                                            _stream()), "mul_mat_id_glu_split")
    return out


def glu_split(gate, up, glu_op=GLU_SWIGLU, swapped=False, out=None, alpha=1.702, limit=7.0):
    """ggml's split GLU over float32 tensors of equal shape [..., F]:
    act(gate) * up (act(up) * gate when swapped); alpha and limit are
    SWIGLU_OAI's parameters."""
    _require_cuda(gate, up)
    if gate.dtype != torch.float32 or up.dtype != torch.float32 or gate.shape != up.shape:
        raise TypeError("glu_split takes two float32 tensors of one shape")
    g2 = gate.reshape(-1, gate.shape[-1]).contiguous()
    u2 = up.reshape(-1, up.shape[-1]).contiguous()
    F = g2.shape[1]
    if out is None:
        out = torch.empty(gate.shape, dtype=torch.float32, device=gate.device)
    if glu_op == GLU_SWIGLU_OAI:
        check(lib().spiral_glu_split_swiglu_oai(int(swapped), alpha, limit, _ptr(g2), F, _ptr(u2), F, F, g2.shape[0],
                                                _ptr(out), F, _stream()), "glu_split_swiglu_oai")
        return out
    check(lib().spiral_glu_split(glu_op, int(swapped), _ptr(g2), F, _ptr(u2), F, F, g2.shape[0], _ptr(out), F,
                                 _stream()), "glu_split")
    return out


def glu(x, glu_op=GLU_SWIGLU, swapped=False, out=None, alpha=1.702, limit=7.0):
    """ggml GLU over the last dimension of a float32 tensor [..., 2F] -> [..., F];
    alpha and limit are SWIGLU_OAI's parameters."""
    _require_cuda(x)
    if x.dtype != torch.float32:
        raise TypeError("glu takes float32")
    x2 = x.reshape(-1, x.shape[-1]).contiguous()
    F = x2.shape[1] // 2
    if out is None:
        out = torch.empty(x.shape[:-1] + (F,), dtype=torch.float32, device=x.device)
    if glu_op == GLU_SWIGLU_OAI:
        check(lib().spiral_glu_swiglu_oai(int(swapped), alpha, limit, _ptr(x2), x2.shape[1], F, x2.shape[0],
                                          _ptr(out), F, _stream()), "glu_swiglu_oai")
        return out
    check(lib().spiral_glu(glu_op, int(swapped), _ptr(x2), x2.shape[1], F, x2.shape[0], _ptr(out), F, _stream()),
          "glu")
    return out


def unpack_all(qtype, packed, weights_rows, weights_cols):
    """quants_unpack_all over reference records -> bf16 in reference order."""
    _require_cuda(packed)
    out = torch.empty(weights_rows * weights_cols, dtype=torch.bfloat16, device=packed.device)
    check(lib().quants_unpack_all(qtype, _ptr(packed), weights_rows, weights_cols, _ptr(out), _stream()),
          "unpack_all")
    return out


def unpack_mmul_all(qtype, packed, inputs, weights_rows, weights_cols):
    """quants_unpack_mmul_all: inputs bf16 [K/8][4][8] -> f32 [N/8][4][8]."""
    _require_cuda(packed, inputs)
    out = torch.empty((weights_cols // 8) * 32, dtype=torch.float32, device=packed.device)
    check(lib().quants_unpack_mmul_all(qtype, _ptr(packed), _ptr(inputs), _ptr(out), weights_rows,
                                       weights_cols, _stream()), "unpack_mmul_all")
    return out


def block_elems(qtype):
    return BLOCK_ELEMS[qtype]
