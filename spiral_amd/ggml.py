"""ctypes mirror of the ggml-backend-shaped surface (include/spiral_ggml.h).

Tensors, graphs, buffers and the backend as a llama.cpp-side shim would use
them: build op nodes with mul_mat / get_rows / mul_mat_id / glu (the ggml
builder names), place tensors in a Buffer, upload canonical GGUF bytes with
Buffer.set, and run a graph on a Backend. All compute happens in
libspiral_quants.so on the device; nothing here computes.
"""

import ctypes
import struct

from ._lib import (TYPE_BF16, TYPE_F16, TYPE_F32, TYPE_I32, TYPE_IQ4_NL, TYPE_IQ4_XS, TYPE_Q4_0,  # noqa: F401
                   TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0, check, lib)

MAX_DIMS, MAX_SRC, MAX_NAME, MAX_OP_PARAMS = 4, 10, 64, 16
(OP_NONE, OP_GET_ROWS, OP_MUL_MAT, OP_MUL_MAT_ID, OP_VIEW, OP_RESHAPE, OP_PERMUTE,
 OP_TRANSPOSE, OP_GLU) = range(9)
# ggml GLU variants (op_params[0] of a GLU node; ggml_glu_op numbering)
GLU_REGLU, GLU_GEGLU, GLU_SWIGLU, GLU_SWIGLU_OAI, GLU_GEGLU_ERF, GLU_GEGLU_QUICK = range(6)
FLAG_OUTPUT = 2  # ggml GGML_TENSOR_FLAG_OUTPUT

# bytes per block and elements per block (ggml type traits)
TYPE_TRAITS = {
    TYPE_F32: (4, 1), TYPE_F16: (2, 1), TYPE_BF16: (2, 1), TYPE_I32: (4, 1),
    TYPE_Q4_0: (18, 32), TYPE_Q8_0: (34, 32), TYPE_Q6_K: (210, 256),
    TYPE_Q4_K: (144, 256), TYPE_Q5_K: (176, 256), TYPE_IQ4_NL: (18, 32), TYPE_IQ4_XS: (136, 256),
}


class Tensor(ctypes.Structure):
    pass


Tensor._fields_ = [
    ("type", ctypes.c_int32),
    ("buffer", ctypes.c_void_p),
    ("ne", ctypes.c_int64 * MAX_DIMS),
    ("nb", ctypes.c_size_t * MAX_DIMS),
    ("op", ctypes.c_int32),
    ("op_params", ctypes.c_int32 * MAX_OP_PARAMS),
    ("flags", ctypes.c_int32),
    ("src", ctypes.POINTER(Tensor) * MAX_SRC),
    ("view_src", ctypes.POINTER(Tensor)),
    ("view_offs", ctypes.c_size_t),
    ("data", ctypes.c_void_p),
    ("name", ctypes.c_char * MAX_NAME),
]


class CGraph(ctypes.Structure):
    _fields_ = [("n_nodes", ctypes.c_int32), ("nodes", ctypes.POINTER(ctypes.POINTER(Tensor)))]


_T = ctypes.POINTER(Tensor)
_p, _sz, _int = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int

SIGNATURES = {
    "spiral_buft_name": (ctypes.c_char_p, []),
    "spiral_buft_alignment": (_sz, []),
    "spiral_buft_max_size": (_sz, []),
    "spiral_buft_alloc_size": (_sz, [_T]),
    "spiral_buft_alloc_buffer": (_p, [_sz]),
    "spiral_buffer_free": (None, [_p]),
    "spiral_buffer_get_base": (_p, [_p]),
    "spiral_buffer_get_size": (_sz, [_p]),
    "spiral_buffer_init_tensor": (_int, [_p, _T]),
    "spiral_buffer_set_tensor": (_int, [_p, _T, _p, _sz, _sz]),
    "spiral_buffer_get_tensor": (_int, [_p, _T, _p, _sz, _sz]),
    "spiral_buffer_memset_tensor": (_int, [_p, _T, ctypes.c_uint8, _sz, _sz]),
    "spiral_buffer_clear": (_int, [_p, ctypes.c_uint8]),
    "spiral_supports_op": (_int, [_T]),
    "spiral_backend_init": (_p, [_int]),
    "spiral_backend_free": (None, [_p]),
    "spiral_backend_name": (ctypes.c_char_p, [_p]),
    "spiral_backend_stream": (_p, [_p]),
    "spiral_backend_graph_compute": (_int, [_p, ctypes.POINTER(CGraph)]),
    "spiral_backend_synchronize": (_int, [_p]),
}

_bound = False


def _lib():
    global _bound
    L = lib()
    if not _bound:
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _bound = True
    return L


def new_tensor(qtype, ne, name=""):
    """ggml_new_tensor: contiguous strides, no data yet."""
    ne = list(ne) + [1] * (MAX_DIMS - len(ne))
    ts, blck = TYPE_TRAITS[qtype]
    if ne[0] % blck != 0:
        raise ValueError(f"ne[0]={ne[0]} is not a multiple of the block size {blck}")
    t = Tensor()
    t.type = qtype
    for i, v in enumerate(ne):
        t.ne[i] = v
    t.nb[0] = ts
    t.nb[1] = ts * ne[0] // blck
    for i in range(2, MAX_DIMS):
        t.nb[i] = t.nb[i - 1] * ne[i - 1]
    t.op = OP_NONE
    t.name = name.encode()[:MAX_NAME - 1]
    return t


def nbytes(t):
    return _lib().spiral_buft_alloc_size(ctypes.byref(t))


def _node(qtype, ne, op, srcs, name):
    t = new_tensor(qtype, ne, name)
    t.op = op
    for i, s in enumerate(srcs):
        t.src[i] = ctypes.pointer(s)
    t._keep = list(srcs)  # keep the sources alive as long as the node
    return t


def view(a, ne, nb, offset, name="view"):
    """ggml_view_4d(a, ne..., nb1..., offset): a VIEW node of type a.type over
    a's memory; view_src is the tensor that owns the memory (never a view)
    and view_offs the byte offset into it, as ggml records them."""
    ne = list(ne) + [1] * (MAX_DIMS - len(ne))
    t = new_tensor(a.type, ne, name)
    t.nb[0] = a.nb[0]
    for i, v in enumerate(nb, start=1):
        t.nb[i] = v
    t.op = OP_VIEW
    t.src[0] = ctypes.pointer(a)
    base = a.view_src.contents if a.view_src else a
    t.view_src = ctypes.pointer(base)
    t.view_offs = (a.view_offs if a.view_src else 0) + offset
    if a.data:
        t.data = a.data + offset
    t.buffer = a.buffer
    t._keep = [a, base]
    return t


def mul_mat(a, b, name="mul_mat"):
    """ggml_mul_mat(a, b): [a.ne1, b.ne1, b.ne2, b.ne3] F32."""
    return _node(TYPE_F32, [a.ne[1], b.ne[1], b.ne[2], b.ne[3]], OP_MUL_MAT, [a, b], name)


def get_rows(a, ids, out_type=TYPE_F32, name="get_rows"):
    """ggml_get_rows(a, ids): [a.ne0, ids.ne0, ids.ne1, ids.ne2]."""
    return _node(out_type, [a.ne[0], ids.ne[0], ids.ne[1], ids.ne[2]], OP_GET_ROWS, [a, ids], name)


def mul_mat_id(a, b, ids, name="mul_mat_id"):
    """ggml_mul_mat_id(as, b, ids): [as.ne1, ids.ne0, ids.ne1] F32."""
    return _node(TYPE_F32, [a.ne[1], ids.ne[0], ids.ne[1], 1], OP_MUL_MAT_ID, [a, b, ids], name)


def _glu_params(t, op, swapped, alpha, limit):
    t.op_params[0] = op
    t.op_params[1] = int(swapped)
    if op == GLU_SWIGLU_OAI:  # ggml_swiglu_oai: alpha and limit as float bits in op_params[2], [3]
        t.op_params[2] = struct.unpack("<i", struct.pack("<f", alpha))[0]
        t.op_params[3] = struct.unpack("<i", struct.pack("<f", limit))[0]


def glu(a, op=GLU_SWIGLU, swapped=False, name="glu", alpha=1.702, limit=7.0):
    """ggml_glu(a, op, swapped) (single-tensor form): [a.ne0 / 2, a.ne1, ...] F32;
    SWIGLU_OAI as ggml_swiglu_oai with alpha and limit."""
    t = _node(TYPE_F32, [a.ne[0] // 2, a.ne[1], a.ne[2], a.ne[3]], OP_GLU, [a], name)
    _glu_params(t, op, swapped, alpha, limit)
    return t


def glu_split(a, b, op=GLU_SWIGLU, swapped=False, name="glu_split", alpha=1.702, limit=7.0):
    """ggml_glu_split(a, b, op) (split form): act(a) * b over equal shapes, F32;
    SWIGLU_OAI as ggml_swiglu_oai(a, b, alpha, limit). `swapped` only sets
    op_params[1], which the split form ignores, as in ggml."""
    t = _node(TYPE_F32, list(a.ne), OP_GLU, [a, b], name)
    _glu_params(t, op, swapped, alpha, limit)
    return t


def supports_op(t):
    return bool(_lib().spiral_supports_op(ctypes.byref(t)))


class Buffer:
    """A device buffer with a bump allocator for tensors (ggml_backend_buffer
    plus the part of ggml-alloc a test needs)."""

    def __init__(self, size):
        L = _lib()
        self.ptr = L.spiral_buft_alloc_buffer(size)
        if not self.ptr:
            raise MemoryError(f"spiral_buft_alloc_buffer({size}) failed")
        self.base = L.spiral_buffer_get_base(self.ptr)
        self.size = L.spiral_buffer_get_size(self.ptr)
        self.align = L.spiral_buft_alignment()
        self.used = 0

    def alloc(self, t):
        n = nbytes(t)
        off = (self.used + self.align - 1) // self.align * self.align
        if n == 0 or off + n > self.size:
            raise MemoryError("buffer too small for tensor")
        t.data = self.base + off
        self.used = off + n
        check(_lib().spiral_buffer_init_tensor(self.ptr, ctypes.byref(t)), "init_tensor")
        return t

    def set(self, t, data, offset=0):
        data = bytes(data) if not isinstance(data, (bytes, bytearray)) else data
        buf = (ctypes.c_uint8 * len(data)).from_buffer_copy(data)
        check(_lib().spiral_buffer_set_tensor(self.ptr, ctypes.byref(t), buf, offset, len(data)), "set_tensor")

    def get(self, t, size=None, offset=0):
        size = nbytes(t) - offset if size is None else size
        buf = (ctypes.c_uint8 * size)()
        check(_lib().spiral_buffer_get_tensor(self.ptr, ctypes.byref(t), buf, offset, size), "get_tensor")
        return bytes(buf)

    def memset(self, t, value, offset=0, size=None):
        size = nbytes(t) - offset if size is None else size
        check(_lib().spiral_buffer_memset_tensor(self.ptr, ctypes.byref(t), value, offset, size), "memset_tensor")

    def clear(self, value):
        check(_lib().spiral_buffer_clear(self.ptr, value), "clear")

    def free(self):
        if self.ptr:
            _lib().spiral_buffer_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Backend:
    def __init__(self, device=0):
        self.ptr = _lib().spiral_backend_init(device)
        if not self.ptr:
            raise RuntimeError(f"spiral_backend_init({device}) failed: no such HIP device")

    @property
    def name(self):
        return _lib().spiral_backend_name(self.ptr).decode()

    def graph_compute(self, nodes):
        arr = (ctypes.POINTER(Tensor) * len(nodes))(*[ctypes.pointer(n) for n in nodes])
        g = CGraph(len(nodes), arr)
        return _lib().spiral_backend_graph_compute(self.ptr, ctypes.byref(g))

    def synchronize(self):
        check(_lib().spiral_backend_synchronize(self.ptr), "synchronize")

    def free(self):
        if self.ptr:
            _lib().spiral_backend_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
