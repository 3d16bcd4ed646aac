"""ctypes view of the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Loads oracle/liboracle.so (built by oracle/Makefile) and, when present, the
reference's own repack shims compiled into oracle/_ref/. Only tests/,
__graft_entry__.smoke() and bench.py's CPU-baseline leg import this module;
the product library never does.
"""

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS = 2, 8, 12, 13, 14, 20, 23
BLOCK_ELEMS = {Q4_0: 32, Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256, IQ4_NL: 32, IQ4_XS: 256}
BLOCK_BYTES = {Q4_0: 18, Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210, IQ4_NL: 18, IQ4_XS: 136}
FORMAT_NAMES = {Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_k", Q5_K: "q5_k", Q6_K: "q6_k", IQ4_NL: "iq4_nl",
                IQ4_XS: "iq4_xs"}

_i64 = ctypes.c_int64
_p = ctypes.c_void_p


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


_lib = None


def lib():
    global _lib
    if _lib is None:
        path = HERE / "liboracle.so"
        if not path.exists():
            raise RuntimeError(f"{path} missing: run `make -C oracle`")
        L = ctypes.CDLL(str(path))
        L.oq_fp16_ieee.argtypes = [ctypes.c_uint16]
        L.oq_fp16_ieee.restype = ctypes.c_float
        L.oq_fp16_device.argtypes = [ctypes.c_uint16]
        L.oq_fp16_device.restype = ctypes.c_float
        L.oq_bf16_rne.argtypes = [ctypes.c_float]
        L.oq_bf16_rne.restype = ctypes.c_uint16
        L.oq_fp16_device_array.argtypes = [_p, _p, _i64]
        L.oq_fp16_device_array.restype = None
        L.oq_bf16_rne_array.argtypes = [_p, _p, _i64]
        L.oq_bf16_rne_array.restype = None
        L.oq_aie_q_times_d.argtypes = [ctypes.c_int, ctypes.c_uint16]
        L.oq_aie_q_times_d.restype = ctypes.c_uint16
        L.oq_aie_q6_k.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_uint16]
        L.oq_aie_q6_k.restype = ctypes.c_uint16
        L.oq_check_q_times_d.argtypes = [ctypes.POINTER(_i64)]
        L.oq_check_q_times_d.restype = _i64
        L.oq_check_q6_k.argtypes = [ctypes.c_int, ctypes.POINTER(_i64)]
        L.oq_check_q6_k.restype = _i64
        L.oq_check_split_identity.argtypes = []
        L.oq_check_split_identity.restype = _i64
        L.oq_dequant.argtypes = [ctypes.c_int, _p, _i64, _i64, _i64, _p, _i64]
        L.oq_dequant.restype = ctypes.c_int
        L.oq_dequant_f64.argtypes = [ctypes.c_int, _p, _i64, _i64, _i64, _p, _i64]
        L.oq_dequant_f64.restype = ctypes.c_int
        L.oq_matmul_f64_exact.argtypes = [_p, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64]
        L.oq_matmul_f64_exact.restype = None
        L.oq_get_rows.argtypes = [ctypes.c_int, _p, _i64, _i64, _i64, _p, _i64, _p, _i64]
        L.oq_get_rows.restype = ctypes.c_int
        L.oq_ref_record_count.argtypes = [ctypes.c_int, _i64, _i64]
        L.oq_ref_record_count.restype = _i64
        L.oq_ref_packed_bytes.argtypes = [ctypes.c_int, _i64, _i64]
        L.oq_ref_packed_bytes.restype = _i64
        L.oq_ref_repack.argtypes = [ctypes.c_int, _p, _i64, _p, _i64, _i64, _i64,
                                    ctypes.POINTER(ctypes.c_int)]
        L.oq_ref_repack.restype = _i64
        L.oq_ref_unpack.argtypes = [ctypes.c_int, _p, _i64, _i64, _p]
        L.oq_ref_unpack.restype = ctypes.c_int
        L.oq_matmul_f64.argtypes = [_p, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64]
        L.oq_matmul_f64.restype = None
        L.oq_matmul_f32.argtypes = [_p, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64]
        L.oq_matmul_f32.restype = None
        L.oq_quant_matmul_f32.argtypes = [ctypes.c_int, _p, _i64, _i64, _i64, _p, _i64,
                                          _i64, _p, _i64, ctypes.c_int]
        L.oq_quant_matmul_f32.restype = ctypes.c_int
        _lib = L
    return _lib


def fp16_device(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().oq_fp16_device_array(_ptr(h), _ptr(out), h.size)
    return out


def bf16_rne(f):
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, dtype=np.uint16)
    lib().oq_bf16_rne_array(_ptr(f), _ptr(out), f.size)
    return out


def row_bytes(qtype, k):
    return (k // BLOCK_ELEMS[qtype]) * BLOCK_BYTES[qtype]


def dequant(qtype, raw, n_rows, k, row_stride=None):
    """Canonical rows -> uint16 bf16 bits, shape [n_rows, k]."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    row_stride = row_bytes(qtype, k) if row_stride is None else row_stride
    out = np.empty((n_rows, k), dtype=np.uint16)
    rc = lib().oq_dequant(qtype, _ptr(raw), row_stride, n_rows, k, _ptr(out), k)
    if rc != 0:
        raise ValueError("oracle dequant: bad shape")
    return out


def dequant_exact(qtype, raw, n_rows, k, row_stride=None):
    """Canonical rows -> the exact weights (float64, shape [n_rows, k]) that
    dequant rounds to bf16 once."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    row_stride = row_bytes(qtype, k) if row_stride is None else row_stride
    out = np.empty((n_rows, k), dtype=np.float64)
    rc = lib().oq_dequant_f64(qtype, _ptr(raw), row_stride, n_rows, k, _ptr(out), k)
    if rc != 0:
        raise ValueError("oracle dequant_exact: bad shape")
    return out


def get_rows(qtype, raw, n_rows, k, ids):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    out = np.empty((ids.size, k), dtype=np.uint16)
    rc = lib().oq_get_rows(qtype, _ptr(raw), row_bytes(qtype, k), n_rows, k,
                           _ptr(ids), ids.size, _ptr(out), k)
    if rc != 0:
        raise ValueError("oracle get_rows: bad shape or id")
    return out


def ref_packed_bytes(qtype, weights_rows, weights_cols):
    return lib().oq_ref_packed_bytes(qtype, weights_rows, weights_cols)


def ref_repack(qtype, raw, weights_rows, weights_cols, stride=None):
    """Canonical column-major bytes -> reference NPU records; (bytes, warnings)."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    stride = row_bytes(qtype, weights_rows) if stride is None else stride
    n = ref_packed_bytes(qtype, weights_rows, weights_cols)
    dst = np.zeros(max(n, 1), dtype=np.uint8)
    warn = ctypes.c_int(0)
    written = lib().oq_ref_repack(qtype, _ptr(raw), stride, _ptr(dst), n,
                                  weights_rows, weights_cols, ctypes.byref(warn))
    if written != n or n == 0:
        raise ValueError("oracle ref_repack failed")
    return dst[:n], warn.value


def ref_unpack(qtype, packed, weights_rows, weights_cols):
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.empty(weights_rows * weights_cols, dtype=np.uint16)
    rc = lib().oq_ref_unpack(qtype, _ptr(packed), weights_rows, weights_cols, _ptr(out))
    if rc != 0:
        raise ValueError("oracle ref_unpack: bad shape")
    return out


def ref_order(values_nk, record_rows):
    """Row-major [N][K] -> the reference output order
    [N/8][K/record_rows][record_rows][8] (formats/q4_0.py:65-79)."""
    n, k = values_nk.shape
    return (values_nk.T.reshape(k // record_rows, record_rows, n // 8, 8)
            .transpose(2, 0, 1, 3).reshape(-1))


REF_RECORD_ROWS = {Q4_0: 64, Q8_0: 256, Q6_K: 256}


def matmul_f64(w_bf16, x_bf16):
    """y[m, n] = sum_k x[m, k] * w[n, k] in float64 over bf16 bit arrays."""
    w = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    n, k = w.shape
    m = x.shape[0]
    y = np.empty((m, n), dtype=np.float64)
    lib().oq_matmul_f64(_ptr(w), k, n, k, _ptr(x), k, m, _ptr(y), n)
    return y


def matmul_f64_exact(w_f64, x_bf16):
    """y[m, n] = sum_k x[m, k] * w[n, k] in float64 over float64 weights."""
    w = np.ascontiguousarray(w_f64, dtype=np.float64)
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    n, k = w.shape
    m = x.shape[0]
    y = np.empty((m, n), dtype=np.float64)
    lib().oq_matmul_f64_exact(_ptr(w), k, n, k, _ptr(x), k, m, _ptr(y), n)
    return y


# ggml GLU variants (ggml_glu_op numbering), used by the fused MUL_MAT_ID + GLU.
GLU_REGLU, GLU_GEGLU, GLU_SWIGLU, GLU_SWIGLU_OAI, GLU_GEGLU_ERF, GLU_GEGLU_QUICK = 0, 1, 2, 3, 4, 5


def glu_f64(h, op, swapped=False, alpha=None, limit=None):
    """ggml's GLU over the last axis of h (..., 2F) in float64: act(a) * b with
    (a, b) the first and second halves of each row, (b, a) when swapped.

    ggml is not vendored by the reference (its MoE FFN is a plan:
    src/quants/TODO.md:55,214-220); act follows the published definitions of
    ggml's GLU ops: REGLU relu; GEGLU gelu in its tanh form
    0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))); SWIGLU silu x / (1 + e^-x);
    GEGLU_ERF 0.5 x (1 + erf(x / sqrt(2))); GEGLU_QUICK x / (1 + e^(-1.702 x)).
    SWIGLU_OAI (gpt-oss's FFN; alpha and limit given) combines both halves:
    x = min(a, limit), y = clip(b, -limit, limit), x / (1 + e^(-alpha x)) * (y + 1).
    """
    from scipy.special import erf

    h = np.asarray(h, dtype=np.float64)
    F = h.shape[-1] // 2
    a, b = h[..., :F], h[..., F:]
    if swapped:
        a, b = b, a
    if op == GLU_REGLU:
        act = np.maximum(a, 0.0)
    elif op == GLU_GEGLU:
        act = 0.5 * a * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (a + 0.044715 * a ** 3)))
    elif op == GLU_SWIGLU:
        act = a / (1.0 + np.exp(-a))
    elif op == GLU_GEGLU_ERF:
        act = 0.5 * a * (1.0 + erf(a / np.sqrt(2.0)))
    elif op == GLU_GEGLU_QUICK:
        act = a / (1.0 + np.exp(-1.702 * a))
    elif op == GLU_SWIGLU_OAI:
        x = np.minimum(a, limit)
        y = np.clip(b, -limit, limit)
        return x / (1.0 + np.exp(-alpha * x)) * (y + 1.0)
    else:
        raise ValueError(f"GLU op {op}")
    return act * b


def matmul_f32(w_bf16, x_bf16):
    w = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    n, k = w.shape
    m = x.shape[0]
    y = np.empty((m, n), dtype=np.float32)
    lib().oq_matmul_f32(_ptr(w), k, n, k, _ptr(x), k, m, _ptr(y), n)
    return y


def quant_matmul_f32(qtype, raw, n_rows, k, x_bf16, threads=1):
    """Streaming dequantize-and-multiply on the CPU (the CPU baseline)."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16).reshape(-1, k)
    m = x.shape[0]
    y = np.empty((m, n_rows), dtype=np.float32)
    rc = lib().oq_quant_matmul_f32(qtype, _ptr(raw), row_bytes(qtype, k), n_rows, k,
                                   _ptr(x), k, m, _ptr(y), n_rows, threads)
    if rc != 0:
        raise ValueError("oracle quant_matmul: bad shape")
    return y


# ---- the reference's own repack, compiled from its sources into _ref/ ----

def ref_shim(qtype):
    """ctypes handle on oracle/_ref/libref_repack_<fmt>.so, or None."""
    path = HERE / "_ref" / f"libref_repack_{FORMAT_NAMES[qtype]}.so"
    if not path.exists():
        return None
    L = ctypes.CDLL(str(path))
    L.quants_record_count.argtypes = [_i64, _i64]
    L.quants_record_count.restype = _i64
    L.quants_packed_bytes.argtypes = [_i64, _i64]
    L.quants_packed_bytes.restype = _i64
    L.quants_repack.argtypes = [_p, _i64, _p, _i64, _i64, _i64]
    L.quants_repack.restype = _i64
    return L


def cpu_count():
    return len(os.sched_getaffinity(0))


# ---- the CPU baseline (oracle/cpu_baseline.c), timed by bench.py -------------

_cb = None


def cpu_baseline():
    """ctypes handle on oracle/libcpu_baseline.so."""
    global _cb
    if _cb is None:
        path = HERE / "libcpu_baseline.so"
        if not path.exists():
            raise RuntimeError(f"{path} missing: run `make -C oracle`")
        L = ctypes.CDLL(str(path))
        L.cb_gemv_q8_0.argtypes = [_p, _i64, _i64, _p, _p, ctypes.c_int]
        L.cb_gemv_q8_0.restype = ctypes.c_int
        L.cb_dequant_q4_0.argtypes = [_p, _i64, _i64, _p, ctypes.c_int]
        L.cb_dequant_q4_0.restype = ctypes.c_int
        L.cb_gemm_q4_0.argtypes = [_p, _i64, _i64, _p, _i64, _p, ctypes.c_int]
        L.cb_gemm_q4_0.restype = ctypes.c_int
        L.cb_gemv_q6_k.argtypes = [_p, _i64, _i64, _p, _p, ctypes.c_int]
        L.cb_gemv_q6_k.restype = ctypes.c_int
        L.cb_dequant_q6_k.argtypes = [_p, _i64, _i64, _p, ctypes.c_int]
        L.cb_dequant_q6_k.restype = ctypes.c_int
        L.cb_moe_q4_0.argtypes = [_p, _i64, _i64, _i64, _i64, _p, _i64, _p, _i64, _i64, _p, ctypes.c_int]
        L.cb_moe_q4_0.restype = ctypes.c_int
        _cb = L
    return _cb


def cb_gemv_q8_0(raw, n_rows, k, x_bf16, threads):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16).reshape(-1)
    y = np.empty(n_rows, dtype=np.float32)
    if cpu_baseline().cb_gemv_q8_0(_ptr(raw), n_rows, k, _ptr(x), _ptr(y), threads) != 0:
        raise ValueError("cb_gemv_q8_0: bad shape")
    return y


def cb_dequant_q4_0(raw, n_rows, k, threads, out=None):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty((n_rows, k), dtype=np.uint16) if out is None else out
    if cpu_baseline().cb_dequant_q4_0(_ptr(raw), n_rows, k, _ptr(out), threads) != 0:
        raise ValueError("cb_dequant_q4_0: bad shape")
    return out


def cb_gemm_q4_0(raw, n_rows, k, x_bf16, threads):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16).reshape(-1, k)
    y = np.empty((x.shape[0], n_rows), dtype=np.float32)
    if cpu_baseline().cb_gemm_q4_0(_ptr(raw), n_rows, k, _ptr(x), x.shape[0], _ptr(y), threads) != 0:
        raise ValueError("cb_gemm_q4_0: bad shape")
    return y


def cb_gemv_q6_k(raw, n_rows, k, x_bf16, threads):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16).reshape(-1)
    y = np.empty(n_rows, dtype=np.float32)
    if cpu_baseline().cb_gemv_q6_k(_ptr(raw), n_rows, k, _ptr(x), _ptr(y), threads) != 0:
        raise ValueError("cb_gemv_q6_k: bad shape")
    return y


def cb_dequant_q6_k(raw, n_rows, k, threads, out=None):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty((n_rows, k), dtype=np.uint16) if out is None else out
    if cpu_baseline().cb_dequant_q6_k(_ptr(raw), n_rows, k, _ptr(out), threads) != 0:
        raise ValueError("cb_dequant_q6_k: bad shape")
    return out


def cb_moe_q4_0(raw, expert_bytes, n_expert, n_rows, k, x_bf16, ids, threads):
    """MUL_MAT_ID over canonical Q4_0 experts stacked at expert_bytes: x is
    [n_tokens][x_slots][k] bf16 bits, ids [n_tokens][top_k] int32; returns
    y [n_tokens][top_k][n_rows] float32."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    n_tokens, top_k = ids.shape
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16).reshape(n_tokens, -1, k)
    y = np.empty((n_tokens, top_k, n_rows), dtype=np.float32)
    if cpu_baseline().cb_moe_q4_0(_ptr(raw), expert_bytes, n_expert, n_rows, k, _ptr(x), x.shape[1], _ptr(ids),
                                  n_tokens, top_k, _ptr(y), threads) != 0:
        raise ValueError("cb_moe_q4_0: bad shape")
    return y


def host_cpu():
    """What the CPU baseline ran on: logical CPUs, the usable set, OMP_NUM_THREADS, model."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "affinity": cpu_count(),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS"), "cpu_model": model}
