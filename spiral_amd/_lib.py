"""ctypes binding of libspiral_quants.so (the C ABI in include/spiral_quants.h).

The library is built in-tree by spiral_amd.build. Loading fails loudly when it
is missing: there is no CPU or PyTorch fallback for any op.
"""

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libspiral_quants.so"

TYPE_F32, TYPE_F16, TYPE_Q4_0, TYPE_Q8_0, TYPE_Q6_K, TYPE_I32, TYPE_BF16 = 0, 1, 2, 8, 14, 26, 30
TYPE_Q4_K, TYPE_Q5_K = 12, 13
TYPE_IQ4_NL, TYPE_IQ4_XS = 20, 23

STATUS = {
    0: "SPIRAL_OK", 1: "SPIRAL_ERR_SHAPE", 2: "SPIRAL_ERR_ALIGN", 3: "SPIRAL_ERR_NULL",
    4: "SPIRAL_ERR_NO_DEVICE", 5: "SPIRAL_ERR_HIP", 6: "SPIRAL_ERR_TYPE",
    7: "SPIRAL_ERR_CAPACITY", 8: "SPIRAL_ERR_RANGE",
}


class SpiralError(RuntimeError):
    def __init__(self, status, what):
        self.status = status
        super().__init__(f"{what}: {STATUS.get(status, status)}")


_i64, _int, _p, _f32 = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_float

# name -> (restype, argtypes)
SIGNATURES = {
    "spiral_status_string": (ctypes.c_char_p, [_int]),
    "spiral_device_count": (_int, []),
    "quants_q4_0_record_count": (_i64, [_i64, _i64]),
    "quants_q4_0_packed_bytes": (_i64, [_i64, _i64]),
    "quants_q4_0_repack": (_i64, [_p, _i64, _p, _i64, _i64, _i64]),
    "quants_q8_0_record_count": (_i64, [_i64, _i64]),
    "quants_q8_0_packed_bytes": (_i64, [_i64, _i64]),
    "quants_q8_0_repack": (_i64, [_p, _i64, _p, _i64, _i64, _i64]),
    "quants_q6_k_record_count": (_i64, [_i64, _i64]),
    "quants_q6_k_packed_bytes": (_i64, [_i64, _i64]),
    "quants_q6_k_repack": (_i64, [_p, _i64, _p, _i64, _i64, _i64]),
    "quants_set_repack_warn": (None, [_p, _p]),
    "quants_unpack_all": (_int, [_int, _p, _i64, _i64, _p, _p]),
    "quants_unpack_mmul_all": (_int, [_int, _p, _p, _p, _i64, _i64, _p]),
    "spiral_row_bytes": (_i64, [_int, _i64]),
    "spiral_tensor_bytes": (_i64, [_int, _i64, _i64]),
    "spiral_to_planar": (_int, [_int, _p, _i64, _i64, _i64, _p, _p]),
    "spiral_from_planar": (_int, [_int, _p, _i64, _i64, _p, _i64, _p]),
    "spiral_dequant_bf16": (_int, [_int, _p, _i64, _i64, _p, _i64, _p]),
    "spiral_get_rows": (_int, [_int, _p, _i64, _i64, _p, _i64, _p, _int, _i64, _p]),
    "spiral_mul_mat_workspace_bytes": (_i64, [_int, _i64, _i64, _i64]),
    "spiral_mul_mat": (_int, [_int, _p, _i64, _i64, _p, _i64, _i64, _p, _int, _i64, _p, _i64, _p]),
    "spiral_gemv_relaxed_max_k": (_i64, [_int]),
    "spiral_gemv_relaxed": (_int, [_int, _p, _i64, _i64, _p, _p, _int, _p]),
    "spiral_mul_mat_id_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "spiral_mul_mat_id": (_int, [_int, _p, _i64, _i64, _i64, _i64, _p, _i64, _p, _i64, _i64, _p, _int,
                                 _p, _i64, _p]),
    "spiral_mul_mat_id_noalloc": (_int, [_int, _p, _i64, _i64, _i64, _i64, _p, _i64, _p, _i64, _i64, _p, _int,
                                         _p]),
    "spiral_mul_mat_id_glu_fits": (_int, [_int, _i64, _i64]),
    "spiral_mul_mat_id_glu": (_int, [_int, _p, _i64, _i64, _i64, _i64, _p, _i64, _p, _i64, _i64, _int, _int,
                                     _p, _int, _p, _i64, _p]),
    "spiral_glu": (_int, [_int, _int, _p, _i64, _i64, _i64, _p, _i64, _p]),
    "spiral_mul_mat_id_glu_split": (_int, [_int, _p, _p, _i64, _i64, _i64, _i64, _p, _i64, _p, _i64, _i64, _int,
                                           _int, _p, _int, _p, _i64, _p]),
    "spiral_glu_split": (_int, [_int, _int, _p, _i64, _p, _i64, _i64, _i64, _p, _i64, _p]),
    "spiral_glu_swiglu_oai": (_int, [_int, _f32, _f32, _p, _i64, _i64, _i64, _p, _i64, _p]),
    "spiral_glu_split_swiglu_oai": (_int, [_int, _f32, _f32, _p, _i64, _p, _i64, _i64, _i64, _p, _i64, _p]),
}

_lib = None


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m spiral_amd.build` "
                "(there is no fallback implementation)")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status, what):
    if status != 0:
        raise SpiralError(status, what)
