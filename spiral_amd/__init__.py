"""spiral_amd: MI355X (gfx950) quantized-weight hot path of spiral.

GGUF Q4_0 / Q8_0 / Q4_K / Q5_K / Q6_K / IQ4_NL / IQ4_XS exact dequantization to bf16 and the dequant-fused
GEMV / GEMM / MoE expert products behind a ggml-style MUL_MAT / GET_ROWS /
MUL_MAT_ID surface, as hand-written HIP kernels in libspiral_quants.so.

    spiral_amd._lib     ctypes binding of the C ABI (include/spiral_quants.h)
    spiral_amd.ops      device-tensor wrappers used by tests and bench.py
    spiral_amd.quants   host mirror of the reference's repack harness
    spiral_amd.synth    seeded synthetic GGUF tensors
    spiral_amd.build    hipcc build of the library
"""

from ._lib import (TYPE_BF16, TYPE_F32, TYPE_I32, TYPE_IQ4_NL, TYPE_IQ4_XS, TYPE_Q4_0, TYPE_Q4_K,  # noqa: F401
                   TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0, SpiralError, lib)

FORMATS = {"q4_0": TYPE_Q4_0, "q8_0": TYPE_Q8_0, "q4_k": TYPE_Q4_K, "q5_k": TYPE_Q5_K, "q6_k": TYPE_Q6_K,
           "iq4_nl": TYPE_IQ4_NL, "iq4_xs": TYPE_IQ4_XS}
BLOCK_ELEMS = {TYPE_Q4_0: 32, TYPE_Q8_0: 32, TYPE_Q4_K: 256, TYPE_Q5_K: 256, TYPE_Q6_K: 256,
               TYPE_IQ4_NL: 32, TYPE_IQ4_XS: 256}
BLOCK_BYTES = {TYPE_Q4_0: 18, TYPE_Q8_0: 34, TYPE_Q4_K: 144, TYPE_Q5_K: 176, TYPE_Q6_K: 210,
               TYPE_IQ4_NL: 18, TYPE_IQ4_XS: 136}


def row_bytes(qtype, k):
    return (k // BLOCK_ELEMS[qtype]) * BLOCK_BYTES[qtype]
