"""numpy access to the reference-layout host repack in libspiral_quants.so.

quants_<fmt>_record_count / packed_bytes / repack are the library's C
counterparts of the reference's per-format repack API
(src/quants/q4_0/repack.h:10-111, src/quants/q8_0/repack.h:10-91,
src/quants/q6_k/repack.h:11-115). They validate every argument themselves
and return 0 on a bad shape, stride, capacity or pointer; this module sizes
the output array, makes sure the source array covers the strided view the C
code will read, and turns a 0 into ValueError.
"""

import ctypes

import numpy as np

from ._lib import lib

FORMATS = ("q4_0", "q8_0", "q6_k")

# Record geometry of the reference's NPU layout (src/quants/TODO.md:366-444):
# k-rows (the reference's weights_rows) per record and bytes per record of
# 8 columns; a canonical column is k / block blocks of block_bytes bytes.
RECORD_ROWS = {"q4_0": 64, "q8_0": 256, "q6_k": 256}
RECORD_BYTES = {"q4_0": 288, "q8_0": 2176, "q6_k": 1680}
BLOCK = {"q4_0": (32, 18), "q8_0": (32, 34), "q6_k": (256, 210)}


def _entry(fmt, what):
    if fmt not in FORMATS:
        raise ValueError(f"unknown format {fmt!r}; expected one of {FORMATS}")
    return getattr(lib(), f"quants_{fmt}_{what}")


def record_count(fmt, weights_rows, weights_cols):
    return _entry(fmt, "record_count")(weights_rows, weights_cols)


def packed_bytes(fmt, weights_rows, weights_cols):
    return _entry(fmt, "packed_bytes")(weights_rows, weights_cols)


def column_bytes(fmt, weights_rows):
    """Canonical bytes of one column (one ggml row) of weights_rows elements."""
    elems, nbytes = BLOCK[fmt]
    return weights_rows // elems * nbytes


def repack(fmt, canonical, weights_rows, weights_cols, col_stride=None):
    """Canonical GGUF columns (column c at byte c * col_stride of `canonical`)
    -> the reference's record stream as a new uint8 array."""
    fn = _entry(fmt, "repack")
    used = column_bytes(fmt, weights_rows)
    stride = used if col_stride is None else int(col_stride)
    size = packed_bytes(fmt, weights_rows, weights_cols)
    if size <= 0:
        raise ValueError(f"{fmt}: no record layout for {weights_rows} x {weights_cols}")
    src = np.ascontiguousarray(canonical, dtype=np.uint8).reshape(-1)
    # the C side reads used bytes at each of weights_cols column starts
    if stride >= used and src.size < (weights_cols - 1) * stride + used:
        raise ValueError(f"{fmt}: {src.size} source bytes do not cover {weights_cols} columns at stride {stride}")
    out = np.zeros(size, dtype=np.uint8)
    written = fn(src.ctypes.data_as(ctypes.c_void_p), stride, out.ctypes.data_as(ctypes.c_void_p), size,
                 weights_rows, weights_cols)
    if written != size:
        raise ValueError(f"quants_{fmt}_repack refused the arguments (returned {written})")
    return out
