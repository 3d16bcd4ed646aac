"""Host mirror of the reference's repack harness (src/quants/tests/common.py).

Same names and argument meaning as the reference's Python helpers around its
C shim (quants_record_count / quants_packed_bytes / quants_repack,
src/quants/tests/common.py:283-341), backed by libspiral_quants.so's
quants_<fmt>_* entry points instead of a per-format JIT-compiled shim.
"""

import ctypes

import numpy as np

from ._lib import lib

FORMAT_NAMES = ("q4_0", "q8_0", "q6_k")

# Layout constants the reference harness parses from its layout headers
# (src/quants/tests/common.py:109-170), per format.
CONSTANTS = {
    "q4_0": dict(kBlockRows=32, kBlockBytes=18, kTileCols=8, kRecordRows=64, kUnpackTileRows=64,
                 kChunksPerRecord=1, kPackedRecordBytes=288, kRowsMultiple=256),
    "q8_0": dict(kBlockRows=32, kBlockBytes=34, kTileCols=8, kRecordRows=256, kUnpackTileRows=256,
                 kChunksPerRecord=1, kPackedRecordBytes=2176, kRowsMultiple=256),
    "q6_k": dict(kBlockRows=256, kBlockBytes=210, kTileCols=8, kRecordRows=256, kUnpackTileRows=64,
                 kChunksPerRecord=4, kPackedRecordBytes=1680, kRowsMultiple=256),
}


def _fn(format_name, what):
    if format_name not in FORMAT_NAMES:
        raise ValueError(f"unknown format: {format_name}")
    return getattr(lib(), f"quants_{format_name}_{what}")


def record_count(format_name, weights_rows, weights_cols):
    return _fn(format_name, "record_count")(weights_rows, weights_cols)


def packed_bytes(format_name, weights_rows, weights_cols):
    return _fn(format_name, "packed_bytes")(weights_rows, weights_cols)


def resolve_shape(format_name, rows, cols):
    """Shape check of src/quants/tests/common.py:187-201."""
    c = CONSTANTS[format_name]
    if rows <= 0 or cols <= 0:
        raise ValueError("rows and cols must be positive")
    if rows % c["kRowsMultiple"] != 0:
        raise ValueError(f"rows must be a multiple of {c['kRowsMultiple']}")
    if cols % c["kTileCols"] != 0:
        raise ValueError(f"cols must be a multiple of {c['kTileCols']}")
    return rows, cols, c


def repack_host(format_name, raw, weights_rows, weights_cols, stride):
    """Repack canonical column-major bytes into the reference's records
    (src/quants/tests/common.py:308-341)."""
    if weights_rows <= 0 or weights_cols <= 0:
        raise ValueError("weights_rows and weights_cols must be positive")
    if stride < 0:
        raise ValueError("stride must be non-negative")
    expected = packed_bytes(format_name, weights_rows, weights_cols)
    if expected <= 0:
        raise ValueError(f"{format_name}: invalid shape {weights_rows}x{weights_cols}")
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    if raw.size < weights_cols * stride:
        raise ValueError(f"{format_name}: source buffer is smaller than the strided view")
    packed = np.zeros(expected, dtype=np.uint8)
    written = _fn(format_name, "repack")(
        raw.ctypes.data_as(ctypes.c_void_p), stride, packed.ctypes.data_as(ctypes.c_void_p),
        expected, weights_rows, weights_cols)
    if written != expected:
        raise RuntimeError(f"{format_name}: repack wrote {written} bytes, expected {expected}")
    return packed
