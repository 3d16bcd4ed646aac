"""CPU tests of libspiral_quants.so's C ABI (no GPU needed).

- every function declared in include/*.h is exported;
- the reference-layout host repack (quants_<fmt>_*) is byte-identical to the
  reference's own repack (oracle/_ref when built here, committed fixtures
  everywhere) with the same 0-on-error convention and warning lines;
- argument validation returns its status codes before any device work.
"""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O
from spiral_amd import _lib, quants

ROOT = Path(__file__).resolve().parent.parent
GOLDEN = ROOT / "tests" / "golden"
NAMES = {O.Q4_0: "q4_0", O.Q8_0: "q8_0", O.Q6_K: "q6_k"}


def declared_functions():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"\b([A-Za-z_]\w*)\s*\(", text):
            name = m.group(1)
            if name.startswith(("spiral_", "quants_")):
                names.add(name)
    return sorted(names)


def test_every_declared_symbol_is_exported(spiral_lib):
    names = declared_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(spiral_lib, n)]
    assert not missing, missing


def test_ctypes_signatures_cover_the_header():
    from spiral_amd import ggml
    assert set(declared_functions()) == set(_lib.SIGNATURES) | set(ggml.SIGNATURES)


@pytest.mark.parametrize("qtype", [O.Q4_0, O.Q8_0, O.Q6_K])
def test_host_repack_matches_reference_fixture(spiral_lib, qtype):
    fx = np.load(GOLDEN / "ref_records.npz")
    name = NAMES[qtype]
    raw = fx[f"{name}_raw"]
    rows, cols = (int(v) for v in fx[f"{name}_shape"])
    got = quants.repack(name, raw, rows, cols, O.row_bytes(qtype, rows))
    assert np.array_equal(got, fx[f"{name}_records"])


@pytest.mark.parametrize("qtype", [O.Q4_0, O.Q8_0, O.Q6_K])
def test_host_repack_matches_reference_build(spiral_lib, qtype, capfd):
    shim = O.ref_shim(qtype)
    if shim is None:
        pytest.skip("reference repack not built here (oracle/_ref)")
    name = NAMES[qtype]
    rng = np.random.default_rng(77 + qtype)
    rows, cols = 768, 40
    stride = O.row_bytes(qtype, rows) + 10  # padded column view
    raw = rng.integers(0, 256, cols * stride, dtype=np.uint8)
    blocks_view = raw.reshape(cols, stride)[:, :O.row_bytes(qtype, rows)].reshape(cols, -1, O.BLOCK_BYTES[qtype])
    dpos = 208 if qtype == O.Q6_K else 0
    blocks_view[:, ::3, dpos + 1] &= 0x83
    want = np.zeros(shim.quants_packed_bytes(rows, cols), dtype=np.uint8)
    assert shim.quants_repack(raw.ctypes.data, stride, want.ctypes.data, want.size, rows, cols) == want.size
    ref_err = capfd.readouterr().err
    got = quants.repack(name, raw, rows, cols, stride)
    ours_err = capfd.readouterr().err
    assert np.array_equal(got, want)
    assert ours_err == ref_err and ours_err.count("\n") == 1


@pytest.mark.parametrize("name", ["q4_0", "q8_0", "q6_k"])
def test_host_repack_errors_return_zero(spiral_lib, name):
    L = spiral_lib
    rc = getattr(L, f"quants_{name}_record_count")
    pb = getattr(L, f"quants_{name}_packed_bytes")
    rp = getattr(L, f"quants_{name}_repack")
    record_rows = quants.RECORD_ROWS[name]
    assert rc(record_rows, 8) == 1 and rc(record_rows, 7) == 0 and rc(record_rows - 32, 8) == 0
    assert rc(0, 8) == 0 and rc(record_rows, 0) == 0 and rc(-record_rows, 8) == 0
    assert pb(record_rows * 2, 16) == 4 * quants.RECORD_BYTES[name]
    qtype = {"q4_0": O.Q4_0, "q8_0": O.Q8_0, "q6_k": O.Q6_K}[name]
    stride = O.row_bytes(qtype, record_rows)
    src = np.zeros(8 * stride, dtype=np.uint8)
    dst = np.zeros(pb(record_rows, 8), dtype=np.uint8)
    vp = ctypes.c_void_p
    assert rp(vp(src.ctypes.data), stride, vp(dst.ctypes.data), dst.size, record_rows, 8) == dst.size
    assert rp(vp(src.ctypes.data), stride, vp(dst.ctypes.data), dst.size - 1, record_rows, 8) == 0
    assert rp(vp(src.ctypes.data), stride - 1, vp(dst.ctypes.data), dst.size, record_rows, 8) == 0
    assert rp(None, stride, vp(dst.ctypes.data), dst.size, record_rows, 8) == 0
    assert rp(vp(src.ctypes.data), stride, None, dst.size, record_rows, 8) == 0


def test_sizes(spiral_lib):
    L = spiral_lib
    assert L.spiral_row_bytes(_lib.TYPE_Q4_0, 4096) == 2304
    assert L.spiral_row_bytes(_lib.TYPE_Q8_0, 4096) == 4352
    assert L.spiral_row_bytes(_lib.TYPE_Q6_K, 14336) == 11760
    assert L.spiral_row_bytes(_lib.TYPE_Q6_K, 100) == 0
    assert L.spiral_row_bytes(_lib.TYPE_F32, 64) == 0
    assert L.spiral_tensor_bytes(_lib.TYPE_Q8_0, 14336, 4096) == 62_390_272
    assert L.spiral_tensor_bytes(_lib.TYPE_Q6_K, 4096, 14336) == 48_168_960
    assert L.spiral_tensor_bytes(_lib.TYPE_Q4_0, 4096, 4096) == 9_437_184
    assert L.spiral_mul_mat_id_workspace_bytes(128, 64, 8) == 4 * (129 + 512)
    # GEMV (m = 1) and the small-batch form (m = 2..16) need no workspace; the
    # GEMM packs m rows (rounded up to 16) of k bf16
    assert L.spiral_mul_mat_workspace_bytes(_lib.TYPE_Q8_0, 14336, 4096, 1) == 0
    for m in (2, 4, 16):
        assert L.spiral_mul_mat_workspace_bytes(_lib.TYPE_Q4_0, 14336, 4096, m) == 0
        assert L.spiral_mul_mat_workspace_bytes(_lib.TYPE_Q6_K, 4096, 14336, m) == 0
    assert L.spiral_mul_mat_workspace_bytes(_lib.TYPE_Q4_0, 4096, 4096, 17) == 32 * 4096 * 2
    assert L.spiral_mul_mat_workspace_bytes(_lib.TYPE_Q4_0, 4096, 4096, 512) == 512 * 4096 * 2
    assert L.spiral_mul_mat_workspace_bytes(_lib.TYPE_Q4_0, 4096, 4096, 130) == 144 * 4096 * 2
    assert L.spiral_mul_mat_workspace_bytes(_lib.TYPE_Q6_K, 4096, 100, 4) == 0  # k not a block multiple


def test_validation_before_device_work(spiral_lib):
    """Bad arguments are reported without touching a device; with valid
    arguments and no device the call says so (SPIRAL_ERR_NO_DEVICE) instead
    of falling back to anything."""
    L = spiral_lib
    p = ctypes.c_void_p(4096)  # aligned dummy pointer, never dereferenced
    q4 = _lib.TYPE_Q4_0
    assert L.spiral_dequant_bf16(_lib.TYPE_F32, p, 4, 64, p, 64, None) == 6
    assert L.spiral_dequant_bf16(q4, None, 4, 64, p, 64, None) == 3
    assert L.spiral_dequant_bf16(q4, p, 4, 48, p, 64, None) == 1
    assert L.spiral_dequant_bf16(q4, p, 0, 64, p, 64, None) == 1
    assert L.spiral_dequant_bf16(q4, ctypes.c_void_p(4100), 4, 64, p, 64, None) == 2
    assert L.spiral_mul_mat(q4, p, 4, 64, p, 64, 1, p, _lib.TYPE_I32, 4, None, 0, None) == 6
    assert L.spiral_mul_mat(q4, p, 4, 64, p, 60, 1, p, _lib.TYPE_F32, 4, None, 0, None) == 1
    assert L.spiral_mul_mat(_lib.TYPE_Q6_K, p, 4, 64, p, 64, 1, p, _lib.TYPE_F32, 4, None, 0, None) == 1
    # the GEMM path (m > 16) needs its workspace: missing -> NULL, short -> CAPACITY, misaligned -> ALIGN
    assert L.spiral_mul_mat(q4, p, 4, 64, p, 64, 20, p, _lib.TYPE_F32, 4, None, 0, None) == 3
    assert L.spiral_mul_mat(q4, p, 4, 64, p, 64, 20, p, _lib.TYPE_F32, 4, p, 32 * 64 * 2 - 1, None) == 7
    assert L.spiral_mul_mat(q4, p, 4, 64, p, 64, 20, p, _lib.TYPE_F32, 4, ctypes.c_void_p(4104), 8192, None) == 2
    # the small-batch form (m = 2..16) takes none
    assert L.spiral_mul_mat(q4, p, 4, 64, p, 60, 8, p, _lib.TYPE_F32, 4, None, 0, None) == 1
    assert L.spiral_get_rows(q4, p, 4, 64, p, 0, p, _lib.TYPE_F32, 64, None) == 0  # empty is a no-op
    assert L.spiral_mul_mat_id(q4, p, 32, 4, 4, 64, p, 3, p, 2, 2, p, _lib.TYPE_F32, p, 1 << 20, None) == 1
    assert L.spiral_mul_mat_id(q4, p, 144, 4, 4, 64, p, 1, p, 2, 2, p, _lib.TYPE_F32, p, 4, None) == 7
    assert L.quants_unpack_all(q4, p, 96, 8, p, None) == 1
    # fused MUL_MAT_ID + GLU: unknown / unimplemented GLU op, bad swapped flag, odd row count
    assert L.spiral_mul_mat_id_glu(q4, p, 144, 4, 4, 64, p, 1, p, 2, 2, 3, 0, p, _lib.TYPE_F32, p, 1 << 20, None) == 6
    assert L.spiral_mul_mat_id_glu(q4, p, 144, 4, 4, 64, p, 1, p, 2, 2, 2, 2, p, _lib.TYPE_F32, p, 1 << 20, None) == 6
    assert L.spiral_mul_mat_id_glu(q4, p, 144, 4, 5, 64, p, 1, p, 2, 2, 2, 0, p, _lib.TYPE_F32, p, 1 << 20, None) == 1
    assert L.spiral_glu(7, 0, p, 8, 4, 2, p, 4, None) == 6
    assert L.spiral_glu(2, 0, p, 7, 4, 2, p, 4, None) == 1  # ldx < 2F
    assert L.spiral_glu(2, 0, p, 8, 4, 0, p, 4, None) == 0  # no rows: a no-op
    # SWIGLU_OAI needs alpha and limit: its own entry points, TYPE from the plain ones
    assert L.spiral_glu(3, 0, p, 8, 4, 2, p, 4, None) == 6
    assert L.spiral_glu_split(3, 0, p, 4, p, 4, 4, 2, p, 4, None) == 6
    assert L.spiral_glu_swiglu_oai(2, 1.702, 7.0, p, 8, 4, 2, p, 4, None) == 6  # swapped not 0 / 1
    assert L.spiral_glu_swiglu_oai(0, 1.702, 7.0, p, 7, 4, 2, p, 4, None) == 1  # ldx < 2F
    assert L.spiral_glu_swiglu_oai(0, 1.702, 7.0, p, 8, 4, 0, p, 4, None) == 0  # no rows
    assert L.spiral_glu_split_swiglu_oai(0, 1.702, 7.0, p, 3, p, 4, 4, 2, p, 4, None) == 1  # ldg < F
    assert L.spiral_glu_split_swiglu_oai(0, 1.702, 7.0, None, 4, p, 4, 4, 2, p, 4, None) == 3
    if L.spiral_device_count() == 0:
        assert L.spiral_mul_mat_id_glu(q4, p, 144, 4, 4, 64, p, 1, p, 2, 2, 2, 0, p, _lib.TYPE_F32, p, 1 << 20,
                                       None) == 4
        assert L.spiral_glu(2, 1, p, 8, 4, 2, p, 4, None) == 4
        assert L.spiral_glu_swiglu_oai(1, 1.702, 7.0, p, 8, 4, 2, p, 4, None) == 4
        assert L.spiral_dequant_bf16(q4, p, 4, 64, p, 64, None) == 4
        assert L.spiral_mul_mat(q4, p, 4, 64, p, 64, 1, p, _lib.TYPE_F32, 4, None, 0, None) == 4
        assert L.spiral_mul_mat(q4, p, 4, 64, p, 64, 20, p, _lib.TYPE_F32, 4, p, 8192, None) == 4
        assert L.spiral_mul_mat(q4, p, 4, 64, p, 64, 8, p, _lib.TYPE_F32, 4, None, 0, None) == 4
        assert L.quants_unpack_all(q4, p, 64, 8, p, None) == 4


def test_repack_warning_route(spiral_lib, capfd):
    """quants_set_repack_warn reroutes the one warning line of a repack (the
    reference's QUANTS_REPACK_WARN, src/quants/common/repack.h:9-14): to the
    callback while one is set, to nothing with a callback that drops it, and
    back to stderr after resetting to NULL."""
    rows, cols = 64, 8
    raw = synth_q4_0_columns(rows, cols)
    raw.reshape(cols, -1, 18)[3, 1, :2] = (0x01, 0x00)  # one subnormal scale
    lines = []
    cb_type = ctypes.CFUNCTYPE(None, ctypes.c_char_p, ctypes.c_void_p)
    keep = cb_type(lambda line, user: lines.append((line.decode(), user)))
    drop = cb_type(lambda line, user: None)
    L = spiral_lib
    try:
        L.quants_set_repack_warn(ctypes.cast(keep, ctypes.c_void_p), ctypes.c_void_p(1234))
        quants.repack("q4_0", raw, rows, cols)
        assert lines == [("quants: Q4_0 repack flushed subnormal fp16 scales to zero\n", 1234)]
        assert capfd.readouterr().err == ""
        L.quants_set_repack_warn(ctypes.cast(drop, ctypes.c_void_p), None)
        quants.repack("q4_0", raw, rows, cols)
        assert capfd.readouterr().err == "" and len(lines) == 1
    finally:
        L.quants_set_repack_warn(None, None)
    quants.repack("q4_0", raw, rows, cols)
    assert capfd.readouterr().err == "quants: Q4_0 repack flushed subnormal fp16 scales to zero\n"


def synth_q4_0_columns(rows, cols):
    from spiral_amd import synth
    return synth.make_weights(O.Q4_0, cols, rows, 3)


def test_repack_wrapper_checks_the_source_span(spiral_lib):
    """The numpy wrapper refuses a source array shorter than the strided view
    the C entry point reads, and reports the entry point's 0 as an error."""
    rows, cols = 64, 8
    raw = synth_q4_0_columns(rows, cols)
    with pytest.raises(ValueError, match="do not cover"):
        quants.repack("q4_0", raw[:-1], rows, cols)
    with pytest.raises(ValueError, match="do not cover"):
        quants.repack("q4_0", raw, rows, cols, col_stride=O.row_bytes(O.Q4_0, rows) + 1)
    with pytest.raises(ValueError, match="refused"):
        quants.repack("q4_0", raw, rows, cols, col_stride=O.row_bytes(O.Q4_0, rows) - 1)
    with pytest.raises(ValueError, match="no record layout"):
        quants.repack("q4_0", raw, rows - 32, cols)
    assert quants.repack("q4_0", raw, rows, cols).size == quants.RECORD_BYTES["q4_0"]


def test_glu_fits_predicate(spiral_lib):
    L = spiral_lib
    q4, q6 = _lib.TYPE_Q4_0, _lib.TYPE_Q6_K
    assert L.spiral_mul_mat_id_glu_fits(q4, 1536, 2048) == 1
    assert L.spiral_mul_mat_id_glu_fits(q4, 1536, 4096) == 1
    assert L.spiral_mul_mat_id_glu_fits(q4, 1536, 4096 + 32) == 0
    assert L.spiral_mul_mat_id_glu_fits(q4, 1535, 2048) == 0
    assert L.spiral_mul_mat_id_glu_fits(q6, 64, 2048) == 1
    assert L.spiral_mul_mat_id_glu_fits(q6, 64, 2048 + 32) == 0
    assert L.spiral_mul_mat_id_glu_fits(_lib.TYPE_F32, 64, 2048) == 0
