"""Pins the CPU oracle (oracle/) before anything is checked against it.

Each oracle function is checked by something other than its own formula:
  - fp16 decode: numpy's IEEE binary16 for normal exponents, the reference's
    documented special cases (src/quants/common/scale.aie.h:14-27) for the rest;
  - bf16 rounding: torch's float32 -> bfloat16 conversion;
  - dequant closed form: the reference's split-scale device arithmetic, step by
    step, exhaustively (oq_check_*); exact rational arithmetic on random blocks;
    hand-computed golden blocks (tests/golden/special_blocks.json);
  - record layout: the reference's own repack.h compiled into oracle/_ref, and
    fixtures made from it (tests/golden/ref_records.npz);
  - exact (unrounded) weights: exact fractions, a numpy restatement of Q4_0,
    and rounding them once to bf16 gives dequant's bits;
  - matmul: numpy float64.
"""

import ctypes
import json
from fractions import Fraction
from pathlib import Path

import math

import numpy as np
import pytest
import torch

from oracle import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"
FORMATS = [O.Q4_0, O.Q8_0, O.Q6_K]


# ---- scalar conversions ---------------------------------------------------

def _fp16_expected(h):
    """Device decode rule from the reference text, via numpy for normals."""
    h = np.asarray(h, dtype=np.uint16)
    e = (h >> 10) & 31
    out = h.view(np.float16).astype(np.float32)
    out = np.where(e == 0, np.float32(0.0), out)
    m = (h & 0x3FF).astype(np.float64)
    sign = np.where(h & 0x8000, -1.0, 1.0)
    big = (sign * 65536.0 * (1.0 + m / 1024.0)).astype(np.float32)
    return np.where(e == 31, big, out)


def test_fp16_device_every_pattern(oracle):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.fp16_device(h)
    exp = _fp16_expected(h)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))
    # exponent 0 (both zeros and every subnormal) decodes to +0 bits exactly
    zeros = got[((h >> 10) & 31) == 0]
    assert np.all(zeros.view(np.uint32) == 0)


def test_fp16_ieee_matches_numpy(oracle):
    L = O.lib()
    for h in list(range(0, 65536, 7)) + [0x0001, 0x03FF, 0x8001, 0x7C00, 0xFC00]:
        want = np.array([h], dtype=np.uint16).view(np.float16).astype(np.float32)[0]
        got = np.float32(L.oq_fp16_ieee(h))
        if np.isnan(want):
            assert np.isnan(got)
        else:
            assert got.view(np.uint32) == want.view(np.uint32), hex(h)


def test_bf16_rne_matches_torch(oracle):
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, 400_000, dtype=np.uint64).astype(np.uint32)
    # keep finite values; add exact ties (low half 0x8000) with even and odd keep bits
    exp = (bits >> 23) & 0xFF
    bits = bits[exp != 0xFF]
    ties = (rng.integers(0, 2**16, 50_000, dtype=np.uint32) << 16) | 0x8000
    ties = ties[((ties >> 23) & 0xFF) < 0xFE]
    bits = np.concatenate([bits, ties, np.array([0x00000000, 0x80000000, 0x3F808000, 0x3F818000,
                                                 0x7F7FFFFF & 0x7F7F7FFF], dtype=np.uint32)])
    f = bits.view(np.float32)
    want = torch.from_numpy(f.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = O.bf16_rne(f)
    assert np.array_equal(got, want)


# ---- Appendix-B exhaustiveness: reference device arithmetic == closed form ----

def test_split_hi_lo_is_exact(oracle):
    assert O.lib().oq_check_split_identity() == 0


def test_q_times_d_exhaustive(oracle):
    """Every normal fp16 d (both signs) x every int8 code: the reference's
    two-term bf16 scale arithmetic (src/quants/q4_0/unpack.aie.h:41-45,
    src/quants/q8_0/unpack.aie.h:44-51) rounds to the same bf16 as the closed
    form. Results that differ only in the sign of a zero are counted apart:
    they arise for code 0 with negative d, where the two-term sum gives +0."""
    sz = ctypes.c_int64(0)
    assert O.lib().oq_check_q_times_d(ctypes.byref(sz)) == 0
    assert sz.value <= 30720  # at most one per negative normal d (code 0 only)


def test_q6_k_exhaustive(oracle):
    """Every normal fp16 d x every int8 sub-scale x every centred 6-bit code:
    the reference's three-term split (src/quants/q6_k/unpack.aie.h:33-61,81-91)
    equals bf16_rne(d * sc * (q - 32))."""
    sz = ctypes.c_int64(0)
    assert O.lib().oq_check_q6_k(1, ctypes.byref(sz)) == 0


def test_aie_emulation_catches_a_dropped_term(oracle):
    """The exhaustive check can fail: a one-term scale (hi only, the relaxed
    mode the reference rejects, src/quants/NOTES.md:327-335) differs from the
    closed form for some d."""
    L = O.lib()
    mism = 0
    for h in range(0x3C00, 0x3C00 + 1024, 3):  # d in [1, 2)
        d = np.float32(np.array([h], dtype=np.uint16).view(np.float16)[0])
        hi = O.bf16_rne(np.array([d], dtype=np.float32)).astype(np.uint32) << 16
        one_term = O.bf16_rne((np.float32(7) * hi.view(np.float32)).astype(np.float32))[0]
        if one_term != L.oq_aie_q_times_d(7, h):
            mism += 1
    assert mism > 0


# ---- dequant closed form vs exact arithmetic --------------------------------

def _fp16_exact(bits):
    """Exact rational value of the device-decoded scale."""
    e = (bits >> 10) & 31
    if e == 0:
        return Fraction(0)
    m = bits & 0x3FF
    s = -1 if bits & 0x8000 else 1
    return s * Fraction(1024 + m, 1024) * (Fraction(2) ** (e - 15 if e != 31 else 16))


def _bf16_of_fraction(v):
    # exact value -> float32 (exact for these products) -> torch RNE to bf16
    f = np.array([float(v)], dtype=np.float32)
    assert Fraction(float(f[0])) == v
    return int(torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)[0])


def _exact_values(qtype, blk):
    """Element values of one canonical block, written from the format
    description (src/quants/tests/formats/*.py) with exact fractions."""
    out = []
    if qtype == O.Q4_0:
        d = _fp16_exact(int(blk[0]) | (int(blk[1]) << 8))
        codes = [int(b) & 15 for b in blk[2:18]] + [int(b) >> 4 for b in blk[2:18]]
        out = [(c - 8) * d for c in codes]
    elif qtype == O.Q8_0:
        d = _fp16_exact(int(blk[0]) | (int(blk[1]) << 8))
        out = [int(np.int8(np.uint8(b))) * d for b in blk[2:34]]
    else:
        ql, qh = blk[:128].astype(int), blk[128:192].astype(int)
        sc = blk[192:208].view(np.int8).astype(int)
        d = _fp16_exact(int(blk[208]) | (int(blk[209]) << 8))
        out = [None] * 256
        for e in range(256):
            h, r = divmod(e, 128)
            j, l = divmod(r, 32)
            byte = ql[64 * h + 32 * (j % 2) + l]
            nib = (byte >> 4) if j >= 2 else (byte & 15)
            q = nib | (((qh[32 * h + l] >> (2 * j)) & 3) << 4)
            out[e] = d * sc[8 * h + l // 16 + 2 * j] * (q - 32)
    return out


def _exact_block(qtype, blk):
    return [_bf16_of_fraction(v) for v in _exact_values(qtype, blk)]


@pytest.mark.parametrize("qtype", FORMATS)
def test_dequant_matches_exact_arithmetic(oracle, qtype):
    rng = np.random.default_rng(qtype)
    k = O.BLOCK_ELEMS[qtype] * 2
    n = 3
    raw = rng.integers(0, 256, n * O.row_bytes(qtype, k), dtype=np.uint8)
    bb = O.BLOCK_BYTES[qtype]
    dpos = 0 if qtype != O.Q6_K else 208
    blocks = raw.reshape(-1, bb)
    # random but finite-product scales: any fp16 except exponent 31 on most
    # blocks, plus one block each with exponent 0 and exponent 31
    dbits = rng.integers(0, 0x7C00, blocks.shape[0]).astype(np.uint16) | (
        rng.integers(0, 2, blocks.shape[0]).astype(np.uint16) << 15)
    dbits[0] = 0x0123   # subnormal -> +0
    dbits[1] = 0x7C05   # exponent 31 -> finite 2^16 * (1 + 5/1024)
    blocks[:, dpos] = dbits & 0xFF
    blocks[:, dpos + 1] = dbits >> 8
    got = O.dequant(qtype, raw, n, k)
    want = np.array([_exact_block(qtype, b) for b in blocks], dtype=np.uint16).reshape(n, k)
    # zero results may differ only in sign (see test_q_times_d_exhaustive)
    both_zero = ((got & 0x7FFF) == 0) & ((want & 0x7FFF) == 0)
    assert np.array_equal(np.where(both_zero, 0, got), np.where(both_zero, 0, want))


@pytest.mark.parametrize("qtype", FORMATS)
def test_dequant_exact_matches_fractions_and_rounds_to_dequant(oracle, qtype):
    """The unrounded weights: equal to the exact rational values, and their
    one rounding to bf16 is dequant's output."""
    rng = np.random.default_rng(100 + qtype)
    k = O.BLOCK_ELEMS[qtype] * 3
    n = 4
    raw = rng.integers(0, 256, n * O.row_bytes(qtype, k), dtype=np.uint8)
    blocks = raw.reshape(-1, O.BLOCK_BYTES[qtype])
    dpos = 0 if qtype != O.Q6_K else 208
    dbits = rng.integers(0, 0x7C00, blocks.shape[0]).astype(np.uint16) | (
        rng.integers(0, 2, blocks.shape[0]).astype(np.uint16) << 15)
    dbits[0] = 0x0123   # subnormal -> +0
    dbits[1] = 0x7C05   # exponent 31 -> finite
    blocks[:, dpos] = dbits & 0xFF
    blocks[:, dpos + 1] = dbits >> 8
    got = O.dequant_exact(qtype, raw, n, k)
    want = [v for b in blocks for v in _exact_values(qtype, b)]
    assert all(Fraction(float(g)) == w for g, w in zip(got.reshape(-1), want))
    rounded = O.bf16_rne(got.astype(np.float32))
    bits16 = O.dequant(qtype, raw, n, k)
    both_zero = ((rounded & 0x7FFF) == 0) & ((bits16 & 0x7FFF) == 0)
    assert np.array_equal(np.where(both_zero, 0, rounded), np.where(both_zero, 0, bits16))


def test_dequant_exact_q4_0_numpy_restatement(oracle):
    """Q4_0 from its bytes with numpy alone: (nibble - 8) * d."""
    rng = np.random.default_rng(7)
    n, k = 5, 128
    raw = rng.integers(0, 256, n * O.row_bytes(O.Q4_0, k), dtype=np.uint8)
    blocks = raw.reshape(-1, 18)
    blocks[:, 1] &= 0x7B  # normal, finite scales
    blocks[:, 1] |= 0x04
    d = blocks[:, :2].copy().view(np.float16).astype(np.float64)[:, 0]
    qs = blocks[:, 2:].astype(np.int64)
    vals = np.concatenate([(qs & 15) - 8, (qs >> 4) - 8], axis=1) * d[:, None]
    assert np.array_equal(O.dequant_exact(O.Q4_0, raw, n, k), vals.reshape(n, k))


def test_golden_special_blocks(oracle):
    """Hand-computed blocks: every Q4_0 code at d = 1, 0.5, -2, a subnormal d,
    d = -0 and the exponent-31 quirk; Q8_0 -128..127; Q6_K with known fields."""
    cases = json.loads((GOLDEN / "special_blocks.json").read_text())
    for c in cases:
        qtype = {"q4_0": O.Q4_0, "q8_0": O.Q8_0, "q6_k": O.Q6_K}[c["format"]]
        raw = np.array(c["block"], dtype=np.uint8)
        got = O.dequant(qtype, raw, 1, O.BLOCK_ELEMS[qtype])[0]
        assert got.tolist() == c["bf16"], c["name"]


# ---- reference record layout --------------------------------------------------

def _raw_with_specials(qtype, weights_rows, weights_cols, seed):
    rng = np.random.default_rng(seed)
    stride = O.row_bytes(qtype, weights_rows)
    raw = rng.integers(0, 256, weights_cols * stride, dtype=np.uint8)
    blocks = raw.reshape(-1, O.BLOCK_BYTES[qtype])
    dpos = 208 if qtype == O.Q6_K else 0
    blocks[::5, dpos + 1] &= 0x83  # exponent 0 -> subnormal or zero scale
    return raw, stride


@pytest.mark.parametrize("qtype", FORMATS)
def test_ref_repack_matches_reference_build(oracle, qtype):
    shim = O.ref_shim(qtype)
    if shim is None:
        pytest.skip("reference repack not built here (oracle/_ref); fixtures cover it")
    rows, cols = 512, 24
    raw, stride = _raw_with_specials(qtype, rows, cols, seed=qtype)
    for pad in (0, 6):
        st = stride + pad
        src = np.zeros(cols * st, dtype=np.uint8)
        src.reshape(cols, st)[:, :stride] = raw.reshape(cols, stride)
        want = np.zeros(shim.quants_packed_bytes(rows, cols), dtype=np.uint8)
        assert shim.quants_repack(src.ctypes.data, st, want.ctypes.data, want.size, rows, cols) == want.size
        got, warn = O.ref_repack(qtype, src, rows, cols, stride=st)
        assert np.array_equal(got, want)
        assert warn & 1
    # the 0-on-error convention, case by case
    buf = np.zeros(O.ref_packed_bytes(qtype, rows, cols), dtype=np.uint8)
    L = O.lib()
    for (r, c, st, cap) in [(rows, 4, stride, buf.size), (rows - 32, cols, stride, buf.size),
                            (rows, cols, stride - 2, buf.size), (rows, cols, stride, buf.size - 1),
                            (0, cols, stride, buf.size), (rows, -8, stride, buf.size)]:
        a = shim.quants_repack(raw.ctypes.data, st, buf.ctypes.data, cap, r, c)
        b = L.oq_ref_repack(qtype, raw.ctypes.data, st, buf.ctypes.data, cap, r, c, None)
        assert a == b == 0
        assert shim.quants_packed_bytes(r, c) == L.oq_ref_packed_bytes(qtype, r, c)


@pytest.mark.parametrize("qtype", FORMATS)
def test_ref_repack_matches_fixture(oracle, qtype):
    fx = np.load(GOLDEN / "ref_records.npz")
    name = O.FORMAT_NAMES[qtype]
    raw = fx[f"{name}_raw"]
    rows, cols = (int(v) for v in fx[f"{name}_shape"])
    got, _ = O.ref_repack(qtype, raw, rows, cols)
    assert np.array_equal(got, fx[f"{name}_records"])


@pytest.mark.parametrize("qtype", FORMATS)
def test_ref_unpack_equals_canonical_dequant(oracle, qtype):
    """Decoding the reference's records (its unpack semantics) gives the
    canonical dequant, re-ordered into the reference output order
    (src/quants/tests/formats/q4_0.py:65-79)."""
    rows, cols = 512, 16
    raw, _ = _raw_with_specials(qtype, rows, cols, seed=10 + qtype)
    rec, _ = O.ref_repack(qtype, raw, rows, cols)
    got = O.ref_unpack(qtype, rec, rows, cols)
    want = O.ref_order(O.dequant(qtype, raw, cols, rows), O.REF_RECORD_ROWS[qtype])
    both_zero = ((got & 0x7FFF) == 0) & ((want & 0x7FFF) == 0)
    assert np.array_equal(np.where(both_zero, 0, got), np.where(both_zero, 0, want))


# ---- matmul -------------------------------------------------------------------

def test_matmul_f64_matches_numpy(oracle):
    rng = np.random.default_rng(3)
    w = O.bf16_rne(rng.standard_normal((40, 96)).astype(np.float32))
    x = O.bf16_rne(rng.standard_normal((5, 96)).astype(np.float32))
    wf = (w.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    xf = (x.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    assert np.allclose(O.matmul_f64(w, x), xf @ wf.T, rtol=1e-12, atol=1e-12)
    assert np.allclose(O.matmul_f32(w, x), xf @ wf.T, rtol=1e-5, atol=1e-4)


def test_matmul_f64_exact_matches_numpy(oracle):
    rng = np.random.default_rng(5)
    w = rng.standard_normal((33, 64))
    x = O.bf16_rne(rng.standard_normal((6, 64)).astype(np.float32))
    xf = (x.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    assert np.allclose(O.matmul_f64_exact(w, x), xf @ w.T, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("qtype", FORMATS)
def test_quant_matmul_matches_dequant_then_matmul(oracle, qtype):
    rng = np.random.default_rng(4)
    n, k = 24, 512
    raw = rng.integers(0, 256, n * O.row_bytes(qtype, k), dtype=np.uint8)
    blocks = raw.reshape(-1, O.BLOCK_BYTES[qtype])
    dpos = 208 if qtype == O.Q6_K else 0
    blocks[:, dpos + 1] = 0x20  # modest finite scales
    x = O.bf16_rne(rng.standard_normal((3, k)).astype(np.float32))
    w = O.dequant(qtype, raw, n, k)
    ref = O.matmul_f64(w, x)
    got = O.quant_matmul_f32(qtype, raw, n, k, x, threads=2)
    assert np.allclose(got, ref, rtol=1e-4, atol=1e-3 * np.abs(ref).max())


def test_glu_oracle_closed_forms():
    """The GLU restatement against values the mathematics fixes: relu, silu
    and the logistic at known points, gelu(1) = Phi(1), the tanh form within
    its published 1e-3 of the erf form, x * act at 0, and swapped = the
    halves exchanged (a wrong half or sign fails one of these)."""
    a = np.array([-2.0, -0.5, 0.0, 1.0, 3.0])
    b = np.array([1.0, 2.0, -1.0, 0.5, -2.0])
    h = np.concatenate([a, b])
    assert np.array_equal(O.glu_f64(h, O.GLU_REGLU), np.array([0.0, 0.0, 0.0, 0.5, -6.0]))
    sig1 = 1.0 / (1.0 + math.exp(-1.0))
    assert math.isclose(O.glu_f64(np.array([1.0, 1.0]), O.GLU_SWIGLU)[0], sig1, rel_tol=1e-15)
    assert math.isclose(O.glu_f64(np.array([1.0, 1.0]), O.GLU_GEGLU_ERF)[0], 0.8413447460685429, rel_tol=1e-14)
    assert math.isclose(O.glu_f64(np.array([1.0, 1.0]), O.GLU_GEGLU_QUICK)[0], 1.0 / (1.0 + math.exp(-1.702)),
                        rel_tol=1e-15)
    xs = np.linspace(-4.0, 4.0, 801)
    ones = np.ones_like(xs)
    tanh_form = O.glu_f64(np.concatenate([xs, ones]), O.GLU_GEGLU)
    erf_form = O.glu_f64(np.concatenate([xs, ones]), O.GLU_GEGLU_ERF)
    assert np.max(np.abs(tanh_form - erf_form)) < 1e-3
    silu = O.glu_f64(np.concatenate([xs, ones]), O.GLU_SWIGLU)
    assert np.allclose(silu, xs / (1.0 + np.exp(-xs)), rtol=1e-15)
    for op in (O.GLU_REGLU, O.GLU_GEGLU, O.GLU_SWIGLU, O.GLU_GEGLU_ERF, O.GLU_GEGLU_QUICK):
        assert O.glu_f64(np.array([0.0, 5.0]), op)[0] == 0.0
        assert np.array_equal(O.glu_f64(h, op, swapped=True), O.glu_f64(np.concatenate([b, a]), op))


def test_glu_swiglu_oai_closed_forms():
    """SWIGLU_OAI against what fixes it: with no limit it is SWIGLU (alpha 1)
    and GEGLU_QUICK (alpha 1.702) of a times b + 1; a is capped at limit (not
    below), b clamped to [-limit, limit]; zero at a = 0 and at b = -1; swapped
    exchanges the halves. A dropped + 1, a clamp on the wrong side or a lost
    alpha fails one of these."""
    a = np.array([-6.0, -1.5, 0.0, 0.7, 2.0, 9.0])
    b = np.array([3.0, -0.25, 4.0, 1.0, -1.0, 0.5])
    h = np.concatenate([a, b])
    hb = np.concatenate([a, b + 1.0])
    oai = lambda hh, alpha, limit, **kw: O.glu_f64(hh, O.GLU_SWIGLU_OAI, alpha=alpha, limit=limit, **kw)
    assert np.allclose(oai(h, 1.0, np.inf), O.glu_f64(hb, O.GLU_SWIGLU), rtol=1e-15)
    assert np.allclose(oai(h, 1.702, np.inf), O.glu_f64(hb, O.GLU_GEGLU_QUICK), rtol=1e-15)
    got = oai(h, 1.702, 7.0)
    sig = lambda z: 1.0 / (1.0 + math.exp(-z))
    assert math.isclose(got[5], 7.0 * sig(1.702 * 7.0) * 1.5, rel_tol=1e-15)  # a = 9 capped at 7
    assert math.isclose(got[0], -6.0 * sig(-1.702 * 6.0) * 4.0, rel_tol=1e-15)  # a = -6 kept (no lower cap)
    assert got[2] == 0.0 and got[4] == 0.0
    clamp = oai(np.array([1.0, 1.0, 50.0, -50.0]), 1.702, 7.0)
    assert math.isclose(clamp[0], sig(1.702) * 8.0, rel_tol=1e-15)   # b = 50 -> 7, times (7 + 1)
    assert math.isclose(clamp[1], sig(1.702) * -6.0, rel_tol=1e-15)  # b = -50 -> -7, times (-7 + 1)
    assert np.array_equal(oai(h, 1.702, 7.0, swapped=True), oai(np.concatenate([b, a]), 1.702, 7.0))


# ---- the CPU baseline bench.py times (oracle/cpu_baseline.c) ---------------------

def test_cpu_baseline_matches_the_oracle(oracle):
    """The vectorized, multi-threaded CPU baseline computes what the oracle
    computes: dequant bit for bit, products to fp32 summation order."""
    from spiral_amd import synth
    n, k = 67, 1024
    q4 = synth.make_weights(O.Q4_0, n, k, 31)
    assert np.array_equal(O.cb_dequant_q4_0(q4, n, k, 4), O.dequant(O.Q4_0, q4, n, k))
    q8 = synth.make_weights(O.Q8_0, n, k, 32)
    x = synth.make_x(1, k, 33)
    ref = O.matmul_f64(O.dequant(O.Q8_0, q8, n, k), x)[0]
    got = O.cb_gemv_q8_0(q8, n, k, x, 4)
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref))
    xm = synth.make_x(9, k, 34)
    ref = O.matmul_f64(O.dequant(O.Q4_0, q4, n, k), xm)
    got = O.cb_gemm_q4_0(q4, n, k, xm, 4)
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref))
    k6 = 768
    q6 = synth.make_weights(O.Q6_K, n, k6, 35)
    assert np.array_equal(O.cb_dequant_q6_k(q6, n, k6, 4), O.dequant(O.Q6_K, q6, n, k6))
    x6 = synth.make_x(1, k6, 36)
    ref = O.matmul_f64(O.dequant(O.Q6_K, q6, n, k6), x6)[0]
    got = O.cb_gemv_q6_k(q6, n, k6, x6, 4)
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref))


def test_cpu_baseline_moe_matches_the_oracle(oracle):
    """The grouped CPU MoE leg: each (token, slot) equals the oracle's product
    with its expert, per-slot and shared inputs, an id routed nowhere gives a
    zero row."""
    from spiral_amd import synth
    n_expert, n, k, n_tokens, top_k = 5, 37, 256, 6, 3
    per = n * k // 32 * 18
    raws = [synth.make_weights(O.Q4_0, n, k, 60 + e) for e in range(n_expert)]
    stack = np.concatenate(raws)
    rng = np.random.default_rng(61)
    ids = rng.integers(0, n_expert, (n_tokens, top_k)).astype(np.int32)
    ids[2, 1] = -1
    ids[4, 0] = n_expert
    for x_slots in (1, top_k):
        x = synth.make_x(n_tokens * x_slots, k, 62).reshape(n_tokens, x_slots, k)
        got = O.cb_moe_q4_0(stack, per, n_expert, n, k, x, ids, 3)
        for t in range(n_tokens):
            for s in range(top_k):
                e = ids[t, s]
                if not 0 <= e < n_expert:
                    assert not got[t, s].any()
                    continue
                ref = O.matmul_f64(O.dequant(O.Q4_0, raws[e], n, k), x[t, s % x_slots][None])[0]
                assert np.max(np.abs(got[t, s] - ref)) <= 1e-5 * np.max(np.abs(ref))
