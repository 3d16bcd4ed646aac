"""Pins the oracle's Q4_K / Q5_K dequantization (CPU, no GPU).

The reference plans these formats (src/quants/TODO.md:16-17,80-107) but holds
no code, records or vectors for them, and ggml (whose block_q4_K / block_q5_K
byte layout they use) is not in this container: parity with ggml itself is
unpinned. The oracle is pinned instead by checks a plausible mistake fails:

  - the 6-bit scale/min fields: blocks packed by an independent field-wise
    packer (spiral_amd.synth.pack_scale_min) over every (scale, min) pair at
    every group decode back to those pairs (a wrong shift, mask, byte offset
    or a swapped scale/min fails);
  - element order, nibble and qh-bit placement and the sign of the min term:
    blocks whose scales and mins reduce the K-quant to d' * (q - c) equal the
    already-pinned Q8_0 oracle on the same codes, element by element;
  - d and dmin: IEEE binary16, subnormals included (numpy);
  - the single rounding: fmaf(d * scale, q, -dmin * min) against exact
    rationals rounded once to float32 and then to bf16 by torch.
"""

from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import oracle as O
from spiral_amd import synth

KQ = [O.Q4_K, O.Q5_K]
ONE = 0x3C00  # fp16 1.0


def _bf16_to_f64(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def _blocks(qtype, fields):
    return np.concatenate([synth.pack_kquant(qtype, *f) for f in fields])


@pytest.mark.parametrize("qtype", KQ)
def test_scale_min_fields_every_pair_every_group(oracle, qtype):
    """4096 blocks; group g of block b carries pair (b + 517 g) % 4096, so each
    group sees every (scale, min) once. Codes 0 in the first 16 elements of a
    group give -min; codes c1 in the last 16 give c1 * scale - min (c1 = 17
    for Q5_K, so its high bit counts). d = dmin = 1.0: every value is an
    integer, exact in float32 and rounded once to bf16."""
    c1 = 17 if qtype == O.Q5_K else 1
    nblk = 4096
    pair = (np.arange(nblk)[:, None] + 517 * np.arange(8)[None, :]) % 4096
    sc, mn = pair // 64, pair % 64
    codes = np.zeros((nblk, 8, 32), dtype=np.int64)
    codes[:, :, 16:] = c1
    raw = _blocks(qtype, [(ONE, ONE, sc[b], mn[b], codes[b]) for b in range(nblk)])
    got = _bf16_to_f64(O.dequant(qtype, raw, nblk, 256)).reshape(nblk, 8, 32)
    hi = torch.tensor((c1 * sc - mn).astype(np.float32)).to(torch.bfloat16).to(torch.float64).numpy()
    assert np.array_equal(got[:, :, :16], np.broadcast_to(-mn[:, :, None], (nblk, 8, 16)).astype(np.float64))
    assert np.array_equal(got[:, :, 16:], np.broadcast_to(hi[:, :, None], (nblk, 8, 16)))


def test_scale_min_packer_places_bits_where_the_layout_says():
    """The packer itself against the layout, byte by byte, for one hand-set
    case: scales 1..8 and mins 33..40 (so the bits above 15 are set for
    groups 4..7's mins only)."""
    sc = np.arange(1, 9)
    mn = np.arange(33, 41)
    b = synth.pack_scale_min(sc, mn)
    assert list(b[0:4]) == [1, 2, 3, 4]                        # scales 0..3; scales 4..7 < 16
    assert list(b[4:8]) == [33 | 0x80, 34 | 0x80, 35 | 0x80, 36 | 0x80]  # mins 0..3; bit 5 of mins 4..7 (37..40 >= 32)
    assert list(b[8:12]) == [5 | (37 & 15) << 4, 6 | (38 & 15) << 4, 7 | (39 & 15) << 4, 8 | (40 & 15) << 4]


def _q8_0_blocks(codes_signed, d_bits):
    """Canonical Q8_0 blocks (fp16 d, int8 codes) for 32-element rows."""
    codes = np.asarray(codes_signed, dtype=np.int64).reshape(-1, 32)
    out = np.empty((codes.shape[0], 34), dtype=np.uint8)
    out[:, 0] = d_bits & 0xFF
    out[:, 1] = d_bits >> 8
    out[:, 2:] = codes.astype(np.int8).view(np.uint8)
    return out.reshape(-1)


@pytest.mark.parametrize("qtype", KQ)
def test_reduces_to_q8_0(oracle, qtype):
    """With dmin = d and min = c * scale, every element is d * scale * (q - c):
    a Q8_0 block with scale d * scale (exact in fp16 for d a power of two) and
    codes q - c. c = 8 (Q4_K) or 16 (Q5_K) keeps the codes in int8. Random
    codes, several scales, the element order taken from nothing but the Q8_0
    oracle's linear order."""
    rng = np.random.default_rng(5)
    top, c = (32, 16) if qtype == O.Q5_K else (16, 8)
    nblk = 24
    d_exp = rng.integers(-12, 0, nblk)
    fields, q8 = [], []
    for b in range(nblk):
        d = np.float16(2.0 ** d_exp[b])
        sc = rng.integers(1, 63 // c + 1, 8)   # min = c * sc <= 63
        codes = rng.integers(0, top, 256)
        fields.append((int(d.view(np.uint16)), int(d.view(np.uint16)), sc, c * sc, codes))
        for g in range(8):
            ds = np.float16(float(d) * sc[g])
            q8.append(_q8_0_blocks(codes[32 * g:32 * g + 32] - c, int(ds.view(np.uint16))))
    raw = _blocks(qtype, fields)
    got = O.dequant(qtype, raw, nblk, 256)
    ref = O.dequant(O.Q8_0, np.concatenate(q8), nblk, 256)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("qtype", KQ)
def test_subnormal_scales_are_ieee(oracle, qtype):
    """d and dmin decode as IEEE binary16, subnormals keeping their value (not
    the +0 of the Q4_0 / Q8_0 / Q6_K device rule)."""
    rng = np.random.default_rng(6)
    for d_bits, dmin_bits in [(0x0001, 0x0003), (0x03FF, 0x0200), (0x0400, 0x0001), (0x8005, 0x0011)]:
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        codes = rng.integers(0, 32 if qtype == O.Q5_K else 16, 256)
        raw = synth.pack_kquant(qtype, d_bits, dmin_bits, sc, mn, codes)
        got = _bf16_to_f64(O.dequant(qtype, raw, 1, 256))[0]
        d = float(np.uint16(d_bits).view(np.float16))
        dmin = float(np.uint16(dmin_bits).view(np.float16))
        exact = np.repeat(d * sc, 32) * codes - np.repeat(dmin * mn, 32)  # exact in float64 here
        ref = torch.tensor(exact, dtype=torch.float64).to(torch.float32).to(torch.bfloat16).to(torch.float64).numpy()
        assert np.array_equal(got, ref), (hex(d_bits), hex(dmin_bits))


@pytest.mark.parametrize("qtype", KQ)
def test_single_rounding_against_exact_rationals(oracle, qtype):
    """Random blocks: each element is the exact rational d*sc*q - dmin*m
    rounded once to float32 (round-to-nearest-even, by torch from a float64
    that holds it exactly) and then to bf16; the unrounded oracle (dequant_exact)
    holds the exact value."""
    raw = synth.make_weights(qtype, 6, 512, 7)
    got = O.dequant(qtype, raw, 6, 512)
    exact = O.dequant_exact(qtype, raw, 6, 512)
    blocks = raw.reshape(-1, O.BLOCK_BYTES[qtype])
    for b in range(0, blocks.shape[0], 3):
        blk = blocks[b]
        d = Fraction(float(blk[0:2].view(np.float16)[0]))
        dmin = Fraction(float(blk[2:4].view(np.float16)[0]))
        s = blk[4:16].astype(np.int64)
        sc = np.concatenate([s[0:4] & 63, (s[8:12] & 15) | ((s[0:4] >> 6) << 4)])
        mn = np.concatenate([s[4:8] & 63, (s[8:12] >> 4) | ((s[4:8] >> 6) << 4)])
        row, col0 = divmod(b * 256, 512)
        for e in range(0, 256, 37):
            g = e // 32
            v = exact[row, col0 + e]
            # the exact value is of the form d*sc*q - dmin*m with an integer q
            q = (Fraction(v) + dmin * int(mn[g])) / (d * int(sc[g])) if sc[g] else None
            assert q is None or q.denominator == 1, (b, e)
            r = torch.tensor(float(Fraction(v)), dtype=torch.float64).to(torch.float32).to(torch.bfloat16)
            assert int(r.view(torch.int16).item()) & 0xFFFF == int(got[row, col0 + e]), (b, e)


@pytest.mark.parametrize("qtype", KQ)
def test_matmul_over_kquant_weights(oracle, qtype):
    """The f64 matmul oracle over K-quant weights equals numpy's."""
    raw = synth.make_weights(qtype, 5, 768, 8)
    w = O.dequant(qtype, raw, 5, 768)
    x = synth.make_x(3, 768, 9)
    ref = _bf16_to_f64(x).reshape(3, 768) @ _bf16_to_f64(w).reshape(5, 768).T
    assert np.allclose(O.matmul_f64(w, x), ref, rtol=1e-12, atol=1e-12)


# ---- IQ4_NL / IQ4_XS (codebook formats) -------------------------------------------
#
# The reference plans both (src/quants/TODO.md:109-124) with ggml's
# kvalues_iq4nl codebook and holds no code or vectors; ggml is absent, so
# parity with it is unpinned. The codebook is the format's own constant:
KV = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]
IQ4 = [O.IQ4_NL, O.IQ4_XS]


def test_iq4_nl_equals_q8_0_on_the_codebook_values(oracle):
    """IQ4_NL blocks equal the Q8_0 oracle's blocks with codes kv[index] and
    the same d, element by element (nibble order, codebook, scaling); every
    index appears, at every position across the blocks."""
    rng = np.random.default_rng(11)
    nblk = 64
    idx = (np.arange(nblk)[:, None] + np.arange(32)[None, :]) % 16
    d = synth._fp16_bits(rng.uniform(1e-3, 1e-1, nblk))
    raw = np.concatenate([synth.pack_iq4(O.IQ4_NL, int(d[b]), idx[b]) for b in range(nblk)])
    q8 = _q8_0_blocks(np.array(KV)[idx], 0).reshape(nblk, 34)
    q8[:, 0] = d & 0xFF
    q8[:, 1] = d >> 8
    assert np.array_equal(O.dequant(O.IQ4_NL, raw, nblk, 32), O.dequant(O.Q8_0, q8.reshape(-1), nblk, 32))


def test_iq4_xs_sub_blocks_equal_iq4_nl(oracle):
    """An IQ4_XS super-block with d a power of two equals eight IQ4_NL blocks
    with d' = d (ls - 32) (exact in fp16), for every 6-bit ls at every
    sub-block position (an independent packer writes scales_l / scales_h)."""
    rng = np.random.default_rng(12)
    rows = []
    nl = []
    for t in range(64):
        ls = (t + 9 * np.arange(8)) % 64
        e = int(rng.integers(-14, -2))
        d = np.float16(2.0 ** e)
        idx = rng.integers(0, 16, 256)
        rows.append(synth.pack_iq4(O.IQ4_XS, int(d.view(np.uint16)), idx, ls))
        for b in range(8):
            db = np.float16(float(d) * (int(ls[b]) - 32))
            nl.append(synth.pack_iq4(O.IQ4_NL, int(db.view(np.uint16)), idx[32 * b:32 * b + 32]))
    got = O.dequant(O.IQ4_XS, np.concatenate(rows), 64, 256)
    ref = O.dequant(O.IQ4_NL, np.concatenate(nl), 64, 256)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("qtype", IQ4)
def test_iq4_subnormal_d_is_ieee_and_products_exact(oracle, qtype):
    """d decodes as IEEE binary16 (subnormals kept) and every element is
    bf16 of the exact product (rounded once, by torch from float64)."""
    rng = np.random.default_rng(13)
    for d_bits in (0x0001, 0x03FF, 0x8200, 0x3C00, 0x7BFF):
        idx = rng.integers(0, 16, O.BLOCK_ELEMS[qtype])
        ls = rng.integers(0, 64, 8)
        raw = synth.pack_iq4(qtype, d_bits, idx, ls)
        got = _bf16_to_f64(O.dequant(qtype, raw, 1, O.BLOCK_ELEMS[qtype]))[0]
        d = float(np.uint16(d_bits).view(np.float16))
        scale = np.repeat(ls - 32, 32) if qtype == O.IQ4_XS else 1
        exact = d * scale * np.array(KV)[idx]
        ref = torch.tensor(exact, dtype=torch.float64).to(torch.float32).to(torch.bfloat16).to(torch.float64).numpy()
        assert np.array_equal(got, ref), hex(d_bits)
        assert np.array_equal(O.dequant_exact(qtype, raw, 1, O.BLOCK_ELEMS[qtype])[0], exact)
