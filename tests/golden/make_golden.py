"""Regenerates the committed fixtures in tests/golden/.

    python tests/golden/make_golden.py

special_blocks.json
    Hand-chosen canonical blocks with expected bf16 outputs computed from the
    format description with exact rational arithmetic, rounded by torch's
    float32 -> bfloat16 conversion (round to nearest even). Covers every
    Q4_0 code at several scales (including d = -0, a subnormal d and an
    exponent-31 d, which the reference decodes as 0, 0 and 2^16 * 1.m), every
    int8 code for Q8_0 including -128, and Q6_K blocks with patterned fields.

ref_records.npz
    Seeded canonical inputs and the record streams the reference's own repack
    (src/quants/<fmt>/repack.h, compiled from /root/reference into oracle/_ref
    by oracle/Makefile) produces for them. Needs oracle/_ref; the file is data
    so that checks run where the reference tree is absent.
"""

import ctypes
import json
import sys
from fractions import Fraction
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

from oracle import oracle as O  # noqa: E402


def fp16_exact(bits):
    """Device-decoded scale as an exact Python float (exponent 0 -> +0.0)."""
    e = (bits >> 10) & 31
    if e == 0:
        return 0.0
    m = bits & 0x3FF
    s = -1 if bits & 0x8000 else 1
    return float(s * Fraction(1024 + m, 1024) * (Fraction(2) ** ((e - 15) if e != 31 else 16)))


def bf16(v):
    """Round an exactly representable product to bf16 with torch (RNE). The
    products are formed in float64, exactly, so a zero keeps its IEEE sign
    (code times scale), as in the reference's numpy oracle."""
    f = np.array([v], dtype=np.float32)
    assert float(f[0]) == v
    return int(torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)[0])


def q4_0_block(d_bits, codes):
    blk = [d_bits & 0xFF, d_bits >> 8] + [codes[j] | (codes[j + 16] << 4) for j in range(16)]
    d = fp16_exact(d_bits)
    return blk, [bf16(float(c - 8) * d) for c in codes]


def q8_0_block(d_bits, codes):
    blk = [d_bits & 0xFF, d_bits >> 8] + [c & 0xFF for c in codes]
    d = fp16_exact(d_bits)
    return blk, [bf16(float(c) * d) for c in codes]


def q6_k_block(ql, qh, sc, d_bits):
    blk = list(ql) + list(qh) + [s & 0xFF for s in sc] + [d_bits & 0xFF, d_bits >> 8]
    d = fp16_exact(d_bits)
    vals = []
    for e in range(256):
        h, r = divmod(e, 128)
        j, l = divmod(r, 32)
        byte = ql[64 * h + 32 * (j % 2) + l]
        nib = (byte >> 4) if j >= 2 else (byte & 15)
        q = nib | (((qh[32 * h + l] >> (2 * j)) & 3) << 4)
        vals.append(bf16((d * float(sc[8 * h + l // 16 + 2 * j])) * float(q - 32)))
    return blk, vals


def special_blocks():
    cases = []
    all16 = list(range(16)) * 2
    for name, d in [("q4_0 d=1", 0x3C00), ("q4_0 d=0.5", 0x3800), ("q4_0 d=-2", 0xC000),
                    ("q4_0 d=0.0999", 0x2E66), ("q4_0 d subnormal", 0x0001), ("q4_0 d=-0", 0x8000),
                    ("q4_0 d exp31", 0x7C01), ("q4_0 d max normal", 0x7BFF)]:
        blk, want = q4_0_block(d, all16)
        cases.append(dict(name=name, format="q4_0", block=blk, bf16=want))
    codes = list(range(-128, 128))
    for i in range(8):
        for name, d in [("q8_0 d=0.00733", 0x1F81), ("q8_0 d=-3.14", 0xC248)]:
            blk, want = q8_0_block(d, codes[32 * i:32 * i + 32])
            cases.append(dict(name=f"{name} codes {32 * i - 128}..", format="q8_0", block=blk, bf16=want))
    ql = [(7 * i + 3) & 0xFF for i in range(128)]
    qh = [(29 * i + 11) & 0xFF for i in range(64)]
    for name, sc, d in [("q6_k ramp", [i - 8 for i in range(16)], 0x1A3D),
                        ("q6_k extremes", [-128, 127, 1, -1, 63, -64, 2, 0, 5, -5, 100, -100, 7, 9, 11, 13], 0xB555),
                        ("q6_k d subnormal", [3] * 16, 0x0200)]:
        blk, want = q6_k_block(ql, qh, sc, d)
        cases.append(dict(name=name, format="q6_k", block=blk, bf16=want))
    return cases


def ref_records():
    out = {}
    for qtype, rows, cols in [(O.Q4_0, 256, 16), (O.Q8_0, 256, 16), (O.Q6_K, 256, 16)]:
        shim = O.ref_shim(qtype)
        if shim is None:
            raise SystemExit("oracle/_ref is not built: run `make -C oracle` with /root/reference present")
        name = O.FORMAT_NAMES[qtype]
        rng = np.random.default_rng(2024 + qtype)
        stride = O.row_bytes(qtype, rows)
        raw = rng.integers(0, 256, cols * stride, dtype=np.uint8)
        blocks = raw.reshape(-1, O.BLOCK_BYTES[qtype])
        dpos = 208 if qtype == O.Q6_K else 0
        blocks[::7, dpos + 1] &= 0x83  # some zero-exponent (flushed) scales
        rec = np.zeros(shim.quants_packed_bytes(rows, cols), dtype=np.uint8)
        n = shim.quants_repack(raw.ctypes.data_as(ctypes.c_void_p), stride,
                               rec.ctypes.data_as(ctypes.c_void_p), rec.size, rows, cols)
        assert n == rec.size
        out[f"{name}_raw"] = raw
        out[f"{name}_shape"] = np.array([rows, cols], dtype=np.int64)
        out[f"{name}_records"] = rec
    return out


def main():
    (HERE / "special_blocks.json").write_text(json.dumps(special_blocks(), separators=(",", ":")))
    np.savez_compressed(HERE / "ref_records.npz", **ref_records())
    print("wrote", HERE / "special_blocks.json", HERE / "ref_records.npz")


if __name__ == "__main__":
    main()
