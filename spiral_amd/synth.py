"""Seeded synthetic GGUF tensors in canonical layout (numpy, host memory).

Distributions follow the benchmark workloads:
  Q4_0  fp16 d ~ U[1e-3, 2e-2], codes U{0..15}
  Q8_0  fp16 d ~ U[1e-3, 1e-2], int8 codes U{-127..127}
  Q6_K  ql, qh random bytes, int8 sub-scales U{1..63}, fp16 d ~ U[1e-4, 1e-3]
  Q4_K / Q5_K  qs (and qh) random bytes, 6-bit scales and mins U{0..63},
        fp16 d ~ U[1e-4, 1e-3], dmin ~ U[1e-5, 1e-4] (below 6.1e-5 it is an
        fp16 subnormal, as it often is in real files)
  IQ4_NL  fp16 d ~ U[1e-3, 1e-2], qs random bytes (codebook indices)
  IQ4_XS  fp16 d ~ U[1e-4, 1e-3], 6-bit sub-block scales U{0..63}, qs random
  x     bf16 rounded from N(0, 1)
Canonical layout: n_rows rows of k/block elements; row n starts at
n * row_bytes. The generator is numpy's PCG64 (np.random.default_rng(seed)),
drawn field by field over the whole tensor.
"""

import numpy as np

from . import (BLOCK_BYTES, BLOCK_ELEMS, TYPE_IQ4_NL, TYPE_IQ4_XS, TYPE_Q4_0, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K,
               TYPE_Q8_0)


def bf16_bits(f32):
    """float32 array -> bf16 bit patterns, round to nearest even (finite)."""
    u = np.ascontiguousarray(f32, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bf16_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def _fp16_bits(values):
    return np.asarray(values, dtype=np.float32).astype(np.float16).view(np.uint16)


def make_q4_0(n_rows, k, rng, d_range=(1e-3, 2e-2)):
    nb = n_rows * (k // 32)
    blocks = np.empty((nb, 18), dtype=np.uint8)
    d = _fp16_bits(rng.uniform(d_range[0], d_range[1], nb))
    codes = rng.integers(0, 16, (nb, 32), dtype=np.uint8)
    blocks[:, 0] = d & 0xFF
    blocks[:, 1] = d >> 8
    blocks[:, 2:] = codes[:, :16] | (codes[:, 16:] << 4)
    return blocks.reshape(-1)


def make_q8_0(n_rows, k, rng, d_range=(1e-3, 1e-2)):
    nb = n_rows * (k // 32)
    blocks = np.empty((nb, 34), dtype=np.uint8)
    d = _fp16_bits(rng.uniform(d_range[0], d_range[1], nb))
    blocks[:, 0] = d & 0xFF
    blocks[:, 1] = d >> 8
    blocks[:, 2:] = rng.integers(-127, 128, (nb, 32), dtype=np.int8).view(np.uint8)
    return blocks.reshape(-1)


def make_q6_k(n_rows, k, rng, d_range=(1e-4, 1e-3), sc_range=(1, 63)):
    nb = n_rows * (k // 256)
    blocks = np.empty((nb, 210), dtype=np.uint8)
    blocks[:, 0:192] = rng.integers(0, 256, (nb, 192), dtype=np.uint8)
    blocks[:, 192:208] = rng.integers(sc_range[0], sc_range[1] + 1, (nb, 16)).astype(np.int8).view(np.uint8)
    d = _fp16_bits(rng.uniform(d_range[0], d_range[1], nb))
    blocks[:, 208] = d & 0xFF
    blocks[:, 209] = d >> 8
    return blocks.reshape(-1)


def pack_scale_min(sc, mn):
    """[..., 8] 6-bit scales and mins -> the [..., 12] packed K-quant bytes.

    Field by field: bytes 0..3 and 4..7 hold groups 0..3's scale and min in
    bits 0..5 and bits 4..5 of groups 4..7's in bits 6..7; bytes 8..11 hold
    bits 0..3 of groups 4..7's scale (low nibble) and min (high nibble)."""
    sc = np.asarray(sc, dtype=np.uint8)
    mn = np.asarray(mn, dtype=np.uint8)
    out = np.zeros(sc.shape[:-1] + (12,), dtype=np.uint8)
    out[..., 0:4] = (sc[..., 0:4] & 63) | ((sc[..., 4:8] >> 4) << 6)
    out[..., 4:8] = (mn[..., 0:4] & 63) | ((mn[..., 4:8] >> 4) << 6)
    out[..., 8:12] = (sc[..., 4:8] & 15) | ((mn[..., 4:8] & 15) << 4)
    return out


def make_kquant(qtype, n_rows, k, rng, d_range=(1e-4, 1e-3), dmin_range=(1e-5, 1e-4)):
    nb = n_rows * (k // 256)
    bb = 176 if qtype == TYPE_Q5_K else 144
    blocks = np.empty((nb, bb), dtype=np.uint8)
    d = _fp16_bits(rng.uniform(d_range[0], d_range[1], nb))
    dmin = _fp16_bits(rng.uniform(dmin_range[0], dmin_range[1], nb))
    blocks[:, 0] = d & 0xFF
    blocks[:, 1] = d >> 8
    blocks[:, 2] = dmin & 0xFF
    blocks[:, 3] = dmin >> 8
    blocks[:, 4:16] = pack_scale_min(rng.integers(0, 64, (nb, 8)), rng.integers(0, 64, (nb, 8)))
    blocks[:, 16:] = rng.integers(0, 256, (nb, bb - 16), dtype=np.uint8)
    return blocks.reshape(-1)


def pack_kquant(qtype, d_bits, dmin_bits, sc, mn, codes):
    """One K-quant super-block from its fields: fp16 bit patterns d and dmin,
    8 scales and 8 mins (0..63), 256 codes (0..15 for Q4_K, 0..31 for Q5_K).

    Element 32 g + l takes the low (g even) or high (g odd) nibble of
    qs[32 (g // 2) + l] and, for Q5_K, bit g of qh[l] as its bit 4."""
    codes = np.asarray(codes, dtype=np.int64).reshape(8, 32)
    qs = np.zeros(128, dtype=np.uint8)
    qh = np.zeros(32, dtype=np.uint8)
    for g in range(8):
        nib = (codes[g] & 15).astype(np.uint8)
        qs[32 * (g // 2):32 * (g // 2) + 32] |= nib << (4 * (g & 1))
        qh |= (((codes[g] >> 4) & 1).astype(np.uint8) << g)
    head = np.array([d_bits & 0xFF, d_bits >> 8, dmin_bits & 0xFF, dmin_bits >> 8], dtype=np.uint8)
    parts = [head, pack_scale_min(sc, mn)] + ([qh] if qtype == TYPE_Q5_K else []) + [qs]
    return np.concatenate(parts)


def pack_iq4_xs_scales(ls):
    """[..., 8] 6-bit sub-block scales -> ([...] scales_h as uint16, [..., 4]
    scales_l): sub-block b's low 4 bits in nibble b % 2 of scales_l[b // 2],
    its high 2 bits in bits 2b..2b+1 of scales_h."""
    ls = np.asarray(ls, dtype=np.int64)
    lo = ls & 15
    sl = (lo[..., 0::2] | (lo[..., 1::2] << 4)).astype(np.uint8)
    sh = np.zeros(ls.shape[:-1], dtype=np.int64)
    for b in range(8):
        sh |= ((ls[..., b] >> 4) & 3) << (2 * b)
    return sh.astype(np.uint16), sl


def make_iq4_nl(n_rows, k, rng, d_range=(1e-3, 1e-2)):
    nb = n_rows * (k // 32)
    blocks = np.empty((nb, 18), dtype=np.uint8)
    d = _fp16_bits(rng.uniform(d_range[0], d_range[1], nb))
    blocks[:, 0] = d & 0xFF
    blocks[:, 1] = d >> 8
    blocks[:, 2:] = rng.integers(0, 256, (nb, 16), dtype=np.uint8)
    return blocks.reshape(-1)


def make_iq4_xs(n_rows, k, rng, d_range=(1e-4, 1e-3)):
    nb = n_rows * (k // 256)
    blocks = np.empty((nb, 136), dtype=np.uint8)
    d = _fp16_bits(rng.uniform(d_range[0], d_range[1], nb))
    sh, sl = pack_iq4_xs_scales(rng.integers(0, 64, (nb, 8)))
    blocks[:, 0] = d & 0xFF
    blocks[:, 1] = d >> 8
    blocks[:, 2] = sh & 0xFF
    blocks[:, 3] = sh >> 8
    blocks[:, 4:8] = sl
    blocks[:, 8:] = rng.integers(0, 256, (nb, 128), dtype=np.uint8)
    return blocks.reshape(-1)


def pack_iq4(qtype, d_bits, idx, ls=None):
    """One IQ4_NL block (32 indices) or IQ4_XS super-block (256 indices and 8
    scales) from its fields: element j of a 32-element (sub-)block is the low
    (j < 16) or high nibble of its qs[j % 16]."""
    idx = np.asarray(idx, dtype=np.int64).reshape(-1, 32)
    qs = (idx[:, :16] | (idx[:, 16:] << 4)).astype(np.uint8).reshape(-1)
    head = np.array([d_bits & 0xFF, d_bits >> 8], dtype=np.uint8)
    if qtype == TYPE_IQ4_NL:
        return np.concatenate([head, qs])
    sh, sl = pack_iq4_xs_scales(np.asarray(ls).reshape(8))
    return np.concatenate([head, np.array([int(sh) & 0xFF, int(sh) >> 8], dtype=np.uint8), sl, qs])


MAKERS = {TYPE_Q4_0: make_q4_0, TYPE_Q8_0: make_q8_0, TYPE_Q6_K: make_q6_k,
          TYPE_IQ4_NL: make_iq4_nl, TYPE_IQ4_XS: make_iq4_xs,
          TYPE_Q4_K: lambda n, k, rng: make_kquant(TYPE_Q4_K, n, k, rng),
          TYPE_Q5_K: lambda n, k, rng: make_kquant(TYPE_Q5_K, n, k, rng)}


def make_weights(qtype, n_rows, k, seed):
    if k % BLOCK_ELEMS[qtype] != 0:
        raise ValueError("k must be a multiple of the block size")
    return MAKERS[qtype](n_rows, k, np.random.default_rng(seed))


def make_x(m, k, seed):
    """bf16 bit patterns [m, k] rounded from N(0, 1)."""
    rng = np.random.default_rng(seed)
    return bf16_bits(rng.standard_normal((m, k), dtype=np.float32))


def tensor_bytes(qtype, n_rows, k):
    return n_rows * (k // BLOCK_ELEMS[qtype]) * BLOCK_BYTES[qtype]
