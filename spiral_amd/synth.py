"""Seeded synthetic GGUF tensors in canonical layout (numpy, host memory).

Distributions follow the benchmark workloads:
  Q4_0  fp16 d ~ U[1e-3, 2e-2], codes U{0..15}
  Q8_0  fp16 d ~ U[1e-3, 1e-2], int8 codes U{-127..127}
  Q6_K  ql, qh random bytes, int8 sub-scales U{1..63}, fp16 d ~ U[1e-4, 1e-3]
  x     bf16 rounded from N(0, 1)
Canonical layout: n_rows rows of k/block elements; row n starts at
n * row_bytes. The generator is numpy's PCG64 (np.random.default_rng(seed)),
drawn field by field over the whole tensor.
"""

import numpy as np

from . import BLOCK_BYTES, BLOCK_ELEMS, TYPE_Q4_0, TYPE_Q6_K, TYPE_Q8_0


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


MAKERS = {TYPE_Q4_0: make_q4_0, TYPE_Q8_0: make_q8_0, TYPE_Q6_K: make_q6_k}


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
