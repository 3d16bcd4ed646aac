"""GPU parity of IQ4_NL / IQ4_XS through the C ABI (every kernel family).

The oracle (oracle/quants_oracle.c, pinned by tests/test_oracle_kquants.py)
follows the reference's plan for these codebook formats
(src/quants/TODO.md:109-124) over ggml's layout and kvalues_iq4nl table:
element bf16_rne(d * kv[index]) (IQ4_NL) and bf16_rne(d * (ls - 32) *
kv[index]) (IQ4_XS), d IEEE binary16, every product exact in fp32. Parity
with ggml itself is unpinned (ggml is not in this container).

Bars, as for the other formats: planar round trip, dequant and GET_ROWS
bit-exact; products within 1e-2 (bf16 out) / 1e-3 (float32 out, every
product form) of the float64 oracle over the exact bf16 weights, the named
relaxed GEMV (scale applied to each block's code sum) within 1e-4 of the
unrounded weights; edge-case weights within TOL * sum_k |w x|.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from spiral_amd import ops, synth
from test_gpu_kquants import (REL_TOL, REL_TOL_EXACT_W, REL_TOL_UNROUNDED_W, _mul_mat, abs_sum, bits,
                              check_bound, dev_bf16, dev_u8, rel_err)

pytestmark = pytest.mark.gpu

IQ4 = [O.IQ4_NL, O.IQ4_XS]
D_SPECIAL = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x8123, 0x7BFF, 0x0400, 0x3C00], dtype=np.uint16)


def iq4_weights(qtype, n_rows, k, seed, specials=True):
    """Synthetic rows; with specials, random blocks get zero, negative,
    subnormal and largest d, and (IQ4_XS) sub-block scales of 0 and 63, and
    all-0 / all-15 indices."""
    raw = synth.make_weights(qtype, n_rows, k, seed)
    if not specials:
        return raw
    blocks = raw.reshape(-1, O.BLOCK_BYTES[qtype])
    rng = np.random.default_rng(seed + 1)
    pick = rng.choice(blocks.shape[0], min(blocks.shape[0], 24), replace=False)
    qs0 = 8 if qtype == O.IQ4_XS else 2
    for i, b in enumerate(pick):
        d = D_SPECIAL[i % 8]
        blocks[b, 0:2] = [d & 0xFF, d >> 8]
        if i % 4 == 1:
            blocks[b, qs0:] = 0x00
        elif i % 4 == 2:
            blocks[b, qs0:] = 0xFF
        if qtype == O.IQ4_XS and i % 3 == 0:
            sh, sl = synth.pack_iq4_xs_scales(np.array([0, 63, 32, 31, 0, 63, 1, 62]))
            blocks[b, 2:4] = [int(sh) & 0xFF, int(sh) >> 8]
            blocks[b, 4:8] = sl
    return raw


@pytest.mark.parametrize("qtype", IQ4)
def test_planar_round_trip_and_planes(cuda, qtype):
    n, k = 37, O.BLOCK_ELEMS[qtype] * 5
    raw = iq4_weights(qtype, n, k, 1)
    rb = O.row_bytes(qtype, k)
    for pad in (0, 14):
        src = np.zeros((n, rb + pad), dtype=np.uint8)
        src[:, :rb] = raw.reshape(n, rb)
        planar = ops.to_planar(qtype, dev_u8(src, cuda), n, k, row_stride=rb + pad)
        back = ops.from_planar(qtype, planar, n, k, row_stride=rb + pad)
        torch.cuda.synchronize()
        assert planar.numel() == raw.size
        assert np.array_equal(back.cpu().numpy().reshape(n, rb + pad)[:, :rb], raw.reshape(n, rb))
    blocks = raw.reshape(-1, O.BLOCK_BYTES[qtype])
    tot = blocks.shape[0]
    p = ops.to_planar(qtype, dev_u8(raw, cuda), n, k).cpu().numpy()
    if qtype == O.IQ4_XS:
        assert np.array_equal(p[:tot * 128].reshape(tot, 128), blocks[:, 8:])
        assert np.array_equal(p[tot * 128:].reshape(tot, 8), blocks[:, :8])
    else:
        assert np.array_equal(p[:tot * 16].reshape(tot, 16), blocks[:, 2:])
        assert np.array_equal(p[tot * 16:].reshape(tot, 2), blocks[:, :2])


@pytest.mark.parametrize("qtype", IQ4)
def test_dequant_bit_exact_with_edge_cases(cuda, qtype):
    n, k = 64, O.BLOCK_ELEMS[qtype] * (24 if qtype == O.IQ4_NL else 8)
    raw = iq4_weights(qtype, n, k, 5)
    w = ops.to_planar(qtype, dev_u8(raw, cuda), n, k)
    assert np.array_equal(bits(ops.dequant(qtype, w, n, k)), O.dequant(qtype, raw, n, k))


@pytest.mark.parametrize("qtype", IQ4)
def test_dequant_4096x4096_bit_exact(cuda, qtype):
    n = k = 4096
    raw = synth.make_weights(qtype, n, k, 3)
    w = ops.to_planar(qtype, dev_u8(raw, cuda), n, k)
    assert np.array_equal(bits(ops.dequant(qtype, w, n, k)), O.dequant(qtype, raw, n, k))


@pytest.mark.parametrize("qtype", IQ4)
def test_get_rows(cuda, qtype):
    n, k = 50, O.BLOCK_ELEMS[qtype] * 4
    raw = iq4_weights(qtype, n, k, 9)
    w = ops.to_planar(qtype, dev_u8(raw, cuda), n, k)
    ids = np.array([0, 49, 7, 7, 23, 1], dtype=np.int32)
    want = O.get_rows(qtype, raw, n, k, ids)
    ids_t = torch.from_numpy(ids).to(cuda)
    assert np.array_equal(bits(ops.get_rows(qtype, w, n, k, ids_t, out_dtype=torch.bfloat16)), want)
    got32 = ops.get_rows(qtype, w, n, k, ids_t, out_dtype=torch.float32).cpu().numpy()
    assert np.array_equal(got32.view(np.uint32), want.astype(np.uint32) << 16)


@pytest.mark.parametrize("qtype,n,k", [(O.IQ4_NL, 1, 32), (O.IQ4_NL, 7, 32 * 17), (O.IQ4_NL, 129, 4096),
                                       (O.IQ4_NL, 70, 14336), (O.IQ4_XS, 5, 256), (O.IQ4_XS, 129, 4096),
                                       (O.IQ4_XS, 70, 14336), (O.IQ4_XS, 33, 256 * 9), (O.IQ4_NL, 46, 32 * 96),
                                       (O.IQ4_XS, 45, 256 * 20)])
def test_gemv(cuda, qtype, n, k):
    """Rows in 16- and 32-lane groups (masked tasks at 32 * 17 and 256 * 9),
    x in registers, several passes with x from LDS."""
    raw = iq4_weights(qtype, n, k, 20 + n, specials=False)
    for out_dtype in (torch.bfloat16, torch.float32):
        y, x = _mul_mat(cuda, qtype, raw, n, k, 1, 21 + n, out_dtype)
        ref = O.matmul_f64(O.dequant(qtype, raw, n, k), x)
        bar = REL_TOL if out_dtype == torch.bfloat16 else REL_TOL_EXACT_W
        assert rel_err(y, ref) <= bar, rel_err(y, ref)
    # the named relaxed mode (weights not rounded to bf16): its own oracle
    w = ops.to_planar(qtype, dev_u8(raw, cuda), n, k)
    y = ops.gemv_relaxed(qtype, w, n, k, dev_bf16(x, cuda), out_dtype=torch.float32).cpu().numpy()
    ref_u = O.matmul_f64_exact(O.dequant_exact(qtype, raw, n, k), x)
    assert rel_err(y, ref_u) <= REL_TOL_UNROUNDED_W, rel_err(y, ref_u)


@pytest.mark.parametrize("qtype", IQ4)
@pytest.mark.parametrize("m", [2, 4, 16])
def test_small_batch(cuda, qtype, m):
    # IQ4_NL: k not a multiple of 128 (a short last step)
    n, k = 300, (32 * 13 if qtype == O.IQ4_NL else 256 * 5)
    raw = iq4_weights(qtype, n, k, 40 + m, specials=False)
    y, x = _mul_mat(cuda, qtype, raw, n, k, m, 41 + m, torch.float32)
    ref = O.matmul_f64(O.dequant(qtype, raw, n, k), x)
    assert rel_err(y, ref) <= REL_TOL_EXACT_W, rel_err(y, ref)


@pytest.mark.parametrize("qtype", IQ4)
def test_small_batch_k_windows(cuda, qtype):
    n, k = 200, 14336
    raw = iq4_weights(qtype, n, k, 60, specials=False)
    y, x = _mul_mat(cuda, qtype, raw, n, k, 16, 61, torch.float32)
    ref = O.matmul_f64(O.dequant(qtype, raw, n, k), x)
    assert rel_err(y, ref) <= REL_TOL_EXACT_W, rel_err(y, ref)


@pytest.mark.parametrize("qtype", IQ4)
@pytest.mark.parametrize("m,n,k_blocks", [(17, 64, 9), (130, 257, 3), (512, 512, 16)])
def test_gemm(cuda, qtype, m, n, k_blocks):
    k = O.BLOCK_ELEMS[qtype] * k_blocks
    raw = iq4_weights(qtype, n, k, 30 + m, specials=False)
    y, x = _mul_mat(cuda, qtype, raw, n, k, m, 31 + m, torch.float32)
    ref = O.matmul_f64(O.dequant(qtype, raw, n, k), x)
    assert rel_err(y, ref) <= REL_TOL_EXACT_W, rel_err(y, ref)


@pytest.mark.parametrize("qtype", IQ4)
@pytest.mark.parametrize("m", [1, 4, 40])
def test_edge_case_weights_every_product(cuda, qtype, m):
    n, k = 96, O.BLOCK_ELEMS[qtype] * (48 if qtype == O.IQ4_NL else 6)
    raw = iq4_weights(qtype, n, k, 70 + m)
    wb = O.dequant(qtype, raw, n, k)
    for out_dtype, tol in ((torch.float32, 1e-3), (torch.bfloat16, 1e-2)):
        y, x = _mul_mat(cuda, qtype, raw, n, k, m, 71 + m, out_dtype)
        check_bound(y, O.matmul_f64(wb, x), wb, x, tol)


def _moe(cuda, qtype, n_expert, n, k, n_tokens, top_k, x_slots, seed, specials=False, glu=False):
    rng = np.random.default_rng(seed)
    per = O.row_bytes(qtype, k) * n
    raws = [iq4_weights(qtype, n, k, seed * 100 + e, specials) for e in range(n_expert)]
    w = torch.empty(n_expert * per, dtype=torch.uint8, device=cuda)
    for e, r in enumerate(raws):
        w[e * per:(e + 1) * per] = ops.to_planar(qtype, dev_u8(r, cuda), n, k)
    ids = np.stack([rng.choice(n_expert, top_k, replace=False) for _ in range(n_tokens)]).astype(np.int32)
    ids[1, 0] = -1
    x = synth.make_x(n_tokens * x_slots, k, seed + 7).reshape(n_tokens, x_slots, k)
    xd, idd = dev_bf16(x, cuda), torch.from_numpy(ids).to(cuda)
    if glu:
        y = ops.mul_mat_id_glu(qtype, w, per, n_expert, n, k, xd, idd, ops.GLU_SWIGLU, out_dtype=torch.float32)
    else:
        y = ops.mul_mat_id(qtype, w, per, n_expert, n, k, xd, idd, out_dtype=torch.float32)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    deq = [O.dequant(qtype, r, n, k) for r in raws]
    ref = np.zeros((n_tokens, top_k, n))
    bound = np.zeros((n_tokens, top_k, n))
    for t in range(n_tokens):
        for s in range(top_k):
            e = ids[t, s]
            if e < 0:
                continue
            xs = x[t, s % x_slots][None, :]
            ref[t, s] = O.matmul_f64(deq[e], xs)[0]
            bound[t, s] = abs_sum(deq[e], xs)[0]
    return y, ref, bound


@pytest.mark.parametrize("qtype", IQ4)
@pytest.mark.parametrize("k,x_slots", [(1024, 1), (2048, 3), (4608, 1)])
def test_mul_mat_id(cuda, qtype, k, x_slots):
    """Streaming form (k <= 4096; one expert past 16 pairs) and the
    LDS-staged form (k = 4608); an id routed nowhere gives a zero row."""
    y, ref, _ = _moe(cuda, qtype, 8, 96, k, 40, 3, x_slots, 11 + k)
    assert not y[1, 0].any()
    assert rel_err(y, ref) <= REL_TOL_EXACT_W, rel_err(y, ref)


def test_mul_mat_id_iq4_nl_ragged_k(cuda):
    """IQ4_NL experts with k not a multiple of 128 (a short last step), both
    MoE forms."""
    for k in (32 * 9, 32 * 145):
        y, ref, _ = _moe(cuda, O.IQ4_NL, 6, 80, k, 30, 2, 1, 15 + k)
        assert rel_err(y, ref) <= REL_TOL_EXACT_W, (k, rel_err(y, ref))


@pytest.mark.parametrize("qtype", IQ4)
def test_mul_mat_id_edge_cases_and_glu(cuda, qtype):
    k = O.BLOCK_ELEMS[qtype] * (48 if qtype == O.IQ4_NL else 6)
    y, ref, bound = _moe(cuda, qtype, 6, 64, k, 30, 2, 2, 12, specials=True)
    assert np.all(np.abs(y - ref) <= 1e-3 * bound + 1e-30)
    F = 80
    y, ref, _ = _moe(cuda, qtype, 8, 2 * F, 1024, 24, 2, 1, 13, glu=True)
    want = O.glu_f64(ref, O.GLU_SWIGLU)
    assert rel_err(y, want) <= REL_TOL_EXACT_W * 4, rel_err(y, want)
