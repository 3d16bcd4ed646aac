"""GPU parity of Q4_K / Q5_K through the C ABI (every kernel family).

The oracle (oracle/quants_oracle.c, pinned by tests/test_oracle_kquants.py)
follows the reference's plan for these formats (src/quants/TODO.md:80-107):
element = d * scale * q - dmin * min with d, dmin IEEE binary16, one rounding
to float (fma), then bf16 RNE. Parity with ggml itself is unpinned (ggml is
not in this container).

Bars, as for the other formats:
  - planar round trip, dequant and GET_ROWS: bit-exact;
  - products against the float64 oracle over the exact bf16 weights:
    max |y - ref| / max(|ref|, rms(ref)) <= 1e-2 (bf16 out) and <= 1e-3 for
    float32 output of every product form (GEMV included); the named relaxed
    GEMV (spiral_gemv_relaxed), which applies d * scale and dmin * min to
    each group's code and x sums, against the unrounded weights to 1e-4;
  - edge-case weights (zero, negative, subnormal and largest d / dmin, scales
    and mins of 0 and 63, all-zero and all-top codes): every output within
    TOL * sum_k |w x| of the float64 product (the scale of an fp32 dot
    product's rounding error, which cancellation cannot shrink).
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from spiral_amd import ops, synth

pytestmark = pytest.mark.gpu

KQ = [O.Q4_K, O.Q5_K]
REL_TOL = 1e-2
REL_TOL_EXACT_W = 1e-3
REL_TOL_UNROUNDED_W = 1e-4


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def dev_u8(a, device):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).to(device)


def dev_bf16(a_u16, device):
    return torch.from_numpy(np.ascontiguousarray(a_u16, dtype=np.uint16).view(np.int16)).view(torch.bfloat16).to(device)


def f64(u16):
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def rel_err(y, ref):
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    rms = np.sqrt(np.mean(ref * ref))
    return float(np.max(np.abs(y - ref) / np.maximum(np.abs(ref), rms)))


D_SPECIAL = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x8123, 0x7BFF, 0x0400, 0x3C00], dtype=np.uint16)
DMIN_SPECIAL = np.array([0x0001, 0x0000, 0x7BFF, 0x8001, 0x0200, 0x3C00, 0xFBFF, 0x0010], dtype=np.uint16)


def kq_weights(qtype, n_rows, k, seed, specials=True):
    """Synthetic K-quant rows; with specials, random super-blocks get the
    edge cases listed in the module docstring."""
    raw = synth.make_weights(qtype, n_rows, k, seed)
    if not specials:
        return raw
    blocks = raw.reshape(-1, O.BLOCK_BYTES[qtype])
    rng = np.random.default_rng(seed + 1)
    nb = blocks.shape[0]
    pick = rng.choice(nb, min(nb, 24), replace=False)
    for i, b in enumerate(pick):
        d, dm = D_SPECIAL[i % 8], DMIN_SPECIAL[(i * 3) % 8]
        blocks[b, 0:2] = [d & 0xFF, d >> 8]
        blocks[b, 2:4] = [dm & 0xFF, dm >> 8]
        if i % 4 == 1:
            blocks[b, 4:16] = synth.pack_scale_min(np.full(8, 63), np.full(8, 63))
        elif i % 4 == 2:
            blocks[b, 4:16] = 0
        elif i % 4 == 3:
            blocks[b, 16:] = 0xFF  # every code at its top (and every Q5_K high bit set)
    return raw


def abs_sum(w_bits, x_bits):
    """sum_k |w[n][k] x[m][k]|, [m, n]."""
    return np.abs(f64(x_bits)) @ np.abs(f64(w_bits)).T


def check_bound(y, ref, w_bits, x_bits, tol):
    bound = tol * abs_sum(w_bits, x_bits) + 1e-30
    err = np.abs(np.asarray(y, np.float64) - ref)
    assert np.all(err <= bound), float(np.max(err / bound)) * tol


# ---- layout, dequant, GET_ROWS ----------------------------------------------------

@pytest.mark.parametrize("qtype", KQ)
def test_planar_round_trip(cuda, qtype):
    n, k = 37, 256 * 3
    raw = kq_weights(qtype, n, k, 1)
    rb = O.row_bytes(qtype, k)
    for pad in (0, 14):
        src = np.zeros((n, rb + pad), dtype=np.uint8)
        src[:, :rb] = raw.reshape(n, rb)
        planar = ops.to_planar(qtype, dev_u8(src, cuda), n, k, row_stride=rb + pad)
        back = ops.from_planar(qtype, planar, n, k, row_stride=rb + pad)
        torch.cuda.synchronize()
        assert planar.numel() == raw.size
        assert np.array_equal(back.cpu().numpy().reshape(n, rb + pad)[:, :rb], raw.reshape(n, rb))


@pytest.mark.parametrize("qtype", KQ)
def test_planar_planes(cuda, qtype):
    """The planes hold what the layout says: qs, (qh), then the 16-byte meta
    entries (d, dmin, packed scales) in block order."""
    n, k = 5, 512
    raw = kq_weights(qtype, n, k, 2)
    planar = ops.to_planar(qtype, dev_u8(raw, cuda), n, k).cpu().numpy()
    blocks = raw.reshape(-1, O.BLOCK_BYTES[qtype])
    tot = blocks.shape[0]
    q5 = qtype == O.Q5_K
    assert np.array_equal(planar[:tot * 128].reshape(tot, 128), blocks[:, 48 if q5 else 16:])
    if q5:
        assert np.array_equal(planar[tot * 128:tot * 160].reshape(tot, 32), blocks[:, 16:48])
    meta0 = tot * (160 if q5 else 128)
    assert np.array_equal(planar[meta0:].reshape(tot, 16), blocks[:, :16])


@pytest.mark.parametrize("qtype", KQ)
def test_dequant_bit_exact_with_edge_cases(cuda, qtype):
    n, k = 64, 256 * 8
    raw = kq_weights(qtype, n, k, 5)
    w = ops.to_planar(qtype, dev_u8(raw, cuda), n, k)
    assert np.array_equal(bits(ops.dequant(qtype, w, n, k)), O.dequant(qtype, raw, n, k))


@pytest.mark.parametrize("qtype", KQ)
def test_dequant_4096x4096_bit_exact(cuda, qtype):
    n = k = 4096
    raw = synth.make_weights(qtype, n, k, 3)
    w = ops.to_planar(qtype, dev_u8(raw, cuda), n, k)
    assert np.array_equal(bits(ops.dequant(qtype, w, n, k)), O.dequant(qtype, raw, n, k))


@pytest.mark.parametrize("qtype", KQ)
def test_get_rows(cuda, qtype):
    n, k = 50, 1024
    raw = kq_weights(qtype, n, k, 9)
    w = ops.to_planar(qtype, dev_u8(raw, cuda), n, k)
    ids = np.array([0, 49, 7, 7, 23, 1], dtype=np.int32)
    want = O.get_rows(qtype, raw, n, k, ids)
    ids_t = torch.from_numpy(ids).to(cuda)
    assert np.array_equal(bits(ops.get_rows(qtype, w, n, k, ids_t, out_dtype=torch.bfloat16)), want)
    got32 = ops.get_rows(qtype, w, n, k, ids_t, out_dtype=torch.float32).cpu().numpy()
    assert np.array_equal(got32.view(np.uint32), want.astype(np.uint32) << 16)


# ---- products -----------------------------------------------------------------------

def _mul_mat(cuda, qtype, raw, n, k, m, seed, out_dtype):
    x = synth.make_x(m, k, seed)
    w = ops.to_planar(qtype, dev_u8(raw, cuda), n, k)
    y = ops.mul_mat(qtype, w, n, k, dev_bf16(x, cuda), out_dtype=out_dtype)
    torch.cuda.synchronize()
    return y.float().cpu().numpy(), x


@pytest.mark.parametrize("qtype", KQ)
@pytest.mark.parametrize("n,k", [(1, 256), (7, 512), (129, 4096), (70, 14336), (33, 256 * 9), (45, 256 * 20)])
def test_gemv(cuda, qtype, n, k):
    """Rows in 16-lane groups, four a unit (256, 512, and 2304 with masked
    tasks), two tasks a lane with x in registers (4096), several passes with
    x from LDS (14336), 32-lane groups over five passes (5120)."""
    raw = kq_weights(qtype, n, k, 20 + n, specials=False)
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


@pytest.mark.parametrize("qtype", KQ)
@pytest.mark.parametrize("m", [2, 4, 16])
def test_small_batch(cuda, qtype, m):
    n, k = 300, 256 * 5
    raw = kq_weights(qtype, n, k, 40 + m, specials=False)
    y, x = _mul_mat(cuda, qtype, raw, n, k, m, 41 + m, torch.float32)
    ref = O.matmul_f64(O.dequant(qtype, raw, n, k), x)
    assert rel_err(y, ref) <= REL_TOL_EXACT_W, rel_err(y, ref)


@pytest.mark.parametrize("qtype", KQ)
def test_small_batch_k_windows(cuda, qtype):
    """16 rows of x over k = 14336 exceed the LDS window: k staged in windows."""
    n, k = 200, 14336
    raw = kq_weights(qtype, n, k, 60, specials=False)
    y, x = _mul_mat(cuda, qtype, raw, n, k, 16, 61, torch.float32)
    ref = O.matmul_f64(O.dequant(qtype, raw, n, k), x)
    assert rel_err(y, ref) <= REL_TOL_EXACT_W, rel_err(y, ref)


@pytest.mark.parametrize("qtype", KQ)
@pytest.mark.parametrize("m,n,k_sb", [(17, 64, 2), (130, 257, 3), (512, 512, 16)])
def test_gemm(cuda, qtype, m, n, k_sb):
    k = 256 * k_sb
    raw = kq_weights(qtype, n, k, 30 + m, specials=False)
    y, x = _mul_mat(cuda, qtype, raw, n, k, m, 31 + m, torch.float32)
    ref = O.matmul_f64(O.dequant(qtype, raw, n, k), x)
    assert rel_err(y, ref) <= REL_TOL_EXACT_W, rel_err(y, ref)


@pytest.mark.parametrize("qtype", KQ)
@pytest.mark.parametrize("m", [1, 4, 40])
def test_edge_case_weights_every_product(cuda, qtype, m):
    """GEMV (m = 1), small batch (4) and GEMM (40) over the edge-case blocks."""
    n, k = 96, 256 * 6
    raw = kq_weights(qtype, n, k, 70 + m)
    wb = O.dequant(qtype, raw, n, k)
    for out_dtype, tol in ((torch.float32, 1e-3), (torch.bfloat16, 1e-2)):
        y, x = _mul_mat(cuda, qtype, raw, n, k, m, 71 + m, out_dtype)
        check_bound(y, O.matmul_f64(wb, x), wb, x, tol)


# ---- MoE ----------------------------------------------------------------------------

def _moe(cuda, qtype, n_expert, n, k, n_tokens, top_k, x_slots, seed, specials=False, glu=False):
    rng = np.random.default_rng(seed)
    per = O.row_bytes(qtype, k) * n
    raws = [kq_weights(qtype, n, k, seed * 100 + e, specials) for e in range(n_expert)]
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
    return y, ref, bound, ids


@pytest.mark.parametrize("qtype", KQ)
@pytest.mark.parametrize("k,x_slots", [(1024, 1), (2048, 3), (4608, 1)])
def test_mul_mat_id(cuda, qtype, k, x_slots):
    """Streaming form (k <= 4096; 40 tokens x 3 slots over 8 experts, one
    expert past 16 pairs) and the LDS-staged form (k = 4608); an id routed
    nowhere gives a zero row."""
    y, ref, _, ids = _moe(cuda, qtype, 8, 96, k, 40, 3, x_slots, 11 + k)
    assert not y[1, 0].any()
    assert rel_err(y, ref) <= REL_TOL_EXACT_W, rel_err(y, ref)


@pytest.mark.parametrize("qtype", KQ)
def test_mul_mat_id_edge_case_weights(cuda, qtype):
    y, ref, bound, _ = _moe(cuda, qtype, 6, 64, 1536, 30, 2, 2, 12, specials=True)
    assert np.all(np.abs(y - ref) <= 1e-3 * bound + 1e-30)


@pytest.mark.parametrize("qtype", KQ)
def test_mul_mat_id_glu_fused(cuda, qtype):
    """MUL_MAT_ID fused with SwiGLU over the merged gate/up rows."""
    F = 80
    y, ref, _, _ = _moe(cuda, qtype, 8, 2 * F, 1024, 24, 2, 1, 13, glu=True)
    want = O.glu_f64(ref, O.GLU_SWIGLU)
    assert rel_err(y, want) <= REL_TOL_EXACT_W * 4, rel_err(y, want)
