"""GPU parity of MUL_MAT for 17 to 64 rows of x (batched decode, short
prefill chunks), the range between the small-batch streaming form (up to 16
rows) and full GEMM tiles: the GEMM runs it with partly filled 128-row
tiles. Held to the product bars of tests/test_gpu_parity.py against the
float64 oracle (the reference's product, src/quants/tests/mmul.py:104-112),
with ragged row counts, k tails, wide k, bf16 and float32 output, strided x
and y, and edge-case weights.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from spiral_amd import ops, synth
from test_gpu_kquants import abs_sum
from test_gpu_parity import REL_TOL, REL_TOL_EXACT_W, _mul_mat_case, dev_bf16, dev_u8, rel_err, weights_with_specials

pytestmark = pytest.mark.gpu

FORMATS = [O.Q4_0, O.Q8_0, O.Q6_K, O.Q4_K, O.Q5_K, O.IQ4_NL, O.IQ4_XS]


MS = (17, 24, 32, 40, 64)


@pytest.mark.parametrize("qtype", FORMATS)
def test_mid_batch_every_format(cuda, qtype):
    """300 weight rows (a ragged last group); k not a multiple of 128 where
    the format allows; every row count from one block and a bit to four."""
    k = O.BLOCK_ELEMS[qtype] * (13 if O.BLOCK_ELEMS[qtype] == 32 else 3)
    for m in MS:
        y, ref = _mul_mat_case(cuda, qtype, 300, k, m, 80 + m, torch.float32)
        assert rel_err(y, ref) <= REL_TOL_EXACT_W, (m, rel_err(y, ref))


@pytest.mark.parametrize("qtype,k", [(O.Q4_0, 4096), (O.Q8_0, 8192), (O.Q6_K, 14336), (O.Q4_K, 4096)])
def test_mid_batch_wide_k(cuda, qtype, k):
    """32 and 64 rows of x over a wide k."""
    for m in (32, 64):
        y, ref = _mul_mat_case(cuda, qtype, 200, k, m, 90 + m, torch.float32)
        assert rel_err(y, ref) <= REL_TOL_EXACT_W, (m, rel_err(y, ref))


@pytest.mark.parametrize("qtype,n,k", [(O.Q4_0, 4096, 4096), (O.Q8_0, 14336, 4096), (O.Q6_K, 4096, 14336)])
def test_mid_batch_workload_shapes_bf16(cuda, qtype, n, k):
    """Model shapes with bf16 output: 32 and 64 rows."""
    for m in (32, 64):
        y, ref = _mul_mat_case(cuda, qtype, n, k, m, 100 + m, torch.bfloat16)
        assert rel_err(y, ref) <= REL_TOL, (m, rel_err(y, ref))


def test_mid_batch_strides(cuda):
    """x rows and y rows with strides wider than k and n, 40 rows."""
    qtype, n, k, m = O.Q4_0, 100, 512, 40
    raw = synth.make_weights(qtype, n, k, 110)
    x = synth.make_x(m, k, 111)
    w = ops.to_planar(qtype, dev_u8(raw, cuda), n, k)
    xw = torch.zeros((m, k + 24), dtype=torch.bfloat16, device=cuda)
    xw[:, :k] = dev_bf16(x, cuda)
    yw = torch.full((m, n + 12), 7.0, dtype=torch.float32, device=cuda)
    ops.mul_mat(qtype, w, n, k, xw[:, :k], out=yw[:, :n])
    torch.cuda.synchronize()
    got = yw.cpu().numpy()
    assert rel_err(got[:, :n], O.matmul_f64(O.dequant(qtype, raw, n, k), x)) <= REL_TOL_EXACT_W
    assert (got[:, n:] == 7.0).all()  # nothing written past n


@pytest.mark.parametrize("qtype", [O.Q4_0, O.Q8_0, O.Q6_K])
def test_mid_batch_edge_case_weights(cuda, qtype):
    """Special scales (exponent 0 and 31, subnormal), negative and -128 Q6_K
    sub-scales, Q8_0 -128 codes: every product within 1e-3 of the sum of its
    terms' magnitudes."""
    n, k, m = 96, O.BLOCK_ELEMS[qtype] * (24 if qtype != O.Q6_K else 3), 32
    raw = weights_with_specials(qtype, n, k, 120)
    x = synth.make_x(m, k, 121)
    w = ops.to_planar(qtype, dev_u8(raw, cuda), n, k)
    y = ops.mul_mat(qtype, w, n, k, dev_bf16(x, cuda), out_dtype=torch.float32)
    torch.cuda.synchronize()
    wb = O.dequant(qtype, raw, n, k)
    ref = O.matmul_f64(wb, x)
    bound = abs_sum(wb, x)
    assert np.all(np.abs(y.cpu().numpy() - ref) <= 1e-3 * bound + 1e-30)
