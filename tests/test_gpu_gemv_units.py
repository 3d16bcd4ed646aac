"""The exact GEMV's unit shapes over every format (spiral_amd/csrc/gemv.hip:
launch_exact picks the unit of least estimated work for a row of T tasks).

Row lengths are chosen so that the launches cover:
  - rows in 16- or 32-lane groups, four or two rows a unit (T up to 256 and
    no multiple of 64), with and without masked tasks;
  - whole-wave units of one, two or four tasks a lane with x in registers
    (one pass) or read from LDS (several passes), with and without a masked
    last pass.

37 rows leave a partial row group at the matrix end. Every product is
checked against the float64 oracle over the exact bf16 weights: float32
output to 1e-3 and bf16 output to 1e-2 of max(|ref|, rms(ref)).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from spiral_amd import ops, synth

pytestmark = pytest.mark.gpu

FORMATS = [O.Q4_0, O.Q8_0, O.Q6_K, O.Q4_K, O.Q5_K, O.IQ4_NL, O.IQ4_XS]
TASK_ELEMS = {O.Q4_0: 32, O.Q8_0: 16, O.Q6_K: 32, O.Q4_K: 32, O.Q5_K: 32, O.IQ4_NL: 32, O.IQ4_XS: 32}
# Row lengths in tasks; formats keep those that are whole blocks.
TASKS = (8, 12, 24, 40, 48, 72, 96, 100, 112, 128, 160, 176, 200, 224, 264, 300, 448)
N_ROWS = 37


def rel_err(y, ref):
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    rms = np.sqrt(np.mean(ref * ref))
    return float(np.max(np.abs(y - ref) / np.maximum(np.abs(ref), rms)))


def cases():
    for qtype in FORMATS:
        for t in TASKS:
            k = t * TASK_ELEMS[qtype]
            if k % O.BLOCK_ELEMS[qtype] == 0:
                yield pytest.param(qtype, k, id=f"{O.FORMAT_NAMES[qtype]}-k{k}")


@pytest.mark.parametrize("qtype,k", list(cases()))
def test_gemv_unit_shapes(cuda, qtype, k):
    raw = synth.make_weights(qtype, N_ROWS, k, 500 + k)
    x = synth.make_x(1, k, 600 + k)
    w = ops.to_planar(qtype, torch.from_numpy(raw).to(cuda), N_ROWS, k)
    xd = torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).view(torch.bfloat16).to(cuda)
    ref = O.matmul_f64(O.dequant(qtype, raw, N_ROWS, k), x)
    y32 = ops.mul_mat(qtype, w, N_ROWS, k, xd, out_dtype=torch.float32).cpu().numpy()
    y16 = ops.mul_mat(qtype, w, N_ROWS, k, xd, out_dtype=torch.bfloat16).float().cpu().numpy()
    assert rel_err(y32, ref) <= 1e-3, rel_err(y32, ref)
    assert rel_err(y16, ref) <= 1e-2, rel_err(y16, ref)


# The reference's first model target instantiates single-row products at
# K = 1536 / 2048 / 4096 (src/quants/TODO.md:48-51); Q4_0 and Q8_0 are held
# at those shapes by test_gpu_parity.py, the other formats here (K = 1536:
# 48 tasks, rows in 16-lane groups).
@pytest.mark.parametrize("qtype", [O.Q6_K, O.Q4_K, O.Q5_K, O.IQ4_NL, O.IQ4_XS])
@pytest.mark.parametrize("k", (1536, 2048, 4096))
@pytest.mark.parametrize("n", (2048, 12288))
def test_gemv_model_shapes(cuda, qtype, k, n):
    raw = synth.make_weights(qtype, n, k, 700 + n + k)
    x = synth.make_x(1, k, 800 + k)
    w = ops.to_planar(qtype, torch.from_numpy(raw).to(cuda), n, k)
    xd = torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).view(torch.bfloat16).to(cuda)
    y32 = ops.mul_mat(qtype, w, n, k, xd, out_dtype=torch.float32).cpu().numpy()
    ref = O.matmul_f64(O.dequant(qtype, raw, n, k), x)
    assert rel_err(y32, ref) <= 1e-3, rel_err(y32, ref)
