"""GPU parity of MUL_MAT_ID at prefill sizes: many routed tokens per expert.

Passes then take 32 or 64 of an expert's tokens (two or four MFMA row blocks
per dequantized weight, as far as the activations of k fit in LDS), and the
passes of one expert run on several workgroups side by side (pass lanes).
Covered: every format, each pass size at the k that limits it, a skewed
routing (one expert with hundreds of pairs, several passes per lane), ids
routed nowhere, bf16 and float32 output, the fused GLU form. The product is
the reference's (src/quants/tests/mmul.py:104-126), held to the bars of
tests/test_gpu_parity.py; each (pair, row) sum is formed exactly as in a
decode-sized call, so a prefill call also equals per-chunk decode calls bit
for bit.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from spiral_amd import ops
from test_gpu_parity import (REL_TOL, REL_TOL_EXACT_W, _moe_case, _moe_inputs, _moe_ref, check_moe, dev_bf16,
                             rel_err)

pytestmark = pytest.mark.gpu

FORMATS = [O.Q4_0, O.Q8_0, O.Q6_K, O.Q4_K, O.Q5_K, O.IQ4_NL, O.IQ4_XS]


@pytest.mark.parametrize("qtype", FORMATS)
def test_prefill_four_row_blocks_every_format(cuda, qtype):
    """320 pairs over 8 experts (40 a expert): passes of 64 tokens; 104 rows
    (not whole 16-row groups; expert matrices stay 16-byte multiples), k = 768."""
    y, ref, _ = _moe_case(cuda, qtype, 8, 104, 768, 160, 2, 1, 61, torch.float32)
    check_moe(y, ref, True)


def test_prefill_two_row_blocks_at_k2048(cuda):
    """k = 2048 leaves LDS for 32 staged tokens: passes of 32 (25 pairs an
    expert on average, some experts with two passes)."""
    y, ref, _ = _moe_case(cuda, O.Q4_0, 8, 64, 2048, 100, 2, 1, 62, torch.float32)
    check_moe(y, ref, True)


def test_prefill_k4096_pass_lanes(cuda):
    """k = 4096 keeps passes of 16 tokens; 50 pairs an expert spread over four
    pass lanes (routing inside the kernel: every workgroup builds the same
    ordered list)."""
    y, ref, _ = _moe_case(cuda, O.Q4_0, 4, 32, 4096, 200, 1, 1, 63, torch.float32)
    check_moe(y, ref, True)


def test_prefill_skewed_routing_and_bad_ids(cuda):
    """1400 pairs (routed by the counting-sort kernel): expert 3 takes 500 of
    them (eight passes of 64 over two pass lanes), the rest spread; ids routed
    nowhere give zero rows; per-slot inputs; bf16 and float32 output."""
    n_expert, n, k, n_tokens, top_k = 16, 48, 512, 700, 2
    rng = np.random.default_rng(64)
    ids = np.stack([rng.choice(n_expert, top_k, replace=False) for _ in range(n_tokens)]).astype(np.int32)
    ids[:500, 0] = 3
    ids[:500, 1] = np.where(ids[:500, 1] == 3, 4, ids[:500, 1])
    ids[::13, 1] = -1
    ids[5::17, 0] = 40
    for out_dtype in (torch.float32, torch.bfloat16):
        y, ref, ids_used = _moe_case(cuda, O.Q4_0, n_expert, n, k, n_tokens, top_k, 2, 65, out_dtype, ids=ids)
        bad = (ids_used < 0) | (ids_used >= n_expert)
        assert not y[bad].any()
        check_moe(y, ref, out_dtype == torch.float32)


@pytest.mark.parametrize("qtype", [O.Q4_0, O.Q6_K])
def test_prefill_equals_decode_calls(cuda, qtype):
    """A prefill call (30 pairs an expert: passes of 32) equals the same tokens
    sent four at a time (decode-sized calls, passes of 16), bit for bit."""
    n_expert, n, k, n_tokens, top_k = 8, 80, 512, 120, 2
    w, per, raws, ids, x = _moe_inputs(cuda, qtype, n_expert, n, k, n_tokens, top_k, 1, 66)
    xd, idd = dev_bf16(x, cuda), torch.from_numpy(ids).to(cuda)
    big = ops.mul_mat_id(qtype, w, per, n_expert, n, k, xd, idd, out_dtype=torch.float32)
    parts = [ops.mul_mat_id(qtype, w, per, n_expert, n, k, xd[t:t + 4].contiguous(), idd[t:t + 4].contiguous(),
                            out_dtype=torch.float32) for t in range(0, n_tokens, 4)]
    torch.cuda.synchronize()
    assert torch.equal(big, torch.cat(parts))
    assert rel_err(big.cpu().numpy(), _moe_ref(qtype, raws, n, k, ids, x)) <= REL_TOL_EXACT_W


def test_prefill_route_past_lds_list(cuda):
    """8800 pairs (1100 tokens, top-8 over 32 experts): past the 8192 whose
    lists the routing kernel builds in LDS, so the lists are scattered
    straight to memory. Equal bit for bit to the same tokens in decode-sized
    calls of 100 (routed inside the kernel), and to the oracle within the
    bars; ids routed nowhere give zero rows."""
    n_expert, n, k, n_tokens, top_k = 32, 64, 256, 1100, 8
    rng = np.random.default_rng(69)
    ids = np.stack([rng.choice(n_expert, top_k, replace=False) for _ in range(n_tokens)]).astype(np.int32)
    ids[::37, 3] = -2
    w, per, raws, ids, x = _moe_inputs(cuda, O.Q4_0, n_expert, n, k, n_tokens, top_k, 1, 70, ids)
    xd, idd = dev_bf16(x, cuda), torch.from_numpy(ids).to(cuda)
    big = ops.mul_mat_id(O.Q4_0, w, per, n_expert, n, k, xd, idd, out_dtype=torch.float32)
    parts = [ops.mul_mat_id(O.Q4_0, w, per, n_expert, n, k, xd[t:t + 100].contiguous(), idd[t:t + 100].contiguous(),
                            out_dtype=torch.float32) for t in range(0, n_tokens, 100)]
    torch.cuda.synchronize()
    assert torch.equal(big, torch.cat(parts))
    y = big.cpu().numpy()
    assert not y[ids < 0].any()
    check_moe(y, _moe_ref(O.Q4_0, raws, n, k, ids, x), True)


@pytest.mark.parametrize("qtype,n_tokens", [(O.Q4_0, 150), (O.Q4_K, 150), (O.Q4_0, 600)])
def test_prefill_glu(cuda, qtype, n_tokens):
    """The fused GLU form at 37 pairs an expert (passes of 32 over two pass
    lanes, routed in the kernel) and at 150 (1200 pairs: the counting-sort
    route kernel, five pass lanes) equals MUL_MAT_ID followed by the
    standalone GLU bit for bit, and the oracle within the product bar."""
    n_expert, F, k, top_k = 8, 48, 512, 2
    w, per, raws, ids, x = _moe_inputs(cuda, qtype, n_expert, 2 * F, k, n_tokens, top_k, 1, 67)
    xd, idd = dev_bf16(x, cuda), torch.from_numpy(ids).to(cuda)
    prod = ops.mul_mat_id(qtype, w, per, n_expert, 2 * F, k, xd, idd, out_dtype=torch.float32)
    fused = ops.mul_mat_id_glu(qtype, w, per, n_expert, 2 * F, k, xd, idd, ops.GLU_SWIGLU, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(fused, ops.glu(prod, ops.GLU_SWIGLU))
    ref = O.glu_f64(_moe_ref(qtype, raws, 2 * F, k, ids, x), ops.GLU_SWIGLU)
    assert rel_err(fused.cpu().numpy(), ref) <= REL_TOL


@pytest.mark.parametrize("stage", ["gate_up", "down"])
def test_prefill_bench_shape_equals_decode_calls(cuda, stage):
    """The prefill workload at its own size (128 experts of 1536 x 2048 /
    2048 x 768 Q4_0, 1024 tokens, top-8, per-slot inputs for down; passes
    of 32 / 64 tokens): bit for bit the same as sixteen decode-sized calls
    of 64 tokens, and sampled rows against the float64 oracle."""
    n_expert, top_k, n_tokens = 128, 8, 1024
    n, k, xs = (1536, 2048, 1) if stage == "gate_up" else (2048, 768, 8)
    w, per, raws, ids, x = _moe_inputs(cuda, O.Q4_0, n_expert, n, k, n_tokens, top_k, xs, 68)
    xd, idd = dev_bf16(x, cuda), torch.from_numpy(ids).to(cuda)
    big = ops.mul_mat_id(O.Q4_0, w, per, n_expert, n, k, xd, idd, out_dtype=torch.float32)
    parts = [ops.mul_mat_id(O.Q4_0, w, per, n_expert, n, k, xd[t:t + 64].contiguous(), idd[t:t + 64].contiguous(),
                            out_dtype=torch.float32) for t in range(0, n_tokens, 64)]
    torch.cuda.synchronize()
    assert torch.equal(big, torch.cat(parts))
    sel = [(t, s) for t in range(0, n_tokens, 97) for s in (0, top_k - 1)]
    ref = np.stack([O.matmul_f64(O.dequant(O.Q4_0, raws[ids[t, s]], n, k), x[t, s % xs][None, :])[0]
                    for t, s in sel])
    got = np.stack([big[t, s].cpu().numpy() for t, s in sel])
    assert rel_err(got, ref) <= REL_TOL_EXACT_W
