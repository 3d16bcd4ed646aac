"""ggml's split GLU form: gate and up experts in two tensors (two MUL_MAT_ID
nodes and a GLU over both, as MoE FFNs stored with separate ffn_gate_exps
and ffn_up_exps tensors), standalone and fused into one streaming pass.

The GLU variants follow ggml's published definitions (restated in the
oracle's glu_f64); the product is the reference's
(src/quants/tests/mmul.py:104-126). The fused pass forms every (pair, row)
sum exactly as MUL_MAT_ID does, so it equals MUL_MAT_ID of each stack
followed by the standalone split GLU bit for bit.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from spiral_amd import ggml, ops, synth
from test_gpu_parity import GLU_OPS, REL_TOL, _moe_inputs, _moe_ref, dev_bf16, rel_err

pytestmark = pytest.mark.gpu

FORMATS = [O.Q4_0, O.Q8_0, O.Q6_K, O.Q4_K, O.Q5_K, O.IQ4_NL, O.IQ4_XS]


def _split_inputs(cuda, qtype, n_expert, F, k, n_tokens, top_k, seed, ids=None):
    """Gate and up expert stacks (separately seeded), ids and x."""
    wg, per, raws_g, ids, x = _moe_inputs(cuda, qtype, n_expert, F, k, n_tokens, top_k, 1, seed, ids)
    wu, _, raws_u, _, _ = _moe_inputs(cuda, qtype, n_expert, F, k, n_tokens, top_k, 1, seed + 500, ids)
    return wg, wu, per, raws_g, raws_u, ids, x


def test_glu_split_standalone(cuda):
    """act(gate) * up over separate float32 tensors (act(up) * gate when
    swapped), every variant, against the oracle's float64 GLU over the
    concatenated halves."""
    rng = np.random.default_rng(31)
    g = (3.0 * rng.standard_normal((5, 3, 40))).astype(np.float32)
    u = (3.0 * rng.standard_normal((5, 3, 40))).astype(np.float32)
    gt, ut = torch.from_numpy(g).to(cuda), torch.from_numpy(u).to(cuda)
    for op in GLU_OPS:
        for swapped in (False, True):
            y = ops.glu_split(gt, ut, op, swapped).cpu().numpy()
            want = O.glu_f64(np.concatenate([g, u], axis=-1), op, swapped)
            assert rel_err(y, want) <= 1e-5, (op, swapped)


def test_glu_swiglu_oai_standalone(cuda):
    """SWIGLU_OAI (gpt-oss's GLU) over merged [.., 2F] rows and over separate
    gate / up tensors, both half orders, inputs well past +-limit (the
    activated half capped from above, the other clamped both ways), at
    gpt-oss's alpha 1.702 / limit 7 and at alpha 1 / limit 3, against the
    oracle's float64 form; both forms give the same bits."""
    rng = np.random.default_rng(33)
    g = (6.0 * rng.standard_normal((4, 3, 56))).astype(np.float32)
    u = (6.0 * rng.standard_normal((4, 3, 56))).astype(np.float32)
    gt, ut = torch.from_numpy(g).to(cuda), torch.from_numpy(u).to(cuda)
    merged = torch.from_numpy(np.concatenate([g, u], axis=-1)).to(cuda)
    for alpha, limit in ((1.702, 7.0), (1.0, 3.0)):
        for swapped in (False, True):
            want = O.glu_f64(np.concatenate([g, u], axis=-1), O.GLU_SWIGLU_OAI, swapped, alpha=alpha, limit=limit)
            y1 = ops.glu_split(gt, ut, ops.GLU_SWIGLU_OAI, swapped, alpha=alpha, limit=limit).cpu().numpy()
            y2 = ops.glu(merged, ops.GLU_SWIGLU_OAI, swapped, alpha=alpha, limit=limit).cpu().numpy()
            assert rel_err(y1, want) <= 1e-5, (alpha, limit, swapped, rel_err(y1, want))
            assert np.array_equal(y1, y2)


@pytest.mark.parametrize("qtype", FORMATS)
def test_fused_split_matches_unfused_and_oracle(cuda, qtype):
    """Every format: the fused split pass equals MUL_MAT_ID of each stack and
    the standalone split GLU bit for bit (F32 out; BF16 out is that value
    rounded), every variant both ways round, and the oracle within the
    product bar. F = 72 is not a whole number of 16-row groups."""
    k = O.BLOCK_ELEMS[qtype] * (2 if O.BLOCK_ELEMS[qtype] == 256 else 8)
    n_expert, F, n_tokens, top_k = 8, 72, 40, 3
    wg, wu, per, raws_g, raws_u, ids, x = _split_inputs(cuda, qtype, n_expert, F, k, n_tokens, top_k, 41)
    xd, idd = dev_bf16(x, cuda), torch.from_numpy(ids).to(cuda)
    pg = ops.mul_mat_id(qtype, wg, per, n_expert, F, k, xd, idd, out_dtype=torch.float32)
    pu = ops.mul_mat_id(qtype, wu, per, n_expert, F, k, xd, idd, out_dtype=torch.float32)
    ref = np.concatenate([_moe_ref(qtype, raws_g, F, k, ids, x), _moe_ref(qtype, raws_u, F, k, ids, x)], axis=-1)
    for op in GLU_OPS:
        for swapped in (False, True):
            fused = ops.mul_mat_id_glu_split(qtype, wg, wu, per, n_expert, F, k, xd, idd, op, swapped,
                                             out_dtype=torch.float32)
            unfused = ops.glu_split(pg, pu, op, swapped)
            torch.cuda.synchronize()
            assert torch.equal(fused, unfused), (op, swapped)
            assert rel_err(fused.cpu().numpy(), O.glu_f64(ref, op, swapped)) <= REL_TOL, (op, swapped)
    fb = ops.mul_mat_id_glu_split(qtype, wg, wu, per, n_expert, F, k, xd, idd, ops.GLU_SWIGLU,
                                  out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(fb, ops.glu_split(pg, pu, ops.GLU_SWIGLU).to(torch.bfloat16))


@pytest.mark.parametrize("n_expert,n_tokens,top_k", [(6, 30, 2), (12, 160, 8), (8, 300, 2)])
def test_fused_split_routing_paths_and_bad_ids(cuda, n_expert, n_tokens, top_k):
    """Routing inside the kernel, the counting-sort route kernel (above 1024
    pairs) and passes of 32 tokens (37 pairs an expert); ids routed nowhere
    give zero rows; the rest equals the unfused chain."""
    qtype, F, k = O.Q4_0, 40, 256
    rng = np.random.default_rng(n_tokens)
    ids = np.stack([rng.choice(n_expert, top_k, replace=False) for _ in range(n_tokens)]).astype(np.int32)
    ids[::7, 0] = -1
    ids[3::11, -1] = 99
    wg, wu, per, _, _, ids, x = _split_inputs(cuda, qtype, n_expert, F, k, n_tokens, top_k, 42, ids)
    xd, idd = dev_bf16(x, cuda), torch.from_numpy(ids).to(cuda)
    out = torch.full((n_tokens, top_k, F), 7.0, device=cuda)
    ops.mul_mat_id_glu_split(qtype, wg, wu, per, n_expert, F, k, xd, idd, ops.GLU_GEGLU, out=out)
    pg = ops.mul_mat_id(qtype, wg, per, n_expert, F, k, xd, idd, out_dtype=torch.float32)
    pu = ops.mul_mat_id(qtype, wu, per, n_expert, F, k, xd, idd, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(out, ops.glu_split(pg, pu, ops.GLU_GEGLU))
    bad = (ids < 0) | (ids >= n_expert)
    assert not out.cpu().numpy()[bad].any()


def test_ggml_split_glu_fused_and_not(cuda):
    """Through the ggml surface, in llama.cpp's node order (up, gate, GLU):
    graph_compute fuses the three nodes (neither product is written); with a
    product flagged OUTPUT it runs them unfused, with the same result bits;
    a split GLU on its own is supported."""
    qtype, k, F, n_expert, top_k, n_tokens = O.Q4_0, 128, 48, 5, 2, 9
    raws_g = [synth.make_weights(qtype, F, k, 90 + e) for e in range(n_expert)]
    raws_u = [synth.make_weights(qtype, F, k, 190 + e) for e in range(n_expert)]
    rng = np.random.default_rng(10)
    ids = np.stack([rng.choice(n_expert, top_k, replace=False) for _ in range(n_tokens)]).astype(np.int32)
    xf = rng.standard_normal((n_tokens, 1, k), dtype=np.float32)
    buf = ggml.Buffer(4 << 20)
    ag = buf.alloc(ggml.new_tensor(qtype, [k, F, n_expert]))
    buf.set(ag, np.concatenate(raws_g).tobytes())
    au = buf.alloc(ggml.new_tensor(qtype, [k, F, n_expert]))
    buf.set(au, np.concatenate(raws_u).tobytes())
    b = buf.alloc(ggml.new_tensor(ggml.TYPE_F32, [k, 1, n_tokens]))
    buf.set(b, xf.tobytes())
    it = buf.alloc(ggml.new_tensor(ggml.TYPE_I32, [top_k, n_tokens]))
    buf.set(it, ids.tobytes())
    up = buf.alloc(ggml.mul_mat_id(au, b, it, name="ffn_up"))
    gate = buf.alloc(ggml.mul_mat_id(ag, b, it, name="ffn_gate"))
    g = buf.alloc(ggml.glu_split(gate, up, ggml.GLU_SWIGLU))
    assert ggml.supports_op(g)
    sentinel = np.full(F * top_k * n_tokens, 7.0, dtype=np.float32).tobytes()
    buf.set(up, sentinel)
    buf.set(gate, sentinel)
    be = ggml.Backend(0)
    assert be.graph_compute([up, gate, g]) == 0
    be.synchronize()
    assert buf.get(up) == sentinel and buf.get(gate) == sentinel  # fused: neither product written
    y = np.frombuffer(buf.get(g), dtype=np.float32).reshape(n_tokens, top_k, F)
    xb = synth.bf16_bits(xf[:, 0])
    for t in range(n_tokens):
        for s in range(top_k):
            e = ids[t, s]
            pg = O.matmul_f64(O.dequant(qtype, raws_g[e], F, k), xb[t][None])[0]
            pu = O.matmul_f64(O.dequant(qtype, raws_u[e], F, k), xb[t][None])[0]
            assert rel_err(y[t, s], O.glu_f64(np.concatenate([pg, pu]), O.GLU_SWIGLU)) <= REL_TOL
    gate.flags = ggml.FLAG_OUTPUT
    assert be.graph_compute([up, gate, g]) == 0
    be.synchronize()
    assert buf.get(gate) != sentinel
    assert np.frombuffer(buf.get(g), dtype=np.float32).tobytes() == y.tobytes()
    be.free()
    buf.free()
