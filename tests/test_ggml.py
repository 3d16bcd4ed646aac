"""The ggml-backend-shaped surface (include/spiral_ggml.h), tested the way
ggml's test-backend-ops tests a backend: build a node, run it through
graph_compute, compare with a CPU reference (here the oracle).

CPU tests: tensor sizes, supports_op's refusals, and that nothing pretends to
work without a device. GPU tests: canonical-bytes set/get round trips through
the planar device layout (whole matrices and arbitrary byte ranges), and
MUL_MAT / GET_ROWS / MUL_MAT_ID / GLU nodes (and MUL_MAT_ID fused with the
GLU over it) against the oracle.
"""

import ctypes
import struct

import numpy as np
import pytest

from oracle import oracle as O
from spiral_amd import ggml, synth
from spiral_amd._lib import STATUS

REL_TOL = 1e-2         # GEMV path (block-scaled sums)
REL_TOL_EXACT_W = 1e-3  # MFMA paths (exact bf16 weights), F32 output


def rel_err(y, ref):
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    rms = np.sqrt(np.mean(ref * ref))
    return float(np.max(np.abs(y - ref) / np.maximum(np.abs(ref), rms)))


def f32_of_bf16(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---- CPU ----------------------------------------------------------------------

def test_alloc_size_matches_ggml_nbytes(spiral_lib):
    assert ggml.nbytes(ggml.new_tensor(ggml.TYPE_Q4_0, [4096, 4096])) == 9_437_184
    assert ggml.nbytes(ggml.new_tensor(ggml.TYPE_Q8_0, [4096, 14336])) == 62_390_272
    assert ggml.nbytes(ggml.new_tensor(ggml.TYPE_Q6_K, [14336, 4096])) == 48_168_960
    assert ggml.nbytes(ggml.new_tensor(ggml.TYPE_Q4_0, [2048, 1536, 128])) == 128 * 1_769_472
    assert ggml.nbytes(ggml.new_tensor(ggml.TYPE_F32, [4, 3, 2])) == 96
    assert ggml.nbytes(ggml.new_tensor(ggml.TYPE_BF16, [8, 5])) == 80
    # a transposed F32 view: ggml_nbytes counts the span it reaches
    t = ggml.new_tensor(ggml.TYPE_F32, [3, 4])
    t.ne[0], t.ne[1] = 4, 3
    t.nb[0], t.nb[1] = 12, 4
    assert ggml.nbytes(t) == 4 + 3 * 12 + 2 * 4
    with pytest.raises(ValueError):
        ggml.new_tensor(ggml.TYPE_Q6_K, [100, 2])


def test_buffer_type_properties(spiral_lib):
    L = ggml._lib()
    assert L.spiral_buft_name() == b"SPIRAL_MI355X"
    assert L.spiral_buft_alignment() == 256
    assert L.spiral_buft_max_size() > 1 << 40


def test_supports_op_refusals(spiral_lib):
    a = ggml.new_tensor(ggml.TYPE_Q4_0, [256, 64])
    b = ggml.new_tensor(ggml.TYPE_F32, [256, 4])
    # src0 has no buffer: not this backend's weights
    assert not ggml.supports_op(ggml.mul_mat(a, b))
    # dense src0, integer activations, shape mismatch, unknown op
    assert not ggml.supports_op(ggml.mul_mat(ggml.new_tensor(ggml.TYPE_F32, [256, 64]), b))
    assert not ggml.supports_op(ggml.mul_mat(a, ggml.new_tensor(ggml.TYPE_I32, [256, 4])))
    assert not ggml.supports_op(ggml.mul_mat(a, ggml.new_tensor(ggml.TYPE_F32, [128, 4])))
    odd = ggml.new_tensor(ggml.TYPE_F32, [1, 1])
    odd.op = 99
    assert not ggml.supports_op(odd)
    for op in (ggml.OP_NONE, ggml.OP_VIEW, ggml.OP_RESHAPE, ggml.OP_PERMUTE, ggml.OP_TRANSPOSE):
        v = ggml.new_tensor(ggml.TYPE_F32, [4])
        v.op = op
        assert ggml.supports_op(v)


def test_supports_op_glu(spiral_lib):
    """GLU nodes: the single-tensor form over F32 rows with a known variant."""
    h = ggml.new_tensor(ggml.TYPE_F32, [192, 3, 5])
    for op in (ggml.GLU_REGLU, ggml.GLU_GEGLU, ggml.GLU_SWIGLU, ggml.GLU_GEGLU_ERF, ggml.GLU_GEGLU_QUICK):
        for swapped in (False, True):
            g = ggml.glu(h, op, swapped)
            assert list(g.ne) == [96, 3, 5, 1]
            assert ggml.supports_op(g)
    # SWIGLU_OAI: alpha and limit ride in op_params[2] and [3] as float bits
    oai = ggml.glu(h, ggml.GLU_SWIGLU_OAI, alpha=1.702, limit=7.0)
    assert ggml.supports_op(oai)
    assert struct.unpack("<ff", struct.pack("<ii", oai.op_params[2], oai.op_params[3])) == (
        struct.unpack("<f", struct.pack("<f", 1.702))[0], 7.0)
    hs = ggml.new_tensor(ggml.TYPE_F32, [96, 3, 5])
    assert ggml.supports_op(ggml.glu_split(hs, hs, ggml.GLU_SWIGLU_OAI, True))
    g = ggml.glu(h)
    g.op_params[1] = 2
    assert not ggml.supports_op(g)
    g = ggml.glu(h)
    g.src[1] = ctypes.pointer(h)  # the split form (separate gate and up tensors)
    assert not ggml.supports_op(g)
    assert not ggml.supports_op(ggml.glu(ggml.new_tensor(ggml.TYPE_BF16, [192, 3])))
    g = ggml.glu(h)
    g.ne[0] = 95
    assert not ggml.supports_op(g)


def test_no_device_means_no_backend(spiral_lib):
    if spiral_lib.spiral_device_count() > 0:
        pytest.skip("a HIP device is visible")
    L = ggml._lib()
    assert not L.spiral_buft_alloc_buffer(1 << 20)
    with pytest.raises(RuntimeError):
        ggml.Backend(0)
    assert L.spiral_backend_graph_compute(None, None) == 3  # SPIRAL_ERR_NULL
    assert L.spiral_buffer_set_tensor(None, None, None, 0, 0) == 3


# ---- GPU ----------------------------------------------------------------------

def weights(qtype, k, n, n_mat, seed):
    """Canonical bytes of n_mat stacked [n][k] matrices."""
    return np.concatenate([synth.make_weights(qtype, n, k, seed + i) for i in range(n_mat)])


@pytest.mark.gpu
@pytest.mark.parametrize("qtype", [O.Q4_0, O.Q8_0, O.Q6_K, O.Q4_K, O.Q5_K, O.IQ4_NL, O.IQ4_XS])
def test_set_get_round_trip_any_range(cuda, qtype):
    k, n, n_mat = O.BLOCK_ELEMS[qtype] * 3, 8, 3   # 24 blocks: each matrix a multiple of 16 bytes
    raw = weights(qtype, k, n, n_mat, 5)
    buf = ggml.Buffer(1 << 20)
    t = buf.alloc(ggml.new_tensor(qtype, [k, n, n_mat]))
    assert ggml.nbytes(t) == raw.size
    buf.set(t, raw.tobytes())                     # whole matrices
    assert buf.get(t) == raw.tobytes()
    buf.memset(t, 0)
    assert buf.get(t) == bytes(raw.size)
    rng = np.random.default_rng(qtype)
    cuts = np.sort(rng.choice(np.arange(1, raw.size), 5, replace=False))
    for lo, hi in zip([0, *cuts], [*cuts, raw.size]):  # arbitrary byte ranges
        buf.set(t, raw[lo:hi].tobytes(), offset=int(lo))
    assert buf.get(t) == raw.tobytes()
    lo, hi = int(cuts[1]), int(cuts[3])
    assert buf.get(t, size=hi - lo, offset=lo) == raw[lo:hi].tobytes()
    buf.memset(t, 0x5A, offset=3, size=11)
    want = raw.copy()
    want[3:14] = 0x5A
    assert buf.get(t) == want.tobytes()
    # the device copy is planar: GET_ROWS reads it as the oracle reads canonical bytes
    buf.set(t, raw.tobytes())
    ids = buf.alloc(ggml.new_tensor(ggml.TYPE_I32, [4, n_mat]))
    idv = np.array([[0, 7, 3, 3], [1, 2, 5, 0], [6, 6, 0, 4]], dtype=np.int32)
    buf.set(ids, idv.tobytes())
    out = buf.alloc(ggml.get_rows(t, ids, ggml.TYPE_BF16))
    be = ggml.Backend(0)
    assert be.graph_compute([out]) == 0
    be.synchronize()
    got = np.frombuffer(buf.get(out), dtype=np.uint16).reshape(n_mat, 4, k)
    mat = raw.size // n_mat
    for i in range(n_mat):
        assert np.array_equal(got[i], O.get_rows(qtype, raw[i * mat:(i + 1) * mat], n, k, idv[i]))
    be.free()
    buf.free()


@pytest.mark.gpu
def test_stacks_must_be_16_byte_matrices(cuda):
    """A stack whose matrices are not whole 16-byte multiples cannot hold the
    per-matrix planar layout and is refused; a single such matrix is fine."""
    buf = ggml.Buffer(1 << 20)
    one = buf.alloc(ggml.new_tensor(O.Q4_0, [96, 7]))  # 378 bytes
    raw = synth.make_weights(O.Q4_0, 7, 96, 9)
    buf.set(one, raw.tobytes())
    assert buf.get(one) == raw.tobytes()
    stack = ggml.new_tensor(O.Q4_0, [96, 7, 2])
    stack.data = buf.base + 4096
    assert STATUS[ggml._lib().spiral_buffer_init_tensor(buf.ptr, ctypes.byref(stack))] == "SPIRAL_ERR_SHAPE"
    buf.free()


@pytest.mark.gpu
def test_quantized_views(cuda):
    """Views into quantized weights (ggml_view_*: view_src / view_offs). The
    planar layout is relative to each matrix's start, so a view inside a
    matrix (a row range, or a matrix-sized window at a partial offset) is
    refused by supports_op, set_tensor, get_tensor and memset_tensor, even
    though its own strides and alignment look like a whole tensor's. A view
    of one whole matrix of a stack is accepted: MUL_MAT over it is that
    matrix's product and get_tensor returns its canonical bytes."""
    qtype, k, n, n_mat, m = O.Q4_0, 256, 64, 3, 2
    raws = [synth.make_weights(qtype, n, k, 80 + i) for i in range(n_mat)]
    buf = ggml.Buffer(4 << 20)
    a = buf.alloc(ggml.new_tensor(qtype, [k, n, n_mat]))
    buf.set(a, np.concatenate(raws).tobytes())
    rb, mat = a.nb[1], a.nb[2]
    xf = np.random.default_rng(5).standard_normal((m, k), dtype=np.float32)
    b = buf.alloc(ggml.new_tensor(ggml.TYPE_F32, [k, m]))
    buf.set(b, xf.tobytes())
    L = ggml._lib()
    bad_views = [ggml.view(a, [k, 32], [rb], 16 * rb),     # rows 16..47 of matrix 0
                 ggml.view(a, [k, n], [rb], 16 * rb),      # a matrix-sized window at a partial offset
                 ggml.view(a, [k, 32], [rb], mat)]         # the first half of matrix 1
    for v in bad_views:
        assert v.data % 16 == 0 and v.buffer
        assert not ggml.supports_op(ggml.mul_mat(v, b))
        assert not ggml.supports_op(ggml.get_rows(v, ggml.new_tensor(ggml.TYPE_I32, [2])))
        host = (ctypes.c_uint8 * rb)()
        for fn in (L.spiral_buffer_set_tensor, L.spiral_buffer_get_tensor):
            assert STATUS[fn(buf.ptr, ctypes.byref(v), host, 0, rb)] == "SPIRAL_ERR_SHAPE"
        assert STATUS[L.spiral_buffer_memset_tensor(buf.ptr, ctypes.byref(v), 0, 0, rb)] == "SPIRAL_ERR_SHAPE"
    one = ggml.view(a, [k, n], [rb], mat)  # matrix 1, whole
    nested = ggml.view(ggml.view(a, [k, n, 2], [rb, mat], mat), [k, n], [rb], mat)  # matrix 2 via a view of a view
    assert nested.view_offs == 2 * mat and ctypes.addressof(nested.view_src.contents) == ctypes.addressof(a)
    be = ggml.Backend(0)
    for v, i in ((one, 1), (nested, 2)):
        node = buf.alloc(ggml.mul_mat(v, b))
        assert ggml.supports_op(node)
        assert be.graph_compute([node]) == 0
        be.synchronize()
        y = np.frombuffer(buf.get(node), dtype=np.float32).reshape(m, n)
        ref = O.matmul_f64(O.dequant(qtype, raws[i], n, k), synth.bf16_bits(xf))
        assert rel_err(y, ref) <= REL_TOL_EXACT_W
        assert buf.get(v) == raws[i].tobytes()
    be.free()
    buf.free()


@pytest.mark.gpu
@pytest.mark.parametrize("qtype", [O.Q4_0, O.Q8_0, O.Q6_K, O.Q4_K, O.Q5_K, O.IQ4_NL, O.IQ4_XS])
@pytest.mark.parametrize("act", [ggml.TYPE_F32, ggml.TYPE_BF16])
@pytest.mark.parametrize("m", [1, 6, 40])
def test_mul_mat_node(cuda, qtype, act, m):
    k, n = O.BLOCK_ELEMS[qtype] * 4, 80
    raw = synth.make_weights(qtype, n, k, 11 + m)
    rng = np.random.default_rng(m)
    xf = rng.standard_normal((m, k), dtype=np.float32)
    xb = synth.bf16_bits(xf)
    buf = ggml.Buffer(4 << 20)
    a = buf.alloc(ggml.new_tensor(qtype, [k, n]))
    buf.set(a, raw.tobytes())
    b = buf.alloc(ggml.new_tensor(act, [k, m]))
    buf.set(b, (xf if act == ggml.TYPE_F32 else xb).tobytes())
    node = buf.alloc(ggml.mul_mat(a, b))
    assert ggml.supports_op(node)
    be = ggml.Backend(0)
    assert be.graph_compute([node]) == 0
    be.synchronize()
    y = np.frombuffer(buf.get(node), dtype=np.float32).reshape(m, n)
    ref = O.matmul_f64(O.dequant(qtype, raw, n, k), xb)   # F32 activations are rounded to bf16
    assert rel_err(y, ref) <= (REL_TOL if m == 1 else REL_TOL_EXACT_W)
    be.free()
    buf.free()


@pytest.mark.gpu
def test_mul_mat_broadcast_batches(cuda):
    """src0 [k, n, 2, 1] against src1 [k, m, 4, 3]: batch (i2, i3) uses
    src0 matrix i2 / 2 (ggml's broadcast rule)."""
    qtype, k, n, m = O.Q8_0, 256, 48, 3
    raws = [synth.make_weights(qtype, n, k, 40 + i) for i in range(2)]
    rng = np.random.default_rng(3)
    xf = rng.standard_normal((3, 4, m, k), dtype=np.float32)
    buf = ggml.Buffer(4 << 20)
    a = buf.alloc(ggml.new_tensor(qtype, [k, n, 2, 1]))
    buf.set(a, np.concatenate(raws).tobytes())
    b = buf.alloc(ggml.new_tensor(ggml.TYPE_F32, [k, m, 4, 3]))
    buf.set(b, xf.tobytes())
    node = buf.alloc(ggml.mul_mat(a, b))
    be = ggml.Backend(0)
    assert be.graph_compute([node]) == 0
    be.synchronize()
    y = np.frombuffer(buf.get(node), dtype=np.float32).reshape(3, 4, m, n)
    for i3 in range(3):
        for i2 in range(4):
            ref = O.matmul_f64(O.dequant(qtype, raws[i2 // 2], n, k), synth.bf16_bits(xf[i3, i2]))
            assert rel_err(y[i3, i2], ref) <= REL_TOL_EXACT_W
    be.free()
    buf.free()


@pytest.mark.gpu
@pytest.mark.parametrize("qtype", [O.Q4_0, O.Q6_K, O.Q5_K])
def test_mul_mat_id_node(cuda, qtype):
    k, n, n_expert, top_k, n_tokens = O.BLOCK_ELEMS[qtype] * 2, 64, 6, 2, 10
    raws = [synth.make_weights(qtype, n, k, 60 + e) for e in range(n_expert)]
    rng = np.random.default_rng(8)
    ids = np.stack([rng.choice(n_expert, top_k, replace=False) for _ in range(n_tokens)]).astype(np.int32)
    xf = rng.standard_normal((n_tokens, 1, k), dtype=np.float32)
    buf = ggml.Buffer(4 << 20)
    a = buf.alloc(ggml.new_tensor(qtype, [k, n, n_expert]))
    buf.set(a, np.concatenate(raws).tobytes())
    b = buf.alloc(ggml.new_tensor(ggml.TYPE_F32, [k, 1, n_tokens]))
    buf.set(b, xf.tobytes())
    it = buf.alloc(ggml.new_tensor(ggml.TYPE_I32, [top_k, n_tokens]))
    buf.set(it, ids.tobytes())
    node = buf.alloc(ggml.mul_mat_id(a, b, it))
    assert ggml.supports_op(node)
    be = ggml.Backend(0)
    assert be.graph_compute([node]) == 0
    be.synchronize()
    y = np.frombuffer(buf.get(node), dtype=np.float32).reshape(n_tokens, top_k, n)
    xb = synth.bf16_bits(xf[:, 0])
    for t in range(n_tokens):
        for s in range(top_k):
            ref = O.matmul_f64(O.dequant(qtype, raws[ids[t, s]], n, k), xb[t][None])[0]
            assert rel_err(y[t, s], ref) <= REL_TOL_EXACT_W
    be.free()
    buf.free()


@pytest.mark.gpu
def test_mul_mat_id_then_glu_fused_and_not(cuda):
    """MUL_MAT_ID followed by GLU over it: graph_compute runs the two as one
    pass (the product's own data is not written). Flagged OUTPUT, the
    product is computed and written, and the GLU result is the same bits."""
    qtype, k, F, n_expert, top_k, n_tokens = O.Q4_0, 128, 48, 5, 2, 9
    raws = [synth.make_weights(qtype, 2 * F, k, 80 + e) for e in range(n_expert)]
    rng = np.random.default_rng(9)
    ids = np.stack([rng.choice(n_expert, top_k, replace=False) for _ in range(n_tokens)]).astype(np.int32)
    xf = rng.standard_normal((n_tokens, 1, k), dtype=np.float32)
    buf = ggml.Buffer(4 << 20)
    a = buf.alloc(ggml.new_tensor(qtype, [k, 2 * F, n_expert]))
    buf.set(a, np.concatenate(raws).tobytes())
    b = buf.alloc(ggml.new_tensor(ggml.TYPE_F32, [k, 1, n_tokens]))
    buf.set(b, xf.tobytes())
    it = buf.alloc(ggml.new_tensor(ggml.TYPE_I32, [top_k, n_tokens]))
    buf.set(it, ids.tobytes())
    prod = buf.alloc(ggml.mul_mat_id(a, b, it))
    g = buf.alloc(ggml.glu(prod, ggml.GLU_SWIGLU))
    assert ggml.supports_op(g)
    sentinel = np.full(2 * F * top_k * n_tokens, 7.0, dtype=np.float32).tobytes()
    buf.set(prod, sentinel)
    be = ggml.Backend(0)
    assert be.graph_compute([prod, g]) == 0
    be.synchronize()
    assert buf.get(prod) == sentinel  # fused: the product was never written
    y = np.frombuffer(buf.get(g), dtype=np.float32).reshape(n_tokens, top_k, F)
    xb = synth.bf16_bits(xf[:, 0])
    for t in range(n_tokens):
        for s in range(top_k):
            p_ref = O.matmul_f64(O.dequant(qtype, raws[ids[t, s]], 2 * F, k), xb[t][None])[0]
            assert rel_err(y[t, s], O.glu_f64(p_ref, O.GLU_SWIGLU)) <= REL_TOL
    prod.flags = ggml.FLAG_OUTPUT
    assert be.graph_compute([prod, g]) == 0
    be.synchronize()
    assert buf.get(prod) != sentinel
    p = np.frombuffer(buf.get(prod), dtype=np.float32).reshape(n_tokens, top_k, 2 * F)
    assert np.frombuffer(buf.get(g), dtype=np.float32).reshape(n_tokens, top_k, F).tobytes() == y.tobytes()
    for t in range(n_tokens):
        for s in range(top_k):
            p_ref = O.matmul_f64(O.dequant(qtype, raws[ids[t, s]], 2 * F, k), xb[t][None])[0]
            assert rel_err(p[t, s], p_ref) <= REL_TOL_EXACT_W
    # A GLU output with padded rows (row stride F + 8 floats): the fused pass
    # writes packed rows, so graph_compute must run the two nodes unfused and
    # GLU honours the stride; the pad floats are never written.
    prod.flags = 0
    pad = 8
    gp = ggml.glu(prod, ggml.GLU_SWIGLU)
    gp.nb[1] = (F + pad) * 4
    gp.nb[2] = gp.nb[1] * top_k
    gp.nb[3] = gp.nb[2] * n_tokens
    gp_bytes = ggml.nbytes(gp)  # ggml_nbytes: the last row's pad is not part of the tensor
    assert gp_bytes == gp.nb[3] - pad * 4
    gp = buf.alloc(gp)
    assert ggml.supports_op(gp)
    L = ggml._lib()
    fill = (ctypes.c_uint8 * gp_bytes).from_buffer_copy(np.full(gp_bytes // 4, 5.0, np.float32).tobytes())
    assert L.spiral_buffer_set_tensor(buf.ptr, ctypes.byref(gp), fill, 0, gp_bytes) == 0
    assert be.graph_compute([prod, gp]) == 0
    be.synchronize()
    out = (ctypes.c_uint8 * gp.nb[3]).from_buffer_copy(np.full(gp.nb[3] // 4, 5.0, np.float32).tobytes())
    assert L.spiral_buffer_get_tensor(buf.ptr, ctypes.byref(gp), out, 0, gp_bytes) == 0
    rows = np.frombuffer(bytes(out), dtype=np.float32).reshape(n_tokens, top_k, F + pad)
    assert rows[:, :, :F].tobytes() == y.tobytes()
    assert (rows[:, :, F:] == 5.0).all()
    be.free()
    buf.free()


@pytest.mark.gpu
def test_mul_mat_id_then_swiglu_oai(cuda):
    """ggml_swiglu_oai over MUL_MAT_ID output, in the single-tensor form and
    the split form (separate gate and up expert stacks): graph_compute runs
    the products and the GLU as separate nodes (no fused form takes alpha and
    limit), and the result matches the float64 oracle of each product
    followed by SWIGLU_OAI. Outputs are scaled so both halves cross
    +-limit."""
    qtype, k, F, n_expert, top_k, n_tokens = O.Q4_0, 128, 32, 4, 2, 6
    alpha, limit = 1.702, 3.0
    raws = [synth.make_weights(qtype, 2 * F, k, 90 + e) for e in range(n_expert)]
    rng = np.random.default_rng(19)
    ids = np.stack([rng.choice(n_expert, top_k, replace=False) for _ in range(n_tokens)]).astype(np.int32)
    xf = (40.0 * rng.standard_normal((n_tokens, 1, k))).astype(np.float32)
    xb = synth.bf16_bits(xf[:, 0])
    buf = ggml.Buffer(4 << 20)
    a = buf.alloc(ggml.new_tensor(qtype, [k, 2 * F, n_expert]))
    buf.set(a, np.concatenate(raws).tobytes())
    b = buf.alloc(ggml.new_tensor(ggml.TYPE_F32, [k, 1, n_tokens]))
    buf.set(b, xf.tobytes())
    it = buf.alloc(ggml.new_tensor(ggml.TYPE_I32, [top_k, n_tokens]))
    buf.set(it, ids.tobytes())
    prod = buf.alloc(ggml.mul_mat_id(a, b, it))
    g = buf.alloc(ggml.glu(prod, ggml.GLU_SWIGLU_OAI, alpha=alpha, limit=limit))
    assert ggml.supports_op(g)
    sentinel = np.full(2 * F * top_k * n_tokens, 7.0, dtype=np.float32).tobytes()
    buf.set(prod, sentinel)
    be = ggml.Backend(0)
    assert be.graph_compute([prod, g]) == 0
    be.synchronize()
    assert buf.get(prod) != sentinel  # not fused: the product was written
    y = np.frombuffer(buf.get(g), dtype=np.float32).reshape(n_tokens, top_k, F)
    p = np.frombuffer(buf.get(prod), dtype=np.float32).reshape(n_tokens, top_k, 2 * F)
    assert np.abs(p).max() > limit and (p[..., :F] > limit).any() and (p[..., F:] < -limit).any()
    for t in range(n_tokens):
        for s in range(top_k):
            p_ref = O.matmul_f64(O.dequant(qtype, raws[ids[t, s]], 2 * F, k), xb[t][None])[0]
            want = O.glu_f64(p_ref, O.GLU_SWIGLU_OAI, alpha=alpha, limit=limit)
            assert rel_err(y[t, s], want) <= REL_TOL
    # The split form: gate and up experts in two tensors, two MUL_MAT_ID nodes.
    ag = buf.alloc(ggml.new_tensor(qtype, [k, F, n_expert]))
    au = buf.alloc(ggml.new_tensor(qtype, [k, F, n_expert]))
    rb = O.row_bytes(qtype, k)
    buf.set(ag, b"".join(r[: F * rb].tobytes() for r in raws))
    buf.set(au, b"".join(r[F * rb:].tobytes() for r in raws))
    pg = buf.alloc(ggml.mul_mat_id(ag, b, it))
    pu = buf.alloc(ggml.mul_mat_id(au, b, it))
    gs = buf.alloc(ggml.glu_split(pg, pu, ggml.GLU_SWIGLU_OAI, alpha=alpha, limit=limit))
    assert ggml.supports_op(gs)
    assert be.graph_compute([pg, pu, gs]) == 0
    be.synchronize()
    ys = np.frombuffer(buf.get(gs), dtype=np.float32).reshape(n_tokens, top_k, F)
    assert ys.tobytes() == y.tobytes()  # same products, same GLU: the same bits
    # ggml applies op_params[1] (swapped) to the single-tensor form only; a
    # split node carrying 1 still activates src0 (the gate), here unfused
    # (SWIGLU_OAI) and fused (SWIGLU over the two MUL_MAT_ID nodes).
    gsw = buf.alloc(ggml.glu_split(pg, pu, ggml.GLU_SWIGLU_OAI, swapped=True, alpha=alpha, limit=limit))
    assert be.graph_compute([pg, pu, gsw]) == 0
    be.synchronize()
    assert buf.get(gsw) == buf.get(gs)
    g0 = buf.alloc(ggml.glu_split(pg, pu, ggml.GLU_SWIGLU))
    g1 = buf.alloc(ggml.glu_split(pg, pu, ggml.GLU_SWIGLU, swapped=True))
    assert be.graph_compute([pg, pu, g0]) == 0
    assert be.graph_compute([pg, pu, g1]) == 0
    be.synchronize()
    assert buf.get(g1) == buf.get(g0)
    be.free()
    buf.free()


@pytest.mark.gpu
def test_mul_mat_id_then_glu_past_the_fused_shapes(cuda):
    """k > 4096: the fused pass is refused (SPIRAL_ERR_SHAPE), and
    graph_compute runs MUL_MAT_ID (its non-streaming kernel) and then the
    standalone GLU, with the same result as the oracle."""
    import torch
    from spiral_amd import ops

    qtype, k, F, n_expert, top_k, n_tokens = O.Q4_0, 4096 + 256, 24, 3, 2, 5
    raws = [synth.make_weights(qtype, 2 * F, k, 90 + e) for e in range(n_expert)]
    rng = np.random.default_rng(10)
    ids = np.stack([rng.choice(n_expert, top_k, replace=False) for _ in range(n_tokens)]).astype(np.int32)
    xf = rng.standard_normal((n_tokens, 1, k), dtype=np.float32)
    per = O.row_bytes(qtype, k) * 2 * F
    w = torch.cat([ops.to_planar(qtype, torch.from_numpy(r).to(cuda), 2 * F, k) for r in raws])
    xb = synth.bf16_bits(xf[:, 0])
    xd = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).to(cuda).view(n_tokens, 1, k)
    with pytest.raises(RuntimeError, match="SHAPE"):
        ops.mul_mat_id_glu(qtype, w, per, n_expert, 2 * F, k, xd, torch.from_numpy(ids).to(cuda), ops.GLU_GEGLU_ERF)
    buf = ggml.Buffer(4 << 20)
    a = buf.alloc(ggml.new_tensor(qtype, [k, 2 * F, n_expert]))
    buf.set(a, np.concatenate(raws).tobytes())
    b = buf.alloc(ggml.new_tensor(ggml.TYPE_F32, [k, 1, n_tokens]))
    buf.set(b, xf.tobytes())
    it = buf.alloc(ggml.new_tensor(ggml.TYPE_I32, [top_k, n_tokens]))
    buf.set(it, ids.tobytes())
    prod = buf.alloc(ggml.mul_mat_id(a, b, it))
    g = buf.alloc(ggml.glu(prod, ggml.GLU_GEGLU_ERF, swapped=True))
    be = ggml.Backend(0)
    assert be.graph_compute([prod, g]) == 0
    be.synchronize()
    y = np.frombuffer(buf.get(g), dtype=np.float32).reshape(n_tokens, top_k, F)
    for t in range(n_tokens):
        for s in range(top_k):
            p_ref = O.matmul_f64(O.dequant(qtype, raws[ids[t, s]], 2 * F, k), xb[t][None])[0]
            assert rel_err(y[t, s], O.glu_f64(p_ref, O.GLU_GEGLU_ERF, swapped=True)) <= REL_TOL
    be.free()
    buf.free()


@pytest.mark.gpu
def test_graph_of_several_nodes_and_refusal(cuda):
    qtype, k, n = O.Q4_0, 128, 32
    raw = synth.make_weights(qtype, n, k, 70)
    buf = ggml.Buffer(1 << 20)
    a = buf.alloc(ggml.new_tensor(qtype, [k, n]))
    buf.set(a, raw.tobytes())
    ids = buf.alloc(ggml.new_tensor(ggml.TYPE_I32, [3]))
    buf.set(ids, np.array([5, 0, 31], dtype=np.int32).tobytes())
    emb = buf.alloc(ggml.get_rows(a, ids))                 # [k, 3] F32
    view = ggml.new_tensor(ggml.TYPE_F32, [1])
    view.op = ggml.OP_VIEW
    prod = buf.alloc(ggml.mul_mat(a, emb))                  # [n, 3]
    be = ggml.Backend(0)
    assert be.graph_compute([emb, view, prod]) == 0
    be.synchronize()
    w = O.dequant(qtype, raw, n, k)
    e = np.frombuffer(buf.get(emb), dtype=np.float32).reshape(3, k)
    assert np.array_equal(e.view(np.uint32), w[[5, 0, 31]].astype(np.uint32) << 16)
    y = np.frombuffer(buf.get(prod), dtype=np.float32).reshape(3, n)
    assert rel_err(y, O.matmul_f64(w, w[[5, 0, 31]])) <= REL_TOL_EXACT_W
    bad = ggml.mul_mat(a, ggml.new_tensor(ggml.TYPE_I32, [k, 2]))
    before = buf.get(prod)
    assert STATUS[be.graph_compute([prod, bad])] == "SPIRAL_ERR_TYPE"
    be.synchronize()
    assert buf.get(prod) == before  # refused before anything ran
    be.free()
    buf.free()
