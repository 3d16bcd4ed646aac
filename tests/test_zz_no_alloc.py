"""spiral_mul_mat_id_noalloc: MUL_MAT_ID with the routing lists in the
library's own device array instead of a caller workspace (for callers that
cannot allocate). Called through the C ABI and compared with
spiral_mul_mat_id on the same inputs: the same kernels run, so the outputs
must be equal bit for bit. Two calls in a row, the second with fewer
(token, slot) pairs, so the second reads lists the first one's larger run
left behind in the shared array; both above 1024 pairs, where the routing
lists are written to that array, and a decode-size third call."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from spiral_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _noalloc(qtype, w, per, n_expert, n, k, x, ids, y, y_type):
    L = _lib.lib()
    n_tokens, top_k = ids.shape
    return L.spiral_mul_mat_id_noalloc(qtype, _ptr(w), per, n_expert, n, k, _ptr(x), x.shape[1], _ptr(ids),
                                       n_tokens, top_k, _ptr(y), y_type,
                                       ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


def test_noalloc_matches_workspace_form(cuda):
    qtype, n_expert, n, k = O.Q4_0, 24, 96, 512
    per = O.row_bytes(qtype, k) * n
    w = torch.cat([ops.to_planar(qtype, torch.from_numpy(synth.make_weights(qtype, n, k, 500 + e)).to(cuda), n, k)
                   for e in range(n_expert)])
    rng = np.random.default_rng(3)
    for n_tokens, top_k, x_slots in ((200, 8, 1), (150, 8, 8), (40, 4, 1)):  # 1600, 1200, 160 pairs
        ids = np.stack([rng.choice(n_expert, top_k, replace=False) for _ in range(n_tokens)]).astype(np.int32)
        ids[::13, 0] = -1  # routed nowhere: zero rows on both paths
        x = synth.make_x(n_tokens * x_slots, k, n_tokens).reshape(n_tokens, x_slots, k)
        xd = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(cuda)
        idd = torch.from_numpy(ids).to(cuda)
        for out_dtype, y_type in ((torch.float32, _lib.TYPE_F32), (torch.bfloat16, _lib.TYPE_BF16)):
            want = ops.mul_mat_id(qtype, w, per, n_expert, n, k, xd, idd, out_dtype=out_dtype)
            got = torch.full((n_tokens, top_k, n), 3.0, dtype=out_dtype, device=cuda)
            assert _noalloc(qtype, w, per, n_expert, n, k, xd, idd, got, y_type) == 0
            torch.cuda.synchronize()
            assert torch.equal(got, want), (n_tokens, top_k, out_dtype)
        assert not got[torch.from_numpy(ids < 0).to(cuda)].any()


def test_noalloc_refuses_lists_beyond_the_array(cuda):
    """More experts plus pairs than the array holds: SPIRAL_ERR_CAPACITY,
    reported before anything runs (the pointers are never touched)."""
    L = _lib.lib()
    cap = 1 << 20
    assert L.spiral_mul_mat_id_workspace_bytes(1, cap // 4 - 1, 1) > cap
    p = ctypes.c_void_p(4096)
    assert L.spiral_mul_mat_id_noalloc(O.Q4_0, p, 144, 1, 4, 64, p, 1, p, cap // 4 - 1, 1, p, _lib.TYPE_F32,
                                       None) == 7
