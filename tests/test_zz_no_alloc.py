"""q4mi_moe_exec_noalloc (intermediates in a static device array, no
allocation) against q4_hip_moe_exec on the same inputs: the same kernels, so
y must match bit for bit.  Two calls in a row, the second with a smaller
input (fewer experts, smaller n_ff and hidden size), then the size limit."""
import ctypes

import numpy as np
import pytest

import q4mi
from q4mi import synth

pytestmark = pytest.mark.gpu
T = q4mi.T_IQ3_S


def _run(L, fn, d_arena, stride, og, ou, od, ids, wts, x, n_ff, n_embd, noalloc):
    import torch
    dx = torch.from_numpy(x).cuda()
    y = torch.zeros(n_embd, dtype=torch.float32, device="cuda")
    ids = np.ascontiguousarray(ids, np.int32)
    wts = np.ascontiguousarray(wts, np.float32)
    pi, pw = ids.ctypes.data_as(ctypes.c_void_p), wts.ctypes.data_as(ctypes.c_void_p)
    if noalloc:
        ok = L.q4mi_moe_exec_noalloc(d_arena.data_ptr(), stride, pi, pw, len(ids), T, og, T, ou,
                                     T, od, dx.data_ptr(), y.data_ptr(), n_ff, n_embd, n_embd)
    else:
        ok = L.q4_hip_moe_exec(d_arena.data_ptr(), stride, pi, pw, len(ids), T, og, T, ou, T, od,
                               dx.data_ptr(), None, None, None, y.data_ptr(), n_ff, n_embd,
                               n_embd)
    q4mi.check(ok, fn)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def test_noalloc_matches_exec(gpu):
    import torch
    for step, (n_embd, n_ff, n_exp, n_pick) in enumerate([(2048, 1024, 40, 33),
                                                          (1024, 512, 12, 5)]):
        rng = np.random.default_rng(700 + step)
        arena = synth.expert_arena(rng, n_exp, n_embd, n_ff)
        stride, og, ou, od = synth.expert_stride(n_embd, n_ff)
        d_arena = torch.from_numpy(arena).cuda()
        ids = rng.choice(n_exp, n_pick, replace=False).astype(np.int32)
        wts = rng.random(n_pick).astype(np.float32)
        x = rng.standard_normal(n_embd).astype(np.float32)
        args = (d_arena, stride, og, ou, od, ids, wts, x, n_ff, n_embd)
        want = _run(gpu, "q4_hip_moe_exec", *args, noalloc=False)
        got = _run(gpu, "q4mi_moe_exec_noalloc", *args, noalloc=True)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), step
        assert np.abs(want).max() > 0
    # beyond the static array (n_ff > 1024): rejected before any launch
    ids = np.array([0], np.int32)
    w = np.array([1.0], np.float32)
    assert not gpu.q4mi_moe_exec_noalloc(1, 0, ids.ctypes.data_as(ctypes.c_void_p),
                                         w.ctypes.data_as(ctypes.c_void_p), 1, T, 0, T, 0, T,
                                         0, 16, 16, 2048, 2048, 2048)
    assert "static scratch" in q4mi.last_error()
