"""q4mi_moe_exec_noalloc (intermediates in a static device array, no
allocation) against q4_hip_moe_exec on the same inputs: the same kernels, so
y must match bit for bit.  Two calls in a row, the second with a smaller
input (fewer experts, smaller n_ff and hidden size), then the size limit."""
import ctypes
import os
import subprocess
import sys
import textwrap

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


FRESH = textwrap.dedent(r"""
    import ctypes, sys
    import numpy as np
    import torch
    import q4mi
    from q4mi import synth
    M = q4mi.meas()                        # product ABI + the allocation counter
    torch.cuda.set_device(0)
    q4mi.use_torch_stream(M)
    T = q4mi.T_IQ3_S
    outs = []
    for step, (n_embd, n_ff, n_exp, n_pick) in enumerate([(2048, 1024, 24, 11), (1024, 512, 8, 5)]):
        rng = np.random.default_rng(900 + step)
        arena = synth.expert_arena(rng, n_exp, n_embd, n_ff)
        stride, og, ou, od = synth.expert_stride(n_embd, n_ff)
        d_arena = torch.from_numpy(arena).cuda()
        ids = rng.choice(n_exp, n_pick, replace=False).astype(np.int32)
        wts = rng.random(n_pick).astype(np.float32)
        dx = torch.from_numpy(rng.standard_normal(n_embd).astype(np.float32)).cuda()
        y = torch.zeros(n_embd, dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        before = M.q4mi_alloc_count()
        ok = M.q4mi_moe_exec_noalloc(d_arena.data_ptr(), stride, ids.ctypes.data_as(ctypes.c_void_p),
                                     wts.ctypes.data_as(ctypes.c_void_p), n_pick, T, og, T, ou, T,
                                     od, dx.data_ptr(), y.data_ptr(), n_ff, n_embd, n_embd)
        q4mi.check(ok, "q4mi_moe_exec_noalloc", M)
        torch.cuda.synchronize()
        assert M.q4mi_alloc_count() == before == 0, ("library allocated", before, M.q4mi_alloc_count())
        outs.append((y.cpu().numpy(), (d_arena, stride, og, ou, od, ids, wts, dx, n_ff, n_embd)))
    # the allocating entry point afterwards, on the same inputs: same bits
    for got, (d_arena, stride, og, ou, od, ids, wts, dx, n_ff, n_embd) in outs:
        y = torch.zeros(n_embd, dtype=torch.float32, device="cuda")
        ok = M.q4_hip_moe_exec(d_arena.data_ptr(), stride, ids.ctypes.data_as(ctypes.c_void_p),
                               wts.ctypes.data_as(ctypes.c_void_p), len(ids), T, og, T, ou, T, od,
                               dx.data_ptr(), None, None, None, y.data_ptr(), n_ff, n_embd, n_embd)
        q4mi.check(ok, "q4_hip_moe_exec", M)
        torch.cuda.synchronize()
        assert np.array_equal(got.view(np.uint32), y.cpu().numpy().view(np.uint32))
    assert M.q4mi_alloc_count() > 0          # the allocating path did allocate
    print("noalloc fresh process ok")
""")


def test_noalloc_first_in_fresh_process():
    """The allocation-free entry point called first in a new process, before
    any allocating entry point has warmed the library: the library's
    allocation counter stays at 0 through two calls (the second smaller), and
    the allocating entry point then gives the same bits."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join([os.path.join(root, "suzuku-engine-q4_amd"),
                                         env.get("PYTHONPATH", "")])
    r = subprocess.run([sys.executable, "-c", FRESH], env=env, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "noalloc fresh process ok" in r.stdout
