"""GPU parity of the decode layer and the verify window over Q8_0 experts and
mixed layers (IQ3_S gate/up with Q8_0 down and the reverse), against the C
oracle (src/q4_cpuexp.c: the per-type rows of q4_cpuex_dispatch2 /
q4_cpuex_dispatch_win).  Same bar and conditioning rule as the IQ3_S
decode tests: fp32 y within 1e-3 elementwise when the oracle's h is clear of
q8 rounding ties, else within twice the oracle's own shift under a 1e-7
perturbation of h.
"""
import ctypes

import numpy as np
import pytest

from conftest import layer_err, rel_err
from test_gpu_decode import dev, h_tie_margin, host, routed_ids

import oracle as om
import q4mi
from q4mi import synth

pytestmark = pytest.mark.gpu
T_IQ3_S, T_Q8_0 = q4mi.T_IQ3_S, q4mi.T_Q8_0
TOL = 1e-3
N_EMBD, N_FF, N_EXP = 2048, 512, 24


def arena_of(rng, gt, dt):
    """N_EXP packed experts gate[F][H] | up[F][H] | down[H][F] with the given
    gate/up and down types."""
    rg, rd = om.row_bytes(gt, N_EMBD), om.row_bytes(dt, N_FF)
    stride = 2 * N_FF * rg + N_EMBD * rd
    parts = []
    for _ in range(N_EXP):
        parts.append(synth.matrix(rng, gt, 2 * N_FF, N_EMBD))
        parts.append(synth.matrix(rng, dt, N_EMBD, N_FF))
    arena = np.concatenate(parts)
    assert arena.size == N_EXP * stride
    return arena, stride, 0, N_FF * rg, 2 * N_FF * rg


def conditioned_ok(oracle, y, yo, h, arena, stride, od, dt, ids, wts):
    """True when y meets the bar: elementwise 1e-3 on well-conditioned h,
    else the oracle's own sensitivity to a 1e-7 change of h."""
    if min(h_tie_margin(hj) for hj in h) >= 2e-5:
        return rel_err(y, yo) <= TOL
    rd = om.row_bytes(dt, N_FF)
    pr = np.random.default_rng(1)
    yp = np.zeros(N_EMBD, np.float32)
    for j, e in enumerate(ids):
        hj = (h[j] * (1 + 1e-7 * pr.standard_normal(N_FF))).astype(np.float32)
        wd = arena[e * stride + od:e * stride + od + N_EMBD * rd]
        yp += wts[j] * oracle.dot8_rows(dt, wd, N_EMBD, N_FF, hj[None])[0]
    return layer_err(y, yo) <= max(TOL, 2 * layer_err(yp, yo))


@pytest.mark.parametrize("gt,dt", [(T_Q8_0, T_Q8_0), (T_IQ3_S, T_Q8_0), (T_Q8_0, T_IQ3_S)])
def test_moe_decode_types(gpu, oracle, gt, dt):
    rng = np.random.default_rng(60 + 3 * gt + dt)
    arena, stride, og, ou, od = arena_of(rng, gt, dt)
    d_arena = dev(arena)
    for trial in range(3):
        x = rng.standard_normal(N_EMBD).astype(np.float32)
        ids, wts = routed_ids(oracle, rng, k=10, E=N_EXP - 1)
        ids = np.append(ids, N_EXP - 1).astype(np.int32)       # the last expert: shared
        wts = np.append(wts, 1.0).astype(np.float32)
        dx, y = dev(x), dev(np.zeros(N_EMBD, np.float32))
        ok = gpu.q4_hip_moe_exec(q4mi.ptr(d_arena), stride, ids.ctypes.data_as(ctypes.c_void_p),
                                 wts.ctypes.data_as(ctypes.c_void_p), len(ids), gt, og, gt, ou,
                                 dt, od, q4mi.ptr(dx), None, None, None, q4mi.ptr(y), N_FF,
                                 N_EMBD, N_EMBD)
        q4mi.check(ok, "q4_hip_moe_exec")
        yo, h = oracle.moe_tokens(N_EMBD, N_FF, gt, dt, arena, stride, x, ids[None], wts[None],
                                  want_h=True)
        assert conditioned_ok(oracle, host(y), yo[0], h, arena, stride, od, dt, ids, wts), trial


@pytest.mark.parametrize("gt,dt", [(T_Q8_0, T_Q8_0), (T_IQ3_S, T_Q8_0)])
def test_moe_window_types(gpu, oracle, gt, dt):
    """Two tokens through the window, each with its own top-8 + shared."""
    rng = np.random.default_rng(70 + 3 * gt + dt)
    arena, stride, og, ou, od = arena_of(rng, gt, dt)
    d_arena = dev(arena)
    n_tok = 2
    x = rng.standard_normal((n_tok, N_EMBD)).astype(np.float32)
    es = np.full((n_tok, 64), -1, np.int32)
    ew = np.zeros((n_tok, 64), np.float32)
    nh = np.zeros(n_tok, np.int32)
    all_ids, all_w = [], []
    for t in range(n_tok):
        ids, wts = routed_ids(oracle, rng, k=8, E=N_EXP - 1)
        ids = np.append(ids, N_EXP - 1).astype(np.int32)
        wts = np.append(wts, 1.0).astype(np.float32)
        es[t, :len(ids)], ew[t, :len(ids)], nh[t] = ids, wts, len(ids)
        all_ids.append(ids)
        all_w.append(wts)
    assert gpu.q4_hip_moe_win_ok(gt, gt, dt, N_EMBD, N_FF, n_tok)
    d_es, d_ew, d_nh, dx = dev(es), dev(ew), dev(nh), dev(x)
    y = dev(np.zeros((n_tok, N_EMBD), np.float32))
    q4mi.check(gpu.q4_hip_moe_exec_win(q4mi.ptr(d_arena), stride, q4mi.ptr(d_es), q4mi.ptr(d_ew),
                                       q4mi.ptr(d_nh), n_tok, gt, og, gt, ou, dt, od,
                                       q4mi.ptr(dx), None, q4mi.ptr(y), N_FF, N_EMBD, N_EMBD),
               "q4_hip_moe_exec_win")
    got = host(y)
    for t in range(n_tok):
        yo, h = oracle.moe_tokens(N_EMBD, N_FF, gt, dt, arena, stride, x[t], all_ids[t][None],
                                  all_w[t][None], want_h=True)
        assert conditioned_ok(oracle, got[t], yo[0], h, arena, stride, od, dt, all_ids[t],
                              all_w[t]), t
