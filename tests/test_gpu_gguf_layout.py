"""The GGUF expert layout (gate, up and down as separate stacked tensors,
blk.N.ffn_{gate,up,down}_exps; the slices src/q4_expert.c:962-982 reads)
through q4mi_moe_exec_parts and q4mi_mmq_gate_up_parts.  The kernels are the
packed-arena ones with other addresses, so results equal the packed path bit
for bit; a mixed layer (IQ3_S gate/up, Q8_0 down: different strides) is
checked against the oracle (max rel error <= 1e-3)."""
import numpy as np
import pytest

from conftest import rel_err

import oracle as om
import q4mi
from q4mi import synth

pytestmark = pytest.mark.gpu
T_IQ3_S, T_Q8_0 = q4mi.T_IQ3_S, q4mi.T_Q8_0


# device copies made by dev() stay referenced until host() has synchronized:
# a temporary passed straight into an asynchronous launch would otherwise
# return its memory to torch's cache before the kernel has read it
_KEEP = []


def dev(a):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    _KEEP.append(t)
    return t


def host(t):
    import torch
    torch.cuda.synchronize()
    _KEEP.clear()
    return t.cpu().numpy()


def zeros(shape, dtype=None):
    import torch
    return torch.zeros(shape, dtype=dtype or torch.float32, device="cuda")


def split(arena, n_exp, stride, og, ou, od, gu_bytes, d_bytes):
    """Packed experts -> the three stacked tensors of a GGUF layer."""
    a = arena.reshape(n_exp, stride)
    return (np.ascontiguousarray(a[:, og:og + gu_bytes]).reshape(-1),
            np.ascontiguousarray(a[:, ou:ou + gu_bytes]).reshape(-1),
            np.ascontiguousarray(a[:, od:od + d_bytes]).reshape(-1))


def lists(rng, n_tok, n_exp, k):
    es = np.full((n_tok, 64), -1, np.int32)
    ew = np.zeros((n_tok, 64), np.float32)
    ids = np.stack([rng.choice(n_exp, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
    w = rng.random((n_tok, k)).astype(np.float32)
    es[:, :k], ew[:, :k] = ids, w
    return es, ew, np.full(n_tok, k, np.int32), ids, w


@pytest.mark.parametrize("n_tok", [1, 4])
def test_decode_parts_equals_packed(gpu, n_tok):
    H, F, E = 2048, 512, 40
    rng = np.random.default_rng(500 + n_tok)
    arena = synth.expert_arena(rng, E, H, F)
    stride, og, ou, od = synth.expert_stride(H, F)
    g, u, d = split(arena, E, stride, og, ou, od, F * 880, H * 220)
    dg, du, dd, da = dev(g), dev(u), dev(d), dev(arena)
    es, ew, nh, _, _ = lists(rng, n_tok, E, 10)
    x = rng.standard_normal((n_tok, H)).astype(np.float32)
    P = q4mi.ptr
    d_es, d_ew, d_nh, dx = dev(es), dev(ew), dev(nh), dev(x)
    y1, y2 = zeros((n_tok, H)), zeros((n_tok, H))
    q4mi.check(gpu.q4mi_moe_exec_parts(P(dg), P(du), P(dd), F * 880, H * 220, P(d_es), P(d_ew),
                                       P(d_nh), n_tok, T_IQ3_S, T_IQ3_S, P(dx), P(y1), F, H, H),
               "exec_parts")
    if n_tok == 1:
        q4mi.check(gpu.q4_hip_moe_exec_dev(P(da), stride, P(d_es), P(d_ew), P(d_nh), T_IQ3_S, og,
                                           T_IQ3_S, ou, T_IQ3_S, od, P(dx), None, None, None,
                                           P(y2), F, H, H), "exec_dev")
    else:
        q4mi.check(gpu.q4_hip_moe_exec_win(P(da), stride, P(d_es), P(d_ew), P(d_nh), n_tok,
                                           T_IQ3_S, og, T_IQ3_S, ou, T_IQ3_S, od, P(dx), None,
                                           P(y2), F, H, H), "exec_win")
    a, b = host(y1), host(y2)
    assert np.abs(a).max() > 0
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_decode_parts_mixed_types(gpu, oracle):
    """IQ3_S gate/up with a Q8_0 down tensor (down stride != gate stride),
    4 tokens, against the oracle on the equivalent packed experts."""
    H, F, E = 2048, 512, 24
    rng = np.random.default_rng(77)
    g = synth.matrix(rng, T_IQ3_S, E * F, H)
    u = synth.matrix(rng, T_IQ3_S, E * F, H)
    d = synth.matrix(rng, T_Q8_0, E * H, F)
    rg, rd = om.row_bytes(T_IQ3_S, H), om.row_bytes(T_Q8_0, F)
    gs, ds = F * rg, H * rd
    packed = np.concatenate([np.concatenate([g[e * gs:(e + 1) * gs], u[e * gs:(e + 1) * gs],
                                             d[e * ds:(e + 1) * ds]]) for e in range(E)])
    stride = 2 * gs + ds
    n_tok = 4
    es, ew, nh, ids, w = lists(rng, n_tok, E, 8)
    x = rng.standard_normal((n_tok, H)).astype(np.float32)
    P = q4mi.ptr
    dg, du, dd = dev(g), dev(u), dev(d)
    d_es, d_ew, d_nh, dx = dev(es), dev(ew), dev(nh), dev(x)
    y = zeros((n_tok, H))
    q4mi.check(gpu.q4mi_moe_exec_parts(P(dg), P(du), P(dd), gs, ds, P(d_es), P(d_ew), P(d_nh),
                                       n_tok, T_IQ3_S, T_Q8_0, P(dx), P(y), F, H, H),
               "exec_parts")
    yo = oracle.moe_tokens(H, F, T_IQ3_S, T_Q8_0, packed, stride, x, ids, w)
    assert rel_err(host(y), yo) <= 1e-3


def test_mmq_gate_up_parts_equals_packed(gpu):
    """Fused gate/up MMQ over separate gate/up tensors plus a shared expert
    kept in its own tensors: q8(h) codes and scales equal the packed
    q4mi_mmq_gate_up_x launch bit for bit."""
    import torch
    H, F, E, T = 2048, 512, 12, 300
    rng = np.random.default_rng(88)
    arena = synth.expert_arena(rng, E + 1, H, F)
    stride, og, ou, od = synth.expert_stride(H, F)
    g, u, _ = split(arena, E + 1, stride, og, ou, od, F * 880, H * 220)
    gs = F * 880
    per = [40, 0, 7, 130, 1, 33, 64, 5, 20, 0, 77, 9]
    rows = sum(per)
    a_tok = np.concatenate([np.concatenate([rng.integers(0, T, n) for n in per]),
                            np.arange(T)]).astype(np.int32)
    bounds = np.concatenate([[0], np.cumsum(per), [rows + T]]).astype(np.int32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    P = q4mi.ptr
    L = gpu
    xq = zeros(int(L.q4_mmq_q8_bytes(T, H)), torch.uint8)
    q4mi.check(L.q4_mmq_quantize(P(dev(x)), None, P(xq), T_IQ3_S, H, T), "q8 x")
    d_tok, d_b = dev(a_tok), dev(bounds)
    n_all = rows + T
    hq1 = zeros(int(L.q4_mmq_q8_bytes(n_all, F)), torch.uint8)
    hq2 = zeros(int(L.q4_mmq_q8_bytes(n_all, F)), torch.uint8)
    dg, du = dev(g[:E * gs]), dev(u[:E * gs])
    sg_, su_ = dev(g[E * gs:]), dev(u[E * gs:])
    da = dev(arena)
    q4mi.check(L.q4mi_mmq_gate_up_parts(P(dg), P(du), T_IQ3_S, F, H, gs, E, P(xq), T, P(d_tok),
                                        P(d_b), n_all, P(hq1), P(sg_), P(su_)), "gate_up_parts")
    q4mi.check(L.q4mi_mmq_gate_up_x(P(da), P(da) + E * stride, T_IQ3_S, F, H, stride, E, P(xq),
                                    T, P(d_tok), P(d_b), n_all, P(hq2)), "gate_up_x")
    a, b = host(hq1), host(hq2)
    n = n_all * F * 2 + n_all * F // 32 * 4
    assert np.abs(a[:n_all * F * 2].view(np.float16)).max() > 0
    assert np.array_equal(a[:n], b[:n])
