"""GPU parity for the router front q4mi_moe_route (router GEMV + shared-expert
gate + softmax/top-k into per-token device lists) against the C oracle, and
the layer it feeds (decode / verify window with the gated shared expert).

Bars: logits bit-exact (the dot order is fixed: or_router restates it);
routing ids bit-exact; routing weights and the gate <= 1e-6 relative (GPU
exp vs the host's expf); layer outputs max rel error <= 1e-3.
"""
import numpy as np
import pytest

from conftest import rel_err

import oracle as om
import q4mi
from q4mi import synth

pytestmark = pytest.mark.gpu
T_IQ3_S = q4mi.T_IQ3_S
TOL = 1e-3


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


def router_rows(rng, ty, n_exp, K):
    w = (rng.standard_normal((n_exp, K)) * 0.05).astype(np.float32)
    if ty == 0:
        return w
    if ty == 1:
        return w.astype(np.float16).view(np.uint8)
    return (w.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)


def route(L, wr, ty, sgw, x, n_exp, topk, shared, ostride=64):
    import torch
    T, K = x.shape
    lg = zeros((T, n_exp))
    ids = torch.full((T, ostride), -7, dtype=torch.int32, device="cuda")
    wts = zeros((T, ostride))
    nh = zeros(T, torch.int32)
    sg = zeros(T)
    q4mi.check(L.q4mi_moe_route(q4mi.ptr(wr), ty, q4mi.ptr(sgw), q4mi.ptr(dev(x)), T, K, n_exp,
                                topk, q4mi.ptr(lg), q4mi.ptr(ids), q4mi.ptr(wts), q4mi.ptr(nh),
                                ostride, shared, q4mi.ptr(sg) if sgw is not None else None),
               "q4mi_moe_route")
    return host(lg), host(ids), host(wts), host(nh), host(sg)


@pytest.mark.parametrize("ty,T,K,gate", [(0, 1, 2048, True), (0, 4, 2048, True),
                                         (30, 4, 2048, False), (1, 37, 1024, True),
                                         (0, 300, 4096, True), (30, 2048, 2048, True)])
def test_route_front_matches_oracle(gpu, oracle, ty, T, K, gate):
    rng = np.random.default_rng(ty * 100 + T + K)
    n_exp, topk = 512, 10
    w = router_rows(rng, ty, n_exp, K)
    x = rng.standard_normal((T, K)).astype(np.float32)
    g = (rng.standard_normal(K) * 0.02).astype(np.float32) if gate else None
    lg, ids, wts, nh, sg = route(gpu, dev(w), ty, dev(g) if gate else None, x, n_exp, topk,
                                 512)
    res = oracle.router(ty, w, n_exp, K, x, sgw=g)
    olg, osg = res if gate else (res, None)
    assert np.array_equal(lg.view(np.uint32), olg.view(np.uint32))
    oid, ow = oracle.softmax_topk(olg, topk)
    assert np.array_equal(ids[:, :topk], oid)
    assert np.allclose(wts[:, :topk], ow, rtol=1e-6, atol=1e-9)
    # the shared expert's entry and the per-token counts
    assert np.all(ids[:, topk] == 512) and np.all(nh == topk + 1)
    if gate:
        assert np.allclose(sg, osg, rtol=1e-6, atol=0)
        assert np.allclose(wts[:, topk], osg, rtol=1e-6, atol=0)
    else:
        assert np.all(wts[:, topk] == 1.0)
    assert np.all(ids[:, topk + 1:] == -7)     # nothing written past the row's entries


def test_route_front_rejects(gpu):
    import torch
    x = zeros((1, 2048))
    lg, ids, wts = zeros((1, 512)), zeros((1, 64), torch.int32), zeros((1, 64))
    P = q4mi.ptr
    assert not gpu.q4mi_moe_route(P(x), 2, None, P(x), 1, 2048, 512, 10, P(lg), P(ids), P(wts),
                                  None, 64, -1, None)          # router type
    assert not gpu.q4mi_moe_route(P(x), 0, None, P(x), 1, 2000, 512, 10, P(lg), P(ids), P(wts),
                                  None, 64, -1, None)          # n_embd % 256
    assert not gpu.q4mi_moe_route(P(x), 0, None, P(x), 1, 2048, 512, 10, P(lg), P(ids), P(wts),
                                  None, 10, 512, None)         # ostride too small
    assert not gpu.q4mi_moe_route(P(x), 0, P(x), P(x), 1, 2048, 512, 10, P(lg), P(ids), P(wts),
                                  None, 64, 512, None)         # gate without d_sg


@pytest.mark.parametrize("n_tok", [1, 4])
def test_routed_layer_with_gated_shared_expert(gpu, oracle, n_tok):
    """Router front -> device lists -> decode (1 token, q4_hip_moe_exec_dev)
    or verify window (4 tokens): y = sum_k w_k FFN_k(x) + sg * FFN_shared(x)
    against the oracle's layer with the oracle's routing and gate."""
    from test_gpu_decode import layer
    ly = layer()
    H, F = ly.n_embd, ly.n_ff
    rng = np.random.default_rng(60 + n_tok)
    w = router_rows(rng, 0, 512, H)
    g = (rng.standard_normal(H) * 0.02).astype(np.float32)
    x = rng.standard_normal((n_tok, H)).astype(np.float32)
    import torch
    dx = dev(x)
    lg, ids, wts, nh = zeros((n_tok, 512)), zeros((n_tok, 64), torch.int32), zeros((n_tok, 64)), \
        zeros(n_tok, torch.int32)
    sg = zeros(n_tok)
    P = q4mi.ptr
    q4mi.check(gpu.q4mi_moe_route(P(dev(w)), 0, P(dev(g)), P(dx), n_tok, H, 512, 10, P(lg),
                                  P(ids), P(wts), P(nh), 64, 512, P(sg)), "route")
    y = zeros((n_tok, H))
    if n_tok == 1:
        q4mi.check(gpu.q4_hip_moe_exec_dev(P(ly.d_arena), ly.stride, P(ids), P(wts), P(nh),
                                           T_IQ3_S, ly.og, T_IQ3_S, ly.ou, T_IQ3_S, ly.od, P(dx),
                                           None, None, None, P(y), F, H, H), "exec_dev")
    else:
        q4mi.check(gpu.q4_hip_moe_exec_win(P(ly.d_arena), ly.stride, P(ids), P(wts), P(nh),
                                           n_tok, T_IQ3_S, ly.og, T_IQ3_S, ly.ou, T_IQ3_S, ly.od,
                                           P(dx), None, P(y), F, H, H), "exec_win")
    olg, osg = oracle.router(0, w, 512, H, x, sgw=g)
    oid, ow = oracle.softmax_topk(olg, 10)
    sid = np.concatenate([oid, np.full((n_tok, 1), 512, np.int32)], 1)
    sw = np.concatenate([ow, osg[:, None]], 1).astype(np.float32)
    yo = oracle.moe_tokens(H, F, T_IQ3_S, T_IQ3_S, ly.arena, ly.stride, x, sid, sw)
    assert rel_err(host(y), yo) <= TOL


@pytest.mark.parametrize("gate,rtype,n_exp,topk", [(True, 0, 512, 10), (False, 30, 512, 10),
                                                   (True, 1, 200, 63), (True, 0, 8, 10)])
def test_route_exec_equals_route_then_exec_dev(gpu, oracle, gate, rtype, n_exp, topk):
    """q4mi_moe_route_exec (top-k taken inside the layer's gate/up blocks)
    against q4mi_moe_route + q4_hip_moe_exec_dev on the same inputs: logits,
    gate, lists and y equal bit for bit (the same top-k code on the same
    logits); and y against the oracle's layer with the oracle's routing.
    Covers fewer experts than picks (n_exp 8 < topk 10: ids -1 past n_exp)
    and 63 picks + the shared entry (the 64-entry bound)."""
    import torch
    from test_gpu_decode import layer
    ly = layer()
    H, F = ly.n_embd, ly.n_ff
    rng = np.random.default_rng(90 + topk + n_exp)
    w = router_rows(rng, rtype, n_exp, H)
    g = (rng.standard_normal(H) * 0.02).astype(np.float32) if gate else None
    x = rng.standard_normal((1, H)).astype(np.float32)
    dx, dw = dev(x), dev(w)
    dg = dev(g) if gate else None
    P = q4mi.ptr
    shared = 512
    outs = []
    for fused in (False, True):
        lg, ids, wts, nh = zeros((1, n_exp)), zeros((1, 64), torch.int32), zeros((1, 64)), \
            zeros(1, torch.int32)
        ids.fill_(-7)
        sg, y = zeros(1), zeros((1, H))
        gp = P(dg) if gate else None
        if fused:
            q4mi.check(gpu.q4mi_moe_route_exec(P(dw), rtype, gp, P(dx), H, n_exp, topk, P(lg),
                                               P(ids), P(wts), P(nh), shared, P(sg),
                                               P(ly.d_arena), ly.stride, T_IQ3_S, ly.og,
                                               T_IQ3_S, ly.ou, T_IQ3_S, ly.od, P(y), F),
                       "route_exec")
        else:
            q4mi.check(gpu.q4mi_moe_route(P(dw), rtype, gp, P(dx), 1, H, n_exp, topk, P(lg),
                                          P(ids), P(wts), P(nh), 64, shared, P(sg)), "route")
            q4mi.check(gpu.q4_hip_moe_exec_dev(P(ly.d_arena), ly.stride, P(ids), P(wts), P(nh),
                                               T_IQ3_S, ly.og, T_IQ3_S, ly.ou, T_IQ3_S, ly.od,
                                               P(dx), None, None, None, P(y), F, H, H),
                       "exec_dev")
        E = topk + 1
        outs.append([host(t) for t in (lg, sg, y)] + [host(ids)[:, :E], host(wts)[:, :E],
                                                      host(nh)])
    for a, b in zip(*outs):
        assert np.array_equal(a, b)
    oid, ow = oracle.softmax_topk(outs[1][0], min(topk, n_exp))
    got = outs[1][3][0, :min(topk, n_exp)]
    assert np.array_equal(got, oid[0])
    sgv = outs[1][1][0] if gate else 1.0
    sid = np.concatenate([oid, np.full((1, 1), shared, np.int32)], 1)
    sw = np.concatenate([ow, np.full((1, 1), sgv, np.float32)], 1).astype(np.float32)
    yo = oracle.moe_tokens(H, F, T_IQ3_S, T_IQ3_S, ly.arena, ly.stride, x, sid, sw)
    assert rel_err(outs[1][2], yo) <= TOL


def test_route_exec_rejects(gpu):
    """Partial list outputs and more than 64 entries are refused before any
    launch."""
    import torch
    P = q4mi.ptr
    b = zeros(4096)
    i = zeros(64, torch.int32)
    assert not gpu.q4mi_moe_route_exec(P(b), 0, None, P(b), 256, 8, 10, P(b), P(i), None, None,
                                       -1, None, P(b), 0, T_IQ3_S, 0, T_IQ3_S, 0, T_IQ3_S, 0,
                                       P(b), 256)
    assert not gpu.q4mi_moe_route_exec(P(b), 0, None, P(b), 256, 64, 64, P(b), None, None, None,
                                       5, None, P(b), 0, T_IQ3_S, 0, T_IQ3_S, 0, T_IQ3_S, 0,
                                       P(b), 256)


def test_sgate_axpy_and_dot_sigmoid(gpu, oracle):
    """q4_hip_sgate_axpy / q4_hip_dot_sigmoid (the reference's separate gate
    application): sg equals the oracle's gate (the router's dot order) to
    1e-6, y += sg * sh."""
    import torch
    rng = np.random.default_rng(71)
    n, T = 2048, 5
    g = (rng.standard_normal(n) * 0.02).astype(np.float32)
    x = rng.standard_normal((T, n)).astype(np.float32)
    sh = rng.standard_normal((T, n)).astype(np.float32)
    y0 = rng.standard_normal((T, n)).astype(np.float32)
    y = dev(y0)
    q4mi.check(gpu.q4_hip_sgate_axpy(q4mi.ptr(y), q4mi.ptr(dev(sh)), q4mi.ptr(dev(g)),
                                     q4mi.ptr(dev(x)), n, T), "sgate_axpy")
    out = zeros(1)
    q4mi.check(gpu.q4_hip_dot_sigmoid(q4mi.ptr(dev(g)), q4mi.ptr(dev(x[2])), q4mi.ptr(out), n),
               "dot_sigmoid")
    _, osg = oracle.router(0, np.zeros((1, n), np.float32), 1, n, x, sgw=g)
    want = y0 + osg[:, None] * sh
    assert rel_err(host(y), want) <= 1e-5
    assert abs(float(host(out)[0]) - osg[2]) <= 1e-6 * abs(osg[2])
    assert not gpu.q4_hip_sgate_axpy(q4mi.ptr(y), q4mi.ptr(y), q4mi.ptr(y), q4mi.ptr(y), 0, 1)


@pytest.mark.parametrize("n,off", [(1000, 0), (2048, 1), (77, 3), (4096 + 130, 2)])
def test_sgate_any_size_and_alignment(gpu, n, off):
    """Any n and any (float) alignment, as the reference accepts: the gate
    matches a float64 sigmoid(w . x) to 1e-6 relative, and y += sg * sh to
    1e-4 (one fp32 rounding of y0 + sg sh against float64, near-cancelling
    sums included)."""
    rng = np.random.default_rng(n + off)
    T = 3
    g = (rng.standard_normal(n) * 0.02).astype(np.float32)
    x = rng.standard_normal((T, n)).astype(np.float32)
    sh = rng.standard_normal((T, n)).astype(np.float32)
    y0 = rng.standard_normal((T, n)).astype(np.float32)
    # misalign w and x by `off` floats inside padded device buffers
    dg = dev(np.concatenate([np.zeros(off, np.float32), g]))
    dx = dev(np.concatenate([np.zeros(off, np.float32), x.ravel()]))
    y = dev(y0)
    pw, px = q4mi.ptr(dg) + 4 * off, q4mi.ptr(dx) + 4 * off
    q4mi.check(gpu.q4_hip_sgate_axpy(q4mi.ptr(y), q4mi.ptr(dev(sh)), pw, px, n, T), "sgate_axpy")
    out = zeros(1)
    q4mi.check(gpu.q4_hip_dot_sigmoid(pw, px + 4 * n, q4mi.ptr(out), n), "dot_sigmoid")
    d = x.astype(np.float64) @ g.astype(np.float64)
    sg = 1.0 / (1.0 + np.exp(-d))
    assert abs(float(host(out)[0]) - sg[1]) <= 1e-6 * sg[1]
    want = y0.astype(np.float64) + sg[:, None] * sh
    assert rel_err(host(y), want.astype(np.float32)) <= 1e-4


def test_routed_window_graph_replays(gpu):
    """Router front + verify window captured once in a HIP graph and
    replayed over three inputs (new x copied in between, eager work and
    synchronizations between replays): every replay equals the eager call
    bit for bit (no memset nodes; deterministic kernels)."""
    import torch
    from test_gpu_decode import layer
    ly = layer()
    H, F, n_tok = ly.n_embd, ly.n_ff, 4
    rng = np.random.default_rng(88)
    w = dev(router_rows(rng, 0, 512, H))
    g = dev((rng.standard_normal(H) * 0.02).astype(np.float32))
    xs = [rng.standard_normal((n_tok, H)).astype(np.float32) for _ in range(3)]
    x = dev(xs[0])
    lg, ids, wts = zeros((n_tok, 512)), zeros((n_tok, 64), torch.int32), zeros((n_tok, 64))
    nh, sg, y = zeros(n_tok, torch.int32), zeros(n_tok), zeros((n_tok, H))
    P = q4mi.ptr

    def layer_call():
        q4mi.check(gpu.q4mi_moe_route(P(w), 0, P(g), P(x), n_tok, H, 512, 10, P(lg), P(ids),
                                      P(wts), P(nh), 64, 512, P(sg)), "route")
        q4mi.check(gpu.q4_hip_moe_exec_win(P(ly.d_arena), ly.stride, P(ids), P(wts), P(nh),
                                           n_tok, T_IQ3_S, ly.og, T_IQ3_S, ly.ou, T_IQ3_S, ly.od,
                                           P(x), None, P(y), F, H, H), "exec_win")
    eager = []
    for xi in xs:
        x.copy_(torch.from_numpy(xi).cuda())
        y.zero_()
        layer_call()
        eager.append(host(y).copy())
    gr = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    with torch.cuda.graph(gr, stream=s):
        q4mi.use_torch_stream()
        layer_call()
    q4mi.use_torch_stream()
    for i, xi in enumerate(xs):
        x.copy_(torch.from_numpy(xi).cuda())
        y.zero_()
        torch.cuda.synchronize()
        gr.replay()
        got = host(y)
        assert np.array_equal(got.view(np.uint32), eager[i].view(np.uint32)), i
