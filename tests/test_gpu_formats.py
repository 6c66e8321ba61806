"""GPU parity for the weight formats beside IQ3_S / Q8_0 (IQ4_NL, Q2_0,
IQ2_S, Q6_K; IQ2_XXS, IQ2_XS, IQ3_XXS, IQ4_XS as decode / window gate/up),
through the C ABI, against the C oracle (whose decoders and
int8 dots are pinned bit for bit against the reference's CPU code in
tests/test_oracle_formats.py).

Bars: int32 group sums bit-exact; fp32 outputs max rel error <= 1e-3."""
import ctypes

import numpy as np
import pytest

from conftest import rel_err

import oracle as om
import q4mi
from q4mi import synth

pytestmark = pytest.mark.gpu
T_IQ3_S, T_Q8_0 = q4mi.T_IQ3_S, q4mi.T_Q8_0
T_Q6_K, T_IQ4_NL, T_IQ2_S, T_Q2_0 = 14, 20, 22, 42
T_IQ2_XXS, T_IQ2_XS, T_IQ3_XXS, T_IQ4_XS = 16, 17, 18, 23
IQXX = [T_IQ2_XXS, T_IQ2_XS, T_IQ3_XXS, T_IQ4_XS]
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


def empty(shape, dtype):
    import torch
    return torch.empty(shape, dtype=dtype, device="cuda")


@pytest.mark.parametrize("ty", [T_IQ4_NL, T_Q2_0, T_IQ2_S, T_Q6_K])
@pytest.mark.parametrize("K,rows,nt", [(512, 131, 1), (2048, 300, 3), (4096, 64, 8)])
def test_mmvq_formats_sums_and_y(gpu, oracle, ty, K, rows, nt):
    import torch
    rng = np.random.default_rng(ty * 1000 + K + nt)
    w = synth.matrix(rng, ty, rows, K)
    x = rng.standard_normal((nt, K)).astype(np.float32)
    qs = np.stack([oracle.quant8(x[t])[0] for t in range(nt)])
    ds = np.stack([oracle.quant8(x[t])[1] for t in range(nt)])
    y = empty((nt, rows), torch.float32)
    s = empty((nt, rows, K // 32), torch.int32)
    q4mi.check(gpu.q4mi_mmvq(ty, q4mi.ptr(dev(w)), rows, K, q4mi.ptr(dev(qs)), q4mi.ptr(dev(ds)),
                             nt, q4mi.ptr(y), 1.0, q4mi.ptr(s)), "q4mi_mmvq")
    sg = host(s)
    rb = om.row_bytes(ty, K)
    for t in range(nt):
        for r in range(0, rows, 5):
            assert np.array_equal(sg[t, r], oracle.group_sums(ty, w[r * rb:(r + 1) * rb], K,
                                                              qs[t])), (t, r)
    assert rel_err(host(y), oracle.dot8_rows(ty, w, rows, K, x)) <= TOL


@pytest.mark.parametrize("n", [1, 4])
def test_q6k_lm_head(gpu, oracle, n):
    """A Q6_K LM head (the reference's wgv_q6_k_k case) through q4_mmvq_n:
    40000 x 2048, fp32 x quantized by the library."""
    import torch
    rows, K = 40000, 2048
    rng = np.random.default_rng(600 + n)
    w = synth.matrix(rng, T_Q6_K, rows, K)
    x = rng.standard_normal((n, K)).astype(np.float32)
    y = empty((n, rows), torch.float32)
    gpu.q4_mmvq_warm()
    q4mi.check(gpu.q4_mmvq_n(T_Q6_K, q4mi.ptr(dev(w)), rows, K, q4mi.ptr(dev(x)), q4mi.ptr(y),
                             1.0, n), "q4_mmvq_n")
    assert rel_err(host(y), oracle.dot8_rows(T_Q6_K, w, rows, K, x)) <= TOL


def packed_experts(rng, E, H, F, tg, td):
    g = synth.matrix(rng, tg, E * F, H)
    u = synth.matrix(rng, tg, E * F, H)
    d = synth.matrix(rng, td, E * H, F)
    gs, ds = F * om.row_bytes(tg, H), H * om.row_bytes(td, F)
    arena = np.concatenate([np.concatenate([g[e * gs:(e + 1) * gs], u[e * gs:(e + 1) * gs],
                                            d[e * ds:(e + 1) * ds]]) for e in range(E)])
    return arena, 2 * gs + ds, 0, gs, 2 * gs


@pytest.mark.parametrize("tg,td", [(T_IQ3_S, T_IQ4_NL), (T_IQ3_S, T_Q2_0), (T_IQ2_S, T_IQ4_NL),
                                   (T_IQ2_S, T_Q2_0), (T_IQ2_S, T_IQ2_S), (T_Q8_0, T_IQ2_S)])
@pytest.mark.parametrize("n_tok", [1, 4])
def test_moe_layer_formats(gpu, oracle, tg, td, n_tok):
    """Decode (1 token, host list) and the 4-token verify window over
    layers mixing the reference models' formats: IQ2_S / IQ3_S / Q8_0
    gate/up with IQ4_NL / Q2_0 / IQ2_S down (hidden 2048, n_ff 512)."""
    H, F, E = 2048, 512, 24
    rng = np.random.default_rng(tg * 100 + td + n_tok)
    arena, stride, og, ou, od = packed_experts(rng, E, H, F, tg, td)
    d_arena = dev(arena)
    x = rng.standard_normal((n_tok, H)).astype(np.float32)
    ids = np.stack([rng.choice(E, 9, replace=False) for _ in range(n_tok)]).astype(np.int32)
    w = rng.random((n_tok, 9)).astype(np.float32)
    yo = oracle.moe_tokens(H, F, tg, td, arena, stride, x, ids, w)
    P = q4mi.ptr
    if n_tok == 1:
        y = dev(np.zeros(H, np.float32))
        i0, w0 = np.ascontiguousarray(ids[0]), np.ascontiguousarray(w[0])
        q4mi.check(gpu.q4_hip_moe_exec(P(d_arena), stride, i0.ctypes.data_as(ctypes.c_void_p),
                                       w0.ctypes.data_as(ctypes.c_void_p), 9, tg, og, tg, ou, td,
                                       od, P(dev(x[0])), None, None, None, P(y), F, H, H),
                   "q4_hip_moe_exec")
        assert rel_err(host(y), yo[0]) <= TOL
        return
    es = np.full((n_tok, 64), -1, np.int32)
    ew = np.zeros((n_tok, 64), np.float32)
    es[:, :9], ew[:, :9] = ids, w
    assert gpu.q4_hip_moe_win_ok(tg, tg, td, H, F, n_tok)
    y = dev(np.zeros((n_tok, H), np.float32))
    q4mi.check(gpu.q4_hip_moe_exec_win(P(d_arena), stride, P(dev(es)), P(dev(ew)),
                                       P(dev(np.full(n_tok, 9, np.int32))), n_tok, tg, og, tg, ou,
                                       td, od, P(dev(x)), None, P(y), F, H, H), "exec_win")
    assert rel_err(host(y), yo) <= TOL


def h_tie_margin(h):
    """Smallest distance of h*127/amax (per 32-value group) from a q8
    rounding boundary."""
    g = np.asarray(h, np.float64).reshape(-1, 32)
    v = g * 127.0 / np.maximum(np.abs(g).max(1, keepdims=True), 1e-30)
    return float(np.abs(np.abs(v - np.floor(v)) - 0.5).min())


def check_tokens(oracle, y, yo, h, ids, w, arena, stride, od, td, H, F):
    """Per token: a token whose oracle h is at least 2e-5 from every q8
    rounding tie must match to TOL (a 1e-7 relative change of h, the size of
    fp32 sum-order differences, moves h*127/amax by at most ~1.3e-5).  A token
    with h values nearer a tie must match to TOL the oracle's layer with those
    codes rounded either way: the down projection is recomputed from the
    oracle's own q8(h) codes (or_dot8q_rows) with every subset of the near-tie
    codes moved to the other neighbour.  Returns the number of tokens on a
    tie."""
    rd = om.row_bytes(td, F)
    k = ids.shape[1]
    ties = 0
    for t in range(ids.shape[0]):
        ht = h[t * k:(t + 1) * k]
        if min(h_tie_margin(hj) for hj in ht) >= 2e-5:
            assert rel_err(y[t], yo[t]) <= TOL, t
            continue
        ties += 1
        qd = [oracle.quant8(ht[j].astype(np.float32)) for j in range(k)]
        near = []
        for j in range(k):
            g = ht[j].astype(np.float64).reshape(-1, 32)
            v = (g * 127.0 / np.maximum(np.abs(g).max(1, keepdims=True), 1e-30)).ravel()
            for i in np.nonzero(np.abs(np.abs(v - np.floor(v)) - 0.5) < 2e-5)[0]:
                q = int(qd[j][0][i])
                near.append((j, int(i), q + 1 if v[i] > q else q - 1))
        assert 0 < len(near) <= 4, (t, len(near))
        best = rel_err(y[t], yo[t])
        for mask in range(1, 1 << len(near)):
            qs = [qd[j][0].copy() for j in range(k)]
            for b, (j, i, alt) in enumerate(near):
                if (mask >> b) & 1:
                    qs[j][i] = alt
            ya = np.zeros(H, np.float32)
            for j, e in enumerate(ids[t]):
                wd = arena[e * stride + od:e * stride + od + H * rd]
                ya += w[t, j] * oracle.dot8q_rows(td, wd, H, F, qs[j][None], qd[j][1][None])[0]
            best = min(best, rel_err(y[t], ya))
        assert best <= TOL, (t, best)
    return ties


@pytest.mark.parametrize("tg", IQXX)
@pytest.mark.parametrize("td", [T_IQ4_NL, T_IQ3_S])
@pytest.mark.parametrize("n_tok", [1, 4, 8])
def test_moe_layer_iq_gate_up(gpu, oracle, tg, td, n_tok):
    """The reference window's other gate/up formats (IQ2_XXS, IQ2_XS,
    IQ3_XXS, IQ4_XS; win_iq_bb, src/q4_rocm.cu:7333-7343) through the decode
    layer (1 token, host list) and the 2..8-token window, against the
    oracle (whose window layer matches the reference's q4_cpuex_dispatch_win
    for these formats), token by token with the q8(h) tie rule of
    check_tokens."""
    H, F, E = 2048, 512, 24
    rng = np.random.default_rng(tg * 1000 + td * 10 + n_tok)
    arena, stride, og, ou, od = packed_experts(rng, E, H, F, tg, td)
    d_arena = dev(arena)
    x = rng.standard_normal((n_tok, H)).astype(np.float32)
    k = 9 if n_tok <= 4 else 7   # n_tok * k <= 64, the window's entry bound
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
    w = rng.random((n_tok, k)).astype(np.float32)
    yo, h = oracle.moe_tokens(H, F, tg, td, arena, stride, x, ids, w, want_h=True)
    P = q4mi.ptr
    if n_tok == 1:
        y = dev(np.zeros(H, np.float32))
        i0, w0 = np.ascontiguousarray(ids[0]), np.ascontiguousarray(w[0])
        q4mi.check(gpu.q4_hip_moe_exec(P(d_arena), stride, i0.ctypes.data_as(ctypes.c_void_p),
                                       w0.ctypes.data_as(ctypes.c_void_p), k, tg, og, tg, ou, td,
                                       od, P(dev(x[0])), None, None, None, P(y), F, H, H),
                   "q4_hip_moe_exec")
        got = host(y)[None]
    else:
        es = np.full((n_tok, 64), -1, np.int32)
        ew = np.zeros((n_tok, 64), np.float32)
        es[:, :k], ew[:, :k] = ids, w
        assert gpu.q4_hip_moe_win_ok(tg, tg, td, H, F, n_tok)
        y = dev(np.zeros((n_tok, H), np.float32))
        q4mi.check(gpu.q4_hip_moe_exec_win(P(d_arena), stride, P(dev(es)), P(dev(ew)),
                                           P(dev(np.full(n_tok, k, np.int32))), n_tok, tg, og, tg,
                                           ou, td, od, P(dev(x)), None, P(y), F, H, H), "exec_win")
        got = host(y)
    ties = check_tokens(oracle, got, yo, h, ids, w, arena, stride, od, td, H, F)
    assert ties <= max(1, n_tok // 2)


def test_format_coverage_rules(gpu):
    """IQ4_NL and Q2_0 are down-projection types here (gate/up rejected);
    IQ2_XXS, IQ2_XS, IQ3_XXS and IQ4_XS gate/up types (down rejected), as in
    the reference's window; Q6_K is an LM-head type (not in the routed
    layer)."""
    assert gpu.q4_hip_moe_win_ok(T_IQ2_S, T_IQ2_S, T_Q2_0, 2048, 512, 4)
    assert not gpu.q4_hip_moe_win_ok(T_IQ4_NL, T_IQ4_NL, T_IQ3_S, 2048, 512, 4)
    assert not gpu.q4_hip_moe_win_ok(T_IQ3_S, T_IQ3_S, T_Q6_K, 2048, 512, 4)
    for t in IQXX:
        assert gpu.q4_hip_moe_win_ok(t, t, T_IQ4_NL, 2048, 512, 4)
        assert not gpu.q4_hip_moe_win_ok(T_IQ3_S, T_IQ3_S, t, 2048, 512, 4)
    # IQ2_XXS rows must be whole dwords: 66 B per 256 values -> K % 512
    assert not gpu.q4_hip_moe_win_ok(T_IQ2_XXS, T_IQ2_XXS, T_IQ4_NL, 256 * 3, 512, 4)


def mmq_q8(L, x, rows_idx, K):
    import torch
    xq = torch.zeros(int(L.q4_mmq_q8_bytes(len(rows_idx), K)), dtype=torch.uint8, device="cuda")
    q4mi.check(L.q4_mmq_quantize(q4mi.ptr(dev(x)), q4mi.ptr(dev(np.asarray(rows_idx, np.int32))),
                                 q4mi.ptr(xq), 21, K, len(rows_idx)), "q4_mmq_quantize")
    return xq


@pytest.mark.parametrize("ty,N,K", [(T_IQ4_NL, 2048, 512), (T_Q2_0, 2048, 512),
                                    (T_IQ2_S, 1024, 2048), (T_IQ2_S, 2048, 512),
                                    (T_IQ4_NL, 256, 2048)])
def test_mmq_formats_mul_id(gpu, oracle, ty, N, K):
    """The prefill MMQ over the other formats, ragged experts (empty, tile
    edges, single rows), against the oracle's int8 row dot."""
    import torch
    rng = np.random.default_rng(ty * 7 + N + K)
    per = [70, 0, 1, 129, 5, 33]
    E = len(per)
    rb = om.row_bytes(ty, K)
    W = synth.matrix(rng, ty, E * N, K)
    T = 200
    x = rng.standard_normal((T, K)).astype(np.float32)
    a_tok = np.concatenate([rng.integers(0, T, n) for n in per]).astype(np.int32)
    bounds = np.concatenate([[0], np.cumsum(per)]).astype(np.int32)
    total = int(bounds[-1])
    assert gpu.q4_mmq_supported(ty, N)
    xq = mmq_q8(gpu, x, a_tok, K)
    dst = torch.zeros((total, N), dtype=torch.float32, device="cuda")
    q4mi.check(gpu.q4_mmq_mul_id(q4mi.ptr(dev(W)), ty, N, K, N * rb, E, q4mi.ptr(xq),
                                 q4mi.ptr(dev(bounds)), 0, total, q4mi.ptr(dst), N),
               "q4_mmq_mul_id")
    d = host(dst)
    for e in range(E):
        if per[e] == 0:
            continue
        rows = a_tok[bounds[e]:bounds[e + 1]]
        ref = oracle.dot8_rows(ty, W[e * N * rb:(e + 1) * N * rb], N, K, x[rows])
        assert rel_err(d[bounds[e]:bounds[e + 1]], ref) <= TOL, e


def test_mmq_iq2s_gate_up_fused(gpu, oracle):
    """Fused gate/up (SwiGLU + q8(h)) over IQ2_S experts: the q8(h) codes
    against or_quant8 of the oracle's h (at most 1e-4 of them differ: h
    rounding near a q8 boundary)."""
    import torch
    rng = np.random.default_rng(91)
    H, F = 2048, 512
    per = [40, 3, 0, 130]
    E = len(per)
    rb = om.row_bytes(T_IQ2_S, H)
    W = synth.matrix(rng, T_IQ2_S, E * 2 * F, H)      # per expert: gate rows then up rows
    T = 150
    x = rng.standard_normal((T, H)).astype(np.float32)
    a_tok = np.concatenate([rng.integers(0, T, n) for n in per]).astype(np.int32)
    bounds = np.concatenate([[0], np.cumsum(per)]).astype(np.int32)
    rows = int(bounds[-1])
    xq = mmq_q8(gpu, x, np.arange(T), H)
    hq = torch.zeros(int(gpu.q4_mmq_q8_bytes(rows, F)), dtype=torch.uint8, device="cuda")
    q4mi.check(gpu.q4mi_mmq_gate_up(q4mi.ptr(dev(W)), T_IQ2_S, F, H, 2 * F * rb, E, q4mi.ptr(xq),
                                    T, q4mi.ptr(dev(a_tok)), q4mi.ptr(dev(bounds)), rows,
                                    q4mi.ptr(hq)), "gate_up")
    hb = host(hq)
    codes = hb[:rows * F * 2].view(np.float16).reshape(rows, F).astype(np.int32)
    diff = 0
    for e in range(E):
        if not per[e]:
            continue
        Wg = W[e * 2 * F * rb:(e + 1) * 2 * F * rb]
        gu = oracle.dot8_rows(T_IQ2_S, Wg, 2 * F, H, x[a_tok[bounds[e]:bounds[e + 1]]])
        h = (gu[:, :F] / (1 + np.exp(-gu[:, :F].astype(np.float64))) * gu[:, F:]).astype(np.float32)
        for i in range(per[e]):
            q, _, _ = oracle.quant8(h[i])
            diff += int(np.count_nonzero(q.astype(np.int32) != codes[bounds[e] + i]))
    assert diff <= 1e-3 * rows * F, diff


# The reference model's shapes: hidden 2560 (80 q8 groups per row) and
# expert intermediate 640 (20 groups), rows the power-of-two layouts do not
# divide (16 lanes x 5 groups, 4 lanes x 5 groups).
@pytest.mark.parametrize("ty,K", [(T_IQ3_S, 2560), (T_Q8_0, 2560), (T_IQ2_S, 2560),
                                  (T_IQ4_NL, 640), (T_Q2_0, 640), (T_Q8_0, 640)])
@pytest.mark.parametrize("nt", [1, 4])
def test_mmvq_reference_model_shapes(gpu, oracle, ty, K, nt):
    """q4mi_mmvq (int32 group sums bit-exact) and q4_mmvq_n (y <= TOL, the
    library quantizing fp32 x) at K = 2560 and 640."""
    import torch
    rows = 300
    rng = np.random.default_rng(ty * 100 + K + nt)
    w = synth.matrix(rng, ty, rows, K)
    x = rng.standard_normal((nt, K)).astype(np.float32)
    qs = np.stack([oracle.quant8(x[t])[0] for t in range(nt)])
    ds = np.stack([oracle.quant8(x[t])[1] for t in range(nt)])
    y = empty((nt, rows), torch.float32)
    s = empty((nt, rows, K // 32), torch.int32)
    q4mi.check(gpu.q4mi_mmvq(ty, q4mi.ptr(dev(w)), rows, K, q4mi.ptr(dev(qs)), q4mi.ptr(dev(ds)),
                             nt, q4mi.ptr(y), 1.0, q4mi.ptr(s)), "q4mi_mmvq")
    sg = host(s)
    rb = om.row_bytes(ty, K)
    for t in range(nt):
        for r in range(0, rows, 7):
            assert np.array_equal(sg[t, r], oracle.group_sums(ty, w[r * rb:(r + 1) * rb], K,
                                                              qs[t])), (t, r)
    y2 = empty((nt, rows), torch.float32)
    gpu.q4_mmvq_warm()
    q4mi.check(gpu.q4_mmvq_n(ty, q4mi.ptr(dev(w)), rows, K, q4mi.ptr(dev(x)), q4mi.ptr(y2), 1.0,
                             nt), "q4_mmvq_n")
    assert rel_err(host(y2), oracle.dot8_rows(ty, w, rows, K, x)) <= TOL


@pytest.mark.parametrize("tg", [T_IQ3_S, T_IQ2_S, T_IQ3_XXS, T_IQ2_XXS, T_IQ4_XS])
@pytest.mark.parametrize("n_tok", [1, 4])
def test_moe_layer_reference_model_shapes(gpu, oracle, tg, n_tok):
    """Decode (1 token) and the 4-token window at the reference model's
    shapes (hidden 2560, expert intermediate 640) with its window formats
    (gate/up IQ2_S / IQ3_XXS / IQ3_S and the others, IQ4_NL down), against
    the oracle with the q8(h) tie rule of check_tokens."""
    H, F, E, td = 2560, 640, 20, T_IQ4_NL
    rng = np.random.default_rng(tg * 7 + n_tok)
    arena, stride, og, ou, od = packed_experts(rng, E, H, F, tg, td)
    d_arena = dev(arena)
    x = rng.standard_normal((n_tok, H)).astype(np.float32)
    k = 11
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
    w = rng.random((n_tok, k)).astype(np.float32)
    yo, h = oracle.moe_tokens(H, F, tg, td, arena, stride, x, ids, w, want_h=True)
    P = q4mi.ptr
    if n_tok == 1:
        y = dev(np.zeros(H, np.float32))
        i0, w0 = np.ascontiguousarray(ids[0]), np.ascontiguousarray(w[0])
        q4mi.check(gpu.q4_hip_moe_exec(P(d_arena), stride, i0.ctypes.data_as(ctypes.c_void_p),
                                       w0.ctypes.data_as(ctypes.c_void_p), k, tg, og, tg, ou, td,
                                       od, P(dev(x[0])), None, None, None, P(y), F, H, H),
                   "q4_hip_moe_exec")
        got = host(y)[None]
    else:
        es = np.full((n_tok, 64), -1, np.int32)
        ew = np.zeros((n_tok, 64), np.float32)
        es[:, :k], ew[:, :k] = ids, w
        assert gpu.q4_hip_moe_win_ok(tg, tg, td, H, F, n_tok)
        y = dev(np.zeros((n_tok, H), np.float32))
        q4mi.check(gpu.q4_hip_moe_exec_win(P(d_arena), stride, P(dev(es)), P(dev(ew)),
                                           P(dev(np.full(n_tok, k, np.int32))), n_tok, tg, og, tg,
                                           ou, td, od, P(dev(x)), None, P(y), F, H, H), "exec_win")
        got = host(y)
    ties = check_tokens(oracle, got, yo, h, ids, w, arena, stride, od, td, H, F)
    assert ties <= max(1, n_tok // 2)
