"""GPU parity for the prefill MMQ path (q4_mmq_quantize / q4_mmq_mul_id /
q4_mmq_swiglu / q4_hip_expert_reduce and the routing pack), against the C
oracle.  fp32 outputs: max relative error <= 1e-3."""
import numpy as np
import pytest

from conftest import rel_err

import oracle as om
import q4mi
from q4mi import synth

pytestmark = pytest.mark.gpu
T_IQ3_S, T_Q8_0 = q4mi.T_IQ3_S, q4mi.T_Q8_0
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


def mmq_quant(L, x, ids, cols, rows):
    import torch
    xq = zeros(int(L.q4_mmq_q8_bytes(rows, cols)), torch.uint8)
    q4mi.check(L.q4_mmq_quantize(q4mi.ptr(x), q4mi.ptr(ids), q4mi.ptr(xq), T_IQ3_S, cols, rows),
               "q4_mmq_quantize")
    return xq


def mul_id(L, w, ty, N, K, estride, n_exp, xq, bounds, total, ld):
    dst = zeros((total, ld))
    q4mi.check(L.q4_mmq_mul_id(q4mi.ptr(w), ty, N, K, estride, n_exp, q4mi.ptr(xq),
                               q4mi.ptr(bounds), 0, total, q4mi.ptr(dst), ld), "q4_mmq_mul_id")
    return dst


@pytest.mark.parametrize("ty,N,K", [(T_IQ3_S, 1024, 2048), (T_IQ3_S, 2048, 512),
                                    (T_Q8_0, 256, 2048), (T_Q8_0, 128, 512)])
def test_mul_id_ragged(gpu, oracle, ty, N, K):
    rng = np.random.default_rng(N + K + ty)
    per = [100, 0, 1, 40, 128, 129, 3, 257]       # ragged, incl. empty and tile edges
    E = len(per)
    rb = om.row_bytes(ty, K)
    W = synth.matrix(rng, ty, E * N, K)
    estride = N * rb
    T = 300
    x = rng.standard_normal((T, K)).astype(np.float32)
    a_tok = np.concatenate([rng.integers(0, T, n) for n in per]).astype(np.int32)
    bounds = np.concatenate([[0], np.cumsum(per)]).astype(np.int32)
    total = int(bounds[-1])
    dx, dids = dev(x), dev(a_tok)
    xq = mmq_quant(gpu, dx, dids, K, total)
    dW, dbounds = dev(W), dev(bounds)
    dst = host(mul_id(gpu, dW, ty, N, K, estride, E, xq, dbounds, total, N))
    for e in range(E):
        if per[e] == 0:
            continue
        rows = a_tok[bounds[e]:bounds[e + 1]]
        ref = oracle.dot8_rows(ty, W[e * estride:(e + 1) * estride], N, K, x[rows])
        assert rel_err(dst[bounds[e]:bounds[e + 1]], ref) <= TOL, e


@pytest.mark.parametrize("ty", [T_IQ3_S, T_Q8_0])
def test_mul_id_misaligned_experts(gpu, oracle, ty):
    """Expert bases 2 bytes into a dword (stride = matrix bytes + 2): every
    superblock then starts at the other in-dword offset."""
    rng = np.random.default_rng(17 + ty)
    N, K, E = 256, 1024, 3
    per = [37, 130, 5]
    rb = om.row_bytes(ty, K)
    W = synth.matrix(rng, ty, E * N, K)
    estride = N * rb + 2
    buf = np.zeros(E * estride + 8, np.uint8)
    for e in range(E):
        buf[e * estride:e * estride + N * rb] = W[e * N * rb:(e + 1) * N * rb]
    T = 200
    x = rng.standard_normal((T, K)).astype(np.float32)
    a_tok = np.concatenate([rng.integers(0, T, n) for n in per]).astype(np.int32)
    bounds = np.concatenate([[0], np.cumsum(per)]).astype(np.int32)
    total = int(bounds[-1])
    xq = mmq_quant(gpu, dev(x), dev(a_tok), K, total)
    dst = host(mul_id(gpu, dev(buf), ty, N, K, estride, E, xq, dev(bounds), total, N))
    for e in range(E):
        rows = a_tok[bounds[e]:bounds[e + 1]]
        ref = oracle.dot8_rows(ty, W[e * N * rb:(e + 1) * N * rb], N, K, x[rows])
        assert rel_err(dst[bounds[e]:bounds[e + 1]], ref) <= TOL, e


def test_mmq_group_sums_exact(gpu, oracle):
    """With d_w = 1 and activations whose q8 scale is exactly 1, the MMQ
    output of each 512-value row equals the oracle's exact integer sums."""
    rng = np.random.default_rng(77)
    N, K = 128, 512
    rb = om.row_bytes(T_IQ3_S, K)
    W = synth.matrix(rng, T_IQ3_S, N, K)
    Wb = W.reshape(-1, 110)
    Wb[:, 0:2] = np.array([1.0], np.float16).view(np.uint8)
    x = rng.integers(-127, 128, (3, K)).astype(np.float32)
    x[:, ::32] = 127.0                               # amax 127 -> d = 1, q = x exactly
    bounds = np.array([0, 3], np.int32)
    dx, dW, dbounds = dev(x), dev(W), dev(bounds)
    xq = mmq_quant(gpu, dx, None, K, 3)
    dst = host(mul_id(gpu, dW, T_IQ3_S, N, K, N * rb, 1, xq, dbounds, 3, N))
    for t in range(3):
        q, d, _ = oracle.quant8(x[t])
        assert np.all(d == 1.0) and np.array_equal(q.astype(np.float32), x[t])
        for n in range(N):
            s = oracle.group_sums(T_IQ3_S, W[n * rb:(n + 1) * rb], K, q)
            assert dst[t, n] == float(s.sum())


def test_prefill_layer_config3(gpu, oracle):
    """BASELINE config 3-prefill: 2048 tokens, Zipf-skewed top-10 over 512
    experts + the shared expert; route -> stable pack -> quantize ->
    MMQ gate/up -> SwiGLU -> quantize -> MMQ down -> weighted reduce.
    Checked on a sample of tokens against the oracle's composition."""
    import torch
    E, H, F, T, k = 512, 2048, 512, 2048, 10
    rng = np.random.default_rng(3)
    arena = synth.expert_arena(rng, E + 1, H, F)
    stride, og, ou, od = synth.expert_stride(H, F)
    x = rng.standard_normal((T, H)).astype(np.float32)
    lg = synth.logits(rng, T, E, zipf=True)
    d_arena, dx, dlg = dev(arena), dev(x), dev(lg)
    L = gpu
    ids, wts = zeros((T, k), torch.int32), zeros((T, k))
    q4mi.check(L.q4_hip_route_pf(q4mi.ptr(dlg), q4mi.ptr(ids), q4mi.ptr(wts), T, E, k), "route")
    a_tok, rsrc, rw = zeros(T * k, torch.int32), zeros(T * k, torch.int32), zeros(T * k)
    stg, stgn, ek = zeros(512, torch.int32), zeros(1, torch.int32), zeros(512, torch.int32)
    bounds = zeros(E + 1, torch.int32)
    q4mi.check(L.q4mi_assign(q4mi.ptr(ids), q4mi.ptr(wts), q4mi.ptr(a_tok), q4mi.ptr(rsrc),
                             q4mi.ptr(rw), q4mi.ptr(stg), q4mi.ptr(stgn), q4mi.ptr(ek),
                             q4mi.ptr(bounds), T, k, E, T), "assign")
    rows = T * k
    # routed experts: gate|up are contiguous (gate rows then up rows) = one
    # 2F x H matrix per expert at arena + e*stride.  Reference sequence:
    # quantize(x, a_tok) -> mul_id -> swiglu -> quantize(h); fast path:
    # quantize(x) per token -> fused gate/up (gathered through a_tok).
    xq = mmq_quant(L, dx, a_tok, H, rows)
    gu = mul_id(L, d_arena, T_IQ3_S, 2 * F, H, stride, E, xq, bounds, rows, 2 * F)
    h = zeros((rows, F))
    q4mi.check(L.q4_mmq_swiglu(q4mi.ptr(gu), q4mi.ptr(h), rows, F), "swiglu")
    hq_ref_path = mmq_quant(L, h, None, F, rows)
    xq_tok = mmq_quant(L, dx, None, H, T)
    hq = zeros(int(L.q4_mmq_q8_bytes(rows, F)), torch.uint8)
    q4mi.check(L.q4mi_mmq_gate_up(q4mi.ptr(d_arena), T_IQ3_S, F, H, stride, E, q4mi.ptr(xq_tok),
                                  T, q4mi.ptr(a_tok), q4mi.ptr(bounds), rows, q4mi.ptr(hq)),
               "gate_up")
    # both paths give the same q8(h) codes up to 1 (fp32 rounding of h)
    ca = host(hq)[:rows * F * 2].view(np.float16).astype(np.float32)
    cb = host(hq_ref_path)[:rows * F * 2].view(np.float16).astype(np.float32)
    assert np.abs(ca - cb).max() <= 1
    dn_w = d_arena[od:]
    pd = mul_id(L, dn_w, T_IQ3_S, H, F, stride, E, hq, bounds, rows, H)
    y = zeros((T, H))
    q4mi.check(L.q4_hip_expert_reduce(q4mi.ptr(y), q4mi.ptr(pd), q4mi.ptr(rsrc), q4mi.ptr(rw),
                                      T, k, H), "reduce")
    # shared expert: one "expert" over all tokens, weight 1
    sb = dev(np.array([0, T], np.int32))
    sxq = mmq_quant(L, dx, None, H, T)
    sgu = mul_id(L, d_arena[E * stride:], T_IQ3_S, 2 * F, H, stride, 1, sxq, sb, T, 2 * F)
    sh = zeros((T, F))
    q4mi.check(L.q4_mmq_swiglu(q4mi.ptr(sgu), q4mi.ptr(sh), T, F), "swiglu")
    shq = mmq_quant(L, sh, None, F, T)
    spd = mul_id(L, d_arena[E * stride + od:], T_IQ3_S, H, F, stride, 1, shq, sb, T, H)
    ones = dev(np.ones(T, np.float32))
    iden = dev(np.arange(T, dtype=np.int32))
    q4mi.check(L.q4_hip_expert_reduce(q4mi.ptr(y), q4mi.ptr(spd), q4mi.ptr(iden), q4mi.ptr(ones),
                                      T, 1, H), "reduce shared")
    yg = host(y)
    # routing and pack are bit-exact against the oracle
    oid, ow = oracle.softmax_topk(lg, k)
    assert np.array_equal(host(ids), oid)
    pk = oracle.pack(oid, ow, E, T)
    assert np.array_equal(host(a_tok), pk["a_tok"][:rows])
    assert np.array_equal(host(bounds), pk["bounds"])
    # sampled tokens through the oracle (routed picks + shared, weight 1)
    samp = np.concatenate([[0, T - 1], rng.choice(np.arange(1, T - 1), 22, replace=False)])
    sid = np.concatenate([oid[samp], np.full((len(samp), 1), E, np.int32)], 1)
    sw = np.concatenate([ow[samp], np.ones((len(samp), 1), np.float32)], 1)
    yo = oracle.moe_tokens(H, F, T_IQ3_S, T_IQ3_S, arena, stride, x[samp], sid, sw, mode=1)
    assert rel_err(yg[samp], yo) <= TOL


def test_gate_up_fused_and_rows(gpu, oracle):
    """q4mi_mmq_gate_up (SwiGLU + q8(h) epilogue) and q4mi_mmq_mul_id_rows
    (activation rows gathered through a_tok) against the oracle."""
    import torch
    rng = np.random.default_rng(31)
    H, F = 2048, 512
    per = [130, 0, 7, 64, 200]
    E = len(per)
    arena = synth.expert_arena(rng, E, H, F)
    stride, og, ou, od = synth.expert_stride(H, F)
    T = 256
    x = rng.standard_normal((T, H)).astype(np.float32)
    a_tok = np.concatenate([rng.integers(0, T, n) for n in per]).astype(np.int32)
    bounds = np.concatenate([[0], np.cumsum(per)]).astype(np.int32)
    rows = int(bounds[-1])
    d_arena, dx, dtok, dbounds = dev(arena), dev(x), dev(a_tok), dev(bounds)
    xq = mmq_quant(gpu, dx, None, H, T)              # one q8 row per token
    hq = zeros(int(gpu.q4_mmq_q8_bytes(rows, F)), torch.uint8)
    q4mi.check(gpu.q4mi_mmq_gate_up(q4mi.ptr(d_arena), T_IQ3_S, F, H, stride, E, q4mi.ptr(xq), T,
                                    q4mi.ptr(dtok), q4mi.ptr(dbounds), rows, q4mi.ptr(hq)),
               "gate_up")
    gu = zeros((rows, 2 * F))
    q4mi.check(gpu.q4mi_mmq_mul_id_rows(q4mi.ptr(d_arena), T_IQ3_S, 2 * F, H, stride, E,
                                        q4mi.ptr(xq), T, q4mi.ptr(dtok), q4mi.ptr(dbounds), rows,
                                        q4mi.ptr(gu), 2 * F), "mul_id_rows")
    hqh = host(hq)
    codes = hqh[:rows * F * 2].view(np.float16).reshape(rows, F).astype(np.float32)
    hd = hqh[rows * F * 2: rows * F * 2 + rows * (F // 32) * 4].view(np.float32).reshape(rows, -1)
    guh = host(gu)
    for e in range(E):
        if per[e] == 0:
            continue
        W = arena[e * stride:(e + 1) * stride]
        toks = a_tok[bounds[e]:bounds[e + 1]]
        ref_gu = oracle.dot8_rows(T_IQ3_S, W[:2 * F * 880], 2 * F, H, x[toks])
        got = guh[bounds[e]:bounds[e + 1]]
        assert rel_err(got, ref_gu) <= TOL
        g, u = ref_gu[:, :F], ref_gu[:, F:]
        h = g / (1 + np.exp(-g)) * u
        hdeq = codes[bounds[e]:bounds[e + 1]] * np.repeat(hd[bounds[e]:bounds[e + 1]], 32, 1)
        # q8(h): codes times scale track h to half a step (plus the fp32 noise of h)
        step = np.repeat(hd[bounds[e]:bounds[e + 1]], 32, 1)
        assert np.all(np.abs(hdeq - h) <= 0.5 * step + 2e-3 * np.abs(h).max())
        # and they are exactly the q8 codes of the kernel's own h (rows of
        # h recomputed from the plain gate/up output agree to 1 code)
        hg = got[:, :F] / (1 + np.exp(-got[:, :F])) * got[:, F:]
        for r in range(0, len(toks), 17):
            q, d, _ = oracle.quant8(hg[r].astype(np.float32))
            assert np.abs(q.astype(np.float32) - codes[bounds[e] + r]).max() <= 1


def test_shared_expert_in_routed_launch(gpu):
    """The _x entry points (routed experts + a shared expert stored apart,
    appended as expert E over every token) give the separate launches'
    results: q8(h) codes bit-exact, y within fp32 reduction order."""
    import torch
    E, H, F, T, k = 64, 2048, 512, 512, 4
    rng = np.random.default_rng(41)
    arena = synth.expert_arena(rng, E + 1, H, F)
    stride, og, ou, od = synth.expert_stride(H, F)
    x = rng.standard_normal((T, H)).astype(np.float32)
    lg = synth.logits(rng, T, E, zipf=True)
    sw = rng.uniform(0.1, 1.0, T).astype(np.float32)          # per-token shared-expert gate
    L, P, chk = gpu, q4mi.ptr, q4mi.check
    d_routed = dev(arena[:E * stride])
    d_shared = dev(arena[E * stride:(E + 1) * stride].copy())  # its own allocation
    dx, dlg, dsw = dev(x), dev(lg), dev(sw)
    ids, wts = zeros((T, k), torch.int32), zeros((T, k))
    chk(L.q4_hip_route_pf(P(dlg), P(ids), P(wts), T, E, k), "route")
    rows = T * k
    a_tok = zeros(rows + T, torch.int32)
    a_tok[rows:] = torch.arange(T, dtype=torch.int32, device="cuda")
    rsrc, rw = zeros(rows, torch.int32), zeros(rows)
    stg, stgn, ek = zeros(512, torch.int32), zeros(1, torch.int32), zeros(512, torch.int32)
    bounds = zeros(E + 2, torch.int32)
    bounds[E + 1] = rows + T
    chk(L.q4mi_assign(P(ids), P(wts), P(a_tok), P(rsrc), P(rw), P(stg), P(stgn), P(ek),
                      P(bounds), T, k, E, T), "assign")
    xq = mmq_quant(L, dx, None, H, T)
    # separate launches
    hq = zeros(int(L.q4_mmq_q8_bytes(rows, F)), torch.uint8)
    chk(L.q4mi_mmq_gate_up(P(d_routed), T_IQ3_S, F, H, stride, E, P(xq), T, P(a_tok), P(bounds),
                           rows, P(hq)), "gate_up")
    pd = zeros((rows, H))
    chk(L.q4_mmq_mul_id(P(d_routed) + od, T_IQ3_S, H, F, stride, E, P(hq), P(bounds), 0, rows,
                        P(pd), H), "down")
    y1 = zeros((T, H))
    chk(L.q4_hip_expert_reduce(P(y1), P(pd), P(rsrc), P(rw), T, k, H), "reduce")
    sb = dev(np.array([0, T], np.int32))
    hq_s = zeros(int(L.q4_mmq_q8_bytes(T, F)), torch.uint8)
    chk(L.q4mi_mmq_gate_up(P(d_shared), T_IQ3_S, F, H, stride, 1, P(xq), T, None, P(sb), T,
                           P(hq_s)), "gate_up shared")
    pd_s = zeros((T, H))
    chk(L.q4_mmq_mul_id(P(d_shared) + od, T_IQ3_S, H, F, stride, 1, P(hq_s), P(sb), 0, T,
                        P(pd_s), H), "down shared")
    chk(L.q4_hip_expert_reduce(P(y1), P(pd_s), P(dev(np.arange(T, dtype=np.int32))), P(dsw), T,
                               1, H), "reduce shared")
    # one launch each
    hq_x = zeros(int(L.q4_mmq_q8_bytes(rows + T, F)), torch.uint8)
    chk(L.q4mi_mmq_gate_up_x(P(d_routed), P(d_shared), T_IQ3_S, F, H, stride, E, P(xq), T,
                             P(a_tok), P(bounds), rows + T, P(hq_x)), "gate_up_x")
    pd_x = zeros((rows + T, H))
    chk(L.q4mi_mmq_mul_id_x(P(d_routed) + od, P(d_shared) + od, T_IQ3_S, H, F, stride, E,
                            P(hq_x), P(bounds), rows + T, P(pd_x), H), "down_x")
    y2 = zeros((T, H))
    chk(L.q4mi_expert_reduce_x(P(y2), P(pd_x), P(rsrc), P(rw), T, k, H, rows, P(dsw)), "reduce_x")
    # the q8(h) layout: fp16 codes [rows][F] then fp32 scales [rows][F/32]
    def codes(buf, n):
        b = host(buf)
        return (b[:n * F * 2].view(np.float16), b[n * F * 2:n * F * 2 + n * F // 32 * 4].view(np.float32))
    cx, dxs = codes(hq_x, rows + T)
    cr, dr = codes(hq, rows)
    cs, ds = codes(hq_s, T)
    assert np.array_equal(cx[:rows * F], cr) and np.array_equal(dxs[:rows * F // 32], dr)
    assert np.array_equal(cx[rows * F:], cs) and np.array_equal(dxs[rows * F // 32:], ds)
    assert np.array_equal(host(pd_x)[:rows], host(pd)) and np.array_equal(host(pd_x)[rows:], host(pd_s))
    assert rel_err(host(y2), host(y1)) <= 1e-5


def test_prefill_graph_replays(gpu):
    """The fused prefill sequence (route, pack, q8(x), gate/up, down, reduce)
    captured in a HIP graph and replayed over three inputs equals the eager
    calls bit for bit (no memset nodes; every kernel deterministic)."""
    import torch
    E, H, F, T, k = 64, 2048, 512, 256, 6
    rng = np.random.default_rng(51)
    arena = synth.expert_arena(rng, E + 1, H, F)
    stride, og, ou, od = synth.expert_stride(H, F)
    d_arena = dev(arena)
    xs = [rng.standard_normal((T, H)).astype(np.float32) for _ in range(3)]
    lgs = [synth.logits(rng, T, E, zipf=True) for _ in range(3)]
    x, lg = dev(xs[0]), dev(lgs[0])
    i32 = torch.int32
    rows = T * k
    ids, wts = zeros((T, k), i32), zeros((T, k))
    a_tok = zeros(rows + T, i32)
    a_tok[rows:] = torch.arange(T, dtype=i32, device="cuda")
    rsrc, rw = zeros(rows, i32), zeros(rows)
    stg, stgn, ek = zeros(512, i32), zeros(1, i32), zeros(512, i32)
    bounds = zeros(E + 2, i32)
    bounds[E + 1] = rows + T
    xq = zeros(int(gpu.q4_mmq_q8_bytes(T, H)), torch.uint8)
    hq = zeros(int(gpu.q4_mmq_q8_bytes(rows + T, F)), torch.uint8)
    pd = zeros((rows + T, H))
    y = zeros((T, H))
    L, P, chk = gpu, q4mi.ptr, q4mi.check
    A = d_arena.data_ptr()
    S = A + E * stride

    def layer():
        chk(L.q4_hip_route_pf(P(lg), P(ids), P(wts), T, E, k), "route")
        chk(L.q4mi_assign(P(ids), P(wts), P(a_tok), P(rsrc), P(rw), P(stg), P(stgn), P(ek),
                          P(bounds), T, k, E, T), "assign")
        chk(L.q4_mmq_quantize(P(x), None, P(xq), T_IQ3_S, H, T), "q8 x")
        chk(L.q4mi_mmq_gate_up_x(A, S, T_IQ3_S, F, H, stride, E, P(xq), T, P(a_tok),
                                 P(bounds), rows + T, P(hq)), "gate/up")
        chk(L.q4mi_mmq_mul_id_x(A + od, S + od, T_IQ3_S, H, F, stride, E, P(hq), P(bounds),
                                rows + T, P(pd), H), "down")
        chk(L.q4mi_expert_reduce_x(P(y), P(pd), P(rsrc), P(rw), T, k, H, rows, None), "reduce")
    eager = []
    for xi, li in zip(xs, lgs):
        x.copy_(torch.from_numpy(xi).cuda())
        lg.copy_(torch.from_numpy(li).cuda())
        y.zero_()
        layer()
        eager.append(host(y).copy())
    gr = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    with torch.cuda.graph(gr, stream=s):
        q4mi.use_torch_stream()
        layer()
    q4mi.use_torch_stream()
    for i, (xi, li) in enumerate(zip(xs, lgs)):
        x.copy_(torch.from_numpy(xi).cuda())
        lg.copy_(torch.from_numpy(li).cuda())
        y.zero_()
        torch.cuda.synchronize()
        gr.replay()
        assert np.array_equal(host(y).view(np.uint32), eager[i].view(np.uint32)), i
