"""GPU parity at the BASELINE configurations' full shapes, through the C ABI,
against the C oracle:

- config 4: the Q8_0 151936 x 2048 lm-head through q4_mmvq_n, 1 and 4 tokens;
- config 3-prefill: the fused prefill sequence the benchmark times
  (route, q4mi_assign, q8(x), q4mi_mmq_gate_up_x, q4mi_mmq_mul_id_x,
  q4mi_expert_reduce_x, the shared expert riding in the routed launches),
  on 288 sampled tokens including the first and the last;
- the q8(h) codes of the prefill and decode paths, counted against the
  oracle's q8 of its own h;
- the decode layer and window at the wider hidden sizes (4096, 8192) whose
  lane layouts the config shapes do not reach.

Bars: fp32 outputs max rel error <= 1e-3 (|err| / max(|ref|, 1e-3 max|ref|));
routing ids and the pack bit-exact; at most 1e-4 of the q8(h) codes differ
from the oracle's (h is fp32 from differently ordered sums and a hardware
exp in silu, so a value within a few ulp of a q8 rounding boundary may round
the other way; the codes of every group away from a boundary are equal).
"""
import concurrent.futures as cf
import os

import numpy as np
import pytest

from conftest import rel_err

import oracle as om
import q4mi
from q4mi import synth

pytestmark = pytest.mark.gpu
T_IQ3_S, T_Q8_0 = q4mi.T_IQ3_S, q4mi.T_Q8_0
TOL = 1e-3
CODE_DIFF_MAX = 1e-4
WORKERS = min(16, os.cpu_count() or 1)


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


def oracle_tokens(oracle, H, F, arena, stride, x, ids, wts, mode, want_h):
    """or_moe_tokens over token chunks on a thread pool (the C call releases
    the GIL); same results as one call."""
    T = x.shape[0]
    step = max(1, (T + WORKERS - 1) // WORKERS)
    parts = [(i, min(T, i + step)) for i in range(0, T, step)]

    def run(p):
        a, b = p
        return oracle.moe_tokens(H, F, T_IQ3_S, T_IQ3_S, arena, stride, x[a:b], ids[a:b],
                                 wts[a:b], mode=mode, want_h=want_h)
    with cf.ThreadPoolExecutor(len(parts)) as ex:
        res = list(ex.map(run, parts))
    if not want_h:
        return np.concatenate(res)
    return np.concatenate([r[0] for r in res]), np.concatenate([r[1] for r in res])


def code_diff_fraction(oracle, h_ref, codes_got):
    """Fraction of q8 codes of the oracle's h rows (or_quant8, the
    reference's quantizer) that differ from codes_got, and the rows with a
    difference."""
    diff = 0
    rows = np.zeros(h_ref.shape[0], bool)
    for r in range(h_ref.shape[0]):
        q, _, _ = oracle.quant8(h_ref[r])
        n = int(np.count_nonzero(q.astype(np.int32) != codes_got[r].astype(np.int32)))
        diff += n
        rows[r] = n > 0
    return diff / h_ref.size, rows


def down_from_codes(oracle, arena, stride, od, H, F, ids, wts, codes, scales):
    """The oracle's down projection and weighted sum fed with given q8(h)
    codes/scales: y[t] = sum_j wts[t,j] * (down_{ids[t,j]} . codes[t,j]),
    summed in pick order in fp32 (or_moe_tokens mode 1).  Isolates the
    exact-integer down path from how h rounded."""
    T, k = ids.shape
    rd = om.row_bytes(T_IQ3_S, F)

    def one(t):
        acc = np.zeros(H, np.float32)
        for j in range(k):
            e = int(ids[t, j])
            wd = arena[e * stride + od:e * stride + od + H * rd]
            dv = oracle.dot8q_rows(T_IQ3_S, wd, H, F, codes[t, j][None], scales[t, j][None])[0]
            acc = acc + np.float32(wts[t, j]) * dv
        return acc
    with cf.ThreadPoolExecutor(WORKERS) as ex:
        return np.stack(list(ex.map(one, range(T))))


# ------------------------------------------------------------ config 4

@pytest.mark.parametrize("n", [1, 4])
def test_config4_lmhead_full(gpu, oracle, n):
    """BASELINE config 4 at its stated shape: Q8_0 151936 x 2048 (330 MB),
    fp32 x quantized inside q4_mmvq_n, 1 and 4 tokens."""
    import torch
    rows, K = 151936, 2048
    rng = np.random.default_rng(4000 + n)
    w = synth.matrix(rng, T_Q8_0, rows, K)
    x = rng.standard_normal((n, K)).astype(np.float32)
    dw, dx = dev(w), dev(x)
    y = torch.empty((n, rows), dtype=torch.float32, device="cuda")
    gpu.q4_mmvq_warm()
    q4mi.check(gpu.q4_mmvq_n(T_Q8_0, q4mi.ptr(dw), rows, K, q4mi.ptr(dx), q4mi.ptr(y), 1.0, n),
               "q4_mmvq_n")
    yg = host(y)
    del dw

    def run(p):
        a, b = p
        return oracle.dot8_rows(T_Q8_0, w[a * 2176:b * 2176], b - a, K, x)
    step = (rows + WORKERS - 1) // WORKERS
    parts = [(i, min(rows, i + step)) for i in range(0, rows, step)]
    with cf.ThreadPoolExecutor(len(parts)) as ex:
        yo = np.concatenate(list(ex.map(run, parts)), axis=1)
    assert rel_err(yg, yo) <= TOL


# -------------------------------------------------------- config 3-prefill

def test_prefill_fused_path_config3(gpu, oracle):
    """The benchmark's prefill sequence at config 3-prefill (2048 tokens,
    Zipf-skewed top-10 over 512 experts, the shared expert as expert 512 at
    weight 1 in the routed launches) against the oracle on 288 tokens; the
    q8(h) codes of every sampled (token, pick) row are counted against the
    oracle's."""
    import torch
    E, H, F, T, k = 512, 2048, 512, 2048, 10
    rng = np.random.default_rng(33)
    arena = synth.expert_arena(rng, E + 1, H, F)
    stride, og, ou, od = synth.expert_stride(H, F)
    x = rng.standard_normal((T, H)).astype(np.float32)
    lg = synth.logits(rng, T, E, zipf=True)
    L, P, chk = gpu, q4mi.ptr, q4mi.check
    d_arena, dx, dlg = dev(arena), dev(x), dev(lg)
    i32 = torch.int32
    rows = T * k
    ids, wts = zeros((T, k), i32), zeros((T, k))
    a_tok = zeros(rows + T, i32)
    a_tok[rows:] = torch.arange(T, dtype=i32, device="cuda")
    rsrc, rw = zeros(rows, i32), zeros(rows)
    stg, stgn, ek = zeros(512, i32), zeros(1, i32), zeros(512, i32)
    bounds = zeros(E + 2, i32)
    bounds[E + 1] = rows + T
    xq = zeros(int(L.q4_mmq_q8_bytes(T, H)), torch.uint8)
    hq = zeros(int(L.q4_mmq_q8_bytes(rows + T, F)), torch.uint8)
    pd = zeros((rows + T, H))
    y = zeros((T, H))
    A = d_arena.data_ptr()
    S = A + E * stride
    # exactly bench.py's bench_prefill layer()
    chk(L.q4_hip_route_pf(P(dlg), P(ids), P(wts), T, E, k), "route")
    chk(L.q4mi_assign(P(ids), P(wts), P(a_tok), P(rsrc), P(rw), P(stg), P(stgn), P(ek),
                      P(bounds), T, k, E, T), "assign")
    chk(L.q4_mmq_quantize(P(dx), None, P(xq), T_IQ3_S, H, T), "q8 x")
    chk(L.q4mi_mmq_gate_up_x(A, S, T_IQ3_S, F, H, stride, E, P(xq), T, P(a_tok), P(bounds),
                             rows + T, P(hq)), "mmq gate/up")
    chk(L.q4mi_mmq_mul_id_x(A + od, S + od, T_IQ3_S, H, F, stride, E, P(hq), P(bounds),
                            rows + T, P(pd), H), "mmq down")
    chk(L.q4mi_expert_reduce_x(P(y), P(pd), P(rsrc), P(rw), T, k, H, rows, None), "reduce")
    yg = host(y)
    # routing and the pack: bit-exact
    oid, ow = oracle.softmax_topk(lg, k)
    assert np.array_equal(host(ids), oid)
    pk = oracle.pack(oid, ow, E, T)
    assert np.array_equal(host(a_tok)[:rows], pk["a_tok"][:rows])
    assert np.array_equal(host(bounds)[:E + 1], pk["bounds"])
    assert np.array_equal(host(rsrc), pk["rsrc"])
    # sampled tokens: first, last and 286 others
    samp = np.concatenate([[0, T - 1], rng.choice(np.arange(1, T - 1), 286, replace=False)])
    sid = np.concatenate([oid[samp], np.full((len(samp), 1), E, np.int32)], 1)
    sw = np.concatenate([ow[samp], np.ones((len(samp), 1), np.float32)], 1)
    yo, ho = oracle_tokens(oracle, H, F, arena, stride, x[samp], sid, sw, 1, True)
    # q8(h) of those rows: pick (t, j) is packed row rsrc[t, j]; the shared
    # expert's row of token t is rows + t
    hqh = host(hq)
    n_all = rows + T
    codes = hqh[:n_all * F * 2].view(np.float16).reshape(n_all, F)
    scales = hqh[n_all * F * 2:n_all * F * 2 + n_all * F // 32 * 4].view(np.float32)
    scales = scales.reshape(n_all, F // 32)
    src = np.concatenate([pk["rsrc"].reshape(T, k)[samp], (rows + samp)[:, None]], 1)
    cg = codes[src.reshape(-1)].astype(np.float32)
    frac, flipped = code_diff_fraction(oracle, ho, cg)
    print("prefill q8(h) codes differing: %.3g of %d" % (frac, ho.size))
    assert frac <= CODE_DIFF_MAX, frac
    # the down path fed with the GPU's own q8(h): every sampled token
    yc = down_from_codes(oracle, arena, stride, od, H, F, sid, sw,
                         cg.astype(np.int8).reshape(len(samp), k + 1, F),
                         scales[src.reshape(-1)].reshape(len(samp), k + 1, F // 32))
    assert rel_err(yg[samp], yc) <= TOL
    # end to end against the oracle: every token whose q8(h) codes all equal
    # the oracle's (a flipped code moves y by that code's step times its
    # down column, which the check above accounts for exactly)
    clean = ~flipped.reshape(len(samp), k + 1).any(1)
    print("prefill tokens without a flipped code: %d of %d" % (clean.sum(), len(samp)))
    assert clean.sum() >= 0.8 * len(samp), int(clean.sum())
    assert rel_err(yg[samp][clean], yo[clean]) <= TOL


# ------------------------------------------------------- decode h codes

def test_decode_h_codes(gpu, oracle):
    """The decode layer's fp32 h (read back with q4mi_moe_copy_h) against the
    oracle's h over 20 config-2 seeds: h within 1e-5 of each row's scale;
    q8(h) codes equal to the oracle's on all but <= 1e-4 of the values; y
    equal to the oracle's down path fed with the GPU's own q8(h) on every
    seed, and to the oracle end to end on every seed without a flipped code."""
    from test_gpu_decode import layer, moe_exec_host, routed_ids
    ly = layer()
    F, H = ly.n_ff, ly.n_embd
    hbuf = zeros(64 * 8 * F)
    diff = tot = clean = 0
    worst = 0.0
    for seed in range(21, 41):
        rng = np.random.default_rng(seed)
        x = rng.standard_normal(H).astype(np.float32)
        ids, wts = routed_ids(oracle, rng)
        ids = np.append(ids, 512).astype(np.int32)
        wts = np.append(wts, 1.0).astype(np.float32)
        y = moe_exec_host(gpu, ly, x, ids, wts)
        q4mi.check(gpu.q4mi_moe_copy_h(q4mi.ptr(hbuf), F), "q4mi_moe_copy_h")
        hg = host(hbuf).reshape(64, 8, F)[:len(ids), 0]     # unique experts, token 0
        yo, ho = oracle.moe_tokens(H, F, T_IQ3_S, T_IQ3_S, ly.arena, ly.stride, x,
                                   ids[None], wts[None], want_h=True)
        worst = max(worst, float(np.abs(hg - ho).max() / np.abs(ho).max()))
        qs, ds, nflip = [], [], 0
        for j in range(len(ids)):
            qg, dg, _ = oracle.quant8(hg[j])      # the GPU quantizer's codes (bit-exact)
            qo, _, _ = oracle.quant8(ho[j])
            nflip += int(np.count_nonzero(qg != qo))
            qs.append(qg)
            ds.append(dg)
        diff += nflip
        tot += len(ids) * F
        yc = down_from_codes(oracle, ly.arena, ly.stride, ly.od, H, F, ids[None], wts[None],
                             np.array(qs)[None], np.array(ds)[None])[0]
        assert rel_err(y, yc) <= TOL, seed
        if nflip == 0:
            clean += 1
            assert rel_err(y, yo[0]) <= TOL, seed
    print("decode h: worst rel %.3g; codes differing %d of %d; clean seeds %d of 20"
          % (worst, diff, tot, clean))
    assert worst <= 1e-5, worst
    assert diff / tot <= CODE_DIFF_MAX, (diff, tot)
    assert clean >= 16, clean


# ------------------------------------------- wider hidden sizes (layouts)

@pytest.mark.parametrize("n_embd,n_tok", [(4096, 1), (4096, 4), (8192, 1), (8192, 4)])
def test_moe_wide_hidden(gpu, oracle, n_embd, n_tok):
    """Decode (1 token, host list) and window (4 tokens) at hidden 4096 and
    8192, n_ff 512: the paired-group lane layouts (32 lanes x 4 groups,
    64 x 2, 64 x 4) that hidden 2048 does not use, and the register-heavy
    window at K >= 4096."""
    from test_gpu_decode import Layer, moe_exec_host
    n_exp = 24
    ly = Layer(90 + n_embd // 1024, n_exp=n_exp, n_embd=n_embd, n_ff=512)
    rng = np.random.default_rng(n_embd + n_tok)
    x = rng.standard_normal((n_tok, n_embd)).astype(np.float32)
    ids = np.stack([rng.choice(n_exp, 8, replace=False) for _ in range(n_tok)]).astype(np.int32)
    w = rng.random((n_tok, 8)).astype(np.float32)
    w /= w.sum(1, keepdims=True)
    yo = oracle.moe_tokens(n_embd, 512, T_IQ3_S, T_IQ3_S, ly.arena, ly.stride, x, ids, w)
    if n_tok == 1:
        y = moe_exec_host(gpu, ly, x[0], ids[0], w[0])
        assert rel_err(y, yo[0]) <= TOL
        return
    es = np.full((n_tok, 64), -1, np.int32)
    ew = np.zeros((n_tok, 64), np.float32)
    es[:, :8], ew[:, :8] = ids, w
    assert gpu.q4_hip_moe_win_ok(T_IQ3_S, T_IQ3_S, T_IQ3_S, n_embd, 512, n_tok)
    d_es, d_ew, d_nh, dx = dev(es), dev(ew), dev(np.full(n_tok, 8, np.int32)), dev(x)
    y = dev(np.zeros((n_tok, n_embd), np.float32))
    q4mi.check(gpu.q4_hip_moe_exec_win(q4mi.ptr(ly.d_arena), ly.stride, q4mi.ptr(d_es),
                                       q4mi.ptr(d_ew), q4mi.ptr(d_nh), n_tok, T_IQ3_S, ly.og,
                                       T_IQ3_S, ly.ou, T_IQ3_S, ly.od, q4mi.ptr(dx), None,
                                       q4mi.ptr(y), 512, n_embd, n_embd), "exec_win")
    assert rel_err(host(y), yo) <= TOL


def test_device_status_clean(gpu):
    """After the decode tests, no bounded in-kernel wait gave up."""
    assert gpu.q4mi_device_status(1) == 0, q4mi.last_error()
