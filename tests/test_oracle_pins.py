"""Pin the C oracle (oracle/q4_oracle.c) before trusting it.

Each check is independent of the oracle's own formula: the reference's kernels
compiled from source (oracle/_ref, when present), closed-form known answers,
integer brute force over the float dequantization, and a stable sort for the
pack.  CPU only.
"""
import numpy as np
import pytest

from conftest import rel_err

import oracle as om
from q4mi import synth

T_IQ3_S, T_Q8_0 = om.T_IQ3_S, om.T_Q8_0


def grid_entries():
    import os
    import re
    from conftest import ROOT
    text = open(os.path.join(ROOT, "include", "q4mi_iq3s_grid.h")).read()
    body = text.split("#define Q4MI_IQ3S_CODES", 1)[1].split("static const", 1)[0]
    codes = [int(c, 16) for c in re.findall(r"0x[0-9a-f]+", body)]
    return [sum((2 * ((c >> (3 * j)) & 7) + 1) << (8 * j) for j in range(4)) for c in codes]


def test_grid_table_structure():
    g = grid_entries()
    assert len(g) == 512
    # reference src/q4_test.c:51-57: entry 0 is 0x01010101
    assert g[0] == 0x01010101
    # the codebook is strictly increasing as u32 and every byte is odd 1..15
    assert all(g[i] < g[i + 1] for i in range(511))
    b = np.array(g, np.uint32).view(np.uint8)
    assert set(np.unique(b)) == {1, 3, 5, 7, 9, 11, 13, 15}


def test_iq3s_known_answer(oracle):
    """src/q4_test.c:51-57: zero codeword, d=1, x=1 gives 256."""
    blk = np.zeros(110, np.uint8)
    blk[0:2] = np.array([1.0], np.float16).view(np.uint8)
    y = oracle.dequant_row(T_IQ3_S, blk, 256)
    assert np.all(y == 1.0) and y.sum() == 256.0
    x = np.ones(256, np.float32)
    q, d, bs = oracle.quant8(x)
    assert np.all(q == 127) and np.all(bs == 32 * 127)
    s = oracle.group_sums(T_IQ3_S, blk, 256, q)
    assert np.all(s == 32 * 127)
    yd = oracle.dot8_rows(T_IQ3_S, blk, 1, 256, x)[0, 0]
    assert abs(yd - 256.0) < 1e-3


def test_quant8_closed_form(oracle):
    rng = np.random.default_rng(1)
    x = rng.standard_normal(4096).astype(np.float32)
    x[0:32] = 0.0                      # amax = 0 -> all zero
    x[32:64] = np.arange(32) - 15.5    # amax = 15.5
    x[64:96] = (np.arange(32) - 16) + 0.5  # amax 15.5, x*127/15.5 ties? no
    # exact ties: amax = 127 -> scale 1 -> k + 0.5 rounds to even
    x[96:128] = np.arange(32, dtype=np.float32) - 16.5
    x[127] = 127.0
    q, d, bs = oracle.quant8(x)
    assert np.all(q[0:32] == 0) and d[0] == 0 and bs[0] == 0
    ties = x[96:127]
    assert np.array_equal(q[96:127], np.round(ties).astype(np.int8))  # numpy rounds half-even
    a = np.abs(x.reshape(-1, 32)).max(1)
    assert np.array_equal(d, (a / np.float32(127)).astype(np.float32))
    assert np.array_equal(bs, q.reshape(-1, 32).astype(np.int32).sum(1))
    # invariant of the reference's selftest (src/q4_cpuexp.c:2989-2999)
    err = np.abs(q.astype(np.float32) * np.repeat(d, 32) - x)
    assert np.all(err <= np.repeat(d, 32) * 0.51 + 1e-6)


def test_group_sums_bruteforce(oracle):
    """Exact int32 group sums vs a brute-force dot over the float
    dequantization with d = 1 (values are then exact integers)."""
    rng = np.random.default_rng(2)
    for ty, K in ((T_IQ3_S, 2048), (T_Q8_0, 1024)):
        w = synth.matrix(rng, ty, 8, K)
        bb = 110 if ty == T_IQ3_S else 34
        wb = w.reshape(-1, bb)
        wb[:, 0:2] = np.array([1.0], np.float16).view(np.uint8)
        x = rng.standard_normal(K).astype(np.float32)
        q, d, _ = oracle.quant8(x)
        rbytes = om.row_bytes(ty, K)
        for r in range(8):
            row = w[r * rbytes:(r + 1) * rbytes]
            deq = oracle.dequant_row(ty, row, K)
            assert np.all(deq == np.round(deq))
            brute = (deq.astype(np.int64).reshape(-1, 32) *
                     q.astype(np.int64).reshape(-1, 32)).sum(1)
            s = oracle.group_sums(ty, row, K, q)
            assert np.array_equal(s.astype(np.int64), brute)


def test_dot_matches_double(oracle):
    """fp32 row dots vs a float64 sum of exact group sums * d_w * d_x."""
    rng = np.random.default_rng(3)
    K, rows = 4096, 32
    w = synth.matrix(rng, T_IQ3_S, rows, K)
    x = rng.standard_normal(K).astype(np.float32)
    q, d, _ = oracle.quant8(x)
    y = oracle.dot8_rows(T_IQ3_S, w, rows, K, x)[0]
    rb = om.row_bytes(T_IQ3_S, K)
    for r in range(rows):
        row = w[r * rb:(r + 1) * rb]
        s = oracle.group_sums(T_IQ3_S, row, K, q).astype(np.float64)
        dw = np.repeat(row.reshape(-1, 110)[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0], 8)
        ref = (s * dw * d.astype(np.float64)).sum()
        assert abs(y[r] - ref) <= 1e-5 * max(abs(ref), 1e-3)


def test_routing_topk_invariants(oracle):
    rng = np.random.default_rng(4)
    lg = rng.standard_normal((64, 512)).astype(np.float32)
    lg[0, 10] = lg[0, 20] = lg[0, 30] = 9.0   # planted ties: lower index first
    ids, wts = oracle.softmax_topk(lg, 10)
    assert list(ids[0, :3]) == [10, 20, 30]
    for t in range(64):
        order = np.lexsort((np.arange(512), -lg[t]))[:10]
        assert np.array_equal(ids[t], order)
        assert abs(float(wts[t].sum()) - 1.0) < 1e-6
        assert np.all(np.diff(wts[t]) <= 0)


def test_pack_is_stable_sort(oracle):
    rng = np.random.default_rng(5)
    T, k, E = 300, 10, 512
    lg = synth.logits(rng, T, E, zipf=True)
    ids, wts = oracle.softmax_topk(lg, k)
    ids[3, 2] = -1                      # invalid pick: rsrc -1, weight 0
    for gsz in (300, 64, 17):
        pk = oracle.pack(ids, wts, E, gsz)
        n_g = (T + gsz - 1) // gsz
        for g in range(n_g):
            t0, t1 = g * gsz, min(T, (g + 1) * gsz)
            e = ids[t0:t1].reshape(-1)
            tk = np.repeat(np.arange(t0, t1), k)
            valid = e >= 0
            order = np.argsort(np.where(valid, e, 1 << 20), kind="stable")[:valid.sum()]
            seg = pk["a_tok"][g * gsz * k: g * gsz * k + valid.sum()]
            assert np.array_equal(seg, tk[order])
            cnt = np.bincount(e[valid], minlength=E)
            assert np.array_equal(pk["ek"][g * 512:g * 512 + E], cnt)
            b = pk["bounds"][g * (E + 1):(g + 1) * (E + 1)]
            assert np.array_equal(b[:-1], np.concatenate([[0], np.cumsum(cnt)[:-1]]))
            assert b[-1] == valid.sum()
            used = np.nonzero(cnt)[0]
            assert pk["stgn"][g] == len(used)
            assert np.array_equal(pk["stg"][g * 512:g * 512 + len(used)], used)
        # rsrc maps every pick back to its token and weight
        for t in range(T):
            g = t // gsz
            for j in range(k):
                p = pk["rsrc"][t * k + j]
                if ids[t, j] < 0:
                    assert p == -1 and pk["rw"][t * k + j] == 0
                else:
                    assert pk["a_tok"][g * gsz * k + p] == t
                    assert pk["rw"][t * k + j] == wts[t, j]


# ----------------------------------------------- against the reference build

def test_quant8_bitexact_vs_reference(oracle, ref):
    rng = np.random.default_rng(6)
    x = (rng.standard_normal(1 << 15) * rng.choice([1e-3, 1, 30], 1 << 15)).astype(np.float32)
    x[0:32] = 0
    x[64:96] = np.arange(32) - 16.5
    x[95] = 127
    for a, b in zip(oracle.quant8(x), ref.quant8(x)):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("ty,K,nt", [(T_IQ3_S, 2048, 1), (T_IQ3_S, 4096, 1),
                                     (T_IQ3_S, 512, 4), (T_Q8_0, 2048, 1),
                                     (T_Q8_0, 2048, 4)])
def test_dot8_bitexact_vs_reference(oracle, ref, ty, K, nt):
    rng = np.random.default_rng(7 + K + nt)
    rows = 64
    w = synth.matrix(rng, ty, rows, K)
    x = rng.standard_normal((nt, K)).astype(np.float32)
    a = oracle.dot8_rows(ty, w, rows, K, x)
    b = ref.dot8_rows(ty, w, rows, K, x)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_softmax_topk_vs_reference(oracle, ref):
    rng = np.random.default_rng(8)
    lg = synth.logits(rng, 256, 512, zipf=True)
    lg[0, 5] = lg[0, 6] = 50.0
    a = oracle.softmax_topk(lg, 10)
    b = ref.softmax_topk(lg, 10)
    assert np.array_equal(a[0], b[0])
    assert np.array_equal(a[1].view(np.uint32), b[1].view(np.uint32))


def test_moe_decode_vs_reference(oracle, ref):
    rng = np.random.default_rng(9)
    n_embd, n_ff, E = 512, 256, 24
    arena = synth.expert_arena(rng, E, n_embd, n_ff)
    stride = synth.expert_stride(n_embd, n_ff)[0]
    x = rng.standard_normal(n_embd).astype(np.float32)
    ids = np.array([3, 17, 5, 23, 0, 9], np.int32)
    wts = np.array([0.3, 0.2, 0.2, 0.1, 0.1, 0.1], np.float32)
    yr = ref.moe_decode(n_embd, n_ff, T_IQ3_S, T_IQ3_S, E, arena, stride, x, ids, wts)
    yo = oracle.moe_tokens(n_embd, n_ff, T_IQ3_S, T_IQ3_S, arena, stride, x, ids, wts)[0]
    assert rel_err(yo, yr) < 1e-5


def test_moe_window_vs_reference(oracle, ref):
    rng = np.random.default_rng(10)
    n_embd, n_ff, E, T, k = 512, 256, 16, 4, 4
    arena = synth.expert_arena(rng, E, n_embd, n_ff)
    stride = synth.expert_stride(n_embd, n_ff)[0]
    x = rng.standard_normal((T, n_embd)).astype(np.float32)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    wts = rng.random((T, k)).astype(np.float32)
    yr = ref.moe_win(n_embd, n_ff, T_IQ3_S, T_IQ3_S, E, arena, stride, x, ids, wts,
                     np.full(T, k, np.uint32))
    yo = oracle.moe_tokens(n_embd, n_ff, T_IQ3_S, T_IQ3_S, arena, stride, x, ids, wts)
    assert rel_err(yo, yr) < 1e-5


def test_dot8q_rows_is_dot8_of_quantized(oracle):
    """or_dot8q_rows (pre-quantized activations) equals or_dot8_rows bit for
    bit when fed or_quant8's codes and scales."""
    from q4mi import synth
    rng = np.random.default_rng(8)
    for ty, K in ((om.T_IQ3_S, 512), (om.T_Q8_0, 256)):
        w = synth.matrix(rng, ty, 40, K)
        x = rng.standard_normal((3, K)).astype(np.float32)
        q = np.stack([oracle.quant8(x[t])[0] for t in range(3)])
        d = np.stack([oracle.quant8(x[t])[1] for t in range(3)])
        a = oracle.dot8q_rows(ty, w, 40, K, q, d)
        b = oracle.dot8_rows(ty, w, 40, K, x)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _router_rows(rng, ty, n_exp, K):
    w = (rng.standard_normal((n_exp, K)) * 0.05).astype(np.float32)
    if ty == 0:
        return w, w
    if ty == 1:
        h = w.astype(np.float16)
        return h.view(np.uint8), h.astype(np.float32)
    b = (w.view(np.uint32) >> 16).astype(np.uint16)      # BF16 by truncation
    return b.view(np.uint8), (b.astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("ty", [0, 1, 30])
def test_router_logits_vs_reference_and_exact(oracle, ref, ty):
    """or_router (the library's fixed dot order) against the reference's own
    router GEMV q4_gemv (src/q4_quant.c:595-622, another order) and a
    float64 dot: within 1e-5 of each row's sum of |w x|; and the routing the
    reference takes from its logits equals the oracle's from its own."""
    rng = np.random.default_rng(40 + ty)
    n_exp, K, T = 512, 2048, 6
    wb, wf = _router_rows(rng, ty, n_exp, K)
    x = rng.standard_normal((T, K)).astype(np.float32)
    lg = oracle.router(ty, wb, n_exp, K, x)
    for t in range(T):
        rl = ref.gemv(ty, wb, n_exp, K, x[t])
        exact = wf.astype(np.float64) @ x[t].astype(np.float64)
        scale = np.abs(wf.astype(np.float64)) @ np.abs(x[t].astype(np.float64))
        assert np.all(np.abs(lg[t] - exact) <= 1e-5 * scale)
        assert np.all(np.abs(rl - exact) <= 1e-5 * scale)
        oid, _ = oracle.softmax_topk(lg[t], 10)
        rid, _ = ref.softmax_topk(rl, 10)
        assert np.array_equal(oid, rid)


def test_router_dot_order_closed_form(oracle):
    """The fixed order on inputs where every partial sum is exact (small
    integers): the logits are the exact integer dots; and a single non-zero
    product lands unchanged wherever it sits."""
    rng = np.random.default_rng(9)
    n_exp, K = 64, 512
    w = rng.integers(-8, 9, (n_exp, K)).astype(np.float32)
    x = rng.integers(-8, 9, (2, K)).astype(np.float32)
    lg = oracle.router(0, w, n_exp, K, x)
    assert np.array_equal(lg, (x.astype(np.int64) @ w.T.astype(np.int64)).astype(np.float32))
    w1 = np.zeros((K, K), np.float32)
    w1[np.arange(K), np.arange(K)] = 3.0
    lg1 = oracle.router(0, w1, K, K, x[:1])
    assert np.array_equal(lg1[0], 3.0 * x[0])


def test_sgate_closed_form(oracle):
    """sigmoid(sgw . x): a zero gate vector gives exactly 0.5, a large
    positive dot gives 1, a large negative one 0; otherwise 1/(1+e^-d)."""
    rng = np.random.default_rng(10)
    K = 1024
    w = np.zeros((4, K), np.float32)
    x = rng.standard_normal((3, K)).astype(np.float32)
    _, sg = oracle.router(0, w, 4, K, x, sgw=np.zeros(K, np.float32))
    assert np.all(sg == 0.5)
    _, sg = oracle.router(0, w, 4, K, x, sgw=x[0] * 10)
    assert sg[0] == 1.0
    _, sg = oracle.router(0, w, 4, K, x, sgw=-x[0] * 10)
    assert sg[0] == 0.0
    g = (rng.standard_normal(K) * 0.01).astype(np.float32)
    _, sg = oracle.router(0, w, 4, K, x, sgw=g)
    d = x.astype(np.float64) @ g.astype(np.float64)
    assert np.allclose(sg, 1 / (1 + np.exp(-d)), rtol=1e-6, atol=0)


def test_xg_fp16_rounding(oracle):
    """The XG oracle's fp32 -> fp16 conversion equals numpy's (IEEE round to
    nearest even) on normals, subnormals, ties, overflow and signed zero."""
    rng = np.random.default_rng(12)
    v = np.concatenate([rng.standard_normal(4000) * 10 ** rng.uniform(-9, 5, 4000),
                        np.array([0.0, -0.0, 65504.0, 65520.0, 70000.0, 6e-8, 3e-8, 1e-9,
                                  1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, -2049.0, 2051.0])
                        ]).astype(np.float32)
    got = np.array([oracle.L.or_f16_bits(float(f)) for f in v], np.uint16)
    with np.errstate(over="ignore"):     # 65520 and 70000 overflow to inf, as intended
        want = v.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_xg_dequant_close_to_float_dequant(oracle):
    """XG weights (fp16 of the integer times fp16(scale * 256)) are the
    float dequantization times 256 to two fp16 roundings."""
    rng = np.random.default_rng(13)
    for ty in (om.T_IQ3_S, om.T_Q8_0):
        w = synth.matrix(rng, ty, 3, 2048)
        rb = om.row_bytes(ty, 2048)
        for r in range(3):
            a = oracle.xg_dequant_row(ty, w[r * rb:(r + 1) * rb], 2048).astype(np.float64)
            b = oracle.dequant_row(ty, w[r * rb:(r + 1) * rb], 2048).astype(np.float64) * 256
            assert np.all(np.abs(a - b) <= 2 * 2 ** -11 * np.abs(b) + 1e-30)
