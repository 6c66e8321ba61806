"""GPU parity for the remaining drop-in entry points, through the C ABI:

- q4_hip_moe_stage / q4_hip_moe_exec_staged (src/q4.h:1306-1311): the staged
  list equals the host-list layer, and a captured graph replays with the list
  staged last;
- q4_hip_moe_tok_ok / q4_hip_moe_exec_tok (src/q4.h:893-901): ragged
  per-token lists equal the single-token layer per token, equal counts equal
  the verify window;
- q4_mmq_gather / q4_mmq_wbuf / q4_mmq_wbuf_lend / q4_mmq_pad
  (src/q4.h:1161-1174): gathered bytes and zero tails exactly, and MMQ over
  the gathered buffer equals MMQ over the arena.

The references here are entry points pinned against the oracle elsewhere
(test_gpu_decode, test_gpu_mmq).  The same kernels run on both sides, so
the bar is 1e-6 relative (in practice bit-identical), not the oracle's 1e-3.
"""
import ctypes

import numpy as np
import pytest

from conftest import rel_err
from test_gpu_decode import dev, host, layer, moe_exec_host, routed_ids
from test_gpu_mmq import mmq_quant, mul_id

import oracle as om
import q4mi
from q4mi import synth

pytestmark = pytest.mark.gpu
T_IQ3_S = q4mi.T_IQ3_S
SAME = 1e-6


def host_arr(a, dtype):
    a = np.ascontiguousarray(a, dtype)
    return a, a.ctypes.data_as(ctypes.c_void_p)


def stage(L, ids, wts):
    ids, pi = host_arr(ids, np.int32)
    wts, pw = host_arr(wts, np.float32)
    q4mi.check(L.q4_hip_moe_stage(pi, pw, len(ids)), "q4_hip_moe_stage")


def exec_staged(L, ly, dx, y):
    q4mi.check(L.q4_hip_moe_exec_staged(q4mi.ptr(ly.d_arena), ly.stride, T_IQ3_S, ly.og, T_IQ3_S,
                                        ly.ou, T_IQ3_S, ly.od, q4mi.ptr(dx), None, None, None,
                                        q4mi.ptr(y), ly.n_ff, ly.n_embd, ly.n_embd),
               "q4_hip_moe_exec_staged")


def top(oracle, rng, k):
    ids, wts = routed_ids(oracle, rng, k=k)
    return np.append(ids, 512).astype(np.int32), np.append(wts, 1.0).astype(np.float32)


def test_staged_matches_host_exec(gpu, oracle):
    ly = layer()
    rng = np.random.default_rng(41)
    x = rng.standard_normal(ly.n_embd).astype(np.float32)
    ids, wts = top(oracle, rng, 10)
    want = moe_exec_host(gpu, ly, x, ids, wts)
    stage(gpu, ids, wts)
    dx, y = dev(x), dev(np.zeros(ly.n_embd, np.float32))
    exec_staged(gpu, ly, dx, y)
    assert rel_err(host(y), want) <= SAME
    # an empty staged list adds nothing
    stage(gpu, ids[:0], wts[:0])
    exec_staged(gpu, ly, dx, y)
    assert rel_err(host(y), want) <= SAME


def test_staged_graph_replays_current_list(gpu, oracle):
    """One capture, six replays over three lists of different lengths: each
    replay reads the list staged just before it (eager work and syncs run
    between replays; every replay is checked against the eager layer)."""
    import torch
    ly = layer()
    rng = np.random.default_rng(42)
    x = rng.standard_normal(ly.n_embd).astype(np.float32)
    lists = [top(oracle, rng, k) for k in (10, 7, 4)]
    dx, y = dev(x), dev(np.zeros(ly.n_embd, np.float32))
    gpu.q4_hip_moe_scratch_warm()
    stage(gpu, *lists[0])
    exec_staged(gpu, ly, dx, y)          # warm every launch configuration eagerly
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        q4mi.use_torch_stream()
        exec_staged(gpu, ly, dx, y)
    q4mi.use_torch_stream()
    for ids, wts in lists + lists[::-1]:
        want = moe_exec_host(gpu, ly, x, ids, wts)
        stage(gpu, ids, wts)
        y.zero_()
        g.replay()
        assert rel_err(host(y), want) <= SAME


def run_tok(L, ly, x, lists):
    n_tok = len(lists)
    off = np.zeros(n_tok + 1, np.uint32)
    off[1:] = np.cumsum([len(i) for i, _ in lists])
    flat_i = np.concatenate([i for i, _ in lists] + [np.zeros(1, np.int32)])
    flat_w = np.concatenate([w for _, w in lists] + [np.zeros(1, np.float32)])
    d_s, d_w, dx = dev(flat_i), dev(flat_w), dev(x)
    y = dev(np.zeros((n_tok, ly.n_embd), np.float32))
    off, po = host_arr(off, np.uint32)
    assert L.q4_hip_moe_tok_ok(T_IQ3_S, T_IQ3_S, T_IQ3_S, ly.n_embd, ly.n_ff)
    q4mi.check(L.q4_hip_moe_exec_tok(q4mi.ptr(ly.d_arena), ly.stride, q4mi.ptr(d_s),
                                     q4mi.ptr(d_w), po, n_tok, T_IQ3_S, ly.og, T_IQ3_S, ly.ou,
                                     T_IQ3_S, ly.od, q4mi.ptr(dx), None, None, q4mi.ptr(y),
                                     ly.n_ff, ly.n_embd, ly.n_embd), "q4_hip_moe_exec_tok")
    return host(y)


@pytest.mark.parametrize("counts", [[11, 5, 0, 3], [11] * 8, [2]])
def test_exec_tok_per_token(gpu, oracle, counts):
    """Ragged counts (incl. an empty token), equal counts past the window's
    64 picks, and a single token: one layer per token."""
    ly = layer()
    rng = np.random.default_rng(43 + len(counts))
    x = rng.standard_normal((len(counts), ly.n_embd)).astype(np.float32)
    lists = [top(oracle, rng, c - 1) if c else (np.zeros(0, np.int32), np.zeros(0, np.float32))
             for c in counts]
    got = run_tok(gpu, ly, x, lists)
    for t, (ids, wts) in enumerate(lists):
        if not len(ids):
            assert not got[t].any()
            continue
        assert rel_err(got[t], moe_exec_host(gpu, ly, x[t], ids, wts)) <= SAME, t


def test_exec_tok_equal_counts_is_the_window(gpu, oracle):
    ly = layer()
    rng = np.random.default_rng(47)
    n_tok = 4
    x = rng.standard_normal((n_tok, ly.n_embd)).astype(np.float32)
    lists = [top(oracle, rng, 10) for _ in range(n_tok)]
    got = run_tok(gpu, ly, x, lists)
    es = np.full((n_tok, 64), -1, np.int32)
    ew = np.zeros((n_tok, 64), np.float32)
    nh = np.zeros(n_tok, np.int32)
    for t, (ids, wts) in enumerate(lists):
        es[t, :len(ids)], ew[t, :len(ids)], nh[t] = ids, wts, len(ids)
    d_es, d_ew, d_nh, dx = dev(es), dev(ew), dev(nh), dev(x)
    y = dev(np.zeros((n_tok, ly.n_embd), np.float32))
    q4mi.check(gpu.q4_hip_moe_exec_win(q4mi.ptr(ly.d_arena), ly.stride, q4mi.ptr(d_es),
                                       q4mi.ptr(d_ew), q4mi.ptr(d_nh), n_tok, T_IQ3_S, ly.og,
                                       T_IQ3_S, ly.ou, T_IQ3_S, ly.od, q4mi.ptr(dx), None,
                                       q4mi.ptr(y), ly.n_ff, ly.n_embd, ly.n_embd),
               "q4_hip_moe_exec_win")
    assert rel_err(got, host(y)) <= SAME


def gather(L, abase, astride, goff, gu_bytes, doff, d_bytes, gu_dst, d_dst, eid, slot, d_gu,
           d_d):
    d_eid, d_slot = dev(np.asarray(eid, np.int32)), dev(np.asarray(slot, np.int32))
    q4mi.check(L.q4_mmq_gather(abase, astride, goff, gu_bytes, doff, d_bytes, gu_dst, d_dst,
                               q4mi.ptr(d_eid), q4mi.ptr(d_slot), len(eid), d_gu, d_d),
               "q4_mmq_gather")


@pytest.mark.parametrize("shift,gu_bytes,d_bytes,pad", [(0, 901120, 450560, 4096),
                                                         (4, 1000, 500, 12),
                                                         (3, 999, 501, 7)])
def test_mmq_gather_bytes(gpu, shift, gu_bytes, d_bytes, pad):
    """16-, 4- and 1-byte copy paths: every gathered byte equals its source
    and every tail byte up to the destination stride is zero (the buffers
    start filled with 0xAB)."""
    import torch
    rng = np.random.default_rng(48 + shift)
    E, astride = 6, gu_bytes + d_bytes + 64 + shift
    arena = rng.integers(0, 256, E * astride + 64, dtype=np.uint8)
    d_arena = dev(arena)
    goff, doff = shift, shift + gu_bytes + 32
    slot, eid = [4, 1, 5], [2, 0, 3]
    n_exp = 4
    gu_dst, d_dst = gu_bytes + pad, d_bytes + pad
    d_gu = torch.full((n_exp * gu_dst + 16,), 0xAB, dtype=torch.uint8, device="cuda")
    d_d = torch.full((n_exp * d_dst + 16,), 0xAB, dtype=torch.uint8, device="cuda")
    gather(gpu, q4mi.ptr(d_arena), astride, goff, gu_bytes, doff, d_bytes, gu_dst, d_dst, eid,
           slot, q4mi.ptr(d_gu), q4mi.ptr(d_d))
    gu, dd = host(d_gu), host(d_d)
    for e, s in zip(eid, slot):
        src = arena[s * astride:]
        assert np.array_equal(gu[e * gu_dst:e * gu_dst + gu_bytes], src[goff:goff + gu_bytes])
        assert not gu[e * gu_dst + gu_bytes:(e + 1) * gu_dst].any()
        assert np.array_equal(dd[e * d_dst:e * d_dst + d_bytes], src[doff:doff + d_bytes])
        assert not dd[e * d_dst + d_bytes:(e + 1) * d_dst].any()
    # expert 1 was never gathered: untouched
    assert (gu[1 * gu_dst:2 * gu_dst] == 0xAB).all()


def test_mmq_gathered_experts_match_arena(gpu):
    """The reference's prefill sequence: gather the used experts into the
    library's id-indexed buffers (q4_mmq_wbuf, stride = bytes + q4_mmq_pad),
    then mul_id over them; each expert's rows equal mul_id on the arena."""
    rng = np.random.default_rng(49)
    H, F, E = 2048, 512, 6
    arena = synth.expert_arena(rng, E, H, F)
    stride, og, ou, od = synth.expert_stride(H, F)
    d_arena = dev(arena)
    rb_g = om.row_bytes(T_IQ3_S, H)
    gu_bytes, d_bytes = od - og, stride - od
    assert gpu.q4_mmq_pad(rb_g) == 0
    gu_dst, d_dst = gu_bytes + gpu.q4_mmq_pad(rb_g), d_bytes
    slot, eid = [5, 2, 3], [0, 1, 2]
    p_gu, p_d = ctypes.c_void_p(), ctypes.c_void_p()
    q4mi.check(gpu.q4_mmq_wbuf(gu_dst, d_dst, 3, ctypes.byref(p_gu), ctypes.byref(p_d)),
               "q4_mmq_wbuf")
    gather(gpu, q4mi.ptr(d_arena), stride, og, gu_bytes, od, d_bytes, gu_dst, d_dst, eid, slot,
           p_gu.value, p_d.value)
    per = [70, 130, 9]
    T = 160
    x = rng.standard_normal((T, H)).astype(np.float32)
    a_tok = np.concatenate([rng.integers(0, T, n) for n in per]).astype(np.int32)
    bounds = np.concatenate([[0], np.cumsum(per)]).astype(np.int32)
    total = int(bounds[-1])
    xq = mmq_quant(gpu, dev(x), dev(a_tok), H, total)

    class Raw:      # a device address mul_id can take
        def __init__(self, p):
            self.p = p

        def data_ptr(self):
            return self.p

    got = host(mul_id(gpu, Raw(p_gu.value), T_IQ3_S, 2 * F, H, gu_dst, 3, xq, dev(bounds),
                      total, 2 * F))
    for e, s in zip(eid, slot):
        one = dev(np.array([0, per[e]], np.int32))
        xe = mmq_quant(gpu, dev(x), dev(a_tok[bounds[e]:bounds[e + 1]]), H, per[e])
        ref = host(mul_id(gpu, Raw(d_arena.data_ptr() + s * stride + og), T_IQ3_S, 2 * F, H,
                          gu_dst, 1, xe, one, per[e], 2 * F))
        assert np.array_equal(got[bounds[e]:bounds[e + 1]], ref), e


def test_mmq_wbuf_lend(gpu):
    """Lend mode: q4_mmq_wbuf hands out the borrowed (zeroed) buffers and
    refuses sizes beyond them.  Runs last among the pool tests: lending is
    permanent for the process."""
    import torch
    gu = torch.full((1 << 20,), 7, dtype=torch.uint8, device="cuda")
    d = torch.full((1 << 19,), 7, dtype=torch.uint8, device="cuda")
    q4mi.check(gpu.q4_mmq_wbuf_lend(q4mi.ptr(gu), gu.numel(), q4mi.ptr(d), d.numel()),
               "q4_mmq_wbuf_lend")
    assert not host(gu).any() and not host(d).any()
    p_gu, p_d = ctypes.c_void_p(), ctypes.c_void_p()
    assert gpu.q4_mmq_wbuf(1 << 18, 1 << 17, 4, ctypes.byref(p_gu), ctypes.byref(p_d))
    assert p_gu.value == gu.data_ptr() and p_d.value == d.data_ptr()
    assert not gpu.q4_mmq_wbuf(1 << 18, 1 << 17, 5, ctypes.byref(p_gu), ctypes.byref(p_d))
