"""GPU parity for routing, the stable expert pack and the weighted
scatter-back, against the C oracle (ids, permutation: bit-exact)."""
import ctypes

import numpy as np
import pytest

import q4mi
from q4mi import synth

pytestmark = pytest.mark.gpu


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


def empty(n, dtype):
    import torch
    return torch.empty(n, dtype=dtype, device="cuda")


def route_gpu(L, lg, k):
    import torch
    T, E = lg.shape
    ids, wts = empty((T, k), torch.int32), empty((T, k), torch.float32)
    d = dev(lg)
    q4mi.check(L.q4_hip_route_pf(q4mi.ptr(d), q4mi.ptr(ids), q4mi.ptr(wts), T, E, k), "route_pf")
    return host(ids), host(wts)


@pytest.mark.parametrize("T,E,k,zipf", [(1, 512, 10, False), (2048, 512, 10, True),
                                        (33, 512, 64, False), (7, 100, 8, False)])
def test_route_matches_oracle(gpu, oracle, T, E, k, zipf):
    rng = np.random.default_rng(T + E + k)
    lg = synth.logits(rng, T, E, zipf=zipf)
    if T > 1:
        lg[1, 3] = lg[1, 40] = lg[1, E - 1] = 12.0     # planted ties
    ids, wts = route_gpu(gpu, lg, k)
    oid, ow = oracle.softmax_topk(lg, k)
    assert np.array_equal(ids, oid)
    assert np.allclose(wts, ow, rtol=1e-6, atol=1e-9)


def test_route_probability_ties(gpu, oracle, ref):
    """Different logits whose probabilities round to the same value go to the
    lower index, as q4_topk ranks them (src/q4_quant.c:728-750):
    - logits 1 ulp apart right at the maximum (both exp to exactly 1.0);
    - a token where only 4 experts have a non-zero probability: the other
      6 picks are the lowest-index experts among the underflowed ones,
      whatever their logits."""
    E, k = 512, 10
    rng = np.random.default_rng(5)
    lg = np.stack([rng.standard_normal(E) for _ in range(3)]).astype(np.float32)
    # token 0: the maximum 1e-3 at index 300, its 1-ulp-lower neighbour at 7
    # and 200 (lower index), and at 450; exp(-1 ulp) rounds to 1.0
    lg[0] = rng.uniform(-30, -20, E).astype(np.float32)
    top = np.float32(1e-3)
    lg[0, 300] = top
    lg[0, [7, 450]] = np.nextafter(top, np.float32(-1))
    lg[0, 200] = np.nextafter(np.nextafter(top, np.float32(-1)), np.float32(-1))
    # token 1: 4 live experts; the rest sit 200..300 below (exp underflows
    # to 0), with the larger of those logits at the higher indices
    lg[1] = (-200.0 - np.linspace(100, 0, E)).astype(np.float32)
    lg[1, [11, 99, 300, 480]] = [1.0, 0.5, 0.25, 2.0]
    # token 2: all equal
    lg[2] = 0.75
    ids, wts = route_gpu(gpu, lg, k)
    oid, ow = oracle.softmax_topk(lg, k)
    rid, rw = ref.softmax_topk(lg, k)
    assert np.array_equal(oid, rid) and np.array_equal(ow.view(np.uint32), rw.view(np.uint32))
    assert np.array_equal(ids, oid)
    assert list(oid[1, 4:]) == [0, 1, 2, 3, 4, 5]
    assert list(oid[2]) == list(range(10))
    assert np.allclose(wts, ow, rtol=1e-6, atol=1e-9)


def test_softmax_topk_host_copy(gpu, oracle):
    rng = np.random.default_rng(3)
    lg = rng.standard_normal(512).astype(np.float32)
    d = dev(lg)
    ids = np.empty(10, np.int32)
    w = np.empty(10, np.float32)
    q4mi.check(gpu.q4_hip_softmax_topk(q4mi.ptr(d), 512, 10, ids.ctypes.data_as(ctypes.c_void_p),
                                       w.ctypes.data_as(ctypes.c_void_p)), "softmax_topk")
    oid, ow = oracle.softmax_topk(lg[None], 10)
    assert np.array_equal(ids, oid[0]) and np.allclose(w, ow[0], rtol=1e-6)


def pack_gpu(L, ids, wts, E, gsz):
    import torch
    T, k = ids.shape
    n_g = (T + gsz - 1) // gsz
    a_tok = dev(np.full(n_g * gsz * k, -7, np.int32))
    rsrc, rw = empty(T * k, torch.int32), empty(T * k, torch.float32)
    stg = dev(np.full(n_g * 512, -7, np.int32))
    stgn, ek = empty(n_g, torch.int32), empty(n_g * 512, torch.int32)
    bounds = empty(n_g * (E + 1), torch.int32)
    di, dw = dev(ids), dev(wts)
    q4mi.check(L.q4mi_assign(q4mi.ptr(di), q4mi.ptr(dw), q4mi.ptr(a_tok), q4mi.ptr(rsrc),
                             q4mi.ptr(rw), q4mi.ptr(stg), q4mi.ptr(stgn), q4mi.ptr(ek),
                             q4mi.ptr(bounds), gsz, k, E, T), "q4mi_assign")
    return dict(a_tok=host(a_tok), rsrc=host(rsrc), rw=host(rw), stg=host(stg),
                stgn=host(stgn).astype(np.uint32), ek=host(ek).astype(np.uint32),
                bounds=host(bounds))


@pytest.mark.parametrize("T,k,gsz", [(2048, 10, 2048), (17, 10, 8), (300, 64, 300),
                                     (4, 10, 4), (1000, 10, 333)])
def test_pack_bitexact(gpu, oracle, T, k, gsz):
    rng = np.random.default_rng(T * k + gsz)
    E = 512
    lg = synth.logits(rng, T, E, zipf=True)
    ids, wts = oracle.softmax_topk(lg, k)
    ids[0, 1] = -1              # invalid pick
    if T > 2:
        ids[2, 0] = 700         # out of range pick
    got = pack_gpu(gpu, ids, wts, E, gsz)
    ref = oracle.pack(ids, wts, E, gsz)
    n_rows = [int(b) for b in ref["bounds"][E::E + 1]]
    n_g = len(n_rows)
    for g in range(n_g):
        s = g * gsz * k
        assert np.array_equal(got["a_tok"][s:s + n_rows[g]], ref["a_tok"][s:s + n_rows[g]])
        assert np.array_equal(got["stg"][g * 512:g * 512 + ref["stgn"][g]],
                              ref["stg"][g * 512:g * 512 + ref["stgn"][g]])
    for key in ("rsrc", "rw", "stgn", "ek", "bounds"):
        assert np.array_equal(got[key], ref[key]), key


def test_expert_reduce(gpu):
    import torch
    rng = np.random.default_rng(5)
    T, k, n = 64, 10, 2048
    rows = T * k
    pd = rng.standard_normal((rows, n)).astype(np.float32)
    rsrc = rng.permutation(rows).astype(np.int32).reshape(T, k)
    rsrc[3, 4] = -1
    rw = rng.random((T, k)).astype(np.float32)
    y0 = rng.standard_normal((T, n)).astype(np.float32)
    # keep every device buffer referenced until the kernel has run: a freed
    # temporary's block can be handed to the next allocation of the same size
    y, d_pd, d_rsrc, d_rw = dev(y0), dev(pd), dev(rsrc), dev(rw)
    q4mi.check(gpu.q4_hip_expert_reduce(q4mi.ptr(y), q4mi.ptr(d_pd), q4mi.ptr(d_rsrc),
                                        q4mi.ptr(d_rw), T, k, n), "expert_reduce")
    ref = y0.astype(np.float64).copy()
    for t in range(T):
        for j in range(k):
            if rsrc[t, j] >= 0:
                ref[t] += rw[t, j] * pd[rsrc[t, j]].astype(np.float64)
    assert np.abs(host(y) - ref).max() < 1e-4
