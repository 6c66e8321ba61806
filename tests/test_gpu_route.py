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


MAIL_BYTES = 1240           # the reference mailbox prefix copied to the host (through seq)


def mail_fields(raw):
    """Fields of the reference's q4_mail_t prefix (src/q4_moe.c:368-386)."""
    b = raw.tobytes()
    i32 = lambda o, n: np.frombuffer(b, np.int32, n, o)
    return {"ids": i32(0, 64), "wts": np.frombuffer(b, np.float32, 64, 256),
            "n": int(i32(512, 1)[0]), "ntok": int(i32(516, 1)[0]), "tn": i32(520, 8),
            "hs": i32(552, 128), "hn": i32(1064, 8), "rk": np.frombuffer(b, np.uint8, 64, 1096),
            "routed": i32(1160, 16), "rseq": int(np.frombuffer(b, np.uint64, 1, 1224)[0]),
            "seq": int(np.frombuffer(b, np.uint64, 1, 1232)[0])}


@pytest.mark.parametrize("T,E,k,resident", [(1, 512, 10, "all"), (4, 512, 10, "all"),
                                            (4, 512, 10, "half"), (6, 1024, 10, "half"),
                                            (8, 700, 8, "none")])
def test_route_dev_n_reference_signature(gpu, oracle, T, E, k, resident):
    """q4_hip_route_dev_n through the reference's signature (src/q4.h:1289-1294):
    hits land in the stride-64 device lists as slots, misses in the mailbox
    in token order with their ranks, seq / rseq bumped once per call; ids and
    weights are q4_topk's (the oracle), ids bit-exact."""
    import torch
    L = gpu
    rng = np.random.default_rng(T * 31 + E)
    lg = synth.logits(rng, T, E, zipf=False)
    if resident == "all":
        devtab = np.arange(E, dtype=np.int32)[::-1].copy()       # slot = E - 1 - id
    elif resident == "half":
        devtab = np.where(np.arange(E) % 2 == 0, np.arange(E) // 2, -1).astype(np.int32)
    else:
        devtab = np.full(E, -1, np.int32)
    d_lg, d_tab = dev(lg), dev(devtab)
    es = torch.full((T, 64), -9, dtype=torch.int32, device="cuda")
    ew = torch.zeros((T, 64), dtype=torch.float32, device="cuda")
    nh = torch.full((T,), -9, dtype=torch.int32, device="cuda")
    mail = torch.zeros(1280, dtype=torch.uint8, device="cuda")
    seq = torch.tensor([41], dtype=torch.uint64, device="cuda")
    rseq = torch.tensor([7], dtype=torch.uint64, device="cuda")
    prof = torch.zeros(2, dtype=torch.uint64, device="cuda")
    P = q4mi.ptr
    for call in range(2):
        q4mi.check(L.q4_hip_route_dev_n(P(d_lg), P(d_tab), P(es), P(ew), P(nh), P(mail), P(seq),
                                        P(rseq), P(prof), E, k, T), "q4_hip_route_dev_n")
    es_h, ew_h, nh_h = host(es), host(ew), host(nh)
    m = mail_fields(host(mail)[:MAIL_BYTES])
    oid, ow = oracle.softmax_topk(lg, k)
    assert m["seq"] == 43 and m["rseq"] == 9 and int(host(prof)[1]) == 2
    assert m["ntok"] == T
    miss_ids, miss_w, miss_rk = [], [], []
    for t in range(T):
        slots = devtab[oid[t]]
        hit = slots >= 0
        nhit = int(hit.sum())
        assert nh_h[t] == nhit and m["hn"][t] == nhit and m["tn"][t] == k - nhit
        assert np.array_equal(es_h[t, :nhit], slots[hit])
        assert np.array_equal(m["hs"][16 * t:16 * t + nhit], slots[hit])
        assert np.allclose(ew_h[t, :nhit], ow[t][hit], rtol=1e-6, atol=1e-9)
        assert np.all(es_h[t, nhit:] == -9)                     # nothing past the hits
        miss_ids += list(oid[t][~hit])
        miss_w += list(ow[t][~hit])
        miss_rk += list(np.nonzero(~hit)[0])
    n = len(miss_ids)
    assert m["n"] == n
    assert np.array_equal(m["ids"][:n], np.array(miss_ids, np.int32))
    assert np.allclose(m["wts"][:n], np.array(miss_w, np.float32), rtol=1e-6, atol=1e-9)
    assert np.array_equal(m["rk"][:n], np.array(miss_rk, np.uint8))
    assert np.all(m["tn"][T:] == 0) and np.all(m["hn"][T:] == 0)
    assert np.array_equal(m["routed"][:k], oid[0]) and np.all(m["routed"][k:] == 0)


def test_route_dev_n_rejects(gpu):
    """The reference's bounds: n_tok * topk <= 64, topk <= 16, n_exp <= 1024,
    n_tok <= 8 -> false before any launch."""
    import torch
    L = gpu
    z = torch.zeros(8 * 2048, dtype=torch.float32, device="cuda")
    P = q4mi.ptr
    for E, k, T in ((512, 10, 7), (512, 17, 1), (1025, 4, 1), (512, 4, 9), (512, 0, 1)):
        assert not L.q4_hip_route_dev_n(P(z), P(z), P(z), P(z), P(z), P(z), P(z), None, None,
                                        E, k, T)
