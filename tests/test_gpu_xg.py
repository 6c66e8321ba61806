"""GPU parity for the XG (fp16-activation) prefill GEMMs q4_xg_gu / q4_xg_dn
(the reference's q4_xg A/B, src/q4_xg.cu) against the C oracle's XG layer
(or_xg_tokens: the same fp16 weight and activation rounding, exact products
summed in double).

Bars, per launch:
- q4_xg_gu: every h16 value is the oracle's h rounded to fp16 or its
  neighbour (the GPU sums in fp32 MFMA order, the oracle in double, so h may
  cross an fp16 rounding boundary) or, for h near zero (cancelling sums),
  within 1e-5 of the row's largest |h|; at most 1% of them differ from the
  oracle's rounding;
- q4_xg_dn: the down rows fed with the GPU's own h16, max rel error <= 1e-3;
- the layer: max rel error <= 1e-3 against the oracle's down path on the
  GPU's h16, and normwise <= 1e-3 against the oracle's own XG layer.
The synthetic activations are scaled by 0.05 so that h stays inside fp16's
range with these weights (|h| would otherwise reach ~1e5 > 65504)."""
import numpy as np
import pytest

from conftest import rel_err

import oracle as om
import q4mi
from q4mi import synth

pytestmark = pytest.mark.gpu
T_IQ3_S, T_Q8_0 = q4mi.T_IQ3_S, q4mi.T_Q8_0

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


def packed(rng, E, H, F, tg, td):
    """Packed experts gate | up | down with gate/up type tg, down type td."""
    g = synth.matrix(rng, tg, E * F, H)
    u = synth.matrix(rng, tg, E * F, H)
    d = synth.matrix(rng, td, E * H, F)
    gs, ds = F * om.row_bytes(tg, H), H * om.row_bytes(td, F)
    arena = np.concatenate([np.concatenate([g[e * gs:(e + 1) * gs], u[e * gs:(e + 1) * gs],
                                            d[e * ds:(e + 1) * ds]]) for e in range(E)])
    return arena, 2 * gs + ds, 0, gs, 2 * gs


@pytest.mark.parametrize("ty,td", [(T_IQ3_S, T_IQ3_S), (T_Q8_0, T_Q8_0), (22, 20), (22, 42),
                                   (T_IQ3_S, 22)])
def test_xg_layer_matches_oracle(gpu, oracle, ty, td):
    import torch
    E, H, F, T, k = 48, 2048, 512, 384, 6
    rng = np.random.default_rng(70 + ty + td)
    if ty == td:
        arena = synth.expert_arena(rng, E, H, F, ty)
        stride, og, ou, od = synth.expert_stride(H, F, ty)
    else:
        arena, stride, og, ou, od = packed(rng, E, H, F, ty, td)
    x = (rng.standard_normal((T, H)) * 0.05).astype(np.float32)
    lg = synth.logits(rng, T, E, zipf=True)
    ids, wts = oracle.softmax_topk(lg, k)
    pk = oracle.pack(ids, wts, E, T)
    rows = T * k
    tiles = np.zeros(4 * (rows // 128 + E), np.int32)
    ek = pk["ek"][:E].astype(np.uint32)
    ebase = pk["bounds"][:E].astype(np.uint32)
    slot = np.arange(E, dtype=np.int32)
    assert gpu.q4_xg_shape_ok(H, F) and gpu.q4_xg_gu_type(ty) and gpu.q4_xg_dn_type(td)
    cap = gpu.q4_xg_tile_cap(rows, E)
    nt = gpu.q4_xg_tiles(ek.ctypes.data, ebase.ctypes.data, slot.ctypes.data, E,
                         tiles.ctypes.data, cap)
    assert nt > 0
    P = q4mi.ptr
    d_arena, dx, d_tiles = dev(arena), dev(x), dev(tiles[:4 * nt])
    x16 = zeros((T, H), torch.float16)
    h16 = zeros((rows, F), torch.float16)
    pd = zeros((rows, H))
    y = zeros((T, H))
    q4mi.check(gpu.q4_xg_cvt(P(dx), P(x16), T * H), "q4_xg_cvt")
    q4mi.check(gpu.q4_xg_gu(ty, P(d_arena), stride, og, ou, H, F, P(d_tiles), nt, P(x16),
                            P(dev(pk["a_tok"][:rows])), P(h16)), "q4_xg_gu")
    q4mi.check(gpu.q4_xg_dn(td, P(d_arena), stride, od, F, H, P(d_tiles), nt, P(h16), P(pd)),
               "q4_xg_dn")
    q4mi.check(gpu.q4_hip_expert_reduce(P(y), P(pd), P(dev(pk["rsrc"])), P(dev(pk["rw"])), T, k,
                                        H), "reduce")
    assert np.array_equal(host(x16), x.astype(np.float16))
    h16g = host(h16).astype(np.float32)
    pdg = host(pd)
    yg = host(y)
    samp = np.concatenate([[0, T - 1], rng.choice(np.arange(1, T - 1), 30, replace=False)])
    rsrc = pk["rsrc"].reshape(T, k)
    nh = nflip = 0
    yc = np.zeros((len(samp), H), np.float32)
    tok_flips = np.zeros(len(samp), np.int64)
    for si, t in enumerate(samp):
        for j in range(k):
            e, p = int(ids[t, j]), int(rsrc[t, j])
            pe = arena[e * stride:(e + 1) * stride]
            ho = oracle.xg_gu_row(H, F, ty, pe, x[t])
            # h16 is the oracle's h rounded to fp16, or its fp16 neighbour
            r16 = ho.astype(np.float16)
            up = np.nextafter(r16, np.float16(np.inf)).astype(np.float32)
            dn = np.nextafter(r16, np.float16(-np.inf)).astype(np.float32)
            g = h16g[p]
            exact = g == r16.astype(np.float32)
            # near-zero h come from cancelling sums: there the fp32 sum
            # error, not the fp16 step, bounds the difference
            near = np.abs(g - ho) <= 1e-5 * np.abs(ho).max()
            assert np.all(exact | (g == up) | (g == dn) | near), (t, j)
            nh += F
            nflip += int(np.count_nonzero(~exact))
            tok_flips[si] += int(np.count_nonzero(~exact))
            # the down launch on the GPU's own h16
            pdo = oracle.xg_dn_row(F, H, td, pe[od:], g)
            assert rel_err(pdg[p], pdo) <= 1e-3, (t, j)
            yc[si] = yc[si] + np.float32(wts[t, j]) * pdo
    print("xg h16 values off by one fp16 step: %d of %d" % (nflip, nh))
    assert nflip <= 0.01 * nh
    # the layer output against the oracle's down path on those h16 (a step
    # of h16 moves y by more than the bar wherever y is small, so the end to
    # end comparison with the oracle's own h16 is reported, not asserted)
    assert rel_err(yg[samp], yc) <= 1e-3
    yo = oracle.xg_tokens(H, F, ty, td, arena, stride, x[samp], ids[samp], wts[samp])
    print("xg layer vs oracle xg layer (own h16 rounding): max rel %.3g, normwise %.3g"
          % (rel_err(yg[samp], yo), np.abs(yg[samp] - yo).max() / np.abs(yo).max()))
    assert np.abs(yg[samp] - yo).max() <= 1e-3 * np.abs(yo).max()
    # elementwise: a token whose h16 all round as the oracle's is within the
    # 1e-3 bar of it; a token with an fp16 step in h moves by that step's
    # weight only (measured max rel 0.026 over the sampled tokens; bar 0.05)
    clean = tok_flips == 0
    if clean.any():
        assert rel_err(yg[samp][clean], yo[clean]) <= 1e-3
    assert rel_err(yg[samp], yo) <= 0.05
    print("xg tokens without an h16 step: %d of %d" % (int(clean.sum()), len(samp)))
    # the A/B: the q8 path's layer on the same input differs by the q8
    # quantization of x and h (reported, loosely bounded)
    yq = oracle.moe_tokens(H, F, ty, td, arena, stride, x[samp], ids[samp], wts[samp], mode=1)
    nw = np.abs(yg[samp] - yq).max() / np.abs(yq).max()
    print("xg vs q8 layer: normwise %.3g" % nw)
    assert nw <= 0.05


def test_xg_rejects(gpu):
    assert not gpu.q4_xg_shape_ok(2048, 500)
    assert not gpu.q4_xg_gu_type(20) and not gpu.q4_xg_dn_type(14)
    assert gpu.q4_xg_tiles(None, None, None, 0, None, 0) == 0


def test_xg_rejects_bad_tile_records(gpu):
    """A caller's XG tile record with more rows than the 128-row tile, a
    negative slot or a negative first row is skipped on the device (its rows
    are not written) and reported by q4mi_device_status; the valid records of
    the same table still run."""
    import torch
    P = q4mi.ptr
    H, F = 2048, 512
    rng = np.random.default_rng(12)
    arena = synth.expert_arena(rng, 2, H, F)
    stride, og, ou, od = synth.expert_stride(H, F)
    d_arena = dev(arena)
    rows = 64
    h16 = torch.from_numpy((rng.standard_normal((rows, F)) * 0.05).astype(np.float16)).cuda()
    pd = torch.full((rows, H), 7.0, dtype=torch.float32, device="cuda")
    assert gpu.q4mi_device_status(1) == 0
    # record 0 valid (rows 0..31 of slot 1), then bad records: 200 rows,
    # slot -1, first row -5
    tiles = np.array([0, 32, 1, 1, 32, 200, 0, 0, 32, 8, -1, 0, -5, 8, 0, 0], np.int32)
    d_tiles = dev(tiles)
    q4mi.check(gpu.q4_xg_dn(q4mi.T_IQ3_S, P(d_arena), stride, od, F, H, P(d_tiles), 4, P(h16),
                            P(pd)), "q4_xg_dn")
    out = host(pd)
    st = gpu.q4mi_device_status(1)
    assert st & 4, st
    assert "XG tile record" in q4mi.last_error()
    assert np.all(out[32:] == 7.0)              # the rejected records wrote nothing
    assert np.all(np.isfinite(out[:32])) and not np.all(out[:32] == 7.0)
    assert gpu.q4mi_device_status(1) == 0       # cleared
