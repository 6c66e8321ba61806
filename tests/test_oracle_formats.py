"""The oracle's other weight formats (IQ4_NL, Q2_0, IQ2_S, Q6_K, IQ2_XXS,
IQ2_XS, IQ3_XXS, IQ4_XS) pinned against the reference's own code compiled
from source (oracle/_ref): dequantization bit for bit against
q4_dequant_row; the int8 row dot bit for bit against the CPU expert kernels
(dq8_iq4_nl, dq8_q2_0, dq8_iq2_s, dq8_iq2_xxs, dq8_iq2_xs, dq8_iq3_xxs,
dq8_iq4_xs); and
the exact integer group sums against the dequantized values (d * S_g equals
sum_i v_i q_i in exact arithmetic)."""
import numpy as np
import pytest

import oracle as om
from q4mi import synth

IQXX = [om.T_IQ2_XXS, om.T_IQ2_XS, om.T_IQ3_XXS, om.T_IQ4_XS]
FMTS = [om.T_IQ4_NL, om.T_Q2_0, om.T_IQ2_S, om.T_Q6_K] + IQXX
CPU_Q8 = [om.T_IQ4_NL, om.T_Q2_0, om.T_IQ2_S] + IQXX   # types with a reference int8 CPU kernel
# the fp16 block scale's factor in the value (d * factor * multiplier * integer)
DFAC = {om.T_IQ2_S: 0.125, om.T_IQ2_XXS: 0.125, om.T_IQ2_XS: 0.125, om.T_IQ3_XXS: 0.25}


@pytest.mark.parametrize("ty", FMTS)
def test_dequant_matches_reference(oracle, ref, ty):
    rng = np.random.default_rng(ty)
    n = 2048
    w = synth.matrix(rng, ty, 5, n)
    rb = om.row_bytes(ty, n)
    for r in range(5):
        a = oracle.dequant_row(ty, w[r * rb:(r + 1) * rb], n)
        b = ref.dequant_row(ty, w[r * rb:(r + 1) * rb], n)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), r


@pytest.mark.parametrize("ty", CPU_Q8)
@pytest.mark.parametrize("nt", [1, 3, 8])
def test_dot8_matches_reference(oracle, ref, ty, nt):
    rng = np.random.default_rng(ty * 10 + nt)
    rows, n = 37, 1024
    w = synth.matrix(rng, ty, rows, n)
    x = (rng.standard_normal((nt, n)) * rng.choice([1e-3, 1, 30], (nt, n))).astype(np.float32)
    a = oracle.dot8_rows(ty, w, rows, n, x)
    b = ref.dot8_rows(ty, w, rows, n, x)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("ty", FMTS)
def test_group_sums_exact(oracle, ty):
    rng = np.random.default_rng(100 + ty)
    n = 1024
    w = synth.matrix(rng, ty, 4, n)
    rb = om.row_bytes(ty, n)
    x = rng.standard_normal(n).astype(np.float32)
    q, d, _ = oracle.quant8(x)
    for r in range(4):
        row = w[r * rb:(r + 1) * rb]
        s = oracle.group_sums(ty, row, n, q)
        v = oracle.dequant_row(ty, row, n).astype(np.float64)
        vals, nb, doff = synth.BLOCKS[ty]
        blk = row.reshape(-1, nb)
        dscale = blk[:, doff:doff + 2].copy().view(np.float16).astype(np.float64).ravel()
        per_group = np.repeat(dscale, vals // 32) * DFAC.get(ty, 1.0)
        exact = (v * q.astype(np.float64)).reshape(-1, 32).sum(1)
        got = per_group * s.astype(np.float64)
        if ty == om.T_Q6_K:   # fp32 value d*sc*(q-32) may round (25 bits)
            assert np.allclose(got, exact, rtol=0, atol=1e-6 * np.abs(v).max() * 127 * 32)
        else:
            assert np.array_equal(got, exact)


def test_q2_0_zero_codes_and_known_values(oracle):
    """Q2_0 known answer: codes 1 everywhere give value 0 (c - 1); codes 3
    give +2d; code 0 gives -d."""
    b = np.zeros(18, np.uint8)
    b[0:2] = np.array([0.5], np.float16).view(np.uint8)
    b[2:] = 0x55                                    # all codes 1
    assert np.all(oracle.dequant_row(om.T_Q2_0, b, 64) == 0)
    b[2:] = 0xFF                                    # all codes 3
    assert np.all(oracle.dequant_row(om.T_Q2_0, b, 64) == 1.0)
    b[2:] = 0x00
    assert np.all(oracle.dequant_row(om.T_Q2_0, b, 64) == -0.5)


def _arena(rng, E, H, F, tg, td):
    g = synth.matrix(rng, tg, E * F, H)
    u = synth.matrix(rng, tg, E * F, H)
    d = synth.matrix(rng, td, E * H, F)
    gs, ds = F * om.row_bytes(tg, H), H * om.row_bytes(td, F)
    arena = np.concatenate([np.concatenate([g[e * gs:(e + 1) * gs], u[e * gs:(e + 1) * gs],
                                            d[e * ds:(e + 1) * ds]]) for e in range(E)])
    return arena, 2 * gs + ds


@pytest.mark.parametrize("tg", IQXX)
def test_moe_window_formats_vs_reference(oracle, ref, tg):
    """The oracle's verify-window layer with IQ2_XXS / IQ2_XS / IQ3_XXS /
    IQ4_XS gate/up (the reference window's gate/up formats, win_iq_bb
    src/q4_rocm.cu:7333-7343) and IQ4_NL down against the reference's own
    q4_cpuex_dispatch_win on the same arena."""
    from conftest import rel_err
    rng = np.random.default_rng(300 + tg)
    H, F, E, T, k = 512, 256, 12, 4, 4
    arena, stride = _arena(rng, E, H, F, tg, om.T_IQ4_NL)
    x = rng.standard_normal((T, H)).astype(np.float32)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    wts = rng.random((T, k)).astype(np.float32)
    yr = ref.moe_win(H, F, tg, om.T_IQ4_NL, E, arena, stride, x, ids, wts,
                     np.full(T, k, np.uint32))
    yo = oracle.moe_tokens(H, F, tg, om.T_IQ4_NL, arena, stride, x, ids, wts)
    assert np.abs(yr).max() > 0
    # (the reference's pool splits the layer's jobs over threads; a q8(h) code
    # at a rounding boundary may differ, ~1e-5 of the output norm)
    assert rel_err(yo, yr) < 1e-4
