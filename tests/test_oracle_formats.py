"""The oracle's other weight formats (IQ4_NL, Q2_0, IQ2_S, Q6_K) pinned
against the reference's own code compiled from source (oracle/_ref):
dequantization bit for bit against q4_dequant_row; the int8 row dot bit for
bit against the CPU expert kernels (dq8_iq4_nl, dq8_q2_0, dq8_iq2_s); and
the exact integer group sums against the dequantized values (d * S_g equals
sum_i v_i q_i in exact arithmetic)."""
import numpy as np
import pytest

import oracle as om
from q4mi import synth

FMTS = [om.T_IQ4_NL, om.T_Q2_0, om.T_IQ2_S, om.T_Q6_K]
CPU_Q8 = [om.T_IQ4_NL, om.T_Q2_0, om.T_IQ2_S]   # types with a reference int8 CPU kernel


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
        per_group = np.repeat(dscale, vals // 32) * (0.125 if ty == om.T_IQ2_S else 1.0)
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
