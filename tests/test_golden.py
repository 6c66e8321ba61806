"""The oracle against golden vectors written by the reference's own CPU
expert path (tests/golden/make_golden.py).  Runs without the reference."""
import hashlib
import os

import numpy as np
import pytest

from conftest import GOLDEN, rel_err

import oracle as om
from q4mi import synth

G = np.load(os.path.join(GOLDEN, "reference_vectors.npz"))


def sha(*arrs):
    h = hashlib.sha256()
    for a in arrs:
        h.update(np.ascontiguousarray(a).tobytes())
    return np.frombuffer(h.digest(), np.uint8)


def test_quant8_golden(oracle):
    q, d, bs = oracle.quant8(G["q8_x"])
    assert np.array_equal(q, G["q8_q"])
    assert np.array_equal(d.view(np.uint32), G["q8_d"].view(np.uint32))
    assert np.array_equal(bs, G["q8_bs"])


@pytest.mark.parametrize("i", range(5))
def test_dot_golden(oracle, i):
    ty, K, nt, seed, rows = (int(v) for v in G["dot%d_case" % i])
    rng = np.random.default_rng(seed)
    w = synth.matrix(rng, ty, rows, K)
    x = rng.standard_normal((nt, K)).astype(np.float32)
    assert np.array_equal(sha(w, x), G["dot%d_sha" % i]), "generator changed"
    y = oracle.dot8_rows(ty, w, rows, K, x)
    assert np.array_equal(y.view(np.uint32), G["dot%d_y" % i].view(np.uint32))


def test_routing_golden(oracle):
    ids, wts = oracle.softmax_topk(G["route_logits"], 10)
    assert np.array_equal(ids, G["route_ids"])
    assert np.allclose(wts, G["route_wts"], rtol=1e-6, atol=0)


def test_moe_golden(oracle):
    n_embd, n_ff, E, seed = (int(v) for v in G["moe_shape"])
    rng = np.random.default_rng(seed)
    arena = synth.expert_arena(rng, E, n_embd, n_ff)
    assert np.array_equal(sha(arena), G["moe_sha"]), "generator changed"
    stride = synth.expert_stride(n_embd, n_ff)[0]
    y = oracle.moe_tokens(n_embd, n_ff, om.T_IQ3_S, om.T_IQ3_S, arena, stride, G["moe_x"],
                          G["moe_ids"][None], G["moe_wts"][None])[0]
    assert rel_err(y, G["moe_y"]) < 1e-5
    yw = oracle.moe_tokens(n_embd, n_ff, om.T_IQ3_S, om.T_IQ3_S, arena, stride, G["win_x"],
                           G["win_ids"], G["win_wts"])
    assert rel_err(yw, G["win_y"]) < 1e-5


@pytest.mark.parametrize("ty", [om.T_IQ4_NL, om.T_Q2_0, om.T_IQ2_S, om.T_Q6_K])
def test_formats_golden(oracle, ty):
    """Dequantized rows (bit for bit) and int8 row dots (bit for bit, the
    three formats with a reference CPU int8 kernel) of the other formats."""
    rng = np.random.default_rng(500 + ty)
    K = 1024
    w = synth.matrix(rng, ty, 6, K)
    assert np.array_equal(sha(w), G["fmt%d_sha" % ty]), "generator changed"
    rb = om.row_bytes(ty, K)
    deq = np.stack([oracle.dequant_row(ty, w[r * rb:(r + 1) * rb], K) for r in range(6)])
    assert np.array_equal(deq.view(np.uint32), G["fmt%d_deq" % ty].view(np.uint32))
    if ty != om.T_Q6_K:
        y = oracle.dot8_rows(ty, w, 6, K, G["fmt%d_x" % ty])
        assert np.array_equal(y.view(np.uint32), G["fmt%d_y" % ty].view(np.uint32))


def test_router_golden(oracle):
    """The oracle's fixed-order router dot against the reference's q4_gemv
    (another order): within 1e-5 of each row's sum of |w x|."""
    w, x = G["router_w"], G["router_x"]
    scale = np.abs(w.astype(np.float64)) @ np.abs(x.astype(np.float64))
    lg = oracle.router(0, w, 32, 512, x)[0]
    assert np.all(np.abs(lg - G["router_f32"]) <= 1e-5 * scale)
    wb = (w.view(np.uint32) >> 16).astype(np.uint16)
    lb = oracle.router(30, wb.view(np.uint8), 32, 512, x)[0]
    assert np.all(np.abs(lb - G["router_bf16"]) <= 1e-5 * scale)
