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
