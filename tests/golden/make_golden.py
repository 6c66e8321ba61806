"""Write golden vectors from the reference's own CPU expert path.

Runs where /root/reference exists and oracle/_ref/libq4ref.so was built
(`make -C oracle ref`).  Inputs come from the seeded generators in
q4mi.synth; each fixture stores the seeds, a SHA-256 of the generated input
bytes (so a generator change is detected) and the reference outputs.
Output: tests/golden/reference_vectors.npz (data only).
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "oracle"), os.path.join(ROOT, "suzuku-engine-q4_amd")]
import oracle as om  # noqa: E402
from q4mi import synth  # noqa: E402


def sha(*arrs):
    h = hashlib.sha256()
    for a in arrs:
        h.update(np.ascontiguousarray(a).tobytes())
    return np.frombuffer(h.digest(), np.uint8)


def main():
    ref = om.Ref()
    out = {}
    # q8 quantizer, with zero groups and exact .5 ties
    rng = np.random.default_rng(101)
    x = (rng.standard_normal(4096) * rng.choice([1e-3, 1, 40], 4096)).astype(np.float32)
    x[0:32] = 0
    x[32:64] = np.arange(32) - 16.5
    x[63] = 127
    q, d, bs = ref.quant8(x)
    out.update(q8_x=x, q8_q=q, q8_d=d, q8_bs=bs)
    # row dots: (type, K, nt, seed)
    cases = [(om.T_IQ3_S, 4096, 1, 201), (om.T_IQ3_S, 2048, 4, 202), (om.T_IQ3_S, 512, 2, 203),
             (om.T_Q8_0, 2048, 1, 204), (om.T_Q8_0, 2048, 4, 205)]
    for i, (ty, K, nt, seed) in enumerate(cases):
        rng = np.random.default_rng(seed)
        w = synth.matrix(rng, ty, 16, K)
        xx = rng.standard_normal((nt, K)).astype(np.float32)
        out["dot%d_case" % i] = np.array([ty, K, nt, seed, 16], np.int64)
        out["dot%d_sha" % i] = sha(w, xx)
        out["dot%d_y" % i] = ref.dot8_rows(ty, w, 16, K, xx)
    # routing (softmax + top-10 + renorm), Zipf-biased, with a planted tie
    rng = np.random.default_rng(301)
    lg = synth.logits(rng, 24, 512, zipf=True)
    lg[0, 7] = lg[0, 300] = 40.0
    ids, wts = ref.softmax_topk(lg, 10)
    out.update(route_logits=lg, route_ids=ids, route_wts=wts)
    # decode MoE job and a 4-token window (small experts)
    n_embd, n_ff, E = 512, 256, 12
    rng = np.random.default_rng(401)
    arena = synth.expert_arena(rng, E, n_embd, n_ff)
    stride = synth.expert_stride(n_embd, n_ff)[0]
    xd = rng.standard_normal(n_embd).astype(np.float32)
    dids = np.array([4, 11, 0, 7, 2], np.int32)
    dw = np.array([0.35, 0.25, 0.2, 0.15, 0.05], np.float32)
    out["moe_shape"] = np.array([n_embd, n_ff, E, 401], np.int64)
    out["moe_sha"] = sha(arena)
    out.update(moe_x=xd, moe_ids=dids, moe_wts=dw,
               moe_y=ref.moe_decode(n_embd, n_ff, om.T_IQ3_S, om.T_IQ3_S, E, arena, stride,
                                    xd, dids, dw))
    xw = rng.standard_normal((4, n_embd)).astype(np.float32)
    wids = np.array([[1, 2, 3], [2, 5, 9], [10, 1, 6], [0, 11, 2]], np.int32)
    ww = rng.random((4, 3)).astype(np.float32)
    out.update(win_x=xw, win_ids=wids, win_wts=ww,
               win_y=ref.moe_win(n_embd, n_ff, om.T_IQ3_S, om.T_IQ3_S, E, arena, stride, xw,
                                 wids, ww, np.full(4, 3, np.uint32)))
    # the other weight formats: dequantized rows (all four) and int8 row
    # dots (the three with a reference CPU int8 kernel)
    for ty in (om.T_IQ4_NL, om.T_Q2_0, om.T_IQ2_S, om.T_Q6_K):
        rng = np.random.default_rng(500 + ty)
        K = 1024
        w = synth.matrix(rng, ty, 6, K)
        rb = om.row_bytes(ty, K)
        out["fmt%d_sha" % ty] = sha(w)
        out["fmt%d_deq" % ty] = np.stack([ref.dequant_row(ty, w[r * rb:(r + 1) * rb], K)
                                          for r in range(6)])
        if ty != om.T_Q6_K:
            xx = rng.standard_normal((3, K)).astype(np.float32)
            out["fmt%d_x" % ty] = xx
            out["fmt%d_y" % ty] = ref.dot8_rows(ty, w, 6, K, xx)
    # the router GEMV (q4_gemv) on F32 and BF16 rows
    rng = np.random.default_rng(601)
    wr = (rng.standard_normal((32, 512)) * 0.05).astype(np.float32)
    xr = rng.standard_normal(512).astype(np.float32)
    wb = (wr.view(np.uint32) >> 16).astype(np.uint16)
    out.update(router_w=wr, router_x=xr, router_f32=ref.gemv(0, wr, 32, 512, xr),
               router_bf16=ref.gemv(30, wb.view(np.uint8), 32, 512, xr))
    path = os.path.join(HERE, "reference_vectors.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
