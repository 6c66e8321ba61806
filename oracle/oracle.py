"""ctypes bindings for the checkers (TEST INFRASTRUCTURE ONLY).

`Oracle` wraps build/liboracle.so, this repo's plain-C restatement of the
reference path (oracle/q4_oracle.c).  `Ref` wraps _ref/libq4ref.so, the
reference's own CPU expert path compiled from its sources (oracle/Makefile
`ref`); it exists only where that build was made.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, as the thing results are checked against or timed beside.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
T_Q8_0 = 8
T_Q6_K = 14
T_IQ2_XXS = 16
T_IQ2_XS = 17
T_IQ3_XXS = 18
T_IQ4_NL = 20
T_IQ3_S = 21
T_IQ2_S = 22
T_IQ4_XS = 23
T_Q2_0 = 42

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_i8p = ctypes.POINTER(ctypes.c_int8)
_u8p = ctypes.POINTER(ctypes.c_uint8)


def _p(a, t):
    return a.ctypes.data_as(t)


_BLOCK = {T_IQ3_S: (256, 110), T_Q8_0: (32, 34), T_IQ4_NL: (32, 18), T_Q2_0: (64, 18),
          T_IQ2_S: (256, 82), T_Q6_K: (256, 210), T_IQ2_XXS: (256, 66), T_IQ2_XS: (256, 74),
          T_IQ3_XXS: (256, 98), T_IQ4_XS: (256, 136)}


def row_bytes(ty, n):
    if ty not in _BLOCK:
        raise ValueError(ty)
    vals, nb = _BLOCK[ty]
    return n // vals * nb


class Oracle:
    def __init__(self, path=None):
        path = path or os.path.join(HERE, "build", "liboracle.so")
        if not os.path.exists(path):
            raise FileNotFoundError(path + " (run: make -C oracle)")
        self.L = ctypes.CDLL(path)
        L = self.L
        L.or_f16_to_f32.restype = ctypes.c_float
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_quant8.argtypes = [_f32p, ctypes.c_uint64, _i8p, _f32p, _i32p]
        L.or_dequant_row.argtypes = [ctypes.c_uint32, _u8p, ctypes.c_uint64, _f32p]
        L.or_group_sums.argtypes = [ctypes.c_uint32, _u8p, ctypes.c_uint64, _i8p, _i32p]
        L.or_dot8.restype = ctypes.c_float
        L.or_dot8.argtypes = [ctypes.c_uint32, _u8p, ctypes.c_uint64, _i8p, _f32p]
        L.or_dot8_rows.argtypes = [ctypes.c_uint32, _u8p, ctypes.c_uint64, ctypes.c_uint64,
                                   _f32p, ctypes.c_uint32, _f32p]
        L.or_dot8q_rows.argtypes = [ctypes.c_uint32, _u8p, ctypes.c_uint64, ctypes.c_uint64,
                                    _i8p, _f32p, ctypes.c_uint32, _f32p]
        L.or_xg_tokens.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                   ctypes.c_uint32, _u8p, ctypes.c_uint64, _f32p,
                                   ctypes.c_uint32, _i32p, _f32p, ctypes.c_uint32, _f32p]
        L.or_f16_bits.restype = ctypes.c_uint16
        L.or_f16_bits.argtypes = [ctypes.c_float]
        L.or_xg_dequant_row.argtypes = [ctypes.c_uint32, _u8p, ctypes.c_uint64, _f32p]
        L.or_xg_gu_row.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, _u8p,
                                   _f32p, _f32p]
        L.or_xg_dn_row.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, _u8p,
                                   _f32p, _f32p]
        L.or_router.argtypes = [ctypes.c_uint32, _u8p, ctypes.c_uint32, ctypes.c_uint32, _f32p,
                                ctypes.c_uint32, _f32p, _f32p, _f32p]
        L.or_softmax_topk.argtypes = [_f32p, ctypes.c_uint32, ctypes.c_uint32, _i32p, _f32p]
        L.or_pack.argtypes = [_i32p, _f32p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                              ctypes.c_uint32, _i32p, _i32p, _f32p, _u32p, _i32p, _u32p, _i32p]
        L.or_moe_tokens.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                    ctypes.c_uint32, _u8p, ctypes.c_uint64, _f32p,
                                    ctypes.c_uint32, _i32p, _f32p, ctypes.c_uint32, _f32p,
                                    ctypes.c_int, _f32p]

    def quant8(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        n = x.size
        q = np.empty(n, np.int8)
        d = np.empty(n // 32, np.float32)
        bs = np.empty(n // 32, np.int32)
        self.L.or_quant8(_p(x, _f32p), n, _p(q, _i8p), _p(d, _f32p), _p(bs, _i32p))
        return q, d, bs

    def dequant_row(self, ty, w, n):
        w = np.ascontiguousarray(w, dtype=np.uint8)
        y = np.empty(n, np.float32)
        assert self.L.or_dequant_row(ty, _p(w, _u8p), n, _p(y, _f32p))
        return y

    def group_sums(self, ty, w_row, n, q):
        w_row = np.ascontiguousarray(w_row, dtype=np.uint8)
        q = np.ascontiguousarray(q, dtype=np.int8)
        s = np.empty(n // 32, np.int32)
        assert self.L.or_group_sums(ty, _p(w_row, _u8p), n, _p(q, _i8p), _p(s, _i32p))
        return s

    def dot8_rows(self, ty, w, rows, n, x):
        """x: [nt, n] fp32 -> y [nt, rows]"""
        x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.uint8)
        nt = x.shape[0]
        y = np.empty((nt, rows), np.float32)
        assert self.L.or_dot8_rows(ty, _p(w, _u8p), rows, n, _p(x, _f32p), nt, _p(y, _f32p))
        return y

    def dot8q_rows(self, ty, w, rows, n, q, d):
        """Rows of w dotted with pre-quantized activations: q [nt, n] codes,
        d [nt, n/32] scales -> y [nt, rows]."""
        q = np.ascontiguousarray(np.atleast_2d(q), dtype=np.int8)
        d = np.ascontiguousarray(np.atleast_2d(d), dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.uint8)
        nt = q.shape[0]
        y = np.empty((nt, rows), np.float32)
        assert self.L.or_dot8q_rows(ty, _p(w, _u8p), rows, n, _p(q, _i8p), _p(d, _f32p), nt,
                                    _p(y, _f32p))
        return y

    def router(self, ty, w, n_exp, K, x, sgw=None):
        """Router logits [T, n_exp] (and the shared-expert gate sg [T] when
        sgw is given) in the library's fixed dot order."""
        x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
        w = np.ascontiguousarray(w).view(np.uint8).reshape(-1)
        T = x.shape[0]
        lg = np.empty((T, n_exp), np.float32)
        sg = np.empty(T, np.float32)
        g = None if sgw is None else np.ascontiguousarray(sgw, dtype=np.float32)
        assert self.L.or_router(ty, _p(w, _u8p), n_exp, K, _p(x, _f32p), T,
                                None if g is None else _p(g, _f32p), _p(lg, _f32p),
                                _p(sg, _f32p))
        return (lg, sg) if sgw is not None else lg

    def softmax_topk(self, logits, k):
        logits = np.ascontiguousarray(np.atleast_2d(logits), dtype=np.float32)
        T, n = logits.shape
        ids = np.empty((T, k), np.int32)
        wts = np.empty((T, k), np.float32)
        for t in range(T):
            self.L.or_softmax_topk(_p(logits[t], _f32p), n, k, _p(ids[t], _i32p),
                                   _p(wts[t], _f32p))
        return ids, wts

    def pack(self, ids, wts, n_exp, gsz):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        wts = np.ascontiguousarray(wts, dtype=np.float32)
        T, k = ids.shape
        n_g = (T + gsz - 1) // gsz
        a_tok = np.full(n_g * gsz * k, -7, np.int32)
        rsrc = np.empty(T * k, np.int32)
        rw = np.empty(T * k, np.float32)
        ek = np.empty(n_g * 512, np.uint32)
        stg = np.full(n_g * 512, -7, np.int32)
        stgn = np.empty(n_g, np.uint32)
        bounds = np.empty(n_g * (n_exp + 1), np.int32)
        self.L.or_pack(_p(ids, _i32p), _p(wts, _f32p), T, k, n_exp, gsz, _p(a_tok, _i32p),
                       _p(rsrc, _i32p), _p(rw, _f32p), _p(ek, _u32p), _p(stg, _i32p),
                       _p(stgn, _u32p), _p(bounds, _i32p))
        return dict(a_tok=a_tok, rsrc=rsrc, rw=rw, ek=ek, stg=stg, stgn=stgn, bounds=bounds)

    def xg_dequant_row(self, ty, w, n):
        w = np.ascontiguousarray(w, dtype=np.uint8)
        y = np.empty(n, np.float32)
        self.L.or_xg_dequant_row(ty, _p(w, _u8p), n, _p(y, _f32p))
        return y

    def xg_gu_row(self, n_embd, n_ff, t_gu, expert, x):
        """h = silu(g) * u of one token and expert, before the fp16 rounding."""
        expert = np.ascontiguousarray(expert, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32)
        h = np.empty(n_ff, np.float32)
        assert self.L.or_xg_gu_row(n_embd, n_ff, t_gu, _p(expert, _u8p), _p(x, _f32p),
                                   _p(h, _f32p))
        return h

    def xg_dn_row(self, n_ff, n_embd, t_d, down, h16):
        down = np.ascontiguousarray(down, dtype=np.uint8)
        h16 = np.ascontiguousarray(h16, dtype=np.float32)
        pd = np.empty(n_embd, np.float32)
        assert self.L.or_xg_dn_row(n_ff, n_embd, t_d, _p(down, _u8p), _p(h16, _f32p),
                                   _p(pd, _f32p))
        return pd

    def xg_tokens(self, n_embd, n_ff, t_gu, t_d, arena, stride, x, ids, wts):
        """The XG (fp16-activation) prefill layer, y [T, n_embd] from zero."""
        x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
        ids = np.ascontiguousarray(np.atleast_2d(ids), dtype=np.int32)
        wts = np.ascontiguousarray(np.atleast_2d(wts), dtype=np.float32)
        T, k = ids.shape
        y = np.zeros((T, n_embd), np.float32)
        assert self.L.or_xg_tokens(n_embd, n_ff, t_gu, t_d, _p(arena, _u8p), stride,
                                   _p(x, _f32p), T, _p(ids, _i32p), _p(wts, _f32p), k,
                                   _p(y, _f32p))
        return y

    def moe_tokens(self, n_embd, n_ff, t_gu, t_d, arena, stride, x, ids, wts, mode=0,
                   y_init=None, want_h=False):
        x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
        ids = np.ascontiguousarray(np.atleast_2d(ids), dtype=np.int32)
        wts = np.ascontiguousarray(np.atleast_2d(wts), dtype=np.float32)
        T, k = ids.shape
        y = (np.zeros((T, n_embd), np.float32) if y_init is None
             else np.array(y_init, dtype=np.float32, copy=True))
        h = np.empty((T * k, n_ff), np.float32) if want_h else None
        assert self.L.or_moe_tokens(n_embd, n_ff, t_gu, t_d, _p(arena, _u8p), stride,
                                    _p(x, _f32p), T, _p(ids, _i32p), _p(wts, _f32p), k,
                                    _p(y, _f32p), mode,
                                    _p(h, _f32p) if want_h else None)
        return (y, h) if want_h else y


class Ref:
    """The reference's CPU expert path compiled from source (oracle/_ref)."""

    def __init__(self, path=None):
        path = path or os.path.join(HERE, "_ref", "libq4ref.so")
        if not os.path.exists(path):
            raise FileNotFoundError(path + " (run: make -C oracle ref)")
        self.L = ctypes.CDLL(path)
        L = self.L
        L.qref_quant8.argtypes = [_f32p, ctypes.c_uint64, _i8p, _f32p, _i32p]
        L.qref_dot8_rows.argtypes = [ctypes.c_uint32, _u8p, ctypes.c_uint64, ctypes.c_uint64,
                                     _f32p, ctypes.c_uint32, _f32p, ctypes.c_int]
        L.qref_moe_decode.argtypes = [ctypes.c_uint32] * 5 + [_u8p, ctypes.c_uint64, _f32p,
                                                              _i32p, _f32p, ctypes.c_uint32,
                                                              _f32p]
        L.qref_moe_win.argtypes = [ctypes.c_uint32] * 5 + [_u8p, ctypes.c_uint64, _f32p,
                                                           ctypes.c_uint32, _i32p, _f32p,
                                                           _u32p, _f32p]
        L.qref_softmax_topk.argtypes = [_f32p, ctypes.c_uint32, ctypes.c_uint32, _i32p, _f32p]
        L.q4_dequant_row.restype = ctypes.c_bool
        L.q4_dequant_row.argtypes = [ctypes.c_uint32, _u8p, ctypes.c_uint64, _f32p]
        L.q4_gemv.restype = ctypes.c_bool
        L.q4_gemv.argtypes = [ctypes.c_uint32, _u8p, ctypes.c_uint64, ctypes.c_uint64, _f32p,
                              _f32p, ctypes.c_float]

    def quant8(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        n = x.size
        q = np.empty(n, np.int8)
        d = np.empty(n // 32, np.float32)
        bs = np.empty(n // 32, np.int32)
        assert self.L.qref_quant8(_p(x, _f32p), n, _p(q, _i8p), _p(d, _f32p), _p(bs, _i32p))
        return q, d, bs

    def dot8_rows(self, ty, w, rows, n, x, threads=1):
        x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.uint8)
        nt = x.shape[0]
        y = np.empty((nt, rows), np.float32)
        assert self.L.qref_dot8_rows(ty, _p(w, _u8p), rows, n, _p(x, _f32p), nt,
                                     _p(y, _f32p), threads)
        return y

    def moe_decode(self, n_embd, n_ff, t_gu, t_d, n_exp, arena, stride, x, ids, wts):
        x = np.ascontiguousarray(x, dtype=np.float32)
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        wts = np.ascontiguousarray(wts, dtype=np.float32)
        y = np.empty(n_embd, np.float32)
        assert self.L.qref_moe_decode(n_embd, n_ff, t_gu, t_d, n_exp, _p(arena, _u8p), stride,
                                      _p(x, _f32p), _p(ids, _i32p), _p(wts, _f32p), ids.size,
                                      _p(y, _f32p))
        return y

    def moe_win(self, n_embd, n_ff, t_gu, t_d, n_exp, arena, stride, x, ids, wts, tn):
        x = np.ascontiguousarray(x, dtype=np.float32)
        ids = np.ascontiguousarray(ids, dtype=np.int32).ravel()
        wts = np.ascontiguousarray(wts, dtype=np.float32).ravel()
        tn = np.ascontiguousarray(tn, dtype=np.uint32)
        n_tok = x.shape[0]
        y = np.empty((n_tok, n_embd), np.float32)
        assert self.L.qref_moe_win(n_embd, n_ff, t_gu, t_d, n_exp, _p(arena, _u8p), stride,
                                   _p(x, _f32p), n_tok, _p(ids, _i32p), _p(wts, _f32p),
                                   _p(tn, _u32p), _p(y, _f32p))
        return y

    def dequant_row(self, ty, w, n):
        """The reference's float dequantizer (q4_dequant_row)."""
        w = np.ascontiguousarray(w).view(np.uint8).reshape(-1)
        y = np.empty(n, np.float32)
        assert self.L.q4_dequant_row(ty, _p(w, _u8p), n, _p(y, _f32p))
        return y

    def gemv(self, ty, w, rows, cols, x):
        """The reference's float GEMV q4_gemv (src/q4_quant.c:595-622): the
        router logits of its CPU path."""
        w = np.ascontiguousarray(w).view(np.uint8).reshape(-1)
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.zeros(rows, np.float32)
        assert self.L.q4_gemv(ty, _p(w, _u8p), rows, cols, _p(x, _f32p), _p(y, _f32p), 1.0)
        return y

    def softmax_topk(self, logits, k):
        logits = np.ascontiguousarray(np.atleast_2d(logits), dtype=np.float32)
        T, n = logits.shape
        ids = np.empty((T, k), np.int32)
        wts = np.empty((T, k), np.float32)
        for t in range(T):
            self.L.qref_softmax_topk(_p(logits[t], _f32p), n, k, _p(ids[t], _i32p),
                                     _p(wts[t], _f32p))
        return ids, wts


def have_ref():
    return os.path.exists(os.path.join(HERE, "_ref", "libq4ref.so"))
