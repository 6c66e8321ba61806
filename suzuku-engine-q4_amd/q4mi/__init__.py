"""Host-side mirror of the reference's routed-expert GPU entry points.

The product is the C-ABI library lib/libq4mi.so (declared in
include/q4mi.h).  This module binds it with ctypes so Python callers and the
tests drive exactly the entry points a C host engine would link: the
reference's q4.h names (q4_hip_moe_exec, q4_hip_moe_exec_win, q4_mmvq_n,
q4_mmq_*, q4_hip_route_pf, q4_hip_assign_pf, q4_hip_expert_reduce, ...)
plus this library's additions (q4mi_*).

Arguments are device pointers (ints) or torch CUDA tensors; PyTorch supplies
device memory and the stream, nothing else.  There is no CPU fallback: if the
library is missing, importing `lib()` raises.
"""
import ctypes
import os

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# Q4MI_LIB selects another build of the same library (same ABI).
LIB_PATH = os.environ.get("Q4MI_LIB") or os.path.join(PKG, "lib", "libq4mi.so")
# The measurement build (-DQ4MI_MEASURE): the same ABI plus the hooks of
# include/q4mi_measure.h.  Benchmarks and LDS-ring tests load it beside the
# product library; its state (stream, scratch) is its own.
MEAS_PATH = os.path.join(PKG, "lib", "libq4mi_meas.so")

T_Q8_0 = 8
T_IQ3_S = 21

_c = ctypes
_vp = _c.c_void_p
_u32 = _c.c_uint32
_u64 = _c.c_uint64
_f32 = _c.c_float
_b = _c.c_bool

# name: (restype, argtypes)
_SIGS = {
    "q4_hip_stream": (_vp, []),
    "q4mi_set_stream": (None, [_vp]),
    "q4mi_last_error": (_c.c_char_p, []),
    "q4mi_device_ok": (_c.c_int, []),
    "q4mi_quant8": (_b, [_vp, _vp, _u64, _u64, _vp, _vp, _vp]),
    "q4_mmvq_on": (_c.c_int, []),
    "q4_mmvq_set": (None, [_c.c_int]),
    "q4_mmvq_verify": (None, [_c.c_int]),
    "q4_mmvq_warm": (None, []),
    "q4_mmvq_hold": (None, [_vp]),
    "q4_mmvq_release": (None, []),
    "q4_mmvq_n": (_b, [_u32, _vp, _u64, _u64, _vp, _vp, _f32, _u32]),
    "q4mi_mmvq": (_b, [_u32, _vp, _u64, _u64, _vp, _vp, _u32, _vp, _f32, _vp]),
    "q4_hip_moe_scratch_warm": (None, []),
    "q4mi_device_status": (_u32, [_c.c_int]),
    "q4mi_status_text": (_c.c_char_p, [_u32]),
    "q4mi_moe_copy_h": (_b, [_vp, _u32]),
    "q4_hip_moe_exec": (_b, [_vp, _u64, _vp, _vp, _u32, _u32, _u64, _u32, _u64, _u32, _u64,
                             _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32]),
    "q4mi_moe_exec_noalloc": (_b, [_vp, _u64, _vp, _vp, _u32, _u32, _u64, _u32, _u64, _u32,
                                   _u64, _vp, _vp, _u32, _u32, _u32]),
    "q4_hip_moe_exec_dev": (_b, [_vp, _u64, _vp, _vp, _vp, _u32, _u64, _u32, _u64, _u32, _u64,
                                 _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32]),
    "q4_hip_moe_win_ok": (_b, [_u32, _u32, _u32, _u32, _u32, _u32]),
    "q4_hip_moe_exec_win": (_b, [_vp, _u64, _vp, _vp, _vp, _u32, _u32, _u64, _u32, _u64, _u32,
                                 _u64, _vp, _vp, _vp, _u32, _u32, _u32]),
    "q4mi_moe_exec_parts": (_b, [_vp, _vp, _vp, _u64, _u64, _vp, _vp, _vp, _u32, _u32, _u32,
                                 _vp, _vp, _u32, _u32, _u32]),
    "q4_hip_moe_tok_ok": (_b, [_u32, _u32, _u32, _u32, _u32]),
    "q4_hip_moe_exec_tok": (_b, [_vp, _u64, _vp, _vp, _vp, _u32, _u32, _u64, _u32, _u64, _u32,
                                 _u64, _vp, _vp, _vp, _vp, _u32, _u32, _u32]),
    "q4_hip_moe_stage": (_b, [_vp, _vp, _u32]),
    "q4_hip_moe_exec_staged": (_b, [_vp, _u64, _u32, _u64, _u32, _u64, _u32, _u64, _vp, _vp,
                                    _vp, _vp, _vp, _u32, _u32, _u32]),
    "q4_hip_route_pf": (_b, [_vp, _vp, _vp, _u32, _u32, _u32]),
    "q4_hip_route_dev_n": (_b, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32]),
    "q4_hip_softmax_topk_launch": (_b, [_vp, _u32, _u32, _vp, _vp]),
    "q4_hip_softmax_topk": (_b, [_vp, _u32, _u32, _vp, _vp]),
    "q4mi_moe_route": (_b, [_vp, _u32, _vp, _vp, _u32, _u32, _u32, _u32, _vp, _vp, _vp, _vp,
                            _u32, _c.c_int32, _vp]),
    "q4mi_moe_route_exec": (_b, [_vp, _u32, _vp, _vp, _u32, _u32, _u32, _vp, _vp, _vp, _vp,
                                 _c.c_int32, _vp, _vp, _u64, _u32, _u64, _u32, _u64, _u32,
                                 _u64, _vp, _u32]),
    "q4_hip_sgate_axpy": (_b, [_vp, _vp, _vp, _vp, _u32, _u32]),
    "q4_hip_dot_sigmoid": (_b, [_vp, _vp, _vp, _u32]),
    "q4mi_assign": (_b, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32]),
    "q4_hip_assign_pf": (_b, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32]),
    "q4_hip_expert_reduce": (_b, [_vp, _vp, _vp, _vp, _u32, _u32, _u32]),
    "q4_mmq_on": (_c.c_int, []),
    "q4_mmq_group": (_u32, []),
    "q4_mmq_supported": (_b, [_u32, _u64]),
    "q4_mmq_q8_bytes": (_u64, [_u64, _u64]),
    "q4_mmq_quantize": (_b, [_vp, _vp, _vp, _u32, _u64, _u64]),
    "q4_mmq_mul_id": (_b, [_vp, _u32, _u64, _u64, _u64, _u32, _vp, _vp, _u32, _u64, _vp, _u64]),
    "q4_mmq_swiglu": (_b, [_vp, _vp, _u64, _u64]),
    "q4_mmq_pad": (_u64, [_u64]),
    "q4_mmq_wbuf": (_b, [_u64, _u64, _u32, _vp, _vp]),
    "q4_mmq_wbuf_lend": (_b, [_vp, _u64, _vp, _u64]),
    "q4_mmq_gather": (_b, [_vp, _u64, _u64, _u64, _u64, _u64, _u64, _u64, _vp, _vp, _u32, _vp,
                           _vp]),
    "q4mi_mmq_mul_id_rows": (_b, [_vp, _u32, _u64, _u64, _u64, _u32, _vp, _u64, _vp, _vp, _u64,
                                  _vp, _u64]),
    "q4mi_mmq_gate_up": (_b, [_vp, _u32, _u64, _u64, _u64, _u32, _vp, _u64, _vp, _vp, _u64,
                              _vp]),
    "q4mi_mmq_gate_up_x": (_b, [_vp, _vp, _u32, _u64, _u64, _u64, _u32, _vp, _u64, _vp, _vp,
                                _u64, _vp]),
    "q4mi_mmq_mul_id_x": (_b, [_vp, _vp, _u32, _u64, _u64, _u64, _u32, _vp, _vp, _u64, _vp,
                               _u64]),
    "q4mi_mmq_gate_up_parts": (_b, [_vp, _vp, _u32, _u64, _u64, _u64, _u32, _vp, _u64, _vp,
                                    _vp, _u64, _vp, _vp, _vp]),
    "q4_xg_on": (_c.c_int, []),
    "q4_xg_gu_type": (_b, [_u32]),
    "q4_xg_dn_type": (_b, [_u32]),
    "q4_xg_shape_ok": (_b, [_u32, _u32]),
    "q4_xg_tile_cap": (_u32, [_u32, _u32]),
    "q4_xg_tiles": (_u32, [_vp, _vp, _vp, _u32, _vp, _u32]),
    "q4_xg_cvt": (_b, [_vp, _vp, _u64]),
    "q4_xg_gu": (_b, [_u32, _vp, _u64, _u64, _u64, _u32, _u32, _vp, _u32, _vp, _vp, _vp]),
    "q4_xg_dn": (_b, [_u32, _vp, _u64, _u64, _u32, _u32, _vp, _u32, _vp, _vp]),
    "q4mi_expert_reduce_x": (_b, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u64, _vp]),
}

# measurement build only
_MEAS_SIGS = {
    "q4mi_moe_phases": (None, [_c.c_int]),
    "q4mi_moe_lds_cap": (None, [_u32]),
    "q4mi_mfma_probe": (_c.c_bool, [_c.c_int, _u32, _c.POINTER(_c.c_uint64)]),
    "q4mi_stream_probe": (_c.c_bool, [_vp, _u32, _u32, _c.POINTER(_c.c_uint64)]),
    "q4mi_plain_stream_probe": (_c.c_bool, [_vp, _c.c_uint64, _u32]),
    "q4mi_mmq_ab_probe": (_c.c_bool, [_c.c_int, _u32, _c.POINTER(_c.c_uint64)]),
    "q4mi_alloc_count": (_c.c_uint64, []),
    "q4mi_grow_selftest": (_c.c_int, []),
}

_lib = None
_meas = None


def _load(path, sigs):
    if not os.path.exists(path):
        raise RuntimeError("q4mi: %s is missing; build it with __graft_entry__.build()" % path)
    L = _c.CDLL(path)
    for name, (res, args) in sigs.items():
        f = getattr(L, name, None)
        if f is None:
            continue
        f.restype = res
        f.argtypes = args
    return L


def lib():
    """The loaded library (raises if it was not built: no silent fallback)."""
    global _lib
    if _lib is None:
        _lib = _load(LIB_PATH, _SIGS)
    return _lib


def meas():
    """The measurement build (product ABI + the measurement hooks)."""
    global _meas
    if _meas is None:
        _meas = _load(MEAS_PATH, dict(_SIGS, **_MEAS_SIGS))
    return _meas


def exported_symbols():
    return list(_SIGS)


def measurement_symbols():
    return list(_MEAS_SIGS)


def ptr(t):
    """Device pointer of a torch tensor (or an int / None)."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def last_error(L=None):
    e = (L or lib()).q4mi_last_error()
    return e.decode() if e else ""


def check(ok, what, L=None):
    if not ok:
        raise RuntimeError("%s failed: %s" % (what, last_error(L)))


def use_torch_stream(L=None):
    """Launch on torch's current stream (so torch ops and ours are ordered);
    L: the library handle (default: the product library)."""
    import torch
    (L or lib()).q4mi_set_stream(_c.c_void_p(torch.cuda.current_stream().cuda_stream))


def row_bytes(ty, n):
    if ty == T_IQ3_S:
        return n // 256 * 110
    if ty == T_Q8_0:
        return n // 32 * 34
    raise ValueError(ty)
