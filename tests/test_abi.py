"""The C-ABI library: it loads without a GPU, exports every entry point the
public header declares, the Python mirror binds the same set, and host-side
argument checks reject bad calls before any device work (no GPU needed)."""
import ctypes
import os
import re
import subprocess

import pytest

from conftest import ROOT

import q4mi

HEADER = os.path.join(ROOT, "include", "q4mi.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(q4(?:mi)?_\w+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_entry_points():
    names = declared()
    for must in ("q4_hip_moe_exec", "q4_hip_moe_exec_win", "q4_mmvq_n", "q4_mmq_mul_id",
                 "q4_hip_route_pf", "q4_hip_assign_pf", "q4_hip_expert_reduce", "q4mi_quant8"):
        assert must in names


def test_library_exports_every_declared_symbol():
    assert os.path.exists(q4mi.LIB_PATH), "build the library first"
    out = subprocess.run(["nm", "-D", "--defined-only", q4mi.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(l.split()[-1] for l in out.splitlines() if " T " in l)
    missing = [n for n in declared() if n not in exported]
    assert not missing, missing


def test_python_mirror_binds_header():
    assert set(q4mi.exported_symbols()) == set(declared())


def test_loads_and_rejects_without_gpu():
    L = q4mi.lib()
    # host-side shape/type checks run before any HIP call
    assert not L.q4_mmvq_n(99, 1, 16, 2048, 1, 1, 1.0, 1)
    assert not L.q4_mmvq_n(q4mi.T_IQ3_S, 1, 16, 2000, 1, 1, 1.0, 1)
    assert not L.q4_mmvq_n(q4mi.T_IQ3_S, 1, 16, 2048, 1, 1, 1.0, 9)
    assert "not covered" in q4mi.last_error()
    assert not L.q4_hip_moe_win_ok(q4mi.T_IQ3_S, q4mi.T_IQ3_S, q4mi.T_IQ3_S, 2048, 512, 1)
    assert not L.q4_hip_moe_win_ok(q4mi.T_IQ3_S, q4mi.T_IQ3_S, q4mi.T_IQ3_S, 2048, 512, 9)
    assert L.q4_hip_moe_win_ok(q4mi.T_IQ3_S, q4mi.T_IQ3_S, q4mi.T_IQ3_S, 2048, 512, 4)
    assert not L.q4_hip_route_pf(1, 1, 1, 4, 513, 10)
    assert not L.q4_hip_route_pf(1, 1, 1, 4, 512, 65)
    assert not L.q4mi_assign(1, 1, 1, 1, 1, 1, 1, 1, None, 8, 0, 512, 4)
    assert L.q4_mmq_supported(q4mi.T_IQ3_S, 1024)
    assert not L.q4_mmq_supported(q4mi.T_IQ3_S, 1000)
    assert not L.q4_mmq_supported(12, 1024)
    assert L.q4_mmq_q8_bytes(10, 2048) == 10 * 2048 * 2 + 10 * 64 * 4 + 256
    assert not L.q4_mmq_mul_id(1, q4mi.T_IQ3_S, 1000, 2048, 0, 8, 16, 1, 0, 10, 16, 1000)
    # IQ3_S rows must be whole dwords (an even number of 110-byte superblocks)
    assert not L.q4_mmq_mul_id(16, q4mi.T_IQ3_S, 1024, 256, 0, 8, 16, 16, 0, 10, 16, 1024)
    assert "not covered" in q4mi.last_error()
    ids = (ctypes.c_int32 * 65)()
    w = (ctypes.c_float * 65)()
    # 65 experts exceeds the per-call bound (src/q4_test.c:1652-1663)
    assert not L.q4_hip_moe_exec(1, 0, ids, w, 65, 21, 0, 21, 0, 21, 0, 16, None, None, None,
                                 16, 512, 2048, 2048)
    assert not L.q4_hip_moe_exec(1, 0, ids, w, 0, 21, 0, 21, 0, 21, 0, 16, None, None, None,
                                 16, 512, 2048, 2048)


def test_boundary_extras_reject_without_gpu():
    """The staged / per-token decode and MMQ gather entry points check their
    arguments on the host before any device work."""
    L = q4mi.lib()
    T = q4mi.T_IQ3_S
    assert L.q4_hip_moe_tok_ok(T, T, T, 2048, 512)
    assert not L.q4_hip_moe_tok_ok(T, q4mi.T_Q8_0, T, 2048, 512)
    assert not L.q4_hip_moe_tok_ok(T, T, T, 2048, 2048)
    off = (ctypes.c_uint32 * 3)(0, 70, 70)          # token 0: 70 picks > 64
    assert not L.q4_hip_moe_exec_tok(1, 1, 1, 1, off, 2, T, 0, T, 0, T, 0, 16, None, None, 16,
                                     512, 2048, 2048)
    assert "pick range" in q4mi.last_error()
    assert not L.q4_hip_moe_exec_tok(1, 1, 1, 1, off, 2, T, 0, T, 0, T, 0, 16, None, None, 16,
                                     512, 2048, 1024)   # n_embd != in_dim
    assert not L.q4_hip_moe_stage(None, None, 65)
    assert L.q4_mmq_pad(880) == 0
    # destination stride below the slice size
    assert not L.q4_mmq_gather(1, 0, 0, 100, 0, 100, 50, 100, 1, 1, 1, 1, 1)
    assert L.q4_mmq_gather(None, 0, 0, 0, 0, 0, 0, 0, None, None, 0, None, None)   # n = 0
    assert not L.q4_mmq_wbuf(1, 1, 0, None, None)


MEAS_HEADER = os.path.join(ROOT, "include", "q4mi_measure.h")


def _exports(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True,
                         check=True).stdout
    return set(l.split()[-1] for l in out.splitlines() if " T " in l)


def test_measurement_hooks_only_in_measurement_build():
    """The hooks that change process-global behaviour (run one kernel of the
    decode pair, shrink the decode LDS, the MFMA probe) are exported by the
    measurement build only; it also carries the whole product ABI."""
    text = re.sub(r"/\*.*?\*/", "", open(MEAS_HEADER).read(), flags=re.S)
    hooks = sorted(set(re.findall(r"\b(q4mi_\w+)\s*\(", text)))
    assert hooks == sorted(q4mi.measurement_symbols())
    prod = _exports(q4mi.LIB_PATH)
    assert not [h for h in hooks if h in prod]
    assert os.path.exists(q4mi.MEAS_PATH), "build the library first"
    meas = _exports(q4mi.MEAS_PATH)
    assert not [n for n in declared() + hooks if n not in meas]


def test_status_text():
    """The timeout word of the decode kernels' bounded waits, as text
    (q4mi_device_status sets it as the last error when a wait gave up)."""
    L = q4mi.lib()
    assert L.q4mi_status_text(0) == b"ok"
    t1 = L.q4mi_status_text(1).decode()
    assert "consumer" in t1 and "producer" not in t1 and "wrong" in t1
    t2 = L.q4mi_status_text(2).decode()
    assert "producer" in t2 and "consumer" not in t2
    assert "consumer, producer" in L.q4mi_status_text(3).decode()
    assert "not readable" in L.q4mi_status_text(0x80000000).decode()


def test_grow_policy_selftest():
    """Library scratch grows by one policy: never inside a stream capture (the
    call fails instead), and an outgrown buffer is retired, not freed, so a
    graph captured before the growth keeps valid memory.  The measurement
    build runs the policy on host fakes (no device needed)."""
    M = q4mi.meas()
    assert M.q4mi_grow_selftest() == 1


def test_status_text_xg_tiles():
    L = q4mi.lib()
    t = L.q4mi_status_text(4).decode()
    assert "XG tile record" in t and "skipped" in t and "bounded wait" not in t
    t5 = L.q4mi_status_text(5).decode()
    assert "consumer" in t5 and "XG tile" in t5


def test_xg_tiles_host_table():
    """q4_xg_tiles (host code, no device): the reference's tile record
    {first routed row, rows, slot, expert}, every tile at most 128 rows, the
    rows of each expert covered once in order; a too-small capacity gives 0."""
    import ctypes
    import numpy as np
    L = q4mi.lib()
    rng = np.random.default_rng(3)
    E = 40
    ek = rng.integers(0, 400, E).astype(np.uint32)
    ek[[3, 9]] = [128, 129]
    eb = np.concatenate([[0], np.cumsum(ek)[:-1]]).astype(np.uint32)
    slot = rng.permutation(E).astype(np.int32)
    cap = int(L.q4_xg_tile_cap(int(ek.sum()), E))
    out = np.full(4 * cap, -1, np.int32)
    n = L.q4_xg_tiles(ek.ctypes.data, eb.ctypes.data, slot.ctypes.data, E, out.ctypes.data, cap)
    tiles = out[:4 * n].reshape(n, 4)
    assert n == int(sum((int(c) + 127) // 128 for c in ek))
    assert tiles[:, 1].max() <= 128 and tiles[:, 1].min() >= 1
    for e in range(E):
        te = tiles[tiles[:, 3] == e]
        assert te[:, 1].sum() == ek[e]
        assert np.all(te[:, 2] == slot[e])
        assert np.array_equal(te[:, 0], eb[e] + 128 * np.arange(len(te)))
    small = np.zeros(4 * (n - 1), np.int32)
    assert L.q4_xg_tiles(ek.ctypes.data, eb.ctypes.data, slot.ctypes.data, E, small.ctypes.data,
                         n - 1) == 0
