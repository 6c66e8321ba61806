"""Benchmark: IQ3_S routed-expert decode on one MI355X.

A step is one decode token through a stack of L (default 48) MoE layers, each
with its own 513 resident IQ3_S experts (512 routed + 1 shared; hidden 2048,
expert intermediate 512), top-10 routing + the shared expert at weight 1.
The stack holds L x 693 MB of distinct experts, far beyond the 256 MB
Infinity Cache, so every layer streams its 11 experts from HBM.  The L layer
calls (2 kernels each) are captured once in a HIP graph and replayed.

value = sustained algorithmic GB/s per layer: (11 experts x 1,351,680 B +
x 8 KB + y 8 KB) / layer time.  roofline = the gate/up kernel timed alone
(its own graph of L launches), algorithmic bytes 11 x 901,120 + 8,192 per
launch.  Also reported: single-layer latency, config 0 (IQ3_S 4096x4096
GEMV) and config 4 (Q8_0 151936x2048 lm-head, n=1 and n=4).

cpu_baseline: the reference's CPU expert job (q4_cpuex_dispatch2, compiled
from its sources into oracle/_ref) on this host's cores, on the same layer
shape; the repo's scalar C oracle when that build is absent.
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "suzuku-engine-q4_amd"))

METRIC = "IQ3_S MoE MMVQ GB/s (% of 8 TB/s) + prefill MMQ tok/s, 1 MI355X"
HBM_PEAK = 8000.0  # GB/s
N_EMBD, N_FF, N_EXP, TOPK = 2048, 512, 512, 10
EXPERT_BYTES = 1351680
LAYER_BYTES = 11 * EXPERT_BYTES + 2 * 4 * N_EMBD   # 14,884,864
GU_BYTES = 11 * 901120 + 4 * N_EMBD


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter
    summary (FETCH_SIZE + WRITE_SIZE, calibrated against a plain copy);
    None when the summary is absent."""
    path = os.path.join(ROOT, "profiles", "moe_decode_config2_hbm_traffic.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch " + kernel + ":"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def routes(rng, L):
    import numpy as np
    out = []
    for _ in range(L):
        lg = rng.standard_normal(N_EXP).astype(np.float32)
        p = np.exp(lg - lg.max())
        p /= p.sum()
        ids = np.lexsort((np.arange(N_EXP), -lg))[:TOPK]
        w = p[ids] / p[ids].sum()
        out.append((np.append(ids, N_EXP).astype(np.int32),
                    np.append(w, 1.0).astype(np.float32)))
    return out


def cpu_baseline(seconds=12.0):
    """The reference CPU expert job on this host (bounded sample)."""
    import numpy as np
    from q4mi import synth
    om = _oracle()
    rng = np.random.default_rng(5)
    arena = synth.expert_arena(rng, N_EXP + 1, N_EMBD, N_FF)
    stride = synth.expert_stride(N_EMBD, N_FF)[0]
    x = rng.standard_normal(N_EMBD).astype(np.float32)
    rts = routes(rng, 64)
    if om.have_ref():
        R = om.Ref()
        kind, cores = "reference", int(R.L.qref_threads())

        def run(i):
            ids, w = rts[i % len(rts)]
            R.moe_decode(N_EMBD, N_FF, om.T_IQ3_S, om.T_IQ3_S, N_EXP + 1, arena, stride, x,
                         ids, w)
    else:
        O = om.Oracle()
        kind, cores = "port", 1

        def run(i):
            ids, w = rts[i % len(rts)]
            O.moe_tokens(N_EMBD, N_FF, om.T_IQ3_S, om.T_IQ3_S, arena, stride, x, ids[None],
                         w[None])
    for i in range(3):
        run(i)
    times = []
    t_end = time.perf_counter() + seconds
    i = 0
    while time.perf_counter() < t_end or len(times) < 5:
        t0 = time.perf_counter()
        run(i)
        times.append(time.perf_counter() - t0)
        i += 1
    med = float(np.median(times))
    return {"value": round(LAYER_BYTES / med / 1e9, 3), "unit": "GB/s", "cores": cores,
            "kind": kind,
            "sample": "%d config-2 decode layers (11 IQ3_S experts each, routes rotating over "
                      "a 693 MB arena), median %.1f us/layer" % (len(times), med * 1e6)}


def _oracle():
    """The checker package (oracle/: the reference's CPU path and the C
    restatement), used only for the CPU baselines."""
    p = os.path.join(ROOT, "oracle")
    if p not in sys.path:
        sys.path.insert(0, p)
    import oracle as om
    return om


def host_facts():
    """nproc, CPU model and the ISA path the reference's CPU kernels take."""
    om = _oracle()
    model = "?"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        nproc = len(os.sched_getaffinity(0))
    except AttributeError:
        nproc = os.cpu_count() or 1
    isa = None
    if om.have_ref():
        isa = ("AVX-512 VNNI/VBMI/BITALG (c6_* kernels)" if om.Ref().L.qref_has512()
               else "AVX2 (+FMA/F16C) kernels")
    return {"nproc": nproc, "cpu_model": model, "isa_path": isa}


def _timed(run, seconds, min_n=3):
    import numpy as np
    run(0)
    times, i = [], 1
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < min_n:
        t0 = time.perf_counter()
        run(i)
        times.append(time.perf_counter() - t0)
        i += 1
    return float(np.median(times)), len(times)


def cpu_baselines(facts, seconds=4.0):
    """The reference's CPU path (oracle/_ref, compiled from its sources) on
    the other BASELINE configs, each a bounded sample: configs[0] (cpx_dot8
    IQ3_S rows, OpenMP over rows), configs[2] (q4_cpuex_dispatch_win, 4
    tokens), configs[3] (no CPU prefill exists: q4_cpuex_dispatch_win over
    4-token windows, a sample of the 512 windows of the 2048-token prompt)
    and configs[4] (cpx_dot8 / cpx_dot8n Q8_0 rows, n = 1 and 4)."""
    import numpy as np
    from q4mi import synth
    om = _oracle()
    if not om.have_ref():
        return None
    R = om.Ref()
    th = min(16, facts["nproc"])
    out = {"threads_rows": th, "threads_expert_pool": int(R.L.qref_threads())}
    rng = np.random.default_rng(8)
    # 4096 x 4096 IQ3_S, copies rotated beyond the host caches
    K = 4096
    ws = [synth.matrix(rng, om.T_IQ3_S, K, K) for _ in range(100)]
    x = rng.standard_normal(K).astype(np.float32)
    med, n = _timed(lambda i: R.dot8_rows(om.T_IQ3_S, ws[i % len(ws)], K, K, x, th), seconds)
    nb = 4096 * 4096 // 256 * 110 + 2 * 4 * K
    out["config0_gemv"] = {"us": round(med * 1e6, 1), "GB/s": round(nb / med / 1e9, 2),
                           "sample": "%d calls over 100 rotating 7.2 MB copies (720 MB)" % n}
    del ws
    # configs[2] / [3]: one layer's arena (693 MB)
    arena = synth.expert_arena(rng, N_EXP + 1, N_EMBD, N_FF)
    stride = synth.expert_stride(N_EMBD, N_FF)[0]

    def win(xs, rts):
        ids = np.concatenate([r[0] for r in rts])
        w = np.concatenate([r[1] for r in rts])
        tn = np.array([len(r[0]) for r in rts], np.uint32)
        R.moe_win(N_EMBD, N_FF, om.T_IQ3_S, om.T_IQ3_S, N_EXP + 1, arena, stride, xs, ids, w, tn)
        return len(set(ids.tolist()))

    x4 = rng.standard_normal((4, N_EMBD)).astype(np.float32)
    w4 = [routes(rng, 4) for _ in range(32)]
    med, n = _timed(lambda i: win(x4, w4[i % 32]), seconds)
    uq = np.mean([len(set(np.concatenate([r[0] for r in rr]).tolist())) for rr in w4])
    nb = uq * EXPERT_BYTES + 2 * 4 * 4 * N_EMBD
    out["config3_window"] = {"us": round(med * 1e6, 1), "GB/s": round(nb / med / 1e9, 2),
                             "sample": "%d 4-token windows (q4_cpuex_dispatch_win)" % n}
    # the reference's window takes at most 64 (token, expert) entries, so
    # top-10 + shared (11 per token) fits 4 tokens, not 8
    xw = rng.standard_normal((4, N_EMBD)).astype(np.float32)
    lgz = synth.logits(rng, 64, N_EXP, zipf=True)
    idz, wz = R.softmax_topk(lgz, TOPK)
    wzs = [[(np.append(idz[4 * j + t], N_EXP).astype(np.int32),
             np.append(wz[4 * j + t], 1.0).astype(np.float32)) for t in range(4)]
           for j in range(16)]
    med, n = _timed(lambda i: win(xw, wzs[i % 16]), seconds)
    out["config3_prefill"] = {"us_per_4_token_window": round(med * 1e6, 1),
                              "layer_us_512_windows": round(512 * med * 1e6, 1),
                              "tok_per_s": round(4 / med, 1),
                              "sample": "%d 4-token windows of Zipf-routed tokens (top-10 + "
                                        "shared); the reference has no CPU prefill, so the "
                                        "2048-token layer is 512 such windows (its window takes "
                                        "at most 64 (token, expert) entries: 8 tokens x 11 do "
                                        "not fit)" % n}
    del arena
    # Q8_0 151936 x 2048
    rows = 151936
    w3 = [synth.matrix(rng, om.T_Q8_0, rows, N_EMBD) for _ in range(3)]
    for nt in (1, 4):
        xs = rng.standard_normal((nt, N_EMBD)).astype(np.float32)
        med, n = _timed(lambda i: R.dot8_rows(om.T_Q8_0, w3[i % 3], rows, N_EMBD, xs, th),
                        seconds / 2)
        nb = rows * 2176 + 4 * nt * N_EMBD + 4 * nt * rows
        out["config4_lmhead_n%d" % nt] = {"us": round(med * 1e6, 1),
                                          "GB/s": round(nb / med / 1e9, 2),
                                          "sample": "%d calls rotating 3 copies (990 MB)" % n}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--profile", choices=["decode", "window", "prefill", "mmq", "gemv"],
                    help="a short run of one workload for rocprofv3 (no CPU baseline); mmq: "
                         "time the configs[3] prefill's gate/up and down MMQ launches alone "
                         "(with Q4MI_LIB naming a library variant, its knockouts); gemv: "
                         "the configs[0] and configs[4] GEMV lines alone")
    args = ap.parse_args()
    if args.profile == "mmq":
        sys.stdout.write(json.dumps(bench_mmq_launches()) + "\n")
        return
    if args.profile == "gemv":
        sys.stdout.write(json.dumps(bench_gemv_lines()) + "\n")
        return
    if args.profile:
        args.no_cpu = True
        args.no_prefill = args.profile != "prefill"
        args.no_extra = args.profile != "window"
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the routed-expert path is a "
              "single-GPU kernel set; multi-GPU sharding is a design note, not built).",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import q4mi
    from q4mi import synth

    L = q4mi.lib()
    # the measurement build runs one kernel of the decode pair alone
    M = q4mi.meas()
    torch.cuda.set_device(0)
    q4mi.use_torch_stream()
    q4mi.use_torch_stream(M)
    L.q4_hip_moe_scratch_warm()
    M.q4_hip_moe_scratch_warm()
    stride, og, ou, od = synth.expert_stride(N_EMBD, N_FF)
    rng = np.random.default_rng(1234)
    NL = args.layers
    arenas = [synth.device_iq3s((N_EXP + 1) * stride, seed=1000 + l) for l in range(NL)]
    xs = torch.randn(NL, N_EMBD, device="cuda", generator=torch.Generator("cuda").manual_seed(9))
    ys = torch.zeros(NL, N_EMBD, device="cuda")
    rts = routes(rng, NL)
    T = q4mi.T_IQ3_S

    def layer_call(l, lib=L):
        ids, w = rts[l]
        ok = lib.q4_hip_moe_exec(arenas[l].data_ptr(), stride, ids.ctypes.data_as(ctypes.c_void_p),
                               w.ctypes.data_as(ctypes.c_void_p), len(ids), T, og, T, ou, T, od,
                               xs[l].data_ptr(), None, None, None, ys[l].data_ptr(), N_FF,
                               N_EMBD, N_EMBD)
        q4mi.check(ok, "q4_hip_moe_exec", lib)

    def capture(fn):
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn()   # eager warm-up on the capture stream
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            q4mi.use_torch_stream()
            q4mi.use_torch_stream(M)
            fn()
        q4mi.use_torch_stream()
        q4mi.use_torch_stream(M)
        return g

    def stack(lib=L):
        for l in range(NL):
            layer_call(l, lib)

    def timed(g, steps, warmup):
        for _ in range(warmup):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1)

    # replay vs eager: identical bits (no memset nodes; deterministic reduce)
    g_full = capture(stack)
    ys.zero_()
    g_full.replay()
    torch.cuda.synchronize()
    y_graph = ys.clone()
    ys.zero_()
    stack()
    torch.cuda.synchronize()
    if not os.environ.get("Q4MI_DBG"):
        assert torch.equal(y_graph, ys), "graph replay differs from eager"

    ms = timed(g_full, args.steps, args.warmup)
    t_layer = ms * 1e-3 / (args.steps * NL)
    value = LAYER_BYTES / t_layer / 1e9

    # the gate/up kernel alone (dominant kernel: 2/3 of the bytes)
    # (measurement build; its kernels are the product's, compiled alike)
    M.q4mi_moe_phases(1)
    g_gu = capture(lambda: stack(M))
    ms_gu = timed(g_gu, args.steps, args.warmup)
    M.q4mi_moe_phases(2)
    g_dn = capture(lambda: stack(M))
    ms_dn = timed(g_dn, args.steps, args.warmup)
    M.q4mi_moe_phases(3)
    t_gu = ms_gu * 1e-3 / (args.steps * NL)
    t_dn = ms_dn * 1e-3 / (args.steps * NL)
    gu_gbs = GU_BYTES / t_gu / 1e9

    # single-layer latency (eager, synchronised)
    torch.cuda.synchronize()
    lat = []
    for i in range(50):
        t0 = time.perf_counter()
        layer_call(i % NL)
        torch.cuda.synchronize()
        lat.append(time.perf_counter() - t0)
    single_us = float(np.median(lat[5:])) * 1e6

    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded IQ3_S experts generated in HBM; N(0,1) activations)",
        "config": {"workload": "BASELINE.json configs[1] (config 2): IQ3_S MoE decode layer, "
                               "1 token, hidden 2048, "
                               "512 routed experts top-10 + 1 shared, expert intermediate 512; "
                               "sustained over a %d-layer stack of distinct experts" % NL,
                   "layers_per_step": NL, "bytes_per_layer": LAYER_BYTES},
        "pct_of_hbm": round(100 * value / HBM_PEAK, 2),
        "layer_us": round(t_layer * 1e6, 3),
        "kernel_us": {"moe_gu_k": round(t_gu * 1e6, 3), "moe_dn_k": round(t_dn * 1e6, 3)},
        "single_layer_latency_us": round(single_us, 2),
        "roofline": {"bound": "hbm", "achieved": round(gu_gbs, 2), "peak": HBM_PEAK,
                     "unit": "GB/s", "frac": round(gu_gbs / HBM_PEAK, 4),
                     "traffic": measured_traffic("moe_gu_k"),
                     "kernel": "moe_gu_k", "bytes_per_launch": GU_BYTES},
    }
    if not args.no_extra:
        out["config3_window"] = bench_window(L, torch, np, q4mi, arenas, stride, og, ou, od, NL,
                                             capture, timed, args)
        if not args.profile and not args.no_extra:
            out["window_reference_shapes"] = bench_window_mixes(L, torch, np, q4mi, synth,
                                                                capture, timed, args)
        if not args.profile:
            out["config2_routed"] = bench_routed(L, torch, np, q4mi, arenas, stride, og, ou,
                                                 od, NL, capture, timed, args)
    del g_full, g_gu, g_dn, arenas
    torch.cuda.empty_cache()

    if not args.no_extra and not args.profile:
        out["decode_floors"] = bench_floors(M, torch, q4mi)
    if not args.no_prefill:
        out["mfma_peak"] = bench_mfma_peak(M, torch, q4mi)
        out["mmq_inner_ab"] = bench_mmq_ab(M, torch, q4mi)
        out["prefill"] = bench_prefill(L, torch, np, q4mi, synth, args)
        out["prefill"]["pct_of_measured_int8_peak"] = round(
            100 * out["prefill"]["mmq_TOPS"] / out["mfma_peak"]["int8_TOPS"], 2)
        out["prefill_xg"] = bench_prefill_xg(L, torch, np, q4mi, synth, args)
    if not args.no_extra and not args.profile:
        out["config0_gemv"] = bench_gemv(L, torch, np, q4mi, synth, T, 4096, 4096, 80, 1,
                                         "configs[0]")
        out["config4_lmhead_n1"] = bench_gemv(L, torch, np, q4mi, synth, q4mi.T_Q8_0, 151936,
                                              2048, 2, 1, "configs[4]")
        out["config4_lmhead_n4"] = bench_gemv(L, torch, np, q4mi, synth, q4mi.T_Q8_0, 151936,
                                              2048, 2, 4, "configs[4]")
    if not args.no_cpu:
        facts = host_facts()
        out["cpu_baseline"] = cpu_baseline()
        out["cpu_baseline"].update({k: facts[k] for k in ("cpu_model", "isa_path")})
        out["cpu_baseline"]["nproc"] = facts["nproc"]
        out["cpu_baselines"] = cpu_baselines(facts)
    sys.stdout.write(json.dumps(out) + "\n")
    sys.stdout.flush()


def bench_floors(M, torch, q4mi, n=48, reps=20):
    """Floors of the decode kernels' structure on this GPU (measurement
    build's stream probe, one 1024-thread block per CU as moe_gu_k /
    moe_dn_k): a graph of n back-to-back launches, each streaming its own
    per-CU share into LDS from distinct memory (beyond the Infinity Cache);
    per-launch time = graph time / n."""
    import ctypes
    P = q4mi.ptr
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    res = {"n_cu": cus, "launches_per_graph": n}
    per_cases = [(0, 4), (20 * 1024, 4), (40 * 1024, 4), (60 * 1024, 4), (140 * 1024, 4),
                 (140 * 1024, 8)]
    src = torch.empty(n * cus * 140 * 1024, dtype=torch.uint8, device="cuda")
    src.fill_(1)
    for per, waves in per_cases:
        b = ctypes.c_uint64(0)

        def launches():
            for i in range(n):
                q4mi.check(M.q4mi_stream_probe(P(src) + i * cus * per, per, waves,
                                               ctypes.byref(b)), "stream probe", M)
        launches()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            q4mi.use_torch_stream(M)
            launches()
        q4mi.use_torch_stream(M)
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) * 1e-3 / (reps * n)
        key = "empty" if not per else "%dKB_per_cu_%dwaves" % (per // 1024, waves)
        res[key] = {"us_per_launch": round(t * 1e6, 2)}
        if per:
            res[key]["MB"] = round(b.value / 1e6, 2)
            res[key]["GB/s"] = round(b.value / t / 1e9, 1)
        del g
    del src
    torch.cuda.empty_cache()
    # the chip's own floor: plain register-load streaming with many
    # 256-thread blocks (no LDS, one block per 4096*unroll bytes), same
    # graph of n back-to-back launches over distinct memory
    plain = {}
    for mb in (5, 10, 37):
        for unroll in (1, 4, 8):
            per = 4096 * unroll
            nbytes = (mb * 1000 * 1000 + per - 1) // per * per
            buf = torch.empty(n * nbytes, dtype=torch.uint8, device="cuda")
            buf.fill_(1)

            def plaunch():
                for i in range(n):
                    q4mi.check(M.q4mi_plain_stream_probe(P(buf) + i * nbytes, nbytes, unroll),
                               "plain stream probe", M)
            plaunch()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                q4mi.use_torch_stream(M)
                plaunch()
            q4mi.use_torch_stream(M)
            g.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                g.replay()
            e1.record()
            torch.cuda.synchronize()
            t = e0.elapsed_time(e1) * 1e-3 / (reps * n)
            plain["%dMB_unroll%d" % (mb, unroll)] = {
                "us_per_launch": round(t * 1e6, 2), "blocks": nbytes // per,
                "GB/s": round(nbytes / t / 1e9, 1)}
            del g, buf
            torch.cuda.empty_cache()
    res["plain_stream"] = plain
    return res


def bench_mfma_peak(L, torch, q4mi, iters=16384, reps=5):
    """Measured dense MFMA rate of this GPU (the int8 32x32x32 and fp16
    32x32x16 instructions the datasheet peaks are quoted for), from the
    library's throughput probe timed with events on the library stream."""
    import ctypes
    res = {}
    for kind, key in ((0, "int8_TOPS"), (1, "fp16_TFLOPS")):
        ops = ctypes.c_uint64(0)
        q4mi.check(L.q4mi_mfma_probe(kind, iters, ctypes.byref(ops)), "mfma probe", L)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            q4mi.check(L.q4mi_mfma_probe(kind, iters, ctypes.byref(ops)), "mfma probe", L)
        e1.record()
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) * 1e-3 / reps
        res[key] = round(ops.value / t / 1e12, 1)
    res["datasheet_int8_TOPS"] = 5000.0
    res["datasheet_fp16_TFLOPS"] = 2500.0
    return res


def bench_mmq_ab(M, torch, q4mi, groups=2048, reps=5):
    """The prefill MMQ inner loop on the same work, two ways (measurement
    build's probe): exact-integer fp16 MFMA (this library's design: the IQ3_S
    multiplier folded into fp16 operands, one scale FMA per output and group)
    against int8 MFMA (the multiplier does not fit int8, so each output takes
    an integer multiply, a conversion and an FMA per group).  Rates are the
    GEMM ops the loop performs, timed with events on the library stream."""
    import ctypes
    res = {}
    for kind, key in ((0, "fp16_exact_TOPS"), (1, "int8_TOPS")):
        ops = ctypes.c_uint64(0)
        q4mi.check(M.q4mi_mmq_ab_probe(kind, groups, ctypes.byref(ops)), "mmq A/B probe", M)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            q4mi.check(M.q4mi_mmq_ab_probe(kind, groups, ctypes.byref(ops)), "mmq A/B probe", M)
        e1.record()
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) * 1e-3 / reps
        res[key] = round(ops.value / t / 1e12, 1)
    res["int8_over_fp16"] = round(res["int8_TOPS"] / res["fp16_exact_TOPS"], 3)
    res["note"] = ("inner loop only (operands in LDS, 32 x 128 outputs per wave, 2 blocks per "
                   "CU): IQ3_S decode + MFMA + per-group scaling, no copies or epilogue")
    return res


PF_T, PF_K = 2048, 10
PF_OPS = (PF_T * PF_K + PF_T) * 2 * 3 * N_EMBD * N_FF   # 141.7 G (routed + shared)


def bench_prefill(L, torch, np, q4mi, synth, args, copies=3, reps=10):
    """Config 3-prefill: 2048 tokens, Zipf-skewed top-10 over 512 experts +
    the shared expert, one MoE layer: route -> stable pack -> q8(x) ->
    MMQ gate/up -> SwiGLU -> q8(h) -> MMQ down -> weighted reduce.  `copies`
    distinct 693 MB layers rotate so weights stream from HBM."""
    T, k, E, H, F = PF_T, PF_K, N_EXP, N_EMBD, N_FF
    stride, og, ou, od = synth.expert_stride(H, F)
    rows = T * k
    rng = np.random.default_rng(99)
    arenas = [synth.device_iq3s((E + 1) * stride, seed=500 + c) for c in range(copies)]
    x = torch.randn(T, H, device="cuda")
    lg = torch.from_numpy(synth.logits(rng, T, E, zipf=True)).cuda()
    i32 = torch.int32
    ids, wts = torch.empty(T, k, dtype=i32, device="cuda"), torch.empty(T, k, device="cuda")
    # packed rows: the routed pack, then the shared expert's rows (every
    # token, in order), which ride in the routed MMQ launches as expert E
    a_tok = torch.empty(rows + T, dtype=i32, device="cuda")
    a_tok[rows:] = torch.arange(T, dtype=i32, device="cuda")
    rsrc = torch.empty(rows, dtype=i32, device="cuda")
    rw = torch.empty(rows, device="cuda")
    stg, stgn = torch.empty(512, dtype=i32, device="cuda"), torch.empty(1, dtype=i32, device="cuda")
    ek = torch.empty(512, dtype=i32, device="cuda")
    bounds = torch.empty(E + 2, dtype=i32, device="cuda")
    bounds[E + 1] = rows + T                      # the pack writes bounds[0..E]
    xq = torch.empty(int(L.q4_mmq_q8_bytes(T, H)), dtype=torch.uint8, device="cuda")
    hq = torch.empty(int(L.q4_mmq_q8_bytes(rows + T, F)), dtype=torch.uint8, device="cuda")
    pd = torch.empty(rows + T, H, device="cuda")
    y = torch.zeros(T, H, device="cuda")
    P = q4mi.ptr
    TY = q4mi.T_IQ3_S
    chk = q4mi.check

    def layer(c):
        A = arenas[c].data_ptr()
        chk(L.q4_hip_route_pf(P(lg), P(ids), P(wts), T, E, k), "route")
        chk(L.q4mi_assign(P(ids), P(wts), P(a_tok), P(rsrc), P(rw), P(stg), P(stgn), P(ek),
                          P(bounds), T, k, E, T), "assign")
        # q8(x) once per token; routed rows gather it through a_tok
        chk(L.q4_mmq_quantize(P(x), None, P(xq), TY, H, T), "q8 x")
        # routed experts + the shared expert (its own weight base S; every
        # token, weight 1) in one gate/up, one down and one reduce launch
        S = A + E * stride
        chk(L.q4mi_mmq_gate_up_x(A, S, TY, F, H, stride, E, P(xq), T, P(a_tok), P(bounds),
                                 rows + T, P(hq)), "mmq gate/up")
        chk(L.q4mi_mmq_mul_id_x(A + od, S + od, TY, H, F, stride, E, P(hq), P(bounds), rows + T,
                                P(pd), H), "mmq down")
        chk(L.q4mi_expert_reduce_x(P(y), P(pd), P(rsrc), P(rw), T, k, H, rows, None), "reduce")

    def run_all():
        for c in range(copies):
            layer(c)

    run_all()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        q4mi.use_torch_stream()
        run_all()
    q4mi.use_torch_stream()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) * 1e-3 / (reps * copies)
    used = int((ek > 0).sum().item())
    wbytes = (used + 1) * EXPERT_BYTES
    del arenas
    return {"baseline_config": "configs[3]", "layer_us": round(t * 1e6, 1),
            "tok_per_s": round(T / t, 1), "mmq_TOPS": round(PF_OPS / t / 1e12, 2),
            "pct_of_int8_peak": round(100 * PF_OPS / t / 5.0e15, 2),
            "experts_touched": used, "weight_bytes": wbytes,
            "weight_GB_per_s": round(wbytes / t / 1e9, 1),
            "note": "whole routed layer incl. route, pack, quantize, SwiGLU, reduce and the "
                    "shared expert; ops = (20480 + 2048) rows x 3 x 2048 x 512 x 2"}


def bench_mmq_launches(copies=3, reps=8):
    """The configs[3] prefill's two MMQ launches timed alone (eager, events
    on the library stream over `copies` rotating weight arenas): gate/up
    (routed + shared, fused SwiGLU + q8(h)) and down.  Used with library
    variants built by `python -m q4mi.build --lib ... --define ...` to
    attribute the kernels' time (Q4MI_MMQ_KO knockouts)."""
    import numpy as np
    import torch
    import q4mi
    from q4mi import synth
    L = q4mi.lib()
    torch.cuda.set_device(0)
    q4mi.use_torch_stream(L)
    T, k, E, H, F = PF_T, PF_K, N_EXP, N_EMBD, N_FF
    stride, og, ou, od = synth.expert_stride(H, F)
    rows = T * k
    rng = np.random.default_rng(99)
    arenas = [synth.device_iq3s((E + 1) * stride, seed=500 + c) for c in range(copies)]
    x = torch.randn(T, H, device="cuda")
    lg = torch.from_numpy(synth.logits(rng, T, E, zipf=True)).cuda()
    i32 = torch.int32
    ids, wts = torch.empty(T, k, dtype=i32, device="cuda"), torch.empty(T, k, device="cuda")
    a_tok = torch.empty(rows + T, dtype=i32, device="cuda")
    a_tok[rows:] = torch.arange(T, dtype=i32, device="cuda")
    rsrc = torch.empty(rows, dtype=i32, device="cuda")
    rw = torch.empty(rows, device="cuda")
    stg, stgn = torch.empty(512, dtype=i32, device="cuda"), torch.empty(1, dtype=i32, device="cuda")
    ek = torch.empty(512, dtype=i32, device="cuda")
    bounds = torch.empty(E + 2, dtype=i32, device="cuda")
    bounds[E + 1] = rows + T
    xq = torch.empty(int(L.q4_mmq_q8_bytes(T, H)), dtype=torch.uint8, device="cuda")
    hq = torch.empty(int(L.q4_mmq_q8_bytes(rows + T, F)), dtype=torch.uint8, device="cuda")
    pd = torch.empty(rows + T, H, device="cuda")
    P, TY, chk = q4mi.ptr, q4mi.T_IQ3_S, q4mi.check
    chk(L.q4_hip_route_pf(P(lg), P(ids), P(wts), T, E, k), "route", L)
    chk(L.q4mi_assign(P(ids), P(wts), P(a_tok), P(rsrc), P(rw), P(stg), P(stgn), P(ek),
                      P(bounds), T, k, E, T), "assign", L)
    chk(L.q4_mmq_quantize(P(x), None, P(xq), TY, H, T), "q8 x", L)

    def gu(c):
        A = arenas[c].data_ptr()
        chk(L.q4mi_mmq_gate_up_x(A, A + E * stride, TY, F, H, stride, E, P(xq), T, P(a_tok),
                                 P(bounds), rows + T, P(hq)), "mmq gate/up", L)

    def dn(c):
        A = arenas[c].data_ptr()
        chk(L.q4mi_mmq_mul_id_x(A + od, A + E * stride + od, TY, H, F, stride, E, P(hq),
                                P(bounds), rows + T, P(pd), H), "mmq down", L)

    def clock(fn):
        for c in range(copies):
            fn(c)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            for c in range(copies):
                fn(c)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (reps * copies)
    res = {"gate_up_us": round(clock(gu), 1), "down_us": round(clock(dn), 1),
           "library": os.path.basename(q4mi.LIB_PATH)}
    del arenas
    return res


def bench_prefill_xg(L, torch, np, q4mi, synth, args, copies=3, reps=10):
    """The XG A/B of the prefill layer (the reference's q4_xg: fp16
    activations, fp16-dequantized weights, fp32 accumulation) on the same
    routing as bench_prefill: q4_xg_cvt -> q4_xg_gu -> q4_xg_dn -> reduce, the
    shared expert as one more tile set over every token.  The tile table is
    built on the host from the pack (as the reference does) before timing;
    x is N(0,1) * 0.05 so h stays in fp16's range."""
    T, k, E, H, F = PF_T, PF_K, N_EXP, N_EMBD, N_FF
    stride, og, ou, od = synth.expert_stride(H, F)
    rows = T * k
    rng = np.random.default_rng(99)
    arenas = [synth.device_iq3s((E + 1) * stride, seed=500 + c) for c in range(copies)]
    x = torch.randn(T, H, device="cuda") * 0.05
    lg = torch.from_numpy(synth.logits(rng, T, E, zipf=True)).cuda()
    i32 = torch.int32
    P, chk, TY = q4mi.ptr, q4mi.check, q4mi.T_IQ3_S
    ids, wts = torch.empty(T, k, dtype=i32, device="cuda"), torch.empty(T, k, device="cuda")
    a_tok = torch.empty(rows + T, dtype=i32, device="cuda")
    a_tok[rows:] = torch.arange(T, dtype=i32, device="cuda")
    rsrc = torch.empty(rows, dtype=i32, device="cuda")
    rw = torch.empty(rows, device="cuda")
    stg, stgn = torch.empty(512, dtype=i32, device="cuda"), torch.empty(1, dtype=i32, device="cuda")
    ek = torch.empty(512, dtype=i32, device="cuda")
    bounds = torch.empty(E + 1, dtype=i32, device="cuda")
    chk(L.q4_hip_route_pf(P(lg), P(ids), P(wts), T, E, k), "route")
    chk(L.q4mi_assign(P(ids), P(wts), P(a_tok), P(rsrc), P(rw), P(stg), P(stgn), P(ek),
                      P(bounds), T, k, E, T), "assign")
    torch.cuda.synchronize()
    ekh = np.append(ek.cpu().numpy()[:E], T).astype(np.uint32)
    ebh = np.append(bounds.cpu().numpy()[:E], rows).astype(np.uint32)
    slot = np.arange(E + 1, dtype=np.int32)
    cap = L.q4_xg_tile_cap(rows + T, E + 1)
    tiles = np.zeros(4 * cap, np.int32)
    nt = L.q4_xg_tiles(ekh.ctypes.data, ebh.ctypes.data, slot.ctypes.data, E + 1,
                       tiles.ctypes.data, cap)
    assert nt > 0
    d_tiles = torch.from_numpy(tiles[:4 * nt]).cuda()
    x16 = torch.empty(T, H, dtype=torch.float16, device="cuda")
    h16 = torch.empty(rows + T, F, dtype=torch.float16, device="cuda")
    pd = torch.empty(rows + T, H, device="cuda")
    y = torch.zeros(T, H, device="cuda")

    def layer(c):
        A = arenas[c].data_ptr()
        chk(L.q4_xg_cvt(P(x), P(x16), T * H), "xg cvt")
        chk(L.q4_xg_gu(TY, A, stride, og, ou, H, F, P(d_tiles), nt, P(x16), P(a_tok), P(h16)),
            "xg gu")
        chk(L.q4_xg_dn(TY, A, stride, od, F, H, P(d_tiles), nt, P(h16), P(pd)), "xg dn")
        chk(L.q4mi_expert_reduce_x(P(y), P(pd), P(rsrc), P(rw), T, k, H, rows, None), "reduce")

    def run_all():
        for c in range(copies):
            layer(c)

    run_all()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        q4mi.use_torch_stream()
        run_all()
    q4mi.use_torch_stream()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) * 1e-3 / (reps * copies)
    del arenas, g
    return {"baseline_config": "configs[3] (A/B)", "layer_us": round(t * 1e6, 1),
            "tok_per_s": round(T / t, 1), "fp16_TFLOPS": round(PF_OPS / t / 1e12, 2),
            "pct_of_fp16_peak": round(100 * PF_OPS / t / 2.5e15, 2), "tiles": int(nt),
            "note": "fp16 activations (XG): excludes routing/pack (the tile table is "
                    "host-built from the pack, as in the reference); includes x->fp16, "
                    "gate/up, down, reduce"}


def bench_routed(L, torch, np, q4mi, arenas, stride, og, ou, od, NL, capture, timed, args):
    """configs[1] with its router in front (the f1/f2 row): per layer
    q4mi_moe_route_exec (fp32 512 x 2048 router GEMV and the shared expert's
    sigmoid gate, then the device-list decode layer whose gate/up blocks take
    the softmax top-10 themselves, the shared expert at weight sg; the lists
    are written as q4mi_moe_route writes them), sustained over the layer
    stack.
    Bytes per layer add the 4 MB router and the 8 KB gate vector."""
    P = q4mi.ptr
    T = q4mi.T_IQ3_S
    g = torch.Generator("cuda").manual_seed(11)
    routers = torch.randn(NL, N_EXP, N_EMBD, device="cuda", generator=g) * 0.05
    sgate = torch.randn(NL, N_EMBD, device="cuda", generator=g) * 0.02
    xs = torch.randn(NL, N_EMBD, device="cuda", generator=g)
    ys = torch.zeros(NL, N_EMBD, device="cuda")
    lg = torch.empty(NL, N_EXP, device="cuda")
    es = torch.empty(NL, 64, dtype=torch.int32, device="cuda")
    ew = torch.empty(NL, 64, device="cuda")
    nh = torch.empty(NL, dtype=torch.int32, device="cuda")
    sg = torch.empty(NL, device="cuda")

    def stack():
        for l in range(NL):
            q4mi.check(L.q4mi_moe_route_exec(P(routers[l]), 0, P(sgate[l]), P(xs[l]), N_EMBD,
                                             N_EXP, TOPK, P(lg[l]), P(es[l]), P(ew[l]), P(nh[l]),
                                             N_EXP, P(sg[l]), arenas[l].data_ptr(), stride, T,
                                             og, T, ou, T, od, P(ys[l]), N_FF),
                       "q4mi_moe_route_exec")
    gr = capture(stack)
    steps = max(args.steps // 4, 10)
    ms = timed(gr, steps, max(args.warmup // 4, 2))
    t = ms * 1e-3 / (steps * NL)
    nbytes = LAYER_BYTES + N_EXP * N_EMBD * 4 + N_EMBD * 4
    del gr
    return {"baseline_config": "configs[1] + router", "layer_us": round(t * 1e6, 3),
            "GB/s": round(nbytes / t / 1e9, 1),
            "pct_of_hbm": round(100 * nbytes / t / 1e9 / HBM_PEAK, 2),
            "bytes_per_layer": nbytes,
            "note": "router GEMV (fp32 512x2048) + sigmoid shared gate, then the device-list "
                    "decode layer taking the top-10 in its gate/up blocks (3 launches); graph "
                    "over the %d-layer stack"
                    % NL}


def bench_window(L, torch, np, q4mi, arenas, stride, og, ou, od, NL, capture, timed, args,
                 n_tok=4):
    """Config 3: the 4-token verify window (1 accepted + 3 drafted tokens, each
    with its own top-10 from seeded N(0,1) logits, plus the shared expert)
    sustained over the same stack of distinct-expert layers.  Bytes per layer
    = every unique expert once (the window reads each expert once for all of
    its tokens) + x and y."""
    rng = np.random.default_rng(4321)
    es = np.full((NL, n_tok, 64), -1, np.int32)
    ew = np.zeros((NL, n_tok, 64), np.float32)
    nh = np.zeros((NL, n_tok), np.int32)
    uniq = []
    for l in range(NL):
        ids_l = set()
        for t, (ids, w) in enumerate(routes(rng, n_tok)):
            es[l, t, :len(ids)], ew[l, t, :len(ids)], nh[l, t] = ids, w, len(ids)
            ids_l.update(int(i) for i in ids)
        uniq.append(len(ids_l))
    d_es, d_ew, d_nh = (torch.from_numpy(a).cuda() for a in (es, ew, nh))
    xs = torch.randn(NL, n_tok, N_EMBD, device="cuda",
                     generator=torch.Generator("cuda").manual_seed(10))
    ys = torch.zeros(NL, n_tok, N_EMBD, device="cuda")
    T = q4mi.T_IQ3_S

    def stack():
        for l in range(NL):
            q4mi.check(L.q4_hip_moe_exec_win(arenas[l].data_ptr(), stride, d_es[l].data_ptr(),
                                             d_ew[l].data_ptr(), d_nh[l].data_ptr(), n_tok, T,
                                             og, T, ou, T, od, xs[l].data_ptr(), None,
                                             ys[l].data_ptr(), N_FF, N_EMBD, N_EMBD),
                       "q4_hip_moe_exec_win")
    g = capture(stack)
    ys.zero_()
    g.replay()
    torch.cuda.synchronize()
    y_graph = ys.clone()
    ys.zero_()
    stack()
    torch.cuda.synchronize()
    assert torch.equal(y_graph, ys), "window graph replay differs from eager"
    steps = max(args.steps // 4, 10)
    ms = timed(g, steps, max(args.warmup // 4, 2))
    t = ms * 1e-3 / (steps * NL)
    nbytes = float(np.mean(uniq)) * EXPERT_BYTES + 2 * 4 * n_tok * N_EMBD
    del g
    return {"baseline_config": "configs[2]", "layer_us": round(t * 1e6, 3),
            "GB/s": round(nbytes / t / 1e9, 1),
            "pct_of_hbm": round(100 * nbytes / t / 1e9 / HBM_PEAK, 2),
            "unique_experts": round(float(np.mean(uniq)), 2), "tokens": n_tok,
            "note": "4 tokens, own top-10 each + shared; each unique expert read once; "
                    "graph over the %d-layer stack" % NL}


def mixed_arena(torch, synth, q4mi_ty_rb, E, H, F, tg, td, seed):
    """An expert arena of E packed experts [gate F x H | up F x H | down H x F]
    with gate/up blocks of type tg and down blocks of type td, generated in
    HBM (uniform bytes, fp16 |N(0,1)| * 0.02 block scales)."""
    rbg, rbd = q4mi_ty_rb(tg, H), q4mi_ty_rb(td, F)
    stride = 2 * F * rbg + H * rbd
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    a = torch.randint(0, 256, (E, stride), dtype=torch.uint8, device="cuda", generator=g)
    for ty, lo, hi in ((tg, 0, 2 * F * rbg), (td, 2 * F * rbg, stride)):
        vals, nb, doff = synth.BLOCKS[ty]
        part = a[:, lo:hi].reshape(E, (hi - lo) // nb, nb)
        d = (torch.randn(E, (hi - lo) // nb, device="cuda", generator=g).abs() * 0.02
             ).to(torch.float16)
        part[:, :, doff:doff + 2] = d.view(torch.uint8).view(E, (hi - lo) // nb, 2)
        a[:, lo:hi] = part.reshape(E, hi - lo)
    return a.view(-1), stride, 0, F * rbg, 2 * F * rbg


def bench_window_mixes(L, torch, np, q4mi, synth, capture, timed, args, NL=24, n_tok=4):
    """The 4-token verify window at the reference model's shapes (hidden 2560,
    expert intermediate 640, 512 experts, top-10 + the shared expert) for the
    gate/up formats the reference quotes its window on (IQ2_S / IQ3_XXS /
    IQ3_S gate/up, IQ4_NL down: 46 / 51 / 53 us per layer on an RX 7900 XTX,
    AGENTS.md:410-414 of the reference), over a stack of NL distinct-expert
    layers (graph replay).  Bytes per layer = every unique expert once + x, y."""
    H, F, E = 2560, 640, N_EXP + 1
    rb = lambda ty, n: n // synth.BLOCKS[ty][0] * synth.BLOCKS[ty][1]
    rng = np.random.default_rng(777)
    es = np.full((NL, n_tok, 64), -1, np.int32)
    ew = np.zeros((NL, n_tok, 64), np.float32)
    nh = np.zeros((NL, n_tok), np.int32)
    uniq = []
    for l in range(NL):
        ids_l = set()
        for t, (ids, w) in enumerate(routes(rng, n_tok)):
            es[l, t, :len(ids)], ew[l, t, :len(ids)], nh[l, t] = ids, w, len(ids)
            ids_l.update(int(i) for i in ids)
        uniq.append(len(ids_l))
    d_es, d_ew, d_nh = (torch.from_numpy(a).cuda() for a in (es, ew, nh))
    xs = torch.randn(NL, n_tok, H, device="cuda", generator=torch.Generator("cuda").manual_seed(3))
    ys = torch.zeros(NL, n_tok, H, device="cuda")
    out = {"shape": "hidden 2560, n_ff 640, 512 experts top-10 + shared, 4 tokens",
           "layers": NL}
    TD = synth.T_IQ4_NL
    for name, tg in (("IQ2_S", synth.T_IQ2_S), ("IQ3_XXS", synth.T_IQ3_XXS),
                     ("IQ3_S", synth.T_IQ3_S)):
        if not L.q4_hip_moe_win_ok(tg, tg, TD, H, F, n_tok):
            out[name] = "not covered"
            continue
        arenas = []
        for l in range(NL):
            arenas.append(mixed_arena(torch, synth, rb, E, H, F, tg, TD, 900 + l))
        stride, og, ou, od = arenas[0][1:]

        def stack():
            for l in range(NL):
                q4mi.check(L.q4_hip_moe_exec_win(arenas[l][0].data_ptr(), stride,
                                                 d_es[l].data_ptr(), d_ew[l].data_ptr(),
                                                 d_nh[l].data_ptr(), n_tok, tg, og, tg, ou, TD,
                                                 od, xs[l].data_ptr(), None, ys[l].data_ptr(),
                                                 F, H, H), "q4_hip_moe_exec_win")
        g = capture(stack)
        steps = max(args.steps // 4, 10)
        ms = timed(g, steps, max(args.warmup // 4, 2))
        t = ms * 1e-3 / (steps * NL)
        nbytes = float(np.mean(uniq)) * stride + 2 * 4 * n_tok * H
        out[name] = {"layer_us": round(t * 1e6, 2), "GB/s": round(nbytes / t / 1e9, 1),
                     "pct_of_hbm": round(100 * nbytes / t / 1e9 / HBM_PEAK, 2)}
        del g, arenas
        torch.cuda.empty_cache()
    out["reference_rx7900xtx_us"] = {"IQ2_S": 46, "IQ3_XXS": 51, "IQ3_S": 53}
    return out


def bench_gemv_lines():
    """The configs[0] and configs[4] GEMV lines alone (library from Q4MI_LIB
    when set)."""
    import numpy as np
    import torch
    import q4mi
    from q4mi import synth
    L = q4mi.lib()
    torch.cuda.set_device(0)
    q4mi.use_torch_stream(L)
    T = q4mi.T_IQ3_S
    out = {"library": os.path.basename(q4mi.LIB_PATH)}
    out["config0_gemv"] = bench_gemv(L, torch, np, q4mi, synth, T, 4096, 4096, 80, 1, "configs[0]")
    out["config4_lmhead_n1"] = bench_gemv(L, torch, np, q4mi, synth, q4mi.T_Q8_0, 151936, 2048,
                                          2, 1, "configs[4]")
    out["config4_lmhead_n4"] = bench_gemv(L, torch, np, q4mi, synth, q4mi.T_Q8_0, 151936, 2048,
                                          2, 4, "configs[4]")
    for v in out.values():
        if isinstance(v, dict):
            v.pop("note", None)
    return out


def bench_gemv(L, torch, np, q4mi, synth, ty, rows, K, copies, nt, label, reps=30):
    """q4_mmvq_n over `copies` distinct weight copies (rotated to defeat the
    Infinity Cache); GB/s = (weights + x + y) / kernel-pair time."""
    rb = q4mi.row_bytes(ty, K)
    gen = synth.device_iq3s if ty == q4mi.T_IQ3_S else synth.device_q80
    ws = [gen(rows * rb, seed=77 + c) for c in range(copies)]
    x = torch.randn(nt, K, device="cuda")
    y = torch.empty(nt, rows, device="cuda")
    L.q4_mmvq_warm()

    def run():
        for w in ws:
            q4mi.check(L.q4_mmvq_n(ty, w.data_ptr(), rows, K, x.data_ptr(), y.data_ptr(), 1.0,
                                   nt), "q4_mmvq_n")
    run()
    torch.cuda.synchronize()

    def clock(fn):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3 / (reps * copies)
    t_eager = clock(run)
    # the same calls captured once and replayed: launch-bound host overhead
    # (a Python call per GEMV) taken out, as a serving loop's graph does
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        q4mi.use_torch_stream()
        run()
    q4mi.use_torch_stream()
    g.replay()
    torch.cuda.synchronize()
    t = clock(g.replay)
    nbytes = rows * rb + 4 * nt * K + 4 * nt * rows
    del ws, g
    return {"baseline_config": label, "us": round(t * 1e6, 2),
            "GB/s": round(nbytes / t / 1e9, 1),
            "pct_of_hbm": round(100 * nbytes / t / 1e9 / HBM_PEAK, 2),
            "us_eager": round(t_eager * 1e6, 2),
            "note": "fp32 x in, q8 quantization included (inside the GEMV blocks for <= 1024 "
                    "row tiles, else one quantize launch); us = graph replay of the %d "
                    "back-to-back calls over distinct weight copies, us_eager = the same "
                    "calls launched eagerly from Python" % copies}


if __name__ == "__main__":
    main()
