"""Build the HIP library (gfx950) in-tree: lib/libq4mi.so.

Every source under csrc/ is compiled by hipcc for gfx950 only and linked
into one shared object exposing the C ABI declared in include/q4mi.h.  The
same sources compiled with -DQ4MI_MEASURE give lib/libq4mi_meas.so, which
adds the measurement hooks of include/q4mi_measure.h (benchmarks and the
LDS-ring tests load it; the product library never exports them).
"""
import concurrent.futures as cf
import glob
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "lib", "libq4mi.so")
MEAS_LIB = os.path.join(PKG, "lib", "libq4mi_meas.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "-O3", "--offload-arch=gfx950", "-std=c++17", "-fPIC",
    # Packed FP32 instructions stay off (the hardware's packed forms are not
    # trusted on this pool); the host pass ignores the feature with a warning.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Wall", "-Wno-unused-function", "-Wno-unknown-pragmas",
]


def _compile(job):
    src, variant = job
    obj = os.path.join(OBJ, variant, os.path.basename(src).replace(".hip", ".o"))
    extra = ["-DQ4MI_MEASURE"] if variant == "meas" else []
    cmd = [HIPCC] + FLAGS + extra + ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l
                    and "target-feature" not in l)
    return obj, r.returncode, err


def _link(objs, lib):
    tmp = lib + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stderr)
        raise RuntimeError("link failed: " + lib)
    os.replace(tmp, lib)


def build_variant(lib, defines, verbose=False):
    """A measurement-build variant with extra preprocessor defines (e.g. the
    MMQ timing knockouts, Q4MI_MMQ_KO=bits, or the decode phase trace,
    Q4MI_TRACE) linked into `lib`; objects go to _build/<lib name>."""
    tag = os.path.splitext(os.path.basename(lib))[0]
    odir = os.path.join(OBJ, tag)
    os.makedirs(odir, exist_ok=True)
    os.makedirs(os.path.dirname(os.path.abspath(lib)), exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")), key=lambda p: -os.path.getsize(p))
    extra = ["-DQ4MI_MEASURE"] + ["-D" + d for d in defines]

    def one(src):
        obj = os.path.join(odir, os.path.basename(src).replace(".hip", ".o"))
        r = subprocess.run([HIPCC] + FLAGS + extra + ["-c", src, "-o", obj], capture_output=True,
                           text=True)
        return obj, r.returncode, r.stderr

    with cf.ThreadPoolExecutor(min(len(srcs), int(os.environ.get("MAX_JOBS", "8")))) as ex:
        res = list(ex.map(one, srcs))
    for obj, rc, err in res:
        if rc != 0:
            sys.stderr.write(err + "\n")
            raise RuntimeError("hipcc failed for " + obj)
    _link([r[0] for r in res], lib)
    return lib


def build(verbose=False, measure=True):
    variants = ["prod", "meas"] if measure else ["prod"]
    for v in variants:
        os.makedirs(os.path.join(OBJ, v), exist_ok=True)
    os.makedirs(os.path.dirname(LIB), exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    # the longest compiles first, so the pool stays busy to the end
    srcs.sort(key=lambda p: -os.path.getsize(p))
    work = [(s, v) for s in srcs for v in variants]
    jobs = min(len(work), int(os.environ.get("MAX_JOBS", "8")))
    objs = {v: [] for v in variants}
    with cf.ThreadPoolExecutor(jobs) as ex:
        for (src, v), (obj, rc, err) in zip(work, ex.map(_compile, work)):
            if rc != 0:
                sys.stderr.write(err + "\n")
                raise RuntimeError("hipcc failed for " + obj)
            if verbose and err.strip():
                sys.stderr.write(err + "\n")
            objs[v].append(obj)
    _link(objs["prod"], LIB)
    if measure:
        _link(objs["meas"], MEAS_LIB)
    return LIB


if __name__ == "__main__":
    import argparse
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--lib", help="build a measurement variant into this path instead")
    ap.add_argument("--define", action="append", default=[],
                    help="NAME[=VALUE] for the variant (repeatable)")
    args = ap.parse_args()
    if args.lib:
        print(build_variant(args.lib, args.define, verbose=True))
    else:
        print(build(verbose=True))
