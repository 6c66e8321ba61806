"""Copy of a known size, for calibrating HBM byte counters.

`python copycal.py [MiB] [reps]` (repo root, beside bench.py) copies a MiB-sized device buffer to
another `reps` times (torch's device copy kernel).  Under
`rocprofv3 --pmc FETCH_SIZE` (or WRITE_SIZE) each dispatch should report
MiB * 1024 KiB; the ratio of the reported to the known size is the factor
that converts the counter readings of the library's kernels into bytes.
"""
import sys


def main():
    import torch
    mib = int(sys.argv[1]) if len(sys.argv) > 1 else 256
    reps = int(sys.argv[2]) if len(sys.argv) > 2 else 3
    n = mib * (1 << 20) // 4
    src = torch.ones(n, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"copied {mib} MiB x {reps} (expect {mib * 1024} KiB read and written per dispatch)")


if __name__ == "__main__":
    main()
