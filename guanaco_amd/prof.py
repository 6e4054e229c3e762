"""Workloads for rocprofv3 runs (the commands recorded under profiles/).

    python3 -m guanaco_amd.prof copy --mib 256 --iters 20
        the plain copy kernel (gq_hip_copy_dev) on a buffer of known size:
        the reference that scales the FETCH_SIZE / WRITE_SIZE counters into
        HBM bytes (expected per dispatch: mib MiB read and mib MiB written).

The decode workload itself is ``python3 bench.py --eager`` (one kernel launch
per op, so per-dispatch counters map onto ops).
"""
import argparse
import time

from . import hip as H


def run_copy(mib, iters):
    ctx = H.Context(0)
    n = mib << 20
    src, dst = ctx.alloc(n), ctx.alloc(n)
    for _ in range(iters):
        ctx.check(H.lib.gq_hip_copy_dev(ctx.h, dst.ptr, src.ptr, n), "copy")
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(iters):
        ctx.check(H.lib.gq_hip_copy_dev(ctx.h, dst.ptr, src.ptr, n), "copy")
    ctx.sync()
    dt = (time.perf_counter() - t0) / iters
    print(f"copy {mib} MiB: {dt * 1e6:.1f} us per launch, {2 * n / dt / 1e9:.0f} GB/s (read + write)", flush=True)
    ctx.close()


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = ap.add_subparsers(dest="cmd", required=True)
    c = sub.add_parser("copy")
    c.add_argument("--mib", type=int, default=256)
    c.add_argument("--iters", type=int, default=20)
    a = ap.parse_args()
    if a.cmd == "copy":
        run_copy(a.mib, a.iters)


if __name__ == "__main__":
    main()
