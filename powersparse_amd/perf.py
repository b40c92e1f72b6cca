"""Profiling workload and rocprofv3 summaries for the hot path.

  python -m powersparse_amd.perf workload [--config C1] [--steps 3]
      Runs, once each after one warm-up: a plain 1 GiB streaming copy
      (ps_copy_f32_async, the counter calibration: it reads and writes exactly
      1 GiB) and the bench operators of the configuration. Meant to run under
      `rocprofv3 --pmc FETCH_SIZE` and `rocprofv3 --pmc WRITE_SIZE`.

  python -m powersparse_amd.perf summarize --trace KT.db [--fetch F.db --write W.db]
        [--config C1] [--json OUT.json]
      Reads rocprofv3 SQLite result databases: per kernel the dispatch count and
      mean duration (kernel trace), and per operator kernel the HBM traffic per
      dispatch = FETCH_SIZE + WRITE_SIZE (KiB), each scaled by the factor that
      makes the calibration copy read and write exactly its size.
"""
import argparse
import collections
import json
import re
import sqlite3
import sys

CALIB_BYTES = 1 << 30

# operators of each bench configuration, in launch order (kernel, N)
CONFIG_OPS = {"C1": [("spmm", 32), ("spmm", 128), ("sddmm", 128)],
              "C3": [("spmm", 32), ("spmm", 128), ("sddmm", 128)],
              "C4": [("spmm", 64), ("sddmm", 64)]}


def short_name(name):
    name = re.sub(r"\(anonymous namespace\)::", "", name)
    return name.split("(")[0].replace("void ", "").strip()


def kernel_op(name):
    """(op, lanes-template) of an operator kernel name, else None."""
    m = re.search(r"(spmm|sddmm)_kernel<(\d+), (true|false)>", short_name(name))
    return (m.group(1), int(m.group(2))) if m else None


def op_of(op, n):
    """Operator kernel template argument for a width N (see pick_lpn / KQ)."""
    if op == "spmm":
        for lanes, width in ((64, 256), (32, 128), (16, 64)):
            if n % width == 0:
                return lanes
        return 8
    return n // 32


def workload(args):
    import numpy as np  # noqa: F401

    import powersparse_amd as ps

    ps.set_device(0)
    src = ps.DeviceBuffer(CALIB_BYTES)
    dst = ps.DeviceBuffer(CALIB_BYTES)
    ps.fill_random(src, CALIB_BYTES // 4, 7, 0.0, 1.0)
    for _ in range(2):
        ps.copy_f32(dst, src, CALIB_BYTES // 4)
    ps.synchronize()
    csr = ps.synth(args.config, seed=1)
    m = ps.PowerSparseMatrixGPU.from_csr(csr)
    rows, cols = csr.rows, csr.cols
    sizes = m.sddmm_output_sizes()
    for op, n in CONFIG_OPS[args.config]:
        if op == "spmm":
            B = ps.DeviceBuffer(cols * n * 4)
            ps.fill_random(B, cols * n, 11, -1.0, 1.0)
            C = ps.DeviceBuffer(rows * n * 4)
            C.zero()
            for _ in range(1 + args.steps):
                ps.SpMMAsync(m, n, B, C)
        else:
            X = ps.DeviceBuffer(rows * n * 4)
            Y = ps.DeviceBuffer(cols * n * 4)
            ps.fill_random(X, rows * n, 12, 0.0, 1.0, normal=True)
            ps.fill_random(Y, cols * n, 13, 0.0, 1.0, normal=True)
            outs = [ps.DeviceBuffer(max(s, 1) * 4) for s in sizes]
            for o in outs:
                o.zero()
            for _ in range(1 + args.steps):
                ps.SDDMMAsync(m, n, X, Y, outs)
        ps.synchronize()
    print(f"workload {args.config}: nnz={csr.nnz} done", flush=True)


def read_counters(db, counter):
    con = sqlite3.connect(db)
    rows = con.execute("select kernel_name, value, grid_size from counters_collection "
                       "where counter_name = ?", (counter,)).fetchall()
    out = collections.defaultdict(list)
    for name, value, grid in rows:
        out[short_name(name)].append((float(value), int(grid)))
    return out


def read_trace(db):
    con = sqlite3.connect(db)
    rows = con.execute("select name, total_calls, average from top_kernels").fetchall()
    return [(short_name(n), int(c), float(a)) for n, c, a in rows]  # average in us


def calibration(counts):
    """Scale factor bytes / (KiB * 1024) from the calibration copy dispatches:
    the copy kernel dispatch whose grid matches a 1 GiB copy."""
    vals = [v for v, g in counts.get("ps::copy_f32_kernel", [])]
    if not vals:
        return None
    return CALIB_BYTES / (max(vals) * 1024.0)


def summarize(args):
    lines = []
    trace = read_trace(args.trace)
    lines.append("| kernel | dispatches | mean duration (us) |")
    lines.append("|---|---|---|")
    for name, calls, avg in trace[:25]:
        lines.append(f"| `{name}` | {calls} | {avg:.1f} |")
    result = {"config": args.config, "kernels": {}}
    for name, calls, avg in trace:
        result["kernels"][name] = {"dispatches": calls, "mean_us": avg}
    if args.fetch and args.write:
        fetch = read_counters(args.fetch, "FETCH_SIZE")
        write = read_counters(args.write, "WRITE_SIZE")
        kf, kw = calibration(fetch), calibration(write)
        lines.append("")
        lines.append(f"Calibration (1 GiB ps::copy_f32_kernel): FETCH x{kf:.4f}, WRITE x{kw:.4f}")
        lines.append("")
        lines.append("| operator | kernel | FETCH (MB) | WRITE (MB) | HBM traffic per launch (MB) |")
        lines.append("|---|---|---|---|---|")
        result["calibration"] = {"fetch": kf, "write": kw}
        result["traffic"] = {}
        # operator dispatches appear in launch order: 1 + steps per operator
        for op, n in CONFIG_OPS[args.config]:
            tmpl = op_of(op, n)
            names = [k for k in fetch if kernel_op(k) == (op, tmpl)]
            if not names:
                continue
            f = [v for k in names for v, _ in fetch[k]]
            w = [v for k in names for v, _ in write.get(k, [])]
            fb = sum(f) / len(f) * 1024.0 * kf
            wb = sum(w) / len(w) * 1024.0 * kw if w else 0.0
            result["traffic"][f"{op}_N{n}"] = {"kernel": names[0], "fetch_bytes": fb,
                                                "write_bytes": wb, "traffic_bytes": fb + wb}
            lines.append(f"| {op} N={n} | `{names[0]}` | {fb / 1e6:.1f} | {wb / 1e6:.1f} | "
                         f"{(fb + wb) / 1e6:.1f} |")
    print("\n".join(lines))
    if args.json:
        with open(args.json, "w") as fh:
            json.dump(result, fh, indent=1)


def main(argv=None):
    ap = argparse.ArgumentParser(prog="python -m powersparse_amd.perf")
    sub = ap.add_subparsers(dest="cmd", required=True)
    w = sub.add_parser("workload")
    w.add_argument("--config", default="C1", choices=sorted(CONFIG_OPS))
    w.add_argument("--steps", type=int, default=3)
    s = sub.add_parser("summarize")
    s.add_argument("--trace", required=True)
    s.add_argument("--fetch")
    s.add_argument("--write")
    s.add_argument("--config", default="C1", choices=sorted(CONFIG_OPS))
    s.add_argument("--json")
    args = ap.parse_args(argv)
    if args.cmd == "workload":
        workload(args)
    else:
        summarize(args)
    return 0


if __name__ == "__main__":
    sys.exit(main())
