#!/usr/bin/env python3
"""Benchmark of the PowerSparse hot path on one MI355X.

One step = one pass of the hot path over the synthetic benchmark graph, each
operator one fused launch covering every workset, enqueued back to back on one
stream with the operands resident in HBM. The default is config C3, the
north-star graph (Chung-Lu n = 1.6e6, gamma 1.8, mean degree 165, degree clip
1e5, ~264 M nonzeros, values U(0,1)): SpMM at N = 32, SpMM at N = 128 and
SDDMM at N = 128, dense operands U(-1,1). `--config C1` runs the C1/C2 graph
(n = 1e6, gamma 2.1, mean 50, clip 5e4): SpMM N = 32 and 128 with B ~ U(-1,1),
SDDMM N = 128 and 32 with X, Y ~ N(0,1); `--config C4` the community graph
(SpMM and SDDMM at N = 64, operands N(0,1)). The outputs are not cleared
between calls, as in the reference harness (benchmarks/benchmark.cu:179-187).

Prints one JSON line: value = total FLOP of the timed steps (2 * nnz * N per
operator, benchmark.cu:189) / wall time between two events, in GFLOPS; the
`roofline` object is for the dominant operator (algorithmic bytes per call /
its mean call time, HIP events around the call on its stream: the fused
sparse launch, plus the dense hub block's kernels when the matrix keeps one,
`config.hub_block` = its rows x columns); `cpu_baseline` is the OpenMP
double-precision restatement of the reference's check path (the oracle) timed
on this host over a bounded row sample of the same graph and operators.
`roofline.traffic` is the bytes one operator call's kernels (the sparse
launch and the hub block's kernels) exchange between the L2 and the memory
fabric (Infinity Cache and HBM; calibrated FETCH_SIZE + WRITE_SIZE), taken
from the committed rocprofv3 summary of the same workload when that summary
was made from the current kernel sources (else null; `kernel_traffic` is the
sparse launch's share); `traffic_GBps` is the call's bytes over this run's
call time;
`profile_call_kernel_us` is the summed duration of one call's kernels in
that summary's traced bench run (`profile_call_kernels` of them: the sparse
launch and the hub block's kernels), to compare with `call_us`.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C3]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "SpMM/SDDMM GFLOPS + achieved HBM GB/s (% of roofline), N=32/128, 1 GPU"
HBM_PEAK_GBPS = 8000.0
GRAPHS = {
    "C1": "C1/C2 power-law graph (Chung-Lu n=1e6, gamma 2.1, target mean degree 50, clip 5e4)",
    "C3": "C3 power-law graph (Chung-Lu n=1.6e6, gamma 1.8, target mean degree 165, clip 1e5)",
    "C4": "C4 community graph (2048 x 1024 nodes, 2% intra, +8 inter, 5% empty, 5% singleton)",
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def algorithmic_bytes(op, nnz, rows, cols, n):
    """Compulsory HBM traffic of one call: every array touched once."""
    if op == "spmm":  # values + columns, row extents, B read, C written
        return 8 * nnz + 4 * (rows + 1) + 4 * n * cols + 4 * n * rows
    return 12 * nnz + 4 * (rows + 1) + 4 * n * rows + 4 * n * cols  # + outputs


def measured_counters(config, op, n):
    """From the committed rocprofv3 summary of the same workload
    (profiles/traffic_<config>.json, made by `python -m powersparse_amd.perf
    summarize`): HBM bytes per launch of the operator kernel (FETCH_SIZE +
    WRITE_SIZE), its L2 hit rate and VALU figures, the summary's path and a
    note. All figures are None when the summary was made from other kernel
    sources than the ones built here."""
    from powersparse_amd.perf import sources_digest

    path = os.path.join(ROOT, "profiles", f"traffic_{config}.json")
    try:
        with open(path) as fh:
            summary = json.load(fh)
    except (OSError, ValueError):
        return None, {}, None, "no profile summary"
    rel = os.path.relpath(path, ROOT)
    if summary.get("sources_digest") != sources_digest():
        return None, {}, rel, "profile summary made from other kernel sources: not used"
    key = f"{op}_N{n}"
    entry = summary.get("traffic", {}).get(key, {})
    traffic = entry.get("traffic_bytes")
    counters = dict(summary.get("counters", {}).get(key, {}))
    counters["kernel_traffic"] = entry.get("kernel_traffic_bytes")
    # the traced bench run's kernels of one call, summed (the call time this
    # run measures with events should agree)
    call = summary.get("operators", {}).get(key, {})
    counters["profile_call_kernel_us"] = call.get("kernel_us_per_call")
    counters["profile_call_kernels"] = call.get("kernels_per_call")
    return traffic, counters, rel, "from the profile summary of the same kernel sources"


def host_description():
    """nproc, the CPU model and the OpenMP thread count of this host."""
    model = None
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": len(os.sched_getaffinity(0)), "cpu_model": model}


def row_sample(csr, stride):
    """Every stride-th row of the CSR: (row ids, row_ptr, col_ind, values)."""
    rows = np.arange(0, csr.rows, stride, dtype=np.int64)
    starts = csr.row_ptr[rows].astype(np.int64)
    lens = csr.row_ptr[rows + 1].astype(np.int64) - starts
    rp = np.zeros(rows.size + 1, np.int64)
    np.cumsum(lens, out=rp[1:])
    idx = np.repeat(starts - rp[:-1], lens) + np.arange(rp[-1], dtype=np.int64)
    return rows.astype(np.int32), rp.astype(np.int32), csr.col_ind[idx], csr.values[idx]


def cpu_baseline(csr, host_ops, stride, reps=3):
    """Times the oracle (OpenMP, double accumulation) over every stride-th row
    of the graph with the same operators and operands: (median seconds per
    step, FLOP per sampled step, sampled nonzeros, threads)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    threads = oracle.max_threads()
    rows, rp, ci, sv = row_sample(csr, stride)

    def run():
        for op, n, a, b in host_ops:
            if op == "spmm":
                oracle.spmm(rp, ci, sv, n, a)
            else:  # one group per sampled row, X rows addressed by row id
                oracle.sddmm(rows, rp, ci, sv, n, a, b)

    run()  # warm-up
    times = []
    for _ in range(reps):
        t = time.perf_counter()
        run()
        times.append(time.perf_counter() - t)
    flop = sum(2.0 * ci.size * n for _, n, _, _ in host_ops)
    return float(np.median(times)), flop, int(ci.size), threads


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="C3", choices=sorted(GRAPHS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU only (the operators run on one device; "
              "multi-GPU sharding is a design note, not part of this build). Use --gpus 1.",
              file=sys.stderr)
        return 2

    import powersparse_amd as ps
    from powersparse_amd.perf import CONFIG_OPS, fill_operand

    ps.set_device(0)
    props = ps.device_props(0)
    log(f"device: {props['name']} {props['arch']} CUs={props['cu_count']}")
    t = time.perf_counter()
    csr = ps.synth(args.config, seed=1)
    gen_s = time.perf_counter() - t
    nnz, rows, cols = csr.nnz, csr.rows, csr.cols
    log(f"graph {args.config}: rows={rows} nnz={nnz} (generated in {gen_s:.1f} s)")

    ps.synchronize()
    t = time.perf_counter()
    m = ps.PowerSparseMatrixGPU.from_csr(csr)
    ps.synchronize()
    preprocess_ms = (time.perf_counter() - t) * 1e3
    S = m.GroupTypeNum()
    log(f"preprocess {preprocess_ms:.1f} ms: S={S} groups={m.GroupNum()} L={m.SignatureLen()}")

    stream = ps.Stream()
    ops = []
    seed = 100
    sizes = m.sddmm_output_sizes()
    for op, n in CONFIG_OPS[args.config]:
        seed += 1
        if op == "spmm":
            B = ps.DeviceBuffer(cols * n * 4)
            fill_operand(B, cols * n, seed, args.config, op, stream=stream)
            C = ps.DeviceBuffer(rows * n * 4)
            C.zero(stream)
            ops.append(dict(op=op, N=n, bufs=(B, C),
                            call=lambda n=n, B=B, C=C: ps.SpMMAsync(m, n, B, C, stream)))
        else:
            X = ps.DeviceBuffer(rows * n * 4)
            Y = ps.DeviceBuffer(cols * n * 4)
            fill_operand(X, rows * n, seed, args.config, op, stream=stream)
            fill_operand(Y, cols * n, seed + 50, args.config, op, stream=stream)
            outs = [ps.DeviceBuffer(max(sz, 1) * 4) for sz in sizes]
            for o in outs:
                o.zero(stream)
            ops.append(dict(op=op, N=n, bufs=(X, Y, outs),
                            call=lambda n=n, X=X, Y=Y, outs=outs: ps.SDDMMAsync(m, n, X, Y, outs,
                                                                                stream)))
    stream.synchronize()

    for _ in range(args.warmup):
        for o in ops:
            o["call"]()
    stream.synchronize()

    K = args.steps
    marks = [[ps.Event() for _ in range(len(ops) + 1)] for _ in range(K)]
    start, stop = ps.Event(), ps.Event()
    ps.synchronize()
    start.record(stream)
    for k in range(K):
        marks[k][0].record(stream)
        for i, o in enumerate(ops):
            o["call"]()
            marks[k][i + 1].record(stream)
    stop.record(stream)
    stop.synchronize()
    ps.synchronize()
    total_ms = start.elapsed_ms(stop)
    flop_step = sum(2.0 * nnz * o["N"] for o in ops)
    value = flop_step * K / (total_ms * 1e-3) / 1e9

    detail = []
    for i, o in enumerate(ops):
        ms = float(np.mean([marks[k][i].elapsed_ms(marks[k][i + 1]) for k in range(K)]))
        alg = algorithmic_bytes(o["op"], nnz, rows, cols, o["N"])
        detail.append({"op": o["op"], "N": o["N"], "ms": ms,
                       "gflops": 2.0 * nnz * o["N"] / (ms * 1e-3) / 1e9,
                       "alg_bytes": alg, "alg_GBps": alg / (ms * 1e-3) / 1e9,
                       "roofline_frac": alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS})
        log(f"{o['op']} N={o['N']}: {ms:.3f} ms  {detail[-1]['gflops']:.1f} GFLOPS  "
            f"{detail[-1]['alg_GBps']:.0f} GB/s ({100 * detail[-1]['roofline_frac']:.1f}% of 8 TB/s)")
    dom = max(detail, key=lambda d: d["ms"])
    kernel = "ps::spmm_kernel" if dom["op"] == "spmm" else "ps::sddmm_kernel"
    if m.hub_block:
        kernel += (" + the hub block's MFMA kernels ("
                   + ("B transpose, ps::hub_spmm_kernel, fix-up" if dom["op"] == "spmm"
                      else "ps::hub_sddmm_kernel") + ")")
    traffic, counters, traffic_src, traffic_note = measured_counters(args.config, dom["op"],
                                                                      dom["N"])

    cpu = None
    if not args.no_cpu_baseline:
        host_ops = []
        for o in ops:
            if o["op"] == "spmm":
                B, _ = o["bufs"]
                host_ops.append(("spmm", o["N"], B.download(np.float32).reshape(cols, o["N"]),
                                 None))
            else:
                X, Y, _ = o["bufs"]
                host_ops.append(("sddmm", o["N"], X.download(np.float32).reshape(rows, o["N"]),
                                 Y.download(np.float32).reshape(cols, o["N"])))
        # about 64 M sampled nonzeros: every row of C1 and C4, every 4th of C3
        stride = max(1, int(round(nnz / 64e6)))
        cpu_s, cpu_flop, cpu_nnz, threads = cpu_baseline(csr, host_ops, stride)
        host = host_description()
        cpu = {"value": cpu_flop / cpu_s / 1e9, "unit": "GFLOPS", "cores": threads,
               "kind": "port", "nproc": host["nproc"], "cpu_model": host["cpu_model"],
               "omp_threads": threads,
               "sample": f"every {stride} row(s) of the {args.config} graph ({cpu_nnz} of "
                         f"{nnz} nonzeros), one step ("
                         + ", ".join(f"{o['op']} N={o['N']}" for o in ops)
                         + "), oracle/oracle.cpp OpenMP double accumulation, median of 3 "
                           f"after 1 warm-up, {cpu_s:.2f} s per sampled step"}
        log(f"cpu baseline: {cpu['value']:.2f} GFLOPS on {threads} threads "
            f"({host['nproc']} CPUs, {host['cpu_model']})")

    line = {
        "metric": METRIC, "value": value, "unit": "GFLOPS", "n_gpus": 1, "steps": K,
        "warmup": args.warmup, "ms_per_step": total_ms / K, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
        "config": {"workload": f"{GRAPHS[args.config]}: {nnz} nonzeros, realized mean degree "
                               f"{nnz / rows:.1f}; "
                               + " + ".join(f"{o['op'].replace('spmm', 'SpMM').replace('sddmm', 'SDDMM')}"
                                            f" N={o['N']}" for o in ops),
                   "graph": args.config, "rows": rows,
                   "nnz": nnz, "worksets": S, "group_num": m.GroupNum(),
                   "hub_block": list(m.hub_block),
                   "preprocess_ms": preprocess_ms, "parallelism": "single GPU",
                   "device": (f"{props['name']} " if props["name"].strip() else "")
                             + f"({props['arch'].split(':')[0]}, {props['cu_count']} CUs)"},
        "ops": detail,
        "roofline": {"bound": "hbm", "kernel": kernel, "op": f"{dom['op']} N={dom['N']}",
                     "achieved": dom["alg_GBps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": dom["roofline_frac"], "traffic": traffic,
                     # bytes the L2 exchanged with the memory fabric per
                     # operator call (Infinity Cache hits and HBM together),
                     # over this run's call time
                     "traffic_scope": "per operator call: L2 to memory fabric (Infinity "
                                      "Cache and HBM), calibrated FETCH_SIZE + WRITE_SIZE, "
                                      "summed over the call's kernels (sparse launch and "
                                      "hub block)",
                     "kernel_traffic": counters.get("kernel_traffic"),
                     "traffic_GBps": traffic / (dom["ms"] * 1e-3) / 1e9 if traffic else None,
                     "l2_hit_pct": counters.get("l2_hit_pct"),
                     "valu_busy_pct": counters.get("valu_busy_pct"),
                     "valu_utilization_pct": counters.get("valu_utilization_pct"),
                     "call_us": dom["ms"] * 1e3,
                     "profile_call_kernel_us": counters.get("profile_call_kernel_us"),
                     "profile_call_kernels": counters.get("profile_call_kernels"),
                     "traffic_source": traffic_src, "traffic_note": traffic_note},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
