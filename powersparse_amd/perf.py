"""Profiling workload and rocprofv3 summaries for the hot path.

  python -m powersparse_amd.perf workload [--config C1] [--steps 3]
      Runs, once each after one warm-up: a plain 1 GiB streaming copy
      (ps_perf_copy_f32_async from lib/libpowersparse_perf.so, `make -C
      powersparse_amd perf`; the counter calibration: it reads and writes
      exactly 1 GiB) and the bench operators of the configuration. Meant to run
      under `rocprofv3 --pmc FETCH_SIZE` and `rocprofv3 --pmc WRITE_SIZE`.

  python -m powersparse_amd.perf csr [--config C1] [--n 128]
      Times the SDDMM output orders on one matrix built with csr_positions:
      workset order (SDDMMAsync), input-CSR order in one launch (SDDMMToCSR),
      and workset order followed by the permutation (SDDMMAsync +
      WorksetToCSR); mean of 20 calls after one warm-up, HIP events.

  python -m powersparse_amd.perf summarize --trace KT.db [--fetch F.db --write W.db]
        [--l2 L.db] [--valu V.db] [--config C1] [--json OUT.json]
      Reads rocprofv3 SQLite result databases: per kernel the dispatch count and
      mean duration (kernel trace); per operator call (the sparse launch and the
      dense hub block's kernels after it) and per sparse launch alone, the
      traffic between the L2 and the memory fabric = FETCH_SIZE + WRITE_SIZE
      (KiB), each scaled by the factor that makes the calibration copy read and
      write exactly its size; with --l2 (a `--pmc TCC_HIT_sum TCC_MISS_sum`
      pass) the L2 hit rate of the whole call, with --valu (a `--pmc VALUBusy
      VALUUtilization` pass) the share of time the VALUs issue and the share of
      active lanes per VALU instruction of the sparse launch; means over the
      operator's calls.
"""
import argparse
import collections
import json
import re
import sqlite3
import sys

import numpy as np

CALIB_BYTES = 1 << 30

# operators of each bench configuration, in launch order (kernel, N)
CONFIG_OPS = {"C1": [("spmm", 32), ("spmm", 128), ("sddmm", 128), ("sddmm", 32)],
              "C3": [("spmm", 32), ("spmm", 128), ("sddmm", 128)],
              "C4": [("spmm", 64), ("sddmm", 64)]}

# Dense operand distributions of each configuration: SpMM's B, SDDMM's X and Y,
# as ("uniform", lo, hi) or ("normal", mean, std). C1: B ~ U(-1, 1); C2 (the
# SDDMM of C1's pattern): X, Y ~ N(0, 1); C3: every dense operand U(-1, 1);
# C4: every dense operand N(0, 1).
OPERANDS = {"C1": {"spmm": ("uniform", -1.0, 1.0), "sddmm": ("normal", 0.0, 1.0)},
            "C3": {"spmm": ("uniform", -1.0, 1.0), "sddmm": ("uniform", -1.0, 1.0)},
            "C4": {"spmm": ("normal", 0.0, 1.0), "sddmm": ("normal", 0.0, 1.0)}}


def fill_operand(buf, count, seed, config, op, stream=None):
    """Fills a device operand of `config`'s operator `op` on the device."""
    import powersparse_amd as ps

    kind, a, b = OPERANDS[config][op]
    ps.fill_random(buf, count, seed, a, b, normal=kind == "normal", stream=stream)


def host_operand(rng, shape, config, op):
    """A host (numpy float32) operand with `config`'s distribution for `op`."""
    kind, a, b = OPERANDS[config][op]
    if kind == "normal":
        return (a + b * rng.standard_normal(shape)).astype(np.float32)
    return rng.uniform(a, b, shape).astype(np.float32)


def code_text(source):
    """The code of a C / C++ / HIP source: comments and blank lines removed and
    runs of whitespace folded (the sources hold no comment markers inside
    string literals)."""
    source = re.sub(r"/\*.*?\*/", " ", source, flags=re.S)
    source = re.sub(r"//[^\n]*", "", source)
    lines = (" ".join(line.split()) for line in source.split("\n"))
    return "\n".join(line for line in lines if line)


def sources_digest(root=None):
    """SHA-256 over the code of the kernel sources and the C ABI header (their
    comments left out): ties a committed profile summary to the kernels it
    measured."""
    import glob
    import hashlib
    import os

    root = root or os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    files = sorted(glob.glob(os.path.join(root, "powersparse_amd", "csrc", "*.hip")) +
                   glob.glob(os.path.join(root, "powersparse_amd", "csrc", "*.hpp")) +
                   [os.path.join(root, "include", "powersparse_hip.h")])
    h = hashlib.sha256()
    for f in files:
        h.update(os.path.basename(f).encode())
        with open(f, encoding="utf-8") as fh:
            h.update(code_text(fh.read()).encode())
    return h.hexdigest()[:16]


def short_name(name):
    name = re.sub(r"\(anonymous namespace\)::", "", name)
    return name.split("(")[0].replace("void ", "").strip()


def kernel_op(name):
    """(op, lanes-template) of an operator kernel name, else None."""
    # spmm_kernel<lanes, buf>, sddmm_kernel<KQ, buf, store mode>; the hub
    # block's kernels (hub_spmm_kernel<..>, hub_sddmm_kernel<..>) are not
    m = re.search(r"(?:^|::)(spmm|sddmm)_kernel<(\d+), (true|false)(, \d+)?>", short_name(name))
    return (m.group(1), int(m.group(2))) if m else None


def copy_f32(dst, src, count, stream=None):
    """The calibration copy: a plain streaming device copy of `count` floats."""
    import powersparse_amd as ps
    from powersparse_amd import _native

    ps._hip_call(_native.perf_lib().ps_perf_copy_f32_async(
        ps._ptr(dst), ps._ptr(src), int(count), ps._ptr(stream)))


def workload(args):
    import numpy as np  # noqa: F401

    import powersparse_amd as ps

    ps.set_device(0)
    src = ps.DeviceBuffer(CALIB_BYTES)
    dst = ps.DeviceBuffer(CALIB_BYTES)
    ps.fill_random(src, CALIB_BYTES // 4, 7, 0.0, 1.0)
    for _ in range(2):
        copy_f32(dst, src, CALIB_BYTES // 4)
    ps.synchronize()
    csr = ps.synth(args.config, seed=1)
    m = ps.PowerSparseMatrixGPU.from_csr(csr)
    rows, cols = csr.rows, csr.cols
    sizes = m.sddmm_output_sizes()
    for op, n in CONFIG_OPS[args.config]:
        if op == "spmm":
            B = ps.DeviceBuffer(cols * n * 4)
            fill_operand(B, cols * n, 11, args.config, op)
            C = ps.DeviceBuffer(rows * n * 4)
            C.zero()
            for _ in range(1 + args.steps):
                ps.SpMMAsync(m, n, B, C)
        else:
            X = ps.DeviceBuffer(rows * n * 4)
            Y = ps.DeviceBuffer(cols * n * 4)
            fill_operand(X, rows * n, 12, args.config, op)
            fill_operand(Y, cols * n, 13, args.config, op)
            outs = [ps.DeviceBuffer(max(s, 1) * 4) for s in sizes]
            for o in outs:
                o.zero()
            for _ in range(1 + args.steps):
                ps.SDDMMAsync(m, n, X, Y, outs)
        ps.synchronize()
    print(f"workload {args.config}: nnz={csr.nnz} done", flush=True)


def csr_order(args):
    """Times the SDDMM output orders (workset / CSR / workset + permutation)."""
    import powersparse_amd as ps

    ps.set_device(0)
    csr = ps.synth(args.config, seed=1)
    m = ps.PowerSparseMatrixGPU.from_csr(csr, csr_positions=True)
    n, rows, cols = args.n, csr.rows, csr.cols
    st = ps.Stream()
    X = ps.DeviceBuffer(rows * n * 4)
    Y = ps.DeviceBuffer(cols * n * 4)
    ps.fill_random(X, rows * n, 12, 0.0, 1.0, normal=True, stream=st)
    ps.fill_random(Y, cols * n, 13, 0.0, 1.0, normal=True, stream=st)
    outs = [ps.DeviceBuffer(max(sz, 1) * 4) for sz in m.sddmm_output_sizes()]
    for o in outs:
        o.zero(st)
    out_csr = ps.DeviceBuffer(csr.nnz * 4)
    t0, t1 = ps.Event(), ps.Event()

    def timed(fn, reps=20):
        fn()
        t0.record(st)
        for _ in range(reps):
            fn()
        t1.record(st)
        t1.synchronize()
        return t0.elapsed_ms(t1) / reps

    def workset_then_csr():
        ps.SDDMMAsync(m, n, X, Y, outs, st)
        ps.WorksetToCSR(m, outs, out_csr, st)

    rows_out = [("workset order (SDDMMAsync)", timed(lambda: ps.SDDMMAsync(m, n, X, Y, outs, st))),
                ("CSR order, one launch (SDDMMToCSR)",
                 timed(lambda: ps.SDDMMToCSR(m, n, X, Y, out_csr, st))),
                ("workset order + WorksetToCSR", timed(workset_then_csr))]
    print(f"SDDMM output order, {args.config} (nnz {csr.nnz}, task order {m.task_order}), "
          f"N = {n}\n\n| output | ms per call |\n|---|---|")
    for name, ms in rows_out:
        print(f"| {name} | {ms:.3f} |")


# ------------------------------------------------ per-class traffic split

def _class_worksets(m, keep=None):
    """ps_workset array of m's public worksets; with `keep`, every other
    workset emptied (group_num 0), so that a launch runs that class alone."""
    from powersparse_amd import _native

    S = m.GroupTypeNum()
    arr = (_native.Workset * S)()
    cps, vps, dps, gn = m.WorksetColInd(), m.WorksetSpData(), m.GroupDestination(), m.GroupNum()
    for s in range(S):
        g = gn[s] if keep is None or keep == s else 0
        arr[s] = _native.Workset(cps[s], vps[s], dps[s], g, 0 if s == 0 else 32 << (s - 1), None)
    return arr


def classes(args):
    """The sparse kernels one workset class at a time: SDDMM N = args.n on the
    public partition in the locality run order, SpMM N = args.n on the tuned
    partition (3 worksets, signature order), each first with every class and
    then with one class kept (the others emptied), `args.reps` launches each,
    on the matrix without the dense hub block. Prints one manifest line per
    launch group (JSON) for `classes-summarize`."""
    import ctypes
    import json

    import powersparse_amd as ps
    from powersparse_amd import _native

    ps.set_device(0)
    src = ps.DeviceBuffer(CALIB_BYTES)
    dst = ps.DeviceBuffer(CALIB_BYTES)
    ps.fill_random(src, CALIB_BYTES // 4, 7, 0.0, 1.0)
    for _ in range(2):
        copy_f32(dst, src, CALIB_BYTES // 4)
    ps.synchronize()
    cfg, n, reps = args.config, args.n, args.reps
    csr = ps.synth(cfg, seed=1)
    rows, cols = csr.rows, csr.cols
    hip = _native.hip()

    def nnz_of(m, s):
        if s != 0:
            return int(m.GroupNum()[s]) * (32 << (s - 1))
        return int(csr.nnz) - sum(int(m.GroupNum()[k]) * (32 << (k - 1))
                                  for k in range(1, m.GroupTypeNum()))

    def groups(m, op):
        out = [("all", None, int(csr.nnz))]
        for s in range(m.GroupTypeNum() - 1, -1, -1):
            if m.GroupNum()[s]:
                label = "residue" if s == 0 else f"groups of {32 << (s - 1)}"
                out.append((label, s, nnz_of(m, s)))
        return out

    # SDDMM: public partition, locality run order (the product's order)
    m = ps.PowerSparseMatrixGPU.from_csr(csr, hub_block="off")
    S = m.GroupTypeNum()
    X = ps.DeviceBuffer(rows * n * 4)
    Y = ps.DeviceBuffer(cols * n * 4)
    fill_operand(X, rows * n, 12, cfg, "sddmm")
    fill_operand(Y, cols * n, 13, cfg, "sddmm")
    outs = [ps.DeviceBuffer(max(k, 1) * 4) for k in m.sddmm_output_sizes()]
    oa = (ctypes.c_void_p * S)(*[o.ptr for o in outs])
    for label, keep, nnz in groups(m, "sddmm"):
        arr = _class_worksets(m, keep)
        count = ctypes.c_uint32()
        ps._hip_call(hip.ps_task_count(_native.PS_OP_SDDMM, n, S, arr, ctypes.byref(count)))
        order = ps.DeviceBuffer(max(count.value, 1) * 4)
        ps._hip_call(hip.ps_task_order_build(_native.PS_OP_SDDMM, n, S, arr, order.ptr,
                                             count.value, None))
        for _ in range(reps):
            ps._hip_call(hip.ps_sddmm_launch_ordered(
                S, arr, m.ResidueOffset(), rows, cols, n, X.ptr, Y.ptr, oa,
                _native.PS_TASK_CHUNK_AUTO, order.ptr, count.value, None))
        ps.synchronize()
        print(json.dumps({"op": "sddmm", "N": n, "class": label, "nnz": nnz,
                          "tasks": count.value, "launches": reps}), flush=True)
    del outs, X, Y
    m.close()
    # SpMM: the tuned partition as the product builds it without a hub block
    m = ps.PowerSparseMatrixGPU.from_csr(csr, hub_block="off", max_group_types=3,
                                         spmm_partition="parity", run_order=False,
                                         task_order="signature")
    S = m.GroupTypeNum()
    B = ps.DeviceBuffer(cols * n * 4)
    fill_operand(B, cols * n, 11, cfg, "spmm")
    C = ps.DeviceBuffer(rows * n * 4)
    C.zero()
    for label, keep, nnz in groups(m, "spmm"):
        arr = _class_worksets(m, keep)
        count = ctypes.c_uint32()
        ps._hip_call(hip.ps_task_count(_native.PS_OP_SPMM, n, S, arr, ctypes.byref(count)))
        for _ in range(reps):
            ps._hip_call(hip.ps_spmm_launch(S, arr, m.ResidueOffset(), m.ResidueAtomic(), rows,
                                            cols, n, B.ptr, C.ptr, _native.PS_TASK_CHUNK_AUTO,
                                            None))
        ps.synchronize()
        print(json.dumps({"op": "spmm", "N": n, "class": label, "nnz": nnz,
                          "tasks": count.value, "launches": reps}), flush=True)
    m.close()
    print(f"classes {cfg}: nnz={csr.nnz} done", flush=True)


def classes_summarize(args):
    """Markdown table of the `classes` launches: per class its nonzeros, mean
    launch time (kernel trace) and calibrated FETCH_SIZE + WRITE_SIZE (bytes
    per launch and per nonzero); the operator-kernel dispatches are matched to
    the manifest lines in order."""
    import json

    manifest = [json.loads(line) for line in open(args.manifest)
                if line.startswith("{") and '"class"' in line]
    durs = [d for k, _, d in read_dispatches(args.trace) if kernel_op(k) is not None]
    fetch = read_counters(args.fetch, "FETCH_SIZE")
    write = read_counters(args.write, "WRITE_SIZE")
    fscale, wscale = calibration(fetch), calibration(write)
    fv = [v for k, _, v in fetch if kernel_op(k) is not None]
    wv = [v for k, _, v in write if kernel_op(k) is not None]
    need = sum(e["launches"] for e in manifest)
    if not (len(durs) == len(fv) == len(wv) == need):
        raise SystemExit(f"dispatch counts differ: trace {len(durs)}, FETCH {len(fv)}, "
                         f"WRITE {len(wv)}, manifest {need}")
    lines = ["| operator | class | nonzeros (M) | tasks | us per launch | fabric MB per launch "
             "(FETCH + WRITE) | bytes per nonzero | share of the all-class bytes |",
             "|---|---|---|---|---|---|---|---|"]
    i, total = 0, {}
    for e in manifest:
        k = e["launches"]
        us = sum(durs[i:i + k]) / k
        mb = (sum(fv[i:i + k]) * 1024 * fscale + sum(wv[i:i + k]) * 1024 * wscale) / k / 1e6
        i += k
        key = (e["op"], e["N"])
        if e["class"] == "all":
            total[key] = mb
        share = f"{100 * mb / total[key]:.1f}%" if key in total and e["class"] != "all" else ""
        lines.append(f"| {e['op']} N={e['N']} | {e['class']} | {e['nnz'] / 1e6:.1f} | "
                     f"{e['tasks']} | {us:.1f} | {mb:.1f} | {mb * 1e6 / max(e['nnz'], 1):.1f} | "
                     f"{share} |")
    print("\n".join(lines))


# The dense hub block's kernels of an operator call (they follow the sparse
# launch on its stream).
HUB_KERNEL = re.compile(r"(?:^|::)(hub_spmm_kernel|hub_sddmm_kernel|gather_hot_kernel|"
                        r"gather_rows_kernel|clear_flags_kernel|fixup_kernel)\b")


def is_hub_kernel(name):
    return HUB_KERNEL.search(short_name(name)) is not None


def read_counters(db, counter):
    """[(kernel, grid, value)] of every dispatch, in dispatch order."""
    con = sqlite3.connect(db)
    rows = con.execute("select kernel_name, grid_size, value from counters_collection "
                       "where counter_name = ? order by dispatch_id", (counter,)).fetchall()
    return [(short_name(k), int(g), float(v)) for k, g, v in rows]


def counter_means(db, counter, ops):
    """{op_N: mean of `counter` over that operator's dispatches}, the runs of
    operator dispatches matched to `ops` in launch order."""
    runs = operator_runs(read_counters(db, counter))
    return {f"{op}_N{n}": sum(v) / len(v) for (op, n), (_, v) in zip(ops, runs)}


def l2_hit_means(db, ops):
    """{op_N: L2 hit rate in percent of one operator call, 100 * TCC_HIT /
    (TCC_HIT + TCC_MISS) summed over the call's kernels (the sparse launch and
    the hub block's kernels), mean over the calls} (rocprofv3 defines no
    L2CacheHit metric for gfx950)."""
    hits, misses = read_counters(db, "TCC_HIT_sum"), read_counters(db, "TCC_MISS_sum")
    hr = call_runs(hits)
    mr = call_runs(misses)
    out = {}
    for (op, n), (_, hv, _), (_, mv, _) in zip(ops, hr, mr):
        rates = [100.0 * h / (h + m) if h + m > 0 else 0.0 for h, m in zip(hv, mv)]
        out[f"{op}_N{n}"] = sum(rates) / len(rates)
    return out


def read_trace(db):
    """Per (kernel, grid): dispatches and mean duration in us, busiest first."""
    con = sqlite3.connect(db)
    rows = con.execute("select name, grid_x * grid_y * grid_z, count(*), avg(duration) "
                       "from kernels group by name, grid_x * grid_y * grid_z").fetchall()
    out = [(short_name(n), int(g), int(c), float(d) / 1e3) for n, g, c, d in rows]
    return sorted(out, key=lambda r: -r[2] * r[3])


def read_dispatches(db):
    """(kernel, grid, duration in us) of every dispatch, in start order."""
    con = sqlite3.connect(db)
    cols = [d[0] for d in con.execute("select * from kernels limit 1").description]
    order = "start" if "start" in cols else "rowid"
    rows = con.execute(f"select name, grid_x * grid_y * grid_z, duration from kernels "
                       f"order by {order}").fetchall()
    return [(short_name(n), int(g), float(d) / 1e3) for n, g, d in rows]


def operator_calls(dispatches, ops):
    """{op_N: (calls, kernels per call, mean summed kernel time per call in us)}.
    A call is an operator kernel's dispatch with the dispatches after it up to
    the next operator kernel (the dense hub block's kernels follow the sparse
    launch); calls take the workload's operators in turn."""
    calls = []
    for k, _, d in dispatches:
        if kernel_op(k) is not None:
            calls.append([d])
        elif calls:
            calls[-1].append(d)
    out = {}
    for i, (op, n) in enumerate(ops):
        mine = calls[i::len(ops)]
        if mine:
            out[f"{op}_N{n}"] = (len(mine), max(len(c) for c in mine),
                                 sum(sum(c) for c in mine) / len(mine))
    return out


def call_runs(dispatches):
    """Groups dispatches into operator calls (an operator kernel's dispatch and
    the hub block's kernels after it; other kernels belong to no call) and the
    calls into runs of equal (operator kernel, grid), in order: [((kernel,
    grid), [summed value per call], kernels per call)], one run per operator
    of the workload."""
    calls = []
    for k, g, v in dispatches:
        if kernel_op(k) is not None:
            calls.append(((k, g), [v]))
        elif calls and is_hub_kernel(k):
            calls[-1][1].append(v)
    runs = []
    for key, vals in calls:
        if runs and runs[-1][0] == key:
            runs[-1][1].append(sum(vals))
            runs[-1][2] = max(runs[-1][2], len(vals))
        else:
            runs.append([key, [sum(vals)], len(vals)])
    return [tuple(r) for r in runs]


def operator_runs(dispatches):
    """Groups operator-kernel dispatches into runs of equal (kernel, grid), in
    order: one run per operator of the workload."""
    runs = []
    for k, g, v in dispatches:
        if kernel_op(k) is None:
            continue
        if runs and runs[-1][0] == (k, g):
            runs[-1][1].append(v)
        else:
            runs.append(((k, g), [v]))
    return runs


def calibration(dispatches):
    """bytes / (KiB * 1024) that makes the 1 GiB calibration copy exact."""
    vals = [v for k, _, v in dispatches if k == "ps::copy_f32_kernel"]
    return CALIB_BYTES / (max(vals) * 1024.0) if vals else None


def summarize(args):
    lines = ["| kernel | grid (work-items) | dispatches | mean duration (us) |",
             "|---|---|---|---|"]
    trace = read_trace(args.trace)
    # the kernel sources these counters belong to; bench.py drops the figures
    # when its own sources differ
    result = {"config": args.config, "sources_digest": sources_digest(), "kernels": []}
    for name, grid, calls, avg in trace:
        result["kernels"].append({"kernel": name, "grid": grid, "dispatches": calls,
                                  "mean_us": avg})
    for name, grid, calls, avg in trace[:25]:
        lines.append(f"| `{name}` | {grid} | {calls} | {avg:.1f} |")
    per_op = operator_calls(read_dispatches(args.trace), CONFIG_OPS[args.config])
    if per_op:
        # what bench.py times with events around each call: the sparse launch
        # and, with the dense hub block, its GEMM, gather and sampling kernels
        lines += ["", "| operator | calls | kernels per call | summed kernel time per call (us) |",
                  "|---|---|---|---|"]
        result["operators"] = {}
        for key, (calls, kernels, us) in per_op.items():
            result["operators"][key] = {"calls": calls, "kernels_per_call": kernels,
                                        "kernel_us_per_call": us}
            op, n = key.rsplit("_N", 1)
            lines.append(f"| {op} N={n} | {calls} | {kernels} | {us:.1f} |")
    if args.fetch and args.write:
        fetch = read_counters(args.fetch, "FETCH_SIZE")
        write = read_counters(args.write, "WRITE_SIZE")
        kf, kw = calibration(fetch), calibration(write)
        lines += ["", f"Calibration (1 GiB ps::copy_f32_kernel): FETCH x{kf:.4f}, "
                      f"WRITE x{kw:.4f}", "",
                  "Per operator call (the sparse launch and the hub block's kernels), and of "
                  "the sparse launch alone:", "",
                  "| operator | kernels per call | FETCH (MB) | WRITE (MB) | traffic per call (MB) "
                  "| sparse kernel | its traffic per launch (MB) |",
                  "|---|---|---|---|---|---|---|"]
        result["calibration"] = {"fetch": kf, "write": kw}
        result["traffic"] = {}
        fr, wr = operator_runs(fetch), operator_runs(write)
        fc, wc = call_runs(fetch), call_runs(write)
        for (op, n), ((k, g), fv), (_, wv), (_, fcv, kpc), (_, wcv, _) in zip(
                CONFIG_OPS[args.config], fr, wr, fc, wc):
            fb = sum(fcv) / len(fcv) * 1024.0 * kf
            wb = sum(wcv) / len(wcv) * 1024.0 * kw
            kfb = sum(fv) / len(fv) * 1024.0 * kf
            kwb = sum(wv) / len(wv) * 1024.0 * kw
            result["traffic"][f"{op}_N{n}"] = {
                "kernel": k, "grid": g, "kernels_per_call": kpc, "fetch_bytes": fb,
                "write_bytes": wb, "traffic_bytes": fb + wb, "kernel_fetch_bytes": kfb,
                "kernel_write_bytes": kwb, "kernel_traffic_bytes": kfb + kwb}
            lines.append(f"| {op} N={n} | {kpc} | {fb / 1e6:.1f} | {wb / 1e6:.1f} | "
                         f"{(fb + wb) / 1e6:.1f} | `{k}` | {(kfb + kwb) / 1e6:.1f} |")
    if args.l2 or args.valu:
        ops = CONFIG_OPS[args.config]
        l2 = l2_hit_means(args.l2, ops) if args.l2 else {}
        busy = counter_means(args.valu, "VALUBusy", ops) if args.valu else {}
        util = counter_means(args.valu, "VALUUtilization", ops) if args.valu else {}
        lines += ["", "L2 hit rate per operator call; VALU figures of the sparse launch:", "",
                  "| operator | L2 hit rate (%) | VALU busy (%) | VALU lanes active (%) |",
                  "|---|---|---|---|"]
        result["counters"] = {}
        for op, n in ops:
            key = f"{op}_N{n}"
            c = {"l2_hit_pct": l2.get(key), "valu_busy_pct": busy.get(key),
                 "valu_utilization_pct": util.get(key)}
            result["counters"][key] = c
            lines.append(f"| {op} N={n} | " + " | ".join(
                "-" if v is None else f"{v:.1f}" for v in c.values()) + " |")
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
    c = sub.add_parser("csr")
    c.add_argument("--config", default="C1", choices=sorted(CONFIG_OPS))
    c.add_argument("--n", type=int, default=128)
    k = sub.add_parser("classes")
    k.add_argument("--config", default="C3", choices=sorted(CONFIG_OPS))
    k.add_argument("--n", type=int, default=128)
    k.add_argument("--reps", type=int, default=3)
    ks = sub.add_parser("classes-summarize")
    ks.add_argument("--manifest", required=True)
    ks.add_argument("--trace", required=True)
    ks.add_argument("--fetch", required=True)
    ks.add_argument("--write", required=True)
    s = sub.add_parser("summarize")
    s.add_argument("--trace", required=True)
    s.add_argument("--fetch")
    s.add_argument("--write")
    s.add_argument("--l2")
    s.add_argument("--valu")
    s.add_argument("--config", default="C1", choices=sorted(CONFIG_OPS))
    s.add_argument("--json")
    args = ap.parse_args(argv)
    if args.cmd == "workload":
        workload(args)
    elif args.cmd == "csr":
        csr_order(args)
    elif args.cmd == "classes":
        classes(args)
    elif args.cmd == "classes-summarize":
        classes_summarize(args)
    else:
        summarize(args)
    return 0


if __name__ == "__main__":
    sys.exit(main())
