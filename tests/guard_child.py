"""Child process of tests/test_gpu_guard.py: runs the operator flows with the
device allocation guards on (PS_DEVICE_GUARD set by the parent) and prints
the guard count as `guard violations: N`.

Flows: the benchmark harness's (preprocessing, the check path's workset
download, 30 + 3 operator calls into the same outputs, SpMM and SDDMM) on
the matrices its tests use (a 6 x 5 MatrixMarket file with an empty row, an
80 x 300 pattern matrix, synth C0 seed 5, synth C4 at scale 2); the golden
fixtures through SpMM, SDDMM and SDDMMToCSR at N = 32 .. 256 with and without
a hub block; and a scaled power-law graph with its automatic hub block."""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import golden_data as gd  # noqa: E402
import powersparse_amd as ps  # noqa: E402
from powersparse_amd import _native  # noqa: E402

SMALL_MTX = """%%MatrixMarket matrix coordinate real general
6 5 9
1 1 0.5
1 3 -1.25
2 2 2.0
3 1 1.0
3 5 3.5
5 4 -0.75
6 1 1.5
6 2 0.25
6 5 -2.0
"""


def say(*a):
    print(*a, flush=True)


def harness_flow(name, csr, n, op, calls=33):
    """What the benchmark binaries do with one matrix and width."""
    m = ps.PowerSparseMatrixGPU.from_csr(csr)
    S = m.GroupTypeNum()
    for s in range(S):
        m.download_workset(s)
    m.residue_offset()
    streams = [ps.Stream()] * S if S > 1 else None
    if op == "spmm":
        B = ps.DeviceBuffer(host=ps.dense_input(1, csr.cols * n))
        C = ps.DeviceBuffer.zeros(csr.rows * n * 4)
        for _ in range(calls):
            ps.SpMM(m, n, B, C, S, streams)
        ps.synchronize()
        C.download(np.float32)
    else:
        X, Y = ps.dense_input(1, csr.rows * n, csr.cols * n)
        dX, dY = ps.DeviceBuffer(host=X), ps.DeviceBuffer(host=Y)
        outs = [ps.DeviceBuffer.zeros(max(sz, 1) * 4) for sz in m.sddmm_output_sizes()]
        for _ in range(calls):
            ps.SDDMM(m, n, dX, dY, outs, S, streams)
        ps.synchronize()
        for o in outs:
            o.download(np.float32)
    say(f"{name} {op} N={n}: S={S} groups={m.GroupNum()} hub={m.hub_block}")
    m.close()


def fixture_flow(name, hub):
    g = gd.load(name)
    csr = ps.HostCsr(g.rows, g.cols, g.row_ptr, g.col_ind, g.values)
    kw = dict(cu_count=g.parts[0].cu, csr_positions=True)
    if hub:
        deg = np.diff(g.row_ptr.astype(np.int64))
        cnt = np.bincount(g.col_ind, minlength=g.cols)
        d = int(np.quantile(deg[deg > 0], 0.8))
        c = max(int(np.quantile(cnt[cnt > 0], 0.6)), 1)
        kw["hub_thresholds"] = [(max(d, 1), c)]
    try:
        m = ps.PowerSparseMatrixGPU.from_csr(csr, **kw)
    except ValueError:
        return  # thresholds the build refuses
    S = m.GroupTypeNum()
    streams = [ps.Stream() for _ in range(S)] if S > 1 else None
    for n in (32, 64, 128, 256):
        B = ps.DeviceBuffer(host=gd.dense(g.cols, n, gd.SALT_B))
        C = ps.DeviceBuffer.zeros(g.rows * n * 4)
        ps.SpMM(m, n, B, C, S, streams)
        X = ps.DeviceBuffer(host=gd.dense(g.rows, n, gd.SALT_X))
        Y = ps.DeviceBuffer(host=gd.dense(g.cols, n, gd.SALT_Y))
        outs = [ps.DeviceBuffer.zeros(max(sz, 1) * 4) for sz in m.sddmm_output_sizes()]
        ps.SDDMM(m, n, X, Y, outs, S, streams)
        csr_out = ps.DeviceBuffer(max(g.nnz, 1) * 4)
        ps.SDDMMToCSR(m, n, X, Y, csr_out)
        ps.synchronize()
    say(f"fixture {name} hub={m.hub_block}: S={S}")
    m.close()


def main():
    ps.set_device(0)
    lib = _native.hip()
    assert lib.ps_guard_violations() == 0, "guards are off or already tripped"
    tmp = os.environ.get("TMPDIR", "/tmp")
    path = os.path.join(tmp, f"guard_small_{os.getpid()}.mtx")
    with open(path, "w") as fh:
        fh.write(SMALL_MTX)
    small = ps.read_mtx(path)
    os.remove(path)
    r = np.arange(80).repeat(40)
    k = np.tile(np.arange(40), 80)
    cols = ((r * 7 + k * 3) % 300).astype(np.int32)
    rows40 = ps.HostCsr(80, 300, (np.arange(81) * 40).astype(np.int32), cols,
                        np.ones(3200, np.float32))
    cases = [("small.mtx", small, 32, "sddmm"), ("small.mtx", small, 64, "sddmm"),
             ("small.mtx", small, 32, "spmm"), ("rows40", rows40, 32, "sddmm"),
             ("rows40", rows40, 64, "sddmm")]
    c0 = ps.synth("C0", seed=5)
    cases += [("synth:C0:5", c0, n, "spmm") for n in (32, 64, 128)]
    cases += [("synth:C0:5", c0, 128, "sddmm")]
    c4 = ps.synth("C4", seed=2, scale=64)
    cases += [("synth:C4:2:64", c4, n, op) for n in (32, 64) for op in ("spmm", "sddmm")]
    for name, csr, n, op in cases:
        harness_flow(name, csr, n, op)
    for name in ("hand_3x4", "hand_44x70", "empty_middle", "skewed", "star_ties", "hubs",
                 "duplicates"):
        for hub in (False, True):
            fixture_flow(name, hub)
    big = ps.synth("C1", seed=1, scale=100)
    harness_flow("synth:C1:1:100", big, 128, "spmm", calls=3)
    harness_flow("synth:C1:1:100", big, 128, "sddmm", calls=3)
    import gc
    gc.collect()
    say(f"guard violations: {lib.ps_guard_violations()}")


if __name__ == "__main__":
    main()
