"""Locality run order (ps_task_order_build and the *_launch_ordered launchers):
the order is a permutation of the launch's tasks with block tiles sorted
stably by their first column and the residue tasks last as stored; the
operators give the same results in it as in the stored order (SDDMM bitwise,
SpMM within the FP32 tolerance) and against the oracle; any permutation gives
those results; a task count that does not match the launch is rejected; the
subset order leaves out the tasks of marked stretches and SDDMM on its prefix
writes exactly the other tasks' outputs."""
import ctypes

import numpy as np
import pytest

import oracle
import powersparse_amd as ps
import tolerance
from gpu_util import random_graph, say, setup
from powersparse_amd import _native

pytestmark = pytest.mark.gpu

SHAPES = {("spmm", 32): (256, 8), ("spmm", 64): (128, 4), ("spmm", 128): (128, 4),
          ("sddmm", 32): (64, 8), ("sddmm", 64): (64, 8), ("sddmm", 128): (64, 8)}


def worksets(m):
    S = m.GroupTypeNum()
    arr = (_native.Workset * S)()
    cps, vps, dps = m.WorksetColInd(), m.WorksetSpData(), m.GroupDestination()
    for s in range(S):
        arr[s] = _native.Workset(cps[s], vps[s], dps[s], m.GroupNum()[s],
                                 0 if s == 0 else 32 << (s - 1), None)
    return arr


def op_code(op):
    return _native.PS_OP_SPMM if op == "spmm" else _native.PS_OP_SDDMM


def build_order(m, op, N):
    arr = worksets(m)
    count = ctypes.c_uint32()
    ps._hip_call(_native.hip().ps_task_count(op_code(op), N, m.GroupTypeNum(), arr,
                                             ctypes.byref(count)))
    n = count.value
    buf = ps.DeviceBuffer(max(n, 1) * 4)
    ps._hip_call(_native.hip().ps_task_order_build(op_code(op), N, m.GroupTypeNum(), arr,
                                                   buf.ptr, n, None))
    return buf, n


def launch_tasks(m, op, N):
    """(workset, local task, first column or None for residue) per task, in
    launch order, from the downloaded worksets (an independent enumeration)."""
    tile, rgroups = SHAPES[(op, N)]
    tasks = []
    for s in range(m.GroupTypeNum() - 1, -1, -1):
        G = m.GroupNum()[s]
        if G == 0:
            continue
        col = m.download_workset(s)[0]
        if s > 0:
            for t in range(-(-col.size // tile)):
                tasks.append((s, t, int(col[t * tile])))
        else:
            for t in range(-(-G // rgroups)):
                tasks.append((s, t, None))
    return tasks


GRAPHS = {
    "c1": (lambda: ps.synth("C1", seed=41, scale=100), 8),
    "c3": (lambda: ps.synth("C3", seed=42, scale=200), 4),
    "c0_fine": (lambda: ps.synth("C0", seed=43), 256),
    "hubs": (lambda: random_graph(np.random.default_rng(44), 700, 900, 60, hubs=9,
                                  hub_deg=700), 2),
}


@pytest.mark.parametrize("name", sorted(GRAPHS))
@pytest.mark.parametrize("op,N", [("spmm", 32), ("spmm", 64), ("sddmm", 32)])
def test_order_is_the_stable_first_column_sort(name, op, N):
    setup()
    make, cu = GRAPHS[name]
    csr = make()
    m = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=cu, task_order="signature")
    say(f"run order {name} {op} N={N} S={m.GroupTypeNum()} groups={m.GroupNum()}")
    buf, n = build_order(m, op, N)
    tasks = launch_tasks(m, op, N)
    assert n == len(tasks)
    order = buf.download(np.uint32, n).astype(np.int64)
    assert np.array_equal(np.sort(order), np.arange(n))  # a permutation
    keys = [tasks[t][2] for t in order]
    blocks = [k for k in keys if k is not None]
    nb = len(blocks)
    assert all(k is None for k in keys[nb:])  # residue tasks last ...
    assert list(order[nb:]) == sorted(order[nb:])  # ... as stored
    assert blocks == sorted(blocks)  # tiles by first column
    for a, b in zip(order[:nb - 1], order[1:nb]):  # stable: ties keep launch order
        if tasks[a][2] == tasks[b][2]:
            assert a < b


@pytest.mark.parametrize("name", sorted(GRAPHS))
def test_operators_in_run_order_match_stored_order(name):
    setup()
    make, cu = GRAPHS[name]
    csr = make()
    # SpMM on the public worksets, so that it runs their run order too
    a = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=cu, task_order="signature",
                                         csr_positions=True, spmm_partition="parity")
    b = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=cu, task_order="signature",
                                         csr_positions=True, run_order=False,
                                         spmm_partition="parity")
    assert a.run_order and not b.run_order
    rng = np.random.default_rng(7)
    rows = np.arange(csr.rows, dtype=np.int32)
    # 32- and 64-float SpMM slices (N = 96: three 32-float slices; 256: four 64-float)
    for N in (32, 64, 96, 128, 256):
        say(f"run order vs stored {name} N={N}")
        B = rng.uniform(-1, 1, (csr.cols, N)).astype(np.float32)
        dB = ps.DeviceBuffer(host=B)
        E, M = oracle.spmm(csr.row_ptr, csr.col_ind, csr.values, N, B, with_mag=True)
        for m in (a, b):
            C = ps.DeviceBuffer.zeros(csr.rows * N * 4)
            ps.SpMMAsync(m, N, dB, C)
            ps.synchronize()
            tolerance.check(C.download(np.float32).reshape(csr.rows, N), E, M,
                            f"SpMM run_order={m.run_order}")
        X = rng.normal(size=(csr.rows, N)).astype(np.float32)
        Y = rng.normal(size=(csr.cols, N)).astype(np.float32)
        dX, dY = ps.DeviceBuffer(host=X), ps.DeviceBuffer(host=Y)
        res = []
        for m in (a, b):
            outs = [ps.DeviceBuffer.zeros(max(k, 1) * 4) for k in m.sddmm_output_sizes()]
            for _ in range(2):  # accumulating calls, as the reference harness
                ps.SDDMMAsync(m, N, dX, dY, outs)
            csr_out = ps.DeviceBuffer(max(csr.nnz, 1) * 4)
            ps.SDDMMToCSR(m, N, dX, dY, csr_out)
            ps.synchronize()
            res.append([o.download(np.float32, k) for o, k in zip(outs, m.sddmm_output_sizes())]
                       + [csr_out.download(np.float32, csr.nnz)])
        for x, y in zip(*res):
            np.testing.assert_array_equal(x.view(np.uint32), y.view(np.uint32))
        E, M = oracle.sddmm(rows, csr.row_ptr, csr.col_ind, csr.values, N, X, Y, with_mag=True)
        tolerance.check(res[0][-1], E, M, f"SDDMMToCSR in run order N={N}")


def test_any_permutation_gives_the_same_results():
    setup()
    csr = ps.synth("C1", seed=45, scale=100)
    m = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=8, task_order="signature",
                                         run_order=False)
    S, arr = m.GroupTypeNum(), worksets(m)
    rng = np.random.default_rng(9)
    N = 64
    X = rng.normal(size=(csr.rows, N)).astype(np.float32)
    Y = rng.normal(size=(csr.cols, N)).astype(np.float32)
    dX, dY = ps.DeviceBuffer(host=X), ps.DeviceBuffer(host=Y)
    sizes = m.sddmm_output_sizes()

    def sddmm(order, chunk=1):
        outs = [ps.DeviceBuffer.zeros(max(k, 1) * 4) for k in sizes]
        oa = (ctypes.c_void_p * S)(*[o.ptr for o in outs])
        if order is None:
            ps._hip_call(_native.hip().ps_sddmm_launch(S, arr, m.ResidueOffset(), csr.rows,
                                                       csr.cols, N, dX.ptr, dY.ptr, oa, 1, None))
        else:
            d = ps.DeviceBuffer(host=order)
            ps._hip_call(_native.hip().ps_sddmm_launch_ordered(
                S, arr, m.ResidueOffset(), csr.rows, csr.cols, N, dX.ptr, dY.ptr, oa, chunk,
                d.ptr, order.size, None))
        ps.synchronize()
        return [o.download(np.float32, k) for o, k in zip(outs, sizes)]

    count = ctypes.c_uint32()
    ps._hip_call(_native.hip().ps_task_count(_native.PS_OP_SDDMM, N, S, arr,
                                             ctypes.byref(count)))
    base = sddmm(None)
    for trial, chunk in enumerate((1, _native.PS_TASK_CHUNK_AUTO, 4)):
        perm = rng.permutation(count.value).astype(np.uint32)
        say(f"random task permutation {trial}: {perm.size} tasks, task_chunk {chunk}")
        for x, y in zip(base, sddmm(perm, chunk)):
            np.testing.assert_array_equal(x.view(np.uint32), y.view(np.uint32))
    # SpMM with a random permutation against the oracle
    B = rng.uniform(-1, 1, (csr.cols, 32)).astype(np.float32)
    dB = ps.DeviceBuffer(host=B)
    ps._hip_call(_native.hip().ps_task_count(_native.PS_OP_SPMM, 32, S, arr,
                                             ctypes.byref(count)))
    perm = ps.DeviceBuffer(host=rng.permutation(count.value).astype(np.uint32))
    C = ps.DeviceBuffer.zeros(csr.rows * 32 * 4)
    ps._hip_call(_native.hip().ps_spmm_launch_ordered(
        S, arr, m.ResidueOffset(), m.ResidueAtomic(), csr.rows, csr.cols, 32, dB.ptr, C.ptr,
        _native.PS_TASK_CHUNK_AUTO, perm.ptr, count.value, None))
    ps.synchronize()
    E, M = oracle.spmm(csr.row_ptr, csr.col_ind, csr.values, 32, B, with_mag=True)
    tolerance.check(C.download(np.float32).reshape(csr.rows, 32), E, M, "SpMM permuted")
    # a task count that does not match the launch is rejected before any work
    rc = _native.hip().ps_spmm_launch_ordered(
        S, arr, m.ResidueOffset(), m.ResidueAtomic(), csr.rows, csr.cols, 32, dB.ptr, C.ptr,
        1, perm.ptr, count.value - 1, None)
    assert rc == _native.PS_ERR_INVALID and b"task order" in _native.hip().ps_last_error()
    # and so is a task_chunk the launchers do not take
    rc = _native.hip().ps_spmm_launch_ordered(
        S, arr, m.ResidueOffset(), m.ResidueAtomic(), csr.rows, csr.cols, 32, dB.ptr, C.ptr,
        -2, perm.ptr, count.value, None)
    assert rc == _native.PS_ERR_INVALID and b"task_chunk" in _native.hip().ps_last_error()


@pytest.mark.parametrize("op,N", [("sddmm", 64), ("spmm", 32)])
def test_subset_order_leaves_out_marked_stretches(op, N):
    """ps_task_order_build_subset: with random 64-nonzero stretches marked, the
    tasks whose stretches are all marked go last and the rest keep the full
    order's sequence; *kept counts them. SDDMM run on that prefix writes
    exactly the unmarked tasks' outputs, bitwise those of the full launch."""
    setup()
    csr = ps.synth("C1", seed=46, scale=100)
    m = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=8, task_order="signature",
                                         run_order=False)
    S, arr = m.GroupTypeNum(), worksets(m)
    tile, _ = SHAPES[(op, N)]
    rng = np.random.default_rng(11)
    marks, dev = [None] * S, [None] * S
    for s in range(1, S):
        nnz = m.GroupNum()[s] * (32 << (s - 1))
        if nnz == 0:
            continue
        f = (rng.random(-(-nnz // 64)) < 0.6).astype(np.uint8)
        f[: max(1, f.size // 8)] = 1  # a run of marked stretches: whole tiles at any tile size
        marks[s], dev[s] = f, ps.DeviceBuffer(host=f)
    skip = (ctypes.c_void_p * S)(*[d.ptr if d is not None else None for d in dev])
    full, n = build_order(m, op, N)
    sub = ps.DeviceBuffer(max(n, 1) * 4)
    kept = ctypes.c_uint32()
    ps._hip_call(_native.hip().ps_task_order_build_subset(op_code(op), N, S, arr, skip, sub.ptr, n,
                                                          ctypes.byref(kept), None))
    tasks = launch_tasks(m, op, N)
    begin = {}
    for i, (s, t, _) in enumerate(tasks):
        begin.setdefault(s, i)

    def left_out(task):
        s, t, _ = tasks[task]
        if s == 0 or marks[s] is None:
            return False
        first, end = t * tile, min((t + 1) * tile, marks[s].size * 64)
        return bool(marks[s][first // 64:(end - 1) // 64 + 1].all())

    full_order = full.download(np.uint32, n).tolist()
    order = sub.download(np.uint32, n).tolist()
    want_kept = [t for t in full_order if not left_out(t)]
    say(f"subset {op} N={N}: {n} tasks, {kept.value} kept")
    assert 0 < kept.value < n and kept.value == len(want_kept)
    assert order[:kept.value] == want_kept
    assert sorted(order[kept.value:]) == sorted(t for t in range(n) if left_out(t))
    if op != "sddmm":
        return
    X = rng.normal(size=(csr.rows, N)).astype(np.float32)
    Y = rng.normal(size=(csr.cols, N)).astype(np.float32)
    dX, dY = ps.DeviceBuffer(host=X), ps.DeviceBuffer(host=Y)
    sizes = m.sddmm_output_sizes()
    sentinel = np.float32(-3.5)

    def run(order_buf, count):
        outs = [ps.DeviceBuffer(host=np.full(max(k, 1), sentinel, np.float32)) for k in sizes]
        oa = (ctypes.c_void_p * S)(*[o.ptr for o in outs])
        ps._hip_call(_native.hip().ps_sddmm_launch_ordered(
            S, arr, m.ResidueOffset(), csr.rows, csr.cols, N, dX.ptr, dY.ptr, oa,
            _native.PS_TASK_CHUNK_AUTO, order_buf.ptr, count, None))
        ps.synchronize()
        return [o.download(np.float32, k) for o, k in zip(outs, sizes)]

    whole, part = run(full, n), run(sub, kept.value)
    for s in range(S):
        if sizes[s] == 0:
            continue
        written = np.ones(sizes[s], bool)
        if s > 0 and marks[s] is not None:
            for i, (q, t, _) in enumerate(tasks):
                if q == s and left_out(i):
                    written[t * tile:(t + 1) * tile] = False
        np.testing.assert_array_equal(part[s][written].view(np.uint32),
                                      whole[s][written].view(np.uint32), err_msg=f"ws {s}")
        assert (part[s][~written] == sentinel).all(), f"ws {s}: a left-out task wrote"
