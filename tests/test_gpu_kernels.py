"""SpMM / SDDMM kernels on worksets built by the CPU oracle and uploaded, so
the kernels are checked independently of the GPU preprocessing. Outputs are
compared with the oracle's double-precision CheckSpmm / CheckSddmm
(tests/tolerance.py states the bound)."""
import numpy as np
import pytest

import oracle
import powersparse_amd as ps
import tolerance
from gpu_util import Uploaded, random_graph, say, setup, star_graph
from powersparse_amd import _native

pytestmark = pytest.mark.gpu

GRAPHS = {
    # name: (builder, cu_count) -- cu_count picks how many worksets appear
    "c0_fine": (lambda: ps.synth("C0", seed=1), 256),
    "c1_small": (lambda: ps.synth("C1", seed=2, scale=200), 1),
    "c3_small": (lambda: ps.synth("C3", seed=3, scale=400), 1),
    "c4_small": (lambda: ps.synth("C4", seed=4, scale=128), 2),
    "hubs": (lambda: random_graph(np.random.default_rng(5), 300, 5000, 40, hubs=6,
                                  hub_deg=4500), 1),
    "dups": (lambda: random_graph(np.random.default_rng(6), 200, 50, 90, dup=True), 1),
    "star": (lambda: star_graph(np.random.default_rng(7), 20000, 9000, 8, long_rows=40,
                                long_deg=700), 4),
}
_cache = {}


def graph(name):
    if name not in _cache:
        build, cu = GRAPHS[name]
        csr = build()
        w = oracle.preprocess(csr.rows, csr.cols, csr.row_ptr, csr.col_ind, csr.values, cu)
        _cache[name] = (csr, w)
    return _cache[name]


def row_factor(csr, w):
    """1 for rows written by a single non-atomic residue group, 2 otherwise:
    the factor two back-to-back calls without clearing C leave on each row."""
    f = np.full(csr.rows, 2.0)
    for g, r in enumerate(w.des[0]):
        if not w.residue_atomic[g]:
            f[r] = 1.0
    return f


@pytest.mark.parametrize("name", sorted(GRAPHS))
@pytest.mark.parametrize("N", [32, 64, 128, 96, 256, 288, 1024])
def test_spmm_kernel(name, N):
    setup()
    csr, w = graph(name)
    say(f"spmm kernel {name} S={w.S} groups={w.group_num} N={N}")
    up = Uploaded(w)
    rng = np.random.default_rng(N)
    B = rng.uniform(-1, 1, (csr.cols, N)).astype(np.float32)
    dB = ps.DeviceBuffer(host=B)
    dC = ps.DeviceBuffer.zeros(csr.rows * N * 4)
    ps.spmm_launch(up.worksets, up.offset, up.atomic, csr.rows, csr.cols, N, dB, dC)
    ps.synchronize()
    C = dC.download(np.float32).reshape(csr.rows, N)
    E, M = oracle.spmm(csr.row_ptr, csr.col_ind, csr.values, N, B, with_mag=True)
    stats = tolerance.check(C, E, M, f"spmm {name} N={N}")
    say("  ", stats)
    # second call without clearing: atomic rows accumulate, stored rows are rewritten
    ps.spmm_launch(up.worksets, up.offset, up.atomic, csr.rows, csr.cols, N, dB, dC)
    ps.synchronize()
    C2 = dC.download(np.float32).reshape(csr.rows, N)
    f = row_factor(csr, w)[:, None]
    tolerance.check(C2, E * f, M * f, f"spmm {name} N={N} second call")


@pytest.mark.parametrize("name", sorted(GRAPHS))
@pytest.mark.parametrize("N", [32, 64, 128, 96, 256, 512])
def test_sddmm_kernel(name, N):
    setup()
    csr, w = graph(name)
    say(f"sddmm kernel {name} S={w.S} groups={w.group_num} N={N}")
    up = Uploaded(w)
    rng = np.random.default_rng(1000 + N)
    X = rng.normal(size=(csr.rows, N)).astype(np.float32)
    Y = rng.normal(size=(csr.cols, N)).astype(np.float32)
    dX, dY = ps.DeviceBuffer(host=X), ps.DeviceBuffer(host=Y)
    outs = [ps.DeviceBuffer.zeros(max(w.col[s].size, 1) * 4) for s in range(w.S)]
    ps.sddmm_launch(up.worksets, up.offset, csr.rows, csr.cols, N, dX, dY, outs)
    ps.synchronize()
    got = []
    for s in range(w.S):
        E, M = oracle.sddmm(w.des[s], w.offsets(s), w.col[s], w.val[s], N, X, Y, with_mag=True)
        G = outs[s].download(np.float32, w.col[s].size)
        got.append(G)
        tolerance.check(G, E, M, f"sddmm {name} N={N} workset {s}")
    # second call: block outputs are stored again, residue outputs accumulate
    ps.sddmm_launch(up.worksets, up.offset, csr.rows, csr.cols, N, dX, dY, outs)
    ps.synchronize()
    for s in range(w.S):
        G2 = outs[s].download(np.float32, w.col[s].size)
        if s == 0:
            np.testing.assert_allclose(G2, 2 * got[0], rtol=1e-6, atol=1e-6)
        else:
            np.testing.assert_array_equal(G2, got[s])


def test_launch_argument_checks():
    setup()
    csr, w = graph("c1_small")
    up = Uploaded(w)
    dB = ps.DeviceBuffer(csr.cols * 48 * 4)
    dC = ps.DeviceBuffer(csr.rows * 48 * 4)
    with pytest.raises(ValueError, match="multiple of 32"):
        ps.spmm_launch(up.worksets, up.offset, up.atomic, csr.rows, csr.cols, 48, dB, dC)
    with pytest.raises(ValueError, match="between 32 and 512"):
        ps.sddmm_launch(up.worksets, up.offset, csr.rows, csr.cols, 544, dB, dB,
                        [dC] * w.S)
    with pytest.raises(ValueError, match="Missing SDDMM output"):
        ps.sddmm_launch(up.worksets, up.offset, csr.rows, csr.cols, 32, dB, dB,
                        [None] * w.S)


def run_order(offsets, kind, seed):
    """A residue run order: 'length' (longest first, ties in stored order) or a
    random permutation."""
    lens = np.diff(np.asarray(offsets, dtype=np.int64))
    if kind == "length":
        return np.argsort(-np.minimum(lens, 255), kind="stable").astype(np.int32)
    return np.random.default_rng(seed).permutation(lens.size).astype(np.int32)


@pytest.mark.parametrize("kind", ["length", "random"])
@pytest.mark.parametrize("name", sorted(GRAPHS))
def test_residue_run_order(name, kind):
    """The operators given a run order for the residue groups (ps_workset.order):
    SpMM within tolerance of the oracle, SDDMM bitwise equal to the call without
    an order (each output is one lane's dot, whichever slot runs the group)."""
    setup()
    csr, w = graph(name)
    if w.group_num[0] == 0:
        pytest.skip("no residue groups")
    say(f"residue run order {kind} {name} S={w.S} groups={w.group_num}")
    up = Uploaded(w)
    d_order = ps.DeviceBuffer(host=run_order(w.residue_offset, kind, 3))
    ordered = [up.worksets[0] + (d_order,)] + list(up.worksets[1:])
    rng = np.random.default_rng(17)
    for N in (32, 64, 128):
        B = rng.uniform(-1, 1, (csr.cols, N)).astype(np.float32)
        dB = ps.DeviceBuffer(host=B)
        dC = ps.DeviceBuffer.zeros(csr.rows * N * 4)
        ps.spmm_launch(ordered, up.offset, up.atomic, csr.rows, csr.cols, N, dB, dC)
        ps.synchronize()
        E, M = oracle.spmm(csr.row_ptr, csr.col_ind, csr.values, N, B, with_mag=True)
        tolerance.check(dC.download(np.float32).reshape(csr.rows, N), E, M,
                        f"spmm {name} N={N} order {kind}")
        X = rng.normal(size=(csr.rows, N)).astype(np.float32)
        Y = rng.normal(size=(csr.cols, N)).astype(np.float32)
        dX, dY = ps.DeviceBuffer(host=X), ps.DeviceBuffer(host=Y)
        plain = [ps.DeviceBuffer.zeros(max(w.col[s].size, 1) * 4) for s in range(w.S)]
        runs = [ps.DeviceBuffer.zeros(max(w.col[s].size, 1) * 4) for s in range(w.S)]
        ps.sddmm_launch(up.worksets, up.offset, csr.rows, csr.cols, N, dX, dY, plain)
        ps.sddmm_launch(ordered, up.offset, csr.rows, csr.cols, N, dX, dY, runs)
        ps.synchronize()
        for s in range(w.S):
            np.testing.assert_array_equal(runs[s].download(np.float32, w.col[s].size),
                                          plain[s].download(np.float32, w.col[s].size))
        E, M = oracle.sddmm(w.des[0], w.offsets(0), w.col[0], w.val[0], N, X, Y, with_mag=True)
        tolerance.check(runs[0].download(np.float32, w.col[0].size), E, M,
                        f"sddmm {name} N={N} order {kind} residue")


@pytest.mark.parametrize("kind", [None, "length", "random"])
def test_long_residue_groups(kind):
    """Residue groups longer than the kernels stage in LDS (up to 150 nonzeros)
    and empty ones, which the preprocessing never builds but the C ABI accepts:
    one group per row, each row's whole CSR row, so SpMM stores every row."""
    setup()
    rng = np.random.default_rng(21)
    rows, cols = 700, 3000
    lens = rng.integers(0, 151, rows)
    lens[::7] = rng.integers(0, 33, lens[::7].size)  # short ones mixed in
    lens[::50] = 0
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    nnz = int(offsets[-1])
    col = rng.integers(0, cols, nnz).astype(np.int32)
    val = rng.uniform(-1, 1, nnz).astype(np.float32)
    rows_of = np.repeat(np.arange(rows), lens)
    bufs = [ps.DeviceBuffer(host=col), ps.DeviceBuffer(host=val),
            ps.DeviceBuffer(host=np.arange(rows, dtype=np.int32))]
    order = None if kind is None else ps.DeviceBuffer(host=run_order(offsets, kind, 5))
    ws = [(bufs[0], bufs[1], bufs[2], rows, 0, order)]
    d_off = ps.DeviceBuffer(host=offsets)
    d_atomic = ps.DeviceBuffer.zeros(rows)
    say(f"long residue groups order={kind} rows={rows} nnz={nnz} max={lens.max()}")
    # the SDDMM kernel's paired dots (K up to 256) and its unpaired form (K = 320)
    for N in (32, 64, 96, 128, 320):
        B = rng.uniform(-1, 1, (cols, N)).astype(np.float32)
        dB = ps.DeviceBuffer(host=B)
        dC = ps.DeviceBuffer.zeros(rows * N * 4)
        ps.spmm_launch(ws, d_off, d_atomic, rows, cols, N, dB, dC)
        ps.synchronize()
        terms = val[:, None].astype(np.float64) * B[col].astype(np.float64)
        E = np.zeros((rows, N))
        M = np.zeros((rows, N))
        np.add.at(E, rows_of, terms)
        np.add.at(M, rows_of, np.abs(terms))
        tolerance.check(dC.download(np.float32).reshape(rows, N), E, M,
                        f"spmm long groups N={N} order={kind}")
        X = rng.normal(size=(rows, N)).astype(np.float32)
        Y = rng.normal(size=(cols, N)).astype(np.float32)
        dX, dY = ps.DeviceBuffer(host=X), ps.DeviceBuffer(host=Y)
        out = ps.DeviceBuffer.zeros(nnz * 4)
        ps.sddmm_launch(ws, d_off, rows, cols, N, dX, dY, [out])
        ps.synchronize()
        prod = X[rows_of].astype(np.float64) * Y[col].astype(np.float64)
        E = val * prod.sum(1)
        M = np.abs(val) * np.abs(prod).sum(1)
        tolerance.check(out.download(np.float32, nnz), E, M,
                        f"sddmm long groups N={N} order={kind}")


def test_residue_order_out_of_range_entries_skipped():
    """Run-order entries outside [0, group_num) are skipped: their slots
    compute nothing and every other group is computed as without an order."""
    setup()
    csr, w = graph("c1_small")
    up = Uploaded(w)
    G = w.group_num[0]
    order = np.arange(G, dtype=np.int32)
    dropped = np.array([0, 5, G // 2, G - 1])
    order[dropped] = np.array([-1, G, G + 1000, -(1 << 30)], dtype=np.int32)
    d_order = ps.DeviceBuffer(host=order)
    ordered = [up.worksets[0] + (d_order,)] + list(up.worksets[1:])
    N = 32
    rng = np.random.default_rng(29)
    X = rng.normal(size=(csr.rows, N)).astype(np.float32)
    Y = rng.normal(size=(csr.cols, N)).astype(np.float32)
    dX, dY = ps.DeviceBuffer(host=X), ps.DeviceBuffer(host=Y)
    n0 = w.col[0].size
    plain, runs = ps.DeviceBuffer.zeros(n0 * 4), ps.DeviceBuffer.zeros(n0 * 4)
    ps.sddmm_launch(up.worksets[:1], up.offset, csr.rows, csr.cols, N, dX, dY, [plain])
    ps.sddmm_launch(ordered[:1], up.offset, csr.rows, csr.cols, N, dX, dY, [runs])
    ps.synchronize()
    expect = plain.download(np.float32, n0)
    off = w.residue_offset
    for g in dropped:
        expect[off[g]:off[g + 1]] = 0.0
    np.testing.assert_array_equal(runs.download(np.float32, n0), expect)


@pytest.mark.parametrize("name", ["c1_small", "c4_small", "hubs"])
def test_task_chunk_mapping(name):
    """The workgroup -> XCD run length (task_chunk) changes only which XCD runs
    a task: SDDMM bitwise equal for every chunk, SpMM within tolerance (atomic
    addition order), invalid chunks rejected before any launch."""
    setup()
    csr, w = graph(name)
    up = Uploaded(w)
    rng = np.random.default_rng(31)
    N = 32
    B = rng.uniform(-1, 1, (csr.cols, N)).astype(np.float32)
    X = rng.normal(size=(csr.rows, N)).astype(np.float32)
    Y = rng.normal(size=(csr.cols, N)).astype(np.float32)
    dB, dX, dY = ps.DeviceBuffer(host=B), ps.DeviceBuffer(host=X), ps.DeviceBuffer(host=Y)
    E, M = oracle.spmm(csr.row_ptr, csr.col_ind, csr.values, N, B, with_mag=True)
    ref = None
    for chunk in (0, 1, 2, 16, 64, 256, 4096, _native.PS_TASK_CHUNK_AUTO):
        dC = ps.DeviceBuffer.zeros(csr.rows * N * 4)
        ps.spmm_launch(up.worksets, up.offset, up.atomic, csr.rows, csr.cols, N, dB, dC,
                       task_chunk=chunk)
        outs = [ps.DeviceBuffer.zeros(max(w.col[s].size, 1) * 4) for s in range(w.S)]
        ps.sddmm_launch(up.worksets, up.offset, csr.rows, csr.cols, N, dX, dY, outs,
                        task_chunk=chunk)
        ps.synchronize()
        tolerance.check(dC.download(np.float32).reshape(csr.rows, N), E, M,
                        f"spmm {name} task_chunk={chunk}")
        got = [outs[s].download(np.float32, w.col[s].size) for s in range(w.S)]
        if ref is None:
            ref = got
        for s in range(w.S):
            np.testing.assert_array_equal(got[s], ref[s], err_msg=f"chunk {chunk} workset {s}")
    dC = ps.DeviceBuffer.zeros(csr.rows * N * 4)
    for bad in (3, 8192, -2):
        with pytest.raises(ValueError, match="task_chunk"):
            ps.spmm_launch(up.worksets, up.offset, up.atomic, csr.rows, csr.cols, N, dB, dC,
                           task_chunk=bad)
        with pytest.raises(ValueError, match="task_chunk"):
            ps.sddmm_launch(up.worksets, up.offset, csr.rows, csr.cols, N, dX, dY,
                            [dC] * w.S, task_chunk=bad)
