"""The product against the golden fixtures (tests/golden/*.npz) on the GPU.

The GPU preprocessing must give the stored worksets bit for bit at each
stored (CU count, workset cap), and every execution path (tuned or parity
SpMM partition, signature or row task order, run order on or off, the raw
launchers on the stored worksets, SDDMM in workset or CSR order) must give
the stored results exactly: the fixtures' values are dyadic rationals for
which every FP32 partial sum is exact, so the results cannot depend on the
order of the additions. N = 64 to 512 are checked against the float64
products of the same inputs (exact as well: below 2^24 at 2^-14 resolution)."""
import numpy as np
import pytest

import golden_data as gd
import powersparse_amd as ps
from gpu_util import say, setup
from powersparse_amd import _native

pytestmark = pytest.mark.gpu

NAMES = gd.names()

# (spmm_partition, task_order, run_order)
PATHS = [("tuned", "auto", True), ("parity", "auto", True), ("tuned", "row", True),
         ("parity", "signature", False)]


def csr_of(g):
    return ps.HostCsr(g.rows, g.cols, g.row_ptr, g.col_ind, g.values)


def stored_rows(p):
    """Rows whose SpMM output the reference stores (one residue group marked
    non-atomic); every other row accumulates over repeated calls."""
    des0 = p.des[0]
    return des0[p.residue_atomic == 0] if des0.size else des0


def expected_spmm(g, N):
    if N == g.n:
        return g.spmm_c.astype(np.float64)
    row_of = np.repeat(np.arange(g.rows), np.diff(g.row_ptr))
    C = np.zeros((g.rows, N))
    B = gd.dense(g.cols, N, gd.SALT_B).astype(np.float64)
    np.add.at(C, row_of, g.values.astype(np.float64)[:, None] * B[g.col_ind])
    return C


def dense_inputs(g, N):
    return (gd.dense(g.cols, N, gd.SALT_B), gd.dense(g.rows, N, gd.SALT_X),
            gd.dense(g.cols, N, gd.SALT_Y))


@pytest.mark.parametrize("name", NAMES)
def test_preprocessing_matches_golden(name):
    setup()
    g = gd.load(name)
    for p in g.parts:
        say(f"golden {name} cu={p.cu} cap={p.cap} S={p.S}")
        m = ps.PowerSparseMatrixGPU.from_csr(csr_of(g), cu_count=p.cu, max_group_types=p.cap)
        assert (m.GroupTypeNum(), m.GroupNum(), m.SignatureLen()) == (p.S, p.group_num, g.L)
        np.testing.assert_array_equal(m.residue_offset(), p.residue_offset)
        np.testing.assert_array_equal(m.residue_atomic(), p.residue_atomic)
        for s in range(p.S):
            if p.group_num[s] == 0:
                continue
            col, val, des = m.download_workset(s)
            np.testing.assert_array_equal(des, p.des[s], err_msg=f"group_des[{s}]")
            np.testing.assert_array_equal(col, p.col[s], err_msg=f"col_ind[{s}]")
            np.testing.assert_array_equal(val.view(np.uint32), p.val[s].view(np.uint32))
        m.close()


@pytest.mark.parametrize("path", PATHS, ids=["-".join(map(str, x)) for x in PATHS])
@pytest.mark.parametrize("name", NAMES)
def test_operators_exact(name, path):
    setup()
    g = gd.load(name)
    part, order, run = path
    p = g.parts[0]
    m = ps.PowerSparseMatrixGPU.from_csr(csr_of(g), cu_count=p.cu, csr_positions=True,
                                         task_order=order, run_order=run, spmm_partition=part)
    S = m.GroupTypeNum()
    assert S == p.S
    streams = [ps.Stream() for _ in range(S)] if S > 1 else None
    keep = stored_rows(p)
    for N in (32, 64, 96, 128, 256, 512):
        say(f"golden {name} {part}/{order}/run={run} N={N} S={S} order={m.task_order}")
        B, X, Y = dense_inputs(g, N)
        want = expected_spmm(g, N)
        dB = ps.DeviceBuffer(host=B)
        dC = ps.DeviceBuffer.zeros(g.rows * N * 4)
        ps.SpMM(m, N, dB, dC, S, streams)
        ps.synchronize()
        np.testing.assert_array_equal(dC.download(np.float32).reshape(g.rows, N), want)
        # a second call without zeroing: stored rows rewritten, the others doubled
        ps.SpMM(m, N, dB, dC, S, streams)
        ps.synchronize()
        twice = 2 * want
        twice[keep] = want[keep]
        np.testing.assert_array_equal(dC.download(np.float32).reshape(g.rows, N), twice)

        dX, dY = ps.DeviceBuffer(host=X), ps.DeviceBuffer(host=Y)
        sizes = m.sddmm_output_sizes()
        outs = [ps.DeviceBuffer.zeros(max(n, 1) * 4) for n in sizes]
        ps.SDDMM(m, N, dX, dY, outs, S, streams)
        ps.synchronize()
        for s in range(S):
            if sizes[s]:
                np.testing.assert_array_equal(outs[s].download(np.float32, sizes[s]),
                                              p.sddmm_expected(s, X, Y), err_msg=f"ws {s}")
        csr_out = ps.DeviceBuffer(max(g.nnz, 1) * 4)
        ps.SDDMMToCSR(m, N, dX, dY, csr_out)
        ps.synchronize()
        got = csr_out.download(np.float32, g.nnz)
        if N == g.n:
            np.testing.assert_array_equal(got, g.sddmm_csr)
        row_of = np.repeat(np.arange(g.rows), np.diff(g.row_ptr))
        dots = np.einsum("ij,ij->i", X[row_of].astype(np.float64),
                         Y[g.col_ind].astype(np.float64))
        np.testing.assert_array_equal(got, g.values.astype(np.float64) * dots)
    m.close()


@pytest.mark.parametrize("chunk", [1, _native.PS_TASK_CHUNK_AUTO])
@pytest.mark.parametrize("name", NAMES)
def test_raw_launchers_on_golden_worksets(name, chunk):
    """The stored worksets uploaded as they are and run through the C ABI's
    launchers (no preprocessing of this build involved)."""
    setup()
    g = gd.load(name)
    for p in g.parts:
        bufs, ws = [], []
        for s in range(p.S):
            col = ps.DeviceBuffer(host=p.col[s]) if p.col[s].size else None
            val = ps.DeviceBuffer(host=p.val[s]) if p.val[s].size else None
            des = ps.DeviceBuffer(host=p.des[s]) if p.des[s].size else None
            bufs += [col, val, des]
            ws.append((col, val, des, p.group_num[s], 0 if s == 0 else 32 << (s - 1)))
        off = ps.DeviceBuffer(host=p.residue_offset)
        atom = ps.DeviceBuffer(host=p.residue_atomic) if p.residue_atomic.size else \
            ps.DeviceBuffer(16)
        B, X, Y = dense_inputs(g, g.n)
        say(f"golden raw {name} cu={p.cu} cap={p.cap} chunk={chunk}")
        dB = ps.DeviceBuffer(host=B)
        dC = ps.DeviceBuffer.zeros(g.rows * g.n * 4)
        ps.spmm_launch(ws, off, atom, g.rows, g.cols, g.n, dB, dC, task_chunk=chunk)
        ps.synchronize()
        np.testing.assert_array_equal(dC.download(np.float32).reshape(g.rows, g.n), g.spmm_c)
        dX, dY = ps.DeviceBuffer(host=X), ps.DeviceBuffer(host=Y)
        outs = [ps.DeviceBuffer.zeros(max(int(p.col[s].size), 1) * 4) for s in range(p.S)]
        ps.sddmm_launch(ws, off, g.rows, g.cols, g.n, dX, dY, outs, task_chunk=chunk)
        ps.synchronize()
        for s in range(p.S):
            n = int(p.col[s].size)
            if n:
                np.testing.assert_array_equal(outs[s].download(np.float32, n),
                                              p.sddmm_expected(s, X, Y), err_msg=f"ws {s}")
