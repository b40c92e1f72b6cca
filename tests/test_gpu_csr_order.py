"""SDDMM output in the input CSR's order (SDDMMToCSR, WorksetToCSR) and the
CSR-position map the preprocessing keeps for it. The map is checked against
the input arrays themselves; the values against the oracle's double SDDMM
evaluated row by row in CSR order (one group per row)."""
import numpy as np
import pytest

import oracle
import powersparse_amd as ps
import tolerance
from gpu_util import random_graph, say, setup

pytestmark = pytest.mark.gpu


def check_positions(csr, m):
    """The kept positions form a bijection onto 0..nnz-1 and every slot holds
    the column, value bits and row of the CSR entry it names."""
    row_of = np.repeat(np.arange(csr.rows), np.diff(csr.row_ptr))
    seen = np.zeros(csr.nnz, np.int32)
    offs0 = m.residue_offset()
    for s in range(m.GroupTypeNum()):
        if m.GroupNum()[s] == 0:
            continue
        col, val, des = m.download_workset(s)
        pos = m.download_csr_position(s)
        assert pos.min() >= 0 and pos.max() < csr.nnz
        np.testing.assert_array_equal(csr.col_ind[pos], col, err_msg=f"columns ws {s}")
        np.testing.assert_array_equal(csr.values[pos].view(np.uint32), val.view(np.uint32))
        lens = np.diff(offs0) if s == 0 else np.full(m.GroupNum()[s], ps.GROUP_SIZE(s))
        np.testing.assert_array_equal(row_of[pos], np.repeat(des, lens), err_msg=f"rows ws {s}")
        np.add.at(seen, pos, 1)
    assert (seen == 1).all()


def expected_csr(csr, N, X, Y):
    rows = np.arange(csr.rows, dtype=np.int32)
    return oracle.sddmm(rows, csr.row_ptr, csr.col_ind, csr.values, N, X, Y, with_mag=True)


CASES = [("C0", 1, 32, 256), ("C1", 20, 128, 256), ("C1", 50, 32, 4), ("C4", 16, 64, 256),
         ("C3", 60, 96, 2)]


@pytest.mark.parametrize("cfg,scale,N,cu", CASES)
def test_sddmm_csr_order(cfg, scale, N, cu):
    setup()
    csr = ps.synth(cfg, seed=21, scale=scale)
    m = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=cu, csr_positions=True)
    say(f"csr order {cfg}/{scale} N={N} S={m.GroupTypeNum()} nnz={csr.nnz}")
    check_positions(csr, m)
    rng = np.random.default_rng(3)
    X = rng.normal(size=(csr.rows, N)).astype(np.float32)
    Y = rng.normal(size=(csr.cols, N)).astype(np.float32)
    dX, dY = ps.DeviceBuffer(host=X), ps.DeviceBuffer(host=Y)
    # no zeroing needed: fill the output with NaN first
    out = ps.DeviceBuffer(host=np.full(csr.nnz, np.nan, np.float32))
    ps.SDDMMToCSR(m, N, dX, dY, out)
    ps.synchronize()
    got = out.download(np.float32, csr.nnz)
    E, M = expected_csr(csr, N, X, Y)
    say("  ", tolerance.check(got, E, M, f"SDDMMToCSR {cfg} N={N}"))
    # the workset-order operator followed by the permutation gives the same bits
    outs = [ps.DeviceBuffer.zeros(max(n, 1) * 4) for n in m.sddmm_output_sizes()]
    ps.SDDMMAsync(m, N, dX, dY, outs)
    moved = ps.DeviceBuffer(host=np.full(csr.nnz, np.nan, np.float32))
    ps.WorksetToCSR(m, outs, moved)
    ps.synchronize()
    np.testing.assert_array_equal(moved.download(np.float32, csr.nnz).view(np.uint32),
                                  got.view(np.uint32))


@pytest.mark.parametrize("seed", range(4))
def test_sddmm_csr_order_random(seed):
    # duplicate (row, column) entries and hub rows: every duplicate keeps its own slot
    setup()
    rng = np.random.default_rng(40 + seed)
    csr = random_graph(rng, int(rng.integers(50, 400)), int(rng.integers(20, 2000)), 80,
                       hubs=2, hub_deg=int(rng.integers(100, 1500)), dup=(seed % 2 == 1))
    if csr.nnz == 0:
        return
    m = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=int(rng.choice([1, 2, 64])),
                                         csr_positions=True)
    say(f"random csr order seed={seed} nnz={csr.nnz} S={m.GroupTypeNum()}")
    check_positions(csr, m)
    N = 32
    X = rng.normal(size=(csr.rows, N)).astype(np.float32)
    Y = rng.normal(size=(csr.cols, N)).astype(np.float32)
    out = ps.DeviceBuffer(host=np.full(csr.nnz, np.nan, np.float32))
    dX, dY = ps.DeviceBuffer(host=X), ps.DeviceBuffer(host=Y)  # alive until the sync
    ps.SDDMMToCSR(m, N, dX, dY, out)
    ps.synchronize()
    E, M = expected_csr(csr, N, X, Y)
    tolerance.check(out.download(np.float32, csr.nnz), E, M, "SDDMMToCSR random")


def test_csr_order_needs_positions():
    setup()
    csr = ps.synth("C0", seed=1)
    m = ps.PowerSparseMatrixGPU.from_csr(csr)
    assert m.csr_position(0) == 0
    X = ps.DeviceBuffer(csr.rows * 32 * 4)
    Y = ps.DeviceBuffer(csr.cols * 32 * 4)
    out = ps.DeviceBuffer(csr.nnz * 4)
    with pytest.raises(ValueError, match="csr_positions"):
        ps.SDDMMToCSR(m, 32, X, Y, out)
    with pytest.raises(ValueError, match="csr_positions"):
        ps.WorksetToCSR(m, [out], out)
    m2 = ps.PowerSparseMatrixGPU.from_csr(csr, csr_positions=True)
    with pytest.raises(ValueError, match="multiple of 32"):
        ps.SDDMMToCSR(m2, 48, X, Y, out)
