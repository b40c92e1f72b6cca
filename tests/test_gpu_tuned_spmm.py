"""Tuned SpMM partition (SpmmPartition::kTuned): the capped partition it runs
on is bit-exact with the oracle's capped partition, and SpMM on it matches the
oracle and the parity partition (FP32 tolerance), including the reference's
accumulate-without-zeroing behaviour over repeated calls; it is built only
when the parity partition has more worksets than the cap and the task order
is the signature order."""
import numpy as np
import pytest

import oracle
import powersparse_amd as ps
import tolerance
from gpu_util import random_graph, say, setup

pytestmark = pytest.mark.gpu

CAP = 3  # kTunedSpmmGroupTypes


def check_capped(csr, cu, cap):
    w = oracle.preprocess(csr.rows, csr.cols, csr.row_ptr, csr.col_ind, csr.values, cu,
                          max_group_types=cap)
    m = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=cu, max_group_types=cap,
                                         spmm_partition="parity")
    say(f"  capped at {cap}: S={m.GroupTypeNum()} groups={m.GroupNum()}")
    assert m.GroupTypeNum() == w.S and m.GroupNum() == w.group_num
    np.testing.assert_array_equal(m.residue_offset(), w.residue_offset)
    np.testing.assert_array_equal(m.residue_atomic(), w.residue_atomic)
    for s in range(w.S):
        if w.group_num[s]:
            col, val, des = m.download_workset(s)
            np.testing.assert_array_equal(des, w.des[s])
            np.testing.assert_array_equal(col, w.col[s])
            np.testing.assert_array_equal(val.view(np.uint32), w.val[s].view(np.uint32))
    m.close()


GRAPHS = {
    "c1": (lambda: ps.synth("C1", seed=51, scale=50), 8),
    "c3": (lambda: ps.synth("C3", seed=52, scale=100), 2),
    "hubs": (lambda: random_graph(np.random.default_rng(53), 900, 1200, 90, hubs=12,
                                  hub_deg=1100), 1),
}


@pytest.mark.parametrize("name", sorted(GRAPHS))
def test_capped_partition_bit_exact(name):
    setup()
    make, cu = GRAPHS[name]
    csr = make()
    say(f"capped partition {name}: rows={csr.rows} nnz={csr.nnz}")
    for cap in (1, 2, CAP, 5):
        check_capped(csr, cu, cap)


def spmm(m, N, B, calls=1):
    dB = ps.DeviceBuffer(host=B)
    C = ps.DeviceBuffer.zeros(m.MatrixRow() * N * 4)
    S = m.GroupTypeNum()
    streams = [ps.Stream() for _ in range(S)] if S > 1 else None
    for _ in range(calls):  # outputs not cleared, as the reference harness
        ps.SpMM(m, N, dB, C, S, streams)
    ps.synchronize()
    return C.download(np.float32).reshape(m.MatrixRow(), N)


@pytest.mark.parametrize("name", sorted(GRAPHS))
@pytest.mark.parametrize("N", [32, 64, 128])
def test_tuned_spmm_matches_oracle_and_parity(name, N):
    setup()
    make, cu = GRAPHS[name]
    csr = make()
    tuned = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=cu, task_order="signature")
    parity = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=cu, task_order="signature",
                                              spmm_partition="parity")
    say(f"tuned SpMM {name} N={N}: parity S={parity.GroupTypeNum()}, "
        f"SpMM on S={tuned.spmm_worksets}")
    assert parity.spmm_worksets == parity.GroupTypeNum()
    assert tuned.GroupTypeNum() == parity.GroupTypeNum()  # the public worksets are unchanged
    assert tuned.spmm_worksets == min(CAP, parity.GroupTypeNum())
    rng = np.random.default_rng(N)
    B = rng.uniform(-1, 1, (csr.cols, N)).astype(np.float32)
    E, M = oracle.spmm(csr.row_ptr, csr.col_ind, csr.values, N, B, with_mag=True)
    for m in (tuned, parity):
        tolerance.check(spmm(m, N, B), E, M, f"SpMM S_exec={m.spmm_worksets}")
    # two calls without zeroing: rows stored by a lone residue group (fewer
    # than 32 nonzeros) hold one product, every other row (a 32-nonzero row is
    # one block group) two, in either partition
    deg = np.diff(csr.row_ptr)
    assert min(tuned.spmm_worksets, parity.GroupTypeNum()) > 1  # the S > 1 rule below
    twice = np.where((deg >= 32)[:, None], 2 * E, E)
    for m in (tuned, parity):
        tolerance.check(spmm(m, N, B, calls=2), twice, 2 * M, f"SpMM x2 S_exec={m.spmm_worksets}")


def test_no_tuned_partition_in_row_order_or_small_partitions():
    setup()
    csr = ps.synth("C4", seed=54, scale=32)
    m = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=1, task_order="row")
    assert m.task_order == "row" and m.spmm_worksets == m.GroupTypeNum()
    m = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=256)
    assert m.spmm_worksets == m.GroupTypeNum() <= CAP
