"""GPU preprocessing (PowerSparseMatrixGPU) against the CPU oracle: every
index array bit-exact, values bitwise equal, at stated CU counts."""
import numpy as np
import pytest

import oracle
import powersparse_amd as ps
from gpu_util import random_graph, say, setup
from test_oracle_preprocess import csr_from_rows

pytestmark = pytest.mark.gpu


def compare(csr, cu):
    w = oracle.preprocess(csr.rows, csr.cols, csr.row_ptr, csr.col_ind, csr.values, cu)
    say(f"  oracle S={w.S} groups={w.group_num} L={w.L}")
    m = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=cu)
    assert m.GroupTypeNum() == w.S
    assert m.GroupNum() == w.group_num
    assert m.SignatureLen() == w.L
    assert m.PartitionCuCount() == cu
    np.testing.assert_array_equal(m.residue_offset(), w.residue_offset)
    np.testing.assert_array_equal(m.residue_atomic(), w.residue_atomic)
    for s in range(w.S):
        if w.group_num[s] == 0:
            assert m.WorksetColInd()[s] == 0
            continue
        col, val, des = m.download_workset(s)
        np.testing.assert_array_equal(des, w.des[s], err_msg=f"group_des[{s}]")
        np.testing.assert_array_equal(col, w.col[s], err_msg=f"col_ind[{s}]")
        np.testing.assert_array_equal(val.view(np.uint32), w.val[s].view(np.uint32),
                                      err_msg=f"sp_data[{s}]")
    m.close()
    return w


def test_hand_cases():
    setup()
    rp, ci, va = csr_from_rows([[0, 1, 2], [0], [3, 0]])
    compare(ps.HostCsr(3, 4, rp, ci, va), 1)
    rows = [list(range(32))] * 40 + [list(range(33)), list(range(64)), [], list(range(64, 69))]
    rp, ci, va = csr_from_rows(rows)
    compare(ps.HostCsr(44, 70, rp, ci, va), 1)


@pytest.mark.parametrize("seed", range(8))
@pytest.mark.parametrize("cu", [1, 2, 4, 64])
def test_random_graphs(seed, cu):
    setup()
    rng = np.random.default_rng(seed)
    csr = random_graph(rng, int(rng.integers(20, 400)), int(rng.integers(10, 3000)),
                       int(rng.choice([20, 80, 300])), hubs=int(rng.integers(0, 4)),
                       hub_deg=int(rng.integers(100, 2000)), dup=(seed % 3 == 2))
    if csr.nnz == 0:
        return
    say(f"random seed={seed} cu={cu} rows={csr.rows} nnz={csr.nnz}")
    compare(csr, cu)


@pytest.mark.parametrize("cfg,scale,cu", [
    ("C0", 1, 256), ("C0", 1, 1), ("C1", 100, 1), ("C1", 20, 8), ("C3", 100, 2),
    ("C4", 64, 1), ("C4", 16, 4)])
def test_configs(cfg, scale, cu):
    setup()
    csr = ps.synth(cfg, seed=7, scale=scale)
    say(f"config {cfg}/{scale} cu={cu} rows={csr.rows} nnz={csr.nnz}")
    compare(csr, cu)


@pytest.mark.parametrize("deg,rows", [(2048, 40), (8192, 36), (16384, 33), (20000, 34)])
def test_large_groups(deg, rows):
    # P = 1: 32+ rows of `deg` nonzeros make GROUP_SIZE up to 16384, exercising
    # the LDS bitonic (<= 8192) and the radix (> 8192) within-group column sorts
    setup()
    rng = np.random.default_rng(deg)
    cols = 3 * deg
    ci = np.concatenate([np.sort(rng.choice(cols, deg, replace=False)) for _ in range(rows)])
    rp = np.arange(rows + 1, dtype=np.int32) * deg
    csr = ps.HostCsr(rows, cols, rp, ci.astype(np.int32),
                     rng.uniform(-1, 1, ci.size).astype(np.float32))
    say(f"large groups deg={deg} rows={rows}")
    w = compare(csr, 1)
    assert w.S >= 2


def test_device_cu_count_default():
    setup()
    csr = ps.synth("C0", seed=1)
    m = ps.PowerSparseMatrixGPU.from_csr(csr)
    assert m.PartitionCuCount() == ps.device_props(0)["cu_count"]
    say("device:", ps.device_props(0))
