"""The golden fixtures (tests/golden/*.npz) on the CPU: the oracle and the
independent brute force both reproduce the stored worksets, and the stored
SpMM / SDDMM results are what the CSR and the dense inputs define.

The fixtures freeze what the pinned oracle made of each graph when they were
written; these tests keep the oracle from drifting away from them, and the
GPU tests (test_gpu_golden.py) compare the product with the same files."""
import numpy as np
import pytest

import brute
import golden_data as gd
import oracle

NAMES = gd.names()


def test_fixture_set():
    assert len(NAMES) >= 7
    S = [p.S for n in NAMES for p in gd.load(n).parts]
    caps = [p.cap for n in NAMES for p in gd.load(n).parts]
    # fine mode, two worksets, five worksets, a capped partition
    assert {1, 2, 5} <= set(S) and 3 in caps


def test_dense_inputs_fixed():
    # the generator of the dense operands is part of the fixture format
    k = gd.dense_k(4, 4, gd.SALT_B)
    assert k.dtype == np.int8 and k.min() >= -16 and k.max() <= 16
    np.testing.assert_array_equal(gd.dense_k(1000, 32, 2)[:2, :4], gd.dense_k(2, 4, 2))
    big = gd.dense_k(1000, 32, 3)
    assert abs(float(big.mean())) < 0.5 and len(np.unique(big)) == 33


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_worksets(name):
    g = gd.load(name)
    for p in g.parts:
        w = oracle.preprocess(g.rows, g.cols, g.row_ptr, g.col_ind, g.values, p.cu,
                              max_group_types=p.cap)
        assert (w.S, w.L, w.group_num) == (p.S, g.L, p.group_num)
        np.testing.assert_array_equal(w.sigbit, g.sigbit)
        np.testing.assert_array_equal(w.residue_offset, p.residue_offset)
        np.testing.assert_array_equal(w.residue_atomic, p.residue_atomic)
        for s in range(p.S):
            np.testing.assert_array_equal(w.des[s], p.des[s], err_msg=f"des {s}")
            np.testing.assert_array_equal(w.col[s], p.col[s], err_msg=f"col {s}")
            np.testing.assert_array_equal(w.val[s].view(np.uint32), p.val[s].view(np.uint32))


@pytest.mark.parametrize("name", NAMES)
def test_brute_force_reproduces_worksets(name):
    g = gd.load(name)
    for p in g.parts:
        S, out = brute.preprocess(g.rows, g.cols, g.row_ptr.tolist(), g.col_ind.tolist(),
                                  g.values.tolist(), p.cu, g.sigbit.tolist(), g.L,
                                  max_group_types=p.cap)
        assert S == p.S
        for s in range(S):
            assert len(out[s]["des"]) == p.group_num[s]
            np.testing.assert_array_equal(np.array(out[s]["des"], np.int32), p.des[s])
            np.testing.assert_array_equal(np.array(out[s]["col"], np.int32), p.col[s])
            np.testing.assert_array_equal(np.array(out[s]["val"], np.float32), p.val[s])
        np.testing.assert_array_equal(np.array(out[0]["offsets"], np.int32), p.residue_offset)
        np.testing.assert_array_equal(np.array(out[0]["atomic"], np.uint8), p.residue_atomic)


@pytest.mark.parametrize("name", NAMES)
def test_expected_results(name):
    g = gd.load(name)
    row_of = np.repeat(np.arange(g.rows), np.diff(g.row_ptr))
    # SpMM: a dense product of the CSR, exact in float64
    A = np.zeros((g.rows, g.cols))
    np.add.at(A, (row_of, g.col_ind), g.values.astype(np.float64))
    np.testing.assert_array_equal(g.spmm_c, (A @ g.B.astype(np.float64)).astype(np.float32))
    # the oracle's CPU check path agrees bit for bit on these exact inputs
    E = oracle.spmm(g.row_ptr, g.col_ind, g.values, g.n, g.B)
    np.testing.assert_array_equal(np.asarray(E, np.float64), g.spmm_c.astype(np.float64))
    # SDDMM in CSR order: value * <X[row], Y[col]>
    D = (g.X.astype(np.float64) @ g.Y.astype(np.float64).T)[row_of, g.col_ind]
    np.testing.assert_array_equal(g.sddmm_csr, (g.values * D).astype(np.float32))
    # each workset order holds the same (row, col, value, result) entries
    want = sorted(zip(row_of, g.col_ind, g.values, g.sddmm_csr))
    for p in g.parts:
        got = []
        for s in range(p.S):
            des = np.repeat(p.des[s], np.diff(p.offsets(s)))
            got += zip(des, p.col[s], p.val[s], p.sddmm_expected(s, g.X, g.Y).astype(np.float32))
        assert sorted(got) == want, f"cu={p.cu} cap={p.cap}"
