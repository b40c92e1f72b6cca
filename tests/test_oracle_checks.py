"""Pins the oracle's check path: CheckSpmm / CheckSddmm in double
(benchmarks/benchmark.cu:64-96) against numpy's dense float64 products and
closed forms, and DenseInput's generator against values fixed by the C++
standard."""
import numpy as np

import oracle


def dense(rows, cols, rp, ci, va):
    A = np.zeros((rows, cols))
    for r in range(rows):
        for p in range(rp[r], rp[r + 1]):
            A[r, ci[p]] += va[p]  # duplicates add, as in the CSR product
    return A


def random_csr(rng, rows, cols, density):
    mask = rng.random((rows, cols)) < density
    rp = np.concatenate([[0], np.cumsum(mask.sum(1))]).astype(np.int32)
    ci = np.nonzero(mask)[1].astype(np.int32)
    va = rng.uniform(-1, 1, ci.size).astype(np.float32)
    return rp, ci, va


def test_spmm_matches_numpy_dense():
    rng = np.random.default_rng(1)
    for n in (32, 64, 96):
        rp, ci, va = random_csr(rng, 50, 40, 0.2)
        B = rng.uniform(-1, 1, (40, n)).astype(np.float32)
        C, mag = oracle.spmm(rp, ci, va, n, B, with_mag=True)
        A = dense(50, 40, rp, ci, va)
        np.testing.assert_allclose(C, A @ B.astype(np.float64), rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(mag, np.abs(A) @ np.abs(B.astype(np.float64)), rtol=1e-12)


def test_spmm_closed_forms():
    rng = np.random.default_rng(2)
    B = rng.uniform(-1, 1, (16, 32)).astype(np.float32)
    eye = np.arange(17, dtype=np.int32)
    # identity: C == B exactly
    C = oracle.spmm(eye, np.arange(16, dtype=np.int32), np.ones(16, np.float32), 32, B)
    np.testing.assert_array_equal(C, B.astype(np.float64))
    # duplicated entries add up; empty rows give zeros
    rp = np.array([0, 3, 3], np.int32)
    C = oracle.spmm(rp, np.array([5, 5, 2], np.int32), np.array([1, 2, 4], np.float32), 32, B)
    Bd = B.astype(np.float64)
    np.testing.assert_allclose(C[0], 3.0 * Bd[5] + 4.0 * Bd[2], rtol=1e-12)
    assert (C[1] == 0).all()


def test_sddmm_matches_numpy():
    rng = np.random.default_rng(3)
    for k in (32, 64, 128):
        X = rng.normal(size=(20, k)).astype(np.float32)
        Y = rng.normal(size=(30, k)).astype(np.float32)
        des = np.array([3, 7, 7, 19], np.int32)
        off = np.array([0, 5, 6, 20, 22], np.int32)
        ci = rng.integers(0, 30, 22).astype(np.int32)
        va = rng.uniform(0, 1, 22).astype(np.float32)
        out, mag = oracle.sddmm(des, off, ci, va, k, X, Y, with_mag=True)
        rows = np.repeat(des, np.diff(off))
        Xd, Yd = X.astype(np.float64), Y.astype(np.float64)
        ref = np.einsum("ij,ij->i", Xd[rows], Yd[ci]) * va
        np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(mag, np.abs(Xd[rows] * Yd[ci]).sum(1) * va, rtol=1e-12)


def test_mt19937_standard_values():
    # [rand.predef]: the 10000th output of a default-constructed (seed 5489)
    # std::mt19937 is 4123659995.
    assert oracle.mt19937_nth(5489, 10000) == 4123659995
    # seed 1, first output 1791095845 -> 1791095845 % 3 = 1 -> DenseInput 0.1f
    assert oracle.mt19937_nth(1, 1) == 1791095845
    a = oracle.dense_input(1, 4)
    assert a[0] == np.float32(0.1)
    assert set(np.unique(oracle.dense_input(1, 1000))) <= {np.float32(0), np.float32(0.1),
                                                           np.float32(0.2)}


def test_dense_input_draw_order():
    # lhs is drawn before rhs from one generator (benchmark.cu:137-140)
    lhs, rhs = oracle.dense_input(1, 10, 7)
    both = oracle.dense_input(1, 17)
    np.testing.assert_array_equal(np.concatenate([lhs, rhs]), both)


def test_tolerance_counts_outputs_passing_only_by_the_condition_bound():
    """tolerance.check: an output beyond 1e-4 relative and 1e-5 absolute but
    within 16 * 2^-24 * sum|a b| passes and is counted in `only_cond`; a planted
    error beyond all three bounds fails."""
    import pytest

    import tolerance
    # a cancelled sum: expected 1e-3, magnitudes summed 1e3, error 5e-5
    exp = np.array([1.0, 1e-3, 2.0, 0.0])
    mag = np.array([1.0, 1e3, 2.0, 1.0])
    act = exp + np.array([5e-5, 5e-5, 1e-4, 5e-6])
    r = tolerance.check(act, exp, mag, "counts")
    # output 0 passes by 1e-4 relative (5e-5 <= 1e-4), output 1 only by the
    # condition bound (5e-5 <= 16 * 2^-24 * 1e3 ~ 9.5e-4), output 2 relative
    # (1e-4 <= 2e-4), output 3 absolute
    assert r["n"] == 4 and r["only_cond"] == 1
    assert r["only_cond_max_abs"] == pytest.approx(5e-5)
    with pytest.raises(AssertionError, match="1 of 4 outputs out of tolerance"):
        tolerance.check(exp + np.array([0, 2e-3, 0, 0]), exp, mag, "planted")
