"""Writes the golden fixtures under tests/golden/ (run from the repository
root after `make -C oracle`):

    python tests/golden/make_golden.py

Each fixture `<graph>.npz` holds one small graph (values k/64) and, for each
(CU count, workset cap) pair listed with it, the worksets that the
reference's preprocessing (ParCIS/PowerSparse utils/matrix_utils.cu:31-663,
restated in oracle/oracle.cpp) makes of it, plus the results of SpMM
(PowerSparse_SpMM/spmm_solution.cu:7-34) and SDDMM
(PowerSparse_SDDMM/sddmm_solution.cu:7-50, CSR order) on the dense inputs
that tests/golden_data.py defines. The format is described there.

The expected outputs are computed here in float64 from the CSR alone (not by
the oracle) and checked to be exact in FP32 before they are stored as
float32.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
TESTS = os.path.dirname(HERE)
ROOT = os.path.dirname(TESTS)
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, TESTS)

import golden_data as gd  # noqa: E402
import oracle  # noqa: E402

N = 32


def random_rows(rng, cols, degrees, dup=False):
    out = []
    for d in degrees:
        d = int(min(d, cols))
        r = rng.integers(0, cols, d) if dup else rng.choice(cols, d, replace=False)
        out.append([int(c) for c in r])
    return out


def graphs():
    """name -> (cols, rows as lists of column ids, [(cu, cap), ...])."""
    rng = np.random.default_rng(20261202)
    g = {}
    # The 3 x 4 case of the hand-derived worksets (fine mode, S = 1).
    g["hand_3x4"] = (4, [[0, 1, 2], [0], [3, 0]], [(1, 0)])
    # 40 rows of 32 + rows of 33, 64, 0 and 5 nonzeros: S = 2.
    g["hand_44x70"] = (70, [list(range(32))] * 40 +
                       [list(range(33)), list(range(64)), [], list(range(64, 69))], [(1, 0)])
    # Skewed degrees with empty rows: S = 2 at one CU, fine mode at 256.
    deg = np.minimum(rng.geometric(0.04, 150), 300)
    deg[rng.choice(150, 12, replace=False)] = 0
    g["skewed"] = (400, random_rows(rng, 400, deg), [(1, 0), (256, 0)])
    # Repeated column ids inside rows.
    g["duplicates"] = (300, random_rows(rng, 300, rng.integers(0, 90, 120), dup=True), [(2, 0)])
    # Hub rows reaching groups of 256 (S = 5 at one CU), and the same graph
    # with the workset count capped at 3, the tuned SpMM partition's cap.
    hub = list(rng.integers(1024, 1100, 8)) + list(rng.integers(0, 40, 30))
    g["hubs"] = (1200, random_rows(rng, 1200, hub), [(1, 0), (1, 3)])
    # Rows of exactly 128 and 32 nonzeros: worksets 1 and 3 filled, workset 2
    # (groups of 64) empty, no residue.
    g["empty_middle"] = (200, random_rows(rng, 200, [128] * 40 + [32] * 10), [(1, 0)])
    # Every row holds the two hub columns 0 and 1, so most other columns tie
    # on their counts; every third row long enough for a group of 32 (S = 2
    # at one CU, fine mode at two).
    rows = []
    for r in range(96):
        d = (68 if r < 2 else 40) if r % 3 == 0 else int(rng.integers(0, 12))
        rows.append([0, 1] + [int(x) for x in rng.choice(np.arange(2, 500), d, replace=False)])
    g["star_ties"] = (500, rows, [(1, 0), (2, 0)])
    return g


def exact32(x, what):
    y = np.asarray(x, np.float64).astype(np.float32)
    assert np.array_equal(y.astype(np.float64), x), f"{what}: not exact in FP32"
    return y


def val_k(v):
    k = np.rint(np.asarray(v, np.float64) * 64)
    assert np.array_equal(k / 64, v) and np.abs(k).max(initial=0) <= 64
    return k.astype(np.int8)


def make(name, cols, row_lists, parts, rng):
    rows = len(row_lists)
    row_ptr = np.zeros(rows + 1, np.int32)
    row_ptr[1:] = np.cumsum([len(r) for r in row_lists])
    col_ind = np.array([c for r in row_lists for c in r], np.int32)
    k = (rng.integers(1, 65, col_ind.size) * rng.choice([-1, 1], col_ind.size)).astype(np.int8)
    values = k.astype(np.float32) / np.float32(64)
    f = {"rows": rows, "cols": cols, "n": N, "row_ptr": row_ptr, "col_ind": col_ind,
         "values_k": k, "parts": np.array(parts, np.int32).reshape(-1, 2)}
    for p, (cu, cap) in enumerate(parts):
        w = oracle.preprocess(rows, cols, row_ptr, col_ind, values, cu, max_group_types=cap)
        if p == 0:
            f["sigbit"], f["L"] = w.sigbit, w.L
        assert np.array_equal(f["sigbit"], w.sigbit) and f["L"] == w.L
        pre = f"p{p}_"
        f[pre + "S"] = w.S
        f[pre + "group_num"] = np.array(w.group_num, np.int32)
        f[pre + "residue_offset"] = w.residue_offset
        f[pre + "residue_atomic"] = w.residue_atomic
        for s in range(w.S):
            f[f"{pre}ws{s}_col"] = w.col[s]
            f[f"{pre}ws{s}_val_k"] = val_k(w.val[s])
            f[f"{pre}ws{s}_des"] = w.des[s]
        print(f"{name}: rows={rows} cols={cols} nnz={col_ind.size} cu={cu} cap={cap} "
              f"S={w.S} groups={w.group_num} L={w.L}")

    B = gd.dense(cols, N, gd.SALT_B).astype(np.float64)
    X = gd.dense(rows, N, gd.SALT_X).astype(np.float64)
    Y = gd.dense(cols, N, gd.SALT_Y).astype(np.float64)
    vals64 = values.astype(np.float64)
    row_of = np.repeat(np.arange(rows), np.diff(row_ptr))
    C = np.zeros((rows, N))
    np.add.at(C, row_of, vals64[:, None] * B[col_ind])
    f["spmm_c"] = exact32(C, f"{name} SpMM")
    f["sddmm_csr"] = exact32(vals64 * np.einsum("ij,ij->i", X[row_of], Y[col_ind]),
                             f"{name} SDDMM")
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **f)


def main():
    rng = np.random.default_rng(7)
    for name, (cols, row_lists, parts) in graphs().items():
        make(name, cols, row_lists, parts, rng)


if __name__ == "__main__":
    main()
