"""Loader of the golden fixtures in tests/golden/ (written by
tests/golden/make_golden.py) and the deterministic dense inputs they are
defined on.

A fixture `<graph>.npz` holds a small CSR matrix whose values are k/64
(int8 k, stored), its column signature bits, the worksets that the
reference's preprocessing (ParCIS/PowerSparse utils/matrix_utils.cu:31-663)
makes of it for one or more (CU count, workset cap) pairs, and the exact
results of SpMM (spmm_solution.cu:7-34) and SDDMM (sddmm_solution.cu:7-50,
in CSR order) on the dense inputs of `dense()` below.

Every value is a small dyadic rational, so every FP32 product and every
partial sum in any order is exact (magnitudes below 2^12, at most 20
significant bits): a correct kernel reproduces the stored float32 results
bit for bit, whatever its summation order.
"""
import glob
import os

import numpy as np

GOLDEN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

# Salts of the three dense operands.
SALT_B, SALT_X, SALT_Y = 1, 2, 3


def dense_k(count, n, salt):
    """int8 k in [-16, 16] for a count x n operand: a 32-bit integer mix of
    (index, feature, salt) reduced mod 33; the operand is k / 16."""
    i = np.arange(count, dtype=np.uint64)[:, None]
    j = np.arange(n, dtype=np.uint64)[None, :]
    m = np.uint64(0xFFFFFFFF)
    h = (i * np.uint64(0x9E3779B1) + j * np.uint64(0x85EBCA77) +
         np.uint64(salt) * np.uint64(0xC2B2AE3D)) & m
    h ^= h >> np.uint64(15)
    h = (h * np.uint64(0x2C1B3C6D)) & m
    h ^= h >> np.uint64(12)
    return ((h % np.uint64(33)).astype(np.int64) - 16).astype(np.int8)


def dense(count, n, salt):
    return (dense_k(count, n, salt).astype(np.float32) / np.float32(16))


class Partition:
    """Worksets of one (cu, cap) pair, as the reference's accessors return them."""

    def __init__(self, z, p):
        self.cu, self.cap = (int(v) for v in z["parts"][p])
        pre = f"p{p}_"
        self.S = int(z[pre + "S"])
        self.group_num = [int(v) for v in z[pre + "group_num"]]
        self.residue_offset = z[pre + "residue_offset"]
        self.residue_atomic = z[pre + "residue_atomic"]
        self.col = [z[f"{pre}ws{s}_col"] for s in range(self.S)]
        self.val = [(z[f"{pre}ws{s}_val_k"].astype(np.float32) / np.float32(64))
                    for s in range(self.S)]
        self.des = [z[f"{pre}ws{s}_des"] for s in range(self.S)]

    def offsets(self, s):
        if s == 0:
            return self.residue_offset.astype(np.int64)
        return np.arange(self.group_num[s] + 1, dtype=np.int64) * (32 << (s - 1))

    def sddmm_expected(self, s, X, Y):
        """value * <X[row], Y[col]> for each entry of workset s, in float64
        (exact for the fixture's inputs)."""
        des = np.repeat(self.des[s], np.diff(self.offsets(s)))
        dots = np.einsum("ij,ij->i", X[des].astype(np.float64),
                         Y[self.col[s]].astype(np.float64))
        return self.val[s].astype(np.float64) * dots


class Golden:
    def __init__(self, path):
        self.name = os.path.splitext(os.path.basename(path))[0]
        with np.load(path, allow_pickle=False) as z:
            self.rows, self.cols, self.n = int(z["rows"]), int(z["cols"]), int(z["n"])
            self.row_ptr = z["row_ptr"]
            self.col_ind = z["col_ind"]
            self.values = z["values_k"].astype(np.float32) / np.float32(64)
            self.sigbit = z["sigbit"]
            self.L = int(z["L"])
            self.spmm_c = z["spmm_c"]
            self.sddmm_csr = z["sddmm_csr"]
            self.parts = [Partition(z, p) for p in range(len(z["parts"]))]
        self.B = dense(self.cols, self.n, SALT_B)
        self.X = dense(self.rows, self.n, SALT_X)
        self.Y = dense(self.cols, self.n, SALT_Y)

    @property
    def nnz(self):
        return int(self.col_ind.size)


def names():
    return sorted(os.path.splitext(os.path.basename(p))[0]
                  for p in glob.glob(os.path.join(GOLDEN_DIR, "*.npz")))


def load(name):
    return Golden(os.path.join(GOLDEN_DIR, name + ".npz"))
