"""TEST INFRASTRUCTURE — ctypes wrapper of the CPU oracle (oracle/liboracle.so).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module, and only as the checker. See oracle.h for the reference files restated.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")
REF_READER = os.path.join(_HERE, "_ref", "mm_reader")

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"oracle library {LIB_PATH} missing; run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        vp, ip = ctypes.c_void_p, ctypes.c_int
        L.or_preprocess.restype = vp
        L.or_preprocess.argtypes = [ip, ip, ip, vp, vp, vp, ip, ctypes.c_char_p, ip]
        L.or_free.argtypes = [vp]
        for name in ("or_group_type_num", "or_signature_len"):
            getattr(L, name).restype = ip
            getattr(L, name).argtypes = [vp]
        L.or_group_num.restype = ip
        L.or_group_num.argtypes = [vp, ip]
        L.or_workset_len.restype = ctypes.c_longlong
        L.or_workset_len.argtypes = [vp, ip]
        L.or_copy_workset.argtypes = [vp, ip, vp, vp, vp]
        L.or_copy_residue.argtypes = [vp, vp, vp]
        L.or_copy_col_nnz.argtypes = [vp, vp]
        L.or_copy_ranked_pos.argtypes = [vp, vp]
        L.or_copy_sigbit.argtypes = [vp, vp]
        L.or_copy_initial_des.argtypes = [vp, ip, vp]
        L.or_copy_initial_residue.argtypes = [vp, vp, vp]
        L.or_copy_signature.argtypes = [vp, ip, vp]
        L.or_copy_group_perm.argtypes = [vp, ip, vp]
        L.or_has_signature.restype = ip
        L.or_has_signature.argtypes = [vp, ip]
        L.or_set_signature_order.argtypes = [ip]
        L.or_set_max_group_types.argtypes = [ip]
        L.or_order_bit_lists.argtypes = [ip, vp, vp, vp]
        L.or_analyze_group_type_num.restype = ip
        L.or_analyze_group_type_num.argtypes = [ip, vp, ip]
        L.or_generate_sigbit.restype = ip
        L.or_generate_sigbit.argtypes = [ip, vp, ip, vp]
        L.or_spmm.argtypes = [ip, vp, vp, vp, ip, vp, vp, vp, ip]
        L.or_sddmm.argtypes = [ip, vp, vp, vp, vp, ip, vp, vp, vp, vp, ip]
        L.or_dense_input.argtypes = [ctypes.c_uint, ctypes.c_size_t, vp, ctypes.c_size_t, vp]
        L.or_mt19937_nth.restype = ctypes.c_uint32
        L.or_mt19937_nth.argtypes = [ctypes.c_uint, ctypes.c_longlong]
        L.or_max_threads.restype = ip
        _lib = L
    return _lib


def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class Worksets:
    """Everything the oracle's preprocessing produced, as numpy arrays."""

    def __init__(self, h, rows, cols, nnz):
        L = lib()
        self.S = L.or_group_type_num(h)
        self.L = L.or_signature_len(h)
        self.group_num = [L.or_group_num(h, s) for s in range(self.S)]
        self.col, self.val, self.des = [], [], []
        for s in range(self.S):
            n = L.or_workset_len(h, s)
            c = np.empty(n, np.int32)
            v = np.empty(n, np.float32)
            d = np.empty(self.group_num[s], np.int32)
            L.or_copy_workset(h, s, c.ctypes.data, v.ctypes.data, d.ctypes.data)
            self.col.append(c)
            self.val.append(v)
            self.des.append(d)
        g0 = self.group_num[0]
        self.residue_offset = np.empty(g0 + 1, np.int32)
        self.residue_atomic = np.empty(g0, np.uint8)
        L.or_copy_residue(h, self.residue_offset.ctypes.data, self.residue_atomic.ctypes.data)
        self.col_nnz = np.empty(cols, np.int32)
        L.or_copy_col_nnz(h, self.col_nnz.ctypes.data)
        self.ranked = np.empty(nnz, np.int32)
        L.or_copy_ranked_pos(h, self.ranked.ctypes.data)
        self.sigbit = np.empty(cols, np.int32)
        L.or_copy_sigbit(h, self.sigbit.ctypes.data)
        self.initial_des, self.signature, self.perm = [], [], []
        words = self.L // 32
        for s in range(self.S):
            d = np.empty(self.group_num[s], np.int32)
            L.or_copy_initial_des(h, s, d.ctypes.data)
            self.initial_des.append(d)
            if L.or_has_signature(h, s):  # None when ordered by bit lists
                sg = np.zeros(self.group_num[s] * words, np.uint32)
                L.or_copy_signature(h, s, sg.ctypes.data)
                self.signature.append(sg.reshape(words, self.group_num[s]))
            else:
                self.signature.append(None)
            p = np.empty(self.group_num[s], np.int32)
            L.or_copy_group_perm(h, s, p.ctypes.data)
            self.perm.append(p)
        self.initial_residue_offset = np.empty(g0 + 1, np.int32)
        self.initial_residue_atomic = np.empty(g0, np.uint8)
        L.or_copy_initial_residue(h, self.initial_residue_offset.ctypes.data,
                                  self.initial_residue_atomic.ctypes.data)

    def offsets(self, s):
        """Group offsets of workset s (residue offsets, or multiples of GROUP_SIZE)."""
        if s == 0:
            return self.residue_offset
        gs = 32 * (1 << (s - 1))
        return np.arange(self.group_num[s] + 1, dtype=np.int64) * gs


ORDER_MODES = {"auto": 0, "bitmap_words": 1, "bit_lists": 2}


def preprocess(rows, cols, row_ptr, col_ind, values, cu_count, signature_order="auto",
               max_group_types=0):
    """Runs the CPU restatement; raises ValueError with the reference message.

    signature_order: how groups are put in signature order (the same order
    either way): "auto", "bitmap_words" (per-word stable sorts of the bitmaps,
    as the reference) or "bit_lists" (comparison of sorted bit lists).
    max_group_types: cap on the workset count S (0: none, the reference's rule)."""
    row_ptr, col_ind, values = _i32(row_ptr), _i32(col_ind), _f32(values)
    err = ctypes.create_string_buffer(256)
    nnz = int(col_ind.size)
    lib().or_set_signature_order(ORDER_MODES[signature_order])
    lib().or_set_max_group_types(int(max_group_types))
    try:
        h = lib().or_preprocess(rows, cols, nnz, row_ptr.ctypes.data if row_ptr.size else None,
                                col_ind.ctypes.data if col_ind.size else None,
                                values.ctypes.data if values.size else None, cu_count, err, 256)
    finally:
        lib().or_set_signature_order(0)
        lib().or_set_max_group_types(0)
    if not h:
        raise ValueError(err.value.decode())
    try:
        return Worksets(h, rows, cols, nnz)
    finally:
        lib().or_free(h)


def order_bit_lists(bit_sets):
    """Stable descending-signature order of groups given as iterables of
    signature bits: perm[k] = group at position k."""
    begin = np.zeros(len(bit_sets) + 1, np.int32)
    flat = []
    for g, bits in enumerate(bit_sets):
        flat.extend(int(b) for b in bits)
        begin[g + 1] = len(flat)
    flat = np.asarray(flat if flat else [0], np.int32)
    perm = np.empty(len(bit_sets), np.int32)
    if len(bit_sets):
        lib().or_order_bit_lists(len(bit_sets), begin.ctypes.data, flat.ctypes.data,
                                 perm.ctypes.data)
    return perm


def analyze_group_type_num(row_ptr, cu_count):
    row_ptr = _i32(row_ptr)
    return lib().or_analyze_group_type_num(row_ptr.size - 1, row_ptr.ctypes.data, cu_count)


def generate_sigbit(col_nnz, ffc=2):
    col_nnz = _i32(col_nnz)
    sig = np.empty_like(col_nnz)
    length = lib().or_generate_sigbit(col_nnz.size, col_nnz.ctypes.data, ffc, sig.ctypes.data)
    return sig, length


def spmm(row_ptr, col_ind, values, n, B, threads=0, with_mag=False):
    """CheckSpmm in double: returns C (rows x n) [and sum |a||b|]."""
    row_ptr, col_ind, values, B = _i32(row_ptr), _i32(col_ind), _f32(values), _f32(B)
    rows = row_ptr.size - 1
    C = np.empty((rows, n), np.float64)
    mag = np.empty((rows, n), np.float64) if with_mag else None
    lib().or_spmm(rows, row_ptr.ctypes.data, col_ind.ctypes.data if col_ind.size else None,
                  values.ctypes.data if values.size else None, n, B.ctypes.data, C.ctypes.data,
                  mag.ctypes.data if with_mag else None, threads)
    return (C, mag) if with_mag else C


def sddmm(des, offsets, col_ind, values, k, X, Y, threads=0, with_mag=False):
    """CheckSddmm in double for one workset given by groups."""
    des, offsets = _i32(des), _i32(offsets)
    col_ind, values, X, Y = _i32(col_ind), _f32(values), _f32(X), _f32(Y)
    n = int(offsets[-1]) if offsets.size else 0
    out = np.empty(n, np.float64)
    mag = np.empty(n, np.float64) if with_mag else None
    if des.size:
        lib().or_sddmm(des.size, des.ctypes.data, offsets.ctypes.data, col_ind.ctypes.data,
                       values.ctypes.data, k, X.ctypes.data, Y.ctypes.data, out.ctypes.data,
                       mag.ctypes.data if with_mag else None, threads)
    return (out, mag) if with_mag else out


def dense_input(seed, n1, n2=0):
    a = np.empty(int(n1), np.float32)
    b = np.empty(int(n2), np.float32)
    lib().or_dense_input(seed, a.size, a.ctypes.data if a.size else None, b.size,
                         b.ctypes.data if b.size else None)
    return (a, b) if n2 else a


def mt19937_nth(seed, index):
    return int(lib().or_mt19937_nth(seed, index))


def max_threads():
    return lib().or_max_threads()
