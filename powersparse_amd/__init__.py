"""PowerSparse on MI355X: FP32 SpMM (node aggregation) and SDDMM (edge messaging)
with GPU-built block/residue worksets.

The Python layer mirrors the reference's C++ interface (ParCIS/PowerSparse
utils/matrix_utils.h:20-76, PowerSparse_SpMM/PowerSparse_SpMM.h:14-17,
PowerSparse_SDDMM/PowerSparse_SDDMM.h:14-18) over the C facade of the C++17
host library; every device call goes through the HIP C ABI. Device buffers are
raw device pointers (DeviceBuffer). Errors keep the reference's exception
split: std::invalid_argument -> ValueError, other failures -> RuntimeError.
"""
import ctypes

import numpy as np

from . import _native
from ._native import PS_ERR_INVALID, PS_OK, DeviceProps, Workset

__all__ = [
    "PowerSparseMatrixGPU", "SpMM", "SpMMAsync", "SDDMM", "SDDMMAsync", "DeviceBuffer",
    "Stream", "Event", "HostCsr", "set_device", "device_count", "device_props", "synchronize",
    "synth", "read_mtx", "read_binary", "write_binary", "generate_sigbit", "workset_count",
    "dense_input", "GROUP_SIZE", "spmm_launch", "sddmm_launch",
]


def GROUP_SIZE(s):
    """GROUP_SIZE(I) = 32 * 2^(I-1) (utils/matrix_utils.h:8)."""
    return 32 * (1 << (s - 1))


def _raise(status, msg):
    msg = msg.decode() if isinstance(msg, bytes) else msg
    if status == PS_ERR_INVALID:
        raise ValueError(msg)
    raise RuntimeError(msg)


def _hip_call(status):
    if status != PS_OK:
        _raise(status, _native.hip().ps_last_error())


def _host_call(status):
    if status != PS_OK:
        _raise(status, _native.host().psx_last_error())


def _ptr(x):
    """Raw handle of a DeviceBuffer / Stream / Event, an int, or None."""
    if x is None:
        return None
    if hasattr(x, "ptr"):  # DeviceBuffer, Stream, Event
        return x.ptr
    return int(x)


# ------------------------------------------------------------------ device

def set_device(device=0):
    _hip_call(_native.hip().ps_set_device(device))


def device_count():
    n = ctypes.c_int(0)
    _hip_call(_native.hip().ps_device_count(ctypes.byref(n)))
    return n.value


def mem_get_info():
    """(free, total) bytes of device memory on the current device."""
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    _hip_call(_native.hip().ps_mem_get_info(ctypes.byref(free), ctypes.byref(total)))
    return free.value, total.value


def device_props(device=0):
    p = DeviceProps()
    _hip_call(_native.hip().ps_get_device_props(device, ctypes.byref(p)))
    return {
        "name": p.name.decode(), "arch": p.arch.decode(), "cu_count": p.cu_count,
        "major": p.major, "minor": p.minor, "lds_per_block": p.lds_per_block,
        "l2_bytes": p.l2_bytes, "clock_khz": p.clock_khz, "mem_clock_khz": p.mem_clock_khz,
        "mem_bus_width": p.mem_bus_width, "global_mem": p.global_mem,
    }


def synchronize():
    _hip_call(_native.hip().ps_device_synchronize())


class DeviceBuffer:
    """Device allocation (ps_malloc) with numpy upload/download."""

    def __init__(self, nbytes=0, host=None):
        if host is not None:
            host = np.ascontiguousarray(host)
            nbytes = host.nbytes
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        _hip_call(_native.hip().ps_malloc(ctypes.byref(p), self.nbytes))
        self.ptr = p.value or 0
        if host is not None:
            self.upload(host)

    @classmethod
    def zeros(cls, nbytes):
        b = cls(nbytes)
        b.zero()
        synchronize()
        return b

    def upload(self, host):
        host = np.ascontiguousarray(host)
        if host.nbytes > self.nbytes:
            raise ValueError("Upload size mismatch")
        if host.nbytes:
            _hip_call(_native.hip().ps_memcpy_htod(self.ptr, host.ctypes.data, host.nbytes))

    def download(self, dtype, count=None):
        dtype = np.dtype(dtype)
        if count is None:
            count = self.nbytes // dtype.itemsize
        out = np.empty(int(count), dtype=dtype)
        if out.nbytes > self.nbytes:
            raise ValueError("Download size mismatch")
        if out.nbytes:
            _hip_call(_native.hip().ps_memcpy_dtoh(out.ctypes.data, self.ptr, out.nbytes))
        return out

    def zero(self, stream=None):
        if self.nbytes:
            _hip_call(_native.hip().ps_memset_async(self.ptr, 0, self.nbytes, _ptr(stream)))

    def free(self):
        if self.ptr:
            _native.hip().ps_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def download(ptr, dtype, count):
    """Copies `count` elements of `dtype` from a raw device pointer."""
    dtype = np.dtype(dtype)
    out = np.empty(int(count), dtype=dtype)
    if out.nbytes:
        _hip_call(_native.hip().ps_memcpy_dtoh(out.ctypes.data, ptr, out.nbytes))
    return out


class Stream:
    def __init__(self):
        s = ctypes.c_void_p()
        _hip_call(_native.hip().ps_stream_create(ctypes.byref(s)))
        self.ptr = s.value

    def synchronize(self):
        _hip_call(_native.hip().ps_stream_synchronize(self.ptr))

    def destroy(self):
        if self.ptr:
            _native.hip().ps_stream_destroy(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        _hip_call(_native.hip().ps_event_create(ctypes.byref(e)))
        self.ptr = e.value

    def record(self, stream=None):
        _hip_call(_native.hip().ps_event_record(self.ptr, _ptr(stream)))

    def synchronize(self):
        _hip_call(_native.hip().ps_event_synchronize(self.ptr))

    def elapsed_ms(self, end):
        ms = ctypes.c_float()
        _hip_call(_native.hip().ps_event_elapsed_ms(ctypes.byref(ms), self.ptr, end.ptr))
        return ms.value

    def __del__(self):
        try:
            if self.ptr:
                _native.hip().ps_event_destroy(self.ptr)
        except Exception:
            pass


def fill_random(buf, count, seed, lo, hi, normal=False, stream=None):
    """Counter-based random fill of `count` floats on the device."""
    _hip_call(_native.hip().ps_fill_random_async(_ptr(buf), int(count), int(seed), float(lo),
                                                 float(hi), int(bool(normal)), _ptr(stream)))


# ---------------------------------------------------------------- host CSR

class HostCsr:
    """CSR matrix in host memory (int32 indices, float32 values)."""

    def __init__(self, rows, cols, row_ptr, col_ind, values):
        self.rows, self.cols = int(rows), int(cols)
        self.row_ptr = np.ascontiguousarray(row_ptr, dtype=np.int32)
        self.col_ind = np.ascontiguousarray(col_ind, dtype=np.int32)
        self.values = np.ascontiguousarray(values, dtype=np.float32)

    @property
    def nnz(self):
        return int(self.col_ind.size)

    @classmethod
    def _from_handle(cls, h):
        host = _native.host()
        try:
            rows, cols, nnz = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
            _host_call(host.psx_csr_info(h, ctypes.byref(rows), ctypes.byref(cols),
                                         ctypes.byref(nnz)))
            rp, ci, va = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
            _host_call(host.psx_csr_arrays(h, ctypes.byref(rp), ctypes.byref(ci),
                                           ctypes.byref(va)))

            def grab(p, n, t):
                if n == 0:
                    return np.zeros(0, dtype=t)
                ct = ctypes.c_int32 if t == np.int32 else ctypes.c_float
                return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ct)), (n,)).copy()

            return cls(rows.value, cols.value, grab(rp.value, rows.value + 1, np.int32),
                       grab(ci.value, nnz.value, np.int32), grab(va.value, nnz.value, np.float32))
        finally:
            host.psx_csr_free(h)

    def write_binary(self, path):
        """Writes the binary CSR format ("PSCSR001")."""
        with open(path, "wb") as f:
            f.write(b"PSCSR001")
            f.write(np.array([self.rows, self.cols, self.nnz], dtype="<i8").tobytes())
            f.write(self.row_ptr.astype("<i4").tobytes())
            f.write(self.col_ind.astype("<i4").tobytes())
            f.write(self.values.astype("<f4").tobytes())


def synth(config, seed=1, scale=1):
    """Seeded synthetic benchmark graph "C0".."C4" (node count / scale)."""
    h = ctypes.c_void_p()
    _host_call(_native.host().psx_csr_synth(config.encode(), int(seed), int(scale),
                                            ctypes.byref(h)))
    return HostCsr._from_handle(h)


def synth_chung_lu(n, gamma, mean_deg, max_deg, val_lo=0.0, val_hi=1.0, seed=1):
    h = ctypes.c_void_p()
    _host_call(_native.host().psx_csr_chung_lu(n, gamma, mean_deg, max_deg, val_lo, val_hi,
                                               seed, ctypes.byref(h)))
    return HostCsr._from_handle(h)


def synth_uniform_degree(rows, cols, deg_lo, deg_hi, val_lo=-1.0, val_hi=1.0, seed=1):
    h = ctypes.c_void_p()
    _host_call(_native.host().psx_csr_uniform_degree(rows, cols, deg_lo, deg_hi, val_lo, val_hi,
                                                     seed, ctypes.byref(h)))
    return HostCsr._from_handle(h)


def synth_community(communities, block, p_intra, inter_mean, empty_frac, single_frac,
                    val_lo=-1.0, val_hi=1.0, seed=1):
    h = ctypes.c_void_p()
    _host_call(_native.host().psx_csr_community(communities, block, p_intra, inter_mean,
                                                empty_frac, single_frac, val_lo, val_hi, seed,
                                                ctypes.byref(h)))
    return HostCsr._from_handle(h)


def read_mtx(path):
    """MatrixMarket reader with the reference semantics (benchmarks/matrix_market.cpp)."""
    h = ctypes.c_void_p()
    _host_call(_native.host().psx_csr_read_mtx(str(path).encode(), ctypes.byref(h)))
    return HostCsr._from_handle(h)


def read_binary(path):
    h = ctypes.c_void_p()
    _host_call(_native.host().psx_csr_read_binary(str(path).encode(), ctypes.byref(h)))
    return HostCsr._from_handle(h)


def write_binary(csr, path):
    csr.write_binary(path)


# ------------------------------------------------------ host preprocessing

def generate_sigbit(col_nnz, ffc=2):
    """GenerateSigBit in FFC mode (utils/matrix_utils.cu:65-128) -> (sigbit, L)."""
    col_nnz = np.ascontiguousarray(col_nnz, dtype=np.int32)
    sig = np.empty_like(col_nnz)
    length = ctypes.c_int()
    _host_call(_native.host().psx_generate_sigbit(col_nnz.size, col_nnz.ctypes.data, ffc,
                                                  sig.ctypes.data, ctypes.byref(length)))
    return sig, length.value


def workset_count(degree_sums, cu_count):
    """AnalyzeMatrix's S (utils/matrix_utils.cu:31-63) from the degree sums."""
    sums = np.zeros(32, dtype=np.uint64)
    sums[:len(degree_sums)] = degree_sums
    s = ctypes.c_int()
    _host_call(_native.host().psx_workset_count(
        sums.ctypes.data_as(_native.c_u64_p), int(cu_count), ctypes.byref(s)))
    return s.value


def dense_input(seed, n1, n2=0):
    """DenseInput (benchmarks/benchmark_utils.h:100-104): n1 then n2 values."""
    a = np.empty(int(n1), dtype=np.float32)
    b = np.empty(int(n2), dtype=np.float32)
    _host_call(_native.host().psx_dense_input(seed, a.size, a.ctypes.data if a.size else None,
                                              b.size, b.ctypes.data if b.size else None))
    return (a, b) if n2 else a


# ----------------------------------------------------------------- matrix

class PowerSparseMatrixGPU:
    """Owns the GPU worksets built from host CSR arrays (utils/matrix_utils.h:20-69).

    cu_count=0 partitions for the current device; a positive value reproduces
    the partition for a device with that many CUs/SMs. signature_order picks
    how groups are put in signature order ("auto", "bitmap_words" or
    "bit_lists"; both methods give the same order). csr_positions=True keeps
    each stored nonzero's CSR position (SDDMMToCSR, WorksetToCSR). task_order
    ("auto", "signature" or "row") picks the group order the operators run in
    (same results); `.task_order` and `.locality` report the choice and the
    scores compared. hub_block ("auto" or "off") keeps the dense hub block
    (rows of highest degree x most popular columns, in up to three tiers of
    row ranges) as dense matrices run on the matrix cores when the cost rule
    finds one, and hub_thresholds = [(min_degree, min_count), ...] (degrees
    decreasing) sets its tiers explicitly; `.hub_block` lists the tiers'
    (rows, columns), [] when none. With timings=True the stage
    times (ms) are kept in `.timings` (the task-order step counts into
    "gather").
    """

    TIMING_KEYS = ("upload", "analyze", "rank", "groups", "sigbit", "signature", "order",
                   "gather", "total")
    ORDER_METHODS = ("auto", "bitmap_words", "bit_lists")
    TASK_ORDERS = ("auto", "signature", "row")

    def __init__(self, row_num, col_num, nnz_num, row_ptr, col_ind, sp_data, cu_count=0,
                 timings=False, signature_order="auto", csr_positions=False,
                 task_order="auto", run_order=True, max_group_types=0,
                 spmm_partition="tuned", hub_block="auto", hub_thresholds=()):
        row_ptr = np.ascontiguousarray(row_ptr, dtype=np.int32)
        col_ind = np.ascontiguousarray(col_ind, dtype=np.int32)
        sp_data = np.ascontiguousarray(sp_data, dtype=np.float32)
        self._h = None
        t = (ctypes.c_double * 9)() if timings else None
        h = ctypes.c_void_p()
        if signature_order not in self.ORDER_METHODS:
            raise ValueError(f"signature_order must be one of {self.ORDER_METHODS}")
        if task_order not in self.TASK_ORDERS:
            raise ValueError(f"task_order must be one of {self.TASK_ORDERS}")
        if spmm_partition not in ("tuned", "parity"):
            raise ValueError("spmm_partition must be 'tuned' or 'parity'")
        if hub_block not in ("auto", "off"):
            raise ValueError("hub_block must be 'auto' or 'off'")
        if len(hub_thresholds) > 3:
            raise ValueError("at most 3 hub block tiers")
        degs = (ctypes.c_int * 3)(*[int(d) for d, _ in hub_thresholds])
        cnts = (ctypes.c_int * 3)(*[int(c) for _, c in hub_thresholds])
        opts = _native.BuildOptions(int(cu_count), self.ORDER_METHODS.index(signature_order),
                                    int(bool(csr_positions)), self.TASK_ORDERS.index(task_order),
                                    int(not run_order), int(max_group_types),
                                    int(spmm_partition == "parity"), int(hub_block == "off"),
                                    degs, cnts)
        _host_call(_native.host().psx_matrix_create_ex(
            int(row_num), int(col_num), int(nnz_num),
            row_ptr.ctypes.data if row_ptr.size else None,
            col_ind.ctypes.data if col_ind.size else None,
            sp_data.ctypes.data if sp_data.size else None, ctypes.byref(opts), t,
            ctypes.byref(h)))
        self._h = h.value
        method = ctypes.c_int()
        _host_call(_native.host().psx_matrix_signature_order(self._h, ctypes.byref(method)))
        self.signature_order = self.ORDER_METHODS[method.value]
        order, sig, row = ctypes.c_int(), ctypes.c_double(), ctypes.c_double()
        _host_call(_native.host().psx_matrix_task_order(self._h, ctypes.byref(order),
                                                        ctypes.byref(sig), ctypes.byref(row)))
        self.task_order = self.TASK_ORDERS[order.value]
        self.locality = {"signature": sig.value, "row": row.value}
        used = ctypes.c_int()
        _host_call(_native.host().psx_matrix_run_order(self._h, ctypes.byref(used)))
        self.run_order = bool(used.value)
        _host_call(_native.host().psx_matrix_spmm_worksets(self._h, ctypes.byref(used)))
        self.spmm_worksets = used.value  # workset count of the partition SpMM runs on
        tiers, hr, hc = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        self.hub_block = []
        _host_call(_native.host().psx_matrix_hub_block(self._h, ctypes.byref(tiers), 0, None, None))
        for k in range(tiers.value):
            _host_call(_native.host().psx_matrix_hub_block(self._h, None, k, ctypes.byref(hr),
                                                           ctypes.byref(hc)))
            self.hub_block.append((hr.value, hc.value))
        self.timings = dict(zip(self.TIMING_KEYS, list(t))) if timings else None
        rows, cols, nnz, S, fine, L, cu = (ctypes.c_int() for _ in range(7))
        _host_call(_native.host().psx_matrix_info(
            self._h, ctypes.byref(rows), ctypes.byref(cols), ctypes.byref(nnz), ctypes.byref(S),
            ctypes.byref(fine), ctypes.byref(L), ctypes.byref(cu)))
        self._rows, self._cols, self._nnz = rows.value, cols.value, nnz.value
        self._S, self._fine, self._L, self._cu = S.value, fine.value, L.value, cu.value
        g = (ctypes.c_int * self._S)()
        _host_call(_native.host().psx_matrix_group_num(self._h, g))
        self._group_num = list(g)

    @classmethod
    def from_csr(cls, csr, cu_count=0, timings=False, signature_order="auto",
                 csr_positions=False, task_order="auto", run_order=True, max_group_types=0,
                 spmm_partition="tuned", hub_block="auto", hub_thresholds=()):
        return cls(csr.rows, csr.cols, csr.nnz, csr.row_ptr, csr.col_ind, csr.values,
                   cu_count=cu_count, timings=timings, signature_order=signature_order,
                   csr_positions=csr_positions, task_order=task_order, run_order=run_order,
                   max_group_types=max_group_types, spmm_partition=spmm_partition,
                   hub_block=hub_block, hub_thresholds=hub_thresholds)

    def close(self):
        if self._h:
            _native.host().psx_matrix_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self):
        return self._h

    # accessors (utils/matrix_utils.h:30-40)
    def MatrixRow(self):
        return self._rows

    def MatrixCol(self):
        return self._cols

    def MatrixNNZ(self):
        return self._nnz

    def GroupTypeNum(self):
        return self._S

    def GroupFineSize(self):
        return self._fine

    def GroupNum(self):
        return list(self._group_num)

    def SignatureLen(self):
        return self._L

    def PartitionCuCount(self):
        return self._cu

    def _workset_ptrs(self, s):
        c, v, d = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
        _host_call(_native.host().psx_matrix_workset(self._h, s, ctypes.byref(c),
                                                     ctypes.byref(v), ctypes.byref(d)))
        return c.value or 0, v.value or 0, d.value or 0

    def WorksetColInd(self):
        return [self._workset_ptrs(s)[0] for s in range(self._S)]

    def WorksetSpData(self):
        return [self._workset_ptrs(s)[1] for s in range(self._S)]

    def GroupDestination(self):
        return [self._workset_ptrs(s)[2] for s in range(self._S)]

    def _residue_ptrs(self):
        o, a = ctypes.c_void_p(), ctypes.c_void_p()
        _host_call(_native.host().psx_matrix_residue(self._h, ctypes.byref(o), ctypes.byref(a)))
        return o.value or 0, a.value or 0

    def ResidueOffset(self):
        return self._residue_ptrs()[0]

    def ResidueAtomic(self):
        return self._residue_ptrs()[1]

    # host copies for checking
    def residue_offset(self):
        return download(self.ResidueOffset(), np.int32, self._group_num[0] + 1)

    def residue_atomic(self):
        return download(self.ResidueAtomic(), np.uint8, self._group_num[0])

    def workset_len(self, s):
        if s == 0:
            return int(self.residue_offset()[-1])
        return self._group_num[s] * GROUP_SIZE(s)

    def download_workset(self, s):
        """(col_ind, sp_data, group_des) of workset s as numpy arrays."""
        c, v, d = self._workset_ptrs(s)
        n = self.workset_len(s)
        return (download(c, np.int32, n), download(v, np.float32, n),
                download(d, np.int32, self._group_num[s]))

    def csr_position(self, s):
        """Device pointer of workset s's CSR positions (0 if not kept or empty)."""
        p = ctypes.c_void_p()
        _host_call(_native.host().psx_matrix_csr_position(self._h, s, ctypes.byref(p)))
        return p.value or 0

    def download_csr_position(self, s):
        """CSR position of every stored nonzero of workset s (numpy int32)."""
        ptr = self.csr_position(s)
        if not ptr:
            raise ValueError("matrix built without csr_positions, or empty workset")
        return download(ptr, np.int32, self.workset_len(s))

    def sddmm_output_sizes(self):
        """Floats per SDDMM output workset (benchmarks/benchmark.cu:147-155)."""
        return [self.workset_len(s) for s in range(self._S)]


def _streams(streams, count):
    if streams is None:
        return None
    arr = (ctypes.c_void_p * max(count, len(streams), 1))()
    for i, s in enumerate(streams):
        arr[i] = _ptr(s)
    return arr


def SpMM(matrix, N, B_gpu, C_gpu, ps_stream_num=None, ps_stream=None):
    """FP32 C = A * B (PowerSparse_SpMM.h:14-17). C must be zeroed by the caller."""
    if ps_stream_num is None:
        ps_stream_num = matrix.GroupTypeNum()
    _host_call(_native.host().psx_spmm(matrix.handle, int(N), _ptr(B_gpu), _ptr(C_gpu),
                                       int(ps_stream_num), _streams(ps_stream, ps_stream_num)))


def SpMMAsync(matrix, N, B_gpu, C_gpu, stream=None):
    """One launch on `stream`, no device synchronisation."""
    _host_call(_native.host().psx_spmm_async(matrix.handle, int(N), _ptr(B_gpu), _ptr(C_gpu),
                                             _ptr(stream)))


def _out_array(outputs, count):
    arr = (ctypes.c_void_p * max(count, 1))()
    for i, o in enumerate(outputs):
        arr[i] = _ptr(o)
    return arr


def SDDMM(matrix, N, lhs_gpu, rhs_gpu, sddmm_output_gpu, ps_stream_num=None, ps_stream=None):
    """FP32 sampled dense-dense product in workset order (PowerSparse_SDDMM.h:14-18)."""
    if ps_stream_num is None:
        ps_stream_num = matrix.GroupTypeNum()
    _host_call(_native.host().psx_sddmm(
        matrix.handle, int(N), _ptr(lhs_gpu), _ptr(rhs_gpu),
        _out_array(sddmm_output_gpu, matrix.GroupTypeNum()), int(ps_stream_num),
        _streams(ps_stream, ps_stream_num)))


def SDDMMAsync(matrix, N, lhs_gpu, rhs_gpu, sddmm_output_gpu, stream=None):
    _host_call(_native.host().psx_sddmm_async(
        matrix.handle, int(N), _ptr(lhs_gpu), _ptr(rhs_gpu),
        _out_array(sddmm_output_gpu, matrix.GroupTypeNum()), _ptr(stream)))


def SDDMMToCSR(matrix, N, lhs_gpu, rhs_gpu, out_csr_gpu, stream=None):
    """SDDMM with the output in the input CSR's order (MatrixNNZ floats, no
    zeroing needed). The matrix must be built with csr_positions=True."""
    _host_call(_native.host().psx_sddmm_csr(matrix.handle, int(N), _ptr(lhs_gpu), _ptr(rhs_gpu),
                                            _ptr(out_csr_gpu), _ptr(stream)))


def WorksetToCSR(matrix, values_gpu, out_csr_gpu, stream=None):
    """Workset-order per-nonzero values (one buffer per workset) into CSR order."""
    _host_call(_native.host().psx_workset_to_csr(
        matrix.handle, _out_array(values_gpu, matrix.GroupTypeNum()), _ptr(out_csr_gpu),
        _ptr(stream)))


# ------------------------------------------------ raw launchers (C ABI)

def _workset_array(worksets):
    arr = (Workset * max(len(worksets), 1))()
    for i, w in enumerate(worksets):
        col, val, des, groups, size = w[:5]
        order = w[5] if len(w) > 5 else None  # residue run order (optional)
        arr[i] = Workset(_ptr(col), _ptr(val), _ptr(des), int(groups), int(size), _ptr(order))
    return arr


def spmm_launch(worksets, residue_offset, residue_atomic, rows, cols, N, B, C, stream=None,
                task_chunk=1):
    """ps_spmm_launch over (col, val, des, group_num, group_size[, order]) tuples,
    s = 0..S-1."""
    _hip_call(_native.hip().ps_spmm_launch(len(worksets), _workset_array(worksets),
                                           _ptr(residue_offset), _ptr(residue_atomic), rows, cols,
                                           N, _ptr(B), _ptr(C), int(task_chunk), _ptr(stream)))


def sddmm_launch(worksets, residue_offset, rows, cols, N, lhs, rhs, outputs, stream=None,
                 task_chunk=1):
    """ps_sddmm_launch; outputs[s] is workset s's output buffer."""
    _hip_call(_native.hip().ps_sddmm_launch(len(worksets), _workset_array(worksets),
                                            _ptr(residue_offset), rows, cols, N, _ptr(lhs),
                                            _ptr(rhs), _out_array(outputs, len(worksets)),
                                            int(task_chunk), _ptr(stream)))
