"""Task order: the operators on the row-ordered execution copy give the same
results as on the public worksets (SDDMM bitwise, SpMM within the FP32
tolerance, since only the order of atomic additions changes), the automatic
choice, and the locality score itself."""
import ctypes

import numpy as np
import pytest

import oracle
import powersparse_amd as ps
import tolerance
from gpu_util import random_graph, say, setup
from powersparse_amd import _native

pytestmark = pytest.mark.gpu


def sddmm_public(m, N, dX, dY, calls=1):
    outs = [ps.DeviceBuffer.zeros(max(n, 1) * 4) for n in m.sddmm_output_sizes()]
    for _ in range(calls):  # outputs not cleared between calls, as the reference harness
        ps.SDDMMAsync(m, N, dX, dY, outs)
    ps.synchronize()
    return [o.download(np.float32, n) for o, n in zip(outs, m.sddmm_output_sizes())]


@pytest.mark.parametrize("cfg,scale,cu,N", [("C0", 1, 256, 32), ("C1", 20, 8, 64),
                                            ("C4", 16, 256, 64), ("C3", 60, 2, 128),
                                            ("C4", 64, 256, 96), ("C4", 64, 256, 256)])
def test_row_order_matches_signature_order(cfg, scale, cu, N):
    setup()
    csr = ps.synth(cfg, seed=31, scale=scale)
    # without a dense hub block: its outputs come from a GEMM, whose summation
    # order differs from the sparse kernels' (test_gpu_hub.py covers it)
    a = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=cu, task_order="signature",
                                         csr_positions=True, hub_block="off")
    b = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=cu, task_order="row",
                                         csr_positions=True)
    assert a.task_order == "signature" and b.task_order == "row"
    say(f"task order {cfg}/{scale} cu={cu} N={N} S={a.GroupTypeNum()}")
    # the public worksets do not depend on the task order
    for s in range(a.GroupTypeNum()):
        if a.GroupNum()[s]:
            for x, y in zip(a.download_workset(s), b.download_workset(s)):
                np.testing.assert_array_equal(x.view(np.uint32), y.view(np.uint32))
    rng = np.random.default_rng(5)
    B = rng.uniform(-1, 1, (csr.cols, N)).astype(np.float32)
    dB = ps.DeviceBuffer(host=B)
    E, M = oracle.spmm(csr.row_ptr, csr.col_ind, csr.values, N, B, with_mag=True)
    for m in (a, b):
        C = ps.DeviceBuffer.zeros(csr.rows * N * 4)
        ps.SpMMAsync(m, N, dB, C)
        ps.synchronize()
        tolerance.check(C.download(np.float32).reshape(csr.rows, N), E, M,
                        f"SpMM {m.task_order}")
    X = rng.normal(size=(csr.rows, N)).astype(np.float32)
    Y = rng.normal(size=(csr.cols, N)).astype(np.float32)
    dX, dY = ps.DeviceBuffer(host=X), ps.DeviceBuffer(host=Y)
    for x, y in zip(sddmm_public(a, N, dX, dY, 2), sddmm_public(b, N, dX, dY, 2)):
        np.testing.assert_array_equal(x.view(np.uint32), y.view(np.uint32))
    got = []
    for m in (a, b):
        out = ps.DeviceBuffer(host=np.full(csr.nnz, np.nan, np.float32))
        ps.SDDMMToCSR(m, N, dX, dY, out)
        ps.synchronize()
        got.append(out.download(np.float32, csr.nnz))
    np.testing.assert_array_equal(got[0].view(np.uint32), got[1].view(np.uint32))
    rows = np.arange(csr.rows, dtype=np.int32)
    E, M = oracle.sddmm(rows, csr.row_ptr, csr.col_ind, csr.values, N, X, Y, with_mag=True)
    tolerance.check(got[1], E, M, "SDDMMToCSR row order")


@pytest.mark.parametrize("seed", range(3))
def test_row_order_random(seed):
    setup()
    rng = np.random.default_rng(70 + seed)
    csr = random_graph(rng, int(rng.integers(100, 500)), int(rng.integers(50, 3000)), 120,
                       hubs=3, hub_deg=int(rng.integers(300, 2500)), dup=(seed == 2))
    cu = int(rng.choice([1, 2, 64]))
    a = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=cu, task_order="signature",
                                         hub_block="off")
    b = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=cu, task_order="row")
    N = 32
    X = rng.normal(size=(csr.rows, N)).astype(np.float32)
    Y = rng.normal(size=(csr.cols, N)).astype(np.float32)
    dX, dY = ps.DeviceBuffer(host=X), ps.DeviceBuffer(host=Y)
    for x, y in zip(sddmm_public(a, N, dX, dY), sddmm_public(b, N, dX, dY)):
        np.testing.assert_array_equal(x.view(np.uint32), y.view(np.uint32))
    B = rng.uniform(-1, 1, (csr.cols, N)).astype(np.float32)
    E, M = oracle.spmm(csr.row_ptr, csr.col_ind, csr.values, N, B, with_mag=True)
    C = ps.DeviceBuffer.zeros(csr.rows * N * 4)
    dB = ps.DeviceBuffer(host=B)  # alive until the sync
    ps.SpMMAsync(b, N, dB, C)
    ps.synchronize()
    tolerance.check(C.download(np.float32).reshape(csr.rows, N), E, M, "SpMM row order")


def test_auto_choice_full_size():
    # community rows are id ranges: C4 runs in row order; C1's hubs favour the
    # signature order
    setup()
    for cfg, expect in (("C4", "row"), ("C1", "signature")):
        csr = ps.synth(cfg, seed=1)
        m = ps.PowerSparseMatrixGPU.from_csr(csr)
        say(f"{cfg}: task order {m.task_order}, scores {m.locality}")
        assert m.task_order == expect
        assert 0 < m.locality["signature"] <= 1 and 0 < m.locality["row"] <= 1
        m.close()


def locality(arrays, window, max_windows=64):
    bufs = [ps.DeviceBuffer(host=np.asarray(a, np.int32)) for a in arrays]
    ptrs = (ctypes.c_void_p * len(arrays))(*[b.ptr for b in bufs])
    lens = (ctypes.c_longlong * len(arrays))(*[len(a) for a in arrays])
    score = ctypes.c_double()
    ps._hip_call(_native.hip().ps_pre_locality_score(len(arrays), ptrs, lens, window,
                                                     max_windows, ctypes.byref(score), None))
    return score.value


def test_locality_score_exact():
    setup()
    W = 1024
    w0 = np.full(W, 7)                      # 1 distinct
    w1 = np.arange(W) + 5000                # W distinct
    w2 = np.repeat(np.arange(W // 2), 2)    # W/2 distinct
    w3 = np.arange(W) % 3 + 10**6           # 3 distinct
    seq = np.concatenate([w0, w1, w2, w3, np.arange(100)])  # a partial tail window is ignored
    split = W + 300                         # the sequence spans two arrays mid-window
    got = locality([seq[:split], seq[split:]], W)
    assert got == pytest.approx((1 + W + W // 2 + 3) / (4 * W), rel=0, abs=1e-12)
    assert locality([seq[:W - 1]], W) == 0.0  # shorter than one window
    # sampling: every other window of 8 when 4 may be sampled
    eight = np.concatenate([w0, w1] * 4)
    assert locality([eight], W, max_windows=4) == pytest.approx(1 / W)
