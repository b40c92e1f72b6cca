"""The drop-in API end to end on the GPU: PowerSparseMatrixGPU (GPU
preprocessing) + SpMM / SDDMM with the reference's stream contract, against
the oracle; argument errors; and checks at the full benchmark sizes."""
import numpy as np
import pytest

import oracle
import powersparse_amd as ps
import tolerance
from gpu_util import say, setup

pytestmark = pytest.mark.gpu


def run_spmm(m, N, B, streams=None):
    dB = ps.DeviceBuffer(host=B)
    dC = ps.DeviceBuffer.zeros(m.MatrixRow() * N * 4)
    S = m.GroupTypeNum()
    if streams is None and S > 1:
        streams = [ps.Stream() for _ in range(S)]
    ps.SpMM(m, N, dB, dC, S, streams)
    ps.synchronize()
    return dC.download(np.float32).reshape(m.MatrixRow(), N)


@pytest.mark.parametrize("cfg,scale,N", [("C0", 1, 32), ("C1", 20, 32), ("C1", 20, 128),
                                         ("C4", 16, 64), ("C3", 40, 128)])
def test_spmm_end_to_end(cfg, scale, N):
    setup()
    csr = ps.synth(cfg, seed=11, scale=scale)
    m = ps.PowerSparseMatrixGPU.from_csr(csr)
    say(f"spmm {cfg}/{scale} N={N} S={m.GroupTypeNum()} groups={m.GroupNum()}")
    B = np.random.default_rng(1).uniform(-1, 1, (csr.cols, N)).astype(np.float32)
    C = run_spmm(m, N, B)
    E, M = oracle.spmm(csr.row_ptr, csr.col_ind, csr.values, N, B, with_mag=True)
    say("  ", tolerance.check(C, E, M, f"SpMM {cfg} N={N}"))


@pytest.mark.parametrize("cfg,scale,N", [("C0", 1, 32), ("C1", 20, 128), ("C4", 16, 64),
                                         ("C1", 20, 32)])
def test_sddmm_end_to_end(cfg, scale, N):
    setup()
    csr = ps.synth(cfg, seed=12, scale=scale)
    m = ps.PowerSparseMatrixGPU.from_csr(csr)
    S = m.GroupTypeNum()
    say(f"sddmm {cfg}/{scale} N={N} S={S} groups={m.GroupNum()}")
    rng = np.random.default_rng(2)
    X = rng.normal(size=(csr.rows, N)).astype(np.float32)
    Y = rng.normal(size=(csr.cols, N)).astype(np.float32)
    dX, dY = ps.DeviceBuffer(host=X), ps.DeviceBuffer(host=Y)
    sizes = m.sddmm_output_sizes()
    outs = [ps.DeviceBuffer.zeros(max(n, 1) * 4) for n in sizes]
    streams = [ps.Stream() for _ in range(S)] if S > 1 else None
    ps.SDDMM(m, N, dX, dY, outs, S, streams)
    ps.synchronize()
    offs0 = m.residue_offset()
    for s in range(S):
        if sizes[s] == 0:
            continue
        col, val, des = m.download_workset(s)
        offs = offs0 if s == 0 else np.arange(m.GroupNum()[s] + 1) * ps.GROUP_SIZE(s)
        E, Mg = oracle.sddmm(des, offs, col, val, N, X, Y, with_mag=True)
        tolerance.check(outs[s].download(np.float32, sizes[s]), E, Mg, f"SDDMM {cfg} ws {s}")


def test_api_argument_errors():
    setup()
    csr = ps.synth("C1", seed=13, scale=50)
    m = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=4)
    S = m.GroupTypeNum()
    assert S > 1
    B = ps.DeviceBuffer(csr.cols * 128 * 4)
    C = ps.DeviceBuffer(csr.rows * 128 * 4)
    streams = [ps.Stream() for _ in range(S)]
    with pytest.raises(ValueError, match="positive multiple of 32"):
        ps.SpMM(m, 48, B, C, S, streams)
    with pytest.raises(ValueError, match="positive multiple of 32"):
        ps.SpMM(m, 0, B, C, S, streams)
    with pytest.raises(ValueError, match="stream count"):
        ps.SpMM(m, 32, B, C, S - 1, streams)
    with pytest.raises(ValueError, match="stream count"):
        ps.SpMM(m, 32, B, C, S, None)
    with pytest.raises(ValueError, match="Invalid SpMM buffers"):
        ps.SpMM(m, 32, None, C, S, streams)
    with pytest.raises(ValueError, match="between 32 and 512"):
        ps.SDDMM(m, 544, B, B, [C] * S, S, streams)
    with pytest.raises(ValueError, match="Missing SDDMM output"):
        ps.SDDMM(m, 32, B, B, [None] * S, S, streams)
    with pytest.raises(ValueError, match="32-bit kernel indexing"):
        ps.SpMM(m, 32 * (2 ** 31 // (32 * csr.cols) + 1), B, C, S, streams)


def test_single_workset_async_default_stream():
    # S == 1: the reference launches on the default stream without syncing
    setup()
    csr = ps.synth("C0", seed=14)
    m = ps.PowerSparseMatrixGPU.from_csr(csr)
    assert m.GroupTypeNum() == 1
    B = np.random.default_rng(3).uniform(-1, 1, (csr.cols, 32)).astype(np.float32)
    C = run_spmm(m, 32, B, streams=None)
    E, M = oracle.spmm(csr.row_ptr, csr.col_ind, csr.values, 32, B, with_mag=True)
    tolerance.check(C, E, M, "SpMM C0 default stream")


def col_hash(col):
    """A 20-bit multiplicative hash of each column id, as float64: a row's sum
    of up to 2^33 of them stays an exact integer in float64 (< 2^53), so the
    per-row sums compare exactly whatever the summation order."""
    return ((col.astype(np.int64) * 2654435761) & 0xFFFFF).astype(np.float64)


def per_row_checks(csr, m):
    """Multiset of (row, col, value) preserved, via per-row counts and sums
    (column sums and column-hash sums are exact integers in float64)."""
    rows = csr.rows
    cnt = np.zeros(rows, np.int64)
    s_col = np.zeros(rows, np.float64)
    s_col2 = np.zeros(rows, np.float64)
    s_val = np.zeros(rows, np.float64)
    offs0 = m.residue_offset()
    for s in range(m.GroupTypeNum()):
        if m.GroupNum()[s] == 0:
            continue
        col, val, des = m.download_workset(s)
        offs = offs0 if s == 0 else np.arange(m.GroupNum()[s] + 1, dtype=np.int64) * ps.GROUP_SIZE(s)
        row_of = np.repeat(des, np.diff(offs))
        cnt += np.bincount(row_of, minlength=rows)
        s_col += np.bincount(row_of, weights=col.astype(np.float64), minlength=rows)
        s_col2 += np.bincount(row_of, weights=col_hash(col), minlength=rows)
        s_val += np.bincount(row_of, weights=val.astype(np.float64), minlength=rows)
        if s > 0:
            g = col.reshape(-1, ps.GROUP_SIZE(s))
            assert (np.diff(g, axis=1) >= 0).all()
    row_of = np.repeat(np.arange(rows), np.diff(csr.row_ptr))
    np.testing.assert_array_equal(cnt, np.diff(csr.row_ptr))
    np.testing.assert_array_equal(s_col, np.bincount(row_of, weights=csr.col_ind.astype(np.float64), minlength=rows))
    np.testing.assert_array_equal(s_col2, np.bincount(row_of, weights=col_hash(csr.col_ind), minlength=rows))
    np.testing.assert_allclose(s_val, np.bincount(row_of, weights=csr.values.astype(np.float64), minlength=rows), rtol=1e-12, atol=1e-9)


@pytest.mark.parametrize("cfg", ["C1", "C4", "C3"])
def test_full_size_properties(cfg):
    """At full benchmark size (the graphs bench.py builds): worksets preserve every row's entries; SpMM against
    an all-ones B gives each row's value sum, and SpMM is linear in B."""
    setup()
    csr = ps.synth(cfg, seed=1)
    say(f"full {cfg}: rows={csr.rows} nnz={csr.nnz}")
    m = ps.PowerSparseMatrixGPU.from_csr(csr, timings=True)
    say("  S", m.GroupTypeNum(), "groups", m.GroupNum(), "timings", m.timings)
    per_row_checks(csr, m)
    N = 32
    ones = np.ones((csr.cols, N), np.float32)
    C1 = run_spmm(m, N, ones)
    row_sum = np.add.reduceat(np.concatenate([csr.values.astype(np.float64), [0]]),
                              csr.row_ptr[:-1]) * (np.diff(csr.row_ptr) > 0)
    row_abs = np.add.reduceat(np.concatenate([np.abs(csr.values.astype(np.float64)), [0]]),
                              csr.row_ptr[:-1]) * (np.diff(csr.row_ptr) > 0)
    tolerance.check(C1, np.repeat(row_sum[:, None], N, 1), np.repeat(row_abs[:, None], N, 1),
                    f"{cfg} SpMM(ones)")
    rng = np.random.default_rng(4)
    B1 = rng.uniform(-1, 1, (csr.cols, N)).astype(np.float32)
    B2 = rng.uniform(-1, 1, (csr.cols, N)).astype(np.float32)
    Ca, Cb, Cab = run_spmm(m, N, B1), run_spmm(m, N, B2), run_spmm(m, N, B1 + B2)
    _, M1 = oracle.spmm(csr.row_ptr, csr.col_ind, csr.values, N, np.abs(B1) + np.abs(B2),
                        with_mag=True)
    tolerance.check(Cab, Ca.astype(np.float64) + Cb, M1, f"{cfg} SpMM linearity")


@pytest.mark.parametrize("cfg", ["C1", "C4", "C3"])
def test_full_size_sddmm_exact(cfg):
    """At full benchmark size, SDDMM with X[i, :] = (i % 5) / 8 and Y[j, :] = j % 7
    (K = 32): every dot is the exact integer 4 * (i % 5) * (j % 7), so every
    output is the float32 product value * dot exactly, whatever the summation
    order; this pins the row and column of every stored nonzero."""
    setup()
    csr = ps.synth(cfg, seed=1)
    m = ps.PowerSparseMatrixGPU.from_csr(csr)
    say(f"full {cfg} SDDMM exact: nnz={csr.nnz} S={m.GroupTypeNum()} task order {m.task_order}")
    N = 32
    X = np.repeat(((np.arange(csr.rows) % 5) / 8.0).astype(np.float32)[:, None], N, 1)
    Y = np.repeat((np.arange(csr.cols) % 7).astype(np.float32)[:, None], N, 1)
    dX, dY = ps.DeviceBuffer(host=X), ps.DeviceBuffer(host=Y)
    del X, Y
    sizes = m.sddmm_output_sizes()
    outs = [ps.DeviceBuffer.zeros(max(n, 1) * 4) for n in sizes]
    ps.SDDMMAsync(m, N, dX, dY, outs)
    ps.synchronize()
    G = m.GroupNum()
    for s in range(m.GroupTypeNum()):
        if G[s] == 0:
            continue
        col, val, des = m.download_workset(s)
        if s == 0:
            rows = np.repeat(des, np.diff(m.residue_offset()))
        else:
            rows = np.repeat(des, 32 << (s - 1))
        dot = (4 * (rows % 5) * (col % 7)).astype(np.float32)
        got = outs[s].download(np.float32, sizes[s])
        # exact equality of values (residue results are added to +0.0, so a
        # product -0.0 arrives as +0.0)
        np.testing.assert_array_equal(got, val * dot, err_msg=f"{cfg} workset {s}")


@pytest.mark.parametrize("cfg,ops", [("C1", [("spmm", 32), ("spmm", 128), ("sddmm", 128),
                                             ("sddmm", 32)]),
                                     ("C3", [("spmm", 32), ("spmm", 128), ("sddmm", 128)]),
                                     ("C4", [("spmm", 64), ("sddmm", 64)])])
def test_full_size_numerics(cfg, ops):
    """The bench's operators on the full-size benchmark graph against the
    oracle's double-precision results (tests/tolerance.py), with the bench's
    input distributions (C1: B ~ U(-1, 1), X and Y ~ N(0, 1); C3: all U(-1, 1);
    C4: all N(0, 1)). SDDMM is checked in CSR order and in workset order (each
    stored nonzero's CSR position maps it back; C4 runs its row-ordered
    execution copy). Prints per operator how many outputs pass only by the
    condition-aware bound (`only_cond`)."""
    from powersparse_amd.perf import host_operand
    setup()
    csr = ps.synth(cfg, seed=1)
    m = ps.PowerSparseMatrixGPU.from_csr(csr, csr_positions=True)
    say(f"full {cfg} numerics: nnz={csr.nnz} task order {m.task_order}")
    rng = np.random.default_rng(8)
    rows = np.arange(csr.rows, dtype=np.int32)
    for op, N in ops:
        if op == "spmm":
            B = host_operand(rng, (csr.cols, N), cfg, op)
            C = run_spmm(m, N, B)
            E, M = oracle.spmm(csr.row_ptr, csr.col_ind, csr.values, N, B, with_mag=True)
            say("  ", tolerance.check(C, E, M, f"{cfg} SpMM N={N}"))
        else:
            X = host_operand(rng, (csr.rows, N), cfg, op)
            Y = host_operand(rng, (csr.cols, N), cfg, op)
            dX, dY = ps.DeviceBuffer(host=X), ps.DeviceBuffer(host=Y)
            out = ps.DeviceBuffer(csr.nnz * 4)
            ps.SDDMMToCSR(m, N, dX, dY, out)
            ps.synchronize()
            E, M = oracle.sddmm(rows, csr.row_ptr, csr.col_ind, csr.values, N, X, Y,
                                with_mag=True)
            say("  ", tolerance.check(out.download(np.float32, csr.nnz), E, M,
                                      f"{cfg} SDDMM N={N} (CSR order)"))
            # the workset-order operator (the bench's call), mapped to CSR order
            sizes = m.sddmm_output_sizes()
            outs = [ps.DeviceBuffer.zeros(max(sz, 1) * 4) for sz in sizes]
            ps.SDDMMAsync(m, N, dX, dY, outs)
            ps.synchronize()
            ws = np.full(csr.nnz, np.nan, np.float32)
            for s, sz in enumerate(sizes):
                if sz:
                    ws[m.download_csr_position(s)] = outs[s].download(np.float32, sz)
            say("  ", tolerance.check(ws, E, M, f"{cfg} SDDMM N={N} (workset order)"))


def test_operands_over_4gib():
    # B / Y of cols x 512 floats = 4.3 GB: beyond 32-bit buffer offsets, so the
    # kernels take their 64-bit global-load path. Only three clusters of
    # columns (start, middle, end of the range) are used and uploaded.
    setup()
    from powersparse_amd import _native
    N = 512
    cols = (1 << 21) + 4096
    assert cols * N * 4 > (1 << 32) and cols * N <= 2**31 - 1
    rng = np.random.default_rng(9)
    starts = [0, 1 << 20, cols - 1024]
    pool = np.concatenate([np.arange(s0, s0 + 1024) for s0 in starts])
    rows = 500
    deg = rng.integers(0, 300, rows)
    deg[:40] = 64  # enough 64-nonzero blocks to make block worksets at cu_count 1
    ci = [np.sort(rng.choice(pool, d, replace=False)) for d in deg]
    rp = np.concatenate([[0], np.cumsum(deg)]).astype(np.int32)
    ci = np.concatenate(ci).astype(np.int32)
    csr = ps.HostCsr(rows, cols, rp, ci, rng.uniform(0, 1, ci.size).astype(np.float32))
    m = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=1, csr_positions=True)
    say(f"4 GiB operands: S={m.GroupTypeNum()} groups={m.GroupNum()} nnz={csr.nnz}")
    assert m.GroupTypeNum() >= 2
    compact = rng.uniform(-1, 1, (3 * 1024, N)).astype(np.float32)
    big = ps.DeviceBuffer(cols * N * 4)
    for k, s0 in enumerate(starts):
        block = np.ascontiguousarray(compact[k * 1024:(k + 1) * 1024])
        ps._hip_call(_native.hip().ps_memcpy_htod(big.ptr + s0 * N * 4, block.ctypes.data,
                                                   block.nbytes))
    remap = np.empty(cols, np.int32)
    for k, s0 in enumerate(starts):
        remap[s0:s0 + 1024] = np.arange(k * 1024, (k + 1) * 1024)
    cc = remap[csr.col_ind]
    C = ps.DeviceBuffer.zeros(rows * N * 4)
    ps.SpMMAsync(m, N, big, C)
    ps.synchronize()
    E, M = oracle.spmm(csr.row_ptr, cc, csr.values, N, compact, with_mag=True)
    say("  ", tolerance.check(C.download(np.float32).reshape(rows, N), E, M, "SpMM > 4 GiB"))
    X = rng.normal(size=(rows, N)).astype(np.float32)
    out = ps.DeviceBuffer(csr.nnz * 4)
    dX = ps.DeviceBuffer(host=X)  # alive until the sync
    ps.SDDMMToCSR(m, N, dX, big, out)
    ps.synchronize()
    E, M = oracle.sddmm(np.arange(rows, dtype=np.int32), csr.row_ptr, cc, csr.values, N, X,
                        compact, with_mag=True)
    say("  ", tolerance.check(out.download(np.float32, csr.nnz), E, M, "SDDMM > 4 GiB"))


def test_misaligned_buffers_rejected():
    # the kernels use 128-bit accesses: the raw launchers refuse buffers that
    # are not 16-byte aligned instead of running on them
    setup()
    csr = ps.synth("C1", seed=13, scale=50)
    m = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=4)
    S = m.GroupTypeNum()
    assert S > 1
    cps, vps, dps = m.WorksetColInd(), m.WorksetSpData(), m.GroupDestination()
    G = m.GroupNum()
    ws = [(cps[s], vps[s], dps[s], G[s], 0 if s == 0 else ps.GROUP_SIZE(s)) for s in range(S)]
    N = 32
    B = ps.DeviceBuffer(csr.cols * N * 4 + 16)
    C = ps.DeviceBuffer(csr.rows * N * 4 + 16)
    with pytest.raises(ValueError, match="16-byte aligned"):
        ps.spmm_launch(ws, m.ResidueOffset(), m.ResidueAtomic(), csr.rows, csr.cols, N,
                       B.ptr + 4, C.ptr)
    with pytest.raises(ValueError, match="16-byte aligned"):
        ps.spmm_launch(ws, m.ResidueOffset(), m.ResidueAtomic(), csr.rows, csr.cols, N, B.ptr,
                       C.ptr + 8)
    bad = list(ws)
    bad[S - 1] = (cps[S - 1] + 4,) + tuple(ws[S - 1][1:])
    with pytest.raises(ValueError, match="16-byte aligned"):
        ps.spmm_launch(bad, m.ResidueOffset(), m.ResidueAtomic(), csr.rows, csr.cols, N, B.ptr,
                       C.ptr)
    X = ps.DeviceBuffer(csr.rows * N * 4 + 16)
    outs = [ps.DeviceBuffer(max(n, 1) * 4) for n in m.sddmm_output_sizes()]
    with pytest.raises(ValueError, match="16-byte aligned"):
        ps.sddmm_launch(ws, m.ResidueOffset(), csr.rows, csr.cols, N, X.ptr + 4, B.ptr, outs)
    with pytest.raises(ValueError, match="16-byte aligned"):
        ps.sddmm_launch(bad, m.ResidueOffset(), csr.rows, csr.cols, N, X.ptr, B.ptr, outs)
    # the same call with aligned buffers runs
    ps.spmm_launch(ws, m.ResidueOffset(), m.ResidueAtomic(), csr.rows, csr.cols, N, B.ptr,
                   C.ptr)
    ps.synchronize()


def test_operators_on_concurrent_streams():
    """SpMM and SDDMM of two matrices enqueued on two streams at once (the
    kernels keep no state between calls) give the results of the same calls
    made one at a time: SDDMM bitwise, SpMM within FP32 atomic reordering."""
    setup()
    a = ps.synth("C1", seed=5, scale=20)
    b = ps.synth("C4", seed=6, scale=16)
    ma = ps.PowerSparseMatrixGPU.from_csr(a)
    mb = ps.PowerSparseMatrixGPU.from_csr(b)
    say(f"concurrent streams: nnz {a.nnz} / {b.nnz}, task orders {ma.task_order} / {mb.task_order}")
    rng = np.random.default_rng(12)
    N = 64
    B = ps.DeviceBuffer(host=rng.uniform(-1, 1, (a.cols, N)).astype(np.float32))
    X = ps.DeviceBuffer(host=rng.standard_normal((b.rows, N), dtype=np.float32))
    Y = ps.DeviceBuffer(host=rng.standard_normal((b.cols, N), dtype=np.float32))
    sizes = mb.sddmm_output_sizes()

    def run(sa, sb):
        C = ps.DeviceBuffer.zeros(a.rows * N * 4)
        outs = [ps.DeviceBuffer.zeros(max(sz, 1) * 4) for sz in sizes]
        ps.synchronize()  # the zero fills first
        for _ in range(3):  # accumulate: C and the residue outputs add up over calls
            ps.SpMMAsync(ma, N, B, C, sa)
            ps.SDDMMAsync(mb, N, X, Y, outs, sb)
        ps.synchronize()
        return (C.download(np.float32),
                [o.download(np.float32, sz) if sz else None for o, sz in zip(outs, sizes)])

    s1, s2 = ps.Stream(), ps.Stream()
    c_cc, o_cc = run(s1, s2)
    c_seq, o_seq = run(s1, s1)
    # the two runs differ only in the order of FP32 atomic additions into C
    # (three calls accumulated): a few units of 2^-24 of the summed magnitudes
    np.testing.assert_allclose(c_cc, c_seq, rtol=1e-4, atol=1e-6 * np.abs(c_seq).max())
    for s, (x, y) in enumerate(zip(o_cc, o_seq)):
        if x is not None:
            np.testing.assert_array_equal(x.view(np.uint32), y.view(np.uint32),
                                          err_msg=f"SDDMM workset {s}")
