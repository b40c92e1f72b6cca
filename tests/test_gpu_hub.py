"""The dense hub block (PartitionPolicy::hub_block) on the GPU.

A matrix built with a hub block runs the block's rows x hot columns as dense
products and the rest on the sparse paths; the results must equal those of
the same matrix without the block. On the golden fixtures' exact inputs
(sparse values k/64, dense values k/16: every FP32 partial sum exact) the
comparison is bit for bit, for SpMM over repeated calls (the block's rows
accumulate), SDDMM in workset and CSR order (also with a block that splits
block groups between the dense and the sparse path), SpMM with Inf / NaN in
B, and explicit tiers that would leave the sparse path nothing (no block is
kept). Scaled power-law graphs are checked against the oracle within the
FP32 tolerance, and the block's C entry points on a hand-built block."""
import numpy as np
import pytest

import golden_data as gd
import oracle
import powersparse_amd as ps
import tolerance
from gpu_util import say, setup

pytestmark = pytest.mark.gpu


def csr_of(g):
    return ps.HostCsr(g.rows, g.cols, g.row_ptr, g.col_ind, g.values)


def thresholds(csr, cu, tiers=1,
               shares=((0.25, 0.5), (0.25, 0.3), (0.1, 0.3), (0.1, 0.15))):
    """Explicit block tiers [(min_degree, min_count), ...]: tier k takes the
    next share of the rows with 64+ nonzeros (heaviest first) and the columns
    whose count reaches a share of those rows' entries; the first shares for
    which the matrix without the block still has more than one workset at
    `cu` CUs (the build drops the block otherwise)."""
    deg = np.diff(csr.row_ptr.astype(np.int64))
    heavy = np.sort(deg[deg >= 64])[::-1]
    assert heavy.size, "no heavy rows"
    cnt = np.bincount(csr.col_ind, minlength=csr.cols)
    rowof = np.repeat(np.arange(csr.rows), deg)
    cu = cu or 256
    for hub_share, hot_share in shares:
        out, block, hi = [], np.zeros(csr.nnz, bool), np.inf
        for k in range(tiers):
            d = int(heavy[max(0, int(heavy.size * hub_share * (k + 1)) - 1)])
            if d >= hi:
                break
            rows_k = (deg[rowof] >= d) & (deg[rowof] < hi)
            c = max(int(np.sort(cnt[csr.col_ind[rows_k]])[int(rows_k.sum() * (1 - hot_share))]), 1)
            block |= rows_k & (cnt[csr.col_ind] >= c)
            out.append((d, c))
            hi = d
        if len(out) < tiers:
            continue
        rest = np.bincount(rowof[~block], minlength=csr.rows)
        rp = np.concatenate([[0], np.cumsum(rest)]).astype(np.int32)
        if rp[-1] > 0 and oracle.analyze_group_type_num(rp, cu) >= 2:
            return out
    raise AssertionError("no block keeps two worksets in the rest")


def run_ops(m, g, N, B, X, Y, calls=1):
    S = m.GroupTypeNum()
    streams = [ps.Stream() for _ in range(S)] if S > 1 else None
    dB = ps.DeviceBuffer(host=B)
    dC = ps.DeviceBuffer.zeros(g.rows * N * 4)
    for _ in range(calls):
        ps.SpMM(m, N, dB, dC, S, streams)
    ps.synchronize()
    C = dC.download(np.float32).reshape(g.rows, N)
    dX, dY = ps.DeviceBuffer(host=X), ps.DeviceBuffer(host=Y)
    sizes = m.sddmm_output_sizes()
    outs = [ps.DeviceBuffer.zeros(max(n, 1) * 4) for n in sizes]
    ps.SDDMM(m, N, dX, dY, outs, S, streams)
    ps.synchronize()
    W = [outs[s].download(np.float32, sizes[s]) for s in range(S)]
    csr_out = ps.DeviceBuffer(max(g.nnz, 1) * 4)
    ps.SDDMMToCSR(m, N, dX, dY, csr_out)
    ps.synchronize()
    return C, W, csr_out.download(np.float32, g.nnz)


@pytest.mark.parametrize("name,tiers", [("hubs", 1), ("skewed", 1), ("duplicates", 1),
                                        ("skewed", 2), ("duplicates", 2)])
def test_hub_block_exact_on_golden(name, tiers):
    setup()
    g = gd.load(name)
    p = g.parts[0]
    csr = csr_of(g)
    th = thresholds(csr, p.cu, tiers)
    kw = dict(cu_count=p.cu, csr_positions=True)
    on = ps.PowerSparseMatrixGPU.from_csr(csr, hub_thresholds=th, **kw)
    off = ps.PowerSparseMatrixGPU.from_csr(csr, hub_block="off", **kw)
    say(f"golden {name}: hub block {on.hub_block} (tiers {th}), S={on.GroupTypeNum()}, "
        f"SpMM worksets {on.spmm_worksets}")
    assert len(on.hub_block) == tiers and all(r > 0 and c > 0 for r, c in on.hub_block), \
        "the block was not built"
    assert off.hub_block == []
    # the public worksets are the reference's either way
    assert on.GroupNum() == off.GroupNum() == p.group_num
    for N in (32, 64, 128, 256):
        B, X, Y = (gd.dense(g.cols, N, gd.SALT_B), gd.dense(g.rows, N, gd.SALT_X),
                   gd.dense(g.cols, N, gd.SALT_Y))
        for calls in (1, 2):
            a = run_ops(on, g, N, B, X, Y, calls)
            b = run_ops(off, g, N, B, X, Y, calls)
            np.testing.assert_array_equal(a[0], b[0], err_msg=f"SpMM N={N} calls={calls}")
            for s in range(on.GroupTypeNum()):
                np.testing.assert_array_equal(a[1][s], b[1][s], err_msg=f"SDDMM N={N} ws {s}")
            np.testing.assert_array_equal(a[2], b[2], err_msg=f"SDDMMToCSR N={N}")
        if N == g.n:
            np.testing.assert_array_equal(a[2], g.sddmm_csr)
    on.close()
    off.close()


def test_hub_sddmm_tile_past_the_pipeline_capacity():
    """SDDMM's dense kernel writes a tile's first 8192 entries (64 x 128, the
    most a tile holds without repeated nonzeros) while it computes the next
    tile, and any further entries afterwards from direct dot products. 64 hub
    rows storing each of 256 hot columns three times (768 nonzeros each) put
    24576 entries into each of two tiles; on exact inputs (values k/64, operands k/16)
    the outputs in workset and CSR order equal the block-off build's bit for
    bit, at widths that run the resident and the streamed kernels."""
    setup()
    rng = np.random.default_rng(31)
    rows, cols, hub, hot = 4096, 8192, 64, 256
    lists = []
    for r in range(rows):
        if r < hub:
            c = np.repeat(np.arange(hot), 3)
        else:
            c = np.sort(rng.choice(np.arange(hot, cols), 8 if r % 2 else 160, replace=False))
        lists.append(c.astype(np.int32))
    rp = np.concatenate([[0], np.cumsum([len(c) for c in lists])]).astype(np.int32)
    ci = np.concatenate(lists)
    sv = (rng.integers(1, 64, ci.size) / 64).astype(np.float32)
    csr = ps.HostCsr(rows, cols, rp, ci, sv)
    kw = dict(cu_count=8, csr_positions=True)
    on = ps.PowerSparseMatrixGPU.from_csr(csr, hub_thresholds=[(768, 100)], **kw)
    off = ps.PowerSparseMatrixGPU.from_csr(csr, hub_block="off", **kw)
    say(f"capacity: hub block {on.hub_block}, S={on.GroupTypeNum()}")
    assert on.hub_block == [(hub, hot)], "the block was not built"

    class G:
        pass
    g = G()
    g.rows, g.cols, g.nnz = rows, cols, int(ci.size)
    for N in (32, 64, 96, 128, 160, 512):
        B, X, Y = (gd.dense(cols, N, gd.SALT_B), gd.dense(rows, N, gd.SALT_X),
                   gd.dense(cols, N, gd.SALT_Y))
        a = run_ops(on, g, N, B, X, Y)
        b = run_ops(off, g, N, B, X, Y)
        for s in range(on.GroupTypeNum()):
            np.testing.assert_array_equal(a[1][s], b[1][s], err_msg=f"SDDMM N={N} ws {s}")
        np.testing.assert_array_equal(a[2], b[2], err_msg=f"SDDMMToCSR N={N}")
        np.testing.assert_array_equal(a[0], b[0], err_msg=f"SpMM N={N}")
    on.close()
    off.close()


def tiles_inside(g, p, th):
    """(tiles inside the block, whole groups inside, groups split) of the
    block workset tiles (64 consecutive nonzeros of a group of 64+) for the
    explicit tiers th, computed on the host."""
    deg = np.diff(g.row_ptr.astype(np.int64))
    cnt = np.bincount(g.col_ind, minlength=g.cols)
    inside = whole = split = 0
    for s in range(1, p.S):
        gs = 32 << (s - 1)
        if gs < 64:
            continue
        for grp in range(p.group_num[s]):
            r, hi, ok = p.des[s][grp], np.inf, None
            for d, c in th:
                if d <= deg[r] < hi:
                    ok = cnt[p.col[s][grp * gs:(grp + 1) * gs]] >= c
                    break
                hi = d
            if ok is None:
                continue
            t = ok.reshape(-1, 64).all(1)
            inside += int(t.sum())
            whole += int(t.all())
            split += int(t.any() and not t.all())
    return inside, whole, split


def test_hub_block_splits_groups_exactly():
    """SDDMM takes the tiles of a block group that lie inside the block and
    leaves the group's other tiles to the sparse kernel: on the hubs fixture
    with a block that splits groups, every output equals the sparse path's
    bit for bit (workset and CSR order, SpMM alongside)."""
    setup()
    g = gd.load("hubs")
    p = g.parts[0]
    th = [(1046, 6)]
    inside, whole, split = tiles_inside(g, p, th)
    say(f"hubs with tier {th}: {inside} tiles inside, {whole} whole groups, {split} split")
    assert split >= 1 and whole >= 1
    csr = csr_of(g)
    kw = dict(cu_count=p.cu, csr_positions=True)
    on = ps.PowerSparseMatrixGPU.from_csr(csr, hub_thresholds=th, **kw)
    off = ps.PowerSparseMatrixGPU.from_csr(csr, hub_block="off", **kw)
    assert len(on.hub_block) == 1
    for N in (32, 64, 128, 256):
        B, X, Y = (gd.dense(g.cols, N, gd.SALT_B), gd.dense(g.rows, N, gd.SALT_X),
                   gd.dense(g.cols, N, gd.SALT_Y))
        a = run_ops(on, g, N, B, X, Y)
        b = run_ops(off, g, N, B, X, Y)
        np.testing.assert_array_equal(a[0], b[0], err_msg=f"SpMM N={N}")
        for s in range(on.GroupTypeNum()):
            np.testing.assert_array_equal(a[1][s], b[1][s], err_msg=f"SDDMM N={N} ws {s}")
        np.testing.assert_array_equal(a[2], b[2], err_msg=f"SDDMMToCSR N={N}")
        if N == g.n:
            np.testing.assert_array_equal(a[2], g.sddmm_csr)
    on.close()
    off.close()


def test_hub_block_nonfinite_b():
    """Inf and NaN in B rows of hot and cold columns reach exactly the rows
    that store those columns, as without the block (0 * Inf never leaks into
    rows that do not store the column)."""
    setup()
    g = gd.load("hubs")
    csr = csr_of(g)
    th = thresholds(csr, 1)
    min_count = th[0][1]
    on = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=1, hub_thresholds=th, csr_positions=True)
    off = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=1, hub_block="off", csr_positions=True)
    assert on.hub_block
    cnt = np.bincount(csr.col_ind, minlength=csr.cols)
    hot = np.flatnonzero(cnt >= min_count)
    cold = np.flatnonzero((cnt > 0) & (cnt < min_count))
    N = 64
    for pattern in range(3):
        B = gd.dense(g.cols, N, gd.SALT_B).copy()
        rng = np.random.default_rng(pattern)
        for c in rng.choice(hot, 3, replace=False):
            B[c, rng.integers(0, N, 4)] = [np.inf, -np.inf, np.nan, np.inf][: 4]
        for c in rng.choice(cold, 2, replace=False):
            B[c, rng.integers(0, N)] = np.inf
        X = gd.dense(g.rows, N, gd.SALT_X)
        Y = gd.dense(g.cols, N, gd.SALT_Y)
        a = run_ops(on, g, N, B, X, Y)
        b = run_ops(off, g, N, B, X, Y)
        assert np.isnan(a[0]).any() and np.isinf(a[0]).any()
        np.testing.assert_array_equal(np.isnan(a[0]), np.isnan(b[0]))
        np.testing.assert_array_equal(a[0], b[0])
    on.close()
    off.close()


def test_hub_block_repeated_slots_keep_per_entry_products():
    """A (hub row, hot column) slot stored twice stays out of the block: SpMM
    adds a1 * b + a2 * b as the reference does, not (a1 + a2) * b. With a1 =
    a2 = 3e38 and b = 1e-10 the sum of the values overflows to Inf while the
    per-entry products stay finite; with non-exact values (0.1, 0.7) the rows
    match the oracle within the FP32 tolerance, and a second build of the same
    matrix gives the same rows (up to the order of the sparse kernels' atomic
    additions)."""
    setup()
    g = gd.load("hubs")
    th = thresholds(csr_of(g), 1)
    d_min, c_min = th[0]
    deg = np.diff(g.row_ptr.astype(np.int64))
    cnt = np.bincount(g.col_ind, minlength=g.cols)
    hub_rows = np.flatnonzero(deg >= d_min)
    hot = np.flatnonzero(cnt >= c_min)
    rows = [list(g.col_ind[g.row_ptr[r]:g.row_ptr[r + 1]]) for r in range(g.rows)]
    vals = [list(g.values[g.row_ptr[r]:g.row_ptr[r + 1]]) for r in range(g.rows)]
    r1, r2 = int(hub_rows[0]), int(hub_rows[-1])
    c1 = int(next(c for c in hot if c not in rows[r1]))
    c2 = int(next(c for c in hot if c not in rows[r2] and c != c1))
    rows[r1] += [c1, c1]
    vals[r1] += [3e38, 3e38]
    rows[r2] += [c2, c2]
    vals[r2] += [0.1, 0.7]
    rp = np.concatenate([[0], np.cumsum([len(x) for x in rows])]).astype(np.int32)
    ci = np.concatenate([np.asarray(x, np.int32) for x in rows])
    sv = np.concatenate([np.asarray(x, np.float32) for x in vals])
    csr = ps.HostCsr(g.rows, g.cols, rp, ci, sv)
    N = 64
    rng = np.random.default_rng(9)
    B = rng.uniform(-1, 1, (g.cols, N)).astype(np.float32)
    B[c1, :] = 1e-10
    results = []
    for build in range(2):
        m = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=1, hub_thresholds=[(d_min, c_min)])
        assert m.hub_block, "the block was not built"
        dB, dC = ps.DeviceBuffer(host=B), ps.DeviceBuffer.zeros(g.rows * N * 4)
        S = m.GroupTypeNum()
        ps.SpMM(m, N, dB, dC, S, [ps.Stream() for _ in range(S)] if S > 1 else None)
        ps.synchronize()
        results.append(dC.download(np.float32).reshape(g.rows, N))
        m.close()
    C = results[0]
    assert np.isfinite(C).all(), "a repeated slot's values were summed before the product"
    E, M = oracle.spmm(rp, ci, sv, N, B, with_mag=True)
    say("  ", tolerance.check(C, E, M, "SpMM with repeated block slots"))
    # the sparse kernels' atomics add in no fixed order; rows r1 and r2 hold
    # the repeated slots, compare them and the overflow row exactly across builds
    np.testing.assert_array_equal(np.isfinite(results[1]), np.isfinite(C))
    np.testing.assert_allclose(results[1][[r1, r2]], C[[r1, r2]], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("cfg,scale", [("C3", 40), ("C1", 20)])
def test_hub_block_on_power_law_graphs(cfg, scale):
    """Scaled power-law graphs with an explicit block against the oracle's
    double-precision results (stated FP32 tolerance)."""
    setup()
    csr = ps.synth(cfg, seed=3, scale=scale)
    th = thresholds(csr, 0, tiers=2, shares=((0.25, 0.5), (0.1, 0.3)))
    m = ps.PowerSparseMatrixGPU.from_csr(csr, hub_thresholds=th)
    say(f"{cfg}/{scale}: nnz={csr.nnz} hub block {m.hub_block} (tiers {th}) S={m.GroupTypeNum()}")
    assert len(m.hub_block) == 2
    rng = np.random.default_rng(5)
    for N in (32, 128):
        B = rng.uniform(-1, 1, (csr.cols, N)).astype(np.float32)
        dB = ps.DeviceBuffer(host=B)
        dC = ps.DeviceBuffer.zeros(csr.rows * N * 4)
        S = m.GroupTypeNum()
        ps.SpMM(m, N, dB, dC, S, [ps.Stream() for _ in range(S)] if S > 1 else None)
        ps.synchronize()
        E, M = oracle.spmm(csr.row_ptr, csr.col_ind, csr.values, N, B, with_mag=True)
        say("  ", tolerance.check(dC.download(np.float32).reshape(csr.rows, N), E, M,
                                  f"SpMM {cfg} N={N}"))
    N = 128
    X = rng.normal(size=(csr.rows, N)).astype(np.float32)
    Y = rng.normal(size=(csr.cols, N)).astype(np.float32)
    dX, dY = ps.DeviceBuffer(host=X), ps.DeviceBuffer(host=Y)
    sizes = m.sddmm_output_sizes()
    outs = [ps.DeviceBuffer.zeros(max(n, 1) * 4) for n in sizes]
    ps.SDDMMAsync(m, N, dX, dY, outs)
    ps.synchronize()
    offs0 = m.residue_offset()
    for s in range(m.GroupTypeNum()):
        if sizes[s] == 0:
            continue
        col, val, des = m.download_workset(s)
        offs = offs0 if s == 0 else np.arange(m.GroupNum()[s] + 1) * ps.GROUP_SIZE(s)
        E, Mg = oracle.sddmm(des, offs, col, val, N, X, Y, with_mag=True)
        tolerance.check(outs[s].download(np.float32, sizes[s]), E, Mg, f"SDDMM {cfg} ws {s}")
    m.close()


def test_hub_block_concurrent_calls_and_memory():
    """Calls on one matrix from two streams share its workspace in turn and
    give the sequential results; constructions and their operator workspaces
    are released."""
    setup()
    g = gd.load("hubs")
    csr = csr_of(g)
    kw = dict(cu_count=1, hub_thresholds=thresholds(csr, 1))
    m = ps.PowerSparseMatrixGPU.from_csr(csr, **kw)
    assert m.hub_block
    N = 128
    B1, B2 = gd.dense(g.cols, N, 11), gd.dense(g.cols, N, 12)
    d1, d2 = ps.DeviceBuffer(host=B1), ps.DeviceBuffer(host=B2)
    c1, c2 = ps.DeviceBuffer.zeros(g.rows * N * 4), ps.DeviceBuffer.zeros(g.rows * N * 4)
    s1, s2 = ps.Stream(), ps.Stream()
    for _ in range(3):
        ps.SpMMAsync(m, N, d1, c1, s1)
        ps.SpMMAsync(m, N, d2, c2, s2)
    ps.synchronize()
    row_of = np.repeat(np.arange(g.rows), np.diff(g.row_ptr))
    for b, c in ((B1, c1), (B2, c2)):
        want = np.zeros((g.rows, N))
        np.add.at(want, row_of, g.values.astype(np.float64)[:, None] * b.astype(np.float64)[g.col_ind])
        got = c.download(np.float32).reshape(g.rows, N)
        # three calls: every row here accumulates except rows stored by the residue
        stored = g.parts[0].des[0][g.parts[0].residue_atomic == 0]
        want3 = 3 * want
        want3[stored] = want[stored]
        np.testing.assert_array_equal(got, want3)
    m.close()
    ps.synchronize()
    free0, _ = ps.mem_get_info()  # the GEMM library is loaded by now
    for _ in range(3):
        m = ps.PowerSparseMatrixGPU.from_csr(csr, **kw)
        ps.SpMMAsync(m, N, d1, c1)
        m.close()
    ps.synchronize()
    free1, _ = ps.mem_get_info()
    assert free1 >= free0 - (4 << 20), (free0, free1)


def test_hub_entry_points_through_the_abi():
    """The block's C entry points on a block built by hand: SpMM adds exactly
    the products of the block entries whose (row, column) slot is stored once
    into the hub rows; SDDMM, from a plan of the listed tiles, writes exactly
    those tiles' outputs (exact inputs, bit for bit against numpy) and skips
    codes that name no tile (residue workset, workset past the count, tile
    past the workset's end, groups under 64 nonzeros)."""
    import ctypes
    from gpu_util import Uploaded
    from powersparse_amd import _native, _ptr, _workset_array, _out_array, _hip_call
    setup()
    hip = _native.hip()
    g = gd.load("hubs")
    csr = csr_of(g)
    p = g.parts[0]
    w = oracle.preprocess(g.rows, g.cols, g.row_ptr, g.col_ind, g.values, p.cu)
    (d, c), = thresholds(csr, p.cu)
    deg = np.diff(g.row_ptr.astype(np.int64))
    cnt = np.bincount(g.col_ind, minlength=g.cols)
    hub_rows = np.flatnonzero(deg >= d).astype(np.int32)
    hot_cols = np.flatnonzero(cnt >= c).astype(np.int32)
    hub_index = np.full(g.rows, -1, np.int32)
    hub_index[hub_rows] = np.arange(hub_rows.size)
    hot_rank = np.full(g.cols, -1, np.int32)
    hot_rank[hot_cols] = np.arange(hot_cols.size)
    R, H = hub_rows.size, hot_cols.size
    say(f"hand-built block {R} x {H} (degree >= {d}, count >= {c}), S={w.S}")
    bufs = {k: ps.DeviceBuffer(host=v) for k, v in dict(
        hub_rows=hub_rows, hub_index=hub_index, hot_cols=hot_cols, hot_rank=hot_rank,
        row_ptr=g.row_ptr, col_ind=g.col_ind, values=g.values).items()}
    hb = _native.HubBlock(matrix_rows=g.rows, matrix_cols=g.cols, rows=R, cols=H)
    for k in ("hub_rows", "hub_index", "hot_cols", "hot_rank"):
        setattr(hb, k, bufs[k].ptr)
    ld = hip.ps_hub_dense_ld(H)
    assert ld % 64 == 0 and H <= ld < H + 64
    R64 = -(-R // 64) * 64
    assert hip.ps_hub_dense_floats(R, H) == R64 * ld
    dense = ps.DeviceBuffer(R64 * ld * 4)
    stored = ps.DeviceBuffer(max(hip.ps_hub_stored_words(ctypes.byref(hb)), 1) * 4)
    hb.dense, hb.stored = dense.ptr, stored.ptr
    _hip_call(hip.ps_hub_dense_build(ctypes.byref(hb), bufs["row_ptr"].ptr, bufs["col_ind"].ptr,
                                     bufs["values"].ptr, dense.ptr, stored.ptr, None))
    rowof = np.repeat(np.arange(g.rows), deg)
    inblock = (hub_index[rowof] >= 0) & (hot_rank[g.col_ind] >= 0)
    # a slot stored more than once stays out of the block
    slot = rowof.astype(np.int64) * g.cols + g.col_ind
    _, inv, times = np.unique(slot, return_inverse=True, return_counts=True)
    once = times[inv] == 1
    say(f"block entries {int(inblock.sum())}, of them in repeated slots {int((inblock & ~once).sum())}")
    # the dense block: stored-once values, zeros elsewhere (padding included),
    # in fragment order: (row block of 32, step of 8 columns, half of the step,
    # row within the block, column within the half)
    want_dense = np.zeros((R64, ld), np.float32)
    sel = inblock & once
    want_dense[hub_index[rowof[sel]], hot_rank[g.col_ind[sel]]] = g.values[sel]
    frag = want_dense.reshape(R64 // 32, 32, ld // 8, 2, 4).transpose(0, 2, 3, 1, 4)
    np.testing.assert_array_equal(dense.download(np.float32, R64 * ld), frag.ravel())
    inblock = sel

    # SpMM: C = 0 + block * B on the hub rows, zero elsewhere
    N = 64
    B = gd.dense(g.cols, N, gd.SALT_B)
    want = np.zeros((g.rows, N))
    np.add.at(want, rowof[inblock],
              g.values[inblock].astype(np.float64)[:, None] * B[g.col_ind[inblock]])
    dB, dC = ps.DeviceBuffer(host=B), ps.DeviceBuffer.zeros(g.rows * N * 4)
    ws = ps.DeviceBuffer(hip.ps_hub_workspace_bytes(ctypes.byref(hb), _native.PS_OP_SPMM, N))
    _hip_call(hip.ps_hub_spmm_launch(ctypes.byref(hb), N, dB.ptr, dC.ptr, ws.ptr, ws.nbytes,
                                     None))
    ps.synchronize()
    np.testing.assert_array_equal(dC.download(np.float32).reshape(g.rows, N),
                                  want.astype(np.float32))

    # SDDMM: the tiles of block groups lying inside the block, plus bad codes
    up = Uploaded(w)
    tiles, expect = [], {}
    X, Y = gd.dense(g.rows, N, gd.SALT_X), gd.dense(g.cols, N, gd.SALT_Y)
    for s in range(1, w.S):
        gs = 32 << (s - 1)
        for grp in range(w.group_num[s] if gs >= 64 else 0):
            cols_g = w.col[s][grp * gs:(grp + 1) * gs]
            row = w.des[s][grp]
            if hub_index[row] < 0 or (hot_rank[cols_g] < 0).any():
                continue
            for j in range(gs // 64):
                tiles.append((s << 27) | (grp * (gs // 64) + j))
                pos = np.arange(grp * gs + 64 * j, grp * gs + 64 * (j + 1))
                expect.setdefault(s, []).append(pos)
    assert tiles, "no block group lies inside the hand-built block"
    bad = [0 << 27, (w.S << 27) | 0,
           (w.S - 1 << 27) | (w.group_num[w.S - 1] * ((32 << (w.S - 2)) // 64))]
    if w.group_num[1]:
        bad.append((1 << 27) | 0)  # groups of 32 nonzeros
    listed = np.array(bad[:2] + tiles + bad[2:], np.uint32)
    dt = ps.DeviceBuffer(host=listed)
    wa = _workset_array(up.worksets)
    plan_bytes = hip.ps_hub_sddmm_plan_bytes(ctypes.byref(hb), listed.size)
    plan = ps.DeviceBuffer(plan_bytes)
    _hip_call(hip.ps_hub_sddmm_plan(ctypes.byref(hb), w.S, wa, dt.ptr, listed.size, plan.ptr,
                                    plan_bytes, None))
    # the plan's tile table: 64 x 128 dense tiles, the listed entries counted once each
    T = -(-R // 64) * -(-H // 128)
    begin = plan.download(np.uint32, T + 1)
    assert begin[0] == 0 and (np.diff(begin.astype(np.int64)) >= 0).all()
    assert begin[T] == 64 * len(tiles), (begin[T], len(tiles))
    sentinel = np.float32(7.0)
    outs = [ps.DeviceBuffer(host=np.full(max(w.col[s].size, 1), sentinel, np.float32))
            for s in range(w.S)]
    dX, dY = ps.DeviceBuffer(host=X), ps.DeviceBuffer(host=Y)
    wsd = ps.DeviceBuffer(hip.ps_hub_workspace_bytes(ctypes.byref(hb), _native.PS_OP_SDDMM, N))
    _hip_call(hip.ps_hub_sddmm_launch(ctypes.byref(hb), w.S, wa, plan.ptr, listed.size, N,
                                      dX.ptr, dY.ptr, _out_array(outs, w.S), None, None,
                                      wsd.ptr, wsd.nbytes, None))
    ps.synchronize()
    for s in range(w.S):
        out = outs[s].download(np.float32, max(w.col[s].size, 1))[:w.col[s].size]
        mask = np.zeros(w.col[s].size, bool)
        for pos in expect.get(s, []):
            mask[pos] = True
        gs = 32 << (s - 1) if s else 1
        rows = w.des[s][np.arange(w.col[s].size) // gs] if s else None
        if mask.any():
            r, col, val = rows[mask], w.col[s][mask], w.val[s][mask]
            dots = (X[r].astype(np.float64) * Y[col]).sum(1) * val
            np.testing.assert_array_equal(out[mask], dots.astype(np.float32), err_msg=f"ws {s}")
        assert (out[~mask] == sentinel).all(), f"workset {s}: a position outside the list written"


@pytest.mark.parametrize("th", [[(1, 1)], [(64, 1)]])
def test_hub_block_falls_back_when_it_would_hold_everything(th):
    """Explicit tiers that leave no nonzero ((1, 1): every row, every column)
    or only one workset's worth ((64, 1): 586 nonzeros of the light rows) to
    the sparse path: the build keeps no block and the operators give the
    block-free results bit for bit."""
    setup()
    g = gd.load("hubs")
    p = g.parts[0]
    csr = csr_of(g)
    on = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=p.cu, hub_thresholds=th,
                                          csr_positions=True)
    off = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=p.cu, hub_block="off",
                                           csr_positions=True)
    say(f"hubs with tiers {th}: block {on.hub_block}")
    assert on.hub_block == []
    N = 64
    B, X, Y = (gd.dense(g.cols, N, gd.SALT_B), gd.dense(g.rows, N, gd.SALT_X),
               gd.dense(g.cols, N, gd.SALT_Y))
    a, b = run_ops(on, g, N, B, X, Y), run_ops(off, g, N, B, X, Y)
    np.testing.assert_array_equal(a[0], b[0])
    for s in range(on.GroupTypeNum()):
        np.testing.assert_array_equal(a[1][s], b[1][s])
    np.testing.assert_array_equal(a[2], b[2])
    on.close()
    off.close()


def test_hub_block_matrices_from_several_host_threads():
    """Four host threads each build a matrix with a hub block and run SpMM
    and SDDMM on it at once (the GEMM plans and the library handle are shared
    per device): every thread's outputs equal the same calls made from one
    thread, bit for bit."""
    import threading
    setup()
    g = gd.load("hubs")
    p = g.parts[0]
    csr = csr_of(g)
    th = thresholds(csr, p.cu)
    N = 128
    inputs = [(gd.dense(g.cols, N, 20 + k), gd.dense(g.rows, N, 30 + k),
               gd.dense(g.cols, N, 40 + k)) for k in range(4)]

    def work(k, out):
        m = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=p.cu, hub_thresholds=th,
                                             csr_positions=True)
        assert m.hub_block
        out[k] = run_ops(m, g, N, *inputs[k], calls=2)
        m.close()

    seq = {}
    for k in range(4):
        work(k, seq)
    par, errors = {}, []

    def guarded(k):
        try:
            work(k, par)
        except Exception as e:  # reported below
            errors.append(e)

    threads = [threading.Thread(target=guarded, args=(k,)) for k in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for k in range(4):
        np.testing.assert_array_equal(par[k][0], seq[k][0], err_msg=f"thread {k} SpMM")
        for a, b in zip(par[k][1], seq[k][1]):
            np.testing.assert_array_equal(a, b, err_msg=f"thread {k} SDDMM")
        np.testing.assert_array_equal(par[k][2], seq[k][2], err_msg=f"thread {k} SDDMMToCSR")


def test_hub_auto_rule_on_c3():
    """The cost rule on the full C3 graph keeps two tiers, rows of degree >=
    16384 x columns >= 512 and rows of degree 1024..16383 x columns >= 8192,
    and each beats its neighbouring power-of-two thresholds on the rule's
    gain (block nonzeros - 0.12 x rows x columns), counted directly from the
    CSR arrays here; both gains clear the rule's 5% / 2% of the nonzeros."""
    setup()
    csr = ps.synth("C3", seed=1)
    m = ps.PowerSparseMatrixGPU.from_csr(csr)
    say(f"C3 auto hub block: {m.hub_block}")
    assert m.hub_block == [(2526, 72840), (20713, 3578)]
    m.close()
    deg = np.diff(csr.row_ptr.astype(np.int64))
    cnt = np.bincount(csr.col_ind, minlength=csr.cols)
    rdeg = np.repeat(deg, deg)   # each nonzero's row degree
    ccnt = cnt[csr.col_ind]      # each nonzero's column count
    big = np.iinfo(np.int64).max

    def gain(lo, hi, c):
        rows = int(((deg >= lo) & (deg < hi)).sum())
        cols = int((cnt >= c).sum())
        nz = int(((rdeg >= lo) & (rdeg < hi) & (ccnt >= c)).sum())
        return nz - 0.12 * rows * cols, rows, cols

    g0, r0, h0 = gain(16384, big, 512)
    assert (r0, h0) == (2526, 72840) and g0 >= 0.05 * csr.nnz
    for lo, c in [(8192, 512), (32768, 512), (16384, 256), (16384, 1024)]:
        assert gain(lo, big, c)[0] <= g0, (lo, c)
    g1, r1, h1 = gain(1024, 16384, 8192)
    assert (r1, h1) == (20713, 3578) and g1 >= 0.02 * csr.nnz
    for lo, c in [(512, 8192), (2048, 8192), (1024, 4096), (1024, 16384)]:
        assert gain(lo, 16384, c)[0] <= g1, (lo, c)
