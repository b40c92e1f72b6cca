"""GPU preprocessing (PowerSparseMatrixGPU) against the CPU oracle: every
index array bit-exact, values bitwise equal, at stated CU counts."""
import numpy as np
import pytest

import oracle
import powersparse_amd as ps
from gpu_util import random_graph, say, setup, star_graph
from test_oracle_preprocess import csr_from_rows

pytestmark = pytest.mark.gpu


ORDERS = ["bitmap_words", "bit_lists"]


def compare(csr, cu, order="auto"):
    w = oracle.preprocess(csr.rows, csr.cols, csr.row_ptr, csr.col_ind, csr.values, cu)
    say(f"  oracle S={w.S} groups={w.group_num} L={w.L}")
    m = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=cu, signature_order=order)
    if order != "auto":
        assert m.signature_order == order
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


@pytest.mark.parametrize("order", ORDERS)
def test_hand_cases(order):
    setup()
    rp, ci, va = csr_from_rows([[0, 1, 2], [0], [3, 0]])
    compare(ps.HostCsr(3, 4, rp, ci, va), 1, order)
    rows = [list(range(32))] * 40 + [list(range(33)), list(range(64)), [], list(range(64, 69))]
    rp, ci, va = csr_from_rows(rows)
    compare(ps.HostCsr(44, 70, rp, ci, va), 1, order)


@pytest.mark.parametrize("order", ORDERS)
@pytest.mark.parametrize("seed", range(8))
@pytest.mark.parametrize("cu", [1, 2, 4, 64])
def test_random_graphs(seed, cu, order):
    setup()
    rng = np.random.default_rng(seed)
    csr = random_graph(rng, int(rng.integers(20, 400)), int(rng.integers(10, 3000)),
                       int(rng.choice([20, 80, 300])), hubs=int(rng.integers(0, 4)),
                       hub_deg=int(rng.integers(100, 2000)), dup=(seed % 3 == 2))
    if csr.nnz == 0:
        return
    say(f"random seed={seed} cu={cu} order={order} rows={csr.rows} nnz={csr.nnz}")
    compare(csr, cu, order)


@pytest.mark.parametrize("order", ORDERS)
@pytest.mark.parametrize("cfg,scale,cu", [
    ("C0", 1, 256), ("C0", 1, 1), ("C1", 100, 1), ("C1", 20, 8), ("C3", 100, 2),
    ("C4", 64, 1), ("C4", 16, 4)])
def test_configs(cfg, scale, cu, order):
    setup()
    csr = ps.synth(cfg, seed=7, scale=scale)
    say(f"config {cfg}/{scale} cu={cu} order={order} rows={csr.rows} nnz={csr.nnz}")
    compare(csr, cu, order)


def test_full_c4_bit_lists():
    # L = 582720 bits: the bitmaps would take groups x 18210 words (~175 GB);
    # the default build takes the bit lists, the oracle its comparison sort
    setup()
    csr = ps.synth("C4", seed=1)
    say(f"full C4 rows={csr.rows} nnz={csr.nnz}")
    m = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=256)
    assert m.signature_order == "bit_lists"
    m.close()
    w = compare(csr, 256)
    assert w.L == 582720 and w.signature[0] is None


@pytest.mark.parametrize("cfg", ["C1", "C3"])
def test_full_size_bit_exact(cfg):
    # the benchmark graphs at full size (C3: ~264 M nonzeros, the north-star
    # graph): every workset array equal to the oracle's, values bitwise
    setup()
    csr = ps.synth(cfg, seed=1)
    say(f"full {cfg} rows={csr.rows} nnz={csr.nnz}")
    compare(csr, 256)


def run_order(group_sets, length):
    """ps_pre_signature_order on worksets given as lists of bit sets."""
    from powersparse_amd import _native
    import ctypes
    flat, begin = [], [0]
    for sets in group_sets:
        for bits in sets:
            flat.extend(sorted(set(bits)))
            begin.append(len(flat))
    lists = ps.DeviceBuffer(host=np.asarray(flat or [0], np.uint32))
    lb = ps.DeviceBuffer(host=np.asarray(begin, np.uint32))
    S = len(group_sets)
    counts = (ctypes.c_int * S)(*[len(x) for x in group_sets])
    perms = [ps.DeviceBuffer(max(len(x), 1) * 4) for x in group_sets]
    ptrs = (ctypes.c_void_p * S)(*[p.ptr for p in perms])
    ps._hip_call(_native.hip().ps_pre_signature_order(lists.ptr, lb.ptr, S, counts, length,
                                                      ptrs, None))
    return [perms[s].download(np.uint32)[:len(x)] for s, x in enumerate(group_sets)]


def test_signature_order_direct():
    setup()
    rng = np.random.default_rng(11)
    length = 4000
    common = sorted(rng.choice(length, 300, replace=False).tolist())
    worksets = []
    for s in range(4):
        sets = []
        if s == 2:
            worksets.append(sets)  # an empty workset
            continue
        for g in range(int(rng.integers(50, 700))):
            kind = rng.random()
            if kind < 0.3:  # a long shared prefix, cut or extended at a random depth
                cut = int(rng.integers(1, len(common) + 1))
                extra = rng.integers(0, length, size=int(rng.integers(0, 3))).tolist()
                sets.append(common[:cut] + extra)
            elif kind < 0.4 and sets:  # an exact repeat
                sets.append(list(sets[int(rng.integers(0, len(sets)))]))
            else:
                sets.append(rng.integers(0, length, size=int(rng.integers(1, 40))).tolist())
        worksets.append(sets)
    say("direct order: groups", [len(x) for x in worksets])
    got = run_order(worksets, length)
    for s, sets in enumerate(worksets):
        np.testing.assert_array_equal(got[s], oracle.order_bit_lists(sets), err_msg=f"ws {s}")


def test_signature_order_single_group():
    setup()
    got = run_order([[[5, 1]], []], 32)
    assert list(got[0]) == [0]


@pytest.mark.parametrize("order", ORDERS)
@pytest.mark.parametrize("deg,rows", [(2048, 40), (8192, 36), (16384, 33), (20000, 34)])
def test_large_groups(deg, rows, order):
    # P = 1: 32+ rows of `deg` nonzeros make GROUP_SIZE up to 16384, exercising
    # the LDS bitonic (<= 8192) and the radix (> 8192) within-group column sorts
    setup()
    rng = np.random.default_rng(deg)
    cols = 3 * deg
    ci = np.concatenate([np.sort(rng.choice(cols, deg, replace=False)) for _ in range(rows)])
    rp = np.arange(rows + 1, dtype=np.int32) * deg
    csr = ps.HostCsr(rows, cols, rp, ci.astype(np.int32),
                     rng.uniform(-1, 1, ci.size).astype(np.float32))
    say(f"large groups deg={deg} rows={rows} order={order}")
    w = compare(csr, 1, order)
    assert w.S >= 2


def test_device_cu_count_default():
    setup()
    csr = ps.synth("C0", seed=1)
    m = ps.PowerSparseMatrixGPU.from_csr(csr)
    assert m.PartitionCuCount() == ps.device_props(0)["cu_count"]
    say("device:", ps.device_props(0))


def test_signature_order_two_pass_keys():
    # 2^21 groups, a 2^30-bit signature and one 4096-element list: the sort key
    # (class, side, divergence, element) needs more than 64 bits, so each round
    # sorts in two stable passes
    setup()
    rng = np.random.default_rng(17)
    length = 1 << 30
    n = 1 << 21
    pool = rng.integers(0, length, 64).tolist()
    sets = [rng.choice(pool, int(rng.integers(1, 4))).tolist() for _ in range(n - 1)]
    sets.append(sorted(set(rng.integers(0, length, 6000).tolist()))[:4096])
    say("two-pass keys: groups", n)
    got = run_order([sets[: n // 2], sets[n // 2:]], length)
    np.testing.assert_array_equal(got[0], oracle.order_bit_lists(sets[: n // 2]))
    np.testing.assert_array_equal(got[1], oracle.order_bit_lists(sets[n // 2:]))


def test_rank_sort_row_classes():
    # every row-length class of ps_pre_rank_sort (one wave up to 256, LDS tiles
    # of 1024 and 8192, radix for longer rows) against numpy's stable sort by
    # (row, count key); few distinct column counts, so most keys tie
    import ctypes
    from powersparse_amd import _native
    setup()
    rng = np.random.default_rng(23)
    degrees = [0, 1, 5, 64, 65, 200, 256, 257, 300, 1024, 1025, 5000, 8192, 8193, 20000, 0, 33,
               9000]
    degrees += rng.integers(0, 150, 3000).tolist()
    cols = 30000
    pool = rng.choice(cols, 400, replace=False)  # columns concentrated on a few hundred
    ci = []
    for d in degrees:
        if d <= 300:
            row = rng.choice(pool, d, replace=False)
        else:
            row = rng.choice(cols, d, replace=False)
        ci.append(np.sort(row))
    ci = np.concatenate(ci).astype(np.int32)
    rp = np.concatenate([[0], np.cumsum(degrees)]).astype(np.int32)
    rows, nnz = len(degrees), ci.size
    cn = np.bincount(ci, minlength=cols).astype(np.int32)
    max_count = int(cn.max())
    cb = max_count.bit_length()
    row_of = np.repeat(np.arange(rows), np.diff(rp))
    ckey = (max_count - cn[ci]).astype(np.uint64)
    order = np.lexsort((np.arange(nnz), ckey, row_of))  # stable by (row, key)
    exp_keys = (row_of[order].astype(np.uint64) << np.uint64(cb)) | ckey[order]
    d_rp, d_ci, d_cn = (ps.DeviceBuffer(host=a) for a in (rp, ci, cn))
    keys = ps.DeviceBuffer(nnz * 8)
    vals = ps.DeviceBuffer(nnz * 4)
    ps._hip_call(_native.hip().ps_pre_rank_sort(d_rp.ptr, rows, d_ci.ptr, nnz, d_cn.ptr,
                                                max_count, cb, keys.ptr, vals.ptr, None))
    np.testing.assert_array_equal(vals.download(np.uint32), order.astype(np.uint32))
    np.testing.assert_array_equal(keys.download(np.uint64), exp_keys)


def _snapshot(m):
    """Every public array of a matrix, on the host."""
    ws = [m.download_workset(s) if m.GroupNum()[s] else None for s in range(m.GroupTypeNum())]
    return m.GroupNum(), m.SignatureLen(), m.residue_offset(), m.residue_atomic(), ws


def _assert_same(a, b, what):
    assert a[0] == b[0] and a[1] == b[1], what
    np.testing.assert_array_equal(a[2], b[2], err_msg=what)
    np.testing.assert_array_equal(a[3], b[3], err_msg=what)
    for s, (x, y) in enumerate(zip(a[4], b[4])):
        if x is None:
            assert y is None, what
            continue
        for k in range(3):
            np.testing.assert_array_equal(x[k].view(np.uint32), y[k].view(np.uint32),
                                          err_msg=f"{what} workset {s}")


def test_concurrent_constructions():
    """Matrices built at the same time from several host threads (the shared
    default stream, the process-wide page-locked staging buffers of the
    full-size upload, each construction's column-bit helper thread) equal the
    same matrices built one at a time, and the small ones the oracle's."""
    from concurrent.futures import ThreadPoolExecutor
    setup()
    graphs = [ps.synth("C4", seed=1), ps.synth("C1", seed=2, scale=20),
              ps.synth("C4", seed=1), ps.synth("C3", seed=3, scale=40)]
    say("concurrent constructions: " + ", ".join(str(g.nnz) for g in graphs))

    def build(csr):
        m = ps.PowerSparseMatrixGPU.from_csr(csr, cu_count=8)
        snap = _snapshot(m)
        m.close()
        return snap

    with ThreadPoolExecutor(len(graphs)) as ex:
        together = list(ex.map(build, graphs))
    alone = [build(g) for g in graphs]
    for i, (a, b) in enumerate(zip(together, alone)):
        _assert_same(a, b, f"graph {i}: concurrent vs sequential")
    for i in (1, 3):
        csr = graphs[i]
        w = oracle.preprocess(csr.rows, csr.cols, csr.row_ptr, csr.col_ind, csr.values, 8)
        gn, L, ro, ra, ws = together[i]
        assert gn == w.group_num and L == w.L
        np.testing.assert_array_equal(ro, w.residue_offset)
        np.testing.assert_array_equal(ra, w.residue_atomic)
        for s in range(w.S):
            if w.group_num[s]:
                col, val, des = ws[s]
                np.testing.assert_array_equal(col, w.col[s])
                np.testing.assert_array_equal(val.view(np.uint32), w.val[s].view(np.uint32))
                np.testing.assert_array_equal(des, w.des[s])


def test_constructions_release_device_memory():
    """Building and closing matrices, with and without the row-ordered
    execution copy and the CSR positions, leaves the device's free memory
    where it was."""
    setup()
    graphs = [ps.synth("C1", seed=2, scale=10), ps.synth("C4", seed=4, scale=8)]
    # one warm-up pass: runtime-internal buffers of first use are not leaks
    for csr in graphs:
        ps.PowerSparseMatrixGPU.from_csr(csr).close()
    ps.synchronize()
    free0, total = ps.mem_get_info()
    say(f"device memory free {free0 >> 20} MB of {total >> 20} MB")
    for rep in range(3):
        for csr in graphs:
            for kw in ({}, {"csr_positions": True}, {"task_order": "row"},
                       {"task_order": "signature", "csr_positions": True}):
                m = ps.PowerSparseMatrixGPU.from_csr(csr, **kw)
                m.close()
    ps.synchronize()
    free1, _ = ps.mem_get_info()
    say(f"after 24 constructions: free {free1 >> 20} MB")
    assert free1 >= free0 - (4 << 20), (free0, free1)


@pytest.mark.parametrize("order", ORDERS)
def test_star_columns(order):
    """Two hub columns in every row (col_nnz = rows for both, the two top
    columns FFC puts in bucket 0), many rows tied on every other column
    count, plus a few long rows: ranking ties, one huge histogram bin and
    signatures that all share their first bit."""
    setup()
    csr = star_graph(np.random.default_rng(77), 120000, 50000, 8, long_rows=40, long_deg=700)
    say(f"star columns rows={csr.rows} nnz={csr.nnz} order={order}")
    w = compare(csr, 4, order)
    assert w.S >= 2
