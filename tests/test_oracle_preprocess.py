"""Pins the CPU oracle's preprocessing (oracle/oracle.cpp) before anything is
checked against it.

The reference ships no tests, fixtures or golden vectors for this path, so the
pins are: worksets derived by hand for small CSRs (derivations inline), the
reference's own multiset invariant (benchmarks/benchmark.cu:45-62), an
independently written brute-force restatement (tests/brute.py) on random tiny
graphs, and structural invariants the algorithm fixes. The one piece only C++
can fix, libstdc++'s std::sort tie order in GenerateSigBit, is pinned by
hand where the sort is an insertion sort (n <= 16, stable) and by invariants
that hold for any tie order.
"""
import numpy as np
import pytest

import brute
import oracle


def csr_from_rows(rows_cols, values=None):
    row_ptr = [0]
    col = []
    for r in rows_cols:
        col += list(r)
        row_ptr.append(len(col))
    if values is None:
        values = [p + 0.5 for p in range(len(col))]
    return np.array(row_ptr, np.int32), np.array(col, np.int32), np.array(values, np.float32)


def test_hand_fine_mode():
    # rows 0..2 = {0,1,2}, {0}, {3,0}; P = 1 -> threshold 32, no row reaches 32,
    # so S = 1 (fine mode, chunks of 16). col_nnz = [3,1,1,1]. GenerateSigBit on
    # 4 columns: std::sort of <= 16 items is an insertion sort (stable), order
    # [0,1,2,3]; ffc=2 gives cols 0,1 bit 0 (mass 4); cols 2,3 join bucket 1
    # (mass 1, 2 < 4); 2 bits -> L = 32. Groups (row order): g0 = row0 ranked
    # [p0,p1,p2]; g1 = row1 [p3]; g2 = row2 ranked by count [p5(col0), p4(col3)].
    # Signatures: g0 bits {0,1} -> 0xC0000000, g1 {0} -> 0x80000000, g2 {0,1}
    # -> 0xC0000000; stable descending -> perm [0, 2, 1]. Within a group,
    # columns ascending: g2 -> cols [0, 3] = values [v5, v4].
    rp, ci, va = csr_from_rows([[0, 1, 2], [0], [3, 0]])
    w = oracle.preprocess(3, 4, rp, ci, va, cu_count=1)
    assert w.S == 1 and w.group_num == [3] and w.L == 32
    assert list(w.sigbit) == [0, 0, 1, 1]
    assert list(w.col_nnz) == [3, 1, 1, 1]
    assert list(w.perm[0]) == [0, 2, 1]
    assert list(w.col[0]) == [0, 1, 2, 0, 3, 0]
    assert list(w.val[0]) == [va[0], va[1], va[2], va[5], va[4], va[3]]
    assert list(w.residue_offset) == [0, 3, 5, 6]
    assert list(w.des[0]) == [0, 2, 1]
    assert list(w.residue_atomic) == [0, 0, 0]
    assert list(w.signature[0][0]) == [0xC0000000, 0x80000000, 0xC0000000]


def test_hand_blocks_and_residue():
    # P = 1 (threshold 32). rows 0..39: cols 0..31 (deg 32); row 40: cols 0..32
    # (deg 33); row 41: cols 0..63 (deg 64); row 42 empty; row 43: cols 64..68.
    # sum floor(d/32) = 40 + 1 + 2 = 43 >= 32, sum floor(d/64) = 1 < 32 -> S = 2.
    # col_nnz: 0..31 -> 42, 32 -> 2, 33..68 -> 1, 69 -> 0.
    # Membership: deg-32 rows: one block each, no residue; row 40: block of
    # cols 0..31 (count 42 beats 2) + residue {32} (atomic: deg > 32); row 41:
    # blocks {0..31} then {32..63}; row 43: residue {64..68}, not atomic.
    # Signature bits, for ANY tie order: two of cols 0..31 take bit 0 (mass 84);
    # each other count-42 column opens a bucket (42 < 84, 84 not < 84): bits
    # 1..30; the bucket of the last one also takes the whole tail, since
    # 42 + 2 + 36 * 1 + 0 = 80 < 84 -> cols 32..69 get bit 30; 31 bits -> L = 32.
    # Every block holding cols 0..31 has word 0xFFFFFFFE, row 41's second block
    # and both residues 0x00000002: the stable sorts keep the initial (row)
    # order in both worksets.
    rows = [list(range(32))] * 40 + [list(range(33)), list(range(64)), [], list(range(64, 69))]
    rp, ci, va = csr_from_rows(rows)
    w = oracle.preprocess(44, 70, rp, ci, va, cu_count=1)
    assert w.S == 2 and w.L == 32
    assert w.group_num == [2, 43]
    assert list(w.des[1]) == list(range(40)) + [40, 41, 41]
    assert list(w.perm[1]) == list(range(43))
    assert list(w.col[1]) == list(range(32)) * 42 + list(range(32, 64))
    # values follow their columns: row r's value for column c sits at CSR position rp[r] + c
    expect_val = [va[rp[r] + c] for r in range(42) for c in range(32)]
    expect_val += [va[rp[41] + c] for c in range(32, 64)]
    assert list(w.val[1]) == expect_val
    assert list(w.des[0]) == [40, 43]
    assert list(w.perm[0]) == [0, 1]
    assert list(w.residue_offset) == [0, 1, 6]
    assert list(w.residue_atomic) == [1, 0]
    assert list(w.col[0]) == [32, 64, 65, 66, 67, 68]
    assert list(w.val[0]) == [va[rp[40] + 32]] + [va[rp[43] + k] for k in range(5)]
    assert set(w.sigbit[32:].tolist()) == {30}
    assert sorted(w.sigbit[:32].tolist()) == [0, 0] + list(range(1, 31))
    assert list(w.signature[1][0]) == [0xFFFFFFFE] * 42 + [2]
    assert list(w.signature[0][0]) == [2, 2]


@pytest.mark.parametrize("degrees,cu,expect", [
    ([31] * 100, 1, 1),             # nothing reaches 32
    ([32] * 32, 1, 2),              # exactly the threshold at size 32
    ([32] * 31, 1, 1),              # one short
    ([64] * 32, 1, 3),              # 64 groups of 32, 32 of 64, 0 of 128
    ([64] * 32, 2, 2),              # threshold 64: 64 groups of 32 only
    ([1000] * 40, 1, 6),            # 1240, 600, 280, 120, 40 >= 32; 0 at 1024
])
def test_workset_count_closed_form(degrees, cu, expect):
    rp = np.concatenate([[0], np.cumsum(degrees)]).astype(np.int32)
    # independent closed form: S = 1 + #{s >= 1 : sum floor(d / (32 * 2^(s-1))) >= 32 * cu}
    thr = 32 * cu
    s = 1
    while sum(d // (32 << (s - 1)) for d in degrees) >= thr:
        s += 1
    assert s == expect
    assert oracle.analyze_group_type_num(rp, cu) == expect


def test_workset_count_thousand():
    # deg 1000, 40 rows, P = 1: floor(1000/32)=31 -> 1240; /64=15 -> 600; /128=7 -> 280;
    # /256=3 -> 120; /512=1 -> 40; /1024=0 -> 0 < 32. Sizes 32..512 pass -> S = 6.
    rp = np.arange(41, dtype=np.int32) * 1000
    assert oracle.analyze_group_type_num(rp, 1) == 6


def test_sigbit_hand():
    # 8 columns (insertion sort, stable): counts [5,9,9,1,0,3,3,2] sort to
    # c1(9) c2(9) c0(5) c5(3) c6(3) c7(2) c3(1) c4(0). Bit 0: c1, c2, mass 18.
    # Bucket 1 takes c0..c4: running 5, 8, 11, 13, 14, 14 all < 18. L = 32.
    sig, L = oracle.generate_sigbit([5, 9, 9, 1, 0, 3, 3, 2])
    assert L == 32 and list(sig) == [1, 0, 0, 1, 1, 1, 1, 1]
    # counts [10,10,15,6,5,4,3]: c2(15) c0(10) c1(10) c3 c4 c5 c6. Bit 0: c2, c0
    # (mass 25). Bucket 1: c1 10, c3 16, c4 21 (< 25), c5 -> 25 not < 25: stop.
    # Bucket 2: c5 (first always taken) 4, c6 7.
    sig, L = oracle.generate_sigbit([10, 10, 15, 6, 5, 4, 3])
    assert L == 32 and list(sig) == [0, 1, 0, 1, 1, 2, 2]
    # a single heavy column after the head still gets its own bucket
    sig, L = oracle.generate_sigbit([1, 1, 50, 1])
    assert list(sig) == [0, 1, 0, 1]  # c2(50), c0(1) head (mass 51); c1,c3 bucket 1


@pytest.mark.parametrize("ncols,expect_len", [(47, 32), (48, 32), (49, 64), (80, 64), (81, 96)])
def test_sigbit_length_rounding(ncols, expect_len):
    # all counts 1: head = 2 columns (mass 2), every later bucket holds exactly
    # one column (1 < 2, then 2 not < 2): ncols - 1 bits. Rounding: < 32 -> 32,
    # bits % 32 < 16 -> floor, else ceil; bits >= L clamp to L - 1. The multiset
    # of bits is the same for any tie order.
    sig, L = oracle.generate_sigbit(np.ones(ncols, np.int32))
    bits = ncols - 1
    assert L == expect_len
    expect = sorted([0, 0] + [min(b, L - 1) for b in range(1, bits)])
    assert sorted(sig.tolist()) == expect


def test_sigbit_bucket_invariants():
    rng = np.random.default_rng(7)
    for trial in range(20):
        n = int(rng.integers(20, 3000))
        counts = rng.integers(0, 12, size=n).astype(np.int32) ** 2
        sig, L = oracle.generate_sigbit(counts)
        assert L % 32 == 0 and L >= 32
        assert sig.min() == 0 and sig.max() <= L - 1
        # buckets are contiguous in count-descending order: every column of a
        # lower bit has a count >= every column of a higher bit (strictly
        # unclamped bits only)
        top = int(sig.max())
        for b in range(top):
            assert counts[sig == b].min() >= counts[sig == b + 1].max() or b + 1 == top
        # head: exactly min(2, n) columns on bit 0 carrying the largest counts
        assert (sig == 0).sum() == 2
        assert sorted(counts[sig == 0]) == sorted(np.sort(counts)[-2:])


def random_graph(rng, rows, cols, max_deg, dup=False, empty_frac=0.1):
    rp = [0]
    ci = []
    for _ in range(rows):
        d = 0 if rng.random() < empty_frac else int(rng.integers(0, max_deg + 1))
        if dup:
            row = rng.integers(0, cols, size=d).tolist()
        else:
            row = rng.choice(cols, size=min(d, cols), replace=False).tolist()
        ci += row
        rp.append(len(ci))
    va = rng.uniform(-1, 1, size=len(ci)).astype(np.float32)
    return np.array(rp, np.int32), np.array(ci, np.int32), va


@pytest.mark.parametrize("order", ["bitmap_words", "bit_lists"])
@pytest.mark.parametrize("seed", range(12))
def test_brute_force_agreement(seed, order):
    rng = np.random.default_rng(100 + seed)
    rows = int(rng.integers(5, 60))
    cols = int(rng.integers(3, 90))
    max_deg = int(rng.choice([12, 40, 140, 300]))
    dup = bool(seed % 4 == 3)
    rp, ci, va = random_graph(rng, rows, cols, max_deg, dup=dup)
    if ci.size == 0:
        return
    for cu in (1, 2, 4, 64):
        w = oracle.preprocess(rows, cols, rp, ci, va, cu, signature_order=order)
        S, b = brute.preprocess(rows, cols, rp.tolist(), ci.tolist(), va.tolist(), cu,
                                w.sigbit.tolist(), w.L)
        assert w.S == S
        for s in range(S):
            assert w.group_num[s] == len(b[s]["des"])
            assert list(w.perm[s]) == b[s]["perm"], (cu, s)
            assert list(w.des[s]) == b[s]["des"]
            assert list(w.col[s]) == b[s]["col"]
            np.testing.assert_array_equal(w.val[s], np.array(b[s]["val"], np.float32))
        assert list(w.residue_offset) == b[0]["offsets"]
        assert [bool(x) for x in w.residue_atomic] == b[0]["atomic"]


@pytest.mark.parametrize("seed", range(8))
def test_capped_partition_brute_force_agreement(seed):
    """The oracle's optional cap on the workset count (the product's tuned SpMM
    partition) against the brute force with the same cap; a cap at or above the
    reference's S changes nothing."""
    rng = np.random.default_rng(300 + seed)
    rows = int(rng.integers(20, 60))
    cols = int(rng.integers(30, 120))
    rp, ci, va = random_graph(rng, rows, cols, int(rng.choice([140, 300])))
    if ci.size == 0:
        return
    for cu in (1, 2):
        full = oracle.preprocess(rows, cols, rp, ci, va, cu)
        for cap in (1, 2, 3, full.S, full.S + 2):
            w = oracle.preprocess(rows, cols, rp, ci, va, cu, max_group_types=cap)
            S, b = brute.preprocess(rows, cols, rp.tolist(), ci.tolist(), va.tolist(), cu,
                                    w.sigbit.tolist(), w.L, max_group_types=cap)
            assert w.S == S == min(cap, full.S)
            for s in range(S):
                assert list(w.perm[s]) == b[s]["perm"], (cu, cap, s)
                assert list(w.des[s]) == b[s]["des"]
                assert list(w.col[s]) == b[s]["col"]
                np.testing.assert_array_equal(w.val[s], np.array(b[s]["val"], np.float32))
            assert list(w.residue_offset) == b[0]["offsets"]
            assert [bool(x) for x in w.residue_atomic] == b[0]["atomic"]
            if cap >= full.S:  # the reference's partition itself
                for s in range(S):
                    np.testing.assert_array_equal(w.col[s], full.col[s])
                    np.testing.assert_array_equal(w.des[s], full.des[s])


def bigint_order(bit_sets, length):
    """Descending order of the L-bit signature integers (bit b weighs
    2^(L-1-b)), ties in group order (sorted() is stable)."""
    value = [sum(1 << (length - 1 - b) for b in set(bits)) for bits in bit_sets]
    return sorted(range(len(bit_sets)), key=lambda g: -value[g])


def test_order_bit_lists_hand():
    # prefix relations, duplicates, an empty set and equal sets
    sets = [[3], [0, 1], [1, 0, 0], [0], [], [0, 1, 2], [2, 5], [3], [0, 2]]
    # 0,1,2 > 0,1 = 1,0,0 > 0,2 > 0 > 2,5 > 3 = 3 > empty
    assert list(oracle.order_bit_lists(sets)) == [5, 1, 2, 8, 3, 6, 0, 7, 4]
    assert list(oracle.order_bit_lists(sets)) == bigint_order(sets, 8)


@pytest.mark.parametrize("seed", range(6))
def test_order_bit_lists_bigint(seed):
    rng = np.random.default_rng(seed)
    length = int(rng.choice([6, 32, 96]))
    groups = int(rng.integers(1, 400))
    sets = []
    for _ in range(groups):
        if sets and rng.random() < 0.2:  # repeat or extend an earlier set
            base = list(sets[int(rng.integers(0, len(sets)))])
            if rng.random() < 0.5:
                base.append(int(rng.integers(0, length)))
            sets.append(base)
        else:
            k = int(rng.integers(1, min(length, 12) + 1))
            sets.append(rng.integers(0, length, size=k).tolist())
    assert list(oracle.order_bit_lists(sets)) == bigint_order(sets, length)


def check_structure(rows, cols, rp, ci, va, w):
    deg = np.diff(rp)
    S = w.S
    # multiset invariant (benchmarks/benchmark.cu:45-62)
    got = []
    for s in range(S):
        offs = w.offsets(s)
        for g in range(w.group_num[s]):
            r = w.des[s][g]
            for p in range(offs[g], offs[g + 1]):
                got.append((r, w.col[s][p], w.val[s][p]))
    exp = [(r, ci[p], va[p]) for r in range(rows) for p in range(rp[r], rp[r + 1])]
    assert sorted(got) == sorted(exp)
    # group sizes per row follow the greedy decomposition
    for s in range(1, S):
        gs = 32 << (s - 1)
        assert w.col[s].size == w.group_num[s] * gs
    lens = np.diff(w.residue_offset)
    if S == 1:
        assert lens.max(initial=0) <= 16
    else:
        assert lens.max(initial=0) <= 31
        assert (w.residue_atomic == (deg[w.des[0]] > 32)).all()
    # each group's columns ascending; signature order non-increasing
    for s in range(S):
        offs = w.offsets(s)
        for g in range(w.group_num[s]):
            seg = w.col[s][offs[g]:offs[g + 1]]
            assert (np.diff(seg) >= 0).all()
        if w.signature[s] is None:  # ordered by bit lists
            continue
        sig = w.signature[s][:, w.perm[s]].T  # sorted groups x words
        for k in range(1, sig.shape[0]):
            assert tuple(sig[k - 1]) >= tuple(sig[k])


def test_structure_c0():
    import powersparse_amd as ps
    csr = ps.synth("C0", seed=1)
    w = oracle.preprocess(csr.rows, csr.cols, csr.row_ptr, csr.col_ind, csr.values, 256)
    assert w.S == 1  # no row reaches 32 nonzeros: fine mode at any CU count
    check_structure(csr.rows, csr.cols, csr.row_ptr, csr.col_ind, csr.values, w)


@pytest.mark.parametrize("cfg,scale,cu", [("C1", 500, 1), ("C3", 800, 1), ("C4", 256, 2)])
def test_structure_scaled_configs(cfg, scale, cu):
    import powersparse_amd as ps
    csr = ps.synth(cfg, seed=3, scale=scale)
    w = oracle.preprocess(csr.rows, csr.cols, csr.row_ptr, csr.col_ind, csr.values, cu)
    assert w.S >= 2
    check_structure(csr.rows, csr.cols, csr.row_ptr, csr.col_ind, csr.values, w)


@pytest.mark.parametrize("cfg,scale,cu", [("C0", 1, 256), ("C1", 500, 1), ("C3", 800, 1),
                                          ("C4", 64, 2), ("C4", 256, 2)])
def test_order_methods_agree(cfg, scale, cu):
    import powersparse_amd as ps
    csr = ps.synth(cfg, seed=5, scale=scale)
    args = (csr.rows, csr.cols, csr.row_ptr, csr.col_ind, csr.values, cu)
    a = oracle.preprocess(*args, signature_order="bitmap_words")
    b = oracle.preprocess(*args, signature_order="bit_lists")
    assert a.S == b.S and b.signature[0] is None
    for s in range(a.S):
        assert (a.perm[s] == b.perm[s]).all()
        assert (a.col[s] == b.col[s]).all() and (a.des[s] == b.des[s]).all()
    assert (a.residue_offset == b.residue_offset).all()


@pytest.mark.parametrize("args,msg", [
    ((0, 4, [0], [], []), "Expected a nonempty CSR matrix with 32-bit indices"),
    ((2, 4, [1, 1, 2], [0, 1], [1, 1]), "Invalid CSR row-pointer endpoints"),
    ((2, 4, [0, 1, 3], [0, 1], [1, 1]), "Invalid CSR row-pointer endpoints"),
    ((3, 4, [0, 2, 1, 3], [0, 1, 2], [1, 1, 1]), "CSR row pointers must be nondecreasing"),
    ((2, 4, [0, 1, 2], [0, 4], [1, 1]), "Invalid CSR column index or sparse value"),
    ((2, 4, [0, 1, 2], [0, 1], [1, float("nan")]), "Invalid CSR column index or sparse value"),
])
def test_invalid_input_messages(args, msg):
    rows, cols, rp, ci, va = args
    with pytest.raises(ValueError, match=msg):
        oracle.preprocess(rows, cols, rp, ci, va, 1)
