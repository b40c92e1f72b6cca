"""CPU-only checks of the product's host side: the libraries load and export
every declared symbol, the host preprocessing steps match the oracle, the
synthetic generators and file readers behave, and argument validation raises
the reference's errors before any device call."""
import os
import re
import subprocess

import numpy as np
import pytest

import oracle
import powersparse_amd as ps
from powersparse_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b((?:ps|psx)_\w+)\s*\(", text, re.M)))


@pytest.mark.parametrize("header,libpath,minimum", [
    ("powersparse_hip.h", _native.HIP_LIB_PATH, 4), ("powersparse.h", _native.HOST_LIB_PATH, 4),
    ("powersparse_bench.h", _native.BENCH_LIB_PATH, 1)])
def test_every_declared_symbol_is_exported(header, libpath, minimum):
    _native.libs()
    _native.bench()
    names = declared(header)
    assert len(names) >= minimum
    out = subprocess.run(["nm", "-D", "--defined-only", libpath], capture_output=True, text=True,
                         check=True).stdout
    exported = set(line.split()[-1] for line in out.splitlines() if line.strip())
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    bound = {n for n, _, _ in (_native.HIP_API + _native.HOST_API + _native.BENCH_API)}
    assert not [n for n in names if n not in bound]


def test_measurement_copy_library_is_separate():
    """The measurement tooling's calibration copy lives in its own library
    (lib/libpowersparse_perf.so), outside the product libraries."""
    _native.perf_lib()
    for lib in (_native.HIP_LIB_PATH, _native.HOST_LIB_PATH):
        out = subprocess.run(["nm", "-D", "--defined-only", lib], capture_output=True,
                             text=True, check=True).stdout
        assert "ps_perf_copy_f32_async" not in out and "probe" not in out
    out = subprocess.run(["nm", "-D", "--defined-only", _native.PERF_LIB_PATH],
                         capture_output=True, text=True, check=True).stdout
    assert [n for n, _, _ in _native.PERF_API] == ["ps_perf_copy_f32_async"]
    assert "ps_perf_copy_f32_async" in out


def test_sigbit_matches_oracle_with_ties():
    # With one distinct count every bucket after the head holds one column, so
    # equal bits mean the same sorted order, ties included. Sizes from 200000
    # up take the product's multi-threaded path, whose order must still be
    # libstdc++ std::sort's.
    rng = np.random.default_rng(11)
    for n in (5, 17, 100, 1000, 50000, 200000, 1000000, 3000000):
        for distinct in (1, 3, 50):
            counts = rng.integers(0, distinct, size=n).astype(np.int32) * 7
            s1, l1 = ps.generate_sigbit(counts)
            s2, l2 = oracle.generate_sigbit(counts)
            assert l1 == l2
            np.testing.assert_array_equal(s1, s2)


def test_workset_count_matches_oracle():
    rng = np.random.default_rng(12)
    for trial in range(30):
        deg = (rng.pareto(1.2, size=int(rng.integers(10, 3000))) * 20).astype(np.int64)
        deg = np.minimum(deg, 200000)
        rp = np.concatenate([[0], np.cumsum(deg)]).astype(np.int32)
        sums = [0] + [int((deg // (32 << (s - 1))).sum()) for s in range(1, 32)]
        for cu in (1, 4, 108, 256):
            assert ps.workset_count(sums, cu) == oracle.analyze_group_type_num(rp, cu)


def test_dense_input_matches_oracle():
    a1, b1 = ps.dense_input(1, 1000, 500)
    a2, b2 = oracle.dense_input(1, 1000, 500)
    np.testing.assert_array_equal(a1, a2)
    np.testing.assert_array_equal(b1, b2)


def rows_sorted_unique(csr):
    for r in range(csr.rows):
        seg = csr.col_ind[csr.row_ptr[r]:csr.row_ptr[r + 1]]
        if seg.size > 1 and not (np.diff(seg) > 0).all():
            return False
    return True


def test_synth_c0_shape_and_determinism():
    a = ps.synth("C0", seed=1)
    b = ps.synth("C0", seed=1)
    c = ps.synth("C0", seed=2)
    assert a.rows == a.cols == 4096
    deg = np.diff(a.row_ptr)
    assert deg.min() >= 1 and deg.max() <= 31 and abs(deg.mean() - 16) < 0.5
    assert rows_sorted_unique(a)
    assert a.values.min() >= -1 and a.values.max() < 1
    np.testing.assert_array_equal(a.col_ind, b.col_ind)
    np.testing.assert_array_equal(a.values, b.values)
    assert not np.array_equal(a.col_ind[:1000], c.col_ind[:1000])


def test_synth_thread_count_independent():
    code = ("import powersparse_amd as ps, hashlib; c = ps.synth('C1', seed=5, scale=200); "
            "print(hashlib.sha1(c.col_ind.tobytes() + c.values.tobytes()).hexdigest())")
    outs = set()
    for threads in ("1", "3"):
        env = dict(os.environ, OMP_NUM_THREADS=threads, PYTHONPATH=ROOT)
        outs.add(subprocess.run(["python", "-c", code], env=env, capture_output=True, text=True,
                                check=True).stdout.strip())
    assert len(outs) == 1


def test_synth_chung_lu_and_community():
    g = ps.synth("C1", seed=1, scale=100)  # 10k nodes
    deg = np.diff(g.row_ptr)
    assert g.rows == 10000 and rows_sorted_unique(g)
    assert deg[:10].mean() > 20 * deg.mean()  # hubs first
    assert 25 < deg.mean() < 55
    c = ps.synth("C4", seed=1, scale=64)  # 32 communities of 1024
    d = np.diff(c.row_ptr)
    assert c.rows == 32 * 1024 and rows_sorted_unique(c)
    assert 0.04 < (d == 0).mean() < 0.07 and 0.04 < (d == 1).mean() < 0.07
    assert 20 < d[d > 1].mean() < 35


def write(tmp_path, name, text):
    p = tmp_path / name
    p.write_text(text)
    return str(p)


MTX_CASES = {
    "real_general.mtx": "%%MatrixMarket matrix coordinate real general\n% c\n\n3 4 5\n"
                        "1 1 1.5\n3 4 -2e-3\n2 2 7\n1 3 0.1\n3 1 1e30\n",
    "pattern_sym.mtx": "%%MatrixMarket matrix coordinate pattern symmetric\n4 4 4\n"
                       "1 1\n2 1\n4 3\n3 2\n",
    "integer.mtx": "%%MatrixMarket matrix coordinate integer general\n2 2 2\n2 1 -3\n1 2 9\n",
    "crlf.mtx": "%%MatrixMarket matrix coordinate real general\r\n2 2 1\r\n1 2 0.25\r\n",
    "bad_banner.mtx": "%%MatrixMarket matrix array real general\n2 2\n1\n2\n3\n4\n",
    "truncated.mtx": "%%MatrixMarket matrix coordinate real general\n2 2 3\n1 1 1\n",
    "extra.mtx": "%%MatrixMarket matrix coordinate real general\n2 2 1\n1 1 1\n2 2 2\n",
    "range.mtx": "%%MatrixMarket matrix coordinate real general\n2 2 1\n3 1 1\n",
    "inf.mtx": "%%MatrixMarket matrix coordinate real general\n2 2 1\n1 1 1e40\n",
    "fields.mtx": "%%MatrixMarket matrix coordinate real general\n2 2 1\n1 1 1 9\n",
    "symrect.mtx": "%%MatrixMarket matrix coordinate real symmetric\n2 3 1\n1 1 1\n",
    "no_final_newline.mtx": "%%MatrixMarket matrix coordinate real general\n2 3 3\n2 3 4\n"
                            "1 1 -1\n2 1 0.5",
    "empty.mtx": "",
    "banner_only.mtx": "%%MatrixMarket matrix coordinate real general\n% no size line\n",
    "blank_first_line.mtx": "\n%%MatrixMarket matrix coordinate real general\n1 1 1\n1 1 1\n",
    "comments_between.mtx": "%%MatrixMarket matrix coordinate integer symmetric\n  % c\n3 3 3\n"
                            "2 1 5\n\n   %x\n3 3 -2\n\t3 1 7 \n% tail\n",
    "integer_real_value.mtx": "%%MatrixMarket matrix coordinate integer general\n2 2 1\n1 1 1.5\n",
    "range_before_value.mtx": "%%MatrixMarket matrix coordinate real general\n2 2 1\n1 3 abc\n",
    "six_words.mtx": "%%MatrixMarket matrix coordinate real general extra\n1 1 1\n1 1 1\n",
    "zero_entries.mtx": "%%MatrixMarket matrix coordinate real general\n2 2 0\n",
    "sym_pattern_dup.mtx": "%%MatrixMarket matrix coordinate pattern symmetric\n3 3 4\n3 1\n"
                           "1 3\n2 2\n3 1\n",
    "nul_in_line.mtx": "%%MatrixMarket matrix coordinate real general\n2 2 1\n1 1 2\x00 junk\n",
}


def ref_read(path):
    out = subprocess.run([oracle.REF_READER, path], capture_output=True, text=True)
    lines = out.stdout.splitlines()
    if lines[0].startswith("ERROR"):
        return lines[0][6:]
    rows, cols, nnz = map(int, lines[0].split())
    rp = np.array(lines[1].split(), dtype=np.int32)
    ci = np.array(lines[2].split(), dtype=np.int32) if nnz else np.zeros(0, np.int32)
    bits = np.array([int(x, 16) for x in lines[3].split()], dtype=np.uint32)
    return rows, cols, rp, ci, bits.view(np.float32)


@pytest.mark.skipif(not os.path.exists(oracle.REF_READER),
                    reason="reference reader not built (needs the reference tree)")
@pytest.mark.parametrize("name", sorted(MTX_CASES))
def test_mtx_reader_matches_reference_reader(tmp_path, name):
    path = write(tmp_path, name, MTX_CASES[name])
    expect = ref_read(path)
    if isinstance(expect, str):
        with pytest.raises(RuntimeError) as e:
            ps.read_mtx(path)
        assert str(e.value) == expect
        return
    got = ps.read_mtx(path)
    rows, cols, rp, ci, va = expect
    assert (got.rows, got.cols) == (rows, cols)
    np.testing.assert_array_equal(got.row_ptr, rp)
    np.testing.assert_array_equal(got.col_ind, ci)
    np.testing.assert_array_equal(got.values.view(np.uint32), va.view(np.uint32))


def test_mtx_reader_semantics(tmp_path):
    g = ps.read_mtx(write(tmp_path, "a.mtx", MTX_CASES["pattern_sym.mtx"]))
    # symmetric: off-diagonals mirrored, file order kept within rows, pattern -> 1
    assert list(g.row_ptr) == [0, 2, 4, 6, 7]
    assert list(g.col_ind) == [0, 1, 0, 2, 3, 1, 2]
    assert (g.values == 1).all()


def test_binary_csr_round_trip(tmp_path):
    a = ps.synth("C0", seed=4, scale=8)
    path = str(tmp_path / "a.pscsr")
    a.write_binary(path)
    b = ps.read_binary(path)
    assert (a.rows, a.cols) == (b.rows, b.cols)
    for x, y in ((a.row_ptr, b.row_ptr), (a.col_ind, b.col_ind), (a.values, b.values)):
        np.testing.assert_array_equal(x, y)


@pytest.mark.parametrize("args,msg", [
    ((0, 4, [0], [], []), "Expected a nonempty CSR matrix with 32-bit indices"),
    ((2, 4, [0, 1, 3], [0, 1], [1, 1]), "Invalid CSR row-pointer endpoints"),
    ((3, 4, [0, 2, 1, 3], [0, 1, 2], [1, 1, 1]), "CSR row pointers must be nondecreasing"),
    ((2, 4, [0, 1, 2], [0, -1], [1, 1]), "Invalid CSR column index or sparse value"),
    ((2, 4, [0, 1, 2], [0, 1], [1, float("inf")]), "Invalid CSR column index or sparse value"),
])
def test_matrix_validation_before_device(args, msg):
    rows, cols, rp, ci, va = args
    with pytest.raises(ValueError, match=msg):
        ps.PowerSparseMatrixGPU(rows, cols, len(ci), rp, ci, va, cu_count=256)
