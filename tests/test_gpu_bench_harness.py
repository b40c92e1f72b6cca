"""The CSV benchmark harness (psx_bench_main, lib/libpowersparse_bench.so: the
code of the powersparse_{spmm,sddmm} command lines) on the GPU, called in this
process: the CSV row, the CHECK path (preprocessing invariant and CPU
reference, as benchmarks/benchmark.cu:45-96), the argument errors and exit
codes, and the batch runner's matrices (a MatrixMarket file with an empty
row, a pattern matrix, a generated graph) at two widths each. stdout and
stderr are captured at the file-descriptor level around each call."""
import csv
import ctypes
import io
import os
import subprocess
import sys
import tempfile

import pytest

from gpu_util import say
from powersparse_amd import _native

pytestmark = pytest.mark.gpu

HEADER = ("algorithm,operator,matrix,rows,cols,nnz,N,device,gpu,compute_capability,"
          "cuda_runtime,cuda_driver,warmup,repeats,seed,check,preprocess_ms,ms,gflops")
OPS = {"spmm": 0, "sddmm": 1}

SMALL_MTX = """%%MatrixMarket matrix coordinate real general
% small test matrix
6 5 9
1 1 0.5
1 3 -1.25
2 2 2.0
3 1 1.0
3 5 3.5
5 4 -0.75
6 1 1.5
6 2 0.25
6 5 -2.0
"""


def dense_mtx(rows, cols, per_row):
    lines = ["%%MatrixMarket matrix coordinate pattern general", f"{rows} {cols} {rows * per_row}"]
    for r in range(rows):
        for k in range(per_row):
            lines.append(f"{r + 1} {(r * 7 + k * 3) % cols + 1}")
    return "\n".join(lines) + "\n"


def harness(op, *args):
    """(exit code, stdout, stderr) of psx_bench_main with argv = program, args."""
    argv = [f"powersparse_{op}".encode()] + [str(a).encode() for a in args]
    arr = (ctypes.c_char_p * (len(argv) + 1))(*argv, None)
    libc = ctypes.CDLL(None)
    with tempfile.TemporaryFile() as out, tempfile.TemporaryFile() as err:
        libc.fflush(None)
        saved = os.dup(1), os.dup(2)
        os.dup2(out.fileno(), 1)
        os.dup2(err.fileno(), 2)
        try:
            rc = _native.bench().psx_bench_main(OPS[op], len(argv), arr)
            libc.fflush(None)
        finally:
            os.dup2(saved[0], 1)
            os.dup2(saved[1], 2)
            os.close(saved[0])
            os.close(saved[1])
        out.seek(0)
        err.seek(0)
        o, e = out.read().decode(), err.read().decode()
    say(f"$ {' '.join(a.decode() for a in argv)} -> {rc}")
    say(e.strip())
    return rc, o, e


def row_of(stdout):
    return next(csv.DictReader(io.StringIO(HEADER + "\n" + stdout)))


@pytest.mark.parametrize("op,N", [("spmm", 32), ("spmm", 64), ("sddmm", 128)])
def test_harness_synth_check(op, N):
    rc, out, err = harness(op, "synth:C0:5", N, 0, 1, 3)
    assert rc == 0
    row = row_of(out)
    assert row["algorithm"] == "PowerSparse" and row["operator"] == {"spmm": "SpMM",
                                                                      "sddmm": "SDDMM"}[op]
    assert row["matrix"] == "synth:C0:5" and int(row["nnz"]) == 64975
    assert row["check"] == "passed" and int(row["N"]) == N and int(row["repeats"]) == 3
    assert int(row["warmup"]) == 30 and int(row["seed"]) == 1
    assert row["compute_capability"].startswith("gfx")
    assert float(row["ms"]) > 0 and float(row["gflops"]) > 0 and float(row["preprocess_ms"]) > 0
    assert "checks passed" in err


def test_harness_errors(tmp_path):
    rc, _, err = harness("spmm", "synth:C0", 48, 0, 0, 1)
    assert rc == 2 and "N=48 was not selected in main" in err
    rc, _, err = harness("sddmm", tmp_path / "missing.mtx", 32, 0, 0, 1)
    assert rc == 1 and "Error: Cannot open matrix" in err
    rc, _, err = harness("spmm", "synth:C0", 32, 0, 2, 1)
    assert rc == 1 and "CHECK 0 or 1" in err
    rc, _, err = harness("spmm")
    assert rc == 2 and err.startswith("Usage:")
    rc, out, _ = harness("sddmm", "--header")
    assert rc == 0 and out.strip() == HEADER


def test_harness_on_the_runner_matrices(tmp_path):
    (tmp_path / "small.mtx").write_text(SMALL_MTX)
    (tmp_path / "rows40.mtx").write_text(dense_mtx(80, 300, 40))
    rows = []
    for name in ("small.mtx", "rows40.mtx", "synth:C4:2:64"):
        spec = name if name.startswith("synth:") else tmp_path / name
        for N in (32, 64):
            rc, out, _ = harness("sddmm", spec, N, 0, 1, 2)
            assert rc == 0, (name, N)
            rows.append(row_of(out))
    assert [int(r["N"]) for r in rows] == [32, 64] * 3
    assert [int(r["nnz"]) for r in rows[:4]] == [9, 9, 3200, 3200]
    assert all(r["check"] == "passed" and r["operator"] == "SDDMM" for r in rows)
    rc, out, _ = harness("spmm", tmp_path / "small.mtx", 32, 0, 1, 2)
    assert rc == 0 and row_of(out)["check"] == "passed" and int(row_of(out)["rows"]) == 6


ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def child(args, env=None):
    """A child process's (exit code, stdout, stderr), its stderr logged in full."""
    say("$", " ".join(str(a) for a in args))
    r = subprocess.run([str(a) for a in args], capture_output=True, text=True, timeout=240,
                       cwd=ROOT, env=env)
    say(f"exit status {r.returncode}")
    say(r.stderr.strip())
    return r.returncode, r.stdout, r.stderr


@pytest.mark.parametrize("op,N", [("spmm", 32), ("sddmm", 128)])
def test_python_launcher_synth_check(op, N):
    """The harness from its own Python process (python -m powersparse_amd.cli):
    the CSV row, the check path and exit code 0 through the process's exit."""
    rc, out, err = child([sys.executable, "-m", "powersparse_amd.cli", op, "synth:C0:5", N, 0,
                          1, 3])
    assert rc == 0
    row = row_of(out)
    assert row["check"] == "passed" and int(row["N"]) == N and int(row["nnz"]) == 64975
    assert float(row["ms"]) > 0 and "checks passed" in err


def test_runner_end_to_end_python_launcher(tmp_path):
    """The batch runner (scripts/run_benchmarks.sh:1-64 contract) over two
    MatrixMarket files and a generated graph at two widths, each run a child
    process of the harness through PS_BENCH_LAUNCHER=python."""
    data = tmp_path / "data"
    data.mkdir()
    (data / "small.mtx").write_text(SMALL_MTX)
    (data / "rows40.mtx").write_text(dense_mtx(80, 300, 40))
    manifest = tmp_path / "list.txt"
    manifest.write_text("# two files and a generated graph\nsmall.mtx\nrows40.mtx\nsynth:C4:2:64\n")
    out = tmp_path / "out" / "sddmm.csv"
    env = dict(os.environ, DATASET_LIST=str(manifest), PS_BENCH_LAUNCHER="python")
    rc, _, err = child([sys.executable, "-m", "powersparse_amd.cli.run_benchmarks",
                        os.path.join(ROOT, "powersparse_amd"), data, "sddmm", 0, out, "32,64", 2,
                        1], env=env)
    assert rc == 0 and "Results saved to" in err
    table = list(csv.DictReader(io.StringIO(out.read_text())))
    assert [(os.path.basename(t["matrix"]), int(t["N"])) for t in table] == [
        ("small.mtx", 32), ("small.mtx", 64), ("rows40.mtx", 32), ("rows40.mtx", 64),
        ("synth:C4:2:64", 32), ("synth:C4:2:64", 64)]
    assert all(t["check"] == "passed" and t["operator"] == "SDDMM" for t in table)
    assert [int(t["nnz"]) for t in table[:4]] == [9, 9, 3200, 3200]
