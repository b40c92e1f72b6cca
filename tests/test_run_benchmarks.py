"""The batch runner (powersparse_amd/cli/run_benchmarks.py) against the
contract of the reference's scripts/run_benchmarks.sh:1-64, driven with a stub
binary that records its arguments (no GPU)."""
import os
import stat
import subprocess
import sys

import pytest

from powersparse_amd.cli import run_benchmarks as rb

STUB = """#!{python}
import sys
if sys.argv[1:] == ["--header"]:
    print("algorithm,matrix,N,device,check,repeats")
    sys.exit(0)
matrix, n, device, check, repeats = sys.argv[1:]
if "bad" in matrix:
    print("stub: failing on", matrix, file=sys.stderr)
    sys.exit(3)
print(f"PowerSparse,{{matrix}},{{n}},{{device}},{{check}},{{repeats}}")
"""


@pytest.fixture
def build(tmp_path):
    d = tmp_path / "build"
    (d / "bin").mkdir(parents=True)
    for op in ("spmm", "sddmm"):
        p = d / "bin" / f"powersparse_{op}"
        p.write_text(STUB.format(python=sys.executable))
        p.chmod(p.stat().st_mode | stat.S_IXUSR)
    return d


@pytest.fixture
def data(tmp_path):
    d = tmp_path / "data"
    (d / "sub").mkdir(parents=True)
    for name in ("b.mtx", "a.mtx", "d.pscsr", "notes.txt", "sub/e.mtx"):
        (d / name).write_text("x")
    return d


def run(args, env=None, capsys=None):
    old = os.environ.get("DATASET_LIST")
    os.environ.pop("DATASET_LIST", None)
    if env:
        os.environ.update(env)
    try:
        return rb.main([str(a) for a in args])
    finally:
        os.environ.pop("DATASET_LIST", None)
        if old is not None:
            os.environ["DATASET_LIST"] = old


def rows(path):
    return path.read_text().splitlines()


@pytest.mark.parametrize("args,msg", [
    (["b", "d", "spmm", "0"], "Usage:"),
    (["b", "d", "spmm", "0", "o", "32", "1", "0", "extra"], "Usage:"),
    (["b", "d", "gemm", "0", "o"], "Operator must be spmm or sddmm."),
    (["b", "d", "spmm", "x", "o"], "Invalid DEVICE, REPEATS or CHECK."),
    (["b", "d", "spmm", "0", "o", "32", "0"], "Invalid DEVICE, REPEATS or CHECK."),
    (["b", "d", "spmm", "0", "o", "32", "5", "2"], "Invalid DEVICE, REPEATS or CHECK."),
    (["b", "d", "spmm", "0", "o", "32,,128"], "Invalid N_LIST."),
    (["b", "d", "spmm", "0", "o", "032"], "Invalid N_LIST."),
    (["b", "d", "sddmm", "0", "o", "32,96"],
     "sddmm benchmark: N=96 was not selected in main; please use N=32, 64 or 128."),
])
def test_argument_errors(args, msg, capsys):
    assert run(args) == 2
    assert msg in capsys.readouterr().err


def test_missing_binary(tmp_path, data, capsys):
    assert run([tmp_path / "nobuild", data, "spmm", "0", tmp_path / "o.csv"]) == 1
    assert "Missing executable:" in capsys.readouterr().err


def test_default_selection_and_order(build, data, tmp_path, capsys):
    out = tmp_path / "res" / "spmm.csv"
    assert run([build, data, "spmm", "3", out, "32,64", "7", "1"]) == 0
    assert "Results saved to" in capsys.readouterr().err
    assert not os.path.exists(str(out) + ".partial")
    lines = rows(out)
    assert lines[0] == "algorithm,matrix,N,device,check,repeats"
    # *.mtx and *.pscsr directly in the root, sorted; widths inner
    expect = [f"PowerSparse,{data / m},{n},3,1,7" for m in ("a.mtx", "b.mtx", "d.pscsr")
              for n in (32, 64)]
    assert lines[1:] == expect


def test_defaults(build, data, tmp_path):
    out = tmp_path / "o.csv"
    assert run([build, data, "sddmm", "0", out]) == 0
    assert rows(out)[1] == f"PowerSparse,{data / 'a.mtx'},32,0,0,100"
    assert rows(out)[2] == f"PowerSparse,{data / 'a.mtx'},128,0,0,100"


def test_manifest(build, data, tmp_path):
    man = tmp_path / "list.txt"
    man.write_bytes(b"# inputs\r\n\r\n   \nsub/e.mtx\r\n  # indented comment\nsynth:C0:3\nb.mtx")
    out = tmp_path / "m.csv"
    assert run([build, data, "spmm", "0", out, "64", "2"], env={"DATASET_LIST": str(man)}) == 0
    assert rows(out)[1:] == [f"PowerSparse,{data / 'sub/e.mtx'},64,0,0,2",
                             "PowerSparse,synth:C0:3,64,0,0,2",
                             f"PowerSparse,{data / 'b.mtx'},64,0,0,2"]


def test_manifest_errors(build, data, tmp_path, capsys):
    out = tmp_path / "m.csv"
    assert run([build, data, "spmm", "0", out], env={"DATASET_LIST": str(tmp_path / "x")}) == 1
    assert "Cannot read manifest:" in capsys.readouterr().err
    man = tmp_path / "list.txt"
    man.write_text("a.mtx\nmissing.mtx\n")
    assert run([build, data, "spmm", "0", out], env={"DATASET_LIST": str(man)}) == 1
    assert "Missing matrix:" in capsys.readouterr().err
    assert not out.exists() and not os.path.exists(str(out) + ".partial")
    man.write_text("# nothing\n\n")
    assert run([build, data, "spmm", "0", out], env={"DATASET_LIST": str(man)}) == 1
    assert "No matrices selected." in capsys.readouterr().err


def test_no_matrices(build, tmp_path, capsys):
    empty = tmp_path / "empty"
    empty.mkdir()
    assert run([build, empty, "spmm", "0", tmp_path / "o.csv"]) == 1
    assert "No matrices selected." in capsys.readouterr().err


def test_refuses_to_overwrite(build, data, tmp_path, capsys):
    out = tmp_path / "o.csv"
    out.write_text("old")
    assert run([build, data, "spmm", "0", out]) == 1
    assert "Output already exists:" in capsys.readouterr().err
    assert out.read_text() == "old"
    out.unlink()
    partial = tmp_path / "o.csv.partial"
    partial.write_text("old")
    assert run([build, data, "spmm", "0", out]) == 1
    assert partial.read_text() == "old" and not out.exists()


def test_failed_run_stays_partial(build, data, tmp_path):
    (data / "bad.mtx").write_text("x")
    out = tmp_path / "o.csv"
    assert run([build, data, "spmm", "0", out, "32"]) == 3
    assert not out.exists()
    lines = rows(tmp_path / "o.csv.partial")
    assert lines == ["algorithm,matrix,N,device,check,repeats",
                     f"PowerSparse,{data / 'a.mtx'},32,0,0,100",
                     f"PowerSparse,{data / 'b.mtx'},32,0,0,100"]


def test_module_entry_point(build, data, tmp_path):
    out = tmp_path / "o.csv"
    env = dict(os.environ)
    env.pop("DATASET_LIST", None)
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-m", "powersparse_amd.cli.run_benchmarks", str(build),
                        str(data), "spmm", "0", str(out), "128"], cwd=root, env=env,
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    assert len(rows(out)) == 4


def test_python_launcher(data, tmp_path, capsys):
    """PS_BENCH_LAUNCHER=python: the in-tree harness library through
    `python -m powersparse_amd.cli`; here (no GPU) the header is written and the
    first run stops at opening the device, so the file stays partial and the
    harness's exit status 1 is returned."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    package = os.path.join(root, "powersparse_amd")
    if not os.path.exists(os.path.join(package, "lib", "libpowersparse_bench.so")):
        pytest.skip("harness library not built")
    out = tmp_path / "o.csv"
    env = {"PS_BENCH_LAUNCHER": "python"}
    try:
        status = run([package, data, "spmm", "0", out, "32"], env=env)
    finally:
        os.environ.pop("PS_BENCH_LAUNCHER", None)
    assert status == 1
    assert not out.exists()
    assert rows(tmp_path / "o.csv.partial")[0].startswith("algorithm,operator,matrix,")


def test_launcher_errors(build, data, tmp_path, capsys):
    try:
        assert run([build, data, "spmm", "0", tmp_path / "o.csv"],
                   env={"PS_BENCH_LAUNCHER": "python"}) == 1
        assert "Missing library:" in capsys.readouterr().err
        assert run([build, data, "spmm", "0", tmp_path / "o.csv"],
                   env={"PS_BENCH_LAUNCHER": "shell"}) == 2
        assert "Unknown PS_BENCH_LAUNCHER: shell" in capsys.readouterr().err
    finally:
        os.environ.pop("PS_BENCH_LAUNCHER", None)
