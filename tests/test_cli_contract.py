"""The benchmark binaries' argument contract on the CPU (no device is opened on
these paths): --header, usage, an unselected N, and argument errors, with the
reference harness's texts and exit codes (benchmarks/benchmark.cu:98-213)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = ("algorithm,operator,matrix,rows,cols,nnz,N,device,gpu,compute_capability,"
          "cuda_runtime,cuda_driver,warmup,repeats,seed,check,preprocess_ms,ms,gflops")


def run(op, *args):
    exe = os.path.join(ROOT, "powersparse_amd", "bin", f"powersparse_{op}")
    if not os.path.exists(exe):
        pytest.skip("CLI binaries not built")
    return subprocess.run([exe] + [str(a) for a in args], capture_output=True, text=True,
                          timeout=60)


@pytest.mark.parametrize("op", ["spmm", "sddmm"])
def test_header_and_usage(op):
    r = run(op, "--header")
    assert r.returncode == 0 and r.stdout.strip() == HEADER
    r = run(op)
    assert r.returncode == 2 and r.stderr.startswith("Usage: ")
    assert "MATRIX N DEVICE CHECK REPEATS" in r.stderr
    r = run(op, "a.mtx", 32, 0)
    assert r.returncode == 2 and "Usage: " in r.stderr


@pytest.mark.parametrize("op,name", [("spmm", "SpMM"), ("sddmm", "SDDMM")])
def test_unselected_width(op, name):
    for n in (48, 256, 16):
        r = run(op, "synth:C0", n, 0, 0, 1)
        assert r.returncode == 2
        assert r.stderr.strip() == (f"{name} benchmark: N={n} was not selected in main; "
                                    "please use N=32, 64 or 128.")


@pytest.mark.parametrize("args,message", [
    (("synth:C0", 32, 0, 2, 1), "Error: DEVICE must be nonnegative, CHECK 0 or 1, and REPEATS positive"),
    (("synth:C0", 32, -1, 0, 1), "Error: DEVICE must be nonnegative, CHECK 0 or 1, and REPEATS positive"),
    (("synth:C0", 32, 0, 0, 0), "Error: DEVICE must be nonnegative, CHECK 0 or 1, and REPEATS positive"),
    (("synth:C0", "x32", 0, 0, 1), "Error: Invalid N: x32"),
    (("synth:C0", "32x", 0, 0, 1), "Error: Invalid N"),
    (("synth:C0", 32, "zero", 0, 1), "Error: Invalid DEVICE: zero"),
    (("synth:C0", 32, 0, 0, "1.5"), "Error: Invalid REPEATS"),
])
def test_argument_errors(args, message):
    r = run("spmm", *args)
    assert r.returncode == 1 and r.stderr.strip() == message


def run_python(*args):
    """The same harness through the Python launcher (python -m powersparse_amd.cli)."""
    if not os.path.exists(os.path.join(ROOT, "powersparse_amd", "lib", "libpowersparse_bench.so")):
        pytest.skip("harness library not built")
    return subprocess.run(["python", "-m", "powersparse_amd.cli"] + [str(a) for a in args],
                          capture_output=True, text=True, timeout=120, cwd=ROOT)


@pytest.mark.parametrize("op,name", [("spmm", "SpMM"), ("sddmm", "SDDMM")])
def test_python_launcher_contract(op, name):
    r = run_python(op, "--header")
    assert r.returncode == 0 and r.stdout.strip() == HEADER
    r = run_python(op)
    assert r.returncode == 2 and r.stderr.startswith("Usage: powersparse_")
    r = run_python(op, "synth:C0", 48, 0, 0, 1)
    assert r.returncode == 2
    assert r.stderr.strip() == (f"{name} benchmark: N=48 was not selected in main; "
                                "please use N=32, 64 or 128.")
    r = run_python(op, "synth:C0", 32, 0, 2, 1)
    assert r.returncode == 1 and r.stderr.strip() == (
        "Error: DEVICE must be nonnegative, CHECK 0 or 1, and REPEATS positive")
    r = run_python("gemm")
    assert r.returncode == 2 and "python -m powersparse_amd.cli {spmm|sddmm}" in r.stderr
