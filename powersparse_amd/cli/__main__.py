"""The CSV benchmark from a Python process:

    python -m powersparse_amd.cli {spmm|sddmm} MATRIX N DEVICE CHECK REPEATS
    python -m powersparse_amd.cli {spmm|sddmm} --header

runs the harness behind powersparse_amd/bin/powersparse_{spmm,sddmm}
(psx_bench_main in lib/libpowersparse_bench.so, include/powersparse_bench.h)
with the same arguments, CSV header and row on stdout, messages on stderr and
exit codes (0 success, 1 error, 2 usage or an unselected N), the contract of
the reference's benchmarks/benchmark.cu:98-213. The process ends through
Python's own exit path, as every process that loads the libraries through
the package does. The batch runner (run_benchmarks.py) uses this launcher
when PS_BENCH_LAUNCHER=python.
"""
import ctypes
import sys

OPS = {"spmm": 0, "sddmm": 1}  # PSX_BENCH_SPMM, PSX_BENCH_SDDMM

USAGE = ("Usage: python -m powersparse_amd.cli {spmm|sddmm} MATRIX N DEVICE CHECK REPEATS\n"
         "       python -m powersparse_amd.cli {spmm|sddmm} --header")


def main(argv=None):
    argv = sys.argv[1:] if argv is None else list(argv)
    if not argv or argv[0] not in OPS:
        print(USAGE, file=sys.stderr)
        return 2
    from powersparse_amd import _native

    op = argv[0]
    args = [f"powersparse_{op}".encode()] + [a.encode() for a in argv[1:]]
    arr = (ctypes.c_char_p * (len(args) + 1))(*args, None)
    libc = ctypes.CDLL(None)
    # the harness writes to the process's file descriptors through C stdio and
    # iostreams: Python's buffers go first, the C library's are flushed after
    sys.stdout.flush()
    sys.stderr.flush()
    rc = _native.bench().psx_bench_main(OPS[op], len(args), arr)
    libc.fflush(None)
    return rc


if __name__ == "__main__":
    sys.exit(main())
