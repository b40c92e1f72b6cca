/* The CSV benchmark harness of the MI355X PowerSparse build
 * (lib/libpowersparse_bench.so), the code behind the powersparse_spmm and
 * powersparse_sddmm command lines.
 *
 * Replaces: main() of the reference's benchmark binaries
 * (benchmarks/benchmark.cu:98-213, with benchmark_utils.h:13-115 and
 * matrix_market.cpp:12-134), the same contract: argv holds the program name
 * and MATRIX N DEVICE CHECK REPEATS (or --header); the CSV header or row goes
 * to stdout, messages to stderr; the return value is the process exit code
 * (0 success, 1 error with "Error: ..." on stderr, 2 usage or an unselected
 * N). As a library call the harness can also run inside a caller's process. */
#ifndef POWERSPARSE_BENCH_H
#define POWERSPARSE_BENCH_H

#ifdef __cplusplus
extern "C" {
#endif

#define PSX_BENCH_SPMM 0
#define PSX_BENCH_SDDMM 1

/* op: PSX_BENCH_SPMM or PSX_BENCH_SDDMM. */
int psx_bench_main(int op, int argc, char** argv);

#ifdef __cplusplus
}
#endif

#endif
