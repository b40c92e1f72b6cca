// powersparse_spmm / powersparse_sddmm: the CSV benchmark command lines, thin
// wrappers of the harness in lib/libpowersparse_bench.so (cli/harness.cpp).
#include "powersparse_bench.h"

#ifndef POWERSPARSE_BENCH_OP
#define POWERSPARSE_BENCH_OP PSX_BENCH_SPMM
#endif

int main(int argc, char** argv) { return psx_bench_main(POWERSPARSE_BENCH_OP, argc, argv); }
