// TEST INFRASTRUCTURE: a main() around the reference's own ReadMatrixMarket
// (benchmarks/matrix_market.cpp:97-134, compiled from the reference tree) that
// prints the CSR it reads, so tests can compare the product's reader with it.
// Output: "rows cols nnz" then row_ptr, col_ind and the values' IEEE bits in
// hex, one array per line; on a reader error "ERROR <message>" and exit 1.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <exception>

#include "matrix_market.h"

int main(int argc, char** argv) {
  if (argc != 2) {
    std::fprintf(stderr, "usage: %s MATRIX.mtx\n", argv[0]);
    return 2;
  }
  try {
    const CsrMatrix m = ReadMatrixMarket(argv[1]);
    std::printf("%d %d %d\n", m.rows, m.cols, m.nnz());
    for (int v : m.row_ptr) std::printf("%d ", v);
    std::printf("\n");
    for (int v : m.col_ind) std::printf("%d ", v);
    std::printf("\n");
    for (float v : m.values) {
      uint32_t bits;
      std::memcpy(&bits, &v, sizeof(bits));
      std::printf("%08x ", bits);
    }
    std::printf("\n");
  } catch (const std::exception& e) {
    std::printf("ERROR %s\n", e.what());
    return 1;
  }
  return 0;
}
