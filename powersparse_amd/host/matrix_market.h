// MatrixMarket coordinate reader (reference semantics: benchmarks/matrix_market.h:1-14).
#pragma once

#include <string>

#include "synth.h"

namespace PowerSparse {

// Reads a coordinate MatrixMarket file into a host CSR; throws std::runtime_error
// with the reference reader's messages on malformed input.
HostCsr ReadMatrixMarket(const std::string& path);

}  // namespace PowerSparse
