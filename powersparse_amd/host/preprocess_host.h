// Host-side steps of the preprocessing that stay on the CPU, as in the reference.
#pragma once

namespace PowerSparse {

// GenerateSigBit in FFC mode (utils/matrix_utils.cu:65-128): column signature
// bits for ffc leading columns; returns the signature length L (a multiple of 32).
int GenerateSigBitFFC(int cols, const int* col_nnz, int ffc, int* sigbit);

// AnalyzeMatrix's workset count (utils/matrix_utils.cu:31-63) from
// degree_sums[s] = sum over rows of floor(deg / GROUP_SIZE(s)), s = 1..31.
int WorksetCount(const unsigned long long* degree_sums, int cu_count);

}  // namespace PowerSparse
