// Seeded synthetic graphs for the benchmark configurations, and a binary CSR
// file format. Not in the reference, whose inputs are external .mtx files
// (dataset/README.md); the configurations follow the benchmark plan.
//
// Every row draws from its own counter-based random stream (splitmix64 seeded
// from (seed, row)), so a graph is identical for any thread count.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace PowerSparse {

struct HostCsr {
  int rows = 0, cols = 0;
  std::vector<int> row_ptr, col_ind;
  std::vector<float> values;
  int nnz() const { return int(col_ind.size()); }
};

// rows x cols, per-row degree uniform in [deg_lo, deg_hi] (clamped to cols),
// distinct columns uniform without replacement, sorted; values U(val_lo, val_hi).
HostCsr SynthUniformDegree(int rows, int cols, int deg_lo, int deg_hi, float val_lo,
                           float val_hi, uint64_t seed);

// Square Chung-Lu graph: weights w_i = c (i+1)^(-1/(gamma-1)), min(w_i, max_deg),
// with c set so the clipped weights average mean_deg; out-degree of row i is
// Poisson(w_i) (capped at n / 2); endpoints drawn proportional to the same
// weights (alias table), a repeat of a column already in the row drawn again,
// so every row holds exactly its degree of distinct columns, sorted; values
// U(val_lo, val_hi). max_deg must be at most n / 4.
HostCsr SynthChungLu(int n, double gamma, double mean_deg, double max_deg, float val_lo,
                     float val_hi, uint64_t seed);

// Community graph: `communities` blocks of `block` nodes; inside its block a row
// links each node with probability p_intra; plus Poisson(inter_mean) endpoints
// uniform over the other blocks; then a fraction `empty_frac` of rows is emptied
// and a fraction `single_frac` keeps exactly one nonzero. Values U(val_lo, val_hi).
HostCsr SynthCommunity(int communities, int block, double p_intra, double inter_mean,
                       double empty_frac, double single_frac, float val_lo, float val_hi,
                       uint64_t seed);

// Named benchmark configurations, optionally scaled down by `scale` (node
// count divided by scale, degree clip capped at a quarter of the nodes):
//   C0  4096 x 4096, degree U[1,31], values U(-1,1)
//   C1  Chung-Lu n=1e6, gamma 2.1, mean 50, clip 5e4, values U(0,1)
//   C2  the C1 graph (the SDDMM configuration uses C1's pattern)
//   C3  Chung-Lu n=1.6e6, gamma 1.8, mean 165, clip 1e5, values U(0,1)
//   C4  2048 communities x 1024 nodes, intra density 0.02, Poisson(8) inter
//       edges, 5% empty and 5% singleton rows, values U(-1,1)
HostCsr SynthConfig(const std::string& name, uint64_t seed, int scale = 1);

// Binary CSR: "PSCSR001", int64 rows, cols, nnz, then int32 row_ptr[rows+1],
// int32 col_ind[nnz], float32 values[nnz], little endian.
void WriteBinaryCsr(const std::string& path, const HostCsr& csr);
HostCsr ReadBinaryCsr(const std::string& path);

}  // namespace PowerSparse
