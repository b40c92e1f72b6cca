// Seeded synthetic graphs and the binary CSR format (see synth.h).
#include "synth.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <limits>
#include <numeric>
#include <stdexcept>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace PowerSparse {
namespace {

// splitmix64 (Steele, Lea, Flood 2014) as a per-row generator.
inline uint64_t Mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

class RowRng {
 public:
  RowRng(uint64_t seed, uint64_t row) : s_(Mix64(seed ^ Mix64(row + 0x632BE59BD9B4E019ull))) {}
  uint64_t Next() { return Mix64(s_ += 0x9E3779B97F4A7C15ull); }
  double Uniform() { return double(Next() >> 11) * (1.0 / 9007199254740992.0); }  // [0,1)
  float UniformF(float lo, float hi) { return lo + (hi - lo) * float(Uniform()); }
  double Normal() {  // Box-Muller
    const double u1 = (double(Next() >> 11) + 0.5) * (1.0 / 9007199254740992.0);
    const double u2 = Uniform();
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
  }
  int Poisson(double lambda) {
    if (lambda <= 0) return 0;
    if (lambda < 30.0) {  // multiplication method
      const double limit = std::exp(-lambda);
      int k = 0;
      double p = Uniform();
      while (p > limit) {
        ++k;
        p *= Uniform();
      }
      return k;
    }
    const double x = std::floor(lambda + std::sqrt(lambda) * Normal() + 0.5);
    return x < 0 ? 0 : int(std::min(x, 2.0e9));
  }

 private:
  uint64_t s_;
};

// Walker / Vose alias table for sampling indices proportional to weights.
struct AliasTable {
  std::vector<double> prob;
  std::vector<int> alias;
  explicit AliasTable(const std::vector<double>& w) {
    const size_t n = w.size();
    prob.assign(n, 0.0);
    alias.assign(n, 0);
    const double total = std::accumulate(w.begin(), w.end(), 0.0);
    std::vector<double> scaled(n);
    std::vector<int> small, large;
    small.reserve(n);
    large.reserve(n);
    for (size_t i = 0; i < n; ++i) {
      scaled[i] = w[i] * double(n) / total;
      (scaled[i] < 1.0 ? small : large).push_back(int(i));
    }
    while (!small.empty() && !large.empty()) {
      const int s = small.back(), l = large.back();
      small.pop_back();
      prob[size_t(s)] = scaled[size_t(s)];
      alias[size_t(s)] = l;
      scaled[size_t(l)] -= 1.0 - scaled[size_t(s)];
      if (scaled[size_t(l)] < 1.0) {
        large.pop_back();
        small.push_back(l);
      }
    }
    for (int i : large) prob[size_t(i)] = 1.0;
    for (int i : small) prob[size_t(i)] = 1.0;
  }
  int Sample(RowRng& rng) const {
    const size_t n = prob.size();
    size_t i = size_t(rng.Uniform() * double(n));
    if (i >= n) i = n - 1;
    return rng.Uniform() < prob[i] ? int(i) : alias[i];
  }
};

// Generates rows in parallel chunks and concatenates them into a CSR.
// gen(row, rng, cols_out, vals_out) appends the row's sorted entries.
template <typename Gen>
HostCsr BuildRows(int rows, int cols, uint64_t seed, Gen gen) {
  constexpr int kChunk = 2048;
  const int chunks = (rows + kChunk - 1) / kChunk;
  std::vector<std::vector<int>> ccols(static_cast<size_t>(chunks)), clen(static_cast<size_t>(chunks));
  std::vector<std::vector<float>> cvals(static_cast<size_t>(chunks));
#pragma omp parallel for schedule(dynamic, 1)
  for (int c = 0; c < chunks; ++c) {
    std::vector<int> rc;
    std::vector<float> rv;
    const int r0 = c * kChunk, r1 = std::min(rows, r0 + kChunk);
    clen[size_t(c)].resize(size_t(r1 - r0));
    for (int r = r0; r < r1; ++r) {
      RowRng rng(seed, uint64_t(r));
      rc.clear();
      rv.clear();
      gen(r, rng, rc, rv);
      clen[size_t(c)][size_t(r - r0)] = int(rc.size());
      ccols[size_t(c)].insert(ccols[size_t(c)].end(), rc.begin(), rc.end());
      cvals[size_t(c)].insert(cvals[size_t(c)].end(), rv.begin(), rv.end());
    }
  }
  HostCsr csr;
  csr.rows = rows;
  csr.cols = cols;
  csr.row_ptr.assign(size_t(rows) + 1, 0);
  std::vector<size_t> chunk_off(static_cast<size_t>(chunks) + 1, 0);
  for (int c = 0; c < chunks; ++c) chunk_off[size_t(c) + 1] = chunk_off[size_t(c)] + ccols[size_t(c)].size();
  if (chunk_off.back() > size_t(std::numeric_limits<int>::max() - 32))
    throw std::runtime_error("Synthetic graph exceeds 32-bit CSR capacity");
  for (int c = 0; c < chunks; ++c)
    for (size_t i = 0; i < clen[size_t(c)].size(); ++i) {
      const int r = c * kChunk + int(i);
      csr.row_ptr[size_t(r) + 1] = clen[size_t(c)][i];
    }
  for (int r = 0; r < rows; ++r) csr.row_ptr[size_t(r) + 1] += csr.row_ptr[size_t(r)];
  csr.col_ind.resize(chunk_off.back());
  csr.values.resize(chunk_off.back());
#pragma omp parallel for schedule(static)
  for (int c = 0; c < chunks; ++c) {
    std::copy(ccols[size_t(c)].begin(), ccols[size_t(c)].end(), csr.col_ind.begin() + long(chunk_off[size_t(c)]));
    std::copy(cvals[size_t(c)].begin(), cvals[size_t(c)].end(), csr.values.begin() + long(chunk_off[size_t(c)]));
  }
  return csr;
}

// Open-addressing set of non-negative ints sized for `expected` members.
class DistinctSet {
 public:
  explicit DistinctSet(int expected) {
    size_t cap = 16;
    while (cap < 2 * size_t(expected)) cap <<= 1;
    slots_.assign(cap, -1);
    mask_ = cap - 1;
  }
  // Adds v; false when it was already present.
  bool Insert(int v) {
    for (size_t h = (uint32_t(v) * 0x9E3779B1u) & mask_;; h = (h + 1) & mask_) {
      if (slots_[h] == v) return false;
      if (slots_[h] < 0) {
        slots_[h] = v;
        return true;
      }
    }
  }

 private:
  std::vector<int> slots_;
  size_t mask_;
};

void SortUnique(std::vector<int>& v) {
  std::sort(v.begin(), v.end());
  v.erase(std::unique(v.begin(), v.end()), v.end());
}

}  // namespace

HostCsr SynthUniformDegree(int rows, int cols, int deg_lo, int deg_hi, float val_lo,
                           float val_hi, uint64_t seed) {
  if (rows <= 0 || cols <= 0 || deg_lo < 0 || deg_hi < deg_lo)
    throw std::invalid_argument("SynthUniformDegree: bad shape or degree range");
  return BuildRows(rows, cols, seed, [&](int, RowRng& rng, std::vector<int>& rc,
                                         std::vector<float>& rv) {
    int d = deg_lo + int(rng.Uniform() * double(deg_hi - deg_lo + 1));
    d = std::min(std::min(d, deg_hi), cols);
    // Floyd's sampling of d distinct columns.
    for (int j = cols - d; j < cols; ++j) {
      const int t = int(rng.Uniform() * double(j + 1));
      if (std::find(rc.begin(), rc.end(), t) == rc.end()) rc.push_back(t);
      else rc.push_back(j);
    }
    std::sort(rc.begin(), rc.end());
    for (size_t i = 0; i < rc.size(); ++i) rv.push_back(rng.UniformF(val_lo, val_hi));
  });
}

HostCsr SynthChungLu(int n, double gamma, double mean_deg, double max_deg, float val_lo,
                     float val_hi, uint64_t seed) {
  if (n <= 0 || gamma <= 1.0 || mean_deg <= 0 || max_deg <= 0 || max_deg > std::max(1.0, n / 4.0))
    throw std::invalid_argument("SynthChungLu: bad parameters");
  const double alpha = 1.0 / (gamma - 1.0);
  std::vector<double> base(static_cast<size_t>(n));
  for (int i = 0; i < n; ++i) base[size_t(i)] = std::pow(double(i) + 1.0, -alpha);
  auto mean_for = [&](double c) {
    double s = 0;
    for (int i = 0; i < n; ++i) s += std::min(c * base[size_t(i)], max_deg);
    return s / n;
  };
  double lo = 0, hi = max_deg;
  while (mean_for(hi) < mean_deg && hi < 1e300) hi *= 2;
  for (int it = 0; it < 200; ++it) {
    const double mid = 0.5 * (lo + hi);
    (mean_for(mid) < mean_deg ? lo : hi) = mid;
  }
  std::vector<double> w(static_cast<size_t>(n));
  for (int i = 0; i < n; ++i) w[size_t(i)] = std::min(hi * base[size_t(i)], max_deg);
  const AliasTable table(w);
  return BuildRows(n, n, seed, [&](int r, RowRng& rng, std::vector<int>& rc,
                                   std::vector<float>& rv) {
    // The row keeps its Poisson degree: endpoints that repeat one already
    // drawn are drawn again, so hub columns do not thin out heavy rows.
    const int d = std::min(rng.Poisson(w[size_t(r)]), n / 2);
    DistinctSet seen(d);
    rc.reserve(size_t(d));
    while (int(rc.size()) < d) {
      const int c = table.Sample(rng);
      if (seen.Insert(c)) rc.push_back(c);
    }
    std::sort(rc.begin(), rc.end());
    for (size_t i = 0; i < rc.size(); ++i) rv.push_back(rng.UniformF(val_lo, val_hi));
  });
}

HostCsr SynthCommunity(int communities, int block, double p_intra, double inter_mean,
                       double empty_frac, double single_frac, float val_lo, float val_hi,
                       uint64_t seed) {
  if (communities <= 0 || block <= 0 || p_intra < 0 || p_intra >= 1 || inter_mean < 0)
    throw std::invalid_argument("SynthCommunity: bad parameters");
  const long long n64 = (long long)communities * block;
  if (n64 > std::numeric_limits<int>::max() - 32)
    throw std::invalid_argument("SynthCommunity: too many nodes");
  const int n = int(n64);
  const double log_q = std::log1p(-p_intra);
  return BuildRows(n, n, seed, [&](int r, RowRng& rng, std::vector<int>& rc,
                                   std::vector<float>& rv) {
    const int c = r / block;
    if (p_intra > 0) {  // geometric skips over the block
      long long j = -1;
      for (;;) {
        const double u = 1.0 - rng.Uniform();  // (0, 1]
        j += 1 + (long long)std::floor(std::log(u) / log_q);
        if (j >= block) break;
        rc.push_back(c * block + int(j));
      }
    }
    if (communities > 1) {
      const int k = rng.Poisson(inter_mean);
      for (int e = 0; e < k; ++e) {
        int other = int(rng.Uniform() * double(communities - 1));
        if (other >= communities - 1) other = communities - 2;
        if (other >= c) ++other;
        int node = int(rng.Uniform() * double(block));
        if (node >= block) node = block - 1;
        rc.push_back(other * block + node);
      }
    }
    SortUnique(rc);
    const double u = rng.Uniform();
    if (u < empty_frac) {
      rc.clear();
    } else if (u < empty_frac + single_frac) {
      if (rc.empty()) {
        int node = int(rng.Uniform() * double(block));
        if (node >= block) node = block - 1;
        rc.push_back(c * block + node);
      } else {
        size_t keep = size_t(rng.Uniform() * double(rc.size()));
        if (keep >= rc.size()) keep = rc.size() - 1;
        const int v = rc[keep];
        rc.assign(1, v);
      }
    }
    for (size_t i = 0; i < rc.size(); ++i) rv.push_back(rng.UniformF(val_lo, val_hi));
  });
}

HostCsr SynthConfig(const std::string& name, uint64_t seed, int scale) {
  if (scale < 1) throw std::invalid_argument("scale must be >= 1");
  auto clip = [&](double max_deg, int n) { return std::min(max_deg, std::max(1.0, n / 4.0)); };
  if (name == "C0") return SynthUniformDegree(4096 / scale, 4096 / scale, 1, 31, -1.f, 1.f, seed);
  if (name == "C1" || name == "C2") {
    const int n = 1000000 / scale;
    return SynthChungLu(n, 2.1, 50.0, clip(50000.0, n), 0.f, 1.f, seed);
  }
  if (name == "C3") {
    const int n = 1600000 / scale;
    return SynthChungLu(n, 1.8, 165.0, clip(100000.0, n), 0.f, 1.f, seed);
  }
  if (name == "C4")
    return SynthCommunity(std::max(2, 2048 / scale), 1024, 0.02, 8.0, 0.05, 0.05, -1.f, 1.f,
                          seed);
  throw std::invalid_argument("Unknown synthetic configuration: " + name);
}

void WriteBinaryCsr(const std::string& path, const HostCsr& csr) {
  std::ofstream out(path, std::ios::binary);
  if (!out) throw std::runtime_error("Cannot write " + path);
  const char magic[8] = {'P', 'S', 'C', 'S', 'R', '0', '0', '1'};
  const int64_t dims[3] = {csr.rows, csr.cols, int64_t(csr.col_ind.size())};
  out.write(magic, 8);
  out.write(reinterpret_cast<const char*>(dims), sizeof(dims));
  out.write(reinterpret_cast<const char*>(csr.row_ptr.data()), std::streamsize(csr.row_ptr.size() * sizeof(int)));
  out.write(reinterpret_cast<const char*>(csr.col_ind.data()), std::streamsize(csr.col_ind.size() * sizeof(int)));
  out.write(reinterpret_cast<const char*>(csr.values.data()), std::streamsize(csr.values.size() * sizeof(float)));
  if (!out) throw std::runtime_error("Error writing " + path);
}

HostCsr ReadBinaryCsr(const std::string& path) {
  std::ifstream in(path, std::ios::binary);
  if (!in) throw std::runtime_error("Cannot open matrix: " + path);
  char magic[8];
  int64_t dims[3];
  in.read(magic, 8);
  in.read(reinterpret_cast<char*>(dims), sizeof(dims));
  if (!in || std::memcmp(magic, "PSCSR001", 8) != 0)
    throw std::runtime_error("Not a PSCSR001 binary CSR file: " + path);
  const int64_t limit = std::numeric_limits<int>::max() - 32;
  if (dims[0] <= 0 || dims[1] <= 0 || dims[2] < 0 || dims[0] > limit || dims[1] > limit ||
      dims[2] > limit)
    throw std::runtime_error("Binary CSR dimensions out of range");
  HostCsr csr;
  csr.rows = int(dims[0]);
  csr.cols = int(dims[1]);
  csr.row_ptr.resize(size_t(dims[0]) + 1);
  csr.col_ind.resize(size_t(dims[2]));
  csr.values.resize(size_t(dims[2]));
  in.read(reinterpret_cast<char*>(csr.row_ptr.data()), std::streamsize(csr.row_ptr.size() * sizeof(int)));
  in.read(reinterpret_cast<char*>(csr.col_ind.data()), std::streamsize(csr.col_ind.size() * sizeof(int)));
  in.read(reinterpret_cast<char*>(csr.values.data()), std::streamsize(csr.values.size() * sizeof(float)));
  if (!in) throw std::runtime_error("Truncated binary CSR file: " + path);
  if (csr.row_ptr[0] != 0 || csr.row_ptr.back() != int(dims[2]))
    throw std::runtime_error("Binary CSR row pointers are inconsistent");
  return csr;
}

}  // namespace PowerSparse
