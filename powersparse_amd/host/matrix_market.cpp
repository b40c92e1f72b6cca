// MatrixMarket coordinate reader with the reference harness's semantics
// (ParCIS/PowerSparse benchmarks/matrix_market.cpp:12-134):
//   banner "%%MatrixMarket matrix coordinate {pattern|real|integer}
//   {general|symmetric}"; '%' lines and blank lines skipped; 1-based indices
//   checked against the declared size; pattern -> 1.0f, integer -> float,
//   real -> strtod then float (finite, within FP32 range); symmetric input
//   mirrors every off-diagonal entry; two passes over the file (count, then
//   fill) so entries keep file order inside each row; 32-bit CSR limits.
// Error texts match the reference's, since the CLI prints them.
#include "matrix_market.h"

#include <cerrno>
#include <cmath>
#include <cstdlib>
#include <fstream>
#include <limits>
#include <sstream>
#include <stdexcept>

namespace PowerSparse {
namespace {

constexpr long long kMaxIndex = std::numeric_limits<int>::max() - 32;

inline bool IsBlank(char c) {
  return c == ' ' || c == '\t' || c == '\r' || c == '\n' || c == '\f' || c == '\v';
}

// Next line that is neither blank nor a comment.
bool NextRecord(std::istream& in, std::string& line) {
  while (std::getline(in, line)) {
    size_t i = 0;
    while (i < line.size() && IsBlank(line[i])) ++i;
    if (i < line.size() && line[i] != '%') return true;
  }
  if (in.bad()) throw std::runtime_error("Error reading MatrixMarket input");
  return false;
}

class Fields {
 public:
  explicit Fields(const std::string& line) : p_(line.c_str()) {}
  long long Int() {
    Skip();
    errno = 0;
    char* end = nullptr;
    const long long v = std::strtoll(p_, &end, 10);
    if (end == p_ || errno == ERANGE || (*end && !IsBlank(*end)))
      throw std::runtime_error("Invalid integer in MatrixMarket input");
    p_ = end;
    return v;
  }
  float Real() {
    Skip();
    char* end = nullptr;
    const double v = std::strtod(p_, &end);
    if (end == p_ || (*end && !IsBlank(*end)) || !std::isfinite(v) ||
        std::fabs(v) > double(std::numeric_limits<float>::max()))
      throw std::runtime_error("Invalid finite FP32 value in MatrixMarket input");
    p_ = end;
    return float(v);
  }
  void End() {
    Skip();
    if (*p_) throw std::runtime_error("Unexpected extra fields in MatrixMarket record");
  }

 private:
  void Skip() {
    while (IsBlank(*p_)) ++p_;
  }
  const char* p_;
};

struct Banner {
  long long rows = 0, cols = 0, entries = 0;
  std::string field, symmetry;
};

Banner ParseBanner(std::istream& in) {
  std::string line;
  if (!std::getline(in, line)) throw std::runtime_error("Empty MatrixMarket file");
  std::istringstream words(line);
  std::string magic, object, format, field, symmetry, extra;
  const bool five = bool(words >> magic >> object >> format >> field >> symmetry);
  if (!five || (words >> extra) || magic != "%%MatrixMarket" || object != "matrix" ||
      format != "coordinate" || (field != "pattern" && field != "real" && field != "integer") ||
      (symmetry != "general" && symmetry != "symmetric"))
    throw std::runtime_error(
        "Expected MatrixMarket coordinate pattern/real/integer general/symmetric");
  if (!NextRecord(in, line)) throw std::runtime_error("Missing MatrixMarket dimensions");
  Fields f(line);
  Banner b;
  b.rows = f.Int();
  b.cols = f.Int();
  b.entries = f.Int();
  f.End();
  b.field = field;
  b.symmetry = symmetry;
  if (b.rows <= 0 || b.cols <= 0 || b.entries <= 0 || b.rows > kMaxIndex || b.cols > kMaxIndex ||
      b.entries > kMaxIndex || (symmetry == "symmetric" && b.rows != b.cols))
    throw std::runtime_error("Matrix must be nonempty and fit 32-bit CSR indices");
  return b;
}

template <typename Sink>
void ForEachEntry(std::istream& in, const Banner& b, Sink sink) {
  std::string line;
  const bool symmetric = b.symmetry == "symmetric";
  for (long long e = 0; e < b.entries; ++e) {
    if (!NextRecord(in, line)) throw std::runtime_error("Truncated MatrixMarket input");
    Fields f(line);
    const long long r = f.Int(), c = f.Int();
    if (r < 1 || r > b.rows || c < 1 || c > b.cols)
      throw std::runtime_error("MatrixMarket index outside the declared dimensions");
    float v = 1.0f;
    if (b.field == "integer") v = float(f.Int());
    else if (b.field == "real") v = f.Real();
    f.End();
    sink(int(r - 1), int(c - 1), v);
    if (symmetric && r != c) sink(int(c - 1), int(r - 1), v);
  }
  if (NextRecord(in, line))
    throw std::runtime_error("More entries than declared in MatrixMarket input");
}

}  // namespace

HostCsr ReadMatrixMarket(const std::string& path) {
  std::ifstream in(path);
  if (!in) throw std::runtime_error("Cannot open matrix: " + path);
  const Banner b = ParseBanner(in);
  HostCsr csr;
  csr.rows = int(b.rows);
  csr.cols = int(b.cols);
  csr.row_ptr.assign(size_t(b.rows) + 1, 0);
  long long count = 0;
  ForEachEntry(in, b, [&](int r, int, float) {
    if (++count > kMaxIndex) throw std::runtime_error("Expanded matrix exceeds 32-bit CSR capacity");
    ++csr.row_ptr[size_t(r) + 1];
  });
  for (int r = 0; r < csr.rows; ++r) csr.row_ptr[size_t(r) + 1] += csr.row_ptr[size_t(r)];
  csr.col_ind.resize(size_t(count));
  csr.values.resize(size_t(count));
  std::vector<int> next(csr.row_ptr.begin(), csr.row_ptr.end() - 1);

  in.clear();
  in.seekg(0);
  if (!in) throw std::runtime_error("Matrix input must be a seekable regular file");
  const Banner again = ParseBanner(in);
  if (again.rows != b.rows || again.cols != b.cols || again.entries != b.entries ||
      again.field != b.field || again.symmetry != b.symmetry)
    throw std::runtime_error("Matrix header changed between reader passes");
  ForEachEntry(in, b, [&](int r, int c, float v) {
    const int at = next[size_t(r)]++;
    if (at >= csr.row_ptr[size_t(r) + 1])
      throw std::runtime_error("Matrix row counts changed between reader passes");
    csr.col_ind[size_t(at)] = c;
    csr.values[size_t(at)] = v;
  });
  for (int r = 0; r < csr.rows; ++r)
    if (next[size_t(r)] != csr.row_ptr[size_t(r) + 1])
      throw std::runtime_error("Matrix row counts changed between reader passes");
  return csr;
}

}  // namespace PowerSparse
