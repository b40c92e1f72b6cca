// MatrixMarket coordinate reader for the CSV harness.
//
// Design: the file is read into memory once (chunked reads, so a pipe works as
// well as a regular file), scanned line by line in place into a list of
// (row, col, value) entries in file order (a symmetric file's mirror entry
// follows its source entry), and the list is turned into CSR by a stable
// counting sort on the row: per-row counts, a prefix sum, then a scatter in
// list order, which keeps file order inside every row.
//
// Accepted input and error texts are those of the reference harness's reader
// (ParCIS/PowerSparse benchmarks/matrix_market.cpp:12-134), since the CLI
// prints them and scripts match on them:
//   first line "%%MatrixMarket matrix coordinate {pattern|real|integer}
//   {general|symmetric}" (exactly five words); later lines that are blank or
//   start with '%' after leading blanks are skipped; the size line holds three
//   integers; each entry line holds a 1-based row and column (checked against
//   the size before its value is parsed), then an integer (integer files) or a
//   finite real within FP32 range, parsed as double and rounded (real files),
//   or nothing (pattern files, value 1); no field may follow; the file must
//   hold exactly the declared number of entry lines; sizes and the expanded
//   entry count stay below INT32_MAX - 32.
#include "matrix_market.h"

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <limits>
#include <stdexcept>
#include <vector>

namespace PowerSparse {
namespace {

constexpr long long kLimit = std::numeric_limits<int>::max() - 32;

[[noreturn]] void Fail(const char* what) { throw std::runtime_error(what); }

bool Blank(char c) {
  return c == ' ' || c == '\t' || c == '\r' || c == '\n' || c == '\f' || c == '\v';
}

const char* SkipBlanks(const char* p) {
  while (Blank(*p)) ++p;
  return p;
}

// The whole input, split into NUL-terminated lines in place.
class LineBuffer {
 public:
  explicit LineBuffer(const std::string& path) {
    std::ifstream in(path, std::ios::binary);
    if (!in) throw std::runtime_error("Cannot open matrix: " + path);
    constexpr size_t kChunk = size_t(1) << 22;
    for (;;) {
      const size_t at = text_.size();
      text_.resize(at + kChunk);
      in.read(&text_[at], std::streamsize(kChunk));
      text_.resize(at + size_t(in.gcount()));
      if (in.bad()) Fail("Error reading MatrixMarket input");
      if (!in) break;
    }
    text_.push_back('\0');  // the last line ends here if the file lacks a final newline
  }

  size_t Bytes() const { return text_.size() - 1; }

  // The next line (without its newline), or nullptr at the end of the input.
  char* Next() {
    if (pos_ + 1 >= text_.size()) return nullptr;
    char* line = &text_[pos_];
    char* nl = static_cast<char*>(std::memchr(line, '\n', text_.size() - 1 - pos_));
    if (nl) {
      *nl = '\0';
      pos_ = size_t(nl - text_.data()) + 1;
    } else {
      pos_ = text_.size() - 1;
    }
    return line;
  }

  // The next line holding data: neither blank nor a '%' comment.
  char* NextData() {
    while (char* line = Next()) {
      const char* p = SkipBlanks(line);
      if (*p && *p != '%') return line;
    }
    return nullptr;
  }

 private:
  std::string text_;
  size_t pos_ = 0;
};

// Reads one whitespace-delimited integer field.
long long IntField(const char*& p) {
  p = SkipBlanks(p);
  char* end = nullptr;
  errno = 0;
  const long long v = std::strtoll(p, &end, 10);
  if (end == p || errno == ERANGE || (*end && !Blank(*end)))
    Fail("Invalid integer in MatrixMarket input");
  p = end;
  return v;
}

// Reads one real field that must be finite and representable as FP32.
float RealField(const char*& p) {
  p = SkipBlanks(p);
  char* end = nullptr;
  const double v = std::strtod(p, &end);
  if (end == p || (*end && !Blank(*end)) || !std::isfinite(v) ||
      std::fabs(v) > double(std::numeric_limits<float>::max()))
    Fail("Invalid finite FP32 value in MatrixMarket input");
  p = end;
  return float(v);
}

void NoMoreFields(const char* p) {
  if (*SkipBlanks(p)) Fail("Unexpected extra fields in MatrixMarket record");
}

enum class Field { kPattern, kReal, kInteger };

struct Shape {
  int rows = 0, cols = 0;
  long long entries = 0;
  Field field = Field::kPattern;
  bool symmetric = false;
};

// Splits the banner line into whitespace-separated words.
std::vector<std::string> Words(const char* p) {
  std::vector<std::string> out;
  for (p = SkipBlanks(p); *p; p = SkipBlanks(p)) {
    const char* q = p;
    while (*q && !Blank(*q)) ++q;
    out.emplace_back(p, size_t(q - p));
    p = q;
  }
  return out;
}

Shape ReadShape(LineBuffer& lines) {
  const char* banner = lines.Next();
  if (!banner) Fail("Empty MatrixMarket file");
  const std::vector<std::string> w = Words(banner);
  Shape s;
  bool ok = w.size() == 5 && w[0] == "%%MatrixMarket" && w[1] == "matrix" &&
            w[2] == "coordinate";
  if (ok) {
    if (w[3] == "real") s.field = Field::kReal;
    else if (w[3] == "integer") s.field = Field::kInteger;
    else ok = w[3] == "pattern";
  }
  if (ok) {
    s.symmetric = w[4] == "symmetric";
    ok = s.symmetric || w[4] == "general";
  }
  if (!ok) Fail("Expected MatrixMarket coordinate pattern/real/integer general/symmetric");
  const char* p = lines.NextData();
  if (!p) Fail("Missing MatrixMarket dimensions");
  const long long rows = IntField(p), cols = IntField(p), entries = IntField(p);
  NoMoreFields(p);
  if (rows <= 0 || cols <= 0 || entries <= 0 || rows > kLimit || cols > kLimit ||
      entries > kLimit || (s.symmetric && rows != cols))
    Fail("Matrix must be nonempty and fit 32-bit CSR indices");
  s.rows = int(rows);
  s.cols = int(cols);
  s.entries = entries;
  return s;
}

struct Entry {
  int row, col;
  float value;
};

}  // namespace

HostCsr ReadMatrixMarket(const std::string& path) {
  LineBuffer lines(path);
  const Shape s = ReadShape(lines);

  std::vector<Entry> list;
  // an entry line takes at least 4 bytes ("1 1\n"): never reserve beyond the input
  const long long fit = std::min<long long>(s.entries, (long long)(lines.Bytes() / 4 + 1));
  list.reserve(size_t(s.symmetric ? 2 * fit : fit));
  auto add = [&](int r, int c, float v) {
    if ((long long)list.size() + 1 > kLimit) Fail("Expanded matrix exceeds 32-bit CSR capacity");
    list.push_back({r, c, v});
  };
  for (long long e = 0; e < s.entries; ++e) {
    const char* p = lines.NextData();
    if (!p) Fail("Truncated MatrixMarket input");
    const long long r = IntField(p), c = IntField(p);
    if (r < 1 || r > s.rows || c < 1 || c > s.cols)
      Fail("MatrixMarket index outside the declared dimensions");
    float v = 1.0f;
    if (s.field == Field::kInteger) v = float(IntField(p));
    else if (s.field == Field::kReal) v = RealField(p);
    NoMoreFields(p);
    add(int(r) - 1, int(c) - 1, v);
    if (s.symmetric && r != c) add(int(c) - 1, int(r) - 1, v);
  }
  if (lines.NextData()) Fail("More entries than declared in MatrixMarket input");

  // stable counting sort of the list by row
  HostCsr csr;
  csr.rows = s.rows;
  csr.cols = s.cols;
  csr.row_ptr.assign(size_t(s.rows) + 1, 0);
  for (const Entry& e : list) ++csr.row_ptr[size_t(e.row) + 1];
  for (size_t r = 1; r < csr.row_ptr.size(); ++r) csr.row_ptr[r] += csr.row_ptr[r - 1];
  csr.col_ind.resize(list.size());
  csr.values.resize(list.size());
  std::vector<int> fill(csr.row_ptr.begin(), csr.row_ptr.end() - 1);
  for (const Entry& e : list) {
    const size_t at = size_t(fill[size_t(e.row)]++);
    csr.col_ind[at] = e.col;
    csr.values[at] = e.value;
  }
  return csr;
}

}  // namespace PowerSparse
