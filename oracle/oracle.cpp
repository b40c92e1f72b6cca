// TEST INFRASTRUCTURE — CPU oracle for the PowerSparse hot path. See oracle.h.
// Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it,
// and only as the checker; the product never does.
//
// Each function cites the reference (ParCIS/PowerSparse) file:line it restates.
#include "oracle.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <limits>
#include <numeric>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

// GROUP_SIZE(I) = 32 * 2^(I-1)   (utils/matrix_utils.h:8)
inline int GroupSize(int s) { return 32 * (1 << (s - 1)); }
// CEIL / FLOOR (utils/matrix_utils.h:9-10)
inline int CeilDiv(int x, int y) { return x / y + (x % y != 0); }

int AnalyzeS(int rows, const int* rp, int cu_count) {
  // matrix_utils.cu:37-53: threshold = max_TB_per_SM(8) * SMs * 4; S counts the
  // group sizes 32, 64, ... whose total floor(deg / size) reaches the threshold,
  // plus one for the residue workset.
  const long long threshold = 8LL * cu_count * 4;
  int S = 0;
  long long groups = threshold + 1;
  for (; groups >= threshold; S++) {
    const long long size = 32LL << S;  // GROUP_SIZE(S + 1)
    groups = 0;
    for (int r = 0; r < rows; ++r) groups += (rp[r + 1] - rp[r]) / size;
  }
  return S;
}

// GenerateSigBit, FFC branch (matrix_utils.cu:65-75, 91-128). The column order is
// the libstdc++ std::sort of iota by col_nnz descending: the same unstable sort,
// comparator and input as the reference, so equal counts land in the same order.
int SigBits(int cols, const int* col_nnz, int ffc, int* sigbit) {
  std::vector<int> order(cols);
  std::iota(order.begin(), order.end(), 0);
  std::sort(order.begin(), order.end(),
            [col_nnz](const int& a, const int& b) { return col_nnz[a] > col_nnz[b]; });
  int index = 0, bit = 0, first_mass = 0;
  while (index < std::min(ffc, cols)) {  // the ffc most frequent columns share bit 0
    sigbit[order[index]] = bit;
    first_mass += col_nnz[order[index]];
    ++index;
  }
  ++bit;
  while (index < cols) {  // later buckets take columns while their mass stays below
    int mass = 0;
    const int begin = index;
    while (index < cols) {
      mass += col_nnz[order[index]];
      if (mass < first_mass || index == begin) {
        sigbit[order[index]] = bit;
        ++index;
      } else {
        break;
      }
    }
    ++bit;
  }
  int len = bit;  // rounding of matrix_utils.cu:120-122
  if (len < 32) len = 32;
  else if (len % 32 < 16) len = len / 32 * 32;
  else len = CeilDiv(len, 32) * 32;
  for (int c = 0; c < cols; ++c)  // clamp (matrix_utils.cu:123-127)
    if (sigbit[c] >= len) sigbit[c] = len - 1;
  return len;
}

// Stable order of groups by signature, descending, read as one bit string with
// bit b at word b / 32, position 31 - b % 32 (matrix_utils.cu:286-290): bit 0 is
// the most significant. A larger string has a 1 where the other first differs,
// so the order is that of each group's ascending list of distinct bits,
// compared lexicographically ascending, a list's end ranking after every bit;
// equal lists keep group order (the stable sorts of :590-592 start from iota).
// `bits[g]` may hold duplicates, in any order; it is sorted in place.
std::vector<int> OrderByBitLists(std::vector<std::vector<int>>& bits) {
  for (auto& b : bits) {
    std::sort(b.begin(), b.end());
    b.erase(std::unique(b.begin(), b.end()), b.end());
  }
  std::vector<int> perm(bits.size());
  std::iota(perm.begin(), perm.end(), 0);
  std::stable_sort(perm.begin(), perm.end(), [&bits](int x, int y) {
    const std::vector<int>& a = bits[size_t(x)];
    const std::vector<int>& b = bits[size_t(y)];
    const size_t n = std::min(a.size(), b.size());
    for (size_t i = 0; i < n; ++i)
      if (a[i] != b[i]) return a[i] < b[i];
    return a.size() > b.size();  // the shorter list ends first: it ranks after
  });
  return perm;
}

// 0: bitmaps while groups x words stays below kBitmapLimit words, else lists;
// 1: always the per-word sorts of the bitmaps; 2: always the bit lists.
int g_order_mode = 0;
int g_max_group_types = 0;  // cap on S, 0: none
constexpr size_t kBitmapLimit = size_t(1) << 28;

}  // namespace

struct or_worksets {
  int rows = 0, cols = 0, nnz = 0, S = 0, fine = 16, sig_len = 32;
  std::vector<int> group_num;
  std::vector<std::vector<int>> col, des, init_des, perm;
  std::vector<std::vector<float>> val;
  std::vector<std::vector<uint32_t>> signature;  // word-major per workset
  std::vector<int> residue_offset, init_residue_offset;
  std::vector<uint8_t> residue_atomic, init_residue_atomic;
  std::vector<int> col_nnz, ranked, sigbit;
};

extern "C" {

int or_analyze_group_type_num(int rows, const int* row_ptr, int cu_count) {
  return AnalyzeS(rows, row_ptr, cu_count);
}

int or_generate_sigbit(int cols, const int* col_nnz, int ffc, int* sigbit) {
  return SigBits(cols, col_nnz, ffc, sigbit);
}

void or_set_signature_order(int mode) { g_order_mode = mode; }
void or_set_max_group_types(int cap) { g_max_group_types = cap; }

void or_order_bit_lists(int groups, const int* begin, const int* bits, int* perm) {
  std::vector<std::vector<int>> b(static_cast<size_t>(groups));
  for (int g = 0; g < groups; ++g) b[size_t(g)].assign(bits + begin[g], bits + begin[g + 1]);
  const std::vector<int> p = OrderByBitLists(b);
  std::copy(p.begin(), p.end(), perm);
}

or_worksets* or_preprocess(int rows, int cols, int nnz, const int* rp, const int* ci,
                           const float* sv, int cu_count, char* err, int err_len) {
  auto fail = [&](const char* msg) -> or_worksets* {
    if (err && err_len > 0) std::snprintf(err, size_t(err_len), "%s", msg);
    return nullptr;
  };
  // Input validation, same order and messages as matrix_utils.cu:475-488.
  if (rows <= 0 || cols <= 0 || nnz <= 0 || rows > std::numeric_limits<int>::max() - 32 ||
      nnz > std::numeric_limits<int>::max() - 32 || !rp || !ci || !sv)
    return fail("Expected a nonempty CSR matrix with 32-bit indices");
  if (rp[0] != 0 || rp[rows] != nnz) return fail("Invalid CSR row-pointer endpoints");
  for (int r = 0; r < rows; ++r)
    if (rp[r] < 0 || rp[r] > rp[r + 1]) return fail("CSR row pointers must be nondecreasing");
  for (int p = 0; p < nnz; ++p)
    if (ci[p] < 0 || ci[p] >= cols || !std::isfinite(sv[p]))
      return fail("Invalid CSR column index or sparse value");
  if (cu_count <= 0) return fail("cu_count must be positive");

  auto* w = new or_worksets;
  w->rows = rows;
  w->cols = cols;
  w->nnz = nnz;
  int S = AnalyzeS(rows, rp, cu_count);  // matrix_utils.cu:499-506
  // optional cap on S (an extension; with the cap at or above S this is the
  // reference's partition)
  if (g_max_group_types > 0 && S > g_max_group_types) S = g_max_group_types;
  w->S = S;
  const int fine = w->fine;

  // Column histogram (matrix_utils.cu:508-514).
  w->col_nnz.assign(cols, 0);
  for (int p = 0; p < nnz; ++p) w->col_nnz[ci[p]] += 1;
  const std::vector<int>& cn = w->col_nnz;

  // NNZPoint sort by (row asc, col_nnz desc) (matrix_utils.cu:210-223, 518-524).
  // Equal counts keep CSR order: thrust's merge sort is taken to be stable.
  w->ranked.resize(nnz);
  std::iota(w->ranked.begin(), w->ranked.end(), 0);
  for (int r = 0; r < rows; ++r)
    std::stable_sort(w->ranked.begin() + rp[r], w->ranked.begin() + rp[r + 1],
                     [&](int a, int b) { return cn[ci[a]] > cn[ci[b]]; });

  // GetGroupNumArray (matrix_utils.cu:132-156).
  w->group_num.assign(S, 0);
  for (int r = 0; r < rows; ++r) {
    int d = rp[r + 1] - rp[r];
    if (S == 1) {
      w->group_num[0] += CeilDiv(d, fine);
    } else {
      for (int s = S - 1; s > 0; --s) {
        const int n = d / GroupSize(s);
        w->group_num[s] += n;
        d -= n * GroupSize(s);
      }
      if (d) w->group_num[0] += 1;
    }
  }

  // GetGroupMetaInfo (matrix_utils.cu:158-208) together with the membership of
  // every group: group g of workset s holds ranked positions [first, first+len)
  // of its row, where blocks come first from the largest size down
  // (GetBlockSignature / GetSrcBlockWorkset, :295-327, :361-392) and the residue
  // takes the tail (GetResidueSignature / GetSrcResidueWorkset, :261-293, :329-359).
  std::vector<std::vector<int>> member_first(S), member_len(S);
  w->init_des.assign(S, {});
  const int G0 = w->group_num[0];
  w->init_residue_offset.assign(size_t(G0) + 1, 0);
  w->init_residue_atomic.assign(size_t(G0), 0);
  {
    std::vector<int> counter(S, 0);
    for (int s = 0; s < S; ++s) {
      w->init_des[s].resize(w->group_num[s]);
      member_first[s].resize(w->group_num[s]);
      member_len[s].resize(w->group_num[s]);
    }
    for (int r = 0; r < rows; ++r) {
      const int d = rp[r + 1] - rp[r];
      int begin = rp[r];
      if (S == 1) {
        const int chunks = CeilDiv(d, fine);
        for (int j = 0; j < chunks; ++j) {
          const int g = counter[0]++;
          const int len = std::min(d - j * fine, fine);
          w->init_residue_atomic[g] = chunks > 1;
          w->init_residue_offset[g + 1] = w->init_residue_offset[g] + len;
          w->init_des[0][g] = r;
          member_first[0][g] = begin + j * fine;
          member_len[0][g] = len;
        }
      } else {
        int rem = d;
        const bool atomic = d > 32;
        for (int s = S - 1; s > 0; --s) {
          const int n = rem / GroupSize(s);
          for (int j = 0; j < n; ++j) {
            const int g = counter[s]++;
            w->init_des[s][g] = r;
            member_first[s][g] = begin;
            member_len[s][g] = GroupSize(s);
            begin += GroupSize(s);
          }
          rem -= n * GroupSize(s);
        }
        if (rem) {
          const int g = counter[0]++;
          w->init_residue_atomic[g] = atomic;
          w->init_residue_offset[g + 1] = w->init_residue_offset[g] + rem;
          w->init_des[0][g] = r;
          member_first[0][g] = begin;
          member_len[0][g] = rem;
        }
      }
    }
  }

  // Column signature bits (matrix_utils.cu:552-560), FFC with ffc = 2 (:55-60).
  w->sigbit.assign(cols, 0);
  w->sig_len = SigBits(cols, cn.data(), 2, w->sigbit.data());
  const int words = w->sig_len / 32;

  // Signatures and the stable per-word group sort, last word first
  // (matrix_utils.cu:261-327, 394-401, 562-594). Bit for column c sits in word
  // sigbit/32 at position 31 - sigbit%32.
  w->signature.assign(S, {});
  w->perm.assign(S, {});
  for (int s = 0; s < S; ++s) {
    const int G = w->group_num[s];
    w->perm[s].resize(G);
    std::iota(w->perm[s].begin(), w->perm[s].end(), 0);
    if (G == 0) continue;
    const bool lists = g_order_mode == 2 ||
                       (g_order_mode == 0 && size_t(G) * size_t(words) > kBitmapLimit);
    if (lists) {  // same order without the bitmaps (see OrderByBitLists)
      std::vector<std::vector<int>> bits(static_cast<size_t>(G));
      for (int g = 0; g < G; ++g)
        for (int q = 0; q < member_len[s][g]; ++q)
          bits[size_t(g)].push_back(w->sigbit[ci[w->ranked[member_first[s][g] + q]]]);
      w->perm[s] = OrderByBitLists(bits);
      continue;
    }
    std::vector<uint32_t>& sig = w->signature[s];
    sig.assign(size_t(G) * words, 0u);
    for (int g = 0; g < G; ++g)
      for (int q = 0; q < member_len[s][g]; ++q) {
        const int bit = w->sigbit[ci[w->ranked[member_first[s][g] + q]]];
        sig[size_t(bit / 32) * G + g] |= 1u << (31 - bit % 32);
      }
    for (int word = words - 1; word >= 0; --word) {
      const uint32_t* key = sig.data() + size_t(word) * G;
      std::stable_sort(w->perm[s].begin(), w->perm[s].end(),
                       [key](int a, int b) { return key[a] > key[b]; });
    }
  }

  // Final worksets (matrix_utils.cu:596-656): each group's nonzeros sorted by
  // column ascending (NNZPoint2 order, :225-237; stable for duplicate columns),
  // groups laid out in signature order, residue offsets recomputed in that order
  // (GetResidueOffset, :451-464).
  w->col.assign(S, {});
  w->val.assign(S, {});
  w->des.assign(S, {});
  w->residue_offset.assign(size_t(G0) + 1, 0);
  w->residue_atomic.assign(size_t(G0), 0);
  for (int k = 0; k < G0; ++k) {
    const int src = w->perm[0][k];
    w->residue_offset[k + 1] = w->residue_offset[k] + member_len[0][src];
    w->residue_atomic[k] = w->init_residue_atomic[src];
  }
  std::vector<int> tmp;
  for (int s = 0; s < S; ++s) {
    const int G = w->group_num[s];
    const size_t total = s == 0 ? size_t(w->residue_offset[G0]) : size_t(G) * GroupSize(s);
    w->col[s].resize(total);
    w->val[s].resize(total);
    w->des[s].resize(G);
    size_t out = 0;
    for (int k = 0; k < G; ++k) {
      const int src = w->perm[s][k];
      w->des[s][k] = w->init_des[s][src];
      tmp.assign(w->ranked.begin() + member_first[s][src],
                 w->ranked.begin() + member_first[s][src] + member_len[s][src]);
      std::stable_sort(tmp.begin(), tmp.end(), [ci](int a, int b) { return ci[a] < ci[b]; });
      for (int p : tmp) {
        w->col[s][out] = ci[p];
        w->val[s][out] = sv[p];
        ++out;
      }
    }
  }
  return w;
}

void or_free(or_worksets* w) { delete w; }
int or_group_type_num(const or_worksets* w) { return w->S; }
int or_group_num(const or_worksets* w, int s) { return w->group_num[s]; }
int or_signature_len(const or_worksets* w) { return w->sig_len; }
long long or_workset_len(const or_worksets* w, int s) { return (long long)w->col[s].size(); }

void or_copy_workset(const or_worksets* w, int s, int* col, float* val, int* des) {
  if (col) std::copy(w->col[s].begin(), w->col[s].end(), col);
  if (val) std::copy(w->val[s].begin(), w->val[s].end(), val);
  if (des) std::copy(w->des[s].begin(), w->des[s].end(), des);
}
void or_copy_residue(const or_worksets* w, int* offset, uint8_t* atomic) {
  if (offset) std::copy(w->residue_offset.begin(), w->residue_offset.end(), offset);
  if (atomic) std::copy(w->residue_atomic.begin(), w->residue_atomic.end(), atomic);
}
void or_copy_col_nnz(const or_worksets* w, int* out) {
  std::copy(w->col_nnz.begin(), w->col_nnz.end(), out);
}
void or_copy_ranked_pos(const or_worksets* w, int* out) {
  std::copy(w->ranked.begin(), w->ranked.end(), out);
}
void or_copy_sigbit(const or_worksets* w, int* out) {
  std::copy(w->sigbit.begin(), w->sigbit.end(), out);
}
void or_copy_initial_des(const or_worksets* w, int s, int* out) {
  std::copy(w->init_des[s].begin(), w->init_des[s].end(), out);
}
void or_copy_initial_residue(const or_worksets* w, int* offset, uint8_t* atomic) {
  if (offset) std::copy(w->init_residue_offset.begin(), w->init_residue_offset.end(), offset);
  if (atomic) std::copy(w->init_residue_atomic.begin(), w->init_residue_atomic.end(), atomic);
}
void or_copy_signature(const or_worksets* w, int s, uint32_t* out) {
  std::copy(w->signature[s].begin(), w->signature[s].end(), out);
}
int or_has_signature(const or_worksets* w, int s) {
  return w->group_num[s] > 0 && !w->signature[s].empty();
}
void or_copy_group_perm(const or_worksets* w, int s, int* out) {
  std::copy(w->perm[s].begin(), w->perm[s].end(), out);
}

void or_spmm(int rows, const int* rp, const int* ci, const float* sv, int n, const float* B,
             double* C, double* mag, int threads) {
  // CheckSpmm (benchmark.cu:64-77): double(value) * float(B) accumulated in double.
#ifdef _OPENMP
  if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 64) num_threads(threads)
#endif
  for (int r = 0; r < rows; ++r) {
    double* c = C + size_t(r) * n;
    double* m = mag ? mag + size_t(r) * n : nullptr;
    for (int j = 0; j < n; ++j) c[j] = 0.0;
    if (m)
      for (int j = 0; j < n; ++j) m[j] = 0.0;
    for (int p = rp[r]; p < rp[r + 1]; ++p) {
      const double a = double(sv[p]);
      const float* b = B + size_t(ci[p]) * n;
      for (int j = 0; j < n; ++j) c[j] += a * b[j];
      if (m)
        for (int j = 0; j < n; ++j) m[j] += std::fabs(a * b[j]);
    }
  }
}

void or_sddmm(int groups, const int* des, const int* off, const int* ci, const float* sv, int k,
              const float* X, const float* Y, double* out, double* mag, int threads) {
  // CheckSddmm (benchmark.cu:79-96): per position, double dot of lhs[row] and
  // rhs[col], then times the sparse value.
#ifdef _OPENMP
  if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 256) num_threads(threads)
#endif
  for (int g = 0; g < groups; ++g) {
    const float* x = X + size_t(des[g]) * k;
    for (int p = off[g]; p < off[g + 1]; ++p) {
      const float* y = Y + size_t(ci[p]) * k;
      double dot = 0.0, abs_dot = 0.0;
      for (int j = 0; j < k; ++j) {
        const double t = double(x[j]) * y[j];
        dot += t;
        abs_dot += std::fabs(t);
      }
      out[p] = dot * sv[p];
      if (mag) mag[p] = abs_dot * std::fabs(double(sv[p]));
    }
  }
}

void or_dense_input(unsigned seed, size_t n1, float* out1, size_t n2, float* out2) {
  std::mt19937 rng(seed);  // benchmark.cu:137-140, benchmark_utils.h:100-104
  for (size_t i = 0; i < n1; ++i) out1[i] = static_cast<float>(rng() % 3) / 10.0f;
  for (size_t i = 0; i < n2; ++i) out2[i] = static_cast<float>(rng() % 3) / 10.0f;
}

uint32_t or_mt19937_nth(unsigned seed, long long index) {
  std::mt19937 rng(seed);
  uint32_t v = 0;
  for (long long i = 0; i < index; ++i) v = rng();
  return v;
}

int or_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

}  // extern "C"
