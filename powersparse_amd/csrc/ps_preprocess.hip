// Block/residue preprocessing kernels (the GPU side of PowerSparseMatrixGPU).
//
// The C++ host (powersparse_amd/host/matrix_utils.cpp) drives them in order:
//   degree sums (worksets S) -> column histogram -> rank keys + stable radix
//   sort (each row's nonzeros by column count, descending) -> per-row group
//   counts + scans -> group metadata -> signatures -> per-word stable radix sort
//   of group ids -> permuted metadata -> gathered, column-sorted worksets.
// Group membership follows utils/matrix_utils.cu: in a row's ranked order the
// block groups come first, largest size first, and the residue takes the tail;
// in fine mode (S == 1) the row is cut into chunks of `fine` nonzeros.
#include <vector>

#include "ps_common.hpp"

namespace ps {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ int group_size(int s) { return 32 << (s - 1); }

__global__ void degree_sums_kernel(const int* __restrict__ row_ptr, int rows,
                                   unsigned long long* __restrict__ sums) {
  __shared__ unsigned long long acc[32];
  if (threadIdx.x < 32) acc[threadIdx.x] = 0;
  __syncthreads();
  for (int r = blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += gridDim.x * blockDim.x) {
    const int d = row_ptr[r + 1] - row_ptr[r];
    for (int s = 1; s < 32; ++s) {
      const int q = d >> (s + 4);  // floor(d / (32 * 2^(s-1)))
      if (q == 0) break;
      atomicAdd(&acc[s], (unsigned long long)q);
    }
  }
  __syncthreads();
  if (threadIdx.x < 32 && acc[threadIdx.x]) atomicAdd(&sums[threadIdx.x], acc[threadIdx.x]);
}

// Column histogram. Each workgroup counts a chunk of kHistChunk nonzeros in
// an LDS hash table first (keys = column + 1, bounded linear probing) and
// adds each distinct column's count to the global histogram once: hub
// columns, which appear in most rows, then cost one global atomic per chunk
// instead of one per nonzero. Nonzeros that find no slot add directly.
constexpr int kHistSlots = 4096;
constexpr int kHistChunk = 16384;
constexpr int kHistProbes = 8;

__global__ __launch_bounds__(kThreads) void col_hist_kernel(const int* __restrict__ col_ind,
                                                            int nnz, int* __restrict__ col_nnz) {
  __shared__ uint32_t key[kHistSlots];
  __shared__ uint32_t cnt[kHistSlots];
  for (int i = threadIdx.x; i < kHistSlots; i += blockDim.x) {
    key[i] = 0u;
    cnt[i] = 0u;
  }
  __syncthreads();
  const long long first = (long long)blockIdx.x * kHistChunk;
  const long long last = first + kHistChunk < nnz ? first + kHistChunk : nnz;
  for (long long p = first + threadIdx.x; p < last; p += blockDim.x) {
    const int c = col_ind[p];
    const uint32_t k = uint32_t(c) + 1u;
    uint32_t h = (k * 2654435761u) >> (32 - 12);  // 12 bits: kHistSlots slots
    bool counted = false;
    for (int probe = 0; probe < kHistProbes; ++probe) {
      const uint32_t prev = atomicCAS(&key[h], 0u, k);
      if (prev == 0u || prev == k) {
        atomicAdd(&cnt[h], 1u);
        counted = true;
        break;
      }
      h = (h + 1) & (kHistSlots - 1);
    }
    if (!counted) atomicAdd(&col_nnz[c], 1);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < kHistSlots; i += blockDim.x)
    if (key[i]) atomicAdd(&col_nnz[key[i] - 1u], int(cnt[i]));
}

// Row of position p: the last r with row_ptr[r] <= p (binary search).
__device__ __forceinline__ int row_of(const int* __restrict__ row_ptr, int rows, int p) {
  int lo = 0, hi = rows;  // row_ptr[lo] <= p < row_ptr[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (row_ptr[mid] <= p) lo = mid;
    else hi = mid;
  }
  return lo;
}

__global__ void rank_keys_kernel(const int* __restrict__ row_ptr, int rows,
                                 const int* __restrict__ col_ind, int nnz,
                                 const int* __restrict__ col_nnz, int max_count, int count_bits,
                                 uint64_t* __restrict__ keys, uint32_t* __restrict__ vals) {
  for (int p = blockIdx.x * blockDim.x + threadIdx.x; p < nnz; p += gridDim.x * blockDim.x) {
    const int r = row_of(row_ptr, rows, p);
    keys[p] = (uint64_t(r) << count_bits) | uint64_t(max_count - col_nnz[col_ind[p]]);
    vals[p] = uint32_t(p);
  }
}

// ---- ranking each row's nonzeros, row by row ----
//
// Rows arrive in order, so ranking only sorts inside each row: by count key
// (max_count - col_nnz, ascending = column count descending), ties in CSR
// order. Rows of up to 256 nonzeros: one wave per row, each element's rank
// counted against the others. 257 .. 8192: one workgroup per row, bitonic sort of
// (count key, index) pairs in LDS. Longer rows: their elements are compacted
// and radix-sorted (stable) with the row's list index in the high bits.
// Output as the stable sort of (row, count key): keys = row << count_bits |
// count key, vals = CSR position.
constexpr int kRankTileSmall = 1024, kRankTileLarge = 8192;

__device__ __forceinline__ uint32_t count_key(const int* __restrict__ col_ind,
                                              const int* __restrict__ col_nnz, int max_count,
                                              int p) {
  return uint32_t(max_count - col_nnz[col_ind[p]]);
}

constexpr int kRankWavePer = 4;  // elements per lane: one wave ranks rows up to 256

__global__ void rank_small_kernel(const int* __restrict__ row_ptr, int rows,
                                  const int* __restrict__ col_ind,
                                  const int* __restrict__ col_nnz, int max_count, int count_bits,
                                  uint64_t* __restrict__ keys, uint32_t* __restrict__ vals) {
  const int r = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (r >= rows) return;
  const int b = row_ptr[r];
  const int d = row_ptr[r + 1] - b;
  if (d == 0 || d > kWave * kRankWavePer) return;
  const int lane = lane_id();
  // element q * 64 + lane sits in ck[q] of this lane
  uint32_t ck[kRankWavePer];
  int rank[kRankWavePer];
#pragma unroll
  for (int q = 0; q < kRankWavePer; ++q) {
    const int j = q * kWave + lane;
    ck[q] = j < d ? count_key(col_ind, col_nnz, max_count, b + j) : 0xFFFFFFFFu;
    rank[q] = 0;
  }
  const int used = (d + kWave - 1) / kWave;  // element rows of the wave that hold data
  for (int qo = 0; qo < used; ++qo) {
    const int kmax = d - qo * kWave < kWave ? d - qo * kWave : kWave;
    for (int kl = 0; kl < kmax; ++kl) {
      const int k = qo * kWave + kl;
      uint32_t other = 0;
#pragma unroll
      for (int q = 0; q < kRankWavePer; ++q)
        if (q == qo) other = uint32_t(__shfl(int(ck[q]), kl, kWave));
#pragma unroll
      for (int q = 0; q < kRankWavePer; ++q) {
        const int j = q * kWave + lane;
        rank[q] += (other < ck[q] || (other == ck[q] && k < j)) ? 1 : 0;
      }
    }
  }
#pragma unroll
  for (int q = 0; q < kRankWavePer; ++q) {
    const int j = q * kWave + lane;
    if (j < d) {
      keys[b + rank[q]] = (uint64_t(r) << count_bits) | ck[q];
      vals[b + rank[q]] = uint32_t(b + j);
    }
  }
}

// One workgroup per listed row (degree <= tile).
__global__ __launch_bounds__(kThreads) void rank_tile_kernel(
    const uint32_t* __restrict__ row_list, const int* __restrict__ row_ptr,
    const int* __restrict__ col_ind, const int* __restrict__ col_nnz, int max_count,
    int count_bits, uint64_t* __restrict__ keys, uint32_t* __restrict__ vals) {
  extern __shared__ uint64_t pairs[];
  const int r = int(row_list[blockIdx.x]);
  const int b = row_ptr[r];
  const int d = row_ptr[r + 1] - b;
  int pw = 2;
  while (pw < d) pw <<= 1;
  for (int e = threadIdx.x; e < pw; e += blockDim.x)
    pairs[e] = e < d ? (uint64_t(count_key(col_ind, col_nnz, max_count, b + e)) << 32) | uint32_t(e)
                     : ~0ull;
  __syncthreads();
  for (int k2 = 2; k2 <= pw; k2 <<= 1) {
    for (int j = k2 >> 1; j > 0; j >>= 1) {
      for (int e = threadIdx.x; e < pw / 2; e += blockDim.x) {
        const int i = (e / j) * 2 * j + (e % j);
        const int l = i + j;
        const bool asc = (i & k2) == 0;
        const uint64_t x = pairs[i], y = pairs[l];
        if ((x > y) == asc) {
          pairs[i] = y;
          pairs[l] = x;
        }
      }
      __syncthreads();
    }
  }
  for (int e = threadIdx.x; e < d; e += blockDim.x) {
    const uint64_t v = pairs[e];
    keys[b + e] = (uint64_t(r) << count_bits) | (v >> 32);
    vals[b + e] = uint32_t(b) + uint32_t(v & 0xFFFFFFFFu);
  }
}

// Row classes beyond one wave, as flags flag[c * rows + r]: c = 0 up to
// kRankTileSmall nonzeros, 1 up to kRankTileLarge, 2 longer.
__global__ void rank_classify_kernel(const int* __restrict__ row_ptr, int rows,
                                     uint32_t* __restrict__ flag) {
  for (int r = blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += gridDim.x * blockDim.x) {
    const int d = row_ptr[r + 1] - row_ptr[r];
    flag[r] = (d > kWave * kRankWavePer && d <= kRankTileSmall) ? 1u : 0u;
    flag[size_t(rows) + r] = (d > kRankTileSmall && d <= kRankTileLarge) ? 1u : 0u;
    flag[2 * size_t(rows) + r] = d > kRankTileLarge ? 1u : 0u;
  }
}

// list_c[slot_c[r]] = r for the rows of each class (slots scanned per class).
__global__ void rank_lists_kernel(int rows, const uint32_t* __restrict__ flag,
                                  const uint32_t* __restrict__ slot,
                                  uint32_t* __restrict__ list1, uint32_t* __restrict__ list2,
                                  uint32_t* __restrict__ list3) {
  for (int r = blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += gridDim.x * blockDim.x) {
    if (flag[r]) list1[slot[r]] = uint32_t(r);
    if (flag[size_t(rows) + r]) list2[slot[size_t(rows) + r]] = uint32_t(r);
    if (flag[2 * size_t(rows) + r]) list3[slot[2 * size_t(rows) + r]] = uint32_t(r);
  }
}

// long_start[i] = degree of long row list[i] (scanned into element offsets).
__global__ void permute_long_degrees_kernel(const uint32_t* __restrict__ list, uint32_t n,
                                            const int* __restrict__ row_ptr,
                                            uint32_t* __restrict__ long_start) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    const int r = int(list[i]);
    long_start[i] = uint32_t(row_ptr[r + 1] - row_ptr[r]);
  }
}

// Long rows: compacted keys (list index << count_bits | count key), values =
// CSR positions; one workgroup per long row.
__global__ void rank_long_keys_kernel(const uint32_t* __restrict__ list,
                                      const uint32_t* __restrict__ seg_start,
                                      const int* __restrict__ row_ptr,
                                      const int* __restrict__ col_ind,
                                      const int* __restrict__ col_nnz, int max_count,
                                      int count_bits, uint64_t* __restrict__ ck,
                                      uint32_t* __restrict__ cv) {
  const uint32_t i = blockIdx.x;
  const int r = int(list[i]);
  const int b = row_ptr[r];
  const int d = row_ptr[r + 1] - b;
  const size_t o = seg_start[i];
  for (int e = threadIdx.x; e < d; e += blockDim.x) {
    ck[o + e] = (uint64_t(i) << count_bits) | count_key(col_ind, col_nnz, max_count, b + e);
    cv[o + e] = uint32_t(b + e);
  }
}

// After the stable sort the elements of long row i occupy the same compacted
// range as before: element j of it goes to row_ptr[row] + (j - seg_start[i]).
__global__ void rank_long_write_kernel(size_t total, const uint64_t* __restrict__ ck,
                                       const uint32_t* __restrict__ cv,
                                       const uint32_t* __restrict__ list,
                                       const uint32_t* __restrict__ seg_start,
                                       const int* __restrict__ row_ptr, int count_bits,
                                       uint64_t* __restrict__ keys, uint32_t* __restrict__ vals) {
  const uint64_t mask = (uint64_t(1) << count_bits) - 1;
  for (size_t j = size_t(blockIdx.x) * blockDim.x + threadIdx.x; j < total;
       j += size_t(gridDim.x) * blockDim.x) {
    const uint32_t i = uint32_t(ck[j] >> count_bits);
    const int r = int(list[i]);
    const size_t out = size_t(row_ptr[r]) + (j - seg_start[i]);
    keys[out] = (uint64_t(r) << count_bits) | (ck[j] & mask);
    vals[out] = cv[j];
  }
}

// counts[s * (rows + 1) + r]; the extra entry per workset stays 0 so that the
// exclusive scan leaves the workset's group total at index `rows`.
__global__ void group_counts_kernel(const int* __restrict__ row_ptr, int rows, int S, int fine,
                                    uint32_t* __restrict__ counts) {
  const size_t stride = size_t(rows) + 1;
  for (int r = blockIdx.x * blockDim.x + threadIdx.x; r <= rows; r += gridDim.x * blockDim.x) {
    if (r == rows) {
      for (int s = 0; s < S; ++s) counts[s * stride + r] = 0;
      continue;
    }
    int d = row_ptr[r + 1] - row_ptr[r];
    if (S == 1) {
      counts[r] = uint32_t((d + fine - 1) / fine);
      continue;
    }
    for (int s = S - 1; s > 0; --s) {
      const int n = d / group_size(s);
      counts[s * stride + r] = uint32_t(n);
      d -= n * group_size(s);
    }
    counts[r] = d > 0 ? 1u : 0u;
  }
}

struct PtrTable {
  int* p[PS_MAX_WORKSETS];
};
struct SigTable {
  uint32_t* p[PS_MAX_WORKSETS];
  int groups[PS_MAX_WORKSETS];
};

__global__ void group_meta_kernel(const int* __restrict__ row_ptr, int rows, int S, int fine,
                                  const uint32_t* __restrict__ prefix, PtrTable des,
                                  PtrTable start, int* __restrict__ res_len,
                                  uint8_t* __restrict__ res_atomic) {
  const size_t stride = size_t(rows) + 1;
  for (int r = blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += gridDim.x * blockDim.x) {
    const int base = row_ptr[r];
    const int d = row_ptr[r + 1] - base;
    if (S == 1) {
      const int chunks = (d + fine - 1) / fine;
      const int g0 = int(prefix[r]);
      for (int j = 0; j < chunks; ++j) {
        des.p[0][g0 + j] = r;
        start.p[0][g0 + j] = base + j * fine;
        res_len[g0 + j] = min(fine, d - j * fine);
        res_atomic[g0 + j] = chunks > 1;
      }
      continue;
    }
    int rem = d, off = 0;
    for (int s = S - 1; s > 0; --s) {
      const int gs = group_size(s);
      const int n = rem / gs;
      const int g0 = int(prefix[s * stride + r]);
      for (int j = 0; j < n; ++j) {
        des.p[s][g0 + j] = r;
        start.p[s][g0 + j] = base + off;
        off += gs;
      }
      rem -= n * gs;
    }
    if (rem > 0) {
      const int g = int(prefix[r]);
      des.p[0][g] = r;
      start.p[0][g] = base + off;
      res_len[g] = rem;
      res_atomic[g] = d > 32;
    }
  }
}

// Workset s and group g of the nonzero at ranked position i of row r: block
// groups of the largest size first, the residue takes the tail (fine mode:
// chunks of `fine`).
__device__ __forceinline__ void locate_group(const int* __restrict__ row_ptr, int r, int i, int S,
                                             int fine, const uint32_t* __restrict__ prefix,
                                             size_t stride, int& s, int& g) {
  const int base = row_ptr[r];
  const int j = i - base;  // rank of this nonzero inside its row
  s = 0;
  if (S == 1) {
    g = int(prefix[r]) + j / fine;
    return;
  }
  int rem = row_ptr[r + 1] - base, off = 0;
  for (int t = S - 1; t > 0; --t) {
    const int gs = group_size(t);
    const int n = rem / gs;
    if (j < off + n * gs) {
      s = t;
      g = int(prefix[t * stride + r]) + (j - off) / gs;
      return;
    }
    off += n * gs;
    rem -= n * gs;
  }
  g = int(prefix[r]);
}

__global__ void signatures_kernel(const int* __restrict__ row_ptr, int rows, int S, int fine,
                                  const uint64_t* __restrict__ ranked_keys, int count_bits,
                                  const uint32_t* __restrict__ ranked_vals, int nnz,
                                  const int* __restrict__ col_ind, const int* __restrict__ sigbit,
                                  const uint32_t* __restrict__ prefix, SigTable sig) {
  const size_t stride = size_t(rows) + 1;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < nnz; i += gridDim.x * blockDim.x) {
    int s, g;
    locate_group(row_ptr, int(ranked_keys[i] >> count_bits), i, S, fine, prefix, stride, s, g);
    const int bit = sigbit[col_ind[ranked_vals[i]]];
    atomicOr(&sig.p[s][size_t(bit >> 5) * sig.groups[s] + g], 1u << (31 - (bit & 31)));
  }
}

// ---- signature order from sorted bit lists ----
//
// The stable per-word sort orders groups by their signature read as one
// big-endian bit string (bit b of the string is bit 31 - b % 32 of word b / 32),
// descending, ties in group order. Equivalently: by the ascending list of the
// group's distinct signature bits, compared lexicographically ascending with
// the end of a list ranking after every bit, ties in group order. The lists
// cost at most one entry per nonzero, whatever the signature length.

// First group id of each workset in one global numbering; base[S] = total.
struct GroupBase {
  uint32_t base[PS_MAX_WORKSETS + 1];
  int S;
};

__device__ __forceinline__ int workset_of(const GroupBase& gb, uint32_t global) {
  int s = 0;
  while (global >= gb.base[s + 1]) ++s;
  return s;
}

// entry[i] = (global group of ranked position i) << bit_bits | signature bit.
__global__ void signature_entries_kernel(const int* __restrict__ row_ptr, int rows, int S,
                                         int fine, const uint64_t* __restrict__ ranked_keys,
                                         int count_bits, const uint32_t* __restrict__ ranked_vals,
                                         int nnz, const int* __restrict__ col_ind,
                                         const int* __restrict__ sigbit,
                                         const uint32_t* __restrict__ prefix, GroupBase gb,
                                         int bit_bits, uint64_t* __restrict__ entries) {
  const size_t stride = size_t(rows) + 1;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < nnz; i += gridDim.x * blockDim.x) {
    int s, g;
    locate_group(row_ptr, int(ranked_keys[i] >> count_bits), i, S, fine, prefix, stride, s, g);
    const uint32_t bit = uint32_t(sigbit[col_ind[ranked_vals[i]]]);
    entries[i] = (uint64_t(gb.base[s] + uint32_t(g)) << bit_bits) | bit;
  }
}

// flag[i] = 1 where sorted entry i differs from entry i - 1 (first of its value).
__global__ void entry_flags_kernel(const uint64_t* __restrict__ e, uint32_t n,
                                   uint32_t* __restrict__ flag) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    flag[i] = (i == 0 || e[i] != e[i - 1]) ? 1u : 0u;
}

// Distinct entries compacted into lists; list_begin[g] = first list slot of
// group g, list_begin[total] = number of distinct entries.
__global__ void entry_lists_kernel(const uint64_t* __restrict__ e, uint32_t n, int bit_bits,
                                   const uint32_t* __restrict__ flag,
                                   const uint32_t* __restrict__ pos, uint32_t total,
                                   uint32_t* __restrict__ lists,
                                   uint32_t* __restrict__ list_begin) {
  const uint64_t mask = (uint64_t(1) << bit_bits) - 1;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    if (flag[i]) {
      lists[pos[i]] = uint32_t(e[i] & mask);
      const uint64_t g = e[i] >> bit_bits;
      if (i == 0 || (e[i - 1] >> bit_bits) != g) list_begin[g] = pos[i];
    }
    if (i == n - 1) list_begin[total] = pos[i] + flag[i];
  }
}

// Refinement. The active groups (still tied with another group of their
// class) are kept in class order, each with its class base (final position
// of the class's first member) and class depth (all members have equal lists
// before it). Initially every group is active, the classes are the worksets
// and the depth is 0. Each round compares every member with its class's first
// member r (the reference) from the class depth on: the first position where
// they differ, `lcp`, and which way the member goes:
//   EQ     identical list to r;
//   BEFORE the member's element at lcp is smaller than r's, or r's list ends;
//   AFTER  the member's list ends at lcp, or its element is larger.
// Sorting each class by (side, lcp ascending for BEFORE / descending for
// AFTER, element at lcp, list end last) puts it in final order except within
// runs of equal keys, which become the next round's classes with depth
// lcp + 1 (their lists agree up to and including lcp). EQ runs, runs whose
// lists ended, and single members are placed. Every class loses at least its
// reference each round, and in practice a whole nest of prefix-related lists
// separates in one round.
constexpr uint32_t kBefore = 0, kEq = 1, kAfter = 2;

__global__ void order_init_kernel(uint32_t n, GroupBase gb, uint32_t* __restrict__ act_group,
                                  uint32_t* __restrict__ act_base,
                                  uint32_t* __restrict__ act_depth) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    act_group[i] = i;
    act_base[i] = gb.base[workset_of(gb, i)];
    act_depth[i] = 0;
  }
}

// Longest list (bounds the divergence depth).
__global__ void max_list_kernel(const uint32_t* __restrict__ list_begin, uint32_t groups,
                                uint32_t* __restrict__ out) {
  uint32_t m = 0;
  for (uint32_t g = blockIdx.x * blockDim.x + threadIdx.x; g < groups;
       g += gridDim.x * blockDim.x)
    m = max(m, list_begin[g + 1] - list_begin[g]);
  for (int d = 1; d < kWave; d <<= 1) m = max(m, uint32_t(__shfl_xor(int(m), d, kWave)));
  if (lane_id() == 0) atomicMax(out, m);
}

// head[i] = 1 where a class starts.
__global__ void order_class_heads_kernel(const uint32_t* __restrict__ act_base, uint32_t n,
                                         uint32_t* __restrict__ head) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    head[i] = (i == 0 || act_base[i] != act_base[i - 1]) ? 1u : 0u;
}

// head_at[c] = index of class c's first member (its reference).
__global__ void order_class_start_kernel(uint32_t n, const uint32_t* __restrict__ head,
                                         const uint32_t* __restrict__ rank,
                                         uint32_t* __restrict__ head_at) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    if (head[i]) head_at[rank[i]] = i;
}

// Sort keys of every active member: hi = class * 3 + side; lo = divergence
// key * (end + 1) + element (end for a list that ended). lcp[i] = divergence
// position; idx[i] = i.
__global__ void order_diverge_kernel(const uint32_t* __restrict__ act_group,
                                     const uint32_t* __restrict__ act_depth, uint32_t n,
                                     const uint32_t* __restrict__ lists,
                                     const uint32_t* __restrict__ list_begin,
                                     const uint32_t* __restrict__ head,
                                     const uint32_t* __restrict__ rank,
                                     const uint32_t* __restrict__ head_at, uint32_t end,
                                     uint32_t max_len, uint64_t* __restrict__ hi,
                                     uint64_t* __restrict__ lo, uint32_t* __restrict__ lcp_out,
                                     uint32_t* __restrict__ idx) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    const uint32_t c = rank[i] + head[i] - 1;
    const uint32_t g = act_group[i];
    const uint32_t r = act_group[head_at[c]];
    const uint32_t* m = lists + list_begin[g];
    const uint32_t* q = lists + list_begin[r];
    const uint32_t nm = list_begin[g + 1] - list_begin[g];
    const uint32_t nq = list_begin[r + 1] - list_begin[r];
    uint32_t d = act_depth[i];
    if (g != r)
      while (d < nm && d < nq && m[d] == q[d]) ++d;
    uint32_t side, key = 0, elem = 0;
    if (g == r || (d == nm && d == nq)) {
      side = kEq;
      d = nm;
    } else if (d == nm) {
      side = kAfter;
      key = max_len - d;
      elem = end;
    } else if (d == nq || m[d] < q[d]) {
      side = kBefore;
      key = d;
      elem = m[d];
    } else {
      side = kAfter;
      key = max_len - d;
      elem = m[d];
    }
    hi[i] = uint64_t(c) * 3u + side;
    lo[i] = uint64_t(key) * (uint64_t(end) + 1u) + elem;
    lcp_out[i] = d;
    idx[i] = i;
  }
}

// ---- refinement tail in one workgroup ----
//
// Once at most kFinishMax groups are still tied, one 1024-thread workgroup
// runs the remaining rounds with the whole state in LDS (no host round trip
// per round): the same rounds as above, the sort being an LDS bitonic sort of
// (key, slot) pairs (slots unique, so equal keys keep their class order) and
// run / class starts coming from block max-scans.
constexpr int kFinishMax = 2048;
constexpr int kFinishThreads = 1024;
constexpr int kFinishPer = kFinishMax / kFinishThreads;  // elements per thread
// LDS of order_finish_kernel: one uint64 key and seven uint32 arrays per
// element, plus the scan partials.
constexpr size_t kFinishLds =
    size_t(kFinishMax) * (sizeof(uint64_t) + 7 * sizeof(uint32_t)) +
    (kFinishThreads / kWave) * sizeof(uint32_t);

// Exclusive sum (kSum) or inclusive max over v[0 .. kFinishMax) in LDS;
// wsum holds kFinishThreads / kWave partials. Ends with a barrier.
template <bool kSum>
__device__ void block_scan(uint32_t* v, uint32_t* wsum) {
  const int t = threadIdx.x;
  uint32_t x[kFinishPer];
  uint32_t run = 0;
#pragma unroll
  for (int q = 0; q < kFinishPer; ++q) {  // thread t owns v[kFinishPer * t + q]
    x[q] = v[kFinishPer * t + q];
    run = kSum ? run + x[q] : max(run, x[q]);
  }
  uint32_t inc = run;
  const int lane = lane_id();
  for (int d = 1; d < kWave; d <<= 1) {
    const uint32_t y = uint32_t(__shfl_up(int(inc), d, kWave));
    if (lane >= d) inc = kSum ? inc + y : max(inc, y);
  }
  if (lane == kWave - 1) wsum[t / kWave] = inc;
  __syncthreads();
  if (t < kWave) {
    uint32_t w = t < kFinishThreads / kWave ? wsum[t] : 0u;
    for (int d = 1; d < kWave; d <<= 1) {
      const uint32_t y = uint32_t(__shfl_up(int(w), d, kWave));
      if (t >= d) w = kSum ? w + y : max(w, y);
    }
    if (t < kFinishThreads / kWave) wsum[t] = w;
  }
  __syncthreads();
  const uint32_t before_wave = t >= kWave ? wsum[t / kWave - 1] : 0u;
  uint32_t before_me = uint32_t(__shfl_up(int(inc), 1, kWave));
  if (lane == 0) before_me = 0u;  // identity of both sum and max (values >= 0)
  uint32_t acc = kSum ? before_wave + before_me : max(before_wave, before_me);
#pragma unroll
  for (int q = 0; q < kFinishPer; ++q) {
    if (kSum) {
      v[kFinishPer * t + q] = acc;
      acc += x[q];
    } else {
      acc = max(acc, x[q]);
      v[kFinishPer * t + q] = acc;
    }
  }
  __syncthreads();
}

__global__ __launch_bounds__(kFinishThreads) void order_finish_kernel(
    uint32_t n0, const uint32_t* __restrict__ act_group, const uint32_t* __restrict__ act_base,
    const uint32_t* __restrict__ act_depth, const uint32_t* __restrict__ lists,
    const uint32_t* __restrict__ list_begin, uint32_t end, uint32_t max_len, int lo_bits,
    GroupBase gb, SigTable perm, uint32_t* __restrict__ status) {
  extern __shared__ __attribute__((aligned(16))) uint64_t finish_lds[];
  constexpr int P = kFinishMax;
  uint64_t* key = finish_lds;                            // [P]
  uint32_t* grp = reinterpret_cast<uint32_t*>(key + P);  // [P] state by slot
  uint32_t* bas = grp + P;
  uint32_t* dep = bas + P;
  uint32_t* lcp = dep + P;                               // [P] by slot
  uint32_t* idx = lcp + P;                               // [P] sorted -> slot
  uint32_t* t0 = idx + P;                                // [P] scratch
  uint32_t* t1 = t0 + P;                                 // [P] scratch
  uint32_t* wsum = t1 + P;                               // [kFinishThreads / kWave]
  static_assert(sizeof(uint64_t) * P + 7 * sizeof(uint32_t) * P +
                        (kFinishThreads / kWave) * sizeof(uint32_t) == kFinishLds,
                "LDS layout and kFinishLds disagree");
  const int t = threadIdx.x;
  const uint64_t lo_mask = (uint64_t(1) << lo_bits) - 1;
  const uint64_t end1 = uint64_t(end) + 1u;
  uint32_t n = n0;
  for (int e = t; e < P; e += kFinishThreads) {
    if (uint32_t(e) < n) {
      grp[e] = act_group[e];
      bas[e] = act_base[e];
      dep[e] = act_depth[e];
    }
  }
  __syncthreads();
  for (uint32_t round = 0; n > 0; ++round) {
    if (round > n0) {  // cannot happen: every round places each class's reference
      if (t == 0) status[0] = 1u;
      return;
    }
    // class starts -> class ranks (t0 = head flags, then exclusive ranks)
    for (int e = t; e < P; e += kFinishThreads)
      t0[e] = (uint32_t(e) < n && (e == 0 || bas[e] != bas[e - 1])) ? 1u : 0u;
    __syncthreads();
    block_scan<true>(t0, wsum);  // t0[e] = classes before e
    // t1[c] = first slot of class c
    for (int e = t; e < P; e += kFinishThreads)
      if (uint32_t(e) < n && (e == 0 || bas[e] != bas[e - 1])) t1[t0[e]] = uint32_t(e);
    __syncthreads();
    // divergence from each class's first member; keys (hi << lo_bits | lo)
    uint64_t k_reg[kFinishPer];
    uint32_t lcp_reg[kFinishPer];
#pragma unroll
    for (int q = 0; q < kFinishPer; ++q) {
      const int e = t + q * kFinishThreads;
      k_reg[q] = ~0ull;
      lcp_reg[q] = 0u;
      if (uint32_t(e) >= n) continue;
      const bool head = e == 0 || bas[e] != bas[e - 1];
      const uint32_t c = head ? t0[e] : t0[e] - 1u;
      const uint32_t g = grp[e];
      const uint32_t r = grp[t1[c]];
      const uint32_t* m = lists + list_begin[g];
      const uint32_t* rq = lists + list_begin[r];
      const uint32_t nm = list_begin[g + 1] - list_begin[g];
      const uint32_t nq = list_begin[r + 1] - list_begin[r];
      uint32_t d = dep[e];
      if (g != r)
        while (d < nm && d < nq && m[d] == rq[d]) ++d;
      uint32_t side, kk = 0, el = 0;
      if (g == r || (d == nm && d == nq)) {
        side = kEq;
        d = nm;
      } else if (d == nm) {
        side = kAfter;
        kk = max_len - d;
        el = end;
      } else if (d == nq || m[d] < rq[d]) {
        side = kBefore;
        kk = d;
        el = m[d];
      } else {
        side = kAfter;
        kk = max_len - d;
        el = m[d];
      }
      k_reg[q] = ((uint64_t(c) * 3u + side) << lo_bits) | (uint64_t(kk) * end1 + el);
      lcp_reg[q] = d;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kFinishPer; ++q) {
      const int e = t + q * kFinishThreads;
      key[e] = k_reg[q];
      idx[e] = uint32_t(e);
      lcp[e] = lcp_reg[q];
    }
    __syncthreads();
    // bitonic sort of (key, slot) over the next power of two >= n
    uint32_t pw = 2;
    while (pw < n) pw <<= 1;
    for (uint32_t kb = 2; kb <= pw; kb <<= 1) {
      for (uint32_t j = kb >> 1; j > 0; j >>= 1) {
        for (uint32_t e = t; e < pw / 2; e += kFinishThreads) {
          const uint32_t i = (e / j) * 2 * j + (e % j);
          const uint32_t l = i + j;
          const bool asc = (i & kb) == 0;
          const uint64_t ka = key[i], kl = key[l];
          const uint32_t ia = idx[i], il = idx[l];
          const bool greater = ka > kl || (ka == kl && ia > il);
          if (greater == asc) {
            key[i] = kl;
            key[l] = ka;
            idx[i] = il;
            idx[l] = ia;
          }
        }
        __syncthreads();
      }
    }
    // run starts (t0) and class starts (t1) of every sorted position
    for (int e = t; e < P; e += kFinishThreads) {
      uint32_t rs = 0, cs = 0;
      if (uint32_t(e) < n) {
        rs = (e == 0 || key[e] != key[e - 1]) ? uint32_t(e) : 0u;
        cs = (e == 0 || (key[e] >> lo_bits) / 3u != (key[e - 1] >> lo_bits) / 3u) ? uint32_t(e)
                                                                                    : 0u;
      }
      t0[e] = rs;
      t1[e] = cs;
    }
    __syncthreads();
    block_scan<false>(t0, wsum);
    block_scan<false>(t1, wsum);
    // place or keep
    uint32_t keep_reg[kFinishPer], ng[kFinishPer], nb[kFinishPer], nd[kFinishPer];
#pragma unroll
    for (int q = 0; q < kFinishPer; ++q) {
      const int j = t + q * kFinishThreads;
      keep_reg[q] = 0u;
      if (uint32_t(j) >= n) continue;
      const uint32_t i = idx[j];
      const uint32_t hn = t0[j], ho = t1[j];
      const uint32_t base = bas[i] + (hn - ho);
      const uint64_t kj = key[j];
      const bool single = hn == uint32_t(j) && (uint32_t(j) + 1 == n || key[j + 1] != kj);
      const bool ended = uint32_t((kj >> lo_bits) % 3u) == kEq || (kj & lo_mask) % end1 == end;
      const uint32_t g = grp[i];
      if (single || ended) {
        const int s = workset_of(gb, g);
        const uint32_t at = base + (uint32_t(j) - hn) - gb.base[s];
        if (at < uint32_t(perm.groups[s])) perm.p[s][at] = g - gb.base[s];
        else status[0] = 2u;  // a position outside the workset: never written
      } else {
        keep_reg[q] = 1u;
        ng[q] = g;
        nb[q] = base;
        nd[q] = lcp[i] + 1u;
      }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kFinishPer; ++q) t0[t + q * kFinishThreads] = keep_reg[q];
    __syncthreads();
    const uint32_t kept_last = t0[P - 1];
    __syncthreads();
    block_scan<true>(t0, wsum);
    const uint32_t next_n = t0[P - 1] + kept_last;
#pragma unroll
    for (int q = 0; q < kFinishPer; ++q) {
      if (!keep_reg[q]) continue;
      const uint32_t slot = t0[t + q * kFinishThreads];
      grp[slot] = ng[q];
      bas[slot] = nb[q];
      dep[slot] = nd[q];
    }
    __syncthreads();
    n = next_n;
  }
}

// or_and[0] |= OR of the keys, or_and[1] &= AND of the keys.
__global__ void key_span_kernel(const uint64_t* __restrict__ keys, uint32_t n,
                                unsigned long long* __restrict__ or_and) {
  unsigned long long o = 0ull, a = ~0ull;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    o |= keys[i];
    a &= keys[i];
  }
  for (int d = 1; d < kWave; d <<= 1) {
    o |= __shfl_xor(o, d, kWave);
    a &= __shfl_xor(a, d, kWave);
  }
  if (lane_id() == 0) {
    atomicOr(&or_and[0], o);
    atomicAnd(&or_and[1], a);
  }
}

// Combined key when both parts fit: hi << lo_bits | lo.
__global__ void order_combine_kernel(uint32_t n, const uint64_t* __restrict__ hi,
                                     const uint64_t* __restrict__ lo, int lo_bits,
                                     uint64_t* __restrict__ key) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    key[i] = (hi[i] << lo_bits) | lo[i];
}

// key[j] = part[src[j]] (the second key of a two-pass sort, in first-pass order).
__global__ void order_permute_key_kernel(uint32_t n, const uint32_t* __restrict__ src,
                                         const uint64_t* __restrict__ part,
                                         uint64_t* __restrict__ key) {
  for (uint32_t j = blockIdx.x * blockDim.x + threadIdx.x; j < n; j += gridDim.x * blockDim.x)
    key[j] = part[src[j]];
}

// After the sort: new_head / old_head flag the starts of runs of equal keys and
// of classes; the members' group, base and lcp follow their sorted positions.
__global__ void order_runs_kernel(uint32_t n, const uint32_t* __restrict__ src,
                                  const uint64_t* __restrict__ hi, const uint64_t* __restrict__ lo,
                                  uint32_t* __restrict__ new_head, uint32_t* __restrict__ old_head) {
  for (uint32_t j = blockIdx.x * blockDim.x + threadIdx.x; j < n; j += gridDim.x * blockDim.x) {
    const uint32_t i = src[j];
    if (j == 0) {
      new_head[j] = 1u;
      old_head[j] = 1u;
      continue;
    }
    const uint32_t p = src[j - 1];
    new_head[j] = (hi[i] != hi[p] || lo[i] != lo[p]) ? 1u : 0u;
    old_head[j] = (hi[i] / 3u != hi[p] / 3u) ? 1u : 0u;
  }
}

// new_at[c] / old_at[c] = sorted index where run c begins (runs numbered by the
// exclusive scans of the head flags).
__global__ void order_heads_kernel(uint32_t n, const uint32_t* __restrict__ new_head,
                                   const uint32_t* __restrict__ new_rank,
                                   const uint32_t* __restrict__ old_head,
                                   const uint32_t* __restrict__ old_rank,
                                   uint32_t* __restrict__ new_at, uint32_t* __restrict__ old_at) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    if (new_head[i]) new_at[new_rank[i]] = i;
    if (old_head[i]) old_at[old_rank[i]] = i;
  }
}

// A run's base = its class base + the run's offset inside the class. Placed
// members write the permutation; the others (keep = 1) carry their new class
// base and depth lcp + 1.
__global__ void order_resolve_kernel(uint32_t n, const uint32_t* __restrict__ src,
                                     const uint64_t* __restrict__ hi,
                                     const uint64_t* __restrict__ lo, uint32_t end,
                                     const uint32_t* __restrict__ act_group,
                                     const uint32_t* __restrict__ act_base,
                                     const uint32_t* __restrict__ lcp,
                                     const uint32_t* __restrict__ new_head,
                                     const uint32_t* __restrict__ new_rank,
                                     const uint32_t* __restrict__ old_head,
                                     const uint32_t* __restrict__ old_rank,
                                     const uint32_t* __restrict__ new_at,
                                     const uint32_t* __restrict__ old_at, GroupBase gb,
                                     SigTable perm, uint32_t* __restrict__ keep,
                                     uint32_t* __restrict__ next_group,
                                     uint32_t* __restrict__ next_base,
                                     uint32_t* __restrict__ next_depth) {
  for (uint32_t j = blockIdx.x * blockDim.x + threadIdx.x; j < n; j += gridDim.x * blockDim.x) {
    const uint32_t i = src[j];
    const uint32_t hn = new_at[new_rank[j] + new_head[j] - 1];
    const uint32_t ho = old_at[old_rank[j] + old_head[j] - 1];
    const uint32_t base = act_base[i] + (hn - ho);
    const bool single = new_head[j] && (j + 1 == n || new_head[j + 1]);
    const bool ended = uint32_t(hi[i] % 3u) == kEq || lo[i] % (uint64_t(end) + 1u) == end;
    const uint32_t g = act_group[i];
    if (single || ended) {
      const int s = workset_of(gb, g);
      const uint32_t at = base + (j - hn) - gb.base[s];
      if (at < uint32_t(perm.groups[s])) perm.p[s][at] = g - gb.base[s];  // always, if correct
      keep[j] = 0u;
    } else {
      keep[j] = 1u;
    }
    next_group[j] = g;
    next_base[j] = base;
    next_depth[j] = lcp[i] + 1u;
  }
}

__global__ void order_compact_kernel(uint32_t n, const uint32_t* __restrict__ keep,
                                     const uint32_t* __restrict__ slot,
                                     const uint32_t* __restrict__ next_group,
                                     const uint32_t* __restrict__ next_base,
                                     const uint32_t* __restrict__ next_depth,
                                     uint32_t* __restrict__ act_group,
                                     uint32_t* __restrict__ act_base,
                                     uint32_t* __restrict__ act_depth) {
  for (uint32_t j = blockIdx.x * blockDim.x + threadIdx.x; j < n; j += gridDim.x * blockDim.x) {
    if (keep[j]) {
      act_group[slot[j]] = next_group[j];
      act_base[slot[j]] = next_base[j];
      act_depth[slot[j]] = next_depth[j];
    }
  }
}

__global__ void iota_kernel(uint32_t* __restrict__ out, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    out[i] = uint32_t(i);
}

__global__ void signature_keys_kernel(const uint32_t* __restrict__ word,
                                      const uint32_t* __restrict__ perm, int n,
                                      uint32_t* __restrict__ keys) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    keys[i] = ~word[perm[i]];
}

// or_and[2w] |= OR over groups of word w, or_and[2w+1] &= AND (pre-set to 0 / ~0).
__global__ void signature_span_kernel(const uint32_t* __restrict__ sig, int groups,
                                      uint32_t* __restrict__ or_and) {
  const uint32_t* word = sig + size_t(blockIdx.y) * groups;
  uint32_t o = 0u, a = ~0u;
  for (int g = blockIdx.x * blockDim.x + threadIdx.x; g < groups; g += gridDim.x * blockDim.x) {
    const uint32_t v = word[g];
    o |= v;
    a &= v;
  }
  for (int d = 1; d < kWave; d <<= 1) {
    o |= __shfl_xor(o, d, kWave);
    a &= __shfl_xor(a, d, kWave);
  }
  if (lane_id() == 0) {
    atomicOr(&or_and[2 * blockIdx.y], o);
    atomicAnd(&or_and[2 * blockIdx.y + 1], a);
  }
}

__global__ void permute_meta_kernel(const uint32_t* __restrict__ perm, int groups,
                                    const int* __restrict__ src_des, int* __restrict__ des,
                                    const int* __restrict__ src_len, uint32_t* __restrict__ len,
                                    const uint8_t* __restrict__ src_atomic,
                                    uint8_t* __restrict__ atomic) {
  for (int k = blockIdx.x * blockDim.x + threadIdx.x; k <= groups; k += gridDim.x * blockDim.x) {
    if (k == groups) {
      if (len) len[k] = 0;  // scan sentinel
      continue;
    }
    const uint32_t src = perm[k];
    des[k] = src_des[src];
    if (len) len[k] = uint32_t(src_len[src]);
    if (atomic) atomic[k] = src_atomic[src];
  }
}

// Groups of at most 32 nonzeros (residue, or blocks of 32): one 32-lane half
// wave per group, each lane ranks its (column, ranked index) key against the
// group's other keys.
__global__ void gather_small_kernel(int gs, const uint32_t* __restrict__ perm, int groups,
                                    const int* __restrict__ group_start,
                                    const int* __restrict__ offset,
                                    const uint32_t* __restrict__ ranked_vals,
                                    const int* __restrict__ col_ind,
                                    const float* __restrict__ sp_data, int* __restrict__ out_col,
                                    float* __restrict__ out_val, int* __restrict__ out_pos) {
  const int gid = blockIdx.x * blockDim.x + threadIdx.x;
  const int k = gid >> 5;
  const int t = gid & 31;
  const int lane = lane_id();
  const int half = lane & 32;
  const bool has = k < groups;
  int len = 0, dst = 0, col = 0x7fffffff, p = 0;
  if (has) {
    len = gs ? 32 : offset[k + 1] - offset[k];
    dst = gs ? k * 32 : offset[k];
    if (t < len) {
      p = int(ranked_vals[group_start[perm[k]] + t]);
      col = col_ind[p];
    }
  }
  int rank = 0;
  for (int u = 0; u < 32; ++u) {
    const int cu = __shfl(col, half + u, kWave);
    rank += (u < len) && (cu < col || (cu == col && u < t));
  }
  if (has && t < len) {
    out_col[dst + rank] = col;
    out_val[dst + rank] = sp_data[p];
    if (out_pos) out_pos[dst + rank] = p;
  }
}

// Blocks of 64 .. 8192 nonzeros: bitonic sort of (column << 32 | ranked index)
// in LDS, `tile / gs` groups per workgroup.
__global__ __launch_bounds__(kThreads) void gather_bitonic_kernel(
    int gs, int tile, const uint32_t* __restrict__ perm, int groups,
    const int* __restrict__ group_start, const uint32_t* __restrict__ ranked_vals,
    const int* __restrict__ col_ind, const float* __restrict__ sp_data, int* __restrict__ out_col,
    float* __restrict__ out_val, int* __restrict__ out_pos) {
  extern __shared__ uint64_t smem[];
  uint64_t* keys = smem;
  uint32_t* pos = reinterpret_cast<uint32_t*>(smem + tile);
  const int per_block = tile / gs;
  const int first = blockIdx.x * per_block;
  for (int e = threadIdx.x; e < tile; e += blockDim.x) {
    const int k = first + e / gs;
    const int t = e % gs;
    if (k < groups) {
      const uint32_t p = ranked_vals[group_start[perm[k]] + t];
      keys[e] = (uint64_t(uint32_t(col_ind[p])) << 32) | uint32_t(t);
      pos[e] = p;
    } else {
      keys[e] = ~0ull;
      pos[e] = 0;
    }
  }
  __syncthreads();
  for (int k2 = 2; k2 <= gs; k2 <<= 1) {
    for (int j = k2 >> 1; j > 0; j >>= 1) {
      for (int e = threadIdx.x; e < tile / 2; e += blockDim.x) {
        const int i = (e / j) * 2 * j + (e % j);
        const int l = i + j;
        const bool asc = (k2 == gs) || ((i & k2) == 0);
        const uint64_t a = keys[i], b = keys[l];
        if ((a > b) == asc) {
          keys[i] = b;
          keys[l] = a;
          const uint32_t tp = pos[i];
          pos[i] = pos[l];
          pos[l] = tp;
        }
      }
      __syncthreads();
    }
  }
  for (int e = threadIdx.x; e < tile; e += blockDim.x) {
    const int k = first + e / gs;
    if (k < groups) {
      const size_t dst = size_t(k) * gs + (e % gs);
      out_col[dst] = int(keys[e] >> 32);
      out_val[dst] = sp_data[pos[e]];
      if (out_pos) out_pos[dst] = int(pos[e]);
    }
  }
}

// Blocks larger than one LDS tile: lay the members out in group order with key
// (sorted group index << col_bits | column); a stable radix sort of these keys
// then orders each group by column with ties in ranked order.
__global__ void large_group_keys_kernel(int gs, const uint32_t* __restrict__ perm, int groups,
                                        const int* __restrict__ group_start,
                                        const uint32_t* __restrict__ ranked_vals,
                                        const int* __restrict__ col_ind, int col_bits,
                                        uint64_t* __restrict__ keys, uint32_t* __restrict__ vals) {
  const size_t total = size_t(groups) * gs;
  for (size_t e = size_t(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
       e += size_t(gridDim.x) * blockDim.x) {
    const int k = int(e / gs);
    const int t = int(e % gs);
    const uint32_t p = ranked_vals[group_start[perm[k]] + t];
    keys[e] = (uint64_t(k) << col_bits) | uint32_t(col_ind[p]);
    vals[e] = p;
  }
}

__global__ void large_group_write_kernel(size_t total, const uint64_t* __restrict__ keys,
                                         const uint32_t* __restrict__ vals, int col_bits,
                                         const float* __restrict__ sp_data,
                                         int* __restrict__ out_col, float* __restrict__ out_val,
                                         int* __restrict__ out_pos) {
  const uint64_t mask = (1ull << col_bits) - 1;
  for (size_t e = size_t(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
       e += size_t(gridDim.x) * blockDim.x) {
    out_col[e] = int(keys[e] & mask);
    out_val[e] = sp_data[vals[e]];
    if (out_pos) out_pos[e] = int(vals[e]);
  }
}

// ---- task order ----

// out_base[perm[k]] = where public group k (signature order) starts in its
// workset: k * gs for blocks, pub_offset[k] for the residue.
__global__ void exec_positions_kernel(int gs, const uint32_t* __restrict__ perm, int groups,
                                      const int* __restrict__ pub_offset,
                                      int* __restrict__ out_base) {
  for (int k = blockIdx.x * blockDim.x + threadIdx.x; k < groups; k += gridDim.x * blockDim.x)
    out_base[perm[k]] = gs ? k * gs : pub_offset[k];
}

// Locality score: for `windows` windows of `window` consecutive elements of
// the concatenated column sequence (sampled evenly), the number of distinct
// columns, counted by inserting into one open-addressing hash table per
// window (2 * window slots, 0 = empty, keys stored as column + 1).
struct SeqTable {
  const int* p[PS_MAX_WORKSETS];
  uint64_t begin[PS_MAX_WORKSETS + 1];
  int count;
};

__global__ void window_distinct_kernel(SeqTable seq, uint64_t stride, uint32_t window,
                                       uint32_t slots_log2, uint32_t* __restrict__ tables,
                                       unsigned long long* __restrict__ distinct) {
  const uint32_t w = blockIdx.y;
  uint32_t* table = tables + (size_t(w) << slots_log2);
  const uint32_t mask = (1u << slots_log2) - 1;
  const uint64_t first = uint64_t(w) * stride;
  uint32_t added = 0;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < window;
       i += gridDim.x * blockDim.x) {
    const uint64_t e = first + i;
    int a = 0;
    while (a + 1 < seq.count && e >= seq.begin[a + 1]) ++a;
    const uint32_t key = uint32_t(seq.p[a][e - seq.begin[a]]) + 1u;
    uint32_t h = (key * 2654435761u) >> (32 - slots_log2);
    for (;;) {  // load factor <= 1/2: a free slot or the key is always found
      const uint32_t prev = atomicCAS(&table[h], 0u, key);
      if (prev == 0u) {
        ++added;
        break;
      }
      if (prev == key) break;
      h = (h + 1) & mask;
    }
  }
  for (int d = 1; d < kWave; d <<= 1) added += __shfl_xor(added, d, kWave);
  if (lane_id() == 0 && added) atomicAdd(&distinct[0], (unsigned long long)added);
}

unsigned grid_for(size_t n) {
  const size_t b = (n + kThreads - 1) / kThreads;
  return unsigned(b == 0 ? 1 : (b < 1048576 ? b : 1048576));
}

int bits_for(uint64_t v) {  // bits needed to hold values 0..v
  int b = 0;
  while (b < 64 && (v >> b) != 0) ++b;
  return b;
}

// One device allocation cut into 256-byte aligned arrays, freed when the
// object leaves scope (the free waits for the device, so queued work that
// still reads the arrays completes first).
class Scratch {
 public:
  static size_t bytes(size_t n, size_t elem) { return (n * elem + 255) & ~size_t(255); }
  explicit Scratch(size_t total) : err_(dev_malloc(&base_, total ? total : 1)) {}
  ~Scratch() {
    if (base_) dev_free(base_);
  }
  Scratch(const Scratch&) = delete;
  Scratch& operator=(const Scratch&) = delete;
  hipError_t error() const { return err_; }
  template <typename T>
  T* take(size_t n) {
    T* p = reinterpret_cast<T*>(static_cast<char*>(base_) + used_);
    used_ += bytes(n, sizeof(T));
    return p;
  }

 private:
  void* base_ = nullptr;
  size_t used_ = 0;
  hipError_t err_;
};

// Global group numbering over the worksets; false if the total overflows.
bool make_group_base(int S, const int* group_num, GroupBase* gb) {
  uint64_t total = 0;
  for (int s = 0; s <= PS_MAX_WORKSETS; ++s) {
    if (s < S) {
      if (group_num[s] < 0) return false;
      gb->base[s] = uint32_t(total);
      total += uint64_t(group_num[s]);
      if (total >= (uint64_t(1) << 31)) return false;
    } else {
      gb->base[s] = uint32_t(total);
    }
  }
  gb->S = S;
  return true;
}

}  // namespace
}  // namespace ps

extern "C" {

int ps_pre_degree_sums(const int* row_ptr, int rows, unsigned long long* sums_host,
                       ps_stream_t stream) {
  PS_CHECK_ARG(row_ptr && rows > 0 && sums_host, "ps_pre_degree_sums: bad argument");
  hipStream_t st = ps::to_hip(stream);
  unsigned long long* d_sums = nullptr;
  PS_HIP(ps::dev_malloc(&d_sums, 32 * sizeof(unsigned long long)));
  hipError_t e = hipMemsetAsync(d_sums, 0, 32 * sizeof(unsigned long long), st);
  if (e == hipSuccess) {
    const unsigned grid = ps::grid_for(size_t(rows)) < 4096 ? ps::grid_for(size_t(rows)) : 4096;
    ps::degree_sums_kernel<<<grid, ps::kThreads, 0, st>>>(row_ptr, rows, d_sums);
    e = hipGetLastError();
  }
  if (e == hipSuccess)
    e = hipMemcpyAsync(sums_host, d_sums, 32 * sizeof(unsigned long long),
                       hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  ps::dev_free(d_sums);
  PS_HIP(e);
  return PS_OK;
}

int ps_pre_col_histogram(const int* col_ind, int nnz, int* col_nnz, ps_stream_t stream) {
  PS_CHECK_ARG(col_ind && col_nnz && nnz > 0, "ps_pre_col_histogram: bad argument");
  static_assert(ps::kHistSlots == 1 << 12, "col_hist_kernel hashes to 12 bits");
  const unsigned chunks = unsigned((size_t(nnz) + ps::kHistChunk - 1) / ps::kHistChunk);
  ps::col_hist_kernel<<<chunks, ps::kThreads, 0, ps::to_hip(stream)>>>(col_ind, nnz, col_nnz);
  PS_LAUNCHED();
  return PS_OK;
}

int ps_pre_rank_keys(const int* row_ptr, int rows, const int* col_ind, int nnz,
                     const int* col_nnz, int max_count, int count_bits, uint64_t* keys,
                     uint32_t* vals, ps_stream_t stream) {
  PS_CHECK_ARG(row_ptr && col_ind && col_nnz && keys && vals && nnz > 0 && rows > 0,
               "ps_pre_rank_keys: bad argument");
  PS_CHECK_ARG(count_bits >= 0 && count_bits + ps::bits_for(uint64_t(rows - 1)) <= 64,
               "ps_pre_rank_keys: key does not fit 64 bits");
  ps::rank_keys_kernel<<<ps::grid_for(size_t(nnz)), ps::kThreads, 0, ps::to_hip(stream)>>>(
      row_ptr, rows, col_ind, nnz, col_nnz, max_count, count_bits, keys, vals);
  PS_LAUNCHED();
  return PS_OK;
}

int ps_pre_rank_sort(const int* row_ptr, int rows, const int* col_ind, int nnz,
                     const int* col_nnz, int max_count, int count_bits, uint64_t* keys,
                     uint32_t* vals, ps_stream_t stream) {
  PS_CHECK_ARG(row_ptr && col_ind && col_nnz && keys && vals && nnz > 0 && rows > 0,
               "ps_pre_rank_sort: bad argument");
  PS_CHECK_ARG(count_bits >= 0 && count_bits <= 32 &&
                   count_bits + ps::bits_for(uint64_t(rows - 1)) <= 64,
               "ps_pre_rank_sort: key does not fit 64 bits");
  hipStream_t st = ps::to_hip(stream);
  const size_t R = size_t(rows);
  using S = ps::Scratch;
  S ws(S::bytes(3 * R, 4) * 2 + S::bytes(R, 4) * 3 + S::bytes(R + 1, 4) +
       ps_scan_workspace_bytes(R + 1));
  PS_HIP(ws.error());
  uint32_t* flag = ws.take<uint32_t>(3 * R);
  uint32_t* slot = ws.take<uint32_t>(3 * R);
  uint32_t* list1 = ws.take<uint32_t>(R);
  uint32_t* list2 = ws.take<uint32_t>(R);
  uint32_t* list3 = ws.take<uint32_t>(R);
  uint32_t* long_start = ws.take<uint32_t>(R + 1);
  void* scan_ws = ws.take<char>(ps_scan_workspace_bytes(R + 1));
  // rows of up to 64 nonzeros
  {
    const unsigned waves = ps::kThreads / ps::kWave;
    ps::rank_small_kernel<<<unsigned((R + waves - 1) / waves), ps::kThreads, 0, st>>>(
        row_ptr, rows, col_ind, col_nnz, max_count, count_bits, keys, vals);
    PS_LAUNCHED();
  }
  // lists of the longer rows, per class
  ps::rank_classify_kernel<<<ps::grid_for(R), ps::kThreads, 0, st>>>(row_ptr, rows, flag);
  PS_LAUNCHED();
  for (int c = 0; c < 3; ++c) {
    const int rc = ps_exclusive_scan_u32(flag + c * R, slot + c * R, R, scan_ws, stream);
    if (rc != PS_OK) return rc;
  }
  ps::rank_lists_kernel<<<ps::grid_for(R), ps::kThreads, 0, st>>>(rows, flag, slot, list1, list2,
                                                                   list3);
  PS_LAUNCHED();
  uint32_t tail_slot[3], tail_flag[3];
  for (int c = 0; c < 3; ++c) {
    PS_HIP(hipMemcpyAsync(&tail_slot[c], slot + (c + 1) * R - 1, 4, hipMemcpyDeviceToHost, st));
    PS_HIP(hipMemcpyAsync(&tail_flag[c], flag + (c + 1) * R - 1, 4, hipMemcpyDeviceToHost, st));
  }
  PS_HIP(hipStreamSynchronize(st));
  const uint32_t n1 = tail_slot[0] + tail_flag[0];
  const uint32_t n2 = tail_slot[1] + tail_flag[1];
  const uint32_t n3 = tail_slot[2] + tail_flag[2];
  int rc = PS_OK;
  if (n1 > 0) {
    ps::rank_tile_kernel<<<n1, ps::kThreads, ps::kRankTileSmall * sizeof(uint64_t), st>>>(
        list1, row_ptr, col_ind, col_nnz, max_count, count_bits, keys, vals);
    PS_LAUNCHED();
  }
  if (n2 > 0) {
    const size_t lds = size_t(ps::kRankTileLarge) * sizeof(uint64_t);
    PS_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&ps::rank_tile_kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
    ps::rank_tile_kernel<<<n2, ps::kThreads, lds, st>>>(list2, row_ptr, col_ind, col_nnz,
                                                        max_count, count_bits, keys, vals);
    PS_LAUNCHED();
  }
  if (n3 > 0) {
    // element offsets of the long rows, in list order
    PS_HIP(hipMemsetAsync(long_start, 0, (R + 1) * 4, st));
    ps::permute_long_degrees_kernel<<<ps::grid_for(n3), ps::kThreads, 0, st>>>(
        list3, n3, row_ptr, long_start);
    PS_LAUNCHED();
    rc = ps_exclusive_scan_u32(long_start, long_start, size_t(n3) + 1, scan_ws, stream);
    if (rc != PS_OK) return rc;
    uint32_t total = 0;
    PS_HIP(hipMemcpyAsync(&total, long_start + n3, 4, hipMemcpyDeviceToHost, st));
    PS_HIP(hipStreamSynchronize(st));
    const int list_bits = ps::bits_for(uint64_t(n3 - 1));
    PS_CHECK_ARG(list_bits + count_bits <= 64, "ps_pre_rank_sort: key does not fit 64 bits");
    S lw(2 * S::bytes(total, 8) + 2 * S::bytes(total, 4) + ps_radix_workspace_bytes(total));
    PS_HIP(lw.error());
    uint64_t* ck = lw.take<uint64_t>(total);
    uint64_t* ck_alt = lw.take<uint64_t>(total);
    uint32_t* cv = lw.take<uint32_t>(total);
    uint32_t* cv_alt = lw.take<uint32_t>(total);
    void* radix_ws = lw.take<char>(ps_radix_workspace_bytes(total));
    ps::rank_long_keys_kernel<<<n3, ps::kThreads, 0, st>>>(list3, long_start, row_ptr, col_ind,
                                                           col_nnz, max_count, count_bits, ck, cv);
    PS_LAUNCHED();
    int alt = 0;
    rc = ps_radix_sort_pairs_u64(ck, ck_alt, cv, cv_alt, total, 0, list_bits + count_bits,
                                 radix_ws, &alt, stream);
    if (rc != PS_OK) return rc;
    ps::rank_long_write_kernel<<<ps::grid_for(total), ps::kThreads, 0, st>>>(
        total, alt ? ck_alt : ck, alt ? cv_alt : cv, list3, long_start, row_ptr, count_bits,
        keys, vals);
    PS_LAUNCHED();
    PS_HIP(hipStreamSynchronize(st));
  }
  PS_HIP(hipStreamSynchronize(st));
  return PS_OK;
}

int ps_pre_group_counts(const int* row_ptr, int rows, int group_type_num, int fine,
                        uint32_t* counts, ps_stream_t stream) {
  PS_CHECK_ARG(row_ptr && counts && rows > 0 && group_type_num >= 1 &&
                   group_type_num <= PS_MAX_WORKSETS && fine > 0,
               "ps_pre_group_counts: bad argument");
  ps::group_counts_kernel<<<ps::grid_for(size_t(rows) + 1), ps::kThreads, 0,
                            ps::to_hip(stream)>>>(row_ptr, rows, group_type_num, fine, counts);
  PS_LAUNCHED();
  return PS_OK;
}

int ps_pre_group_meta(const int* row_ptr, int rows, int group_type_num, int fine,
                      const uint32_t* prefix, int* const* group_des, int* const* group_start,
                      int* residue_len, uint8_t* residue_atomic, ps_stream_t stream) {
  PS_CHECK_ARG(row_ptr && prefix && group_des && group_start && rows > 0 &&
                   group_type_num >= 1 && group_type_num <= PS_MAX_WORKSETS,
               "ps_pre_group_meta: bad argument");
  ps::PtrTable des{}, start{};
  for (int s = 0; s < group_type_num; ++s) {
    des.p[s] = group_des[s];
    start.p[s] = group_start[s];
  }
  ps::group_meta_kernel<<<ps::grid_for(size_t(rows)), ps::kThreads, 0, ps::to_hip(stream)>>>(
      row_ptr, rows, group_type_num, fine, prefix, des, start, residue_len, residue_atomic);
  PS_LAUNCHED();
  return PS_OK;
}

int ps_pre_signatures(const int* row_ptr, int rows, int group_type_num, int fine,
                      const uint64_t* ranked_keys, int count_bits, const uint32_t* ranked_vals,
                      int nnz, const int* col_ind, const int* sigbit, const uint32_t* prefix,
                      const int* group_num, uint32_t* const* sig, ps_stream_t stream) {
  PS_CHECK_ARG(row_ptr && ranked_keys && ranked_vals && col_ind && sigbit && prefix &&
                   group_num && sig && nnz > 0 && group_type_num >= 1 &&
                   group_type_num <= PS_MAX_WORKSETS,
               "ps_pre_signatures: bad argument");
  ps::SigTable t{};
  for (int s = 0; s < group_type_num; ++s) {
    t.p[s] = sig[s];
    t.groups[s] = group_num[s];
  }
  ps::signatures_kernel<<<ps::grid_for(size_t(nnz)), ps::kThreads, 0, ps::to_hip(stream)>>>(
      row_ptr, rows, group_type_num, fine, ranked_keys, count_bits, ranked_vals, nnz, col_ind,
      sigbit, prefix, t);
  PS_LAUNCHED();
  return PS_OK;
}

int ps_pre_signature_keys(const uint32_t* sig_word, const uint32_t* perm, int n, uint32_t* keys,
                          ps_stream_t stream) {
  PS_CHECK_ARG(sig_word && keys && n >= 0, "ps_pre_signature_keys: bad argument");
  if (n == 0) return PS_OK;
  PS_CHECK_ARG(perm, "ps_pre_signature_keys: null permutation");
  ps::signature_keys_kernel<<<ps::grid_for(size_t(n)), ps::kThreads, 0, ps::to_hip(stream)>>>(
      sig_word, perm, n, keys);
  PS_LAUNCHED();
  return PS_OK;
}

int ps_iota_u32(uint32_t* out, int n, ps_stream_t stream) {
  PS_CHECK_ARG(out && n >= 0, "ps_iota_u32: bad argument");
  if (n == 0) return PS_OK;
  ps::iota_kernel<<<ps::grid_for(size_t(n)), ps::kThreads, 0, ps::to_hip(stream)>>>(out, n);
  PS_LAUNCHED();
  return PS_OK;
}

int ps_pre_signature_span(const uint32_t* sig, int groups, int words, uint32_t* or_host,
                          uint32_t* and_host, ps_stream_t stream) {
  PS_CHECK_ARG(sig && groups > 0 && words > 0 && words <= 65535 && or_host && and_host,
               "ps_pre_signature_span: bad argument");
  hipStream_t st = ps::to_hip(stream);
  std::vector<uint32_t> init(size_t(words) * 2);
  for (int w = 0; w < words; ++w) {
    init[2 * w] = 0u;
    init[2 * w + 1] = ~0u;
  }
  uint32_t* d = nullptr;
  PS_HIP(ps::dev_malloc(&d, init.size() * sizeof(uint32_t)));
  hipError_t e = hipMemcpyAsync(d, init.data(), init.size() * sizeof(uint32_t),
                                hipMemcpyHostToDevice, st);
  if (e == hipSuccess) {
    unsigned gx = ps::grid_for(size_t(groups));
    if (gx > 64) gx = 64;
    ps::signature_span_kernel<<<dim3(gx, unsigned(words)), ps::kThreads, 0, st>>>(sig, groups, d);
    e = hipGetLastError();
  }
  if (e == hipSuccess)
    e = hipMemcpyAsync(init.data(), d, init.size() * sizeof(uint32_t), hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  ps::dev_free(d);
  PS_HIP(e);
  for (int w = 0; w < words; ++w) {
    or_host[w] = init[2 * w];
    and_host[w] = init[2 * w + 1];
  }
  return PS_OK;
}

int ps_pre_permute_meta(const uint32_t* perm, int groups, const int* src_des, int* des,
                        const int* src_len, uint32_t* len, const uint8_t* src_atomic,
                        uint8_t* atomic, ps_stream_t stream) {
  PS_CHECK_ARG(perm && src_des && des && groups > 0, "ps_pre_permute_meta: bad argument");
  PS_CHECK_ARG((src_len == nullptr) == (len == nullptr) &&
                   (src_atomic == nullptr) == (atomic == nullptr),
               "ps_pre_permute_meta: unpaired residue buffers");
  ps::permute_meta_kernel<<<ps::grid_for(size_t(groups) + 1), ps::kThreads, 0,
                            ps::to_hip(stream)>>>(perm, groups, src_des, des, src_len, len,
                                                  src_atomic, atomic);
  PS_LAUNCHED();
  return PS_OK;
}

int ps_pre_gather_workset(int group_size, const uint32_t* perm, int groups,
                          const int* group_start, const int* residue_offset,
                          const uint32_t* ranked_vals, const int* col_ind, const float* sp_data,
                          int* out_col, float* out_val, int* out_csr_pos, ps_stream_t stream) {
  PS_CHECK_ARG(perm && group_start && ranked_vals && col_ind && sp_data && out_col && out_val &&
                   groups > 0,
               "ps_pre_gather_workset: bad argument");
  PS_CHECK_ARG(group_size == 0 || (group_size >= 32 && (group_size & (group_size - 1)) == 0),
               "ps_pre_gather_workset: group size must be 0 (residue) or a power of two >= 32");
  PS_CHECK_ARG(group_size != 0 || residue_offset, "ps_pre_gather_workset: missing offsets");
  hipStream_t st = ps::to_hip(stream);
  if (group_size <= 32) {
    const size_t threads = size_t(groups) * 32;
    ps::gather_small_kernel<<<unsigned((threads + ps::kThreads - 1) / ps::kThreads),
                              ps::kThreads, 0, st>>>(group_size, perm, groups, group_start,
                                                     residue_offset, ranked_vals, col_ind,
                                                     sp_data, out_col, out_val, out_csr_pos);
    PS_LAUNCHED();
    return PS_OK;
  }
  constexpr int kMaxTile = 8192;
  if (group_size <= kMaxTile) {
    const int tile = group_size > 1024 ? group_size : 1024;
    const size_t lds = size_t(tile) * (sizeof(uint64_t) + sizeof(uint32_t));
    PS_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&ps::gather_bitonic_kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
    const int per_block = tile / group_size;
    const unsigned grid = unsigned((groups + per_block - 1) / per_block);
    ps::gather_bitonic_kernel<<<grid, ps::kThreads, lds, st>>>(
        group_size, tile, perm, groups, group_start, ranked_vals, col_ind, sp_data, out_col,
        out_val, out_csr_pos);
    PS_LAUNCHED();
    return PS_OK;
  }
  // Large groups: radix sort on (sorted group index, column).
  const size_t total = size_t(groups) * group_size;
  const int group_bits = ps::bits_for(uint64_t(groups - 1));
  const int col_bits = 31;
  PS_CHECK_ARG(group_bits + col_bits <= 64, "ps_pre_gather_workset: key overflow");
  uint64_t *keys = nullptr, *keys_alt = nullptr;
  uint32_t *vals = nullptr, *vals_alt = nullptr;
  void* ws = nullptr;
  hipError_t e = ps::dev_malloc(&keys, total * sizeof(uint64_t));
  if (e == hipSuccess) e = ps::dev_malloc(&keys_alt, total * sizeof(uint64_t));
  if (e == hipSuccess) e = ps::dev_malloc(&vals, total * sizeof(uint32_t));
  if (e == hipSuccess) e = ps::dev_malloc(&vals_alt, total * sizeof(uint32_t));
  if (e == hipSuccess) e = ps::dev_malloc(&ws, ps_radix_workspace_bytes(total));
  int rc = PS_OK;
  if (e == hipSuccess) {
    ps::large_group_keys_kernel<<<ps::grid_for(total), ps::kThreads, 0, st>>>(
        group_size, perm, groups, group_start, ranked_vals, col_ind, col_bits, keys, vals);
    e = hipGetLastError();
  }
  int alt = 0;
  if (e == hipSuccess) {
    rc = ps_radix_sort_pairs_u64(keys, keys_alt, vals, vals_alt, total, 0,
                                 col_bits + group_bits, ws, &alt, stream);
  }
  if (e == hipSuccess && rc == PS_OK) {
    ps::large_group_write_kernel<<<ps::grid_for(total), ps::kThreads, 0, st>>>(
        total, alt ? keys_alt : keys, alt ? vals_alt : vals, col_bits, sp_data, out_col,
        out_val, out_csr_pos);
    e = hipGetLastError();
  }
  if (e == hipSuccess && rc == PS_OK) e = hipStreamSynchronize(st);
  ps::dev_free(keys);
  ps::dev_free(keys_alt);
  ps::dev_free(vals);
  ps::dev_free(vals_alt);
  ps::dev_free(ws);
  if (rc != PS_OK) return rc;
  PS_HIP(e);
  return PS_OK;
}

int ps_pre_exec_positions(int group_size, const uint32_t* perm, int groups,
                          const int* pub_offset, int* out_base, ps_stream_t stream) {
  PS_CHECK_ARG(perm && out_base && groups >= 0 && group_size >= 0 &&
                   (group_size > 0 || pub_offset),
               "ps_pre_exec_positions: bad argument");
  if (groups == 0) return PS_OK;
  ps::exec_positions_kernel<<<ps::grid_for(size_t(groups)), ps::kThreads, 0,
                              ps::to_hip(stream)>>>(group_size, perm, groups, pub_offset,
                                                    out_base);
  PS_LAUNCHED();
  return PS_OK;
}

int ps_pre_locality_score(int count, const int* const* col_ind, const long long* lengths,
                          int window, int max_windows, double* score, ps_stream_t stream) {
  PS_CHECK_ARG(count >= 1 && count <= PS_MAX_WORKSETS && col_ind && lengths && score &&
                   window >= 64 && window <= (1 << 24) && max_windows >= 1 &&
                   max_windows <= 65535,
               "ps_pre_locality_score: bad argument");
  ps::SeqTable seq{};
  uint64_t total = 0;
  int n = 0;
  for (int a = 0; a < count; ++a) {
    PS_CHECK_ARG(lengths[a] >= 0, "ps_pre_locality_score: negative length");
    if (lengths[a] == 0) continue;
    PS_CHECK_ARG(col_ind[a], "ps_pre_locality_score: null column array");
    seq.p[n] = col_ind[a];
    seq.begin[n] = total;
    total += uint64_t(lengths[a]);
    ++n;
  }
  seq.count = n;
  seq.begin[n] = total;
  *score = 0.0;
  const uint64_t nwin = total / uint64_t(window);
  if (nwin == 0) return PS_OK;  // shorter than one window: no evidence either way
  const uint32_t windows = uint32_t(nwin < uint64_t(max_windows) ? nwin : uint64_t(max_windows));
  const uint64_t stride = nwin / windows * uint64_t(window);
  uint32_t slots_log2 = 1;
  while ((1u << slots_log2) < 2u * uint32_t(window)) ++slots_log2;
  const size_t table_words = size_t(windows) << slots_log2;
  using S = ps::Scratch;
  S ws(S::bytes(table_words, 4) + S::bytes(1, 8));
  PS_HIP(ws.error());
  uint32_t* tables = ws.take<uint32_t>(table_words);
  unsigned long long* distinct = ws.take<unsigned long long>(1);
  hipStream_t st = ps::to_hip(stream);
  PS_HIP(hipMemsetAsync(tables, 0, table_words * 4, st));
  PS_HIP(hipMemsetAsync(distinct, 0, 8, st));
  unsigned gx = unsigned((uint32_t(window) + ps::kThreads - 1) / ps::kThreads);
  if (gx > 64) gx = 64;
  ps::window_distinct_kernel<<<dim3(gx, windows), ps::kThreads, 0, st>>>(
      seq, stride, uint32_t(window), slots_log2, tables, distinct);
  PS_LAUNCHED();
  unsigned long long host = 0;
  PS_HIP(hipMemcpyAsync(&host, distinct, 8, hipMemcpyDeviceToHost, st));
  PS_HIP(hipStreamSynchronize(st));
  *score = double(host) / (double(windows) * double(window));
  return PS_OK;
}

int ps_pre_signature_lists(const int* row_ptr, int rows, int group_type_num, int fine,
                           const uint64_t* ranked_keys, int count_bits,
                           const uint32_t* ranked_vals, int nnz, const int* col_ind,
                           const int* sigbit, int signature_len, const uint32_t* prefix,
                           const int* group_num, uint32_t* lists, uint32_t* list_begin,
                           ps_stream_t stream) {
  PS_CHECK_ARG(row_ptr && ranked_keys && ranked_vals && col_ind && sigbit && prefix &&
                   group_num && lists && list_begin && rows > 0 && nnz > 0 &&
                   group_type_num >= 1 && group_type_num <= PS_MAX_WORKSETS &&
                   signature_len >= 1 && count_bits >= 0 && count_bits < 64 && fine >= 1,
               "ps_pre_signature_lists: bad argument");
  ps::GroupBase gb{};
  PS_CHECK_ARG(ps::make_group_base(group_type_num, group_num, &gb),
               "ps_pre_signature_lists: bad group counts");
  const uint32_t total = gb.base[group_type_num];
  PS_CHECK_ARG(total > 0, "ps_pre_signature_lists: no groups");
  const int bit_bits = ps::bits_for(uint64_t(signature_len - 1)) > 0
                           ? ps::bits_for(uint64_t(signature_len - 1))
                           : 1;
  const int key_bits = bit_bits + ps::bits_for(uint64_t(total - 1));
  PS_CHECK_ARG(key_bits <= 64, "ps_pre_signature_lists: key overflow");
  const size_t n = size_t(nnz);
  using S = ps::Scratch;
  S ws(2 * S::bytes(n, 8) + 2 * S::bytes(n, 4) + ps_radix_workspace_bytes(n) +
       ps_scan_workspace_bytes(n));
  PS_HIP(ws.error());
  uint64_t* e = ws.take<uint64_t>(n);
  uint64_t* e_alt = ws.take<uint64_t>(n);
  uint32_t* flag = ws.take<uint32_t>(n);
  uint32_t* pos = ws.take<uint32_t>(n);
  void* radix_ws = ws.take<char>(ps_radix_workspace_bytes(n));
  void* scan_ws = ws.take<char>(ps_scan_workspace_bytes(n));
  hipStream_t st = ps::to_hip(stream);
  const unsigned grid = ps::grid_for(n);
  ps::signature_entries_kernel<<<grid, ps::kThreads, 0, st>>>(
      row_ptr, rows, group_type_num, fine, ranked_keys, count_bits, ranked_vals, nnz, col_ind,
      sigbit, prefix, gb, bit_bits, e);
  PS_LAUNCHED();
  int alt = 0;
  int rc = ps_radix_sort_pairs_u64(e, e_alt, nullptr, nullptr, n, 0, key_bits, radix_ws, &alt,
                                   stream);
  if (rc != PS_OK) return rc;
  const uint64_t* sorted = alt ? e_alt : e;
  ps::entry_flags_kernel<<<grid, ps::kThreads, 0, st>>>(sorted, uint32_t(n), flag);
  PS_LAUNCHED();
  rc = ps_exclusive_scan_u32(flag, pos, n, scan_ws, stream);
  if (rc != PS_OK) return rc;
  ps::entry_lists_kernel<<<grid, ps::kThreads, 0, st>>>(sorted, uint32_t(n), bit_bits, flag, pos,
                                                         total, lists, list_begin);
  PS_LAUNCHED();
  PS_HIP(hipStreamSynchronize(st));
  return PS_OK;
}

}  // extern "C"

namespace ps {
namespace {

// Stable radix sort of (key, index) pairs over the bits where the keys differ
// (found by an OR/AND reduction); *k / *v point at the sorted data.
int sort_varying(uint64_t* keys, uint64_t* keys_alt, uint32_t* vals, uint32_t* vals_alt,
                 uint32_t n, unsigned long long* span, void* radix_ws, hipStream_t st,
                 const uint64_t** k, const uint32_t** v) {
  static const unsigned long long span_init[2] = {0ull, ~0ull};
  unsigned long long host_span[2] = {0ull, 0ull};
  *k = keys;
  *v = vals;
  PS_HIP(hipMemcpyAsync(span, span_init, sizeof(span_init), hipMemcpyHostToDevice, st));
  const unsigned grid = grid_for(n);
  key_span_kernel<<<grid < 1024 ? grid : 1024, kThreads, 0, st>>>(keys, n, span);
  PS_LAUNCHED();
  PS_HIP(hipMemcpyAsync(host_span, span, sizeof(host_span), hipMemcpyDeviceToHost, st));
  PS_HIP(hipStreamSynchronize(st));
  const uint64_t diff = host_span[0] ^ host_span[1];
  if (diff == 0) return PS_OK;
  const int lo = __builtin_ctzll(diff) / 8 * 8;
  const int hi = 64 - __builtin_clzll(diff);
  int alt = 0;
  const int rc = ps_radix_sort_pairs_u64(keys, keys_alt, vals, vals_alt, n, lo, hi, radix_ws,
                                         &alt, reinterpret_cast<ps_stream_t>(st));
  if (rc != PS_OK) return rc;
  if (alt) {
    *k = keys_alt;
    *v = vals_alt;
  }
  return PS_OK;
}

}  // namespace
}  // namespace ps

extern "C" {

int ps_pre_signature_order(const uint32_t* lists, const uint32_t* list_begin,
                           int group_type_num, const int* group_num, int signature_len,
                           uint32_t* const* perm, ps_stream_t stream) {
  PS_CHECK_ARG(lists && list_begin && group_num && perm && group_type_num >= 1 &&
                   group_type_num <= PS_MAX_WORKSETS && signature_len >= 1,
               "ps_pre_signature_order: bad argument");
  ps::GroupBase gb{};
  PS_CHECK_ARG(ps::make_group_base(group_type_num, group_num, &gb),
               "ps_pre_signature_order: bad group counts");
  ps::SigTable out{};
  for (int s = 0; s < group_type_num; ++s) {
    PS_CHECK_ARG(group_num[s] == 0 || perm[s], "ps_pre_signature_order: null permutation");
    out.p[s] = perm[s];
    out.groups[s] = group_num[s];
  }
  const uint32_t total = gb.base[group_type_num];
  if (total == 0) return PS_OK;
  // List elements take values 0 .. signature_len - 1; signature_len marks a list's end.
  const uint32_t end = uint32_t(signature_len);
  const size_t n0 = total;
  using S = ps::Scratch;
  S ws(6 * S::bytes(n0, 8) + 17 * S::bytes(n0, 4) + S::bytes(2, 8) + S::bytes(1, 4) +
       ps_radix_workspace_bytes(n0) + ps_scan_workspace_bytes(n0));
  PS_HIP(ws.error());
  uint64_t* hi = ws.take<uint64_t>(n0);
  uint64_t* lo = ws.take<uint64_t>(n0);
  uint64_t* keys = ws.take<uint64_t>(n0);
  uint64_t* keys_alt = ws.take<uint64_t>(n0);
  uint64_t* keys2 = ws.take<uint64_t>(n0);
  uint64_t* keys2_alt = ws.take<uint64_t>(n0);
  uint32_t* act_group = ws.take<uint32_t>(n0);
  uint32_t* act_base = ws.take<uint32_t>(n0);
  uint32_t* act_depth = ws.take<uint32_t>(n0);
  uint32_t* head = ws.take<uint32_t>(n0);
  uint32_t* rank = ws.take<uint32_t>(n0);
  uint32_t* head_at = ws.take<uint32_t>(n0);
  uint32_t* lcp = ws.take<uint32_t>(n0);
  uint32_t* idx = ws.take<uint32_t>(n0);
  uint32_t* idx_alt = ws.take<uint32_t>(n0);
  uint32_t* new_head = ws.take<uint32_t>(n0);
  uint32_t* old_head = ws.take<uint32_t>(n0);
  uint32_t* new_rank = ws.take<uint32_t>(n0);
  uint32_t* old_rank = ws.take<uint32_t>(n0);
  uint32_t* new_at = ws.take<uint32_t>(n0);
  uint32_t* old_at = ws.take<uint32_t>(n0);
  uint32_t* keep = ws.take<uint32_t>(n0);
  uint32_t* slot = ws.take<uint32_t>(n0);
  unsigned long long* span = ws.take<unsigned long long>(2);
  uint32_t* max_len_dev = ws.take<uint32_t>(1);
  void* radix_ws = ws.take<char>(ps_radix_workspace_bytes(n0));
  void* scan_ws = ws.take<char>(ps_scan_workspace_bytes(n0));
  // next_group / next_base / next_depth reuse buffers free after the sort
  uint32_t* next_group = head;
  uint32_t* next_base = head_at;
  uint32_t* next_depth = rank;
  hipStream_t st = ps::to_hip(stream);

  uint32_t max_len = 0;
  PS_HIP(hipMemsetAsync(max_len_dev, 0, 4, st));
  {
    unsigned gx = ps::grid_for(n0);
    ps::max_list_kernel<<<gx < 1024 ? gx : 1024, ps::kThreads, 0, st>>>(list_begin, total,
                                                                        max_len_dev);
    PS_LAUNCHED();
  }
  PS_HIP(hipMemcpyAsync(&max_len, max_len_dev, 4, hipMemcpyDeviceToHost, st));
  ps::order_init_kernel<<<ps::grid_for(n0), ps::kThreads, 0, st>>>(total, gb, act_group,
                                                                   act_base, act_depth);
  PS_LAUNCHED();
  PS_HIP(hipStreamSynchronize(st));
  const int lo_bits = ps::bits_for(uint64_t(max_len) * (uint64_t(end) + 1u) + end);
  uint32_t n = total;
  // The finisher holds class ranks < kFinishMax in 13 bits of its keys.
  const bool finisher = 13 + lo_bits <= 64;
  if (finisher) {
    const size_t lds = ps::kFinishLds;
    PS_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&ps::order_finish_kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
  }
  // Every round places at least each class's reference, so a class of k
  // groups needs at most k rounds.
  for (uint32_t round = 0; n > 0; ++round) {
    if (round > total)
      return ps::fail(PS_ERR_RUNTIME, "ps_pre_signature_order: refinement did not converge");
    if (finisher && n <= uint32_t(ps::kFinishMax)) {
      uint32_t flag = 0;
      PS_HIP(hipMemsetAsync(max_len_dev, 0, 4, st));
      const size_t lds = ps::kFinishLds;
      ps::order_finish_kernel<<<1, ps::kFinishThreads, lds, st>>>(
          n, act_group, act_base, act_depth, lists, list_begin, end, max_len, lo_bits, gb, out,
          max_len_dev);
      PS_LAUNCHED();
      PS_HIP(hipMemcpyAsync(&flag, max_len_dev, 4, hipMemcpyDeviceToHost, st));
      PS_HIP(hipStreamSynchronize(st));
      if (flag)
        return ps::fail(PS_ERR_RUNTIME, flag == 1u
                                            ? "ps_pre_signature_order: refinement did not converge"
                                            : "ps_pre_signature_order: position out of range");
      break;
    }
    const unsigned grid = ps::grid_for(n);
    ps::order_class_heads_kernel<<<grid, ps::kThreads, 0, st>>>(act_base, n, head);
    PS_LAUNCHED();
    int rc = ps_exclusive_scan_u32(head, rank, n, scan_ws, stream);
    if (rc != PS_OK) return rc;
    ps::order_class_start_kernel<<<grid, ps::kThreads, 0, st>>>(n, head, rank, head_at);
    PS_LAUNCHED();
    ps::order_diverge_kernel<<<grid, ps::kThreads, 0, st>>>(
        act_group, act_depth, n, lists, list_begin, head, rank, head_at, end, max_len, hi, lo,
        lcp, idx);
    PS_LAUNCHED();
    // Sort by (hi, lo): one pass over the combined key when it fits 64 bits,
    // else lo first and hi second (both stable).
    const int hi_bits = ps::bits_for(3ull * n);
    const uint64_t* k = nullptr;
    const uint32_t* src = nullptr;
    if (hi_bits + lo_bits <= 64) {
      ps::order_combine_kernel<<<grid, ps::kThreads, 0, st>>>(n, hi, lo, lo_bits, keys);
      PS_LAUNCHED();
      rc = ps::sort_varying(keys, keys_alt, idx, idx_alt, n, span, radix_ws, st, &k, &src);
      if (rc != PS_OK) return rc;
    } else {
      ps::order_permute_key_kernel<<<grid, ps::kThreads, 0, st>>>(n, idx, lo, keys);
      PS_LAUNCHED();
      rc = ps::sort_varying(keys, keys_alt, idx, idx_alt, n, span, radix_ws, st, &k, &src);
      if (rc != PS_OK) return rc;
      uint32_t* first = const_cast<uint32_t*>(src);
      uint32_t* first_alt = first == idx ? idx_alt : idx;
      ps::order_permute_key_kernel<<<grid, ps::kThreads, 0, st>>>(n, first, hi, keys2);
      PS_LAUNCHED();
      rc = ps::sort_varying(keys2, keys2_alt, first, first_alt, n, span, radix_ws, st, &k, &src);
      if (rc != PS_OK) return rc;
    }
    ps::order_runs_kernel<<<grid, ps::kThreads, 0, st>>>(n, src, hi, lo, new_head, old_head);
    PS_LAUNCHED();
    rc = ps_exclusive_scan_u32(new_head, new_rank, n, scan_ws, stream);
    if (rc == PS_OK) rc = ps_exclusive_scan_u32(old_head, old_rank, n, scan_ws, stream);
    if (rc != PS_OK) return rc;
    ps::order_heads_kernel<<<grid, ps::kThreads, 0, st>>>(n, new_head, new_rank, old_head,
                                                          old_rank, new_at, old_at);
    PS_LAUNCHED();
    ps::order_resolve_kernel<<<grid, ps::kThreads, 0, st>>>(
        n, src, hi, lo, end, act_group, act_base, lcp, new_head, new_rank, old_head, old_rank,
        new_at, old_at, gb, out, keep, next_group, next_base, next_depth);
    PS_LAUNCHED();
    rc = ps_exclusive_scan_u32(keep, slot, n, scan_ws, stream);
    if (rc != PS_OK) return rc;
    ps::order_compact_kernel<<<grid, ps::kThreads, 0, st>>>(
        n, keep, slot, next_group, next_base, next_depth, act_group, act_base, act_depth);
    PS_LAUNCHED();
    uint32_t tail[2] = {0u, 0u};
    PS_HIP(hipMemcpyAsync(&tail[0], slot + (n - 1), sizeof(uint32_t), hipMemcpyDeviceToHost, st));
    PS_HIP(hipMemcpyAsync(&tail[1], keep + (n - 1), sizeof(uint32_t), hipMemcpyDeviceToHost, st));
    PS_HIP(hipStreamSynchronize(st));
    n = tail[0] + tail[1];
  }
  return PS_OK;
}

}  // extern "C"
