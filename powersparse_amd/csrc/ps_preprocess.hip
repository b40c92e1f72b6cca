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

__global__ void col_hist_kernel(const int* __restrict__ col_ind, int nnz, int* __restrict__ col_nnz) {
  for (int p = blockIdx.x * blockDim.x + threadIdx.x; p < nnz; p += gridDim.x * blockDim.x)
    atomicAdd(&col_nnz[col_ind[p]], 1);
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

__global__ void signatures_kernel(const int* __restrict__ row_ptr, int rows, int S, int fine,
                                  const uint64_t* __restrict__ ranked_keys, int count_bits,
                                  const uint32_t* __restrict__ ranked_vals, int nnz,
                                  const int* __restrict__ col_ind, const int* __restrict__ sigbit,
                                  const uint32_t* __restrict__ prefix, SigTable sig) {
  const size_t stride = size_t(rows) + 1;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < nnz; i += gridDim.x * blockDim.x) {
    const int r = int(ranked_keys[i] >> count_bits);
    const int base = row_ptr[r];
    const int j = i - base;  // rank of this nonzero inside its row
    int s = 0, g;
    if (S == 1) {
      g = int(prefix[r]) + j / fine;
    } else {
      int rem = row_ptr[r + 1] - base, off = 0;
      g = -1;
      for (int t = S - 1; t > 0; --t) {
        const int gs = group_size(t);
        const int n = rem / gs;
        if (j < off + n * gs) {
          s = t;
          g = int(prefix[t * stride + r]) + (j - off) / gs;
          break;
        }
        off += n * gs;
        rem -= n * gs;
      }
      if (g < 0) g = int(prefix[r]);
    }
    const int bit = sigbit[col_ind[ranked_vals[i]]];
    atomicOr(&sig.p[s][size_t(bit >> 5) * sig.groups[s] + g], 1u << (31 - (bit & 31)));
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
                                    float* __restrict__ out_val) {
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
  }
}

// Blocks of 64 .. 8192 nonzeros: bitonic sort of (column << 32 | ranked index)
// in LDS, `tile / gs` groups per workgroup.
__global__ __launch_bounds__(kThreads) void gather_bitonic_kernel(
    int gs, int tile, const uint32_t* __restrict__ perm, int groups,
    const int* __restrict__ group_start, const uint32_t* __restrict__ ranked_vals,
    const int* __restrict__ col_ind, const float* __restrict__ sp_data, int* __restrict__ out_col,
    float* __restrict__ out_val) {
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
                                         int* __restrict__ out_col, float* __restrict__ out_val) {
  const uint64_t mask = (1ull << col_bits) - 1;
  for (size_t e = size_t(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
       e += size_t(gridDim.x) * blockDim.x) {
    out_col[e] = int(keys[e] & mask);
    out_val[e] = sp_data[vals[e]];
  }
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

}  // namespace
}  // namespace ps

extern "C" {

int ps_pre_degree_sums(const int* row_ptr, int rows, unsigned long long* sums_host,
                       ps_stream_t stream) {
  PS_CHECK_ARG(row_ptr && rows > 0 && sums_host, "ps_pre_degree_sums: bad argument");
  hipStream_t st = ps::to_hip(stream);
  unsigned long long* d_sums = nullptr;
  PS_HIP(hipMalloc(&d_sums, 32 * sizeof(unsigned long long)));
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
  (void)hipFree(d_sums);
  PS_HIP(e);
  return PS_OK;
}

int ps_pre_col_histogram(const int* col_ind, int nnz, int* col_nnz, ps_stream_t stream) {
  PS_CHECK_ARG(col_ind && col_nnz && nnz > 0, "ps_pre_col_histogram: bad argument");
  ps::col_hist_kernel<<<ps::grid_for(size_t(nnz)), ps::kThreads, 0, ps::to_hip(stream)>>>(
      col_ind, nnz, col_nnz);
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
  PS_HIP(hipMalloc(&d, init.size() * sizeof(uint32_t)));
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
  (void)hipFree(d);
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
                          int* out_col, float* out_val, ps_stream_t stream) {
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
                                                     sp_data, out_col, out_val);
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
        out_val);
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
  hipError_t e = hipMalloc(&keys, total * sizeof(uint64_t));
  if (e == hipSuccess) e = hipMalloc(&keys_alt, total * sizeof(uint64_t));
  if (e == hipSuccess) e = hipMalloc(&vals, total * sizeof(uint32_t));
  if (e == hipSuccess) e = hipMalloc(&vals_alt, total * sizeof(uint32_t));
  if (e == hipSuccess) e = hipMalloc(&ws, ps_radix_workspace_bytes(total));
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
        out_val);
    e = hipGetLastError();
  }
  if (e == hipSuccess && rc == PS_OK) e = hipStreamSynchronize(st);
  (void)hipFree(keys);
  (void)hipFree(keys_alt);
  (void)hipFree(vals);
  (void)hipFree(vals_alt);
  (void)hipFree(ws);
  if (rc != PS_OK) return rc;
  PS_HIP(e);
  return PS_OK;
}

}  // extern "C"
