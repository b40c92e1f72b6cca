// Dense hub block: the rows of highest degree restricted to the most popular
// columns, run as dense FP32 products on the matrix cores.
//
// On power-law graphs the heaviest rows hold a dense core with the most
// popular columns (C3: rows of degree >= 4096 x columns with >= 2048
// nonzeros hold 21% of the nonzeros at 43% density). The sparse kernels pay
// one row gather per nonzero there; a dense product over the block does the
// same arithmetic from MFMA tiles with each B / Y row read once per tile.
//
//   SpMM:  C[hub_rows[i], :] += sum_h dense[i][h] * B[hot_cols[h], :]
//          (dense holds the block's stored values, zeros elsewhere). B's hot
//          rows are copied with their non-finite elements replaced by 0, and
//          a fix-up adds a * b for every stored block entry (a bit mask marks
//          them) whose b is not finite, so Inf and NaN reach exactly the rows
//          that store that column, as in the reference's per-nonzero
//          products.
//   SDDMM: D = X[hub_rows] * Y[hot_cols]^T, then every listed tile (64
//          consecutive nonzeros of a block group lying in the block) stores
//          sp_data[p] * D[hub_index[row], hot_rank[col_ind[p]]].
//
// The GEMMs run through hipBLASLt in FP32 (compute type 32F). The callers
// pass the workspace (ps_hub_workspace_bytes); the launchers allocate nothing.
// No reference counterpart: the reference runs every nonzero through its
// sparse kernels (spmm_kernel_block.cu, sddmm_kernel_block.cu).
#include <hipblaslt/hipblaslt.h>

#include <array>
#include <map>
#include <mutex>

#include "ps_common.hpp"

namespace ps {
namespace {

constexpr int kThreads = 256;
constexpr size_t kBlasWorkspace = size_t(32) << 20;  // hipBLASLt workspace limit
constexpr int kMaxDevices = 64;

inline size_t round256(size_t b) { return (b + 255) & ~size_t(255); }

// ------------------------------------------------------------- hipBLASLt

// One handle and one algorithm cache per device, created on first use and
// kept until the process ends (never destroyed: nothing runs at exit).
struct Gemm {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  size_t workspace = 0;
};
struct BlasState {
  std::mutex mu;
  hipblasLtHandle_t handle = nullptr;
  std::map<std::array<int, 8>, Gemm*> plans;
};

BlasState* blas_state(int dev) {
  static std::mutex mu;
  static BlasState* states[kMaxDevices] = {};
  std::lock_guard<std::mutex> lock(mu);
  if (!states[dev]) states[dev] = new BlasState;
  return states[dev];
}

#define PS_BLAS(call)                                                                    \
  do {                                                                                   \
    hipblasStatus_t ps_bs_ = (call);                                                     \
    if (ps_bs_ != HIPBLAS_STATUS_SUCCESS)                                                \
      return ps::fail(PS_ERR_RUNTIME, std::string(__FILE__) + ":" +                      \
                                          std::to_string(__LINE__) + ": " #call ": " +   \
                                          "hipBLASLt status " + std::to_string(ps_bs_)); \
  } while (0)

// Column-major C (m x n) = op(A) (m x k) * op(B) (k x n), FP32 in and out,
// FP32 compute, beta = 0.
int gemm_f32(hipStream_t st, bool ta, bool tb, int m, int n, int k, const float* A, int lda,
             const float* B, int ldb, float* C, int ldc, void* ws, size_t ws_bytes) {
  int dev = 0;
  PS_HIP(hipGetDevice(&dev));
  PS_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "hub block: device index out of range");
  BlasState* s = blas_state(dev);
  std::lock_guard<std::mutex> lock(s->mu);
  if (!s->handle) PS_BLAS(hipblasLtCreate(&s->handle));
  const std::array<int, 8> key = {m, n, k, int(ta), int(tb), lda, ldb, ldc};
  Gemm*& g = s->plans[key];
  if (!g) {
    Gemm* p = new Gemm;
    PS_BLAS(hipblasLtMatmulDescCreate(&p->desc, HIPBLAS_COMPUTE_32F, HIP_R_32F));
    const hipblasOperation_t oa = ta ? HIPBLAS_OP_T : HIPBLAS_OP_N;
    const hipblasOperation_t ob = tb ? HIPBLAS_OP_T : HIPBLAS_OP_N;
    PS_BLAS(hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_TRANSA, &oa, sizeof(oa)));
    PS_BLAS(hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_TRANSB, &ob, sizeof(ob)));
    PS_BLAS(hipblasLtMatrixLayoutCreate(&p->a, HIP_R_32F, ta ? k : m, ta ? m : k, lda));
    PS_BLAS(hipblasLtMatrixLayoutCreate(&p->b, HIP_R_32F, tb ? n : k, tb ? k : n, ldb));
    PS_BLAS(hipblasLtMatrixLayoutCreate(&p->c, HIP_R_32F, m, n, ldc));
    hipblasLtMatmulPreference_t pref;
    PS_BLAS(hipblasLtMatmulPreferenceCreate(&pref));
    size_t limit = kBlasWorkspace;
    PS_BLAS(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                  &limit, sizeof(limit)));
    hipblasLtMatmulHeuristicResult_t res[1];
    int found = 0;
    const hipblasStatus_t hs = hipblasLtMatmulAlgoGetHeuristic(s->handle, p->desc, p->a, p->b,
                                                               p->c, p->c, pref, 1, res, &found);
    (void)hipblasLtMatmulPreferenceDestroy(pref);
    PS_BLAS(hs);
    PS_CHECK_ARG(found > 0, "hub block: hipBLASLt has no FP32 algorithm for this shape");
    p->algo = res[0].algo;
    p->workspace = res[0].workspaceSize;
    g = p;
  }
  PS_CHECK_ARG(g->workspace <= ws_bytes, "hub block: GEMM workspace too small");
  const float alpha = 1.0f, beta = 0.0f;
  PS_BLAS(hipblasLtMatmul(s->handle, g->desc, &alpha, A, g->a, B, g->b, &beta, C, g->c, C, g->c,
                          &g->algo, g->workspace ? ws : nullptr, g->workspace, st));
  return PS_OK;
}

// ------------------------------------------------------------- selection

// hist[a][b] += nonzeros of rows with floor(log2(degree)) = a whose column
// has floor(log2(count)) = b; rows of degree < 256 are skipped. One wave per
// row, the block's counts gathered in LDS.
__global__ __launch_bounds__(kThreads) void hist_kernel(const int* __restrict__ row_ptr, int rows,
                                                         const int* __restrict__ col_ind,
                                                         const int* __restrict__ col_nnz,
                                                         unsigned long long* __restrict__ hist) {
  __shared__ unsigned int h[32 * 32];
  for (int i = threadIdx.x; i < 32 * 32; i += kThreads) h[i] = 0;
  __syncthreads();
  const int waves = kThreads / kWave;
  for (int r = blockIdx.x * waves + threadIdx.x / kWave; r < rows; r += gridDim.x * waves) {
    const int b = row_ptr[r], e = row_ptr[r + 1];
    const int deg = e - b;
    if (deg < 256) continue;
    const int a = 31 - __builtin_clz(unsigned(deg));
    for (int p = b + lane_id(); p < e; p += kWave) {
      const int cnt = col_nnz[col_ind[p]];
      const int q = cnt > 0 ? 31 - __builtin_clz(unsigned(cnt)) : 0;
      atomicAdd(&h[a * 32 + q], 1u);
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 32 * 32; i += kThreads)
    if (h[i]) atomicAdd(&hist[i], (unsigned long long)h[i]);
}

// ------------------------------------------------------------- building

// dense[i][hot_rank[c]] += value for every stored entry of hub row i in a hot
// column (repeated entries add up), and its bit in stored (one bit per dense
// element, words of 32 along each dense row). One workgroup per hub row.
__global__ __launch_bounds__(kThreads) void dense_kernel(ps_hub_block hb,
                                                          const int* __restrict__ row_ptr,
                                                          const int* __restrict__ col_ind,
                                                          const float* __restrict__ sp_data,
                                                          float* __restrict__ dense,
                                                          uint32_t* __restrict__ stored) {
  const size_t words = (size_t(hb.cols) + 31) / 32;
  for (int i = blockIdx.x; i < hb.rows; i += gridDim.x) {
    const int r = hb.hub_rows[i];
    const int b = row_ptr[r], e = row_ptr[r + 1];
    float* drow = dense + size_t(i) * size_t(hb.cols);
    uint32_t* srow = stored + size_t(i) * words;
    for (int p = b + threadIdx.x; p < e; p += kThreads) {
      const int h = hb.hot_rank[col_ind[p]];
      if (h >= 0) {
        atomicAdd(drow + h, sp_data[p]);
        atomicOr(srow + h / 32, 1u << (h % 32));
      }
    }
  }
}

// counts[r] = stored entries of row r outside the block. One wave per row.
__global__ __launch_bounds__(kThreads) void kept_kernel(ps_hub_block hb,
                                                         const int* __restrict__ row_ptr,
                                                         const int* __restrict__ col_ind,
                                                         uint32_t* __restrict__ counts) {
  const int waves = kThreads / kWave;
  for (int r = blockIdx.x * waves + threadIdx.x / kWave; r < hb.matrix_rows;
       r += gridDim.x * waves) {
    const int b = row_ptr[r], e = row_ptr[r + 1];
    uint32_t n = uint32_t(e - b);
    if (hb.hub_index[r] >= 0) {
      uint32_t hot = 0;
      for (int p = b + lane_id(); p < e; p += kWave) hot += hb.hot_rank[col_ind[p]] >= 0;
      for (int o = 32; o > 0; o >>= 1) hot += __shfl_xor(hot, o);
      n -= hot;
    }
    if (lane_id() == 0) counts[r] = n;
  }
}

// The CSR without the block's entries, in the original order within rows.
__global__ __launch_bounds__(kThreads) void compact_kernel(ps_hub_block hb,
                                                            const int* __restrict__ row_ptr,
                                                            const int* __restrict__ col_ind,
                                                            const float* __restrict__ sp_data,
                                                            const uint32_t* __restrict__ new_row_ptr,
                                                            int* __restrict__ new_col,
                                                            float* __restrict__ new_val) {
  const int waves = kThreads / kWave;
  for (int r = blockIdx.x * waves + threadIdx.x / kWave; r < hb.matrix_rows;
       r += gridDim.x * waves) {
    const int b = row_ptr[r], e = row_ptr[r + 1];
    const bool hub = hb.hub_index[r] >= 0;
    uint32_t out = new_row_ptr[r];
    for (int p0 = b; p0 < e; p0 += kWave) {
      const int p = p0 + lane_id();
      const int c = p < e ? col_ind[p] : 0;
      const bool keep = p < e && !(hub && hb.hot_rank[c] >= 0);
      const uint64_t m = __ballot(keep);
      if (keep) {
        const uint32_t at = out + uint32_t(__popcll(m & ((1ull << lane_id()) - 1ull)));
        new_col[at] = c;
        new_val[at] = sp_data[p];
      }
      out += uint32_t(__popcll(m));
    }
  }
}

// flags[t] = 1 when the t-th 64-nonzero stretch of a block workset (groups of
// 64 or more nonzeros, so a stretch lies in one group) lies inside the block:
// its group's row is a hub row and all its 64 columns are hot. One wave per
// stretch, one nonzero per lane.
__global__ __launch_bounds__(kThreads) void tile_flags_kernel(ps_hub_block hb, ps_workset w,
                                                               uint8_t* __restrict__ flags) {
  const int waves = kThreads / kWave;
  const size_t tiles = size_t(w.group_num) * size_t(w.group_size / 64);
  for (size_t t = size_t(blockIdx.x) * waves + threadIdx.x / kWave; t < tiles;
       t += size_t(gridDim.x) * waves) {
    const bool hub = hb.hub_index[w.group_des[t * 64 / size_t(w.group_size)]] >= 0;
    const bool hot = hub && hb.hot_rank[w.col_ind[t * 64 + size_t(lane_id())]] >= 0;
    const bool all = __all(hot ? 1 : 0);
    if (lane_id() == 0) flags[t] = all ? 1 : 0;
  }
}

// residue_atomic[g] = 1 for the residue groups of hub rows: a partition of the
// matrix without the block must add those rows' remaining entries to the
// block's product, not overwrite it.
__global__ __launch_bounds__(kThreads) void mark_atomic_kernel(const int* __restrict__ hub_index,
                                                                const int* __restrict__ des, int G,
                                                                uint8_t* __restrict__ atomic) {
  for (int g = blockIdx.x * kThreads + threadIdx.x; g < G; g += gridDim.x * kThreads)
    if (hub_index[des[g]] >= 0) atomic[g] = 1;
}

// ------------------------------------------------------------- operators

__global__ void clear_flag_kernel(int* flag) { *flag = 0; }

// dst[h][:] = src[idx[h]][:] (N floats per row, N a multiple of 4); with
// `sanitize`, non-finite elements become 0, row_flag[h] records whether the
// row had any and *any_flag is set to 1 if so. One wave per row.
__global__ __launch_bounds__(kThreads) void gather_rows_kernel(const float* __restrict__ src,
                                                                const int* __restrict__ idx,
                                                                int count, int N,
                                                                float* __restrict__ dst,
                                                                int sanitize,
                                                                int* __restrict__ row_flag,
                                                                int* __restrict__ any_flag) {
  const int waves = kThreads / kWave;
  const int q = N / 4;
  for (int h = blockIdx.x * waves + threadIdx.x / kWave; h < count; h += gridDim.x * waves) {
    const float4* s = reinterpret_cast<const float4*>(src + size_t(idx[h]) * size_t(N));
    float4* d = reinterpret_cast<float4*>(dst + size_t(h) * size_t(N));
    bool bad = false;
    for (int j = lane_id(); j < q; j += kWave) {
      float4 v = s[j];
      if (sanitize) {
        const bool fx = isfinite(v.x), fy = isfinite(v.y), fz = isfinite(v.z), fw = isfinite(v.w);
        bad |= !(fx && fy && fz && fw);
        v.x = fx ? v.x : 0.f;
        v.y = fy ? v.y : 0.f;
        v.z = fz ? v.z : 0.f;
        v.w = fw ? v.w : 0.f;
      }
      d[j] = v;
    }
    if (sanitize) {
      const bool any = __any(bad ? 1 : 0);
      if (lane_id() == 0) {
        row_flag[h] = any ? 1 : 0;
        if (any) *any_flag = 1;
      }
    }
  }
}

// C[hub_rows[i]][:] += T[i][:]. No other writer touches these rows meanwhile
// (the sparse part runs before or after on the same stream).
__global__ __launch_bounds__(kThreads) void scatter_add_kernel(const float* __restrict__ T,
                                                                const int* __restrict__ hub_rows,
                                                                int rows, int N,
                                                                float* __restrict__ C) {
  const int q = N / 4;
  const size_t total = size_t(rows) * size_t(q);
  for (size_t e = size_t(blockIdx.x) * kThreads + threadIdx.x; e < total;
       e += size_t(gridDim.x) * kThreads) {
    const size_t i = e / size_t(q), j = e % size_t(q);
    float4* c = reinterpret_cast<float4*>(C + size_t(hub_rows[i]) * size_t(N)) + j;
    const float4 t = reinterpret_cast<const float4*>(T + i * size_t(N))[j];
    float4 v = *c;
    v.x += t.x;
    v.y += t.y;
    v.z += t.z;
    v.w += t.w;
    *c = v;
  }
}

// For every stored block entry (hub row i, hot column h) whose B row holds a
// non-finite element: C[row][j] += value * B[c][j] for those elements (the
// sanitised product left them out; repeated entries enter as their sum).
// Exits at once when B's hot rows are all finite. One workgroup per hub row.
__global__ __launch_bounds__(kThreads) void fixup_kernel(ps_hub_block hb, const float* __restrict__ B,
                                                          int N, float* __restrict__ C,
                                                          const int* __restrict__ row_flag,
                                                          const int* __restrict__ any_flag) {
  if (*any_flag == 0) return;
  const size_t words = (size_t(hb.cols) + 31) / 32;
  for (int i = blockIdx.x; i < hb.rows; i += gridDim.x) {
    const int r = hb.hub_rows[i];
    for (int h = threadIdx.x; h < hb.cols; h += kThreads) {
      if (!row_flag[h] || !((hb.stored[size_t(i) * words + h / 32] >> (h % 32)) & 1u)) continue;
      const float a = hb.dense[size_t(i) * size_t(hb.cols) + h];
      const float* brow = B + size_t(hb.hot_cols[h]) * size_t(N);
      for (int j = 0; j < N; ++j) {
        const float v = brow[j];
        if (!isfinite(v)) atomicAdd(C + size_t(r) * size_t(N) + j, a * v);
      }
    }
  }
}

// A listed tile: (workset << kTileBits) | tile index within the workset.
constexpr int kTileBits = 27;
constexpr uint32_t kTileMask = (1u << kTileBits) - 1u;
constexpr int kSampleChunkMax = 256;  // XCD runs of the sample kernel (workgroups)

struct SampleArgs {
  ps_workset ws[PS_MAX_WORKSETS];  // indexed by workset
  int workset_count;
  float* out[PS_MAX_WORKSETS];
  const int* out_pos[PS_MAX_WORKSETS];
  float* out_csr;
  const uint32_t* tiles;
  uint32_t count;
  uint32_t chunk_log2;
};

// Whether a listed tile names a tile of a block workset (groups of 64 or more
// nonzeros): other codes are skipped.
__device__ __forceinline__ bool tile_valid(const SampleArgs& a, uint32_t code) {
  const uint32_t q = code >> kTileBits;
  if (q == 0 || q >= uint32_t(a.workset_count)) return false;
  const ps_workset& w = a.ws[q];
  return w.group_size >= 64 && (w.group_size & 63) == 0 &&
         uint64_t(code & kTileMask) < uint64_t(w.group_num) * uint64_t(w.group_size / 64);
}

// out[s][p] (or out_csr[out_pos[s][p]]) = sp_data[p] * D[doff[e]] for the 64
// nonzeros p of every listed tile t (entry e = 64 t + lane); one wave per
// kSampleTiles consecutive tiles. The tile codes and the D offsets are
// independent loads, the values and the D elements the second and last level
// of the wave's dependent loads (the offsets replace a chain column id ->
// hot rank and group row -> hub index). The list is sorted by hub row and
// first column, and consecutive workgroups go to one XCD in runs, so each L2
// reads a stretch of one D row.
constexpr int kSampleTiles = 4;
__global__ __launch_bounds__(kThreads) void sample_kernel(SampleArgs a, const float* __restrict__ D,
                                                           const uint32_t* __restrict__ doff,
                                                           uint32_t d_elems) {
  const uint32_t blk = balanced_block(blockIdx.x, gridDim.x, a.chunk_log2);
  const uint32_t t0 = (blk * uint32_t(kThreads / kWave) + threadIdx.x / kWave) * kSampleTiles;
  if (t0 >= a.count) return;
  uint32_t code[kSampleTiles], off[kSampleTiles];
#pragma unroll
  for (int k = 0; k < kSampleTiles; ++k) {
    const bool on = t0 + k < a.count;
    code[k] = on ? a.tiles[t0 + k] : 0u;
    off[k] = on ? doff[size_t(t0 + k) * 64 + size_t(lane_id())] : d_elems;
  }
  float v[kSampleTiles];
  size_t p[kSampleTiles];
#pragma unroll
  for (int k = 0; k < kSampleTiles; ++k) {
    p[k] = size_t(code[k] & kTileMask) * 64 + size_t(lane_id());
    const bool on = off[k] < d_elems;  // past the list, or not inside the block
    v[k] = on ? a.ws[code[k] >> kTileBits].sp_data[p[k]] * D[off[k]] : 0.f;
  }
#pragma unroll
  for (int k = 0; k < kSampleTiles; ++k) {
    if (off[k] >= d_elems) continue;
    const int q = int(code[k] >> kTileBits);
    if (a.out_csr) a.out_csr[a.out_pos[q][p[k]]] = v[k];
    else a.out[q][p[k]] = v[k];
  }
}

// doff[64 t + j] = hub_index[row] * cols + hot_rank[col_ind[p]] for the j-th
// nonzero p of listed tile t (its group's row), or d_elems when that entry
// lies outside the block or the code names no tile.
__global__ __launch_bounds__(kThreads) void tile_offsets_kernel(ps_hub_block hb, SampleArgs a,
                                                                 uint32_t* __restrict__ doff,
                                                                 uint32_t d_elems) {
  const size_t n = size_t(a.count) * 64;
  for (size_t e = size_t(blockIdx.x) * kThreads + threadIdx.x; e < n;
       e += size_t(gridDim.x) * kThreads) {
    const uint32_t code = a.tiles[e / 64];
    if (!tile_valid(a, code)) {
      doff[e] = d_elems;
      continue;
    }
    const ps_workset& w = a.ws[code >> kTileBits];
    const size_t p = size_t(code & kTileMask) * 64 + e % 64;
    const int i = hb.hub_index[w.group_des[p / size_t(w.group_size)]];
    const int h = hb.hot_rank[w.col_ind[p]];
    doff[e] = i >= 0 && h >= 0 ? uint32_t(i) * uint32_t(hb.cols) + uint32_t(h) : d_elems;
  }
}

// keys[t] = (hub index of the tile's row << 32) | its first column (all ones
// for a code that names no tile: it sorts last); vals[t] = code.
__global__ __launch_bounds__(kThreads) void tile_keys_kernel(ps_hub_block hb, SampleArgs a,
                                                              uint64_t* __restrict__ keys,
                                                              uint32_t* __restrict__ vals) {
  for (uint32_t t = blockIdx.x * kThreads + threadIdx.x; t < a.count; t += gridDim.x * kThreads) {
    const uint32_t code = a.tiles[t];
    vals[t] = code;
    if (!tile_valid(a, code)) {
      keys[t] = ~0ull;
      continue;
    }
    const ps_workset& w = a.ws[code >> kTileBits];
    const size_t p = size_t(code & kTileMask) * 64;
    const int i = hb.hub_index[w.group_des[int(p / size_t(w.group_size))]];
    keys[t] = (uint64_t(uint32_t(i)) << 32) | uint32_t(w.col_ind[p]);
  }
}

unsigned grid_for(size_t items, size_t per_block) {
  const size_t b = (items + per_block - 1) / per_block;
  return unsigned(b < 1 ? 1 : (b > 65535 ? 65535 : b));
}

int check_block(const ps_hub_block* hb) {
  PS_CHECK_ARG(hb, "hub block: null descriptor");
  PS_CHECK_ARG(hb->rows > 0 && hb->cols > 0 && hb->matrix_rows > 0 && hb->matrix_cols > 0,
               "hub block: empty block");
  PS_CHECK_ARG(hb->hub_rows && hb->hub_index && hb->hot_cols && hb->hot_rank,
               "hub block: missing arrays");
  return PS_OK;
}

}  // namespace
}  // namespace ps

extern "C" {

int ps_hub_histogram(const int* row_ptr, int rows, const int* col_ind, const int* col_nnz,
                     unsigned long long* hist, ps_stream_t stream) {
  PS_CHECK_ARG(row_ptr && col_ind && col_nnz && hist && rows > 0, "ps_hub_histogram: bad arguments");
  hipStream_t st = ps::to_hip(stream);
  PS_HIP(hipMemsetAsync(hist, 0, sizeof(unsigned long long) * 32 * 32, st));
  ps::hist_kernel<<<ps::grid_for(size_t(rows), ps::kThreads / ps::kWave), ps::kThreads, 0, st>>>(
      row_ptr, rows, col_ind, col_nnz, hist);
  PS_LAUNCHED();
  return PS_OK;
}

size_t ps_hub_stored_words(const ps_hub_block* hb) {
  return hb ? size_t(hb->rows) * ((size_t(hb->cols) + 31) / 32) : 0;
}

int ps_hub_dense_build(const ps_hub_block* hb, const int* row_ptr, const int* col_ind,
                       const float* sp_data, float* dense, uint32_t* stored, ps_stream_t stream) {
  const int rc = ps::check_block(hb);
  if (rc != PS_OK) return rc;
  PS_CHECK_ARG(row_ptr && col_ind && sp_data && dense && stored, "ps_hub_dense_build: null argument");
  hipStream_t st = ps::to_hip(stream);
  PS_HIP(hipMemsetAsync(dense, 0, sizeof(float) * size_t(hb->rows) * size_t(hb->cols), st));
  PS_HIP(hipMemsetAsync(stored, 0, sizeof(uint32_t) * ps_hub_stored_words(hb), st));
  ps::dense_kernel<<<ps::grid_for(size_t(hb->rows), 1), ps::kThreads, 0, st>>>(
      *hb, row_ptr, col_ind, sp_data, dense, stored);
  PS_LAUNCHED();
  return PS_OK;
}

int ps_hub_kept_counts(const ps_hub_block* hb, const int* row_ptr, const int* col_ind,
                       uint32_t* counts, ps_stream_t stream) {
  const int rc = ps::check_block(hb);
  if (rc != PS_OK) return rc;
  PS_CHECK_ARG(row_ptr && col_ind && counts, "ps_hub_kept_counts: null argument");
  hipStream_t st = ps::to_hip(stream);
  ps::kept_kernel<<<ps::grid_for(size_t(hb->matrix_rows), ps::kThreads / ps::kWave), ps::kThreads,
                    0, st>>>(*hb, row_ptr, col_ind, counts);
  PS_LAUNCHED();
  return PS_OK;
}

int ps_hub_compact(const ps_hub_block* hb, const int* row_ptr, const int* col_ind,
                   const float* sp_data, const uint32_t* new_row_ptr, int* new_col, float* new_val,
                   ps_stream_t stream) {
  const int rc = ps::check_block(hb);
  if (rc != PS_OK) return rc;
  PS_CHECK_ARG(row_ptr && col_ind && sp_data && new_row_ptr && new_col && new_val,
               "ps_hub_compact: null argument");
  hipStream_t st = ps::to_hip(stream);
  ps::compact_kernel<<<ps::grid_for(size_t(hb->matrix_rows), ps::kThreads / ps::kWave),
                       ps::kThreads, 0, st>>>(*hb, row_ptr, col_ind, sp_data, new_row_ptr, new_col,
                                              new_val);
  PS_LAUNCHED();
  return PS_OK;
}

int ps_hub_mark_atomic(const ps_hub_block* hb, const int* group_des, int group_num,
                       uint8_t* residue_atomic, ps_stream_t stream) {
  const int rc = ps::check_block(hb);
  if (rc != PS_OK) return rc;
  if (group_num <= 0) return PS_OK;
  PS_CHECK_ARG(group_des && residue_atomic, "ps_hub_mark_atomic: null argument");
  hipStream_t st = ps::to_hip(stream);
  ps::mark_atomic_kernel<<<ps::grid_for(size_t(group_num), ps::kThreads), ps::kThreads, 0, st>>>(
      hb->hub_index, group_des, group_num, residue_atomic);
  PS_LAUNCHED();
  return PS_OK;
}

int ps_hub_tile_flags(const ps_hub_block* hb, const ps_workset* workset, uint8_t* flags,
                      ps_stream_t stream) {
  const int rc = ps::check_block(hb);
  if (rc != PS_OK) return rc;
  PS_CHECK_ARG(workset && flags, "ps_hub_tile_flags: bad arguments");
  PS_CHECK_ARG(workset->group_size >= 64 && (workset->group_size & (workset->group_size - 1)) == 0,
               "ps_hub_tile_flags: block groups of at least 64 nonzeros only");
  if (workset->group_num <= 0) return PS_OK;
  PS_CHECK_ARG(workset->col_ind && workset->group_des, "ps_hub_tile_flags: missing workset arrays");
  hipStream_t st = ps::to_hip(stream);
  const size_t tiles = size_t(workset->group_num) * size_t(workset->group_size / 64);
  ps::tile_flags_kernel<<<ps::grid_for(tiles, ps::kThreads / ps::kWave), ps::kThreads, 0, st>>>(
      *hb, *workset, flags);
  PS_LAUNCHED();
  return PS_OK;
}

size_t ps_hub_workspace_bytes(const ps_hub_block* hb, int op, int N) {
  if (!hb || N <= 0) return 0;
  const size_t R = size_t(hb->rows), H = size_t(hb->cols), n = size_t(N);
  if (op == PS_OP_SPMM)  // B's hot rows, the product, row flags, the any-flag, GEMM
    return ps::round256(H * n * 4) + ps::round256(R * n * 4) + ps::round256(H * 4) + 256 +
           ps::kBlasWorkspace;
  // X's hub rows, Y's hot rows, D, GEMM
  return ps::round256(R * n * 4) + ps::round256(H * n * 4) + ps::round256(R * H * 4) +
         ps::kBlasWorkspace;
}

int ps_hub_spmm_launch(const ps_hub_block* hb, int N, const float* B, float* C, void* workspace,
                       size_t workspace_bytes, ps_stream_t stream) {
  const int rc = ps::check_block(hb);
  if (rc != PS_OK) return rc;
  PS_CHECK_ARG(hb->dense && hb->stored, "ps_hub_spmm_launch: missing dense block");
  PS_CHECK_ARG(N > 0 && N % 32 == 0, "SpMM requires N to be a positive multiple of 32");
  PS_CHECK_ARG(B && C && ps::aligned16(B) && ps::aligned16(C),
               "ps_hub_spmm_launch: dense buffers must be 16-byte aligned");
  PS_CHECK_ARG(workspace && workspace_bytes >= ps_hub_workspace_bytes(hb, PS_OP_SPMM, N),
               "ps_hub_spmm_launch: workspace too small");
  const size_t R = size_t(hb->rows), H = size_t(hb->cols), n = size_t(N);
  char* w = static_cast<char*>(workspace);
  float* Bh = reinterpret_cast<float*>(w);
  float* T = reinterpret_cast<float*>(w + ps::round256(H * n * 4));
  int* row_flag = reinterpret_cast<int*>(w + ps::round256(H * n * 4) + ps::round256(R * n * 4));
  int* any_flag = reinterpret_cast<int*>(reinterpret_cast<char*>(row_flag) + ps::round256(H * 4));
  void* blas_ws = reinterpret_cast<char*>(any_flag) + 256;
  hipStream_t st = ps::to_hip(stream);
  ps::clear_flag_kernel<<<1, 1, 0, st>>>(any_flag);
  PS_LAUNCHED();
  ps::gather_rows_kernel<<<ps::grid_for(H, ps::kThreads / ps::kWave), ps::kThreads, 0, st>>>(
      B, hb->hot_cols, hb->cols, N, Bh, 1, row_flag, any_flag);
  PS_LAUNCHED();
  // row-major T (R x N) = dense (R x H) * Bh (H x N): column-major
  // T' (N x R) = Bh' (N x H) * dense' (H x R)
  int r = ps::gemm_f32(st, false, false, N, hb->rows, hb->cols, Bh, N, hb->dense, hb->cols, T, N,
                       blas_ws, ps::kBlasWorkspace);
  if (r != PS_OK) return r;
  ps::scatter_add_kernel<<<ps::grid_for(R * n / 4, ps::kThreads), ps::kThreads, 0, st>>>(
      T, hb->hub_rows, hb->rows, N, C);
  PS_LAUNCHED();
  ps::fixup_kernel<<<ps::grid_for(R, 1), ps::kThreads, 0, st>>>(*hb, B, N, C, row_flag, any_flag);
  PS_LAUNCHED();
  return PS_OK;
}

// SampleArgs over the worksets and a tile list, checked.
static int sample_args(int workset_count, const ps_workset* worksets, const uint32_t* tiles,
                       uint32_t tile_count, ps::SampleArgs* a) {
  PS_CHECK_ARG(workset_count >= 1 && workset_count <= PS_MAX_WORKSETS && worksets,
               "hub block: invalid worksets");
  PS_CHECK_ARG(tile_count == 0 || tiles, "hub block: missing tile list");
  *a = ps::SampleArgs{};
  for (int s = 0; s < workset_count; ++s) a->ws[s] = worksets[s];
  a->workset_count = workset_count;
  a->tiles = tiles;
  a->count = tile_count;
  return PS_OK;
}

int ps_hub_sort_tiles(const ps_hub_block* hb, int workset_count, const ps_workset* worksets,
                      uint32_t* tiles, uint32_t tile_count, ps_stream_t stream) {
  int rc = ps::check_block(hb);
  if (rc != PS_OK) return rc;
  ps::SampleArgs a;
  rc = sample_args(workset_count, worksets, tiles, tile_count, &a);
  if (rc != PS_OK) return rc;
  if (tile_count == 0) return PS_OK;
  const size_t n = tile_count;
  const size_t bytes = 2 * ps::round256(n * 8) + ps::round256(n * 4) +
                       ps::round256(ps_radix_workspace_bytes(n));
  char* base = nullptr;
  PS_HIP(hipMalloc(&base, bytes));
  uint64_t* keys = reinterpret_cast<uint64_t*>(base);
  uint64_t* keys_alt = reinterpret_cast<uint64_t*>(base + ps::round256(n * 8));
  uint32_t* vals = reinterpret_cast<uint32_t*>(base + 2 * ps::round256(n * 8));
  void* ws = base + 2 * ps::round256(n * 8) + ps::round256(n * 4);
  hipStream_t st = ps::to_hip(stream);
  ps::tile_keys_kernel<<<ps::grid_for(n, ps::kThreads), ps::kThreads, 0, st>>>(*hb, a, keys, vals);
  hipError_t e = hipGetLastError();
  int alt = 0, r = PS_OK;
  if (e == hipSuccess)
    r = ps_radix_sort_pairs_u64(keys, keys_alt, vals, tiles, n, 0, 64, ws, &alt, stream);
  if (e == hipSuccess && r == PS_OK && !alt)
    e = hipMemcpyAsync(tiles, vals, n * 4, hipMemcpyDeviceToDevice, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  (void)hipFree(base);
  if (r != PS_OK) return r;
  PS_HIP(e);
  return PS_OK;
}

int ps_hub_tile_offsets(const ps_hub_block* hb, int workset_count, const ps_workset* worksets,
                        const uint32_t* tiles, uint32_t tile_count, uint32_t* doff,
                        ps_stream_t stream) {
  int rc = ps::check_block(hb);
  if (rc != PS_OK) return rc;
  PS_CHECK_ARG(size_t(hb->rows) * size_t(hb->cols) < (size_t(1) << 32),
               "hub block: more dense elements than 32-bit offsets address");
  ps::SampleArgs a;
  rc = sample_args(workset_count, worksets, tiles, tile_count, &a);
  if (rc != PS_OK) return rc;
  if (tile_count == 0) return PS_OK;
  PS_CHECK_ARG(doff, "ps_hub_tile_offsets: null output");
  hipStream_t st = ps::to_hip(stream);
  ps::tile_offsets_kernel<<<ps::grid_for(size_t(tile_count) * 64, ps::kThreads), ps::kThreads, 0,
                            st>>>(*hb, a, doff, uint32_t(hb->rows) * uint32_t(hb->cols));
  PS_LAUNCHED();
  return PS_OK;
}

int ps_hub_sddmm_launch(const ps_hub_block* hb, int workset_count, const ps_workset* worksets,
                        const uint32_t* tiles, const uint32_t* doff, uint32_t tile_count, int N,
                        const float* lhs, const float* rhs, float* const* out,
                        const int* const* out_pos, float* out_csr, void* workspace,
                        size_t workspace_bytes, ps_stream_t stream) {
  int rc = ps::check_block(hb);
  if (rc != PS_OK) return rc;
  PS_CHECK_ARG(size_t(hb->rows) * size_t(hb->cols) < (size_t(1) << 32),
               "hub block: more dense elements than 32-bit offsets address");
  PS_CHECK_ARG(tile_count == 0 || doff, "ps_hub_sddmm_launch: missing tile offsets");
  PS_CHECK_ARG(N > 0 && N % 32 == 0 && N <= 512,
               "SDDMM requires N to be a multiple of 32 between 32 and 512");
  PS_CHECK_ARG(lhs && rhs && ps::aligned16(lhs) && ps::aligned16(rhs),
               "ps_hub_sddmm_launch: dense buffers must be 16-byte aligned");
  PS_CHECK_ARG(out_csr ? (out_pos != nullptr) : (out != nullptr),
               "ps_hub_sddmm_launch: missing outputs");
  PS_CHECK_ARG(workspace && workspace_bytes >= ps_hub_workspace_bytes(hb, PS_OP_SDDMM, N),
               "ps_hub_sddmm_launch: workspace too small");
  ps::SampleArgs a;
  rc = sample_args(workset_count, worksets, tiles, tile_count, &a);
  if (rc != PS_OK) return rc;
  if (tile_count == 0) return PS_OK;
  for (int s = 1; s < workset_count; ++s) {
    a.out[s] = out ? out[s] : nullptr;
    a.out_pos[s] = out_pos ? out_pos[s] : nullptr;
    PS_CHECK_ARG(worksets[s].group_num <= 0 || worksets[s].group_size < 64 ||
                     (out_csr ? a.out_pos[s] != nullptr : a.out[s] != nullptr),
                 "ps_hub_sddmm_launch: missing outputs of a block workset");
  }
  a.out_csr = out_csr;
  const size_t R = size_t(hb->rows), H = size_t(hb->cols), k = size_t(N);
  char* w = static_cast<char*>(workspace);
  float* Xh = reinterpret_cast<float*>(w);
  float* Yh = reinterpret_cast<float*>(w + ps::round256(R * k * 4));
  float* D = reinterpret_cast<float*>(w + ps::round256(R * k * 4) + ps::round256(H * k * 4));
  void* blas_ws = reinterpret_cast<char*>(D) + ps::round256(R * H * 4);
  hipStream_t st = ps::to_hip(stream);
  ps::gather_rows_kernel<<<ps::grid_for(R, ps::kThreads / ps::kWave), ps::kThreads, 0, st>>>(
      lhs, hb->hub_rows, hb->rows, N, Xh, 0, nullptr, nullptr);
  PS_LAUNCHED();
  ps::gather_rows_kernel<<<ps::grid_for(H, ps::kThreads / ps::kWave), ps::kThreads, 0, st>>>(
      rhs, hb->hot_cols, hb->cols, N, Yh, 0, nullptr, nullptr);
  PS_LAUNCHED();
  // row-major D (R x H) = Xh (R x K) * Yh^T: column-major D' (H x R) = Yh'^T (H x K) * Xh' (K x R)
  int r = ps::gemm_f32(st, true, false, hb->cols, hb->rows, N, Yh, N, Xh, N, D, hb->cols, blas_ws,
                       ps::kBlasWorkspace);
  if (r != PS_OK) return r;
  const uint64_t per_block = uint64_t(ps::kThreads / ps::kWave) * ps::kSampleTiles;
  const uint64_t grid = (uint64_t(tile_count) + per_block - 1) / per_block;
  PS_CHECK_ARG(grid < (1ull << 31), "ps_hub_sddmm_launch: too many tiles");
  a.chunk_log2 = uint32_t(ps::task_chunk_log2(PS_TASK_CHUNK_AUTO, grid, ps::kSampleChunkMax));
  ps::sample_kernel<<<unsigned(grid), ps::kThreads, 0, st>>>(a, D, doff,
                                                              uint32_t(hb->rows) * uint32_t(hb->cols));
  PS_LAUNCHED();
  return PS_OK;
}

}  // extern "C"
