// Dense hub block: the rows of highest degree restricted to the most popular
// columns, run as dense FP32 products on the matrix cores (v_mfma_f32_32x32x2f32).
//
// On power-law graphs the heaviest rows hold a dense core with the most
// popular columns (C3: rows of degree >= 16384 x columns with >= 512 nonzeros
// hold 27% of the nonzeros at 38% density). The sparse kernels pay one row
// gather per nonzero there; a dense product over the block does the same
// arithmetic from MFMA tiles with each B / Y row read once per tile.
//
//   SpMM:  C[hub_rows[i], :] += sum_h dense[i][h] * B[hot_cols[h], :]
//          (dense holds the block's stored values, zeros elsewhere). A
//          pre-pass copies B's hot rows transposed (feature-major, so that
//          both MFMA operands run along the hot columns) with non-finite
//          elements replaced by 0; the MFMA kernel splits the hot columns
//          into chunks, and each workgroup adds its partial rows into C with
//          float atomics (whole 128-byte row stretches per instruction). A
//          fix-up adds a * b for every stored block entry whose b is not
//          finite, so Inf and NaN reach exactly the rows that store that
//          column, as in the reference's per-nonzero products.
//   SDDMM: the listed tiles (64 consecutive nonzeros of a block group lying
//          in the block) are planned at build time as per-entry records
//          grouped by the dense tile (64 hub rows x 256 hot columns) they
//          fall in. The MFMA kernel computes each dense tile of
//          D = X[hub_rows] * Y[hot_cols]^T in registers, stages it in LDS and
//          writes sp_data[p] * D[i][h] to every planned output of the tile:
//          D never reaches memory.
//
// MFMA operand layout: for v_mfma_f32_32x32x2f32, lane l supplies A[l % 32][k]
// and B[k][l % 32] for k = l / 32; the 32 x 32 result leaves D[8 j + 4 (l / 32)
// + i][l % 32] in register 4 j + i of lane l. A k-range of 8 is covered by 4
// MFMAs in which lane l supplies k = 4 (l / 32) + step: every lane then loads
// 4 consecutive k of one A row and one B row with a single 128-bit load (both
// operands are stored with k contiguous), and A and B agree on every k.
//
// Repeated entries: a (hub row, hot column) slot stored more than once stays
// on the sparse SpMM path for all its entries (dense slot 0, no stored bit),
// so SpMM still adds a1 * b + a2 * b as the reference's per-nonzero products
// do, and the block is the same for every build. SDDMM plans each entry on
// its own and needs no such rule.
// No reference counterpart: the reference runs every nonzero through its
// sparse kernels (spmm_kernel_block.cu, sddmm_kernel_block.cu).
#include "ps_common.hpp"

namespace ps {
namespace {

constexpr int kThreads = 256;
typedef float v16f __attribute__((ext_vector_type(16)));

inline size_t round256(size_t b) { return (b + 255) & ~size_t(255); }
// Dense rows are padded with zeros to a multiple of 16 hot columns, so the
// MFMA kernels' K loops run in steps of 16 without bounds checks.
__host__ __device__ inline size_t dense_ld(int cols) {
  return (size_t(cols) + 15) & ~size_t(15);
}
// Bit pattern a repeated slot carries in `dense` between the mark and clear
// passes of the build (a NaN; the matrix's values are finite).
constexpr uint32_t kRepeated = 0xFFFFFFFFu;

// SpMM: rows per workgroup (4 waves of 64) and features per feature slice
// (the workspace's transposed copy holds one slice at a time).
constexpr int kSpRows = 256;
constexpr int kSpSlice = 128;
// SDDMM: dense tile of a workgroup (4 waves, each 64 rows x 64 columns), and
// the padded LDS row (a row 4 apart starts 32 banks over: the two half-waves
// of an MFMA result register write disjoint banks).
constexpr int kSdRows = 64;
constexpr int kSdCols = 256;
constexpr int kSdLd = kSdCols + 8;
constexpr int kSdCoordBits = 14;  // 6 row bits + 8 column bits of an entry's tile coordinate
constexpr int kPosBits = 32;
constexpr int kWsBits = 5;        // PS_MAX_WORKSETS = 32
static_assert(PS_MAX_WORKSETS <= (1 << kWsBits), "workset index field too narrow");
static_assert(kPosBits + kWsBits + kSdCoordBits <= 64, "plan entry fields exceed 64 bits");

__device__ __forceinline__ float4 load4(const float* p) { return *reinterpret_cast<const float4*>(p); }

__device__ __forceinline__ float pick(const float4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// acc[rb][cb] += A[rb] * B[cb] over the 8 k of one step (4 MFMAs each).
template <int RB, int CB>
__device__ __forceinline__ void mfma_step(v16f (&acc)[RB][CB], const float4 (&A)[RB],
                                          const float4 (&B)[CB]) {
#pragma unroll
  for (int st = 0; st < 4; ++st)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int cb = 0; cb < CB; ++cb)
        acc[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x2f32(pick(A[rb], st), pick(B[cb], st),
                                                           acc[rb][cb], 0, 0, 0);
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

// Pass 1 of the dense build: the stored bit of every block entry's slot; an
// entry finding its bit already set marks the slot repeated in `dense`. One
// workgroup per hub row.
__global__ __launch_bounds__(kThreads) void dense_mark_kernel(ps_hub_block hb,
                                                               const int* __restrict__ row_ptr,
                                                               const int* __restrict__ col_ind,
                                                               float* __restrict__ dense,
                                                               uint32_t* __restrict__ stored) {
  const size_t words = (size_t(hb.cols) + 31) / 32, ld = dense_ld(hb.cols);
  for (int i = blockIdx.x; i < hb.rows; i += gridDim.x) {
    const int r = hb.hub_rows[i];
    uint32_t* srow = stored + size_t(i) * words;
    uint32_t* drow = reinterpret_cast<uint32_t*>(dense + size_t(i) * ld);
    for (int p = row_ptr[r] + threadIdx.x; p < row_ptr[r + 1]; p += kThreads) {
      const int h = hb.hot_rank[col_ind[p]];
      if (h < 0) continue;
      const uint32_t bit = 1u << (h % 32);
      if (atomicOr(srow + h / 32, bit) & bit) drow[h] = kRepeated;
    }
  }
}

// Pass 2: dense[i][h] = value for every slot stored once (the only writer).
__global__ __launch_bounds__(kThreads) void dense_fill_kernel(ps_hub_block hb,
                                                               const int* __restrict__ row_ptr,
                                                               const int* __restrict__ col_ind,
                                                               const float* __restrict__ sp_data,
                                                               float* __restrict__ dense) {
  const size_t ld = dense_ld(hb.cols);
  for (int i = blockIdx.x; i < hb.rows; i += gridDim.x) {
    const int r = hb.hub_rows[i];
    float* drow = dense + size_t(i) * ld;
    for (int p = row_ptr[r] + threadIdx.x; p < row_ptr[r + 1]; p += kThreads) {
      const int h = hb.hot_rank[col_ind[p]];
      if (h >= 0 && __float_as_uint(drow[h]) != kRepeated) drow[h] = sp_data[p];
    }
  }
}

// Pass 3: repeated slots back to 0 and out of the block (stored bit cleared).
__global__ __launch_bounds__(kThreads) void dense_clear_kernel(ps_hub_block hb,
                                                                const int* __restrict__ row_ptr,
                                                                const int* __restrict__ col_ind,
                                                                float* __restrict__ dense,
                                                                uint32_t* __restrict__ stored) {
  const size_t words = (size_t(hb.cols) + 31) / 32, ld = dense_ld(hb.cols);
  for (int i = blockIdx.x; i < hb.rows; i += gridDim.x) {
    const int r = hb.hub_rows[i];
    uint32_t* srow = stored + size_t(i) * words;
    float* drow = dense + size_t(i) * ld;
    for (int p = row_ptr[r] + threadIdx.x; p < row_ptr[r + 1]; p += kThreads) {
      const int h = hb.hot_rank[col_ind[p]];
      if (h < 0 || __float_as_uint(drow[h]) != kRepeated) continue;
      drow[h] = 0.f;  // every entry of the slot writes the same
      atomicAnd(srow + h / 32, ~(1u << (h % 32)));
    }
  }
}

// Whether entry (hub row i, hot column h) is in the SpMM block: its slot is
// stored once.
__device__ __forceinline__ bool in_block(const ps_hub_block& hb, int i, int h) {
  if (i < 0 || h < 0) return false;
  const size_t words = (size_t(hb.cols) + 31) / 32;
  return (hb.stored[size_t(i) * words + h / 32] >> (h % 32)) & 1u;
}

// counts[r] = stored entries of row r outside the SpMM block. One wave per row.
__global__ __launch_bounds__(kThreads) void kept_kernel(ps_hub_block hb,
                                                         const int* __restrict__ row_ptr,
                                                         const int* __restrict__ col_ind,
                                                         uint32_t* __restrict__ counts) {
  const int waves = kThreads / kWave;
  for (int r = blockIdx.x * waves + threadIdx.x / kWave; r < hb.matrix_rows;
       r += gridDim.x * waves) {
    const int b = row_ptr[r], e = row_ptr[r + 1];
    uint32_t n = uint32_t(e - b);
    const int i = hb.hub_index[r];
    if (i >= 0) {
      uint32_t inside = 0;
      for (int p = b + lane_id(); p < e; p += kWave) inside += in_block(hb, i, hb.hot_rank[col_ind[p]]);
      for (int o = 32; o > 0; o >>= 1) inside += __shfl_xor(inside, o);
      n -= inside;
    }
    if (lane_id() == 0) counts[r] = n;
  }
}

// The CSR without the SpMM block's entries, in the original order within rows.
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
    const int i = hb.hub_index[r];
    uint32_t out = new_row_ptr[r];
    for (int p0 = b; p0 < e; p0 += kWave) {
      const int p = p0 + lane_id();
      const int c = p < e ? col_ind[p] : 0;
      const bool keep = p < e && !(i >= 0 && in_block(hb, i, hb.hot_rank[c]));
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

// ------------------------------------------------------------- SpMM

__global__ void clear_flag_kernel(int* flag) { *flag = 0; }

// Bt[n][h] = B[hot_cols[h]][f0 + n] for the features [f0, f0 + width) (Bt
// rows of ld floats; zero for h >= H), non-finite elements replaced by 0;
// row_flag[h] |= whether the row held a non-finite element there, *any_flag
// set to 1 if any did. A workgroup moves 64 hot columns x 64 features at a
// time through LDS (reads along B rows, writes along Bt rows).
__global__ __launch_bounds__(kThreads) void transpose_hot_kernel(
    const float* __restrict__ B, const int* __restrict__ hot_cols, int H, int N, int ld, int f0,
    int width, float* __restrict__ Bt, int* __restrict__ row_flag, int* __restrict__ any_flag) {
  __shared__ float t[64][65];
  __shared__ int bad[64];
  const int h0 = blockIdx.x * 64;
  if (threadIdx.x < 64) bad[threadIdx.x] = 0;
  for (int n0 = 0; n0 < width; n0 += 64) {
    const int wn = width - n0 < 64 ? width - n0 : 64;
    __syncthreads();
    for (int e = threadIdx.x; e < 64 * 64; e += kThreads) {
      const int hh = e / 64, nn = e % 64;
      float v = 0.f;
      if (h0 + hh < H && nn < wn) {
        v = B[size_t(hot_cols[h0 + hh]) * size_t(N) + size_t(f0 + n0 + nn)];
        if (!isfinite(v)) {
          v = 0.f;
          bad[hh] = 1;
        }
      }
      t[hh][nn] = v;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < 64 * 64; e += kThreads) {
      const int nn = e / 64, hh = e % 64;
      if (nn < wn && h0 + hh < ld) Bt[size_t(n0 + nn) * size_t(ld) + size_t(h0 + hh)] = t[hh][nn];
    }
  }
  __syncthreads();
  if (threadIdx.x < 64 && h0 + int(threadIdx.x) < H) {
    const int b = bad[threadIdx.x];
    if (f0 == 0) row_flag[h0 + threadIdx.x] = b;
    else if (b) row_flag[h0 + threadIdx.x] = 1;
    if (b) *any_flag = 1;
  }
}

struct HubSpmmArgs {
  const float* dense;
  const float* Bt;  // kSpSlice (or fewer) feature rows of ld floats
  float* C;
  const int* hub_rows;
  int R, N, ld;
  int f0;        // first feature of this slice
  int kc;        // hot columns per chunk (multiple of 16)
  int panels;    // row panels of kSpRows rows
  uint32_t chunk_log2;
};

// One workgroup: kSpRows hub rows (64 per wave: 2 MFMA row blocks) x the
// slice's 32 CB features, over one chunk of hot columns; the partial rows are
// added into C with atomics. A (dense) streams from memory once; B (Bt) is
// the same for the 4 waves of a workgroup and for every row panel of a chunk
// (neighbouring workgroups take the chunk's panels on one XCD). ST stages of
// operand loads stay in flight.
template <int CB, int ST>
__global__ __launch_bounds__(kThreads, 2) void hub_spmm_kernel(HubSpmmArgs a) {
  const uint32_t blk = balanced_block(blockIdx.x, gridDim.x, a.chunk_log2);
  const int panel = int(blk % uint32_t(a.panels)), chunk = int(blk / uint32_t(a.panels));
  const int lane = lane_id(), g = lane >> 5, l32 = lane & 31;
  const int m0 = panel * kSpRows + (threadIdx.x / kWave) * 64;
  const int k0 = chunk * a.kc;
  const int k1 = k0 + a.kc < a.ld ? k0 + a.kc : a.ld;
  if (m0 >= a.R || k0 >= k1) return;
  // rows past R load row R - 1; their results are never written
  const float* arow[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int m = m0 + rb * 32 + l32;
    arow[rb] = a.dense + size_t(m < a.R ? m : a.R - 1) * size_t(a.ld) + 4 * g;
  }
  const float* brow[CB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) brow[cb] = a.Bt + size_t(cb * 32 + l32) * size_t(a.ld) + 4 * g;

  v16f acc[2][CB];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = v16f{};
  float4 A[ST][2], Bf[ST][CB];
#pragma unroll
  for (int s = 0; s < ST; ++s)
    if (k0 + 8 * s < k1) {
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) A[s][rb] = load4(arow[rb] + k0 + 8 * s);
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) Bf[s][cb] = load4(brow[cb] + k0 + 8 * s);
    }
  for (int h = k0; h < k1; h += 8 * ST) {
#pragma unroll
    for (int s = 0; s < ST; ++s) {
      if (h + 8 * s < k1) {
        mfma_step<2, CB>(acc, A[s], Bf[s]);
        const int nh = h + 8 * (s + ST);
        if (nh < k1) {
#pragma unroll
          for (int rb = 0; rb < 2; ++rb) A[s][rb] = load4(arow[rb] + nh);
#pragma unroll
          for (int cb = 0; cb < CB; ++cb) Bf[s][cb] = load4(brow[cb] + nh);
        }
      }
    }
  }
  // C[hub_rows[m]][f0 + 32 cb + l32] += acc: register r of a block holds row
  // 8 (r / 4) + 4 g + r % 4, so each atomic instruction adds two 32-float
  // row stretches.
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int mb = m0 + rb * 32;
    const int hr = a.hub_rows[mb + l32 < a.R ? mb + l32 : a.R - 1];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int lr = 8 * (r / 4) + 4 * g + (r % 4);
      const int dst = __shfl(hr, lr);
      if (mb + lr < a.R) {
        float* crow = a.C + size_t(dst) * size_t(a.N) + size_t(a.f0 + l32);
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) unsafeAtomicAdd(crow + cb * 32, acc[rb][cb][r]);
      }
    }
  }
}

// For every stored block entry (hub row i, hot column h) whose B row holds a
// non-finite element: C[row][j] += value * B[c][j] for those elements (the
// sanitised product left them out). Exits at once when B's hot rows are all
// finite. One workgroup per hub row.
__global__ __launch_bounds__(kThreads) void fixup_kernel(ps_hub_block hb, const float* __restrict__ B,
                                                          int N, float* __restrict__ C,
                                                          const int* __restrict__ row_flag,
                                                          const int* __restrict__ any_flag) {
  if (*any_flag == 0) return;
  const size_t words = (size_t(hb.cols) + 31) / 32, ld = dense_ld(hb.cols);
  for (int i = blockIdx.x; i < hb.rows; i += gridDim.x) {
    const int r = hb.hub_rows[i];
    for (int h = threadIdx.x; h < hb.cols; h += kThreads) {
      if (!row_flag[h] || !((hb.stored[size_t(i) * words + h / 32] >> (h % 32)) & 1u)) continue;
      const float a = hb.dense[size_t(i) * ld + h];
      const float* brow = B + size_t(hb.hot_cols[h]) * size_t(N);
      for (int j = 0; j < N; ++j) {
        const float v = brow[j];
        if (!isfinite(v)) atomicAdd(C + size_t(r) * size_t(N) + j, a * v);
      }
    }
  }
}

// ------------------------------------------------------------- SDDMM

// A listed tile: (workset << kTileBits) | tile index within the workset.
constexpr int kTileBits = 27;
constexpr uint32_t kTileMask = (1u << kTileBits) - 1u;

struct Worksets {
  ps_workset ws[PS_MAX_WORKSETS];
  int count;
};

// Whether a listed tile names a tile of a block workset (groups of 64 or more
// nonzeros): other codes are skipped.
__device__ __forceinline__ bool tile_valid(const Worksets& a, uint32_t code) {
  const uint32_t q = code >> kTileBits;
  if (q == 0 || q >= uint32_t(a.count)) return false;
  const ps_workset& w = a.ws[q];
  return w.group_size >= 64 && (w.group_size & 63) == 0 &&
         uint64_t(code & kTileMask) < uint64_t(w.group_num) * uint64_t(w.group_size / 64);
}

// Entry e = 64 t + j of the (code-sorted) list: keys[e] = its dense tile
// (kSdRows hub rows x kSdCols hot columns, row-panel major), or `T` (one past
// the last tile) when the code names no tile or the entry lies outside the
// block; coords[e] = its row and column inside the tile; vals[e] = e.
__global__ __launch_bounds__(kThreads) void plan_keys_kernel(ps_hub_block hb, Worksets a,
                                                              const uint32_t* __restrict__ codes,
                                                              uint32_t count, uint32_t tiles_c,
                                                              uint32_t T, uint32_t* __restrict__ keys,
                                                              uint32_t* __restrict__ vals,
                                                              uint16_t* __restrict__ coords) {
  const size_t n = size_t(count) * 64;
  for (size_t e = size_t(blockIdx.x) * kThreads + threadIdx.x; e < n;
       e += size_t(gridDim.x) * kThreads) {
    vals[e] = uint32_t(e);
    const uint32_t code = codes[e / 64];
    uint32_t key = T;
    if (tile_valid(a, code)) {
      const ps_workset& w = a.ws[code >> kTileBits];
      const size_t p = size_t(code & kTileMask) * 64 + e % 64;
      const int i = hb.hub_index[w.group_des[p / size_t(w.group_size)]];
      const int h = hb.hot_rank[w.col_ind[p]];
      if (i >= 0 && h >= 0) {
        key = uint32_t(i / kSdRows) * tiles_c + uint32_t(h / kSdCols);
        coords[e] = uint16_t(((i % kSdRows) << 8) | (h % kSdCols));
      }
    }
    keys[e] = key;
  }
}

// After the stable sort by tile: tile_begin[t] = first entry of tile t (T + 1
// values; tile_begin[T] = the planned entries), entries[e] = position | workset
// << 32 | tile coordinate << 37, values[e] = the entry's sp_data.
__global__ __launch_bounds__(kThreads) void plan_fill_kernel(Worksets a,
                                                              const uint32_t* __restrict__ codes,
                                                              uint32_t n, uint32_t T,
                                                              const uint32_t* __restrict__ keys,
                                                              const uint32_t* __restrict__ src,
                                                              const uint16_t* __restrict__ coords,
                                                              uint32_t* __restrict__ tile_begin,
                                                              uint64_t* __restrict__ entries,
                                                              float* __restrict__ values) {
  for (uint32_t e = blockIdx.x * kThreads + threadIdx.x; e < n; e += gridDim.x * kThreads) {
    const uint32_t k = keys[e];
    const uint32_t prev = e > 0 ? keys[e - 1] + 1u : 0u;
    for (uint32_t t = prev; t <= k; ++t) tile_begin[t] = e;
    if (e == n - 1)
      for (uint32_t t = k + 1; t <= T; ++t) tile_begin[t] = n;
    if (k >= T) continue;
    const uint32_t e0 = src[e];
    const uint32_t code = codes[e0 / 64];
    const uint32_t s = code >> kTileBits;
    const uint64_t p = uint64_t(code & kTileMask) * 64 + e0 % 64;
    entries[e] = p | (uint64_t(s) << kPosBits) | (uint64_t(coords[e0]) << (kPosBits + kWsBits));
    values[e] = a.ws[s].sp_data[p];
  }
}

struct HubSddmmArgs {
  const float* X;
  const float* Y;
  int K;
  const int* hub_rows;
  const int* hot_cols;
  int R, H;
  const uint32_t* tile_begin;
  const uint64_t* entries;
  const float* values;
  int tiles_r, tiles_c;
  int range;  // column tiles per workgroup
  uint32_t chunk_log2;
  int S;
  float* out[PS_MAX_WORKSETS];
  const int* out_pos[PS_MAX_WORKSETS];
  float* out_csr;
};

__device__ __forceinline__ float* out_of(const HubSddmmArgs& a, int s) {
  float* p = a.out[0];
#pragma unroll
  for (int q = 1; q < PS_MAX_WORKSETS; ++q) {
    if (q >= a.S) break;
    if (s == q) p = a.out[q];
  }
  return p;
}
__device__ __forceinline__ const int* pos_of(const HubSddmmArgs& a, int s) {
  const int* p = a.out_pos[0];
#pragma unroll
  for (int q = 1; q < PS_MAX_WORKSETS; ++q) {
    if (q >= a.S) break;
    if (s == q) p = a.out_pos[q];
  }
  return p;
}

// One workgroup: the dense tiles of one row panel (kSdRows hub rows) over a
// range of column tiles. Wave w computes rows 0..63 x columns 64 w .. 64 w + 63
// of each tile (2 x 2 MFMA blocks) over the K features, passes of 8 KB8; with
// kResident (one pass) its X fragments stay in registers across the column
// tiles, and Y fragments stream one step ahead. The tile then goes through LDS
// and the workgroup writes out[s][p] = value * D[r][c] for the tile's planned
// entries (sorted by output position, so the stores run along the outputs).
// Rows past R and columns past H compute on clamped rows; no entry names them.
template <int KB8, bool kResident>
__global__ __launch_bounds__(kThreads, 2) void hub_sddmm_kernel(HubSddmmArgs a) {
  __shared__ float dt[kSdRows * kSdLd];
  const uint32_t blk = balanced_block(blockIdx.x, gridDim.x, a.chunk_log2);
  const int rp = int(blk % uint32_t(a.tiles_r)), cr = int(blk / uint32_t(a.tiles_r));
  const int cq0 = cr * a.range;
  const int cq1 = cq0 + a.range < a.tiles_c ? cq0 + a.range : a.tiles_c;
  if (cq0 >= cq1) return;  // uniform over the workgroup
  const int wave = threadIdx.x / kWave, lane = lane_id(), g = lane >> 5, l32 = lane & 31;
  const int passes = kResident ? 1 : a.K / (8 * KB8);

  const float* xrow[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int m = rp * kSdRows + rb * 32 + l32;
    xrow[rb] = a.X + size_t(a.hub_rows[m < a.R ? m : a.R - 1]) * size_t(a.K) + 4 * g;
  }
  float4 xa[KB8][2];
  if (kResident) {
#pragma unroll
    for (int kb = 0; kb < KB8; ++kb)
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) xa[kb][rb] = load4(xrow[rb] + 8 * kb);
  }

  for (int cq = cq0; cq < cq1; ++cq) {
    const float* yrow[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int c = cq * kSdCols + wave * 64 + cb * 32 + l32;
      yrow[cb] = a.Y + size_t(a.hot_cols[c < a.H ? c : a.H - 1]) * size_t(a.K) + 4 * g;
    }
    v16f acc[2][2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) acc[rb][cb] = v16f{};
    for (int ps = 0; ps < passes; ++ps) {
      const int f = ps * 8 * KB8;
      if (!kResident) {
#pragma unroll
        for (int kb = 0; kb < KB8; ++kb)
#pragma unroll
          for (int rb = 0; rb < 2; ++rb) xa[kb][rb] = load4(xrow[rb] + f + 8 * kb);
      }
      float4 yb[2][2];
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) yb[0][cb] = load4(yrow[cb] + f);
#pragma unroll
      for (int kb = 0; kb < KB8; ++kb) {
        if (kb + 1 < KB8) {
#pragma unroll
          for (int cb = 0; cb < 2; ++cb) yb[(kb + 1) & 1][cb] = load4(yrow[cb] + f + 8 * (kb + 1));
        }
        mfma_step<2, 2>(acc, xa[kb], yb[kb & 1]);
      }
    }
    __syncthreads();  // the previous tile's entries are done with dt
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          dt[(rb * 32 + 8 * (r / 4) + 4 * g + (r % 4)) * kSdLd + wave * 64 + cb * 32 + l32] =
              acc[rb][cb][r];
    __syncthreads();
    const int t = rp * a.tiles_c + cq;
    const uint32_t e1 = a.tile_begin[t + 1];
    for (uint32_t e = a.tile_begin[t] + threadIdx.x; e < e1; e += kThreads) {
      const uint64_t code = a.entries[e];
      const float v = a.values[e];
      const uint32_t local = uint32_t(code >> (kPosBits + kWsBits));
      const float d = dt[(local >> 8) * kSdLd + (local & 255u)];
      const uint32_t p = uint32_t(code);
      const int s = int((code >> kPosBits) & ((1u << kWsBits) - 1u));
      if (a.out_csr) a.out_csr[pos_of(a, s)[p]] = v * d;
      else out_of(a, s)[p] = v * d;
    }
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

int worksets_of(int workset_count, const ps_workset* worksets, Worksets* a) {
  PS_CHECK_ARG(workset_count >= 1 && workset_count <= PS_MAX_WORKSETS && worksets,
               "hub block: invalid worksets");
  *a = Worksets{};
  for (int s = 0; s < workset_count; ++s) a->ws[s] = worksets[s];
  a->count = workset_count;
  return PS_OK;
}

uint32_t sddmm_tiles_r(const ps_hub_block* hb) { return uint32_t((hb->rows + kSdRows - 1) / kSdRows); }
uint32_t sddmm_tiles_c(const ps_hub_block* hb) { return uint32_t((hb->cols + kSdCols - 1) / kSdCols); }

// Hot columns per SpMM chunk: about 1024 workgroups per feature slice (4 per
// CU), at least 256 columns per chunk, a multiple of 16.
int spmm_chunk(int rows, int ld) {
  const int panels = (rows + kSpRows - 1) / kSpRows;
  int chunks = (1024 + panels - 1) / panels;
  if (chunks > ld / 256) chunks = ld / 256;
  if (chunks < 1) chunks = 1;
  const int kc = (ld + chunks - 1) / chunks;
  return (kc + 15) & ~15;
}

template <int CB>
void spmm_launch_cb(const HubSpmmArgs& a, unsigned grid, hipStream_t st) {
  if (CB >= 2) hub_spmm_kernel<CB, 2><<<grid, kThreads, 0, st>>>(a);
  else hub_spmm_kernel<CB, 4><<<grid, kThreads, 0, st>>>(a);
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

size_t ps_hub_dense_ld(int cols) { return cols > 0 ? ps::dense_ld(cols) : 0; }

int ps_hub_dense_build(const ps_hub_block* hb, const int* row_ptr, const int* col_ind,
                       const float* sp_data, float* dense, uint32_t* stored, ps_stream_t stream) {
  const int rc = ps::check_block(hb);
  if (rc != PS_OK) return rc;
  PS_CHECK_ARG(row_ptr && col_ind && sp_data && dense && stored, "ps_hub_dense_build: null argument");
  PS_CHECK_ARG(ps::aligned16(dense), "ps_hub_dense_build: dense must be 16-byte aligned");
  hipStream_t st = ps::to_hip(stream);
  PS_HIP(hipMemsetAsync(dense, 0, sizeof(float) * size_t(hb->rows) * ps::dense_ld(hb->cols), st));
  PS_HIP(hipMemsetAsync(stored, 0, sizeof(uint32_t) * ps_hub_stored_words(hb), st));
  const unsigned grid = ps::grid_for(size_t(hb->rows), 1);
  ps::dense_mark_kernel<<<grid, ps::kThreads, 0, st>>>(*hb, row_ptr, col_ind, dense, stored);
  PS_LAUNCHED();
  ps::dense_fill_kernel<<<grid, ps::kThreads, 0, st>>>(*hb, row_ptr, col_ind, sp_data, dense);
  PS_LAUNCHED();
  ps::dense_clear_kernel<<<grid, ps::kThreads, 0, st>>>(*hb, row_ptr, col_ind, dense, stored);
  PS_LAUNCHED();
  return PS_OK;
}

int ps_hub_kept_counts(const ps_hub_block* hb, const int* row_ptr, const int* col_ind,
                       uint32_t* counts, ps_stream_t stream) {
  const int rc = ps::check_block(hb);
  if (rc != PS_OK) return rc;
  PS_CHECK_ARG(hb->stored, "ps_hub_kept_counts: missing stored bits");
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
  PS_CHECK_ARG(hb->stored, "ps_hub_compact: missing stored bits");
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
  if (!hb || N <= 0 || op != PS_OP_SPMM) return 0;
  // one feature slice of B's hot rows, transposed; row flags; the any-flag
  const size_t slice = size_t(N < ps::kSpSlice ? N : ps::kSpSlice);
  return ps::round256(slice * ps::dense_ld(hb->cols) * 4) + ps::round256(size_t(hb->cols) * 4) + 256;
}

int ps_hub_spmm_launch(const ps_hub_block* hb, int N, const float* B, float* C, void* workspace,
                       size_t workspace_bytes, ps_stream_t stream) {
  const int rc = ps::check_block(hb);
  if (rc != PS_OK) return rc;
  PS_CHECK_ARG(hb->dense && hb->stored, "ps_hub_spmm_launch: missing dense block");
  PS_CHECK_ARG(N > 0 && N % 32 == 0, "SpMM requires N to be a positive multiple of 32");
  PS_CHECK_ARG(B && C && ps::aligned16(B) && ps::aligned16(C) && ps::aligned16(hb->dense),
               "ps_hub_spmm_launch: dense buffers must be 16-byte aligned");
  PS_CHECK_ARG(workspace && workspace_bytes >= ps_hub_workspace_bytes(hb, PS_OP_SPMM, N),
               "ps_hub_spmm_launch: workspace too small");
  PS_CHECK_ARG(int64_t(hb->matrix_rows) * N <= INT32_MAX && int64_t(hb->matrix_cols) * N <= INT32_MAX,
               "Dense dimensions exceed the 32-bit kernel indexing range");
  const int ld = int(ps::dense_ld(hb->cols));
  const size_t slice = size_t(N < ps::kSpSlice ? N : ps::kSpSlice);
  char* w = static_cast<char*>(workspace);
  float* Bt = reinterpret_cast<float*>(w);
  int* row_flag = reinterpret_cast<int*>(w + ps::round256(slice * size_t(ld) * 4));
  int* any_flag = reinterpret_cast<int*>(reinterpret_cast<char*>(row_flag) +
                                         ps::round256(size_t(hb->cols) * 4));
  hipStream_t st = ps::to_hip(stream);
  ps::clear_flag_kernel<<<1, 1, 0, st>>>(any_flag);
  PS_LAUNCHED();
  ps::HubSpmmArgs a{};
  a.dense = hb->dense;
  a.Bt = Bt;
  a.C = C;
  a.hub_rows = hb->hub_rows;
  a.R = hb->rows;
  a.N = N;
  a.ld = ld;
  a.kc = ps::spmm_chunk(hb->rows, ld);
  a.panels = (hb->rows + ps::kSpRows - 1) / ps::kSpRows;
  const int chunks = (ld + a.kc - 1) / a.kc;
  const uint64_t grid = uint64_t(a.panels) * uint64_t(chunks);
  PS_CHECK_ARG(grid < (1ull << 31), "ps_hub_spmm_launch: block too large");
  // runs of the chunk's row panels on one XCD (up to 64 workgroups)
  a.chunk_log2 = uint32_t(ps::task_chunk_log2(PS_TASK_CHUNK_AUTO, grid, 64));
  for (int f0 = 0; f0 < N; f0 += ps::kSpSlice) {
    const int width = N - f0 < ps::kSpSlice ? N - f0 : ps::kSpSlice;
    ps::transpose_hot_kernel<<<unsigned((ld + 63) / 64), ps::kThreads, 0, st>>>(
        B, hb->hot_cols, hb->cols, N, ld, f0, width, Bt, row_flag, any_flag);
    PS_LAUNCHED();
    a.f0 = f0;
    switch (width / 32) {
      case 1: ps::spmm_launch_cb<1>(a, unsigned(grid), st); break;
      case 2: ps::spmm_launch_cb<2>(a, unsigned(grid), st); break;
      case 3: ps::spmm_launch_cb<3>(a, unsigned(grid), st); break;
      default: ps::spmm_launch_cb<4>(a, unsigned(grid), st); break;
    }
    PS_LAUNCHED();
  }
  ps::fixup_kernel<<<ps::grid_for(size_t(hb->rows), 1), ps::kThreads, 0, st>>>(*hb, B, N, C,
                                                                                row_flag, any_flag);
  PS_LAUNCHED();
  return PS_OK;
}

size_t ps_hub_sddmm_plan_bytes(const ps_hub_block* hb, uint32_t tile_count) {
  if (!hb || hb->rows <= 0 || hb->cols <= 0) return 0;
  const size_t T = size_t(ps::sddmm_tiles_r(hb)) * ps::sddmm_tiles_c(hb);
  const size_t n = size_t(tile_count) * 64;
  return ps::round256((T + 1) * 4) + ps::round256(n * 8) + ps::round256(n * 4);
}

int ps_hub_sddmm_plan(const ps_hub_block* hb, int workset_count, const ps_workset* worksets,
                      const uint32_t* tiles, uint32_t tile_count, void* plan, size_t plan_bytes,
                      ps_stream_t stream) {
  int rc = ps::check_block(hb);
  if (rc != PS_OK) return rc;
  ps::Worksets a;
  rc = ps::worksets_of(workset_count, worksets, &a);
  if (rc != PS_OK) return rc;
  PS_CHECK_ARG(tile_count == 0 || tiles, "hub block: missing tile list");
  PS_CHECK_ARG(plan && plan_bytes >= ps_hub_sddmm_plan_bytes(hb, tile_count),
               "ps_hub_sddmm_plan: plan buffer too small");
  PS_CHECK_ARG(uint64_t(tile_count) * 64 < (1ull << 32), "ps_hub_sddmm_plan: too many tiles");
  const uint32_t tiles_c = ps::sddmm_tiles_c(hb);
  const uint64_t T64 = uint64_t(ps::sddmm_tiles_r(hb)) * tiles_c;
  PS_CHECK_ARG(T64 < (1ull << 31), "ps_hub_sddmm_plan: too many dense tiles");
  const uint32_t T = uint32_t(T64);
  const uint32_t n = tile_count * 64;
  char* pb = static_cast<char*>(plan);
  uint32_t* tile_begin = reinterpret_cast<uint32_t*>(pb);
  uint64_t* entries = reinterpret_cast<uint64_t*>(pb + ps::round256((size_t(T) + 1) * 4));
  float* values = reinterpret_cast<float*>(reinterpret_cast<char*>(entries) +
                                           ps::round256(size_t(n) * 8));
  hipStream_t st = ps::to_hip(stream);
  if (n == 0) {
    PS_HIP(hipMemsetAsync(tile_begin, 0, (size_t(T) + 1) * 4, st));
    PS_HIP(hipStreamSynchronize(st));
    return PS_OK;
  }
  // temporaries: the code list twice, keys / sources twice, coordinates, radix workspace
  const size_t rw = ps_radix_workspace_bytes(n);
  const size_t bytes = 2 * ps::round256(size_t(tile_count) * 4) + 4 * ps::round256(size_t(n) * 4) +
                       ps::round256(size_t(n) * 2) + ps::round256(rw);
  char* base = nullptr;
  PS_HIP(hipMalloc(&base, bytes));
  char* q = base;
  auto take = [&q](size_t b) {
    char* r = q;
    q += ps::round256(b);
    return r;
  };
  uint32_t* codes = reinterpret_cast<uint32_t*>(take(size_t(tile_count) * 4));
  uint32_t* codes_alt = reinterpret_cast<uint32_t*>(take(size_t(tile_count) * 4));
  uint32_t* keys = reinterpret_cast<uint32_t*>(take(size_t(n) * 4));
  uint32_t* keys_alt = reinterpret_cast<uint32_t*>(take(size_t(n) * 4));
  uint32_t* vals = reinterpret_cast<uint32_t*>(take(size_t(n) * 4));
  uint32_t* vals_alt = reinterpret_cast<uint32_t*>(take(size_t(n) * 4));
  uint16_t* coords = reinterpret_cast<uint16_t*>(take(size_t(n) * 2));
  void* radix_ws = take(rw);
  int r = PS_OK, alt = 0;
  hipError_t e = hipMemcpyAsync(codes, tiles, size_t(tile_count) * 4, hipMemcpyDeviceToDevice, st);
  // codes ascending: the entries come out in (workset, position) order, which
  // the stable sort by tile keeps inside every tile
  if (e == hipSuccess)
    r = ps_radix_sort_pairs_u32(codes, codes_alt, nullptr, nullptr, tile_count, 0, 32, radix_ws,
                                &alt, stream);
  const uint32_t* sorted_codes = alt ? codes_alt : codes;
  if (e == hipSuccess && r == PS_OK) {
    ps::plan_keys_kernel<<<ps::grid_for(size_t(n), ps::kThreads), ps::kThreads, 0, st>>>(
        *hb, a, sorted_codes, tile_count, tiles_c, T, keys, vals, coords);
    e = hipGetLastError();
  }
  int kbits = 1;
  while ((uint64_t(1) << kbits) <= uint64_t(T)) ++kbits;
  int alt2 = 0;
  if (e == hipSuccess && r == PS_OK)
    r = ps_radix_sort_pairs_u32(keys, keys_alt, vals, vals_alt, n, 0, kbits, radix_ws, &alt2,
                                stream);
  if (e == hipSuccess && r == PS_OK) {
    ps::plan_fill_kernel<<<ps::grid_for(size_t(n), ps::kThreads), ps::kThreads, 0, st>>>(
        a, sorted_codes, n, T, alt2 ? keys_alt : keys, alt2 ? vals_alt : vals, coords, tile_begin,
        entries, values);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  (void)hipFree(base);
  if (r != PS_OK) return r;
  PS_HIP(e);
  return PS_OK;
}

int ps_hub_sddmm_launch(const ps_hub_block* hb, int workset_count, const ps_workset* worksets,
                        const void* plan, uint32_t tile_count, int N, const float* lhs,
                        const float* rhs, float* const* out, const int* const* out_pos,
                        float* out_csr, ps_stream_t stream) {
  int rc = ps::check_block(hb);
  if (rc != PS_OK) return rc;
  PS_CHECK_ARG(workset_count >= 1 && workset_count <= PS_MAX_WORKSETS && worksets,
               "hub block: invalid worksets");
  PS_CHECK_ARG(tile_count == 0 || plan, "ps_hub_sddmm_launch: missing plan");
  PS_CHECK_ARG(N > 0 && N % 32 == 0 && N <= 512,
               "SDDMM requires N to be a multiple of 32 between 32 and 512");
  PS_CHECK_ARG(lhs && rhs && ps::aligned16(lhs) && ps::aligned16(rhs),
               "ps_hub_sddmm_launch: dense buffers must be 16-byte aligned");
  PS_CHECK_ARG(out_csr ? (out_pos != nullptr) : (out != nullptr),
               "ps_hub_sddmm_launch: missing outputs");
  PS_CHECK_ARG(int64_t(hb->matrix_rows) * N <= INT32_MAX && int64_t(hb->matrix_cols) * N <= INT32_MAX,
               "Dense dimensions exceed the 32-bit kernel indexing range");
  if (tile_count == 0) return PS_OK;
  ps::HubSddmmArgs a{};
  for (int s = 1; s < workset_count; ++s) {
    a.out[s] = out ? out[s] : nullptr;
    a.out_pos[s] = out_pos ? out_pos[s] : nullptr;
    PS_CHECK_ARG(worksets[s].group_num <= 0 || worksets[s].group_size < 64 ||
                     (out_csr ? a.out_pos[s] != nullptr : a.out[s] != nullptr),
                 "ps_hub_sddmm_launch: missing outputs of a block workset");
  }
  a.S = workset_count;
  a.out_csr = out_csr;
  a.X = lhs;
  a.Y = rhs;
  a.K = N;
  a.hub_rows = hb->hub_rows;
  a.hot_cols = hb->hot_cols;
  a.R = hb->rows;
  a.H = hb->cols;
  a.tiles_r = int(ps::sddmm_tiles_r(hb));
  a.tiles_c = int(ps::sddmm_tiles_c(hb));
  const size_t T = size_t(a.tiles_r) * size_t(a.tiles_c);
  const char* pb = static_cast<const char*>(plan);
  a.tile_begin = reinterpret_cast<const uint32_t*>(pb);
  a.entries = reinterpret_cast<const uint64_t*>(pb + ps::round256((T + 1) * 4));
  a.values = reinterpret_cast<const float*>(reinterpret_cast<const char*>(a.entries) +
                                            ps::round256(size_t(tile_count) * 64 * 8));
  // about 1024 workgroups (4 per CU): column ranges per row panel
  int ranges = (1024 + a.tiles_r - 1) / a.tiles_r;
  if (ranges > a.tiles_c) ranges = a.tiles_c;
  a.range = (a.tiles_c + ranges - 1) / ranges;
  ranges = (a.tiles_c + a.range - 1) / a.range;
  const uint64_t grid = uint64_t(a.tiles_r) * uint64_t(ranges);
  PS_CHECK_ARG(grid < (1ull << 31), "ps_hub_sddmm_launch: block too large");
  // runs of one column range's row panels on one XCD share its Y rows in L2
  a.chunk_log2 = uint32_t(ps::task_chunk_log2(PS_TASK_CHUNK_AUTO, grid, 32));
  hipStream_t st = ps::to_hip(stream);
  switch (N) {
    case 32: ps::hub_sddmm_kernel<4, true><<<unsigned(grid), ps::kThreads, 0, st>>>(a); break;
    case 64: ps::hub_sddmm_kernel<8, true><<<unsigned(grid), ps::kThreads, 0, st>>>(a); break;
    case 96: ps::hub_sddmm_kernel<12, true><<<unsigned(grid), ps::kThreads, 0, st>>>(a); break;
    case 128: ps::hub_sddmm_kernel<16, true><<<unsigned(grid), ps::kThreads, 0, st>>>(a); break;
    default: ps::hub_sddmm_kernel<4, false><<<unsigned(grid), ps::kThreads, 0, st>>>(a); break;
  }
  PS_LAUNCHED();
  return PS_OK;
}

}  // extern "C"
