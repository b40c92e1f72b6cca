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
//          (dense holds the block's stored values, zeros elsewhere, in
//          fragment order). A pre-pass gathers B's hot rows into the B
//          operand's fragment order (one feature slice of up to 128 at a
//          time) with non-finite elements replaced by 0; the MFMA kernel
//          splits the row panels' hot columns evenly over its workgroups
//          (up to 64 features each), sums each 32- or 64-column iteration
//          apart before adding it to running sums, and adds those into C
//          with float atomics (whole 128-byte row stretches per instruction). A fix-up adds a * b for every stored
//          block entry whose b is not finite, so Inf and NaN reach exactly
//          the rows that store that column, as in the reference's
//          per-nonzero products.
//   SDDMM: the listed tiles (64 consecutive nonzeros of a block group lying
//          in the block) are planned at build time as per-entry records
//          grouped by the dense tile (64 hub rows x 128 hot columns) they
//          fall in. Pre-passes gather X[hub_rows] and Y[hot_cols] into
//          fragment order; the MFMA kernel computes each dense tile of
//          D = X[hub_rows] * Y[hot_cols]^T in registers, stages it in LDS and
//          writes sp_data[p] * D[i][h] to every planned output of the tile
//          while it computes the next tile: D never reaches memory.
//
// MFMA operand layout: for v_mfma_f32_32x32x2f32, lane l supplies A[l % 32][k]
// and B[k][l % 32] for k = l / 32; the 32 x 32 result leaves D[8 j + 4 (l / 32)
// + i][l % 32] in register 4 j + i of lane l. A k-range of 8 is covered by 4
// MFMAs in which lane l supplies k = 4 (l / 32) + step: every lane then loads
// 4 consecutive k of its A row and B column with a single 128-bit load, and
// A and B agree on every k. Operands are stored in that order (fragment
// order, frag_offset below), so a wave's operand load is one contiguous 1 KB
// read.
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
// Dense rows are padded with zeros to a multiple of kDenseAlign hot columns,
// so the SpMM kernel's K loop runs in whole rings of 8-column steps without
// bounds checks.
constexpr int kDenseAlign = 64;
__host__ __device__ inline size_t dense_ld(int cols) {
  return (size_t(cols) + kDenseAlign - 1) & ~size_t(kDenseAlign - 1);
}
// MFMA fragment order. The kernels' operands are stored so that one 8-column
// step of a 32-row block is 256 consecutive floats, in the order the 64 lanes
// load them (lane l: row l % 32, columns 4 (l / 32) .. + 3 of the step), so
// every operand load is one contiguous 1 KB read. Element (i, h) of a matrix
// with rows padded to kFragRows and ld columns (a multiple of 8):
constexpr int kFragRows = 64;
__host__ __device__ inline size_t frag_offset(size_t i, size_t h, size_t ld) {
  return ((i / 32) * (ld / 8) + h / 8) * 256 + ((h % 8) / 4) * 128 + (i % 32) * 4 + h % 4;
}
__host__ __device__ inline size_t frag_rows(int rows) {
  return (size_t(rows) + kFragRows - 1) & ~size_t(kFragRows - 1);
}
// Bit pattern a repeated slot carries in `dense` between the mark and clear
// passes of the build (a NaN; the matrix's values are finite).
constexpr uint32_t kRepeated = 0xFFFFFFFFu;

// SpMM: rows per workgroup (4 waves of 64) and features per feature slice
// (the workspace's transposed copy holds one slice at a time).
constexpr int kSpRows = 256;
constexpr int kSpSlice = 128;
// SDDMM: dense tile of a workgroup (4 waves, each 64 rows x 32 columns), and
// the padded LDS row (a row 4 apart starts 32 banks over: the two half-waves
// of an MFMA result register write disjoint banks).
constexpr int kSdRows = 64;
constexpr int kSdCols = 128;
constexpr int kSdLd = kSdCols + 8;
// an entry's place in the LDS copy of its dense tile: row * kSdLd + column
constexpr int kSdCoordBits = 15;
static_assert(kSdRows * kSdLd <= (1 << kSdCoordBits), "tile coordinate field too narrow");
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
  uint32_t* d = reinterpret_cast<uint32_t*>(dense);
  for (int i = blockIdx.x; i < hb.rows; i += gridDim.x) {
    const int r = hb.hub_rows[i];
    uint32_t* srow = stored + size_t(i) * words;
    for (int p = row_ptr[r] + threadIdx.x; p < row_ptr[r + 1]; p += kThreads) {
      const int h = hb.hot_rank[col_ind[p]];
      if (h < 0) continue;
      const uint32_t bit = 1u << (h % 32);
      if (atomicOr(srow + h / 32, bit) & bit) d[frag_offset(i, h, ld)] = kRepeated;
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
    for (int p = row_ptr[r] + threadIdx.x; p < row_ptr[r + 1]; p += kThreads) {
      const int h = hb.hot_rank[col_ind[p]];
      if (h < 0) continue;
      float* slot = dense + frag_offset(i, h, ld);
      if (__float_as_uint(*slot) != kRepeated) *slot = sp_data[p];
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
    for (int p = row_ptr[r] + threadIdx.x; p < row_ptr[r + 1]; p += kThreads) {
      const int h = hb.hot_rank[col_ind[p]];
      if (h < 0) continue;
      float* slot = dense + frag_offset(i, h, ld);
      if (__float_as_uint(*slot) != kRepeated) continue;
      *slot = 0.f;  // every entry of the slot writes the same
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

// Bt = the slice's B operand in fragment order: element (n, h) = B[hot_cols[h]][f0
// + n] for the features n < width (a multiple of 32) and hot columns h < ld
// (0 for h >= H), non-finite elements replaced by 0; row_flag[h] |= whether
// B's row hot_cols[h] held a non-finite element there, *any_flag set to 1 if
// any did. An item is one float4 of a 256-float run: lane l of run
// (32-feature block nb, step ks) holds features nb * 32 + l % 32 at hot
// columns 8 ks + 4 (l / 32) + c; each of its 4 reads is a 128-byte stretch of
// a B row shared by 32 lanes. A thread takes 4 items a grid stride apart and
// issues all their index and row loads before any store (C3 SpMM N=128
// 5.662 -> 5.646 ms per call, N=32 1.577 -> 1.573 ms, against one item per
// thread).
__global__ __launch_bounds__(kThreads) void gather_hot_kernel(
    const float* __restrict__ B, const int* __restrict__ hot_cols, int H, int N, int ld, int f0,
    int width, float* __restrict__ Bt, int* __restrict__ row_flag, int* __restrict__ any_flag) {
  constexpr int kItems = 4;  // float4 runs per thread per pass, all loads in flight together
  const size_t runs = size_t(width / 32) * size_t(ld / 8);
  const size_t total = runs * 64;
  const size_t stride = size_t(gridDim.x) * kThreads;
  for (size_t q0 = size_t(blockIdx.x) * kThreads + threadIdx.x; q0 < total;
       q0 += kItems * stride) {
    int h[kItems][4];
    int col[kItems][4];
    int n[kItems];
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
      const size_t q = q0 + size_t(i) * stride;
      const size_t run = q < total ? q / 64 : 0;
      const int l = int(q % 64);
      const int nb = int(run / size_t(ld / 8)), ks = int(run % size_t(ld / 8));
      n[i] = nb * 32 + l % 32;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        h[i][c] = ks * 8 + 4 * (l / 32) + c;
        col[i][c] = q < total && h[i][c] < H ? hot_cols[h[i][c]] : -1;
      }
    }
    float v[kItems][4];
#pragma unroll
    for (int i = 0; i < kItems; ++i)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        v[i][c] = col[i][c] >= 0 ? B[size_t(col[i][c]) * size_t(N) + size_t(f0 + n[i])] : 0.f;
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
      const size_t q = q0 + size_t(i) * stride;
      if (q >= total) continue;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (!isfinite(v[i][c])) {
          v[i][c] = 0.f;
          row_flag[h[i][c]] = 1;  // cleared by clear_flags_kernel before the first slice
          *any_flag = 1;
        }
      }
      *reinterpret_cast<float4*>(Bt + (q / 64) * 256 + size_t(q % 64) * 4) =
          make_float4(v[i][0], v[i][1], v[i][2], v[i][3]);
    }
  }
}

// row_flag[h] = 0 for h < H, *any_flag = 0.
__global__ __launch_bounds__(kThreads) void clear_flags_kernel(int* __restrict__ row_flag, int H,
                                                                int* __restrict__ any_flag) {
  for (int h = blockIdx.x * kThreads + threadIdx.x; h < H; h += gridDim.x * kThreads) row_flag[h] = 0;
  if (blockIdx.x == 0 && threadIdx.x == 0) *any_flag = 0;
}

struct HubSpmmArgs {
  const float* dense;
  const float* Bt;  // the slice's B operand in fragment order (ld columns)
  float* C;
  const int* hub_rows;
  int R, N, ld;
  int f0;        // first feature of this slice
  int panels;    // row panels of kSpRows rows
  int fgroups;   // feature groups of 32 CB features in the slice
};

// One feature group (32 CB of the slice's features) of the hub rows per
// workgroup, each group's work split evenly over its workgroups (the grid is
// one workgroup per slot the CUs hold at once): the row panels' hot columns
// in loop iterations of 8 U columns, panel-major, each workgroup an equal run
// of them, taken as segments of at most one panel each. A segment: kSpRows
// hub rows (64 per wave: 2 MFMA row blocks) over its hot columns. Each loop
// iteration's products are summed in fresh accumulators and then added to
// running sums, so an output's FP32 sum is a chain of 4 U MFMA accumulations
// per iteration plus one addition per iteration (not one chain over the whole
// segment); the running sums are added into C with atomics. The feature
// groups' workgroups for one share run one after another on one XCD, so A
// comes from its L2 for all but the first. A (dense) streams from memory
// through a per-wave ring of RA 8-column steps loaded RA - 1 steps ahead. The
// 4 waves share the group's B fragments: wave w < CB loads the group's
// 32-feature block w of every step (G steps ahead, into registers) and the
// workgroup passes them through a double-buffered LDS stage, one barrier per
// step. Loads past the
// segment's end (never used) read its last step again. Waves whose 64 rows
// lie past R compute on row block 0 and write nothing (every wave takes part
// in the barriers).
// workgroups of hub_spmm_kernel per CU (its registers admit no more)
constexpr int spmm_wg_per_cu(int) { return 2; }
template <int CB, int RA>
__global__ __launch_bounds__(kThreads, spmm_wg_per_cu(CB)) void hub_spmm_kernel(HubSpmmArgs a) {
  constexpr int G = 4;                               // B steps in flight per wave
  constexpr int U = RA > G ? RA : G;                 // steps per loop iteration
  static_assert(U % RA == 0 && U % G == 0 && U % 2 == 0, "ring sizes must divide the unroll");
  static_assert(kDenseAlign % (8 * U) == 0, "a panel's columns must hold whole iterations");
  __shared__ float4 bs[2][CB][kWave];
  const int wave = threadIdx.x / kWave, lane = lane_id(), g = lane >> 5, l32 = lane & 31;
  const size_t steps = size_t(a.ld / 8);
  // the workgroup's feature group fg and its place wi among that group's wn
  // workgroups; with the grid a multiple of kXcd * fgroups, the groups'
  // workgroups for one share run on one XCD one after another (A shared in L2)
  const uint32_t fgs = uint32_t(a.fgroups), wn = gridDim.x / fgs;
  uint32_t fg, wi;
  if (gridDim.x % (kXcd * fgs) == 0) {
    const uint32_t r = blockIdx.x / kXcd;
    fg = r % fgs;
    wi = (r / fgs) * kXcd + blockIdx.x % kXcd;
  } else {
    fg = blockIdx.x % fgs;
    wi = blockIdx.x / fgs;
  }
  const uint32_t ipp = uint32_t(a.ld / (8 * U));  // loop iterations per panel
  const uint64_t total = uint64_t(a.panels) * ipp;
  uint32_t it = uint32_t(total * wi / wn);
  const uint32_t it1 = uint32_t(total * (wi + 1) / wn);
  while (it < it1) {  // uniform over the workgroup
    const int panel = int(it / ipp);
    const uint32_t seg_end = it1 < uint32_t(panel + 1) * ipp ? it1 : uint32_t(panel + 1) * ipp;
    const int k0 = int(it - uint32_t(panel) * ipp) * 8 * U;
    const int k1 = int(seg_end - uint32_t(panel) * ipp) * 8 * U;
    it = seg_end;
    const int m0 = panel * kSpRows + wave * 64;
    const bool active = m0 < a.R;
    const float* arow[2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
      arow[rb] = a.dense + size_t((active ? m0 / 32 : 0) + rb) * steps * 256 + lane * 4;
    const bool loader = wave < CB;  // loads B block `wave` of every step
    const float* bsrc = a.Bt + size_t(fg * CB + (loader ? wave : 0)) * steps * 256 + lane * 4;
    const int klast = k1 - 8;
    auto kclamp = [klast](int k) { return k < klast ? k : klast; };

    v16f acc[2][CB], sum[2][CB];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        acc[rb][cb] = v16f{};
        sum[rb][cb] = v16f{};
      }
    float4 A[RA][2], breg[G];
    // B(0) into LDS slot 0, B(1 .. G) into the register ring (step t in slot t % G)
    if (loader) {
      bs[0][wave][lane] = load4(bsrc + size_t(k0) * 32);
#pragma unroll
      for (int j = 1; j <= G; ++j) breg[j % G] = load4(bsrc + size_t(kclamp(k0 + 8 * j)) * 32);
    }
#pragma unroll
    for (int j = 0; j < RA - 1; ++j)
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) A[j][rb] = load4(arow[rb] + size_t(kclamp(k0 + 8 * j)) * 32);
    __syncthreads();
    for (int h = k0; h < k1; h += 8 * U) {
#pragma unroll
      for (int s = 0; s < U; ++s) {
        const int k = h + 8 * s;  // this step's first hot column
        float4 bf[CB];
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) bf[cb] = bs[s % 2][cb][lane];
        if (loader) {
          bs[(s + 1) % 2][wave][lane] = breg[(s + 1) % G];  // B(t + 1), read after the barrier
          breg[(s + 1) % G] = load4(bsrc + size_t(kclamp(k + 8 * (G + 1))) * 32);
        }
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
          A[(s + RA - 1) % RA][rb] = load4(arow[rb] + size_t(kclamp(k + 8 * (RA - 1))) * 32);
        float4 as[2] = {A[s % RA][0], A[s % RA][1]};
        mfma_step<2, CB>(acc, as, bf);
        __syncthreads();
      }
      // the iteration's partial sums into the running sums
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
          sum[rb][cb] += acc[rb][cb];
          acc[rb][cb] = v16f{};
        }
    }
    // (the last step's barrier has passed: the next segment may refill bs)
    if (active) {
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        const int mb = m0 + rb * 32;
        const int hr = a.hub_rows[mb + l32 < a.R ? mb + l32 : a.R - 1];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int lr = 8 * (r / 4) + 4 * g + (r % 4);
          const int dst = __shfl(hr, lr);
          if (mb + lr < a.R) {
            float* crow = a.C + size_t(dst) * size_t(a.N) + size_t(a.f0 + fg * CB * 32 + l32);
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) unsafeAtomicAdd(crow + cb * 32, sum[rb][cb][r]);
          }
        }
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
      const float a = hb.dense[frag_offset(i, h, ld)];
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
// block; coords[e] = its place in the tile's LDS copy (row * kSdLd + column);
// vals[e] = e.
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
        coords[e] = uint16_t((i % kSdRows) * kSdLd + h % kSdCols);
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

// dst = rows idx[i] of the row-major src (K floats per row, K a multiple of
// 32) in fragment order with ld = K, for i < padded (a multiple of 32); zero
// rows for i >= count. Each thread moves one float4.
__global__ __launch_bounds__(kThreads) void gather_rows_kernel(const float* __restrict__ src,
                                                                const int* __restrict__ idx,
                                                                int count, int padded, int K,
                                                                float* __restrict__ dst) {
  const size_t steps = size_t(K / 8);
  const size_t n = size_t(padded / 32) * steps * 64;
  for (size_t q = size_t(blockIdx.x) * kThreads + threadIdx.x; q < n;
       q += size_t(gridDim.x) * kThreads) {
    const size_t run = q / 64;
    const int l = int(q % 64);
    const int i = int(run / steps) * 32 + l % 32;
    const int k = int(run % steps) * 8 + 4 * (l / 32);
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (i < count) v = load4(src + size_t(idx[i]) * size_t(K) + size_t(k));
    *reinterpret_cast<float4*>(dst + run * 256 + size_t(l) * 4) = v;
  }
}

struct HubSddmmArgs {
  const float* Xf;  // X[hub_rows], fragment order, rows padded to kSdRows
  const float* Yf;  // Y[hot_cols], fragment order, rows padded to kSdCols
  int K;
  const uint32_t* tile_begin;
  const uint64_t* entries;
  const float* values;
  int tiles_r, tiles_c;
  uint32_t chunk_log2;
  float* out[PS_MAX_WORKSETS];
  const int* out_pos[PS_MAX_WORKSETS];
  float* out_csr;
};

// Two workgroups per CU (each holds two D buffers, 68 KB of LDS), each over
// an even share of the dense tiles in row-panel-major order (a row panel is
// kSdRows hub rows, a tile that panel x kSdCols hot columns). The 4 waves sit
// side by side: wave w computes all 64 rows x columns 32 w .. + 31 (two MFMA
// blocks), over the K features in units of 8 KB8 (one unit per tile when
// kResident: the wave's X fragments then stay in registers across a row
// panel's tiles; else K / 32 units, X reloaded per unit). Operands come in
// fragment order (each load one contiguous 1 KB run); no two waves load the
// same Y. Y fragments stream through a ring of 4 steps loaded 3 steps ahead,
// across unit and tile boundaries. A finished tile's D goes to one of the two
// LDS buffers; while the matrix cores compute the next tile, the workgroup
// writes out[s][p] = value * D[r][c] for the finished tile's planned entries
// (sorted by output position), split into one chunk per 8-feature step: a
// step stores the chunk loaded kSdOutAhead steps before and loads the chunk
// kSdOutAhead steps after, so the plan reads and the output stores run under
// the MFMAs. The last tile's outputs are written after the loop. Padding rows
// and columns compute zeros; no entry names them.
// A wave's share of a tile: kSdRb 32-row x kSdNb 32-column MFMA blocks
constexpr int kSdWaveRows = 64;
constexpr int kSdRb = kSdWaveRows / 32;
constexpr int kSdNb = kSdRows * kSdCols / (4 * kSdWaveRows) / 32;
constexpr int kSdDtBytes = 2 * kSdRows * kSdLd * 4;
// workgroups per CU that the two D buffers leave room for in 160 KB of LDS
constexpr int kSdWgPerCu = (160 * 1024 - 1024) / kSdDtBytes;
static_assert(kSdWgPerCu >= 1, "D buffers exceed the LDS");
constexpr int kSdRing = 4;
constexpr int kSdBatch = 16;   // outputs per thread in flight in the final pass
constexpr int kSdOutAhead = 3;  // steps between a chunk's loads and its stores
constexpr int kSdOutSets = kSdOutAhead + 1;
// Pipelined outputs per thread per step: a tile's steps together cover a full
// tile (kSdRows * kSdCols entries); entries past that (only repeated nonzeros
// make them) are written after the last tile from direct dot products.
constexpr int sddmm_out_per(int KB8, bool resident) {
  return resident ? (kSdRows * kSdCols / kThreads + KB8 - 1) / KB8 : 4;
}
using global_float = __attribute__((address_space(1))) float;
// read-only for the kernel's lifetime: uniform reads become scalar loads (a
// vector load there would make the wave wait for every load and store ahead)
using const_u32 = const __attribute__((address_space(4))) uint32_t;
template <int KB8, bool kResident, bool kCsr>
__global__ __launch_bounds__(kThreads, kSdWgPerCu) void hub_sddmm_kernel(HubSddmmArgs a) {
  static_assert(KB8 % kSdRing == 0, "units must hold whole rings of Y steps");
  static_assert(KB8 % kSdOutSets == 0, "units must hold whole cycles of output sets");
  constexpr int OP = sddmm_out_per(KB8, kResident);
  // slot counts of the three forms of a tile's steps (a tile's outputs take
  // the smallest that holds them: a slot costs its loads whether used or not)
  constexpr int OP1 = OP / 4 > 0 ? OP / 4 : 1, OP2 = OP / 2 > 0 ? OP / 2 : 1;
  static_assert(kResident || 20 * OP * kThreads >= kSdRows * kSdCols,
                "non-resident tiles (K >= 160) must cover a full tile in their steps");
  __shared__ float dt[2][kSdRows * kSdLd];
  __shared__ float* s_out[PS_MAX_WORKSETS];
  __shared__ const int* s_pos[PS_MAX_WORKSETS];
  const uint32_t blk = balanced_block(blockIdx.x, gridDim.x, a.chunk_log2);
  const uint64_t T = uint64_t(a.tiles_r) * uint64_t(a.tiles_c);
  const uint32_t t0 = uint32_t(T * blk / gridDim.x), t1 = uint32_t(T * (blk + 1) / gridDim.x);
  if (t0 >= t1) return;  // uniform over the workgroup
  const uint32_t tc = uint32_t(a.tiles_c);
  if (threadIdx.x < PS_MAX_WORKSETS) {
    s_out[threadIdx.x] = a.out[threadIdx.x];
    s_pos[threadIdx.x] = a.out_pos[threadIdx.x];
  }
  __syncthreads();
  const int tid = threadIdx.x;
  const int wave = tid / kWave, lane = lane_id(), g = lane >> 5, l32 = lane & 31;
  constexpr int kWaveCols = kSdNb * 32;
  constexpr int kRowWaves = kSdRows / kSdWaveRows;  // waves down a tile
  const int wr = (wave % kRowWaves) * kSdWaveRows, wc = (wave / kRowWaves) * kWaveCols;
  const int units = kResident ? 1 : a.K / (8 * KB8);  // units per tile
  const int TS = units * KB8;                          // 8-feature steps per tile
  const size_t steps = size_t(a.K / 8);                // 8-feature steps per row block

  // out[s][p] (or out_csr[out_pos[s][p]]) = value * D[r][c] of one planned entry
  auto emit = [&](uint64_t code, float v, const float* d) {
    const float r = v * d[uint32_t(code >> (kPosBits + kWsBits))];
    const int s = int((code >> kPosBits) & ((1u << kWsBits) - 1u));
    if (kCsr) __builtin_nontemporal_store(r, a.out_csr + s_pos[s][uint32_t(code)]);
    else __builtin_nontemporal_store(r, s_out[s] + uint32_t(code));
  };
  // The same in the pipelined form for a lane that may lie past its chunk
  // (`live` false: its clamped entry names a place inside the tile, and it
  // stores nothing); with nothing pending (`pend` false) the loaded entry may
  // be no entry, so code 0 stands in.
  auto emit_pipe = [&](uint64_t code, float v, const float* d, bool live, bool pend) {
    if (!pend) code = 0;
    const float r = v * d[uint32_t(code >> (kPosBits + kWsBits))];
    const int s = int((code >> kPosBits) & ((1u << kWsBits) - 1u));
    if (kCsr) {
      if (live) __builtin_nontemporal_store(r, a.out_csr + s_pos[s][uint32_t(code)]);
    } else {
      // (the empty asm keeps the table read out of the branch: only the store
      // depends on `live`)
      uint64_t base = reinterpret_cast<uint64_t>(s_out[s]);
      asm volatile("" : "+v"(base));
      if (live) __builtin_nontemporal_store(r, (global_float*)base + uint32_t(code));
    }
  };

  // step 0 of the wave's X rows in tile t's row panel
  auto x_run = [&](uint32_t t) {
    return a.Xf + size_t((int(t / tc) * kSdRows + wr) / 32) * steps * 256 + lane * 4;
  };
  float4 xa[KB8][kSdRb];
  // step 0 of the wave's column block cb in tile t (the workgroup's last tile
  // stands in for the one past it)
  auto y_run = [&](uint32_t t, int cb) {
    const int q = int((t < t1 ? t : t1 - 1) % tc);
    return a.Yf + size_t((q * kSdCols + wc) / 32 + cb) * steps * 256 + lane * 4;
  };
  float4 yb[kSdRing][kSdNb];
  // prologue: steps 0 .. kSdRing - 2 of the first unit
#pragma unroll
  for (int j = 0; j < kSdRing - 1; ++j)
#pragma unroll
    for (int cb = 0; cb < kSdNb; ++cb) yb[j][cb] = load4(y_run(t0, cb) + j * 256);

  v16f acc[kSdRb][kSdNb];
#pragma unroll
  for (int rb = 0; rb < kSdRb; ++rb)
#pragma unroll
    for (int cb = 0; cb < kSdNb; ++cb) acc[rb][cb] = v16f{};
  // The finished tile whose outputs are written under the next tile's MFMAs.
  // Its entries [pe0, pe1) go out in TS chunks of clen = ceil((pe1 - pe0) /
  // TS) entries; chunk gs = [pe0 + gs clen, pe0 + (gs + 1) clen) cut at pe1.
  // Before the first tile there is none: every chunk is empty.
  // A tile's first cap entries go through the pipeline, the rest (only
  // repeated nonzeros make a tile hold more) at the end.
  const uint32_t cap = uint32_t(TS * OP * kThreads);
  uint32_t pe0 = 0, pe1 = 0;
  const float* pd = dt[0];
  const const_u32* tb = (const const_u32*)a.tile_begin;
  // the share's tiles, one row panel at a time (no conditional load inside a
  // panel's loop: the wait for one would drain every load and store ahead)
  for (uint32_t t = t0; t < t1;) {
    const uint32_t panel_end = (t / tc + 1) * tc < t1 ? (t / tc + 1) * tc : t1;
    if (kResident) {
#pragma unroll
      for (int kb = 0; kb < KB8; ++kb)
#pragma unroll
        for (int rb = 0; rb < kSdRb; ++rb) xa[kb][rb] = load4(x_run(t) + (rb * steps + kb) * 256);
    }
  for (; t < panel_end; ++t) {
    const uint32_t ne0 = tb[t], ne1 = tb[t + 1];
    const uint32_t clen = (pe1 - pe0 + uint32_t(TS) - 1) / uint32_t(TS);
    // the tile's steps with OPv output slots per thread and step
    auto tile_steps = [&](auto op_count) {
    constexpr int OPv = decltype(op_count)::value;
    uint64_t oc[kSdOutSets][OPv];
    float ov[kSdOutSets][OPv];
    // lanes past the chunk take its last entry (entry 0 when nothing is
    // pending and no entry precedes: a plan holds at least one tile's room)
    auto load_chunk = [&](int gs, int set) {
      const uint32_t cs = pe0 + uint32_t(gs) * clen;
      const uint32_t ce = cs + clen < pe1 ? cs + clen : pe1;
      const uint32_t lim = ce > 0 ? ce - 1 : 0;
#pragma unroll
      for (int j = 0; j < OPv; ++j) {
        uint32_t e = cs + uint32_t(j * kThreads + tid);
        e = e < lim ? e : lim;
        oc[set][j] = __builtin_nontemporal_load(a.entries + e);
        ov[set][j] = __builtin_nontemporal_load(a.values + e);
      }
    };
    auto store_chunk = [&](int gs, int set) {
      const uint32_t cs = pe0 + uint32_t(gs) * clen;
      const uint32_t ce = cs + clen < pe1 ? cs + clen : pe1;
#pragma unroll
      for (int j = 0; j < OPv; ++j)
        emit_pipe(oc[set][j], ov[set][j], pd, cs + uint32_t(j * kThreads + tid) < ce, pe1 > pe0);
    };
#pragma unroll
    for (int j = 0; j < kSdOutAhead; ++j) load_chunk(j, j);
    for (int unit = 0; unit < units; ++unit) {
      const int f8 = unit * KB8;  // first step of this unit
      const bool tile_end = kResident || unit + 1 == units;
      if (!kResident) {
        const float* xrun = x_run(t);
#pragma unroll
        for (int kb = 0; kb < KB8; ++kb)
#pragma unroll
          for (int rb = 0; rb < kSdRb; ++rb) xa[kb][rb] = load4(xrun + (rb * steps + f8 + kb) * 256);
      }
      // the runs the loads ahead read: this tile's, or the next tile's
      const float* ycur[kSdNb];
      const float* ynext[kSdNb];
#pragma unroll
      for (int cb = 0; cb < kSdNb; ++cb) {
        ycur[cb] = y_run(t, cb);
        ynext[cb] = tile_end ? y_run(t + 1, cb) : ycur[cb] + (f8 + KB8) * 256;
      }
#pragma unroll
      for (int kb = 0; kb < KB8; ++kb) {
        float4 xs[kSdRb];
#pragma unroll
        for (int rb = 0; rb < kSdRb; ++rb) xs[rb] = xa[kb][rb];
        float4 ys[kSdNb];
#pragma unroll
        for (int cb = 0; cb < kSdNb; ++cb) ys[cb] = yb[kb % kSdRing][cb];
        mfma_step<kSdRb, kSdNb>(acc, xs, ys);
        // the Y step loaded now: of this unit, of the next unit of this tile,
        // or of the next tile's first unit
        const int ahead = kb + kSdRing - 1;
#pragma unroll
        for (int cb = 0; cb < kSdNb; ++cb)
          yb[ahead % kSdRing][cb] = ahead < KB8 ? load4(ycur[cb] + (f8 + ahead) * 256)
                                                : load4(ynext[cb] + (ahead - KB8) * 256);
        // the previous tile's outputs: this step's chunk out, a later one in
        // (chunks past the tile's last step are not loaded where that is known)
        const int gs = f8 + kb;
        store_chunk(gs, kb % kSdOutSets);
        if (!kResident || kb + kSdOutAhead < KB8)
          load_chunk(gs + kSdOutAhead, (kb + kSdOutAhead) % kSdOutSets);
        // interleave the step's other instructions with its MFMAs (one wave
        // per SIMD: the matrix core idles while the wave issues anything else
        // in a run of its own), and keep them in this step (the scheduler
        // would sink the loads towards their use and shorten the prefetch)
#pragma unroll
        for (int i = 0; i < 4 * kSdRb * kSdNb; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
          __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // VALU
          __builtin_amdgcn_sched_group_barrier(0x040, 1, 0);  // VMEM write
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    };
    const uint32_t n = pe1 - pe0;
    if (n <= uint32_t(TS * OP1 * kThreads)) tile_steps(std::integral_constant<int, OP1>{});
    else if (n <= uint32_t(TS * OP2 * kThreads)) tile_steps(std::integral_constant<int, OP2>{});
    else tile_steps(std::integral_constant<int, OP>{});
    // the tile's D into the buffer the pending tile does not use; after the
    // barrier every wave has finished the pending tile's outputs and sees D
    float* dn = pd == dt[0] ? dt[1] : dt[0];
#pragma unroll
    for (int rb = 0; rb < kSdRb; ++rb)
#pragma unroll
      for (int cb = 0; cb < kSdNb; ++cb) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          dn[(wr + rb * 32 + 8 * (r / 4) + 4 * g + (r % 4)) * kSdLd + wc + cb * 32 + l32] =
              acc[rb][cb][r];
        acc[rb][cb] = v16f{};
      }
    __syncthreads();
    pd = dn;
    pe0 = ne0;
    pe1 = ne1 - ne0 < cap ? ne1 : ne0 + cap;
  }
  }
  // the last tile's outputs, kSdBatch per thread in flight
  for (uint32_t base = pe0; base < pe1; base += kSdBatch * kThreads) {
    uint64_t code[kSdBatch];
    float val[kSdBatch];
#pragma unroll
    for (int j = 0; j < kSdBatch; ++j) {
      const uint32_t e = base + uint32_t(j * kThreads + tid);
      code[j] = e < pe1 ? __builtin_nontemporal_load(a.entries + e) : 0;
      val[j] = e < pe1 ? __builtin_nontemporal_load(a.values + e) : 0.f;
    }
#pragma unroll
    for (int j = 0; j < kSdBatch; ++j)
      if (base + uint32_t(j * kThreads + tid) < pe1) emit(code[j], val[j], pd);
  }
  // entries past a tile's cap: the dot products taken one entry per thread
  // from the fragment-order operands
  for (uint32_t t = t0; t < t1; ++t) {
    const uint32_t e0 = tb[t], count = tb[t + 1] - e0;
    for (uint32_t j = cap + uint32_t(tid); j < count; j += kThreads) {
      const uint32_t e = e0 + j;
      const uint64_t code = a.entries[e];
      const uint32_t local = uint32_t(code >> (kPosBits + kWsBits));
      const size_t hr = size_t(t / tc) * kSdRows + local / kSdLd;  // block row
      const size_t hc = size_t(t % tc) * kSdCols + local % kSdLd;  // block column
      float dot = 0.f;
      for (int f = 0; f < a.K; f += 4) {
        const float4 x = load4(a.Xf + frag_offset(hr, size_t(f), size_t(a.K)));
        const float4 y = load4(a.Yf + frag_offset(hc, size_t(f), size_t(a.K)));
        dot = fmaf(x.x, y.x, dot);
        dot = fmaf(x.y, y.y, dot);
        dot = fmaf(x.z, y.z, dot);
        dot = fmaf(x.w, y.w, dot);
      }
      const float r = a.values[e] * dot;
      const int s = int((code >> kPosBits) & ((1u << kWsBits) - 1u));
      if (kCsr) a.out_csr[s_pos[s][uint32_t(code)]] = r;
      else s_out[s][uint32_t(code)] = r;
    }
  }
}

template <bool kCsr>
void launch_hub_sddmm(const HubSddmmArgs& a, unsigned grid, hipStream_t st) {
  switch (a.K) {
    case 32: hub_sddmm_kernel<4, true, kCsr><<<grid, kThreads, 0, st>>>(a); break;
    case 64: hub_sddmm_kernel<8, true, kCsr><<<grid, kThreads, 0, st>>>(a); break;
    case 96: hub_sddmm_kernel<12, true, kCsr><<<grid, kThreads, 0, st>>>(a); break;
    case 128: hub_sddmm_kernel<16, true, kCsr><<<grid, kThreads, 0, st>>>(a); break;
    default: hub_sddmm_kernel<4, false, kCsr><<<grid, kThreads, 0, st>>>(a); break;
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

// One SpMM feature slice in a.fgroups groups of 32 CB features: the grid
// holds as many workgroups as the CUs run at once (more rounds of shorter
// shares add more partial rows into C and measured slower on C3).
template <int CB>
void spmm_launch_cb(const HubSpmmArgs& a, int cus, uint64_t iterations, hipStream_t st) {
  // as many workgroups as the CUs hold at once, a multiple of the feature
  // groups, each group's over an even share of the loop iterations (at least
  // one each)
  const uint64_t fgs = uint64_t(a.fgroups);
  const uint64_t slots = uint64_t(cus > 0 ? cus : 1) * spmm_wg_per_cu(CB) / fgs;
  const unsigned grid = unsigned((iterations < slots ? iterations : slots) * fgs);
  // a deeper A ring for a single feature block (fewer MFMAs per A load)
  hub_spmm_kernel<CB, (CB == 1 ? 8 : 4)><<<grid, kThreads, 0, st>>>(a);
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

size_t ps_hub_dense_floats(int rows, int cols) {
  return rows > 0 && cols > 0 ? ps::frag_rows(rows) * ps::dense_ld(cols) : 0;
}

int ps_hub_dense_build(const ps_hub_block* hb, const int* row_ptr, const int* col_ind,
                       const float* sp_data, float* dense, uint32_t* stored, ps_stream_t stream) {
  const int rc = ps::check_block(hb);
  if (rc != PS_OK) return rc;
  PS_CHECK_ARG(row_ptr && col_ind && sp_data && dense && stored, "ps_hub_dense_build: null argument");
  PS_CHECK_ARG(ps::aligned16(dense), "ps_hub_dense_build: dense must be 16-byte aligned");
  hipStream_t st = ps::to_hip(stream);
  PS_HIP(hipMemsetAsync(dense, 0, sizeof(float) * ps_hub_dense_floats(hb->rows, hb->cols), st));
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
  if (!hb || N <= 0 || hb->rows <= 0 || hb->cols <= 0) return 0;
  if (op == PS_OP_SDDMM) {
    // X[hub_rows] and Y[hot_cols] in fragment order, padded to whole tiles
    const size_t xrows = size_t(ps::sddmm_tiles_r(hb)) * ps::kSdRows;
    const size_t yrows = size_t(ps::sddmm_tiles_c(hb)) * ps::kSdCols;
    return ps::round256(xrows * size_t(N) * 4) + ps::round256(yrows * size_t(N) * 4);
  }
  if (op != PS_OP_SPMM) return 0;
  // one feature slice of B's hot rows in fragment order; row flags; the any-flag
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
  ps::clear_flags_kernel<<<ps::grid_for(size_t(hb->cols), ps::kThreads), ps::kThreads, 0, st>>>(
      row_flag, hb->cols, any_flag);
  PS_LAUNCHED();
  ps::HubSpmmArgs a{};
  a.dense = hb->dense;
  a.Bt = Bt;
  a.C = C;
  a.hub_rows = hb->hub_rows;
  a.R = hb->rows;
  a.N = N;
  a.ld = ld;
  a.panels = (hb->rows + ps::kSpRows - 1) / ps::kSpRows;
  int cus = 0;
  {
    int dev = 0;
    PS_HIP(hipGetDevice(&dev));
    PS_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  }
  // loop iterations of the coarsest kernel (64 hot columns; the others take 32)
  const uint64_t iterations = uint64_t(a.panels) * uint64_t(ld / 64);
  PS_CHECK_ARG(uint64_t(a.panels) * uint64_t(ld / 32) < (1ull << 32),
               "ps_hub_spmm_launch: block too large");
  for (int f0 = 0; f0 < N; f0 += ps::kSpSlice) {
    const int width = N - f0 < ps::kSpSlice ? N - f0 : ps::kSpSlice;
    ps::gather_hot_kernel<<<ps::grid_for(size_t(width / 32) * size_t(ld / 8) * 64 / 4, ps::kThreads),
                            ps::kThreads, 0, st>>>(B, hb->hot_cols, hb->cols, N, ld, f0, width, Bt,
                                                   row_flag, any_flag);
    PS_LAUNCHED();
    a.f0 = f0;
    switch (width / 32) {
      // 64 features per workgroup at most (its partial and running sums
      // both in registers): 128 features as two groups, 96 as three of 32
      case 1: a.fgroups = 1; ps::spmm_launch_cb<1>(a, cus, iterations, st); break;
      case 2: a.fgroups = 1; ps::spmm_launch_cb<2>(a, cus, iterations, st); break;
      case 3: a.fgroups = 3; ps::spmm_launch_cb<1>(a, cus, iterations, st); break;
      default: a.fgroups = 2; ps::spmm_launch_cb<2>(a, cus, iterations, st); break;
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
  // (entry indices, and the kernel's chunk and tail offsets past them, stay in 32 bits)
  PS_CHECK_ARG(uint64_t(tile_count) * 64 < (1ull << 31), "ps_hub_sddmm_plan: too many tiles");
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
  PS_HIP(ps::dev_malloc(&base, bytes));
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
  ps::dev_free(base);
  if (r != PS_OK) return r;
  PS_HIP(e);
  return PS_OK;
}

int ps_hub_sddmm_launch(const ps_hub_block* hb, int workset_count, const ps_workset* worksets,
                        const void* plan, uint32_t tile_count, int N, const float* lhs,
                        const float* rhs, float* const* out, const int* const* out_pos,
                        float* out_csr, void* workspace, size_t workspace_bytes,
                        ps_stream_t stream) {
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
  PS_CHECK_ARG(uint64_t(tile_count) * 64 < (1ull << 31), "ps_hub_sddmm_launch: too many tiles");
  PS_CHECK_ARG(workspace && ps::aligned16(workspace) &&
                   workspace_bytes >= ps_hub_workspace_bytes(hb, PS_OP_SDDMM, N),
               "ps_hub_sddmm_launch: workspace too small");
  ps::HubSddmmArgs a{};
  for (int s = 1; s < workset_count; ++s) {
    a.out[s] = out ? out[s] : nullptr;
    a.out_pos[s] = out_pos ? out_pos[s] : nullptr;
    PS_CHECK_ARG(worksets[s].group_num <= 0 || worksets[s].group_size < 64 ||
                     (out_csr ? a.out_pos[s] != nullptr : a.out[s] != nullptr),
                 "ps_hub_sddmm_launch: missing outputs of a block workset");
  }
  a.out_csr = out_csr;
  a.K = N;
  a.tiles_r = int(ps::sddmm_tiles_r(hb));
  a.tiles_c = int(ps::sddmm_tiles_c(hb));
  const size_t T = size_t(a.tiles_r) * size_t(a.tiles_c);
  const char* pb = static_cast<const char*>(plan);
  a.tile_begin = reinterpret_cast<const uint32_t*>(pb);
  a.entries = reinterpret_cast<const uint64_t*>(pb + ps::round256((T + 1) * 4));
  a.values = reinterpret_cast<const float*>(reinterpret_cast<const char*>(a.entries) +
                                            ps::round256(size_t(tile_count) * 64 * 8));
  // as many workgroups as the CUs hold at once (the D buffers in LDS bound
  // them), each over an even share of the tiles
  int cus = 0;
  {
    int dev = 0;
    PS_HIP(hipGetDevice(&dev));
    PS_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  }
  const uint64_t slots = uint64_t(cus > 0 ? cus : 1) * ps::kSdWgPerCu;
  const uint64_t grid = T < slots ? T : slots;
  PS_CHECK_ARG(T < (1ull << 32), "ps_hub_sddmm_launch: block too large");
  // neighbouring shares (a row panel's X, Y columns of neighbouring tiles) on
  // one XCD: up to 32 consecutive shares per XCD
  a.chunk_log2 = 0;
  while ((2u << a.chunk_log2) <= 32 && (uint64_t(2) << a.chunk_log2) * ps::kXcd <= grid)
    ++a.chunk_log2;
  hipStream_t st = ps::to_hip(stream);
  // X[hub_rows] and Y[hot_cols] in fragment order
  const int xrows = a.tiles_r * ps::kSdRows, yrows = a.tiles_c * ps::kSdCols;
  float* xf = static_cast<float*>(workspace);
  float* yf = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                       ps::round256(size_t(xrows) * size_t(N) * 4));
  ps::gather_rows_kernel<<<ps::grid_for(size_t(xrows) * size_t(N) / 4, ps::kThreads), ps::kThreads,
                           0, st>>>(lhs, hb->hub_rows, hb->rows, xrows, N, xf);
  PS_LAUNCHED();
  ps::gather_rows_kernel<<<ps::grid_for(size_t(yrows) * size_t(N) / 4, ps::kThreads), ps::kThreads,
                           0, st>>>(rhs, hb->hot_cols, hb->cols, yrows, N, yf);
  PS_LAUNCHED();
  a.Xf = xf;
  a.Yf = yf;
  if (out_csr) ps::launch_hub_sddmm<true>(a, unsigned(grid), st);
  else ps::launch_hub_sddmm<false>(a, unsigned(grid), st);
  PS_LAUNCHED();
  return PS_OK;
}

}  // extern "C"
