// SDDMM (edge messaging), out[p] = a_p * <X[row], Y[col_p]>, FP32, on gfx950.
//
// One launch covers every workset. Wave tasks:
//   block workset: 64 consecutive stored nonzeros (one group when GS >= 64, two
//     groups of 32 when GS == 32);
//   residue workset: 8 groups per wave, one slot per group, as stored or in
//     the workset's run order (ps_workset.order); a slot loads its group's X
//     row once, stages the group's columns and values in LDS and walks it 8
//     nonzeros at a time; in stored order the task's results (one contiguous
//     output range) are collected in LDS and added with whole-wave atomics
//     at the end.
// Lanes form slots of 8; slot q owns 8 consecutive nonzeros and each lane of the
// slot holds K / 8 features of X (float4 pieces 32 floats apart, so a slot reads
// a 128-byte line per piece). Each lane's 8 partial dots go through a
// transposing butterfly (xor 4, 2, 1 via swizzle / DPP; the xor-4 exchange per
// pair of nonzeros j, j + 4 as soon as their partials are summed): each
// exchange halves the number of partials a lane keeps, and at the end lane
// `sub` of slot `q` holds the full dot of nonzero 8q + sub, so the wave's 64
// results are stored with one coalesced write.
//
// Reference behaviour kept (PowerSparse_SDDMM/sddmm_solution.cu:7-50,
// sddmm_kernel_block.cu:155-164, sddmm_kernel_residue.cu:295-305): block
// outputs are stored, residue outputs are added atomically into out[0], the
// output is in workset order.
//
// Run order: a launch may carry a permutation of its tasks (task_map); the
// C++ API passes the locality order (block tiles by first column) for
// signature-ordered worksets. A task's work, and so every output, is the same
// in any order; residue tasks keep their 8 consecutive groups.
//
// Store modes (kMode): 0 = at the nonzero's own position (as above); 1 = per
// nonzero map, out[s][map[s][p]]: CSR order (every out[s] is the one
// CSR-order array, map = CSR positions, plain stores: each position is
// written once, no zeroing needed); 2 = per group base, out[s][base[s][g] + j]
// for member j of group g: a row-ordered execution copy of the worksets
// writing the public workset layout (residue results still added atomically).
#include "ps_common.hpp"

namespace ps {
namespace {

constexpr int kWavesPerBlock = 4;
constexpr int kStage = 32;  // residue columns (and values) staged in LDS per slot
constexpr int kTaskOut = 256;  // residue results of one task collected in LDS
// Longest XCD run of PS_TASK_CHUNK_AUTO (measured in the locality run order,
// C3 N = 128: runs of 256 workgroups 1.4% faster than the round robin, 1024
// slower on C1).
constexpr int kAutoChunkMax = 256;
static_assert(kTaskOut >= 8 * kStage, "a task's slots each collect up to kStage results");

struct SddmmArgs {
  ps_workset ws[PS_MAX_WORKSETS];
  float* out[PS_MAX_WORKSETS];
  uint32_t task_begin[PS_MAX_WORKSETS + 1];
  int32_t count;
  int32_t N;
  uint32_t total_tasks;   // tasks of the worksets
  uint32_t launch_tasks;  // waves with work: total_tasks, or the task map's length
  const int* residue_offset;
  const float* lhs;
  const float* rhs;
  uint64_t lhs_bytes;
  uint64_t rhs_bytes;
  const int* out_pos[PS_MAX_WORKSETS];  // mode 1: per-nonzero map; mode 2: per-group base
  int32_t residue_add;                  // modes 1-2: residue results added, not stored
  uint32_t chunk_log2;                  // workgroup -> XCD mapping (balanced_block)
  const uint32_t* task_map;             // run order of the tasks, or null
};

// Transposing reduction over the 8 lanes of a slot: in p[j] each lane holds
// its partial for nonzero j of the slot; returns the full sum for j == sub.
__device__ __forceinline__ float slot_transpose_sum(const float (&p)[8], int sub) {
  const bool b2 = sub & 4, b1 = sub & 2, b0 = sub & 1;
  float q[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float keep = b2 ? p[i + 4] : p[i];
    const float send = b2 ? p[i] : p[i + 4];
    q[i] = keep + xor_shfl<4>(send);
  }
  float r[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float keep = b1 ? q[i + 2] : q[i];
    const float send = b1 ? q[i] : q[i + 2];
    r[i] = keep + xor_shfl<2>(send);
  }
  const float keep = b0 ? r[1] : r[0];
  const float send = b0 ? r[0] : r[1];
  return keep + xor_shfl<1>(send);
}

// Partial dots of the 8 nonzeros of this lane's slot (Y row byte offsets in
// yoff[]), `kSteps` nonzeros per batch: 8-16 loads in flight per lane.
template <int KQ, bool kBuf>
__device__ __forceinline__ void slot_dots(const Rows<kBuf>& Y,
                                          const typename Rows<kBuf>::Off (&yoff)[8],
                                          const float4 (&x)[KQ], float (&p)[8]) {
  // a power of two dividing the 8 steps: 16 loads for K <= 64, 8 for K = 96,
  // 128 (in the run order, C3 N = 128: 7.69 ms with 16, 7.50 with 8, 7.74
  // with 4; C1 2.272 / 2.278 / 2.342 ms), 16 for K <= 256, 16-32 beyond
  constexpr int kSteps = KQ <= 2 ? 8 : (KQ <= 4 ? 2 : (KQ <= 8 ? 2 : 1));
  static_assert(8 % kSteps == 0, "batches must tile the slot's 8 nonzeros");
#pragma unroll
  for (int b = 0; b < 8; b += kSteps) {
    float4 y[kSteps][KQ];
#pragma unroll
    for (int u = 0; u < kSteps; ++u)
#pragma unroll
      for (int q = 0; q < KQ; ++q) y[u][q] = Y.load(yoff[b + u] + 128u * uint32_t(q));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kSteps; ++u) {
      float s = 0.f;
#pragma unroll
      for (int q = 0; q < KQ; ++q) {
        s = fmaf(x[q].x, y[u][q].x, s);
        s = fmaf(x[q].y, y[u][q].y, s);
        s = fmaf(x[q].z, y[u][q].z, s);
        s = fmaf(x[q].w, y[u][q].w, s);
      }
      p[b + u] = s;
    }
  }
}

// The full dot of nonzero `sub` of this lane's slot, whose 8 nonzeros have
// the columns col_of(0 .. 7). Up to K = 256 the nonzeros are taken in pairs
// (j, j + 4), P pairs per batch, and each pair's partials pass the
// butterfly's first (xor 4) exchange at once, so a lane keeps 4 partials
// instead of 8 and no row offsets (the same sums, bit for bit; with one pair
// per batch the K = 128 kernel took 69 VGPRs instead of 79 and ran C3 SDDMM
// N=128 in 6.26 instead of 6.29 ms).
template <int KQ, bool kBuf, typename ColOf>
__device__ __forceinline__ float slot_dot(const Rows<kBuf>& Y, uint32_t row_bytes, uint32_t piece,
                                          const float4 (&x)[KQ], int sub, ColOf col_of) {
  using Off = typename Rows<kBuf>::Off;
  if constexpr (KQ > 8) {
    float p[8];
    Off yoff[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) yoff[j] = Off(uint32_t(col_of(j))) * row_bytes + piece;
    slot_dots<KQ, kBuf>(Y, yoff, x, p);
    return slot_transpose_sum(p, sub);
  } else {
    // pairs per batch: 8 KQ loads in flight up to K = 64, 16 at K = 128
    // (C3 SDDMM N=128 6.234 -> 6.195 ms, C1 2.250 -> 2.230 ms against 8
    // loads, although the kernel then holds 100 VGPRs, 4 waves per SIMD; 32
    // loads: 6.494 ms; K = 64 with 8 loads instead of 16: C4 1.347 -> 1.372
    // ms), 2 KQ otherwise
    constexpr int P = KQ <= 2 ? 4 : (KQ == 4 ? 2 : 1);
    const bool b2 = sub & 4, b1 = sub & 2, b0 = sub & 1;
    float q[4];
#pragma unroll
    for (int i0 = 0; i0 < 4; i0 += P) {
      float4 y[P][2][KQ];
#pragma unroll
      for (int u = 0; u < P; ++u) {
        const Off o0 = Off(uint32_t(col_of(i0 + u))) * row_bytes + piece;
        const Off o1 = Off(uint32_t(col_of(i0 + u + 4))) * row_bytes + piece;
#pragma unroll
        for (int k = 0; k < KQ; ++k) {
          y[u][0][k] = Y.load(o0 + 128u * uint32_t(k));
          y[u][1][k] = Y.load(o1 + 128u * uint32_t(k));
        }
      }
      // keep the whole batch of loads in flight before the first use
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < P; ++u) {
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int k = 0; k < KQ; ++k) {
          s0 = fmaf(x[k].x, y[u][0][k].x, s0);
          s0 = fmaf(x[k].y, y[u][0][k].y, s0);
          s0 = fmaf(x[k].z, y[u][0][k].z, s0);
          s0 = fmaf(x[k].w, y[u][0][k].w, s0);
          s1 = fmaf(x[k].x, y[u][1][k].x, s1);
          s1 = fmaf(x[k].y, y[u][1][k].y, s1);
          s1 = fmaf(x[k].z, y[u][1][k].z, s1);
          s1 = fmaf(x[k].w, y[u][1][k].w, s1);
        }
        // slot_transpose_sum's first exchange for nonzeros i and i + 4
        const float keep = b2 ? s1 : s0, send = b2 ? s0 : s1;
        q[i0 + u] = keep + xor_shfl<4>(send);
      }
    }
    float r[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float keep = b1 ? q[i + 2] : q[i];
      const float send = b1 ? q[i] : q[i + 2];
      r[i] = keep + xor_shfl<2>(send);
    }
    const float keep = b0 ? r[1] : r[0];
    const float send = b0 ? r[0] : r[1];
    return keep + xor_shfl<1>(send);
  }
}

template <int KQ, bool kBuf, int kMode>
__global__ __launch_bounds__(kWave* kWavesPerBlock) void sddmm_kernel(SddmmArgs args) {
  constexpr int K = 32 * KQ;
  __shared__ __attribute__((aligned(16))) int stage[kWavesPerBlock][8 * kStage];
  __shared__ float task_out[kWavesPerBlock][kTaskOut];  // residue results of a task
  // residue values staged with their columns (no dependent value load after
  // each step's dots: C3 SDDMM N=128 6.303 -> 6.292 ms)
  __shared__ __attribute__((aligned(16))) float stage_val[kWavesPerBlock][8 * kStage];
  const uint32_t blk = balanced_block(blockIdx.x, gridDim.x, args.chunk_log2);
  uint32_t task = __builtin_amdgcn_readfirstlane(blk * kWavesPerBlock + threadIdx.x / kWave);
  if (task >= args.launch_tasks) return;
  if (args.task_map) {  // a permutation of [0, total_tasks), or of a subset of it
    task = __builtin_amdgcn_readfirstlane(args.task_map[task]);
    if (task >= args.total_tasks) return;
  }
  int i = 0;
  while (i + 1 < args.count && task >= args.task_begin[i + 1]) ++i;
  const ps_workset ws = args.ws[i];
  float* __restrict__ out = args.out[i];
  const int* __restrict__ out_pos = args.out_pos[i];
  const int local = int(task - args.task_begin[i]);

  const int lane = lane_id();
  const int slot = lane / 8, sub = lane % 8;
  const Rows<kBuf> X(args.lhs, args.lhs_bytes), Y(args.rhs, args.rhs_bytes);
  using Off = typename Rows<kBuf>::Off;
  const uint32_t row_bytes = uint32_t(K) * 4u;
  const uint32_t piece = uint32_t(sub) * 16u;
  float4 x[KQ];
  int* const wave_stage = stage[threadIdx.x / kWave];

  if (ws.group_size > 0) {
    const int total = ws.group_num * ws.group_size;
    const int p0 = local * 64 + slot * 8;
    const bool valid = p0 < total;
    const int gs_shift = __builtin_ctz(unsigned(ws.group_size));  // a power of two
    const int g = valid ? p0 >> gs_shift : 0;
    const int row = valid ? ws.group_des[g] : 0;
    // the lane's column id and value (one coalesced load each; the column ids
    // go through the wave's LDS to their slots), loaded before the dots (no
    // dependent load at the end of the task: C3 SDDMM N=128 6.346 -> 6.297 ms)
    const int pos = local * 64 + lane;
    const float a_val = valid ? __builtin_nontemporal_load(ws.sp_data + pos) : 0.f;
    // column ids are read once per launch: non-temporal, so that they
    // displace fewer of the L2's Y rows (C3 SDDMM N=128 6.71 -> 6.69 ms)
    wave_stage[lane] = valid ? __builtin_nontemporal_load(ws.col_ind + pos) : 0;
    // the output's index, also loaded up front in the mapped modes
    int dst = pos;
    if constexpr (kMode == 1) {
      if (valid) dst = out_pos[pos];
    } else if constexpr (kMode == 2) {
      const int gl = pos >> gs_shift;
      if (valid) dst = out_pos[gl] + (pos - gl * ws.group_size);
    }
#pragma unroll
    for (int q = 0; q < KQ; ++q) x[q] = X.load(Off(uint32_t(row)) * row_bytes + piece + 128u * q);
    wave_lds_sync();
    const int* const slot_cols = wave_stage + slot * 8;
    const float dot = slot_dot<KQ, kBuf>(Y, row_bytes, piece, x, sub,
                                         [&](int j) { return slot_cols[j]; });
    if (valid) {
      // every output is written once and not read back by the launch:
      // non-temporal stores keep them from displacing Y rows in the L2 (C3
      // SDDMM N=128 6.374 -> 6.348 ms)
      __builtin_nontemporal_store(dot * a_val, out + dst);
    }
  } else {
    // One slot per group (the run order's entry local * 8 + slot: order[]
    // when given, else as stored); the slot's group is walked 8 nonzeros at a
    // time.
    // In stored order the task's 8 groups own one contiguous output range
    // [off[8 local], off[8 local + 8]). When it holds at most kTaskOut results
    // they are collected in LDS and added at the end with atomics covering
    // 256 contiguous bytes per instruction; a slot adding its 8 results per
    // step touches one or two 64-byte sectors for 32 bytes, and float atomics
    // cost per sector touched (128-byte rows: 2.5 G/s with lanes 16 bytes
    // apart, 5.1 G/s with 8 lanes on 32 bytes, 10.3 G/s with 32 lanes per row).
    const int g0 = local * 8;
    const int g_end = g0 + 8 < ws.group_num ? g0 + 8 : ws.group_num;
    const int out0 = kMode == 0 && !ws.order ? args.residue_offset[g0] : 0;
    const int span = kMode == 0 && !ws.order ? args.residue_offset[g_end] - out0 : kTaskOut + 1;
    const bool collect = span <= kTaskOut;
    float* const res_lds = task_out[threadIdx.x / kWave];
    const int kq = local * 8 + slot;
    int g = kq < ws.group_num ? (ws.order ? ws.order[kq] : kq) : -1;
    const bool has = g >= 0 && g < ws.group_num;  // order entries out of range are skipped
    if (!has) g = 0;
    const int beg = has ? args.residue_offset[g] : 0;
    const int len = has ? args.residue_offset[g + 1] - beg : 0;
    const int row = has ? ws.group_des[g] : 0;
    // row-order copy (mode 2) adding its results: a group of up to kStage
    // results is collected in LDS and added with 32 lanes on its output range
    const bool group_collect = kMode == 2 && args.residue_add && len <= kStage;
    // a residue group's X row is read by this task alone in the launch's
    // order (the row's block tiles run long before): non-temporal (C3 SDDMM
    // N=128 6.271 -> 6.254 ms, C4 N=64 1.358 -> 1.348 ms; the block tiles' X
    // rows, shared by a hub row's tiles, measured 2% slower so)
#pragma unroll
    for (int qq = 0; qq < KQ; ++qq)
      x[qq] = X.load_nt(Off(uint32_t(row)) * row_bytes + piece + 128u * qq);
    // The group's columns and values pass through the slot's LDS area in
    // chunks of kStage (one chunk for every group the preprocessing builds),
    // positions past the group's end holding its last column (those
    // nonzeros' dots are dropped); the chunk boundaries are the same for the
    // whole wave (c0 is uniform).
    int* const cols_lds = stage[threadIdx.x / kWave] + slot * kStage;
    float* const vals_lds = stage_val[threadIdx.x / kWave] + slot * kStage;
#pragma unroll 1
    for (int c0 = 0; __any(c0 < len); c0 += 8) {
      const int cs = c0 % kStage;  // place of nonzero c0 in the staged chunk
      if (cs == 0) {
        if (c0 > 0) wave_lds_sync();  // the previous chunk's reads come first
#pragma unroll
        for (int j = sub; j < kStage; j += 8) {
          const int k = c0 + j;
          const int at = beg + (k < len ? k : len - 1);
          cols_lds[j] = len > 0 ? ws.col_ind[at] : 0;
          vals_lds[j] = len > 0 ? ws.sp_data[at] : 0.f;
        }
        wave_lds_sync();
      }
      const float dot = slot_dot<KQ, kBuf>(Y, row_bytes, piece, x, sub,
                                           [&](int j) { return cols_lds[cs + j]; });
      const int k = c0 + sub;
      if (k < len) {
        const float v = dot * vals_lds[cs + sub];
        if constexpr (kMode == 2) {
          if (group_collect) res_lds[slot * kStage + k] = v;
          else if (args.residue_add) unsafeAtomicAdd(out + out_pos[g] + k, v);
          else out[out_pos[g] + k] = v;
        } else if constexpr (kMode == 1) {
          const int at = out_pos[beg + k];
          if (args.residue_add) unsafeAtomicAdd(out + at, v);
          else out[at] = v;
        } else if (collect) {
          res_lds[beg + k - out0] = v;
        } else {
          unsafeAtomicAdd(out + beg + k, v);
        }
      }
    }
    if constexpr (kMode == 2) {
      // groups of up to kStage results, collected per slot: two groups per
      // instruction, 32 lanes on each group's contiguous output range
      if (args.residue_add) {
        const int base = has ? out_pos[g] : 0;
        wave_lds_sync();
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int q = 2 * j + lane / 32, e = lane % 32;
          const int lq = __shfl(len, q * 8), bq = __shfl(base, q * 8);
          if (e < lq && lq <= kStage) unsafeAtomicAdd(out + bq + e, res_lds[q * kStage + e]);
        }
      }
    }
    if (collect) {
      wave_lds_sync();
#pragma unroll
      for (int j = 0; j < kTaskOut / kWave; ++j) {
        const int e = j * kWave + lane;
        if (e < span) unsafeAtomicAdd(out + out0 + e, res_lds[e]);
      }
    }
  }
}

// out[pos[e]] = in[e]: workset-order values to CSR order.
__global__ void to_csr_kernel(const float* __restrict__ in, const int* __restrict__ pos,
                              size_t n, float* __restrict__ out) {
  for (size_t e = size_t(blockIdx.x) * blockDim.x + threadIdx.x; e < n;
       e += size_t(gridDim.x) * blockDim.x)
    out[pos[e]] = in[e];
}

template <int KQ>
void launch_kq(const SddmmArgs& a, bool buf, int mode, unsigned grid, hipStream_t stream) {
  constexpr unsigned kBlock = kWave * kWavesPerBlock;
  if (mode == 1) {
    if (buf) sddmm_kernel<KQ, true, 1><<<grid, kBlock, 0, stream>>>(a);
    else sddmm_kernel<KQ, false, 1><<<grid, kBlock, 0, stream>>>(a);
  } else if (mode == 2) {
    if (buf) sddmm_kernel<KQ, true, 2><<<grid, kBlock, 0, stream>>>(a);
    else sddmm_kernel<KQ, false, 2><<<grid, kBlock, 0, stream>>>(a);
  } else {
    if (buf) sddmm_kernel<KQ, true, 0><<<grid, kBlock, 0, stream>>>(a);
    else sddmm_kernel<KQ, false, 0><<<grid, kBlock, 0, stream>>>(a);
  }
}

// Workset q writes outs[q] at its own positions (mode 0), through the
// per-nonzero map out_pos[q] (mode 1) or after the per-group bases out_pos[q]
// (mode 2); residue results are added when residue_add (modes 1-2).
int launch(int count, const int* order, const ps_workset* worksets, float* const* outs,
           int mode, const int* const* out_pos, int residue_add, const int* residue_offset,
           int rows, int cols, int N, const float* lhs, const float* rhs, int task_chunk,
           const uint32_t* task_map, uint32_t task_map_len, hipStream_t stream) {
  PS_CHECK_ARG(N > 0 && N % 32 == 0 && N <= 512,
               "SDDMM requires N to be a multiple of 32 between 32 and 512");
  PS_CHECK_ARG(int64_t(rows) * N <= INT32_MAX && int64_t(cols) * N <= INT32_MAX,
               "Dense dimensions exceed the 32-bit kernel indexing range");
  PS_CHECK_ARG(lhs && rhs && outs, "Invalid SDDMM buffers");
  PS_CHECK_ARG(aligned16(lhs) && aligned16(rhs), "SDDMM dense buffers must be 16-byte aligned");
  PS_CHECK_ARG(task_chunk_valid(task_chunk),
               "SDDMM task_chunk must be PS_TASK_CHUNK_AUTO, 0 or a power of two up to 4096");
  SddmmArgs a{};
  a.residue_add = residue_add;
  a.N = N;
  a.lhs = lhs;
  a.rhs = rhs;
  const uint64_t lhs_bytes = uint64_t(rows) * uint64_t(N) * 4u;
  const uint64_t rhs_bytes = uint64_t(cols) * uint64_t(N) * 4u;
  const bool buf = lhs_bytes <= 0xFFFFFFFFull && rhs_bytes <= 0xFFFFFFFFull;
  a.lhs_bytes = lhs_bytes;
  a.rhs_bytes = rhs_bytes;
  a.residue_offset = residue_offset;
  uint64_t tasks = 0;
  int n = 0;
  // Validate every workset before submitting any work (sddmm_solution.cu:16-22).
  for (int q = 0; q < count; ++q) {
    const ps_workset& w = worksets[q];
    if (w.group_num <= 0) continue;
    PS_CHECK_ARG(outs[q], "Missing SDDMM output workset");
    if (mode != 0) {
      PS_CHECK_ARG(out_pos && out_pos[q], "Missing output positions of an SDDMM workset");
    }
    PS_CHECK_ARG(w.col_ind && w.sp_data && w.group_des, "Invalid SDDMM workset buffers");
    const int s = order[q];
    uint64_t t;
    if (s > 0) {
      PS_CHECK_ARG(aligned16(w.col_ind), "Block workset arrays must be 16-byte aligned");
      PS_CHECK_ARG(w.group_size >= 32 && (w.group_size & (w.group_size - 1)) == 0,
                   "Block workset group size must be a power of two >= 32");
      // the kernel indexes a block workset's nonzeros (plus a 64-wide tile) in int
      PS_CHECK_ARG(uint64_t(w.group_num) * uint64_t(w.group_size) <= uint64_t(INT32_MAX) - 64,
                   "Block workset exceeds the 32-bit kernel indexing range");
      const uint64_t T = uint64_t(sddmm_task_shape().tile_nnz);
      t = (uint64_t(w.group_num) * w.group_size + T - 1) / T;
    } else {
      PS_CHECK_ARG(residue_offset, "Missing residue offsets");
      const uint64_t R = uint64_t(sddmm_task_shape().residue_groups);  // one slot per group
      t = (uint64_t(w.group_num) + R - 1) / R;
    }
    a.ws[n] = w;
    if (s == 0) a.ws[n].group_size = 0;
    a.out[n] = outs[q];
    if (mode != 0) a.out_pos[n] = out_pos[q];
    a.task_begin[n] = uint32_t(tasks);
    tasks += t;
    ++n;
  }
  if (n == 0) return PS_OK;
  PS_CHECK_ARG(tasks < (1ull << 31), "SDDMM task count exceeds the launch range");
  a.count = n;
  a.task_begin[n] = uint32_t(tasks);
  a.total_tasks = uint32_t(tasks);
  a.launch_tasks = uint32_t(tasks);
  if (task_map) {
    // a subset of the tasks runs when the order lists fewer (the others are
    // computed elsewhere, e.g. by the dense hub block)
    PS_CHECK_ARG(task_map_len <= tasks,
                 "SDDMM task order holds " + std::to_string(task_map_len) + " tasks, the launch " +
                     std::to_string(tasks));
    a.task_map = task_map;
    a.launch_tasks = task_map_len;
  }
  if (a.launch_tasks == 0) return PS_OK;
  const unsigned grid = unsigned((uint64_t(a.launch_tasks) + kWavesPerBlock - 1) / kWavesPerBlock);
  a.chunk_log2 = uint32_t(task_chunk_log2(task_chunk, grid, kAutoChunkMax));
  switch (N / 32) {
    case 1: launch_kq<1>(a, buf, mode, grid, stream); break;
    case 2: launch_kq<2>(a, buf, mode, grid, stream); break;
    case 3: launch_kq<3>(a, buf, mode, grid, stream); break;
    case 4: launch_kq<4>(a, buf, mode, grid, stream); break;
    case 5: launch_kq<5>(a, buf, mode, grid, stream); break;
    case 6: launch_kq<6>(a, buf, mode, grid, stream); break;
    case 7: launch_kq<7>(a, buf, mode, grid, stream); break;
    case 8: launch_kq<8>(a, buf, mode, grid, stream); break;
    case 9: launch_kq<9>(a, buf, mode, grid, stream); break;
    case 10: launch_kq<10>(a, buf, mode, grid, stream); break;
    case 11: launch_kq<11>(a, buf, mode, grid, stream); break;
    case 12: launch_kq<12>(a, buf, mode, grid, stream); break;
    case 13: launch_kq<13>(a, buf, mode, grid, stream); break;
    case 14: launch_kq<14>(a, buf, mode, grid, stream); break;
    case 15: launch_kq<15>(a, buf, mode, grid, stream); break;
    default: launch_kq<16>(a, buf, mode, grid, stream); break;
  }
  PS_LAUNCHED();
  return PS_OK;
}

}  // namespace
}  // namespace ps

extern "C" {

int ps_sddmm_launch(int workset_count, const ps_workset* worksets, const int* residue_offset,
                    int rows, int cols, int N, const float* lhs, const float* rhs,
                    float* const* out, int task_chunk, ps_stream_t stream) {
  PS_CHECK_ARG(workset_count >= 1 && workset_count <= PS_MAX_WORKSETS && worksets && out,
               "Invalid SDDMM workset count");
  int order[PS_MAX_WORKSETS];
  ps_workset ordered[PS_MAX_WORKSETS];
  float* outs[PS_MAX_WORKSETS];
  for (int q = 0; q < workset_count; ++q) {
    order[q] = workset_count - 1 - q;
    ordered[q] = worksets[workset_count - 1 - q];
    outs[q] = out[workset_count - 1 - q];
  }
  return ps::launch(workset_count, order, ordered, outs, 0, nullptr, 0, residue_offset, rows,
                    cols, N, lhs, rhs, task_chunk, nullptr, 0, ps::to_hip(stream));
}

int ps_sddmm_launch_ordered(int workset_count, const ps_workset* worksets,
                            const int* residue_offset, int rows, int cols, int N,
                            const float* lhs, const float* rhs, float* const* out, int task_chunk,
                            const uint32_t* task_order, uint32_t task_count, ps_stream_t stream) {
  PS_CHECK_ARG(workset_count >= 1 && workset_count <= PS_MAX_WORKSETS && worksets && out,
               "Invalid SDDMM workset count");
  int order[PS_MAX_WORKSETS];
  ps_workset ordered[PS_MAX_WORKSETS];
  float* outs[PS_MAX_WORKSETS];
  for (int q = 0; q < workset_count; ++q) {
    order[q] = workset_count - 1 - q;
    ordered[q] = worksets[workset_count - 1 - q];
    outs[q] = out[workset_count - 1 - q];
  }
  return ps::launch(workset_count, order, ordered, outs, 0, nullptr, 0, residue_offset, rows,
                    cols, N, lhs, rhs, task_chunk, task_order, task_count,
                    ps::to_hip(stream));
}

int ps_sddmm_scatter_launch(int workset_count, const ps_workset* worksets,
                            const int* residue_offset, const int* const* out_base, int rows,
                            int cols, int N, const float* lhs, const float* rhs,
                            float* const* out, int task_chunk, ps_stream_t stream) {
  PS_CHECK_ARG(workset_count >= 1 && workset_count <= PS_MAX_WORKSETS && worksets && out_base &&
                   out,
               "Invalid SDDMM workset count");
  int order[PS_MAX_WORKSETS];
  ps_workset ordered[PS_MAX_WORKSETS];
  const int* pos[PS_MAX_WORKSETS];
  float* outs[PS_MAX_WORKSETS];
  for (int q = 0; q < workset_count; ++q) {
    order[q] = workset_count - 1 - q;
    ordered[q] = worksets[workset_count - 1 - q];
    pos[q] = out_base[workset_count - 1 - q];
    outs[q] = out[workset_count - 1 - q];
  }
  return ps::launch(workset_count, order, ordered, outs, 2, pos, 1, residue_offset, rows, cols,
                    N, lhs, rhs, task_chunk, nullptr, 0, ps::to_hip(stream));
}

static int sddmm_csr(int workset_count, const ps_workset* worksets, const int* residue_offset,
                     const int* const* csr_pos, int rows, int cols, int N, const float* lhs,
                     const float* rhs, float* out_csr, int task_chunk, const uint32_t* task_order,
                     uint32_t task_count, ps_stream_t stream) {
  PS_CHECK_ARG(workset_count >= 1 && workset_count <= PS_MAX_WORKSETS && worksets && csr_pos &&
                   out_csr,
               "Invalid SDDMM workset count");
  int order[PS_MAX_WORKSETS];
  ps_workset ordered[PS_MAX_WORKSETS];
  const int* pos[PS_MAX_WORKSETS];
  float* outs[PS_MAX_WORKSETS];
  for (int q = 0; q < workset_count; ++q) {
    order[q] = workset_count - 1 - q;
    ordered[q] = worksets[workset_count - 1 - q];
    pos[q] = csr_pos[workset_count - 1 - q];
    outs[q] = out_csr;
  }
  return ps::launch(workset_count, order, ordered, outs, 1, pos, 0, residue_offset, rows, cols,
                    N, lhs, rhs, task_chunk, task_order, task_count, ps::to_hip(stream));
}

int ps_sddmm_csr_launch(int workset_count, const ps_workset* worksets, const int* residue_offset,
                        const int* const* csr_pos, int rows, int cols, int N, const float* lhs,
                        const float* rhs, float* out_csr, int task_chunk, ps_stream_t stream) {
  return sddmm_csr(workset_count, worksets, residue_offset, csr_pos, rows, cols, N, lhs, rhs,
                   out_csr, task_chunk, nullptr, 0, stream);
}

int ps_sddmm_csr_launch_ordered(int workset_count, const ps_workset* worksets,
                                const int* residue_offset, const int* const* csr_pos, int rows,
                                int cols, int N, const float* lhs, const float* rhs,
                                float* out_csr, int task_chunk, const uint32_t* task_order,
                                uint32_t task_count, ps_stream_t stream) {
  return sddmm_csr(workset_count, worksets, residue_offset, csr_pos, rows, cols, N, lhs, rhs,
                   out_csr, task_chunk, task_order, task_count, stream);
}

int ps_workset_to_csr(int workset_count, const long long* lengths, const int* const* csr_pos,
                      const float* const* in, float* out_csr, ps_stream_t stream) {
  PS_CHECK_ARG(workset_count >= 1 && workset_count <= PS_MAX_WORKSETS && lengths && csr_pos &&
                   in && out_csr,
               "ps_workset_to_csr: bad argument");
  for (int s = 0; s < workset_count; ++s) {
    PS_CHECK_ARG(lengths[s] >= 0, "ps_workset_to_csr: negative length");
    if (lengths[s] == 0) continue;
    PS_CHECK_ARG(csr_pos[s] && in[s], "ps_workset_to_csr: missing workset buffers");
    const size_t n = size_t(lengths[s]);
    size_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    ps::to_csr_kernel<<<unsigned(blocks), 256, 0, ps::to_hip(stream)>>>(in[s], csr_pos[s], n,
                                                                        out_csr);
    PS_LAUNCHED();
  }
  return PS_OK;
}

int ps_sddmm_workset_launch(int s, const ps_workset* workset, const int* residue_offset,
                            int rows, int cols, int N, const float* lhs, const float* rhs,
                            float* out, ps_stream_t stream) {
  PS_CHECK_ARG(s >= 0 && s < PS_MAX_WORKSETS && workset, "Invalid SDDMM workset");
  return ps::launch(1, &s, workset, &out, 0, nullptr, 0, residue_offset, rows, cols, N, lhs,
                    rhs, 1, nullptr, 0, ps::to_hip(stream));
}

}  // extern "C"
