// SpMM (node aggregation), C += A * B, FP32, on gfx950.
//
// One launch covers every workset of a PowerSparse matrix. The grid is a flat
// list of wave tasks; each wave64 decodes its task from a table in the kernel
// arguments. Lanes form SL = 64 / LPN slots of LPN lanes; a slot reads one B-row
// slice of 4 * LPN floats with 128-bit loads, so one wave instruction gathers SL
// B rows. Every lane accumulates a float4 of its slot's output row. Wide N runs
// as column slices of 64 (N a multiple of 64) or 32 floats, all tasks of one
// slice before the next.
//
//   block workset (groups of GS = 32 * 2^(s-1) nonzeros): a task is a tile of
//     T = 32 * SL consecutive stored nonzeros; slot q owns nonzeros
//     [32q, 32q + 32) of the tile. When GS < T a tile holds T / GS whole groups
//     (GS / 32 slots each), otherwise it is a piece of one group. Slots of the
//     same group are summed with DPP / swizzle butterflies and the group's row
//     is added to C with atomics.
//   residue workset: a task is SL groups, as stored or in the workset's run
//     order (ps_workset.order), one per slot; a slot walks its group (at most
//     31 nonzeros) alone, 8 nonzeros at a time, so no cross-slot sum is needed,
//     and writes its row with atomics when the row has other groups, with a
//     plain store otherwise.
//
// Each task first stages its nonzeros in LDS with coalesced loads, as
// (byte offset of the B row, value) pairs, so the gather loop issues batches of
// 8 independent 128-bit B loads per lane with no dependent index load in
// between. B is addressed through a buffer resource with 32-bit offsets when
// cols * N * 4 fits in 32 bits.
//
// Run order: a launch may carry a permutation of one column slice's tasks
// (task_map); task t of every slice then runs task_map[t]. The C++ API passes
// the locality order (block tiles by first column) for signature-ordered
// worksets. Each task's work is the same in any order.
//
// Workgroup -> task mapping: the hardware deals workgroups round-robin over
// the 8 XCDs (workgroups b and b + 8 on the same one). With task_chunk > 1,
// windows of 8 * task_chunk consecutive workgroups are re-dealt so that each
// XCD takes task_chunk consecutive ones: neighbouring tasks share an XCD's
// L2, while every XCD still gets a slice of every window (balance when task
// costs vary along the list). The deal applies before the run order's map.
// PS_TASK_CHUNK_AUTO sizes the runs from the launch (up to kAutoChunkMax).
//
// Reference behaviour kept (PowerSparse_SpMM/spmm_solution.cu:7-34,
// spmm_kernel_block.cu:60-162, spmm_kernel_residue.cu:5-82): block groups and
// flagged residue groups accumulate into C with atomics, unflagged residue
// groups overwrite their row, C is not cleared by the operator.
#include "ps_common.hpp"

namespace ps {
namespace {

// Waves per workgroup: 2 for 8-lane slots (32-float slices: C3 SpMM N=32
// 1.586 -> 1.573 ms, C1 0.502 -> 0.497 ms against 4; 64-float slices run
// best at 4: C3 N=128 5.654 ms against 5.711 at 2 and 5.734 at 8).
constexpr int waves_per_block(int lpn) { return lpn == 8 ? 2 : 4; }
constexpr int kPer = 32;          // nonzeros per slot per block tile
constexpr int kSlotWords = 2 * kPer + 4;  // LDS words per slot (pairs + pad)
// Longest XCD run of PS_TASK_CHUNK_AUTO (measured on the tuned SpMM partition,
// C3: runs of 1024 workgroups 3-4% faster than the round robin, 4096 no better;
// C1: 256 best, 4-5% faster).
constexpr int kAutoChunkMax = 1024;
// B loads in flight per lane. 8 keeps the kernel at 62 VGPRs, i.e. 8 waves per
// SIMD; 16 needs 110 VGPRs (4 waves) and ran 4-9% slower on C1, C3 and C4.
constexpr int kBatch = 8;
// Residue groups are walked 8 nonzeros at a time too: they hold 1..31 nonzeros
// and a wave runs as long as its longest group (16 cost 3% more).
constexpr int kRBatch = 8;

struct SpmmArgs {
  ps_workset ws[PS_MAX_WORKSETS];
  uint32_t task_begin[PS_MAX_WORKSETS + 1];
  int32_t count;
  int32_t N;
  int32_t slices;
  uint32_t total_tasks;
  uint64_t b_bytes;  // size of B in bytes
  const int* residue_offset;
  const uint8_t* residue_atomic;
  const float* B;
  float* C;
  uint32_t chunk_log2;  // workgroup -> XCD mapping (balanced_block)
  const uint32_t* task_map;  // run order of one column slice's tasks, or null
};

__device__ __forceinline__ void fma4(float4& acc, float a, const float4& b) {
  acc.x = fmaf(a, b.x, acc.x);
  acc.y = fmaf(a, b.y, acc.y);
  acc.z = fmaf(a, b.z, acc.z);
  acc.w = fmaf(a, b.w, acc.w);
}

// Adds every slot's output slice (4 * LPN floats; lane `sub` of a slot holds
// floats 4 sub .. 4 sub + 3) to its C row with float atomics, for the slots
// whose `row` is not negative. The slices pass through the wave's LDS so that
// atomic instruction i has lane L add float 64 i + L of the slot-major slices:
// each instruction covers whole contiguous slices (128 or 256 bytes of a row).
// Atomics whose lanes are 16 bytes apart (each lane adding its own float4
// component by component) touch twice the 64-byte sectors per instruction and
// measured 4x fewer row updates per second on MI355X (2.5 G against 10.3 G
// 128-byte rows/s at random rows).
template <int LPN>
__device__ __forceinline__ void add_rows_atomic(float* C, int N, int col0, int* wave_lds,
                                                const float4& acc, int row) {
  constexpr int W = 4 * LPN;  // floats per slice
  if (!__any(row >= 0)) return;
  const int lane = lane_id();
  float* const t = reinterpret_cast<float*>(wave_lds);
  wave_lds_sync();  // earlier reads of this LDS area come first
  *reinterpret_cast<float4*>(t + 4 * lane) = acc;
  wave_lds_sync();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int F = 64 * i + lane;
    const int r = __shfl(row, (F / W) * LPN);
    if (r >= 0) unsafeAtomicAdd(C + r * N + col0 + F % W, t[F]);
  }
}

// Sums acc over the `spg` slots of each group (spg a power of two <= SL).
template <int LPN>
__device__ __forceinline__ float group_sum(float v, int spg) {
  if constexpr (LPN <= 32) {
    if (spg >= 2) v += xor_shfl<LPN>(v);
  }
  if constexpr (LPN <= 16) {
    if (spg >= 4) v += xor_shfl<2 * LPN>(v);
  }
  if constexpr (LPN <= 8) {
    if (spg >= 8) v += xor_shfl<4 * LPN>(v);
  }
  return v;
}

template <int LPN, bool kBuf>
__global__ __launch_bounds__(kWave* waves_per_block(LPN)) void spmm_kernel(SpmmArgs args) {
  constexpr int kWavesPerBlock = waves_per_block(LPN);
  // the tile of kPer * SL nonzeros and the SL residue groups of a task are
  // spmm_task_shape(N)
  constexpr int SL = 64 / LPN;
  // per wave: the slots' staged pairs, and later the 256 floats of add_rows_atomic
  constexpr int kWaveWords = SL * kSlotWords > 256 ? SL * kSlotWords : 256;
  __shared__ __attribute__((aligned(16))) int lds[kWavesPerBlock][kWaveWords];
  const int wave = threadIdx.x / kWave;
  const uint32_t blk = balanced_block(blockIdx.x, gridDim.x, args.chunk_log2);
  const uint32_t task = __builtin_amdgcn_readfirstlane(blk * kWavesPerBlock + wave);
  if (task >= args.total_tasks) return;
  // slice-major: every task of column slice 0, then slice 1, ...
  const uint32_t per_slice = args.total_tasks / uint32_t(args.slices);
  const int slice = int(task / per_slice);
  uint32_t t = task - uint32_t(slice) * per_slice;
  if (args.task_map) {  // a permutation of [0, per_slice)
    t = __builtin_amdgcn_readfirstlane(args.task_map[t]);
    if (t >= per_slice) return;
  }
  int i = 0;
  while (i + 1 < args.count && t >= args.task_begin[i + 1]) ++i;
  const ps_workset ws = args.ws[i];
  const uint32_t local = t - args.task_begin[i];
  const int N = args.N;
  const int col0 = slice * 4 * LPN;

  const int lane = lane_id();
  const int slot = lane / LPN, sub = lane % LPN;
  using Off = typename Rows<kBuf>::Off;
  const uint32_t row_bytes = uint32_t(N) * 4u;
  const Rows<kBuf> Bq(args.B + col0, args.b_bytes - uint64_t(col0) * 4u);
  const uint32_t my_off = uint32_t(sub) * 16u;
  // LDS holds B-row byte offsets when they fit 32 bits, column ids otherwise
  auto stage_key = [&](int c) -> int { return kBuf ? int(uint32_t(c) * row_bytes) : c; };
  auto row_off = [&](int key) -> Off {
    return kBuf ? Off(uint32_t(key)) + my_off : Off(uint32_t(key)) * row_bytes + my_off;
  };
  int* const my_lds = lds[wave];
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);

  if (ws.group_size > 0) {
    // ---------------------------------------------------------- block tile
    constexpr int T = kPer * SL;
    const int GS = ws.group_size;
    const int spg = GS / kPer < SL ? GS / kPer : SL;  // slots per group
    const long long total = (long long)ws.group_num * GS;
    const long long tile = (long long)local * T;
    // stage: lane l holds nonzeros 4l .. 4l+3 of the tile
    if (lane * 4 < T) {
      const long long p = tile + lane * 4;
      int4 c = make_int4(0, 0, 0, 0);
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (p < total) {
        // read once per launch: non-temporal, so that they displace fewer of
        // the L2's B rows (C3 SpMM N=32 / 128: 1.645 / 5.671 -> 1.625 / 5.602 ms)
        const iv4 ci = __builtin_nontemporal_load(reinterpret_cast<const iv4*>(ws.col_ind + p));
        const fv4 vi = __builtin_nontemporal_load(reinterpret_cast<const fv4*>(ws.sp_data + p));
        c = make_int4(ci.x, ci.y, ci.z, ci.w);
        v = make_float4(vi.x, vi.y, vi.z, vi.w);
      }
      const int k = lane * 4, q = k / kPer, j = k % kPer;
      int4* dst = reinterpret_cast<int4*>(my_lds + q * kSlotWords + 2 * j);
      dst[0] = make_int4(stage_key(c.x), __float_as_int(v.x), stage_key(c.y), __float_as_int(v.y));
      dst[1] = make_int4(stage_key(c.z), __float_as_int(v.z), stage_key(c.w), __float_as_int(v.w));
    }
    wave_lds_sync();
    const long long slot_first = tile + slot * kPer;
    const int4* src = reinterpret_cast<const int4*>(my_lds + slot * kSlotWords);
#pragma unroll 1
    for (int b0 = 0; b0 < kPer; b0 += kBatch) {
      Off off[kBatch];
      float val[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; u += 2) {
        const int4 w = src[(b0 + u) / 2];
        off[u] = row_off(w.x);
        val[u] = __int_as_float(w.y);
        off[u + 1] = row_off(w.z);
        val[u + 1] = __int_as_float(w.w);
      }
      float4 bv[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) bv[u] = Bq.load(off[u]);
      // keep the whole batch of loads in flight before the first use
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < kBatch; ++u) fma4(acc, val[u], bv[u]);
    }
    acc.x = group_sum<LPN>(acc.x, spg);
    acc.y = group_sum<LPN>(acc.y, spg);
    acc.z = group_sum<LPN>(acc.z, spg);
    acc.w = group_sum<LPN>(acc.w, spg);
    // every slot of a group holds its sum; the group's first slot adds it
    const bool leader = slot_first < total && slot % spg == 0;
    // GS is a power of two (checked at launch): a shift, not a 64-bit division
    const int row = leader ? ws.group_des[int(slot_first >> __builtin_ctz(unsigned(GS)))] : -1;
    add_rows_atomic<LPN>(args.C, N, col0, my_lds, acc, row);
  } else {
    // ------------------------------------------------------- residue groups
    // Slot q takes group local * SL + q of the run order (order[] when given,
    // else as stored) and stages its (B-row key, value) pairs in its own LDS
    // area; groups built by the preprocessing hold at most 31 nonzeros, longer
    // ones are read directly.
    const int kq = int(local) * SL + slot;
    int g = kq < ws.group_num ? (ws.order ? ws.order[kq] : kq) : -1;
    const bool has = g >= 0 && g < ws.group_num;  // order entries out of range are skipped
    if (!has) g = 0;
    const int start = has ? args.residue_offset[g] : 0;
    const int len = has ? args.residue_offset[g + 1] - start : 0;
    int* const slot_lds = my_lds + slot * kSlotWords;
    const bool staged = len <= kSlotWords / 2;
    if (staged) {
      for (int k = sub; k < len; k += LPN) {
        const int c = ws.col_ind[start + k];
        const float v = ws.sp_data[start + k];
        *reinterpret_cast<int2*>(slot_lds + 2 * k) = make_int2(stage_key(c), __float_as_int(v));
      }
    }
    wave_lds_sync();
#pragma unroll 1
    for (int j0 = 0; __any(j0 < len); j0 += kRBatch) {
      Off off[kRBatch];
      float val[kRBatch];
#pragma unroll
      for (int u = 0; u < kRBatch; ++u) {
        const int j = j0 + u;
        const int jj = j < len ? j : (len > 0 ? len - 1 : 0);
        int2 w;
        if (staged) {
          w = *reinterpret_cast<const int2*>(slot_lds + 2 * jj);
        } else {
          const int p = start + jj;
          w = make_int2(stage_key(len > 0 ? ws.col_ind[p] : 0),
                        __float_as_int(len > 0 ? ws.sp_data[p] : 0.f));
        }
        off[u] = row_off(len > 0 ? w.x : 0);
        val[u] = j < len ? __int_as_float(w.y) : 0.f;
      }
      float4 bv[kRBatch];
#pragma unroll
      for (int u = 0; u < kRBatch; ++u) bv[u] = Bq.load(off[u]);
      // keep the whole batch of loads in flight before the first use
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < kRBatch; ++u) fma4(acc, val[u], bv[u]);
    }
    int atomic_row = -1;
    if (has && len > 0) {
      const int row = ws.group_des[g];
      if (args.residue_atomic[g])
        atomic_row = row;
      else
        // written once per launch: a non-temporal store keeps the row from
        // displacing B rows in the L2 (C3 SpMM N=32 / 128: 1.594 / 5.674 ->
        // 1.585 / 5.650 ms)
        __builtin_nontemporal_store(fv4{acc.x, acc.y, acc.z, acc.w},
                                    reinterpret_cast<fv4*>(args.C + row * N + col0 + sub * 4));
    }
    add_rows_atomic<LPN>(args.C, N, col0, my_lds, acc, atomic_row);
  }
}

// Lanes per B-row slice. N a multiple of 64 runs as N / 64 slices of 64
// floats (16 lanes), any other N as N / 32 slices of 32 floats (8 lanes),
// slice after slice. Narrow slices gather from a smaller working set (cols x
// 32 floats), wide ones read the matrix fewer times and issue half the
// gathers; at N = 128 the 64-float slices won in the run order and on the
// tuned partition (C3: 7.39 -> 6.98 ms tuned, 7.83 -> 7.22 ms run order; C1:
// 2.05 -> 2.03 and 2.23 -> 2.17 ms; one 128-float slice: 7.25 / 7.19 and
// 2.13 / 2.19 ms), where in the first build's stored order the 32-float
// slices had been faster (C1: 2.96 -> 2.53 ms against 128-float slices).
// With the dense hub block they still win (C3 SpMM N=128: 5.65 ms against
// 5.92 ms in 32-float slices and 5.88 ms in one 128-float slice).
int pick_lpn(int N) { return spmm_lanes_per_row(N); }

template <int LPN>
void launch_lpn(const SpmmArgs& a, bool buf, unsigned grid, hipStream_t stream) {
  const dim3 block(kWave * waves_per_block(LPN));
  if (buf) spmm_kernel<LPN, true><<<grid, block, 0, stream>>>(a);
  else spmm_kernel<LPN, false><<<grid, block, 0, stream>>>(a);
}

int launch(int count, const int* order, const ps_workset* worksets, const int* residue_offset,
           const uint8_t* residue_atomic, int rows, int cols, int N, const float* B, float* C,
           int task_chunk, const uint32_t* task_map, uint32_t task_map_len, hipStream_t stream) {
  PS_CHECK_ARG(N > 0 && N % 32 == 0, "SpMM requires N to be a positive multiple of 32");
  PS_CHECK_ARG(task_chunk_valid(task_chunk),
               "SpMM task_chunk must be PS_TASK_CHUNK_AUTO, 0 or a power of two up to 4096");
  PS_CHECK_ARG(int64_t(rows) * N <= INT32_MAX && int64_t(cols) * N <= INT32_MAX,
               "Dense dimensions exceed the 32-bit kernel indexing range");
  PS_CHECK_ARG(B && C, "Invalid SpMM buffers");
  PS_CHECK_ARG(aligned16(B) && aligned16(C), "SpMM dense buffers must be 16-byte aligned");
  const int lpn = pick_lpn(N);
  const TaskShape shape = spmm_task_shape(N);
  SpmmArgs a{};
  a.N = N;
  a.slices = N / (4 * lpn);
  a.B = B;
  a.C = C;
  a.residue_offset = residue_offset;
  a.residue_atomic = residue_atomic;
  const uint64_t b_bytes = uint64_t(cols) * uint64_t(N) * 4u;
  // Buffer offsets are 32-bit: use them when every byte of B is addressable.
  const bool buf = b_bytes <= 0xFFFFFFFFull;
  a.b_bytes = b_bytes;
  uint64_t tasks = 0;
  int n = 0;
  for (int q = 0; q < count; ++q) {
    const int s = order[q];
    const ps_workset& w = worksets[q];
    if (w.group_num <= 0) continue;
    PS_CHECK_ARG(w.col_ind && w.sp_data && w.group_des, "Invalid SpMM workset buffers");
    uint64_t t;
    if (s > 0) {
      PS_CHECK_ARG(aligned16(w.col_ind) && aligned16(w.sp_data),
                   "Block workset arrays must be 16-byte aligned");
      PS_CHECK_ARG(w.group_size >= 32 && (w.group_size & (w.group_size - 1)) == 0,
                   "Block workset group size must be a power of two >= 32");
      const uint64_t T = uint64_t(shape.tile_nnz);
      t = (uint64_t(w.group_num) * uint64_t(w.group_size) + T - 1) / T;
    } else {
      PS_CHECK_ARG(residue_offset && residue_atomic, "Missing residue offsets or flags");
      t = (uint64_t(w.group_num) + shape.residue_groups - 1) / shape.residue_groups;
    }
    a.ws[n] = w;
    if (s == 0) a.ws[n].group_size = 0;
    a.task_begin[n] = uint32_t(tasks);
    tasks += t;
    ++n;
  }
  if (n == 0) return PS_OK;
  a.count = n;
  a.task_begin[n] = uint32_t(tasks);
  if (task_map) {
    PS_CHECK_ARG(task_map_len == tasks,
                 "SpMM task order holds " + std::to_string(task_map_len) + " tasks, the launch " +
                     std::to_string(tasks));
    a.task_map = task_map;
  }
  tasks *= uint64_t(a.slices);
  PS_CHECK_ARG(tasks < (1ull << 31), "SpMM task count exceeds the launch range");
  a.total_tasks = uint32_t(tasks);
  const unsigned wpb = unsigned(waves_per_block(lpn));
  const unsigned grid = unsigned((tasks + wpb - 1) / wpb);
  a.chunk_log2 = uint32_t(task_chunk_log2(task_chunk, grid, kAutoChunkMax));
  switch (lpn) {
    case 8: launch_lpn<8>(a, buf, grid, stream); break;
    case 16: launch_lpn<16>(a, buf, grid, stream); break;
    case 32: launch_lpn<32>(a, buf, grid, stream); break;
    default: launch_lpn<64>(a, buf, grid, stream); break;
  }
  PS_LAUNCHED();
  return PS_OK;
}

}  // namespace
}  // namespace ps

extern "C" {

int ps_spmm_launch(int workset_count, const ps_workset* worksets, const int* residue_offset,
                   const uint8_t* residue_atomic, int rows, int cols, int N, const float* B,
                   float* C, int task_chunk, ps_stream_t stream) {
  PS_CHECK_ARG(workset_count >= 1 && workset_count <= PS_MAX_WORKSETS && worksets,
               "Invalid SpMM workset count");
  // Largest groups first, as the reference submits s = S-1 .. 0
  // (spmm_solution.cu:16).
  int order[PS_MAX_WORKSETS];
  ps_workset ordered[PS_MAX_WORKSETS];
  for (int q = 0; q < workset_count; ++q) {
    order[q] = workset_count - 1 - q;
    ordered[q] = worksets[workset_count - 1 - q];
  }
  return ps::launch(workset_count, order, ordered, residue_offset, residue_atomic, rows, cols,
                    N, B, C, task_chunk, nullptr, 0, ps::to_hip(stream));
}

int ps_spmm_launch_ordered(int workset_count, const ps_workset* worksets,
                           const int* residue_offset, const uint8_t* residue_atomic, int rows,
                           int cols, int N, const float* B, float* C, int task_chunk,
                           const uint32_t* task_order, uint32_t task_count, ps_stream_t stream) {
  PS_CHECK_ARG(workset_count >= 1 && workset_count <= PS_MAX_WORKSETS && worksets,
               "Invalid SpMM workset count");
  int order[PS_MAX_WORKSETS];
  ps_workset ordered[PS_MAX_WORKSETS];
  for (int q = 0; q < workset_count; ++q) {
    order[q] = workset_count - 1 - q;
    ordered[q] = worksets[workset_count - 1 - q];
  }
  return ps::launch(workset_count, order, ordered, residue_offset, residue_atomic, rows, cols,
                    N, B, C, task_chunk, task_order, task_count, ps::to_hip(stream));
}

int ps_spmm_workset_launch(int s, const ps_workset* workset, const int* residue_offset,
                           const uint8_t* residue_atomic, int rows, int cols, int N,
                           const float* B, float* C, ps_stream_t stream) {
  PS_CHECK_ARG(s >= 0 && s < PS_MAX_WORKSETS && workset, "Invalid SpMM workset");
  return ps::launch(1, &s, workset, residue_offset, residue_atomic, rows, cols, N, B, C, 1,
                    nullptr, 0, ps::to_hip(stream));
}

}  // extern "C"
