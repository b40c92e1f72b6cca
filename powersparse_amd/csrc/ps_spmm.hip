// SpMM (node aggregation), C += A * B, FP32, on gfx950.
//
// One launch covers every workset of a PowerSparse matrix. The grid is a flat
// list of wave tasks; each wave64 decodes its task from a small table in the
// kernel arguments:
//   block workset s (groups of GS = 32 * 2^(s-1) nonzeros): a task is a tile of
//     T = min(GS, 256) consecutive nonzeros of one group and one N-slice;
//   residue workset: a task is one residue group and one N-slice.
// Inside a wave the 64 lanes form SL = 64 / LPN slots of LPN lanes; a slot
// reads one B row slice of 4 * LPN floats with 128-bit loads, so one wave
// instruction gathers SL rows. Each slot walks its own run of nonzeros, then
// the slots are summed with DPP / swizzle butterflies and the row result is
// added atomically (or stored, for residue groups whose row has no other group).
//
// Reference behaviour kept (PowerSparse_SpMM/spmm_solution.cu:7-34,
// spmm_kernel_block.cu:60-162, spmm_kernel_residue.cu:5-82): block groups and
// flagged residue groups accumulate into C with atomics, unflagged residue
// groups overwrite their row, C is not cleared by the operator.
#include "ps_common.hpp"

namespace ps {
namespace {

constexpr int kWavesPerBlock = 4;
constexpr int kBlockTile = 256;  // nonzeros per block-workset wave task (max)

struct SpmmArgs {
  ps_workset ws[PS_MAX_WORKSETS];
  uint32_t task_begin[PS_MAX_WORKSETS + 1];
  int32_t tiles_per_group[PS_MAX_WORKSETS];
  int32_t count;
  int32_t N;
  int32_t slices;
  uint32_t total_tasks;
  const int* residue_offset;
  const uint8_t* residue_atomic;
  const float* B;
  float* C;
};

__device__ __forceinline__ void fma4(float4& acc, float a, const float4& b) {
  acc.x = fmaf(a, b.x, acc.x);
  acc.y = fmaf(a, b.y, acc.y);
  acc.z = fmaf(a, b.z, acc.z);
  acc.w = fmaf(a, b.w, acc.w);
}

template <int LPN>
__device__ __forceinline__ float slot_sum(float v) {
  if constexpr (LPN <= 8) v += xor_shfl<8>(v);
  if constexpr (LPN <= 16) v += xor_shfl<16>(v);
  if constexpr (LPN <= 32) v += xor_shfl<32>(v);
  return v;
}

// Adds (atomic) or stores the slot-reduced float4 of every lane into row `row`.
template <int LPN>
__device__ __forceinline__ void write_row(float* C, int row, int N, int col0, float4 acc,
                                          bool atomic) {
  constexpr int SL = 64 / LPN;
  const int lane = lane_id();
  const int slot = lane / LPN, sub = lane % LPN;
  acc.x = slot_sum<LPN>(acc.x);
  acc.y = slot_sum<LPN>(acc.y);
  acc.z = slot_sum<LPN>(acc.z);
  acc.w = slot_sum<LPN>(acc.w);
  float* out = C + row * N + col0 + sub * 4;
  if (atomic) {
    const float v[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (c % SL == slot) unsafeAtomicAdd(out + c, v[c]);
  } else if (slot == 0) {
    *reinterpret_cast<float4*>(out) = acc;
  }
}

template <int LPN>
__global__ __launch_bounds__(kWave* kWavesPerBlock) void spmm_kernel(SpmmArgs args) {
  constexpr int SL = 64 / LPN;
  const uint32_t blk = xcd_remap(blockIdx.x, gridDim.x);
  const uint32_t task =
      __builtin_amdgcn_readfirstlane(blk * kWavesPerBlock + threadIdx.x / kWave);
  if (task >= args.total_tasks) return;
  int i = 0;
  while (i + 1 < args.count && task >= args.task_begin[i + 1]) ++i;
  const ps_workset ws = args.ws[i];
  uint32_t local = task - args.task_begin[i];
  const int N = args.N;
  const int slice = int(local % uint32_t(args.slices));
  local /= uint32_t(args.slices);
  const int col0 = slice * 4 * LPN;

  const int lane = lane_id();
  const int slot = lane / LPN, sub = lane % LPN;
  const float4* __restrict__ B4 = reinterpret_cast<const float4*>(args.B + col0) + sub;
  const int n4 = N / 4;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);

  if (ws.group_size > 0) {
    // Block workset: tile `t` of group `g`, every slot owns per = T / SL
    // consecutive nonzeros (a multiple of 4, so 128-bit index loads).
    const int tiles = args.tiles_per_group[i];
    const int g = int(local / uint32_t(tiles));
    const int t = int(local % uint32_t(tiles));
    const int T = ws.group_size / tiles;
    const int per = T / SL;
    const int begin = g * ws.group_size + t * T + slot * per;
    const int* cp = ws.col_ind + begin;
    const float* vp = ws.sp_data + begin;
    int j = 0;
    for (; j + 8 <= per; j += 8) {
      const int4 c0 = *reinterpret_cast<const int4*>(cp + j);
      const int4 c1 = *reinterpret_cast<const int4*>(cp + j + 4);
      const float4 v0 = *reinterpret_cast<const float4*>(vp + j);
      const float4 v1 = *reinterpret_cast<const float4*>(vp + j + 4);
      const float4 b0 = B4[c0.x * n4], b1 = B4[c0.y * n4], b2 = B4[c0.z * n4],
                   b3 = B4[c0.w * n4], b4 = B4[c1.x * n4], b5 = B4[c1.y * n4],
                   b6 = B4[c1.z * n4], b7 = B4[c1.w * n4];
      fma4(acc, v0.x, b0);
      fma4(acc, v0.y, b1);
      fma4(acc, v0.z, b2);
      fma4(acc, v0.w, b3);
      fma4(acc, v1.x, b4);
      fma4(acc, v1.y, b5);
      fma4(acc, v1.z, b6);
      fma4(acc, v1.w, b7);
    }
    if (j < per) {  // per == 4
      const int4 c0 = *reinterpret_cast<const int4*>(cp + j);
      const float4 v0 = *reinterpret_cast<const float4*>(vp + j);
      const float4 b0 = B4[c0.x * n4], b1 = B4[c0.y * n4], b2 = B4[c0.z * n4],
                   b3 = B4[c0.w * n4];
      fma4(acc, v0.x, b0);
      fma4(acc, v0.y, b1);
      fma4(acc, v0.z, b2);
      fma4(acc, v0.w, b3);
    }
    write_row<LPN>(args.C, ws.group_des[g], N, col0, acc, true);
  } else {
    // Residue workset: one group per wave, nonzero k goes to slot k % SL.
    const int g = int(local);
    const int beg = args.residue_offset[g];
    const int len = args.residue_offset[g + 1] - beg;
    const int* cp = ws.col_ind + beg;
    const float* vp = ws.sp_data + beg;
    for (int k0 = 0; k0 < len; k0 += 4 * SL) {
      int c[4];
      float v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int k = k0 + u * SL + slot;
        const bool ok = k < len;
        c[u] = ok ? cp[k] : 0;
        v[u] = ok ? vp[k] : 0.f;
      }
      float4 b[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) b[u] = B4[c[u] * n4];
#pragma unroll
      for (int u = 0; u < 4; ++u) fma4(acc, v[u], b[u]);
    }
    write_row<LPN>(args.C, ws.group_des[g], N, col0, acc, args.residue_atomic[g] != 0);
  }
}

// Lanes per B row slice: the widest of 64/32/16/8 lanes (256/128/64/32 floats)
// that divides N.
int pick_lpn(int N) {
  if (N % 256 == 0) return 64;
  if (N % 128 == 0) return 32;
  if (N % 64 == 0) return 16;
  return 8;
}

int launch(int count, const int* order, const ps_workset* worksets, const int* residue_offset,
           const uint8_t* residue_atomic, int rows, int cols, int N, const float* B, float* C,
           hipStream_t stream) {
  PS_CHECK_ARG(N > 0 && N % 32 == 0,
               "SpMM requires N to be a positive multiple of 32");
  PS_CHECK_ARG(int64_t(rows) * N <= INT32_MAX && int64_t(cols) * N <= INT32_MAX,
               "Dense dimensions exceed the 32-bit kernel indexing range");
  PS_CHECK_ARG(B && C, "Invalid SpMM buffers");
  const int lpn = pick_lpn(N);
  SpmmArgs a{};
  a.N = N;
  a.slices = N / (4 * lpn);
  a.B = B;
  a.C = C;
  a.residue_offset = residue_offset;
  a.residue_atomic = residue_atomic;
  uint64_t tasks = 0;
  int n = 0;
  for (int q = 0; q < count; ++q) {
    const int s = order[q];
    const ps_workset& w = worksets[q];
    if (w.group_num <= 0) continue;
    PS_CHECK_ARG(w.col_ind && w.sp_data && w.group_des, "Invalid SpMM workset buffers");
    int tiles = 1;
    if (s > 0) {
      PS_CHECK_ARG(w.group_size >= 32 && (w.group_size & (w.group_size - 1)) == 0,
                   "Block workset group size must be a power of two >= 32");
      tiles = w.group_size > kBlockTile ? w.group_size / kBlockTile : 1;
    } else {
      PS_CHECK_ARG(residue_offset && residue_atomic, "Missing residue offsets or flags");
    }
    a.ws[n] = w;
    if (s == 0) a.ws[n].group_size = 0;
    a.tiles_per_group[n] = tiles;
    a.task_begin[n] = uint32_t(tasks);
    tasks += uint64_t(w.group_num) * tiles * a.slices;
    ++n;
  }
  if (n == 0) return PS_OK;
  PS_CHECK_ARG(tasks < (1ull << 31), "SpMM task count exceeds the launch range");
  a.count = n;
  a.task_begin[n] = uint32_t(tasks);
  a.total_tasks = uint32_t(tasks);
  const unsigned grid = unsigned((tasks + kWavesPerBlock - 1) / kWavesPerBlock);
  const dim3 block(kWave * kWavesPerBlock);
  switch (lpn) {
    case 8: spmm_kernel<8><<<grid, block, 0, stream>>>(a); break;
    case 16: spmm_kernel<16><<<grid, block, 0, stream>>>(a); break;
    case 32: spmm_kernel<32><<<grid, block, 0, stream>>>(a); break;
    default: spmm_kernel<64><<<grid, block, 0, stream>>>(a); break;
  }
  PS_LAUNCHED();
  return PS_OK;
}

}  // namespace
}  // namespace ps

extern "C" {

int ps_spmm_launch(int workset_count, const ps_workset* worksets, const int* residue_offset,
                   const uint8_t* residue_atomic, int rows, int cols, int N, const float* B,
                   float* C, ps_stream_t stream) {
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
                    N, B, C, ps::to_hip(stream));
}

int ps_spmm_workset_launch(int s, const ps_workset* workset, const int* residue_offset,
                           const uint8_t* residue_atomic, int rows, int cols, int N,
                           const float* B, float* C, ps_stream_t stream) {
  PS_CHECK_ARG(s >= 0 && s < PS_MAX_WORKSETS && workset, "Invalid SpMM workset");
  return ps::launch(1, &s, workset, residue_offset, residue_atomic, rows, cols, N, B, C,
                    ps::to_hip(stream));
}

}  // extern "C"
