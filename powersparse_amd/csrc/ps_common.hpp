// Shared definitions for the gfx950 kernels and the C ABI glue.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>
#include <type_traits>

#include "powersparse_hip.h"

namespace ps {

// Thread-local last-error text behind ps_last_error().
void set_error(const std::string& msg);
void clear_error();

inline int fail(int code, const std::string& msg) {
  set_error(msg);
  return code;
}

inline hipStream_t to_hip(ps_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Device temporaries of the entry points go through ps_malloc / ps_free, so
// they get the allocation guards (PS_DEVICE_GUARD) like every other block.
template <typename T>
inline hipError_t dev_malloc(T** p, size_t bytes) {
  return ps_malloc(reinterpret_cast<void**>(p), bytes) == PS_OK ? hipSuccess
                                                                : hipErrorOutOfMemory;
}
inline void dev_free(void* p) { (void)ps_free(p); }

// The kernels move dense rows and staged nonzeros with 128-bit accesses.
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace ps

// Returns PS_ERR_RUNTIME with "file:line: call: hip error text" on failure, the
// same shape as the reference's CUDA_CALL message (utils/cuda_utils.h:7-14).
#define PS_HIP(call)                                                                   \
  do {                                                                                 \
    hipError_t ps_status_ = (call);                                                    \
    if (ps_status_ != hipSuccess)                                                      \
      return ps::fail(PS_ERR_RUNTIME, std::string(__FILE__) + ":" +                    \
                                          std::to_string(__LINE__) + ": " #call ": " + \
                                          hipGetErrorString(ps_status_));              \
  } while (0)

#define PS_CHECK_ARG(cond, msg)                        \
  do {                                                 \
    if (!(cond)) return ps::fail(PS_ERR_INVALID, msg); \
  } while (0)

// Checks the launch that was just enqueued.
#define PS_LAUNCHED() PS_HIP(hipGetLastError())

namespace ps {

constexpr int kWave = 64;

// Clang vector types for __builtin_nontemporal_load of 16-byte elements.
typedef int iv4 __attribute__((ext_vector_type(4)));
typedef float fv4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Makes one wave's LDS writes visible to its own later LDS reads.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Cross-lane float moves inside a wave64. Masks 1 and 2 use DPP quad permutes,
// 8 uses a DPP row rotate (xor 8 inside each 16-lane row), 4 and 16 use
// ds_swizzle in bit mode (xor inside 32-lane halves), 32 uses ds_bpermute.
template <int M>
__device__ __forceinline__ float xor_shfl(float v) {
  const int x = __float_as_int(v);
  int r;
  if constexpr (M == 1) {
    r = __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false);
  } else if constexpr (M == 2) {
    r = __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false);
  } else if constexpr (M == 4) {
    r = __builtin_amdgcn_ds_swizzle(x, (4 << 10) | 0x1F);
  } else if constexpr (M == 8) {
    r = __builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false);
  } else if constexpr (M == 16) {
    r = __builtin_amdgcn_ds_swizzle(x, (16 << 10) | 0x1F);
  } else {
    static_assert(M == 32, "xor_shfl supports 1, 2, 4, 8, 16, 32");
    r = __builtin_amdgcn_ds_bpermute((lane_id() ^ 32) << 2, x);
  }
  return __int_as_float(r);
}

// Workgroup -> logical index. The hardware deals a launch's workgroups
// round-robin over the 8 XCDs, each with its own L2: workgroup b runs on XCD
// (x0 + b) mod 8, x0 being where the previous dispatch's dealing stopped, so
// workgroups b and b' share an XCD exactly when b = b' mod 8. With chunk = 2^chunk_log2 > 1, windows of
// 8 * chunk consecutive workgroups are re-dealt so that each XCD takes chunk
// consecutive logical indices: neighbouring tasks run under one L2, while every
// XCD still gets a slice of every window, which keeps the XCDs balanced when
// task costs vary along the list. The last, partial window keeps the hardware
// order; chunk_log2 == 0 keeps it everywhere.
constexpr uint32_t kXcd = 8;
__device__ __forceinline__ uint32_t balanced_block(uint32_t b, uint32_t n, uint32_t chunk_log2) {
  if (chunk_log2 == 0) return b;
  const uint32_t chunk = 1u << chunk_log2;
  const uint32_t win = kXcd * chunk;
  const uint32_t w = b / win;
  if ((w + 1) * win > n) return b;
  return w * win + (b % kXcd) * chunk + (b / kXcd) % chunk;
}

// Task geometry of the fused operator launches, shared by the kernels, their
// launchers and the run-order builder. A launch's tasks are numbered in launch
// order: the worksets from the largest group size down to the residue (empty
// worksets skipped); a block workset of G groups of GS nonzeros gives
// ceil(G * GS / tile_nnz) tile tasks, the residue workset ceil(G0 /
// residue_groups) tasks of consecutive groups.
struct TaskShape {
  int tile_nnz;
  int residue_groups;
};
// SpMM: lanes per B-row slice (16 when N is a multiple of 64: slices of 64
// floats; else 8: slices of 32), slots of lanes per wave, 32 nonzeros per slot
// per tile, one residue group per slot.
inline int spmm_lanes_per_row(int N) { return N % 64 == 0 ? 16 : 8; }
inline TaskShape spmm_task_shape(int N) {
  const int slots = kWave / spmm_lanes_per_row(N);
  return {32 * slots, slots};
}
// SDDMM: 8 slots of 8 lanes, 8 nonzeros per slot per tile, one residue group per slot.
inline TaskShape sddmm_task_shape() { return {64, 8}; }

// Whether task_chunk is one a launcher accepts: PS_TASK_CHUNK_AUTO, 0, or a
// power of two up to 4096.
inline bool task_chunk_valid(int task_chunk) {
  return task_chunk == PS_TASK_CHUNK_AUTO || task_chunk == 0 ||
         (task_chunk > 0 && task_chunk <= 4096 && (task_chunk & (task_chunk - 1)) == 0);
}
// log2 of the run length for a launch of `grid` workgroups. AUTO: the largest
// power of two up to `auto_max` that leaves at least 128 runs in the launch,
// i.e. 16 windows of 8 runs (the last, partial window keeps the hardware's
// order, and within a window the XCDs take runs of unequal cost).
inline int task_chunk_log2(int task_chunk, uint64_t grid, int auto_max) {
  if (task_chunk == PS_TASK_CHUNK_AUTO) {
    int l = 0;
    while ((2 << l) <= auto_max && (uint64_t(2) << l) * 128 <= grid) ++l;
    return l;
  }
  int l = 0;
  while (task_chunk > (1 << l)) ++l;
  return l;
}

// cache-policy operand of the buffer loads: the non-temporal (slc) bit
constexpr int kNonTemporal = 2;
// 128-bit loads at byte offsets from a base: through a buffer resource with
// 32-bit offsets when the whole array fits 4 GiB (Off = uint32_t), plain
// global loads with 64-bit offsets otherwise (Off = uint64_t).
template <bool kBuf>
struct Rows {
  using Off = typename std::conditional<kBuf, uint32_t, uint64_t>::type;
  __amdgpu_buffer_rsrc_t rsrc;
  const char* base;
  __device__ Rows(const float* m, uint64_t bytes) : base(reinterpret_cast<const char*>(m)) {
    if constexpr (kBuf)
      rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(m), (short)0, int(bytes),
                                               0x00020000);
  }
  // the same load with the non-temporal hint: for rows read once, so that
  // they displace fewer of the L2's reused lines
  __device__ __forceinline__ float4 load_nt(Off off) const {
    if constexpr (kBuf)
      return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, kNonTemporal));
    else
      return __builtin_bit_cast(float4, __builtin_nontemporal_load(reinterpret_cast<const fv4*>(base + off)));
  }
  __device__ __forceinline__ float4 load(Off off) const {
    if constexpr (kBuf)
      return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0));
    else
      return *reinterpret_cast<const float4*>(base + off);
  }
};

}  // namespace ps
