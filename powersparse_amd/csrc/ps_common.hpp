// Shared definitions for the gfx950 kernels and the C ABI glue.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

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

__device__ __forceinline__ int lane_id() { return __lane_id(); }

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

// Map a workgroup index to a logical index such that consecutive logical
// indices stay on one XCD: the hardware deals workgroups round-robin over the 8
// XCDs, and each XCD has its own L2, so neighbouring work (which shares B/Y rows
// after the signature ordering) should land on the same XCD.
__device__ __forceinline__ uint32_t xcd_remap(uint32_t block, uint32_t nblocks) {
  constexpr uint32_t kXcd = 8;
  const uint32_t q = nblocks / kXcd, r = nblocks % kXcd;
  const uint32_t xcd = block % kXcd, idx = block / kXcd;
  const uint32_t base = xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q;
  return base + idx;
}

}  // namespace ps
