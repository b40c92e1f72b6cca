// The calibration copy of the measurement tooling (python -m powersparse_amd.perf):
// a plain streaming copy of `count` floats with 128-bit loads and stores (a
// kernel, never a DMA engine), which reads and writes exactly its size, so the
// rocprofv3 FETCH_SIZE / WRITE_SIZE counters can be scaled by it. Built into
// lib/libpowersparse_perf.so; not part of the product ABI and not called by
// the operators or the preprocessing. No reference counterpart.
#include "ps_common.hpp"

namespace ps {
namespace {

__global__ void copy_f32_kernel(float4* __restrict__ dst, const float4* __restrict__ src,
                                size_t n4) {
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n4; i += stride)
    dst[i] = src[i];
}

__global__ void copy_tail_kernel(float* __restrict__ dst, const float* __restrict__ src,
                                 size_t begin, size_t count) {
  const size_t i = begin + size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < count) dst[i] = src[i];
}

}  // namespace
}  // namespace ps

extern "C" int ps_perf_copy_f32_async(float* dst, const float* src, size_t count,
                                      ps_stream_t stream) {
  if (count == 0) return PS_OK;
  PS_CHECK_ARG(dst && src, "ps_perf_copy_f32_async: null pointer");
  PS_CHECK_ARG((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) % 16 == 0,
               "ps_perf_copy_f32_async: buffers must be 16-byte aligned");
  hipStream_t st = ps::to_hip(stream);
  const size_t n4 = count / 4;
  if (n4) {
    // 128 workgroups of 256 per CU, grid-stride
    const size_t blocks = (n4 + 255) / 256;
    ps::copy_f32_kernel<<<unsigned(blocks < 32768 ? blocks : 32768), 256, 0, st>>>(
        reinterpret_cast<float4*>(dst), reinterpret_cast<const float4*>(src), n4);
    PS_LAUNCHED();
  }
  if (count % 4) {
    ps::copy_tail_kernel<<<1, 4, 0, st>>>(dst, src, n4 * 4, count);
    PS_LAUNCHED();
  }
  return PS_OK;
}
