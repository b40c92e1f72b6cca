// Device, memory, stream and event entry points of the C ABI, plus the
// counter-based random fill used for synthetic dense operands.
#include <cstring>
#include <string>

#include "ps_common.hpp"

namespace ps {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

namespace {

// splitmix64 finaliser: a bijective 64-bit mix (Steele, Lea, Flood 2014).
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ float unit_float(uint64_t bits) {
  // 24 high bits -> [0, 1)
  return float(uint32_t(bits >> 40)) * (1.0f / 16777216.0f);
}

__global__ void fill_random_kernel(float* __restrict__ dst, size_t count, uint64_t seed,
                                   float lo, float hi, int normal) {
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride) {
    const uint64_t h = mix64(seed * 0x9E3779B97F4A7C15ull + i);
    if (!normal) {
      dst[i] = lo + (hi - lo) * unit_float(h);
    } else {
      // Box-Muller on two 24-bit uniforms; u1 is kept away from zero.
      const float u1 = (float(uint32_t(h >> 40)) + 0.5f) * (1.0f / 16777216.0f);
      const float u2 = float(uint32_t(h & 0xFFFFFF)) * (1.0f / 16777216.0f);
      const float r = sqrtf(-2.0f * logf(u1));
      dst[i] = lo + hi * r * cosf(6.28318530717958647692f * u2);
    }
  }
}

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

template <int LPN>
__global__ __launch_bounds__(256) void probe_gather_kernel(const float* table, uint32_t rows,
                                                           uint64_t n, uint64_t seed,
                                                           float* out) {
  constexpr int SL = 64 / LPN;
  const int lane = threadIdx.x & 63, slot = lane / LPN, sub = lane % LPN;
  const uint64_t wave = (uint64_t(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  const uint64_t waves = (uint64_t(gridDim.x) * blockDim.x) >> 6;
  const Rows<true> t(table, uint64_t(rows) * LPN * 16);
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (uint64_t base = wave * 16 * SL; base < n; base += waves * 16 * SL) {
    float4 v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const uint64_t k = base + u * SL + slot;
      // 32-bit mix (two xorshift-multiply rounds), range-reduced by a
      // multiply-high, so index arithmetic stays off the critical path
      uint32_t h = uint32_t(k) ^ uint32_t(seed);
      h = (h ^ (h >> 16)) * 0x7feb352du;
      h = (h ^ (h >> 15)) * 0x846ca68bu;
      h ^= h >> 16;
      const uint32_t r = k < n ? uint32_t((uint64_t(h) * rows) >> 32) : 0u;
      v[u] = t.load(r * uint32_t(LPN * 16) + uint32_t(sub) * 16u);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      acc.x += v[u].x;
      acc.y += v[u].y;
      acc.z += v[u].z;
      acc.w += v[u].w;
    }
  }
  const float s = acc.x + acc.y + acc.z + acc.w;
  if (s == -1.2345e-37f) out[0] = s;  // keeps the loads alive; never true for the fills used
}

// 32-bit index mix used by the probes (two xorshift-multiply rounds).
__device__ __forceinline__ uint32_t mix32(uint32_t h) {
  h = (h ^ (h >> 16)) * 0x7feb352du;
  h = (h ^ (h >> 15)) * 0x846ca68bu;
  return h ^ (h >> 16);
}

// n updates of 128-byte rows of C (rows x 32 floats) at uniformly random rows;
// a wave handles 8 rows per step. Modes: 0 plain float4 stores (8 lanes per
// row); 1 float atomics, each of 8 lanes adding its float4 component by
// component (per instruction the lanes of a row are 16 bytes apart); 2 float
// atomics, 8 lanes adding 8 consecutive floats per instruction; 3 float
// atomics, 32 lanes adding a whole row per instruction.
template <int MODE>
__global__ __launch_bounds__(256) void probe_row_update_kernel(float* __restrict__ C,
                                                               uint32_t rows, uint64_t n,
                                                               uint32_t seed) {
  const int lane = threadIdx.x & 63;
  const uint64_t wave = (uint64_t(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  const uint64_t waves = (uint64_t(gridDim.x) * blockDim.x) >> 6;
  auto row_of = [&](uint64_t k) {
    return size_t((uint64_t(mix32(uint32_t(k) ^ seed)) * rows) >> 32) * 32u;
  };
  for (uint64_t base = wave * 8; base < n; base += waves * 8) {
    if constexpr (MODE == 3) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint64_t k = base + 2 * i + lane / 32;
        if (k < n) unsafeAtomicAdd(C + row_of(k) + lane % 32, 1.0f);
      }
    } else {
      const int slot = lane / 8, sub = lane % 8;
      const uint64_t k = base + slot;
      if (k >= n) continue;
      float* const row = C + row_of(k);
      if constexpr (MODE == 0) {
        *reinterpret_cast<float4*>(row + 4 * sub) = make_float4(1.f, 2.f, 3.f, 4.f);
      } else if constexpr (MODE == 1) {
#pragma unroll
        for (int c = 0; c < 4; ++c) unsafeAtomicAdd(row + 4 * sub + c, 1.0f);
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) unsafeAtomicAdd(row + 8 * c + sub, 1.0f);
      }
    }
  }
}

// Writes the XCC (XCD) id of every workgroup: hardware register XCC_ID
// (s_getreg_b32, bits 3:0), read by the workgroup's first lane.
__global__ void probe_xcc_kernel(int* __restrict__ out, int n) {
  if (threadIdx.x == 0 && int(blockIdx.x) < n)
    out[blockIdx.x] = int(__builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 0xF);
}

}  // namespace
}  // namespace ps

extern "C" {

int ps_probe_xcc_ids_async(int* out, int workgroups, ps_stream_t stream) {
  PS_CHECK_ARG(out && workgroups > 0, "ps_probe_xcc_ids_async: bad argument");
  ps::probe_xcc_kernel<<<unsigned(workgroups), 64, 0, ps::to_hip(stream)>>>(out, workgroups);
  PS_LAUNCHED();
  return PS_OK;
}

int ps_probe_row_update_async(float* C, int rows, long long n, int mode, uint64_t seed,
                              ps_stream_t stream) {
  PS_CHECK_ARG(C && rows > 0 && n >= 0 && mode >= 0 && mode <= 3,
               "ps_probe_row_update_async: bad argument");
  PS_CHECK_ARG(ps::aligned16(C), "ps_probe_row_update_async: C must be 16-byte aligned");
  const unsigned grid = 256 * 16;
  hipStream_t st = ps::to_hip(stream);
  const uint32_t r = uint32_t(rows), s = uint32_t(seed);
  switch (mode) {
    case 0: ps::probe_row_update_kernel<0><<<grid, 256, 0, st>>>(C, r, uint64_t(n), s); break;
    case 1: ps::probe_row_update_kernel<1><<<grid, 256, 0, st>>>(C, r, uint64_t(n), s); break;
    case 2: ps::probe_row_update_kernel<2><<<grid, 256, 0, st>>>(C, r, uint64_t(n), s); break;
    default: ps::probe_row_update_kernel<3><<<grid, 256, 0, st>>>(C, r, uint64_t(n), s); break;
  }
  PS_LAUNCHED();
  return PS_OK;
}

int ps_probe_gather_async(const float* table, int rows, int row_floats, long long n,
                          uint64_t seed, float* out, ps_stream_t stream) {
  PS_CHECK_ARG(table && out && rows > 0 && n >= 0 && (row_floats == 32 || row_floats == 128),
               "ps_probe_gather_async: bad argument");
  PS_CHECK_ARG(uint64_t(rows) * uint64_t(row_floats) * 4u <= 0xFFFFFFFFull,
               "ps_probe_gather_async: table must fit 4 GiB");
  const unsigned grid = 256 * 16;
  if (row_floats == 32)
    ps::probe_gather_kernel<8><<<grid, 256, 0, ps::to_hip(stream)>>>(table, uint32_t(rows),
                                                                      uint64_t(n), seed, out);
  else
    ps::probe_gather_kernel<32><<<grid, 256, 0, ps::to_hip(stream)>>>(table, uint32_t(rows),
                                                                       uint64_t(n), seed, out);
  PS_LAUNCHED();
  return PS_OK;
}

int ps_copy_f32_async(float* dst, const float* src, size_t count, ps_stream_t stream) {
  if (count == 0) return PS_OK;
  PS_CHECK_ARG(dst && src, "ps_copy_f32_async: null pointer");
  PS_CHECK_ARG((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) % 16 == 0,
               "ps_copy_f32_async: buffers must be 16-byte aligned");
  hipStream_t st = ps::to_hip(stream);
  const size_t n4 = count / 4;
  if (n4) {
    // 128 workgroups of 256 per CU, grid-stride: 1 GiB copies at 4.9-5.2 TB/s
    // on MI355X (hipMemcpy device to device: 5.3; 32 per CU: 4.7)
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


const char* ps_last_error(void) { return ps::g_last_error.c_str(); }

int ps_set_device(int device) {
  PS_HIP(hipSetDevice(device));
  PS_HIP(hipFree(nullptr));  // create the context before any timing
  return PS_OK;
}

int ps_get_device(int* device) {
  PS_CHECK_ARG(device, "ps_get_device: null output");
  PS_HIP(hipGetDevice(device));
  return PS_OK;
}

int ps_device_count(int* count) {
  PS_CHECK_ARG(count, "ps_device_count: null output");
  PS_HIP(hipGetDeviceCount(count));
  return PS_OK;
}

int ps_get_device_props(int device, ps_device_props* props) {
  PS_CHECK_ARG(props, "ps_get_device_props: null output");
  hipDeviceProp_t p{};
  PS_HIP(hipGetDeviceProperties(&p, device));
  std::memset(props, 0, sizeof(*props));
  std::strncpy(props->name, p.name, sizeof(props->name) - 1);
  std::strncpy(props->arch, p.gcnArchName, sizeof(props->arch) - 1);
  props->cu_count = p.multiProcessorCount;
  props->major = p.major;
  props->minor = p.minor;
  props->lds_per_block = int(p.sharedMemPerBlock);
  props->l2_bytes = p.l2CacheSize;
  props->clock_khz = p.clockRate;
  props->mem_clock_khz = p.memoryClockRate;
  props->mem_bus_width = p.memoryBusWidth;
  props->global_mem = p.totalGlobalMem;
  return PS_OK;
}

int ps_runtime_version(int* version) {
  PS_CHECK_ARG(version, "ps_runtime_version: null output");
  PS_HIP(hipRuntimeGetVersion(version));
  return PS_OK;
}

int ps_driver_version(int* version) {
  PS_CHECK_ARG(version, "ps_driver_version: null output");
  PS_HIP(hipDriverGetVersion(version));
  return PS_OK;
}

int ps_device_synchronize(void) {
  PS_HIP(hipDeviceSynchronize());
  return PS_OK;
}

int ps_malloc(void** ptr, size_t bytes) {
  PS_CHECK_ARG(ptr, "ps_malloc: null output");
  *ptr = nullptr;
  if (bytes == 0) return PS_OK;
  PS_HIP(hipMalloc(ptr, bytes));
  return PS_OK;
}

int ps_free(void* ptr) {
  if (ptr) PS_HIP(hipFree(ptr));
  return PS_OK;
}

int ps_mem_get_info(size_t* free_bytes, size_t* total_bytes) {
  PS_CHECK_ARG(free_bytes && total_bytes, "ps_mem_get_info: null output");
  PS_HIP(hipMemGetInfo(free_bytes, total_bytes));
  return PS_OK;
}

int ps_memcpy_htod(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return PS_OK;
  PS_CHECK_ARG(dst && src, "ps_memcpy_htod: null pointer");
  PS_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  return PS_OK;
}

int ps_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return PS_OK;
  PS_CHECK_ARG(dst && src, "ps_memcpy_dtoh: null pointer");
  PS_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  return PS_OK;
}

int ps_host_malloc(void** ptr, size_t bytes) {
  PS_CHECK_ARG(ptr, "ps_host_malloc: null output");
  *ptr = nullptr;
  if (bytes == 0) return PS_OK;
  PS_HIP(hipHostMalloc(ptr, bytes, hipHostMallocDefault));
  return PS_OK;
}

int ps_host_free(void* ptr) {
  if (ptr) PS_HIP(hipHostFree(ptr));
  return PS_OK;
}

int ps_memcpy_htod_async(void* dst, const void* src, size_t bytes, ps_stream_t stream) {
  if (bytes == 0) return PS_OK;
  PS_CHECK_ARG(dst && src, "ps_memcpy_htod_async: null pointer");
  PS_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ps::to_hip(stream)));
  return PS_OK;
}

int ps_memcpy_dtod_async(void* dst, const void* src, size_t bytes, ps_stream_t stream) {
  if (bytes == 0) return PS_OK;
  PS_CHECK_ARG(dst && src, "ps_memcpy_dtod_async: null pointer");
  PS_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ps::to_hip(stream)));
  return PS_OK;
}

int ps_memset_async(void* dst, int value, size_t bytes, ps_stream_t stream) {
  if (bytes == 0) return PS_OK;
  PS_CHECK_ARG(dst, "ps_memset_async: null pointer");
  PS_HIP(hipMemsetAsync(dst, value, bytes, ps::to_hip(stream)));
  return PS_OK;
}

int ps_fill_random_async(float* dst, size_t count, uint64_t seed, float lo, float hi,
                         int normal, ps_stream_t stream) {
  if (count == 0) return PS_OK;
  PS_CHECK_ARG(dst, "ps_fill_random_async: null pointer");
  const size_t blocks = (count + 255) / 256;
  const unsigned grid = unsigned(blocks < 65536 ? blocks : 65536);
  ps::fill_random_kernel<<<grid, 256, 0, ps::to_hip(stream)>>>(dst, count, seed, lo, hi,
                                                               normal);
  PS_LAUNCHED();
  return PS_OK;
}

int ps_stream_create(ps_stream_t* stream) {
  PS_CHECK_ARG(stream, "ps_stream_create: null output");
  hipStream_t s = nullptr;
  // Default priority only; blocking with respect to the null stream, as the
  // reference's cudaStreamCreate streams are.
  PS_HIP(hipStreamCreate(&s));
  *stream = reinterpret_cast<ps_stream_t>(s);
  return PS_OK;
}

int ps_stream_destroy(ps_stream_t stream) {
  if (stream) PS_HIP(hipStreamDestroy(ps::to_hip(stream)));
  return PS_OK;
}

int ps_stream_synchronize(ps_stream_t stream) {
  PS_HIP(hipStreamSynchronize(ps::to_hip(stream)));
  return PS_OK;
}

int ps_event_create(ps_event_t* event) {
  PS_CHECK_ARG(event, "ps_event_create: null output");
  hipEvent_t e = nullptr;
  PS_HIP(hipEventCreate(&e));
  *event = reinterpret_cast<ps_event_t>(e);
  return PS_OK;
}

int ps_event_destroy(ps_event_t event) {
  if (event) PS_HIP(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)));
  return PS_OK;
}

int ps_event_record(ps_event_t event, ps_stream_t stream) {
  PS_CHECK_ARG(event, "ps_event_record: null event");
  PS_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(event), ps::to_hip(stream)));
  return PS_OK;
}

int ps_event_synchronize(ps_event_t event) {
  PS_CHECK_ARG(event, "ps_event_synchronize: null event");
  PS_HIP(hipEventSynchronize(reinterpret_cast<hipEvent_t>(event)));
  return PS_OK;
}

int ps_event_elapsed_ms(float* ms, ps_event_t start, ps_event_t stop) {
  PS_CHECK_ARG(ms && start && stop, "ps_event_elapsed_ms: null argument");
  PS_HIP(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                             reinterpret_cast<hipEvent_t>(stop)));
  return PS_OK;
}

int ps_stream_wait_event(ps_stream_t stream, ps_event_t event) {
  PS_CHECK_ARG(event, "ps_stream_wait_event: null event");
  PS_HIP(hipStreamWaitEvent(ps::to_hip(stream), reinterpret_cast<hipEvent_t>(event), 0));
  return PS_OK;
}

}  // extern "C"
