// Device, memory, stream and event entry points of the C ABI, plus the
// counter-based random fill used for synthetic dense operands.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "ps_common.hpp"

namespace ps {

namespace {
thread_local std::string g_last_error;

// Device allocation guards (debugging aid, off unless PS_DEVICE_GUARD names a
// byte count): every ps_malloc block gets that many bytes of a known pattern
// before and after it (the count rounded up to a multiple of 256, so blocks
// keep their alignment). ps_free and ps_guard_violations read the guards back
// on the host; a changed byte means some device code wrote outside the block.
constexpr unsigned char kGuardByte = 0xA5;
struct Guarded {
  char* base;    // what hipMalloc returned
  size_t bytes;  // the caller's size
};
struct GuardState {
  size_t guard = 0;
  std::mutex mu;
  std::unordered_map<void*, Guarded> live;
  size_t violations = 0;
};
GuardState& guards() {
  static GuardState* g = [] {
    auto* s = new GuardState;  // never destroyed: frees may come from any exit path
    if (const char* v = std::getenv("PS_DEVICE_GUARD")) {
      const long long n = std::atoll(v);
      if (n > 0) s->guard = (size_t(n) + 255) & ~size_t(255);
    }
    return s;
  }();
  return *g;
}
// Checks both guards of one block (device synchronised by the caller); the
// number of changed bytes, each run of them reported on stderr.
size_t check_guards(size_t guard, void* user, const Guarded& a) {
  std::vector<unsigned char> h(guard);
  size_t bad = 0;
  const char* where[2] = {"before", "after"};
  const char* src[2] = {a.base, a.base + guard + a.bytes};
  for (int k = 0; k < 2; ++k) {
    if (hipMemcpy(h.data(), src[k], guard, hipMemcpyDeviceToHost) != hipSuccess) {
      std::fprintf(stderr, "ps guard: cannot read the guard %s block %p\n", where[k], user);
      ++bad;
      continue;
    }
    size_t first = guard, last = 0, n = 0;
    for (size_t i = 0; i < guard; ++i)
      if (h[i] != kGuardByte) {
        first = i < first ? i : first;
        last = i;
        ++n;
      }
    if (n) {
      std::fprintf(stderr,
                   "ps guard: %zu byte(s) written %s the %zu-byte block at %p (guard offsets "
                   "%zu..%zu of %zu)\n",
                   n, where[k], a.bytes, user, first, last, guard);
      bad += n;
    }
  }
  return bad;
}
}  // namespace

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

}  // namespace
}  // namespace ps

extern "C" {




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
  ps::GuardState& g = ps::guards();
  if (g.guard == 0) {
    PS_HIP(hipMalloc(ptr, bytes));
    return PS_OK;
  }
  char* base = nullptr;
  PS_HIP(hipMalloc(reinterpret_cast<void**>(&base), bytes + 2 * g.guard));
  hipError_t e = hipMemset(base, ps::kGuardByte, g.guard);
  if (e == hipSuccess) e = hipMemset(base + g.guard + bytes, ps::kGuardByte, g.guard);
  if (e != hipSuccess) {
    (void)hipFree(base);
    PS_HIP(e);
  }
  *ptr = base + g.guard;
  std::lock_guard<std::mutex> lock(g.mu);
  g.live[*ptr] = ps::Guarded{base, bytes};
  return PS_OK;
}

int ps_free(void* ptr) {
  if (!ptr) return PS_OK;
  ps::GuardState& g = ps::guards();
  if (g.guard) {
    std::unique_lock<std::mutex> lock(g.mu);
    auto it = g.live.find(ptr);
    if (it != g.live.end()) {
      const ps::Guarded a = it->second;
      g.live.erase(it);
      lock.unlock();
      PS_HIP(hipDeviceSynchronize());
      const size_t bad = ps::check_guards(g.guard, ptr, a);
      lock.lock();
      g.violations += bad;
      lock.unlock();
      PS_HIP(hipFree(a.base));
      return PS_OK;
    }
  }
  PS_HIP(hipFree(ptr));
  return PS_OK;
}

long long ps_guard_violations(void) {
  ps::GuardState& g = ps::guards();
  if (g.guard == 0) return -1;
  if (hipDeviceSynchronize() != hipSuccess) return -2;
  std::lock_guard<std::mutex> lock(g.mu);
  size_t bad = g.violations;
  for (const auto& kv : g.live) bad += ps::check_guards(g.guard, kv.first, kv.second);
  return (long long)bad;
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
