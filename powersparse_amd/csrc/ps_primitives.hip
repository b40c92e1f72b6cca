// Device-wide primitives for the preprocessing: exclusive scan of uint32 and a
// stable least-significant-digit radix sort of (key, uint32 value) pairs, or of
// keys alone when both value buffers are null.
//
// Both use plain reduce-then-scan passes (no inter-workgroup waiting), 256
// threads per workgroup and 4096 items per tile.
//
// Radix pass = histogram kernel + scan of the (digit-major, tile-minor) count
// table + scatter kernel. The scatter ranks each tile's elements stably: wave w
// of the tile owns items [1024w, 1024w + 1024) and walks them in 16 steps of 64
// in order; inside a step the lanes holding the same 8-bit digit are found with
// eight ballots, so an element's offset is (earlier steps' count of its digit in
// this wave) + (lower lanes with the same digit in this step). Wave prefixes and
// the tile's global digit offsets from the scanned table complete the position.
#include <mutex>
#include <vector>

#include "ps_common.hpp"

namespace ps {
namespace {

constexpr int kThreads = 256;
constexpr int kItems = 16;
constexpr int kTile = kThreads * kItems;  // 4096
constexpr int kBins = 256;

__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t v) {
  const int lane = lane_id();
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const uint32_t t = __shfl_up(v, d, kWave);
    if (lane >= d) v += t;
  }
  return v;
}

__global__ __launch_bounds__(kThreads) void scan_reduce_kernel(const uint32_t* __restrict__ in,
                                                               size_t n,
                                                               uint32_t* __restrict__ sums) {
  __shared__ uint32_t wave_sum[kThreads / kWave];
  const size_t base = size_t(blockIdx.x) * kTile;
  uint32_t s = 0;
#pragma unroll
  for (int it = 0; it < kItems; ++it) {
    const size_t i = base + size_t(it) * kThreads + threadIdx.x;
    if (i < n) s += in[i];
  }
  s = wave_inclusive_scan(s);
  if (lane_id() == kWave - 1) wave_sum[threadIdx.x / kWave] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t t = 0;
    for (int w = 0; w < kThreads / kWave; ++w) t += wave_sum[w];
    sums[blockIdx.x] = t;
  }
}

// Exclusive scan of one tile (blocked: thread t owns items 16t .. 16t+15) plus
// the tile's offset from the scanned tile sums (null for a single tile).
__global__ __launch_bounds__(kThreads) void scan_apply_kernel(const uint32_t* in, uint32_t* out,
                                                              size_t n,
                                                              const uint32_t* __restrict__ offsets) {
  __shared__ uint32_t wave_sum[kThreads / kWave];
  const size_t base = size_t(blockIdx.x) * kTile + size_t(threadIdx.x) * kItems;
  uint32_t v[kItems];
  uint32_t total = 0;
#pragma unroll
  for (int it = 0; it < kItems; ++it) {
    const size_t i = base + it;
    v[it] = i < n ? in[i] : 0u;
    total += v[it];
  }
  const uint32_t incl = wave_inclusive_scan(total);
  const int w = threadIdx.x / kWave;
  if (lane_id() == kWave - 1) wave_sum[w] = incl;
  __syncthreads();
  uint32_t run = incl - total + (offsets ? offsets[blockIdx.x] : 0u);
  for (int q = 0; q < w; ++q) run += wave_sum[q];
#pragma unroll
  for (int it = 0; it < kItems; ++it) {
    const size_t i = base + it;
    if (i < n) out[i] = run;
    run += v[it];
  }
}

size_t align_up(size_t x) { return (x + 255) & ~size_t(255); }

size_t scan_ws(size_t n) {
  if (n <= size_t(kTile)) return 0;
  const size_t b = (n + kTile - 1) / kTile;
  return align_up(b * sizeof(uint32_t)) + scan_ws(b);
}

int scan(const uint32_t* in, uint32_t* out, size_t n, char* ws, hipStream_t stream) {
  if (n == 0) return PS_OK;
  const size_t blocks = (n + kTile - 1) / kTile;
  PS_CHECK_ARG(blocks < (1u << 31), "scan too large");
  if (blocks == 1) {
    scan_apply_kernel<<<1, kThreads, 0, stream>>>(in, out, n, nullptr);
    PS_LAUNCHED();
    return PS_OK;
  }
  uint32_t* sums = reinterpret_cast<uint32_t*>(ws);
  scan_reduce_kernel<<<unsigned(blocks), kThreads, 0, stream>>>(in, n, sums);
  PS_LAUNCHED();
  const int rc = scan(sums, sums, blocks, ws + align_up(blocks * sizeof(uint32_t)), stream);
  if (rc != PS_OK) return rc;
  scan_apply_kernel<<<unsigned(blocks), kThreads, 0, stream>>>(in, out, n, sums);
  PS_LAUNCHED();
  return PS_OK;
}

template <typename K>
__global__ __launch_bounds__(kThreads) void radix_hist_kernel(const K* __restrict__ keys, size_t n,
                                                              int shift, uint32_t tiles,
                                                              uint32_t* __restrict__ hist) {
  __shared__ uint32_t cnt[kThreads / kWave][kBins];
  const int w = threadIdx.x / kWave;
  for (int b = threadIdx.x; b < kBins * (kThreads / kWave); b += kThreads) (&cnt[0][0])[b] = 0;
  __syncthreads();
  const size_t base = size_t(blockIdx.x) * kTile;
#pragma unroll 4
  for (int it = 0; it < kItems; ++it) {
    const size_t i = base + size_t(it) * kThreads + threadIdx.x;
    if (i < n) atomicAdd(&cnt[w][uint32_t(keys[i] >> shift) & (kBins - 1)], 1u);
  }
  __syncthreads();
  for (int b = threadIdx.x; b < kBins; b += kThreads) {
    uint32_t s = 0;
#pragma unroll
    for (int q = 0; q < kThreads / kWave; ++q) s += cnt[q][b];
    hist[size_t(b) * tiles + blockIdx.x] = s;
  }
}

template <typename K>
__global__ __launch_bounds__(kThreads) void radix_scatter_kernel(
    const K* __restrict__ keys_in, const uint32_t* __restrict__ vals_in, K* __restrict__ keys_out,
    uint32_t* __restrict__ vals_out, size_t n, int shift, uint32_t tiles,
    const uint32_t* __restrict__ offsets) {
  constexpr int kWaves = kThreads / kWave;
  __shared__ uint32_t cnt[kWaves][kBins];
  __shared__ uint32_t tile_off[kBins];
  const int w = threadIdx.x / kWave;
  const int lane = lane_id();
  for (int b = threadIdx.x; b < kBins * kWaves; b += kThreads) (&cnt[0][0])[b] = 0;
  for (int b = threadIdx.x; b < kBins; b += kThreads)
    tile_off[b] = offsets[size_t(b) * tiles + blockIdx.x];
  __syncthreads();

  const size_t base = size_t(blockIdx.x) * kTile + size_t(w) * (kItems * kWave);
  const uint64_t lower = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  K key[kItems];
  uint32_t val[kItems];
  uint32_t loc[kItems];
#pragma unroll
  for (int r = 0; r < kItems; ++r) {
    const size_t i = base + size_t(r) * kWave + lane;
    const bool valid = i < n;
    key[r] = valid ? keys_in[i] : K(0);
    val[r] = (valid && vals_in) ? vals_in[i] : 0u;
    const uint32_t d = uint32_t(key[r] >> shift) & (kBins - 1);
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const uint64_t m = __ballot((d >> b) & 1);
      peers &= ((d >> b) & 1) ? m : ~m;
    }
    const uint32_t before = cnt[w][d];
    loc[r] = before + uint32_t(__popcll(peers & lower));
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    // the highest lane of each digit class advances the wave's counter
    if (valid && (peers >> lane) == 1ull) cnt[w][d] = before + uint32_t(__popcll(peers));
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  __syncthreads();
  // exclusive prefix of the per-wave counts, digit by digit
  for (int b = threadIdx.x; b < kBins; b += kThreads) {
    uint32_t run = tile_off[b];
#pragma unroll
    for (int q = 0; q < kWaves; ++q) {
      const uint32_t c = cnt[q][b];
      cnt[q][b] = run;
      run += c;
    }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kItems; ++r) {
    const size_t i = base + size_t(r) * kWave + lane;
    if (i < n) {
      const uint32_t d = uint32_t(key[r] >> shift) & (kBins - 1);
      const size_t pos = size_t(cnt[w][d]) + loc[r];
      keys_out[pos] = key[r];
      if (vals_out) vals_out[pos] = val[r];
    }
  }
}

size_t radix_ws(size_t n) {
  const size_t tiles = (n + kTile - 1) / kTile;
  const size_t table = tiles * kBins;
  return align_up(table * sizeof(uint32_t)) + scan_ws(table);
}

template <typename K>
int radix_sort(K* keys, K* keys_alt, uint32_t* vals, uint32_t* vals_alt, size_t n, int begin_bit,
               int end_bit, void* workspace, int* result_in_alt, hipStream_t stream) {
  PS_CHECK_ARG(result_in_alt, "radix sort: null result flag");
  *result_in_alt = 0;
  PS_CHECK_ARG(begin_bit >= 0 && end_bit <= int(8 * sizeof(K)) && begin_bit <= end_bit,
               "radix sort: bad bit range");
  if (n <= 1 || begin_bit == end_bit) return PS_OK;
  PS_CHECK_ARG(keys && keys_alt && workspace && (vals != nullptr) == (vals_alt != nullptr),
               "radix sort: null buffer");
  const size_t tiles = (n + kTile - 1) / kTile;
  PS_CHECK_ARG(tiles < (1u << 31) && n < (size_t(1) << 32), "radix sort: too many items");
  uint32_t* table = reinterpret_cast<uint32_t*>(workspace);
  char* scan_space = reinterpret_cast<char*>(workspace) + align_up(tiles * kBins * sizeof(uint32_t));
  K *kin = keys, *kout = keys_alt;
  uint32_t *vin = vals, *vout = vals_alt;
  int flips = 0;
  for (int shift = begin_bit; shift < end_bit; shift += 8) {
    radix_hist_kernel<K><<<unsigned(tiles), kThreads, 0, stream>>>(kin, n, shift,
                                                                    uint32_t(tiles), table);
    PS_LAUNCHED();
    const int rc = scan(table, table, tiles * kBins, scan_space, stream);
    if (rc != PS_OK) return rc;
    radix_scatter_kernel<K><<<unsigned(tiles), kThreads, 0, stream>>>(
        kin, vin, kout, vout, n, shift, uint32_t(tiles), table);
    PS_LAUNCHED();
    std::swap(kin, kout);
    std::swap(vin, vout);
    flips ^= 1;
  }
  *result_in_alt = flips;
  return PS_OK;
}

}  // namespace
}  // namespace ps

// The tile sums of ps_exclusive_scan_u32_noalloc: every level of the scan
// writes its sums here before reading them, so nothing needs clearing. Each
// GPU holds its own copy for the life of the process; every call on a GPU
// uses that GPU's copy, so calls that overlap on one GPU race.
constexpr size_t kNoAllocScanBytes = size_t(256) << 10;  // 256 KiB: n up to 268,173,312
static __device__ __align__(256) unsigned char scratch[kNoAllocScanBytes];

namespace ps {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxDevices] = {};  // device address of `scratch`, per device

// The current device's copy of `scratch`, resolved once per device (with that
// device current) by hipGetSymbolAddress: host code must never pass the
// array's name itself to a kernel or a copy.
int scratch_address(void** addr) {
  int dev = 0;
  PS_HIP(hipGetDevice(&dev));
  PS_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "device index beyond the scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    void* p = nullptr;
    PS_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    PS_CHECK_ARG(p != nullptr, "hipGetSymbolAddress returned no address for the scratch");
    g_scratch_addr[dev] = p;
  }
  *addr = g_scratch_addr[dev];
  return PS_OK;
}

}  // namespace
}  // namespace ps

extern "C" {

size_t ps_scan_workspace_bytes(size_t n) { return ps::scan_ws(n) + 256; }

int ps_exclusive_scan_u32_noalloc(const uint32_t* in, uint32_t* out, size_t n,
                                  ps_stream_t stream) {
  if (n == 0) return PS_OK;
  PS_CHECK_ARG(ps::scan_ws(n) <= kNoAllocScanBytes,
               "ps_exclusive_scan_u32_noalloc: n = " + std::to_string(n) +
                   " needs more than the " + std::to_string(kNoAllocScanBytes) +
                   "-byte static scratch; use ps_exclusive_scan_u32 with a workspace");
  PS_CHECK_ARG(in && out, "ps_exclusive_scan_u32_noalloc: null buffer");
  void* ws = nullptr;
  const int rc = ps::scratch_address(&ws);
  if (rc != PS_OK) return rc;
  return ps::scan(in, out, n, reinterpret_cast<char*>(ws), ps::to_hip(stream));
}

int ps_exclusive_scan_u32(const uint32_t* in, uint32_t* out, size_t n, void* workspace,
                          ps_stream_t stream) {
  if (n == 0) return PS_OK;
  PS_CHECK_ARG(in && out, "ps_exclusive_scan_u32: null buffer");
  PS_CHECK_ARG(workspace || ps::scan_ws(n) == 0, "ps_exclusive_scan_u32: null workspace");
  return ps::scan(in, out, n, reinterpret_cast<char*>(workspace), ps::to_hip(stream));
}

size_t ps_radix_workspace_bytes(size_t n) { return ps::radix_ws(n) + 256; }

int ps_radix_sort_pairs_u64(uint64_t* keys, uint64_t* keys_alt, uint32_t* vals,
                            uint32_t* vals_alt, size_t n, int begin_bit, int end_bit,
                            void* workspace, int* result_in_alt, ps_stream_t stream) {
  return ps::radix_sort<uint64_t>(keys, keys_alt, vals, vals_alt, n, begin_bit, end_bit,
                                  workspace, result_in_alt, ps::to_hip(stream));
}

int ps_radix_sort_pairs_u32(uint32_t* keys, uint32_t* keys_alt, uint32_t* vals,
                            uint32_t* vals_alt, size_t n, int begin_bit, int end_bit,
                            void* workspace, int* result_in_alt, ps_stream_t stream) {
  return ps::radix_sort<uint32_t>(keys, keys_alt, vals, vals_alt, n, begin_bit, end_bit,
                                  workspace, result_in_alt, ps::to_hip(stream));
}

}  // extern "C"
