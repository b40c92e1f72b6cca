// PowerSparseMatrixGPU: host orchestration of the GPU preprocessing.
//
// Follows ParCIS/PowerSparse utils/matrix_utils.cu:470-663 step by step, with
// every per-nonzero and per-row loop moved to HIP kernels behind the C ABI:
//   validation (host, as :475-488) -> CSR upload -> worksets S (:31-63, device
//   degree sums) -> column histogram (:508-514, device) -> each row's nonzeros
//   ranked by column count descending, ties in CSR order (:518-524, stable
//   radix sort) -> group counts, scans and metadata (:132-208, device) ->
//   column signature bits (:65-128, host std::sort as in the reference) ->
//   signatures and the stable per-word group sort (:261-327, :562-594) ->
//   final worksets (:596-656).
// The host signature-bit step overlaps the device rank sort.
#include "matrix_utils.h"

#include <algorithm>
#include <chrono>
#include <future>
#include <memory>
#include <mutex>
#include <cmath>
#include <cstring>
#include <numeric>
#include <string>
#include <vector>

#include "device_buffer.h"
#include "preprocess_host.h"
#include "staged_upload.h"

#ifdef _OPENMP
#include <omp.h>
#endif

namespace PowerSparse {

void ThrowOnError(int status) {
  if (status == PS_OK) return;
  const std::string msg = ps_last_error();
  if (status == PS_ERR_INVALID) throw std::invalid_argument(msg);
  throw std::runtime_error(msg);
}

namespace {

#if defined(__GLIBCXX__) && defined(_OPENMP)
// libstdc++'s std::sort (bits/stl_algo.h) runs an introsort loop that
// partitions a range, sorts the part right of the cut, then continues on the
// part left of it, and finishes with one insertion-sort pass over the whole
// range. The two parts of a cut never interact, so sorting the right parts of
// the upper levels as concurrent tasks makes exactly the same element moves
// as the sequential call: the order, ties included, is std::sort's. Every
// step is the library's own (partition, sub-range loop, heap-sort fallback,
// final insertion pass); only the dispatch of independent sub-ranges is here.
constexpr long kSpawnBelow = 1 << 15;  // smaller right parts stay on the thread
constexpr int kSpawnDepth = 8;

template <typename It, typename Size, typename Cmp>
void IntrosortTasks(It first, It last, Size depth, Cmp cmp, int spawn) {
  while (last - first > 16) {  // std::sort's insertion-sort threshold
    if (spawn <= 0) {
      std::__introsort_loop(first, last, depth, cmp);
      return;
    }
    if (depth == 0) {
      std::__partial_sort(first, last, last, cmp);
      return;
    }
    --depth;
    It cut = std::__unguarded_partition_pivot(first, last, cmp);
    if (last - cut >= kSpawnBelow) {
#pragma omp task firstprivate(cut, last, depth, cmp, spawn)
      IntrosortTasks(cut, last, depth, cmp, spawn - 1);
    } else {
      std::__introsort_loop(cut, last, depth, cmp);
    }
    last = cut;
    --spawn;
  }
}

template <typename It, typename Less>
void SameOrderAsStdSort(It first, It last, Less less) {
  if (first == last) return;
  auto cmp = __gnu_cxx::__ops::__iter_comp_iter(less);
  const auto depth = std::__lg(last - first) * 2;
  if (last - first < 4 * kSpawnBelow) {
    std::sort(first, last, less);
    return;
  }
#pragma omp parallel
#pragma omp single
  IntrosortTasks(first, last, depth, cmp, kSpawnDepth);
  std::__final_insertion_sort(first, last, cmp);
}
#else
template <typename It, typename Less>
void SameOrderAsStdSort(It first, It last, Less less) {
  std::sort(first, last, less);
}
#endif

}  // namespace

int GenerateSigBitFFC(int cols, const int* col_nnz, int ffc, int* sigbit) {
  // The reference sorts iota by col_nnz descending with libstdc++ std::sort
  // (unstable, matrix_utils.cu:70-75). Sorting (count, column) records with a
  // comparator that reads only the count makes the same comparisons and moves
  // as sorting column ids through an indirect comparator, so the resulting
  // order (ties included) is identical, without the indirect loads.
  struct Rec {
    int count;
    int col;
  };
  std::vector<Rec> order(static_cast<size_t>(cols));
  for (int c = 0; c < cols; ++c) order[size_t(c)] = Rec{col_nnz[c], c};
  SameOrderAsStdSort(order.begin(), order.end(),
                     [](const Rec& a, const Rec& b) { return a.count > b.count; });
  // FFC buckets (matrix_utils.cu:91-118): the ffc most frequent columns take
  // bit 0 and define the bucket mass; each later bucket takes at least one
  // column and keeps taking columns while its running mass stays below it.
  int i = 0, bit = 0, mass0 = 0;
  const int head = std::min(ffc, cols);
  for (; i < head; ++i) {
    sigbit[order[size_t(i)].col] = 0;
    mass0 += order[size_t(i)].count;
  }
  bit = 1;
  while (i < cols) {
    int mass = order[size_t(i)].count;
    sigbit[order[size_t(i)].col] = bit;
    ++i;
    while (i < cols) {
      mass += order[size_t(i)].count;
      if (mass >= mass0) break;
      sigbit[order[size_t(i)].col] = bit;
      ++i;
    }
    ++bit;
  }
  // Length rounded to whole 32-bit words (:120-122), bits clamped (:123-127).
  int len = bit;
  if (len < 32) len = 32;
  else if (len % 32 < 16) len = len / 32 * 32;
  else len = (len + 31) / 32 * 32;
  for (int c = 0; c < cols; ++c)
    if (sigbit[c] >= len) sigbit[c] = len - 1;
  return len;
}

int WorksetCount(const unsigned long long* degree_sums, int cu_count) {
  // matrix_utils.cu:40-53: threshold = 8 blocks per SM * SMs * 4; the number
  // of worksets is one more than the count of leading sizes whose groups reach it.
  const long long threshold = 8LL * cu_count * 4;
  int S = 0;
  long long groups = threshold + 1;
  while (groups >= threshold) {
    groups = S + 1 < 32 ? (long long)degree_sums[S + 1] : 0;
    ++S;
  }
  return S;
}

namespace {

// Groups per workset, as the device kernels split each row (matrix_utils.cu:
// 132-156): S == 1 cuts rows into chunks of `fine`; otherwise the block sizes
// are taken greedily from the largest and the rest is one residue group.
void HostGroupCounts(const int* row_ptr, int rows, int S, int fine, int* group_num) {
  std::vector<long long> total(static_cast<size_t>(S), 0);
#pragma omp parallel
  {
    std::vector<long long> mine(static_cast<size_t>(S), 0);
#pragma omp for schedule(static)
    for (int r = 0; r < rows; ++r) {
      long long d = row_ptr[r + 1] - row_ptr[r];
      if (S == 1) {
        mine[0] += (d + fine - 1) / fine;
        continue;
      }
      for (int s = S - 1; s > 0; --s) {
        const long long n = d / GROUP_SIZE(s);
        mine[size_t(s)] += n;
        d -= n * GROUP_SIZE(s);
      }
      mine[0] += d > 0;
    }
#pragma omp critical
    for (int s = 0; s < S; ++s) total[size_t(s)] += mine[size_t(s)];
  }
  for (int s = 0; s < S; ++s) {
    if (total[size_t(s)] > std::numeric_limits<int>::max())
      throw std::runtime_error("Too many groups in one workset");
    group_num[s] = int(total[size_t(s)]);
  }
}

int BitsFor(uint64_t v) {
  int b = 0;
  while (b < 64 && (v >> b) != 0) ++b;
  return b;
}

class StageClock {
 public:
  explicit StageClock(PreprocessTimings* t) : t_(t), last_(Now()), first_(last_) {}
  // Records the time since the previous mark into `slot` (synchronising the
  // device first) when timings were requested.
  void Mark(double PreprocessTimings::*slot) {
    if (!t_) return;
    ThrowOnError(ps_device_synchronize());
    const auto now = Now();
    t_->*slot += std::chrono::duration<double, std::milli>(now - last_).count();
    last_ = now;
  }
  void Finish() {
    if (t_) t_->total_ms = std::chrono::duration<double, std::milli>(Now() - first_).count();
  }

 private:
  static std::chrono::steady_clock::time_point Now() { return std::chrono::steady_clock::now(); }
  PreprocessTimings* t_;
  std::chrono::steady_clock::time_point last_, first_;
};

}  // namespace

// The partition-independent stages of the preprocessing. Members are declared
// so that the signature-bit thread (sig_len) is joined before the vectors it
// writes are destroyed.
struct PowerSparseMatrixGPU::Prepared {
  StageClock clock;
  DeviceArray<int> row_ptr, col_ind;
  DeviceArray<float> sp_data;
  unsigned long long degree_sums[32] = {};
  DeviceArray<int> col_nnz;  // device column counts
  std::vector<int> col_nnz_host, sigbit;
  int max_count = 0, count_bits = 0;
  // Each row's nonzeros ranked by column count (descending, ties in CSR order).
  DeviceArray<uint64_t> keys;
  DeviceArray<uint32_t> vals;
  DeviceArray<int> sigbit_device;
  int signature_len = 0;
  std::future<int> sig_len;

  Prepared(int rows, int cols, int nnz, const int* host_row_ptr, const int* host_col_ind,
           const float* host_sp_data, PreprocessTimings* timings)
      : clock(timings), row_ptr(size_t(rows) + 1), col_ind(size_t(nnz)), sp_data(size_t(nnz)) {
    StagedUpload(row_ptr.data(), host_row_ptr, sizeof(int) * (size_t(rows) + 1));
    StagedUpload(col_ind.data(), host_col_ind, sizeof(int) * size_t(nnz));
    StagedUpload(sp_data.data(), host_sp_data, sizeof(float) * size_t(nnz));
    clock.Mark(&PreprocessTimings::upload_ms);
    Analyze(rows, cols, nnz);
  }
  // From a CSR already on the device (stage times not recorded).
  Prepared(int rows, int cols, int nnz, DeviceArray<int>&& rp, DeviceArray<int>&& ci,
           DeviceArray<float>&& sv)
      : clock(nullptr), row_ptr(std::move(rp)), col_ind(std::move(ci)), sp_data(std::move(sv)) {
    Analyze(rows, cols, nnz);
  }

  void Analyze(int rows, int cols, int nnz) {
    ps_stream_t st = nullptr;
    // Degree sums (AnalyzeMatrix) and the column histogram.
    ThrowOnError(ps_pre_degree_sums(row_ptr.data(), rows, degree_sums, st));
    col_nnz.Allocate(size_t(cols));
    col_nnz.Zero(st);
    ThrowOnError(ps_pre_col_histogram(col_ind.data(), nnz, col_nnz.data(), st));
    col_nnz_host.resize(size_t(cols));
    col_nnz.Download(col_nnz_host.data(), size_t(cols));
    max_count = *std::max_element(col_nnz_host.begin(), col_nnz_host.end());
    clock.Mark(&PreprocessTimings::analyze_ms);

    // Host: the column signature bits, on a thread of their own while this
    // thread drives the device work that does not need them (joined by
    // SignatureLen()).
    sigbit.resize(size_t(cols));
    sig_len = std::async(std::launch::async, [this, cols] {
      return GenerateSigBitFFC(cols, col_nnz_host.data(), 2, sigbit.data());
    });

    count_bits = BitsFor(uint64_t(max_count));
    keys.Allocate(size_t(nnz));
    vals.Allocate(size_t(nnz));
    ThrowOnError(ps_pre_rank_sort(row_ptr.data(), rows, col_ind.data(), nnz, col_nnz.data(),
                                  max_count, count_bits, keys.data(), vals.data(), st));
    clock.Mark(&PreprocessTimings::rank_ms);
  }

  // Joins the signature-bit thread on the first call (sigbit_ms: the time
  // spent waiting for it) and uploads the bits.
  int SignatureLen() {
    if (sig_len.valid()) {
      signature_len = sig_len.get();
      clock.Mark(&PreprocessTimings::sigbit_ms);
      sigbit_device.Allocate(sigbit.size());
      sigbit_device.Upload(sigbit.data(), sigbit.size());
    }
    return signature_len;
  }
};

PowerSparseMatrixGPU::PowerSparseMatrixGPU(int row_num, int col_num, int nnz_num,
                                           const int* row_ptr, const int* col_ind,
                                           const float* sp_data)
    : PowerSparseMatrixGPU(row_num, col_num, nnz_num, row_ptr, col_ind, sp_data,
                           PartitionPolicy{}) {}

PowerSparseMatrixGPU::PowerSparseMatrixGPU(Unbuilt, int row_num, int col_num, int nnz_num,
                                           int cu_count, const PartitionPolicy& policy)
    : _matrix_row(row_num), _matrix_col(col_num), _matrix_nnz(nnz_num) {
  Configure(policy);
  _cu_count = cu_count;
}

void PowerSparseMatrixGPU::Configure(const PartitionPolicy& policy) {
  if (policy.cu_count < 0) throw std::invalid_argument("PartitionPolicy::cu_count must be >= 0");
  if (int(policy.signature_order) < 0 || int(policy.signature_order) > 2)
    throw std::invalid_argument("PartitionPolicy::signature_order is not a SignatureOrder");
  if (int(policy.task_order) < 0 || int(policy.task_order) > 2)
    throw std::invalid_argument("PartitionPolicy::task_order is not a TaskOrder");
  if (policy.max_group_types < 0)
    throw std::invalid_argument("PartitionPolicy::max_group_types must be >= 0");
  if (int(policy.spmm_partition) < 0 || int(policy.spmm_partition) > 1)
    throw std::invalid_argument("PartitionPolicy::spmm_partition is not an SpmmPartition");
  _cu_count = policy.cu_count;
  _signature_order = policy.signature_order;
  _keep_csr_pos = policy.csr_positions;
  _task_order = policy.task_order;
  _want_run_order = policy.run_order;
  _max_group_types = policy.max_group_types;
}

PowerSparseMatrixGPU::PowerSparseMatrixGPU(int row_num, int col_num, int nnz_num,
                                           const int* row_ptr, const int* col_ind,
                                           const float* sp_data, const PartitionPolicy& policy,
                                           PreprocessTimings* timings)
    : _matrix_row(row_num), _matrix_col(col_num), _matrix_nnz(nnz_num) {
  // Same checks and messages as the reference constructor (matrix_utils.cu:475-488).
  if (row_num <= 0 || col_num <= 0 || nnz_num <= 0 ||
      row_num > std::numeric_limits<int>::max() - 32 ||
      nnz_num > std::numeric_limits<int>::max() - 32 || !row_ptr || !col_ind || !sp_data) {
    throw std::invalid_argument("Expected a nonempty CSR matrix with 32-bit indices");
  }
  if (row_ptr[0] != 0 || row_ptr[row_num] != nnz_num)
    throw std::invalid_argument("Invalid CSR row-pointer endpoints");
  int bad = 0;
#pragma omp parallel for reduction(| : bad) schedule(static)
  for (int r = 0; r < row_num; ++r) bad |= (row_ptr[r] < 0 || row_ptr[r] > row_ptr[r + 1]);
  if (bad) throw std::invalid_argument("CSR row pointers must be nondecreasing");
#pragma omp parallel for reduction(| : bad) schedule(static)
  for (int p = 0; p < nnz_num; ++p)
    bad |= (col_ind[p] < 0 || col_ind[p] >= col_num || !std::isfinite(sp_data[p]));
  if (bad) throw std::invalid_argument("Invalid CSR column index or sparse value");
  Configure(policy);
  if (_cu_count == 0) {
    int dev = 0;
    ThrowOnError(ps_get_device(&dev));
    ps_device_props props;
    ThrowOnError(ps_get_device_props(dev, &props));
    _cu_count = props.cu_count;
  }
  try {
    Prepared in(row_num, col_num, nnz_num, row_ptr, col_ind, sp_data, timings);
    // A tuned SpMM partition may follow only in signature order (kAuto
    // decides the order at the end of the build).
    const bool may_tune =
        policy.spmm_partition == SpmmPartition::kTuned && _task_order != TaskOrder::kRow;
    Build(row_ptr, in, !may_tune);
    bool hub = false;
    if (may_tune && _task_order == TaskOrder::kSignature && _want_run_order &&
        policy.hub_block == HubBlock::kAuto)
      hub = BuildHub(row_ptr, in, policy);
    if (!hub && may_tune && _task_order == TaskOrder::kSignature &&
        _group_type_num > kTunedSpmmGroupTypes) {
      PartitionPolicy tuned;
      tuned.cu_count = _cu_count;
      tuned.task_order = TaskOrder::kSignature;
      tuned.run_order = false;
      tuned.max_group_types = kTunedSpmmGroupTypes;
      tuned.spmm_partition = SpmmPartition::kParity;
      _spmm_tuned =
          new PowerSparseMatrixGPU(Unbuilt{}, row_num, col_num, nnz_num, _cu_count, tuned);
      _spmm_tuned->Build(row_ptr, in, true);
    }
    in.clock.Finish();
  } catch (...) {
    Release();
    throw;
  }
}

void PowerSparseMatrixGPU::Build(const int* row_ptr, Prepared& in, bool last_partition) {
  const int rows = _matrix_row, nnz = _matrix_nnz;
  const int fine = _group_fine_size;
  ps_stream_t st = nullptr;
  StageClock& clock = in.clock;
  DeviceArray<int>& d_rp = in.row_ptr;
  DeviceArray<int>& d_ci = in.col_ind;
  DeviceArray<float>& d_sv = in.sp_data;
  DeviceArray<uint32_t>& vals = in.vals;
  const int count_bits = in.count_bits;

  // Worksets S (AnalyzeMatrix), with the policy's cap.
  int S = WorksetCount(in.degree_sums, _cu_count);
  if (_max_group_types > 0 && S > _max_group_types) S = _max_group_types;
  if (S > PS_MAX_WORKSETS) throw std::runtime_error("Too many worksets");
  _group_type_num = S;
  // No tuned partition follows a partition of at most its cap of worksets.
  if (S <= kTunedSpmmGroupTypes) last_partition = true;

  // Group counts per workset, on the host from row_ptr (the split the device
  // kernels make), so the device arrays are sized without waiting.
  _group_num = new int[S]();
  HostGroupCounts(row_ptr, rows, S, fine, _group_num);
  const int G0 = _group_num[0];
  std::vector<long long> lengths(static_cast<size_t>(S), 0);  // nonzeros per workset
  lengths[0] = nnz;
  for (int s = 1; s < S; ++s) {
    lengths[size_t(s)] = (long long)_group_num[s] * GROUP_SIZE(s);
    lengths[0] -= lengths[size_t(s)];
  }

  // Per-row group counts and their exclusive scans (group ids in row order).
  const size_t stride = size_t(rows) + 1;
  DeviceArray<uint32_t> prefix(static_cast<size_t>(S) * stride);
  ThrowOnError(ps_pre_group_counts(d_rp.data(), rows, S, fine, prefix.data(), st));
  DeviceArray<char> scan_ws(ps_scan_workspace_bytes(stride));
  for (int s = 0; s < S; ++s)
    ThrowOnError(ps_exclusive_scan_u32(prefix.data() + s * stride, prefix.data() + s * stride,
                                       stride, scan_ws.data(), st));

  std::vector<DeviceArray<int>> des0(static_cast<size_t>(S)), start(static_cast<size_t>(S));
  std::vector<int*> des_ptr(static_cast<size_t>(S), nullptr), start_ptr(static_cast<size_t>(S), nullptr);
  for (int s = 0; s < S; ++s) {
    des0[size_t(s)].Allocate(size_t(_group_num[s]));
    start[size_t(s)].Allocate(size_t(_group_num[s]));
    des_ptr[size_t(s)] = des0[size_t(s)].data();
    start_ptr[size_t(s)] = start[size_t(s)].data();
  }
  DeviceArray<int> res_len(static_cast<size_t>(G0));
  DeviceArray<uint8_t> res_atomic0(static_cast<size_t>(G0));
  ThrowOnError(ps_pre_group_meta(d_rp.data(), rows, S, fine, prefix.data(), des_ptr.data(),
                                 start_ptr.data(), res_len.data(), res_atomic0.data(), st));
  clock.Mark(&PreprocessTimings::groups_ms);

  // The row-ordered execution copy (task order) does not depend on the
  // signature order either: build it now, decide whether to keep it later.
  DeviceArray<uint32_t> iota, exec_len;
  DeviceArray<char> exec_ws;
  if (_task_order != TaskOrder::kSignature) {
    size_t gmax = 0;
    for (int s = 0; s < S; ++s) gmax = std::max(gmax, size_t(_group_num[s]));
    iota.Allocate(gmax);
    ThrowOnError(ps_iota_u32(iota.data(), int(gmax), st));
    _exec_col_ind = new int*[S]();
    _exec_sp_data = new float*[S]();
    _exec_group_des = new int*[S]();
    _exec_out_base = new int*[S]();
    if (_keep_csr_pos) _exec_csr_pos = new int*[S]();
    // residue offsets in the initial (row) order
    ThrowOnError(ps_malloc(reinterpret_cast<void**>(&_exec_residue_offset),
                           sizeof(int) * (size_t(G0) + 1)));
    ThrowOnError(ps_memset_async(_exec_residue_offset, 0, sizeof(int) * (size_t(G0) + 1), st));
    if (G0 > 0) {
      exec_len.Allocate(size_t(G0) + 1);
      ThrowOnError(ps_memcpy_dtod_async(exec_len.data(), res_len.data(), sizeof(int) * size_t(G0),
                                        st));
      ThrowOnError(ps_memset_async(exec_len.data() + G0, 0, sizeof(uint32_t), st));
      exec_ws.Allocate(ps_scan_workspace_bytes(size_t(G0) + 1));
      ThrowOnError(ps_exclusive_scan_u32(exec_len.data(),
                                         reinterpret_cast<uint32_t*>(_exec_residue_offset),
                                         size_t(G0) + 1, exec_ws.data(), st));
    }
    for (int s = 0; s < S; ++s) {
      const int G = _group_num[s];
      if (G == 0) continue;
      const size_t size = size_t(lengths[size_t(s)]);
      ThrowOnError(ps_malloc(reinterpret_cast<void**>(&_exec_col_ind[s]), sizeof(int) * size));
      ThrowOnError(ps_malloc(reinterpret_cast<void**>(&_exec_sp_data[s]), sizeof(float) * size));
      if (_keep_csr_pos)
        ThrowOnError(ps_malloc(reinterpret_cast<void**>(&_exec_csr_pos[s]), sizeof(int) * size));
      ThrowOnError(ps_pre_gather_workset(s == 0 ? 0 : GROUP_SIZE(s), iota.data(), G,
                                         start[size_t(s)].data(),
                                         s == 0 ? _exec_residue_offset : nullptr, vals.data(),
                                         d_ci.data(), d_sv.data(), _exec_col_ind[s],
                                         _exec_sp_data[s],
                                         _keep_csr_pos ? _exec_csr_pos[s] : nullptr, st));
    }
  }

  _signature_len = in.SignatureLen();

  // Groups in signature order: perm[s][k] = initial group at position k.
  const int words = _signature_len / 32;
  if (_signature_order == SignatureOrder::kAuto)
    _signature_order = words <= kBitmapMaxWords ? SignatureOrder::kBitmapWords
                                                : SignatureOrder::kBitLists;
  const int* d_sigbit = in.sigbit_device.data();
  const uint64_t* keys = in.keys.data();
  std::vector<DeviceArray<uint32_t>> perm(static_cast<size_t>(S));
  std::vector<uint32_t*> perm_ptr(static_cast<size_t>(S), nullptr);
  for (int s = 0; s < S; ++s) {
    if (_group_num[s] == 0) continue;
    perm[size_t(s)].Allocate(size_t(_group_num[s]));
    perm_ptr[size_t(s)] = perm[size_t(s)].data();
  }
  if (_signature_order == SignatureOrder::kBitLists) {
    // Each group's sorted distinct signature bits, then the tie refinement.
    size_t total = 0;
    for (int s = 0; s < S; ++s) total += size_t(_group_num[s]);
    DeviceArray<uint32_t> lists(static_cast<size_t>(nnz)), list_begin(total + 1);
    ThrowOnError(ps_pre_signature_lists(d_rp.data(), rows, S, fine, keys, count_bits,
                                        vals.data(), nnz, d_ci.data(), d_sigbit,
                                        _signature_len, prefix.data(), _group_num, lists.data(),
                                        list_begin.data(), st));
    if (last_partition) in.keys.Reset();
    clock.Mark(&PreprocessTimings::signature_ms);
    ThrowOnError(ps_pre_signature_order(lists.data(), list_begin.data(), S, _group_num,
                                        _signature_len, perm_ptr.data(), st));
  } else {
    // Signature bitmaps, word-major per workset.
    std::vector<DeviceArray<uint32_t>> sig(static_cast<size_t>(S));
    std::vector<uint32_t*> sig_ptr(static_cast<size_t>(S), nullptr);
    for (int s = 0; s < S; ++s) {
      sig[size_t(s)].Allocate(size_t(_group_num[s]) * words);
      sig[size_t(s)].Zero(st);
      sig_ptr[size_t(s)] = sig[size_t(s)].data();
    }
    ThrowOnError(ps_pre_signatures(d_rp.data(), rows, S, fine, keys, count_bits,
                                   vals.data(), nnz, d_ci.data(), d_sigbit, prefix.data(),
                                   _group_num, sig_ptr.data(), st));
    if (last_partition) in.keys.Reset();
    clock.Mark(&PreprocessTimings::signature_ms);
    // Stable sort of each workset's groups by signature, descending, word 0
    // most significant: one stable pass per word from the last word to the
    // first (matrix_utils.cu:590-592), skipping words and digits that do not vary.
    for (int s = 0; s < S; ++s) {
      const int G = _group_num[s];
      if (G == 0) continue;
      ThrowOnError(ps_iota_u32(perm[size_t(s)].data(), G, st));
      if (G == 1) continue;
      std::vector<uint32_t> w_or(static_cast<size_t>(words)), w_and(static_cast<size_t>(words));
      ThrowOnError(ps_pre_signature_span(sig[size_t(s)].data(), G, words, w_or.data(),
                                         w_and.data(), st));
      DeviceArray<uint32_t> k1(static_cast<size_t>(G)), k2(static_cast<size_t>(G)), p2(static_cast<size_t>(G));
      DeviceArray<char> ws(ps_radix_workspace_bytes(size_t(G)));
      for (int w = words - 1; w >= 0; --w) {
        const uint32_t diff = w_or[size_t(w)] ^ w_and[size_t(w)];
        if (diff == 0) continue;
        const int lo = __builtin_ctz(diff) / 8 * 8;
        const int hi = 32 - __builtin_clz(diff);
        ThrowOnError(ps_pre_signature_keys(sig[size_t(s)].data() + size_t(w) * G,
                                           perm[size_t(s)].data(), G, k1.data(), st));
        int alt = 0;
        ThrowOnError(ps_radix_sort_pairs_u32(k1.data(), k2.data(), perm[size_t(s)].data(),
                                             p2.data(), size_t(G), lo, hi, ws.data(), &alt, st));
        if (alt) std::swap(perm[size_t(s)], p2);
      }
      sig[size_t(s)].Reset();
    }
  }
  clock.Mark(&PreprocessTimings::order_ms);

  // Final metadata and worksets in signature order.
  _workset_col_ind = new int*[S]();
  _workset_sp_data = new float*[S]();
  _group_des = new int*[S]();
  if (_keep_csr_pos) _workset_csr_pos = new int*[S]();
  ThrowOnError(ps_malloc(reinterpret_cast<void**>(&_residue_offset), sizeof(int) * (size_t(G0) + 1)));
  ThrowOnError(ps_memset_async(_residue_offset, 0, sizeof(int) * (size_t(G0) + 1), st));
  if (G0 > 0) {
    ThrowOnError(ps_malloc(reinterpret_cast<void**>(&_residue_atomic), sizeof(bool) * size_t(G0)));
    ThrowOnError(ps_malloc(reinterpret_cast<void**>(&_group_des[0]), sizeof(int) * size_t(G0)));
    DeviceArray<uint32_t> len(static_cast<size_t>(G0) + 1);
    ThrowOnError(ps_pre_permute_meta(perm[0].data(), G0, des0[0].data(), _group_des[0],
                                     res_len.data(), len.data(), res_atomic0.data(),
                                     reinterpret_cast<uint8_t*>(_residue_atomic), st));
    DeviceArray<char> ws(ps_scan_workspace_bytes(size_t(G0) + 1));
    ThrowOnError(ps_exclusive_scan_u32(len.data(), reinterpret_cast<uint32_t*>(_residue_offset),
                                       size_t(G0) + 1, ws.data(), st));
  }
  for (int s = 1; s < S; ++s) {
    const int G = _group_num[s];
    if (G == 0) continue;
    ThrowOnError(ps_malloc(reinterpret_cast<void**>(&_group_des[s]), sizeof(int) * size_t(G)));
    ThrowOnError(ps_pre_permute_meta(perm[size_t(s)].data(), G, des0[size_t(s)].data(),
                                     _group_des[s], nullptr, nullptr, nullptr, nullptr, st));
  }
  for (int s = 0; s < S; ++s) {
    const int G = _group_num[s];
    if (G == 0) continue;
    const size_t size = size_t(lengths[size_t(s)]);
    ThrowOnError(ps_malloc(reinterpret_cast<void**>(&_workset_col_ind[s]), sizeof(int) * size));
    ThrowOnError(ps_malloc(reinterpret_cast<void**>(&_workset_sp_data[s]), sizeof(float) * size));
    if (_keep_csr_pos)
      ThrowOnError(ps_malloc(reinterpret_cast<void**>(&_workset_csr_pos[s]), sizeof(int) * size));
    ThrowOnError(ps_pre_gather_workset(s == 0 ? 0 : GROUP_SIZE(s), perm[size_t(s)].data(), G,
                                       start[size_t(s)].data(), s == 0 ? _residue_offset : nullptr,
                                       vals.data(), d_ci.data(), d_sv.data(), _workset_col_ind[s],
                                       _workset_sp_data[s],
                                       _keep_csr_pos ? _workset_csr_pos[s] : nullptr, st));
  }

  // Task order: keep the row-ordered copy when asked for, or when it scores
  // clearly better than the signature order.
  if (_task_order != TaskOrder::kSignature) {
    if (G0 > 0) _exec_residue_atomic = reinterpret_cast<bool*>(res_atomic0.Release());
    for (int s = 0; s < S; ++s)
      if (_group_num[s] > 0) _exec_group_des[s] = des0[size_t(s)].Release();
    bool keep = _task_order == TaskOrder::kRow;
    if (_task_order == TaskOrder::kAuto) {
      // Launch order of the worksets: largest groups first, the residue last.
      std::vector<const int*> pub(static_cast<size_t>(S)), row(static_cast<size_t>(S));
      std::vector<long long> len(static_cast<size_t>(S));
      for (int q = 0; q < S; ++q) {
        pub[size_t(q)] = _workset_col_ind[S - 1 - q];
        row[size_t(q)] = _exec_col_ind[S - 1 - q];
        len[size_t(q)] = lengths[size_t(S - 1 - q)];
      }
      ThrowOnError(ps_pre_locality_score(S, pub.data(), len.data(), kLocalityWindow,
                                         kLocalityWindows, &_locality[0], st));
      ThrowOnError(ps_pre_locality_score(S, row.data(), len.data(), kLocalityWindow,
                                         kLocalityWindows, &_locality[1], st));
      keep = _locality[1] < kRowOrderGain * _locality[0];
    }
    if (keep) {
      _task_order = TaskOrder::kRow;
      for (int s = 0; s < S; ++s) {
        const int G = _group_num[s];
        if (G == 0) continue;
        ThrowOnError(ps_malloc(reinterpret_cast<void**>(&_exec_out_base[s]),
                               sizeof(int) * size_t(G)));
        ThrowOnError(ps_pre_exec_positions(s == 0 ? 0 : GROUP_SIZE(s), perm[size_t(s)].data(), G,
                                           _residue_offset, _exec_out_base[s], st));
      }
    } else {
      _task_order = TaskOrder::kSignature;
      ThrowOnError(ps_device_synchronize());
      ReleaseExecution();
    }
  }
  if (_task_order == TaskOrder::kSignature && _want_run_order) BuildRunOrders();
  ThrowOnError(ps_device_synchronize());
  clock.Mark(&PreprocessTimings::gather_ms);
}

// ------------------------------------------------------------ hub block

// One tier of the hub block: a row range x its hot columns.
struct HubTier {
  ps_hub_block desc{};
  DeviceArray<int> hub_rows, hub_index, hot_cols, hot_rank;
  DeviceArray<float> dense;
  DeviceArray<uint32_t> stored;
  // the SDDMM plan of the 64-nonzero tiles of the public block groups lying
  // inside this tier (SDDMM writes their outputs from the dense tiles), and
  // the number of tiles it was built from (0: the tier serves SpMM only)
  DeviceArray<char> plan;
  uint32_t plan_tiles = 0;
};

struct PowerSparseMatrixGPU::HubState {
  std::vector<std::unique_ptr<HubTier>> tiers;
  // the operator workspace (allocated with the block for every width, so
  // calls allocate nothing): one call at a time, in GPU order (`done` is
  // recorded after each call's hub kernels, the next call waits for it)
  std::mutex mu;
  DeviceArray<char> ws;
  ps_event_t done = nullptr;
  bool recorded = false;
  ~HubState() {
    if (done) ps_event_destroy(done);
  }
  size_t Workspace(int op, int N) const {
    size_t need = 0;
    for (const auto& t : tiers)
      if (op == PS_OP_SPMM || t->plan_tiles)
        need = std::max(need, ps_hub_workspace_bytes(&t->desc, op, N));
    return need;
  }
};

int PowerSparseMatrixGPU::HubTiers() const { return _hub ? int(_hub->tiers.size()) : 0; }
int PowerSparseMatrixGPU::HubRows(int tier) const {
  return tier >= 0 && tier < HubTiers() ? _hub->tiers[size_t(tier)]->desc.rows : 0;
}
int PowerSparseMatrixGPU::HubCols(int tier) const {
  return tier >= 0 && tier < HubTiers() ? _hub->tiers[size_t(tier)]->desc.cols : 0;
}

namespace {
int FloorLog2(long long v) {
  int b = -1;
  while (v > 0) {
    v >>= 1;
    ++b;
  }
  return b;
}
struct TierSpec {
  long long min_degree, max_degree, min_count;  // rows in [min_degree, max_degree)
};
}  // namespace

bool PowerSparseMatrixGPU::BuildHub(const int* row_ptr, Prepared& in,
                                    const PartitionPolicy& policy) {
  const int rows = _matrix_row, cols = _matrix_col, S = _group_type_num;
  if (S < 2) return false;  // fine mode: its store rule differs from a capped partition's
  const std::vector<int>& cnt = in.col_nnz_host;
  // rows of degree >= 2^a, columns of count >= 2^b (index 32: none)
  std::vector<long long> rows_ge(34, 0), cols_ge(34, 0);
  for (int r = 0; r < rows; ++r) {
    const int d = row_ptr[r + 1] - row_ptr[r];
    if (d > 0) ++rows_ge[size_t(FloorLog2(d))];
  }
  for (int c = 0; c < cols; ++c)
    if (cnt[size_t(c)] > 0) ++cols_ge[size_t(FloorLog2(cnt[size_t(c)]))];
  for (int k = 31; k >= 0; --k) {
    rows_ge[size_t(k)] += rows_ge[size_t(k) + 1];
    cols_ge[size_t(k)] += cols_ge[size_t(k) + 1];
  }
  std::vector<TierSpec> specs;
  const bool forced = policy.hub_min_degree[0] > 0 && policy.hub_min_count[0] > 0;
  if (forced) {
    for (int k = 0; k < kHubMaxTiers; ++k) {
      if (policy.hub_min_degree[k] <= 0 || policy.hub_min_count[k] <= 0) break;
      const long long hi = specs.empty() ? std::numeric_limits<long long>::max()
                                         : specs.back().min_degree;
      if (policy.hub_min_degree[k] >= hi)
        throw std::invalid_argument("PartitionPolicy hub tiers need decreasing row degrees");
      specs.push_back({policy.hub_min_degree[k], hi, policy.hub_min_count[k]});
    }
  } else {
    // nonzeros of rows of degree >= 2^a (a >= 8) in columns of count >= 2^b
    DeviceArray<unsigned long long> hist(32 * 32);
    ThrowOnError(ps_hub_histogram(in.row_ptr.data(), rows, in.col_ind.data(), in.col_nnz.data(),
                                  hist.data(), nullptr));
    std::vector<unsigned long long> h(32 * 32);
    hist.Download(h.data(), h.size());
    std::vector<double> ge(33 * 33, 0.0);
    for (int a = 31; a >= 0; --a)
      for (int b = 31; b >= 0; --b)
        ge[size_t(a) * 33 + size_t(b)] = double(h[size_t(a) * 32 + size_t(b)]) +
                                         ge[size_t(a + 1) * 33 + size_t(b)] +
                                         ge[size_t(a) * 33 + size_t(b + 1)] -
                                         ge[size_t(a + 1) * 33 + size_t(b + 1)];
    int top = 32;  // the rows of earlier tiers have degree >= 2^top
    for (int k = 0; k < kHubMaxTiers; ++k) {
      double best = 0.0;
      int ba = -1, bb = -1;
      for (int a = 8; a < top; ++a)
        for (int b = 0; b < 31; ++b) {
          const long long R = rows_ge[size_t(a)] - rows_ge[size_t(top)], H = cols_ge[size_t(b)];
          if (R < kHubMinRows || H < kHubMinCols || R * H > kHubMaxElements) continue;
          const double nz = ge[size_t(a) * 33 + size_t(b)] - ge[size_t(top) * 33 + size_t(b)];
          const double gain = nz - kHubDenseCost * double(R) * double(H);
          if (gain > best) {
            best = gain;
            ba = a;
            bb = b;
          }
        }
      if (ba < 0 || best < (k == 0 ? kHubMinGain : kHubMinTierGain) * double(_matrix_nnz)) break;
      specs.push_back({1LL << ba, top < 32 ? (1LL << top) : std::numeric_limits<long long>::max(),
                       1LL << bb});
      top = ba;
    }
    if (specs.empty()) return false;
  }

  auto hub = std::make_unique<HubState>();
  for (const TierSpec& spec : specs) {
    auto t = std::make_unique<HubTier>();
    std::vector<int> hub_rows, hub_index(size_t(rows), -1), hot_cols, hot_rank(size_t(cols), -1);
    for (int r = 0; r < rows; ++r) {
      const long long d = row_ptr[r + 1] - row_ptr[r];
      if (d >= spec.min_degree && d < spec.max_degree) {
        hub_index[size_t(r)] = int(hub_rows.size());
        hub_rows.push_back(r);
      }
    }
    for (int c = 0; c < cols; ++c)
      if (cnt[size_t(c)] >= spec.min_count) {
        hot_rank[size_t(c)] = int(hot_cols.size());
        hot_cols.push_back(c);
      }
    const long long R = (long long)hub_rows.size(), H = (long long)hot_cols.size();
    if (R == 0 || H == 0) continue;
    if (R * H > kHubMaxElements) {
      if (forced)
        throw std::invalid_argument("PartitionPolicy hub thresholds give a dense block over " +
                                    std::to_string(kHubMaxElements) + " elements");
      continue;
    }
    t->hub_rows.Allocate(size_t(R));
    t->hub_rows.Upload(hub_rows.data(), size_t(R));
    t->hub_index.Allocate(size_t(rows));
    t->hub_index.Upload(hub_index.data(), size_t(rows));
    t->hot_cols.Allocate(size_t(H));
    t->hot_cols.Upload(hot_cols.data(), size_t(H));
    t->hot_rank.Allocate(size_t(cols));
    t->hot_rank.Upload(hot_rank.data(), size_t(cols));
    ps_hub_block& d = t->desc;
    d.matrix_rows = rows;
    d.matrix_cols = cols;
    d.rows = int(R);
    d.cols = int(H);
    d.hub_rows = t->hub_rows.data();
    d.hub_index = t->hub_index.data();
    d.hot_cols = t->hot_cols.data();
    d.hot_rank = t->hot_rank.data();
    t->dense.Allocate(ps_hub_dense_floats(int(R), int(H)));
    t->stored.Allocate(ps_hub_stored_words(&d));
    d.dense = t->dense.data();
    d.stored = t->stored.data();
    ThrowOnError(ps_hub_dense_build(&d, in.row_ptr.data(), in.col_ind.data(), in.sp_data.data(),
                                    t->dense.data(), t->stored.data(), nullptr));
    hub->tiers.push_back(std::move(t));
  }
  if (hub->tiers.empty()) return false;

  // SpMM: a tuned partition of the matrix without the block, the tiers taken
  // out one after another (their rows are disjoint).
  DeviceArray<int> rp, ci;
  DeviceArray<float> sv;
  std::vector<int> rp_host(size_t(rows) + 1);
  int nnz_rest = _matrix_nnz;
  for (const auto& t : hub->tiers) {
    const int* cur_rp = rp.size() ? rp.data() : in.row_ptr.data();
    const int* cur_ci = ci.size() ? ci.data() : in.col_ind.data();
    const float* cur_sv = sv.size() ? sv.data() : in.sp_data.data();
    DeviceArray<uint32_t> kept(size_t(rows) + 1);
    ThrowOnError(ps_memset_async(kept.data() + rows, 0, sizeof(uint32_t), nullptr));
    ThrowOnError(ps_hub_kept_counts(&t->desc, cur_rp, cur_ci, kept.data(), nullptr));
    DeviceArray<int> next_rp(size_t(rows) + 1);
    {
      DeviceArray<char> scan_ws(ps_scan_workspace_bytes(size_t(rows) + 1));
      ThrowOnError(ps_exclusive_scan_u32(kept.data(), reinterpret_cast<uint32_t*>(next_rp.data()),
                                         size_t(rows) + 1, scan_ws.data(), nullptr));
    }
    ThrowOnError(ps_memcpy_dtoh(&nnz_rest, next_rp.data() + rows, sizeof(int)));
    if (nnz_rest <= 0) return false;  // the block would hold every nonzero
    DeviceArray<int> next_ci{static_cast<size_t>(nnz_rest)};
    DeviceArray<float> next_sv{static_cast<size_t>(nnz_rest)};
    ThrowOnError(ps_hub_compact(&t->desc, cur_rp, cur_ci, cur_sv,
                                reinterpret_cast<const uint32_t*>(next_rp.data()), next_ci.data(),
                                next_sv.data(), nullptr));
    rp = std::move(next_rp);
    ci = std::move(next_ci);
    sv = std::move(next_sv);
  }
  rp.Download(rp_host.data(), rp_host.size());
  Prepared rest(rows, cols, nnz_rest, std::move(rp), std::move(ci), std::move(sv));
  // the rest must keep the public partition's store rule: more than one workset
  if (std::min(WorksetCount(rest.degree_sums, _cu_count), kTunedSpmmGroupTypes) < 2) return false;
  PartitionPolicy tuned;
  tuned.cu_count = _cu_count;
  tuned.task_order = TaskOrder::kSignature;
  tuned.run_order = false;
  tuned.max_group_types = kTunedSpmmGroupTypes;
  tuned.spmm_partition = SpmmPartition::kParity;
  tuned.hub_block = HubBlock::kOff;
  std::unique_ptr<PowerSparseMatrixGPU> part(
      new PowerSparseMatrixGPU(Unbuilt{}, rows, cols, nnz_rest, _cu_count, tuned));
  part->Build(rp_host.data(), rest, true);
  // hub rows add their remaining entries to the block's product
  for (const auto& t : hub->tiers)
    ThrowOnError(ps_hub_mark_atomic(&t->desc, part->_group_des[0], part->_group_num[0],
                                    reinterpret_cast<uint8_t*>(part->_residue_atomic), nullptr));

  // SDDMM: the tiles (64 consecutive nonzeros of a block group) inside the
  // block leave the run order; their outputs come from the dense products.
  // A tier the cost rule chose serves SDDMM only when its tiles hold at least
  // kHubSddmmMinFill nonzeros per dense element (its D is computed whole);
  // explicit tiers serve both operators.
  std::vector<ps_workset> ws = PublicWorksets();
  const size_t T = hub->tiers.size();
  std::vector<std::vector<uint32_t>> tiles(T);
  std::vector<std::vector<std::vector<uint8_t>>> flags(T, std::vector<std::vector<uint8_t>>(size_t(S)));
  DeviceArray<uint8_t> f_dev;
  for (int s = 1; s < S; ++s) {
    const int G = _group_num[s], GS = GROUP_SIZE(s);
    if (G == 0 || GS < 64) continue;
    const size_t n = size_t(G) * size_t(GS / 64);  // 64-nonzero stretches
    f_dev.Allocate(n);
    for (size_t k = 0; k < T; ++k) {
      ThrowOnError(ps_hub_tile_flags(&hub->tiers[k]->desc, &ws[size_t(s)], f_dev.data(), nullptr));
      std::vector<uint8_t>& f = flags[k][size_t(s)];
      f.resize(n);
      f_dev.Download(f.data(), f.size());
      for (size_t t = 0; t < n; ++t)
        if (f[t]) tiles[k].push_back((uint32_t(s) << 27) | uint32_t(t));
    }
  }
  for (size_t k = 0; k < T && !forced; ++k) {
    const ps_hub_block& d = hub->tiers[k]->desc;
    if (double(tiles[k].size()) * 64.0 < kHubSddmmMinFill * double(d.rows) * double(d.cols))
      tiles[k].clear();
  }
  std::vector<DeviceArray<uint8_t>> skip(static_cast<size_t>(S));
  std::vector<const uint8_t*> skip_ptr(static_cast<size_t>(S), nullptr);
  for (int s = 1; s < S; ++s) {
    std::vector<uint8_t> any;
    for (size_t k = 0; k < T; ++k) {
      const std::vector<uint8_t>& f = flags[k][size_t(s)];
      if (tiles[k].empty() || f.empty()) continue;
      any.resize(f.size(), 0);
      for (size_t t = 0; t < f.size(); ++t) any[t] |= f[t];
    }
    if (std::find(any.begin(), any.end(), uint8_t(1)) == any.end()) continue;
    skip[size_t(s)].Allocate(any.size());
    skip[size_t(s)].Upload(any.data(), any.size());  // tiles inside an SDDMM tier
    skip_ptr[size_t(s)] = skip[size_t(s)].data();
  }
  for (size_t k = 0; k < T; ++k) {
    if (tiles[k].empty()) continue;
    HubTier& t = *hub->tiers[k];
    const uint32_t n = uint32_t(tiles[k].size());
    DeviceArray<uint32_t> codes(n);
    codes.Upload(tiles[k].data(), n);
    t.plan.Allocate(ps_hub_sddmm_plan_bytes(&t.desc, n));
    ThrowOnError(ps_hub_sddmm_plan(&t.desc, S, ws.data(), codes.data(), n, t.plan.data(),
                                   t.plan.size(), nullptr));
    t.plan_tiles = n;
  }
  const int k = RunOrderSlot(PS_OP_SDDMM, 32);
  uint32_t count = 0, kept_tasks = 0;
  ThrowOnError(ps_task_count(PS_OP_SDDMM, 32, S, ws.data(), &count));
  uint32_t* order = nullptr;
  if (count > 0) {
    ThrowOnError(ps_malloc(reinterpret_cast<void**>(&order), sizeof(uint32_t) * count));
    const int rc = ps_task_order_build_subset(PS_OP_SDDMM, 32, S, ws.data(), skip_ptr.data(),
                                              order, count, &kept_tasks, nullptr);
    if (rc != PS_OK) {
      ps_free(order);
      ThrowOnError(rc);
    }
  }
  // the workspace for every width: SpMM runs feature slices of at most 128,
  // SDDMM widths go up to 512
  hub->ws.Allocate(std::max(hub->Workspace(PS_OP_SPMM, 128), hub->Workspace(PS_OP_SDDMM, 512)));
  ThrowOnError(ps_event_create(&hub->done));
  ps_free(_run_order[k]);
  _run_order[k] = order;
  _run_order_tasks[k] = kept_tasks;
  _spmm_tuned = part.release();
  _hub = hub.release();
  return true;
}

void PowerSparseMatrixGPU::HubSpmm(int N, const float* B, float* C, ps_stream_t stream) const {
  HubState& h = *_hub;
  std::lock_guard<std::mutex> lock(h.mu);
  if (h.ws.size() < h.Workspace(PS_OP_SPMM, N))  // allocated for every width with the block
    throw std::logic_error("Hub block workspace smaller than the block needs");
  if (h.recorded) ThrowOnError(ps_stream_wait_event(stream, h.done));
  for (const auto& t : h.tiers)
    ThrowOnError(ps_hub_spmm_launch(&t->desc, N, B, C, h.ws.data(), h.ws.size(), stream));
  ThrowOnError(ps_event_record(h.done, stream));
  h.recorded = true;
}

void PowerSparseMatrixGPU::HubSddmm(int N, const float* lhs, const float* rhs, float* const* out,
                                    float* csr_out, ps_stream_t stream) const {
  HubState& h = *_hub;
  const std::vector<ps_workset> ws = PublicWorksets();
  std::lock_guard<std::mutex> lock(h.mu);
  if (h.ws.size() < h.Workspace(PS_OP_SDDMM, N))  // allocated for every width with the block
    throw std::logic_error("Hub block workspace smaller than the block needs");
  if (h.recorded) ThrowOnError(ps_stream_wait_event(stream, h.done));
  for (const auto& t : h.tiers)
    if (t->plan_tiles)
      ThrowOnError(ps_hub_sddmm_launch(&t->desc, _group_type_num, ws.data(), t->plan.data(),
                                       t->plan_tiles, N, lhs, rhs, out,
                                       csr_out ? _workset_csr_pos : nullptr, csr_out, h.ws.data(),
                                       h.ws.size(), stream));
  ThrowOnError(ps_event_record(h.done, stream));
  h.recorded = true;
}

std::vector<ps_workset> PowerSparseMatrixGPU::PublicWorksets() const {
  const int S = _group_type_num;
  std::vector<ps_workset> ws(static_cast<size_t>(S));
  for (int s = 0; s < S; ++s) {
    ws[size_t(s)].col_ind = _workset_col_ind[s];
    ws[size_t(s)].sp_data = _workset_sp_data[s];
    ws[size_t(s)].group_des = _group_des[s];
    ws[size_t(s)].group_num = _group_num[s];
    ws[size_t(s)].group_size = s == 0 ? 0 : GROUP_SIZE(s);
    ws[size_t(s)].order = nullptr;
  }
  return ws;
}

// The locality run order of each operator's fused launch over the public
// (signature-ordered) worksets; see PartitionPolicy::run_order.
void PowerSparseMatrixGPU::BuildRunOrders() {
  const int S = _group_type_num;
  std::vector<ps_workset> ws(static_cast<size_t>(S));
  for (int s = 0; s < S; ++s) {
    ws[size_t(s)].col_ind = _workset_col_ind[s];
    ws[size_t(s)].sp_data = _workset_sp_data[s];
    ws[size_t(s)].group_des = _group_des[s];
    ws[size_t(s)].group_num = _group_num[s];
    ws[size_t(s)].group_size = s == 0 ? 0 : GROUP_SIZE(s);
    ws[size_t(s)].order = nullptr;
  }
  const int shapes[3][2] = {{PS_OP_SPMM, 32}, {PS_OP_SPMM, 64}, {PS_OP_SDDMM, 32}};
  for (int k = 0; k < 3; ++k) {
    const int op = shapes[k][0], n = shapes[k][1];
    uint32_t count = 0;
    ThrowOnError(ps_task_count(op, n, S, ws.data(), &count));
    if (count == 0) continue;
    ThrowOnError(ps_malloc(reinterpret_cast<void**>(&_run_order[k]), sizeof(uint32_t) * count));
    _run_order_tasks[k] = count;
    ThrowOnError(ps_task_order_build(op, n, S, ws.data(), _run_order[k], count, nullptr));
  }
}

ExecutionLayout PowerSparseMatrixGPU::Execution() const {
  ExecutionLayout e;
  if (_task_order == TaskOrder::kRow) {
    e.col_ind = _exec_col_ind;
    e.sp_data = _exec_sp_data;
    e.group_des = _exec_group_des;
    e.residue_offset = _exec_residue_offset;
    e.residue_atomic = _exec_residue_atomic;
    e.out_base = _exec_out_base;
    e.task_chunk = kRowOrderTaskChunk;
    e.csr_pos = _exec_csr_pos;
  } else {
    e.col_ind = _workset_col_ind;
    e.sp_data = _workset_sp_data;
    e.group_des = _group_des;
    e.residue_offset = _residue_offset;
    e.residue_atomic = _residue_atomic;
    e.csr_pos = _workset_csr_pos;
    for (int k = 0; k < 3; ++k) {
      e.run_order[k] = _run_order[k];
      e.run_order_tasks[k] = _run_order_tasks[k];
    }
  }
  return e;
}

PowerSparseMatrixGPU::~PowerSparseMatrixGPU() { Release(); }

void PowerSparseMatrixGPU::ReleaseExecution() noexcept {
  for (int s = 0; s < _group_type_num; ++s) {
    if (_exec_col_ind) ps_free(_exec_col_ind[s]);
    if (_exec_sp_data) ps_free(_exec_sp_data[s]);
    if (_exec_group_des) ps_free(_exec_group_des[s]);
    if (_exec_out_base) ps_free(_exec_out_base[s]);
    if (_exec_csr_pos) ps_free(_exec_csr_pos[s]);
  }
  delete[] _exec_col_ind;
  delete[] _exec_sp_data;
  delete[] _exec_group_des;
  delete[] _exec_out_base;
  delete[] _exec_csr_pos;
  ps_free(_exec_residue_offset);
  ps_free(_exec_residue_atomic);
  _exec_col_ind = nullptr;
  _exec_sp_data = nullptr;
  _exec_group_des = nullptr;
  _exec_out_base = nullptr;
  _exec_csr_pos = nullptr;
  _exec_residue_offset = nullptr;
  _exec_residue_atomic = nullptr;
}

void PowerSparseMatrixGPU::Release() noexcept {
  ReleaseExecution();
  delete _hub;
  _hub = nullptr;
  delete _spmm_tuned;
  _spmm_tuned = nullptr;
  for (int k = 0; k < 3; ++k) {
    ps_free(_run_order[k]);
    _run_order[k] = nullptr;
    _run_order_tasks[k] = 0;
  }
  for (int s = 0; s < _group_type_num; ++s) {
    if (_workset_col_ind) ps_free(_workset_col_ind[s]);
    if (_workset_sp_data) ps_free(_workset_sp_data[s]);
    if (_group_des) ps_free(_group_des[s]);
    if (_workset_csr_pos) ps_free(_workset_csr_pos[s]);
  }
  delete[] _group_num;
  delete[] _workset_col_ind;
  delete[] _workset_sp_data;
  delete[] _group_des;
  delete[] _workset_csr_pos;
  ps_free(_residue_offset);
  ps_free(_residue_atomic);
  _group_num = nullptr;
  _workset_col_ind = nullptr;
  _workset_sp_data = nullptr;
  _group_des = nullptr;
  _workset_csr_pos = nullptr;
  _residue_offset = nullptr;
  _residue_atomic = nullptr;
}

}  // namespace PowerSparse
